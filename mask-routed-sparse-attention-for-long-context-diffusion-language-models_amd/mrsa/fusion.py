"""Output fusion: ``remote + local_weight * local``.

Drop-in for ``ops.hils_bidir_output_fusion_tilelang.fuse_hils_outputs``
(ops/hils_bidir_output_fusion_tilelang.py:138-148), with the backward of
``_FuseHiLSOutputs`` (:90-99) on the gfx950 backward kernel.
"""

from __future__ import annotations

import torch

from . import _lib


def _validate(remote_output, local_output, local_weight):
    # ops/hils_bidir_output_fusion_tilelang.py:103-135
    if remote_output.device.type != "cuda":
        raise ValueError("fuse_hils_outputs requires CUDA tensors")
    if not (remote_output.device == local_output.device == local_weight.device):
        raise ValueError("all fusion tensors must share one CUDA device")
    if remote_output.ndim != 4 or local_output.shape != remote_output.shape:
        raise ValueError(
            "remote_output and local_output must have the same [B,L,H,D] shape"
        )
    if local_weight.shape != remote_output.shape[:-1]:
        raise ValueError(
            f"local_weight shape {tuple(local_weight.shape)} must equal "
            f"{tuple(remote_output.shape[:-1])}"
        )
    if remote_output.shape[-1] > 256:
        raise ValueError(f"head_dim must be <= 256, got {remote_output.shape[-1]}")
    if not (
        remote_output.dtype == local_output.dtype == local_weight.dtype == torch.bfloat16
    ):
        raise ValueError("fuse_hils_outputs requires BF16 tensors")
    if not (
        remote_output.is_contiguous()
        and local_output.is_contiguous()
        and local_weight.is_contiguous()
    ):
        raise ValueError("fuse_hils_outputs requires contiguous tensors")


def _fuse_launch(remote_output, local_output, local_weight):
    return torch.ops.mrsa.fuse_hils_outputs(remote_output, local_output, local_weight)


def _fuse_impl(remote_output, local_output, local_weight):
    out = torch.empty_like(remote_output)
    head_dim = remote_output.shape[-1]
    rows = remote_output.numel() // max(head_dim, 1)
    st = _lib.call(
        "mrsa_fuse_hils_outputs_fwd",
        _lib.ptr(remote_output), _lib.ptr(local_output), _lib.ptr(local_weight),
        _lib.ptr(out), rows, head_dim, _lib.stream_of(out),
    )
    _lib.check(st, "fuse_hils_outputs")
    return out


def fuse_hils_outputs_backward(local_output, local_weight, grad_output):
    """(d_remote, d_local, d_weight), all bf16, for a bf16 upstream gradient."""

    return torch.ops.mrsa.fuse_hils_outputs_bwd(local_output, local_weight, grad_output)


def _fuse_bwd_impl(local_output, local_weight, grad_output):
    grad = grad_output.to(torch.bfloat16).contiguous()
    head_dim = local_output.shape[-1]
    rows = local_output.numel() // max(head_dim, 1)
    d_remote = torch.empty_like(local_output)
    d_local = torch.empty_like(local_output)
    d_weight = torch.empty_like(local_weight)
    st = _lib.call(
        "mrsa_fuse_hils_outputs_bwd",
        _lib.ptr(local_output), _lib.ptr(local_weight), _lib.ptr(grad),
        _lib.ptr(d_remote), _lib.ptr(d_local), _lib.ptr(d_weight), rows, head_dim,
        _lib.stream_of(grad),
    )
    _lib.check(st, "fuse_hils_outputs backward")
    return d_remote, d_local, d_weight


class _FuseHiLSOutputs(torch.autograd.Function):
    # ops/hils_bidir_output_fusion_tilelang.py:80-99
    @staticmethod
    def forward(ctx, remote_output, local_output, local_weight):
        ctx.save_for_backward(local_output, local_weight)
        return _fuse_launch(remote_output, local_output, local_weight)

    @staticmethod
    def backward(ctx, grad_output):
        local_output, local_weight = ctx.saved_tensors
        return fuse_hils_outputs_backward(local_output, local_weight, grad_output)


def fuse_hils_outputs(
    remote_output: torch.Tensor,
    local_output: torch.Tensor,
    local_weight: torch.Tensor,
) -> torch.Tensor:
    """Add the weighted local branch to the already weighted remote branch."""

    _validate(remote_output, local_output, local_weight)
    if torch.is_grad_enabled() and (
        remote_output.requires_grad or local_output.requires_grad or local_weight.requires_grad
    ):
        return _FuseHiLSOutputs.apply(remote_output, local_output, local_weight)
    return _fuse_launch(remote_output, local_output, local_weight)
