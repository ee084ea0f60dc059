"""Layout and chunk-mask helpers.

Mirrors dream_dllm_hils/kernel_utils.py.  ``remote_drop_mask`` runs on the
gfx950 library; the group padding helpers are plain tensor reshapes kept for
callers that still use the physical-G=8 layout (the kernels here take the
logical G=7 layout directly and do not need them).
"""

from __future__ import annotations

from typing import Tuple

import torch

from . import _lib


def _validate_group_layout(x, h_kv, logical_g, physical_g):
    # kernel_utils.py:10-28
    if x.ndim < 2:
        raise ValueError(f"expected at least two dimensions, got {tuple(x.shape)}")
    if h_kv <= 0 or logical_g <= 0 or physical_g < logical_g:
        raise ValueError(
            "expected h_kv > 0 and physical_g >= logical_g > 0; "
            f"got h_kv={h_kv}, logical_g={logical_g}, physical_g={physical_g}"
        )
    expected_heads = h_kv * logical_g
    if x.shape[-2] != expected_heads:
        raise ValueError(
            f"head dimension must be h_kv * logical_g = {expected_heads}, "
            f"got {x.shape[-2]} for shape {tuple(x.shape)}"
        )


def group_pad_to(x, h_kv, logical_g, physical_g, value=0.0):
    """Pad the per-KV-head query-group axis (kernel_utils.py:31-51)."""

    _validate_group_layout(x, h_kv, logical_g, physical_g)
    if physical_g == logical_g:
        return x
    prefix = x.shape[:-2]
    feature = x.shape[-1]
    grouped = x.reshape(*prefix, h_kv, logical_g, feature)
    pad = torch.full(
        (*prefix, h_kv, physical_g - logical_g, feature), value,
        dtype=x.dtype, device=x.device,
    )
    return torch.cat((grouped, pad), dim=-2).reshape(*prefix, h_kv * physical_g, feature)


def group_unpad(x, h_kv, logical_g, physical_g):
    """Remove physical query-group padding (kernel_utils.py:54-72)."""

    if x.ndim < 2 or x.shape[-2] != h_kv * physical_g:
        raise ValueError(
            f"head dimension must be h_kv * physical_g = {h_kv * physical_g}, "
            f"got shape {tuple(x.shape)}"
        )
    prefix = x.shape[:-2]
    feature = x.shape[-1]
    grouped = x.reshape(*prefix, h_kv, physical_g, feature)
    return grouped[..., :logical_g, :].reshape(*prefix, h_kv * logical_g, feature)


def chunk_aligned_local_bounds(
    seq_len: int, window: int, chunk_size: int, device: torch.device
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Inclusive-left / exclusive-right chunk-aligned local bounds (kernel_utils.py:75-99)."""

    if seq_len <= 0:
        raise ValueError(f"seq_len must be positive, got {seq_len}")
    if window < 0:
        raise ValueError(f"window must be non-negative, got {window}")
    if chunk_size <= 0 or seq_len % chunk_size != 0:
        raise ValueError(f"seq_len={seq_len} must be divisible by chunk_size={chunk_size}")
    positions = torch.arange(seq_len, device=device, dtype=torch.long)
    raw_left = (positions - window).clamp_min(0)
    raw_right = (positions + window).clamp_max(seq_len - 1)
    left = torch.div(raw_left, chunk_size, rounding_mode="floor") * chunk_size
    right = (torch.div(raw_right, chunk_size, rounding_mode="floor") + 1) * chunk_size
    return left, right.clamp_max(seq_len)


def remote_drop_mask(
    valid_mask: torch.Tensor,
    window: int,
    chunk_size: int,
    allowed_mask: torch.Tensor | None = None,
) -> torch.Tensor:
    """1 = chunk may not be routed to (local or invalid); int32 [B, L, L/S].

    Same contract as kernel_utils.py:102-161.
    """

    if valid_mask.ndim != 2:
        raise ValueError(
            f"valid_mask must have shape [B, L], got {tuple(valid_mask.shape)}"
        )
    batch, seq_len = valid_mask.shape
    if chunk_size <= 0 or seq_len % chunk_size != 0:
        raise ValueError(
            f"sequence length {seq_len} must be divisible by chunk_size={chunk_size}"
        )
    if allowed_mask is not None and allowed_mask.shape != (batch, seq_len, seq_len):
        raise ValueError(
            "allowed_mask must have shape "
            f"{(batch, seq_len, seq_len)}, got {tuple(allowed_mask.shape)}"
        )
    if valid_mask.device.type != "cuda":
        raise ValueError("remote_drop_mask requires CUDA tensors")
    if window < 0:
        raise ValueError(f"window must be non-negative, got {window}")
    return torch.ops.mrsa.remote_drop_mask(valid_mask, allowed_mask, int(window), int(chunk_size))


def _drop_mask_impl(valid_mask, allowed_mask, window, chunk_size):
    batch, seq_len = valid_mask.shape
    valid = valid_mask.to(torch.bool).contiguous()
    allowed = None if allowed_mask is None else allowed_mask.to(
        device=valid.device, dtype=torch.bool
    ).contiguous()
    out = torch.empty(
        batch, seq_len, seq_len // chunk_size, dtype=torch.int32, device=valid.device
    )
    st = _lib.call(
        "mrsa_remote_drop_mask", _lib.ptr(valid), _lib.ptr(allowed),
        batch, seq_len, int(window), int(chunk_size), _lib.ptr(out), _lib.stream_of(out),
    )
    _lib.check(st, "remote_drop_mask")
    return out


def remote_drop_mask_rows(
    valid_mask: torch.Tensor,
    window: int,
    chunk_size: int,
    query_positions: torch.Tensor,
) -> torch.Tensor:
    """``remote_drop_mask(valid_mask, window, chunk_size)[:, query_positions]``
    without the full [B, L, L/S] mask; int32 [B, len(query_positions), L/S].

    The cached decode path's drop mask (fastdllm_attention.py:295-299).
    """

    if valid_mask.ndim != 2:
        raise ValueError(
            f"valid_mask must have shape [B, L], got {tuple(valid_mask.shape)}"
        )
    batch, seq_len = valid_mask.shape
    if chunk_size <= 0 or seq_len % chunk_size != 0:
        raise ValueError(
            f"sequence length {seq_len} must be divisible by chunk_size={chunk_size}"
        )
    if window < 0:
        raise ValueError(f"window must be non-negative, got {window}")
    if query_positions.ndim != 1 or query_positions.dtype != torch.long:
        raise ValueError("query_positions must be a 1-D torch.long tensor")
    if valid_mask.device.type != "cuda" or query_positions.device != valid_mask.device:
        raise ValueError("remote_drop_mask_rows requires CUDA tensors on one device")
    rows = query_positions.numel()
    if rows and bool(((query_positions < 0) | (query_positions >= seq_len)).any()):
        raise ValueError("query_positions must be in [0, seq_len)")
    return drop_mask_rows_launch(valid_mask, window, chunk_size, query_positions)


def drop_mask_rows_launch(valid_mask, window, chunk_size, query_positions):
    """remote_drop_mask_rows without the argument checks (positions already
    validated by the caller; the kernel ignores none of them)."""

    return torch.ops.mrsa.remote_drop_mask_rows(valid_mask, query_positions, int(window),
                                                int(chunk_size))


def _drop_mask_rows_impl(valid_mask, query_positions, window, chunk_size):
    batch, seq_len = valid_mask.shape
    rows = query_positions.numel()
    valid = valid_mask.to(torch.bool).contiguous()
    pos = query_positions.contiguous()
    out = torch.empty(batch, rows, seq_len // chunk_size, dtype=torch.int32, device=valid.device)
    st = _lib.call(
        "mrsa_remote_drop_mask_rows", _lib.ptr(valid), _lib.ptr(pos), batch, seq_len, rows,
        int(window), int(chunk_size), _lib.ptr(out), _lib.stream_of(out),
    )
    _lib.check(st, "remote_drop_mask_rows")
    return out
