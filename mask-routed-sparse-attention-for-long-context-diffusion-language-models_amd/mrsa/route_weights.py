"""Route weights: normalise routed chunk logits against the local branch.

Drop-ins for ``route_weights`` (ops/hils_bidir_route_weights_tilelang.py:276-290,
topk <= 31) and ``_route_weights_torch`` (dream_dllm_hils/attention.py:126-235,
the path the route layer takes at topk = 32).  The backward recomputes the
row probabilities on the gfx950 backward kernel (mrsa_route_weights_bwd) and
returns the gradients of scores, prior_bias, local_lse and the gate tensors.
"""

from __future__ import annotations

import torch

from . import _lib


def route_weights_launch(
    scores: torch.Tensor,
    indices: torch.Tensor,
    prior_bias: torch.Tensor,
    local_lse: torch.Tensor,
    *,
    temperature: float = 1.0,
    gate_offset: float | None = None,
    gate_scale: float | None = None,
):
    B, L, Hq, K = scores.shape
    _, C, Hkv, G = prior_bias.shape
    sc = scores.to(torch.bfloat16).contiguous()
    idx = indices.to(torch.int32).contiguous()
    bias = prior_bias.to(torch.float32).contiguous()
    lse = local_lse.to(torch.float32).reshape(B, L, Hq).contiguous()
    remote = torch.empty(B, L, Hq, K, dtype=torch.bfloat16, device=scores.device)
    local = torch.empty(B, L, Hq, dtype=torch.bfloat16, device=scores.device)
    st = _lib.call(
        "mrsa_route_weights_fwd",
        _lib.ptr(sc), _lib.ptr(idx), _lib.ptr(bias), _lib.ptr(lse),
        B, L, C, Hkv, G, K, float(temperature),
        0 if gate_offset is None else 1, 0.0 if gate_offset is None else float(gate_offset),
        0 if gate_scale is None else 1, 1.0 if gate_scale is None else float(gate_scale),
        _lib.ptr(remote), _lib.ptr(local), _lib.stream_of(sc),
    )
    _lib.check(st, "route_weights")
    return remote, local


def _prepared(scores, indices, prior_bias, local_lse):
    B, L, Hq, _ = scores.shape
    return (
        scores.to(torch.bfloat16).contiguous(),
        indices.to(torch.int32).contiguous(),
        prior_bias.to(torch.float32).contiguous(),
        local_lse.to(torch.float32).reshape(B, L, Hq).contiguous(),
    )


def route_weights_backward(
    scores, indices, prior_bias, local_lse, grad_remote, grad_local, *,
    temperature: float = 1.0, gate_offset: float | None = None, gate_scale: float | None = None,
):
    """(d_scores fp32, d_bias fp32, d_local_lse fp32, d_gate fp32[2]) for the
    forward inputs and bf16 upstream gradients (grad_local may be None)."""

    sc, idx, bias, lse = _prepared(scores, indices, prior_bias, local_lse)
    B, L, Hq, K = sc.shape
    _, C, Hkv, G = bias.shape
    dev = sc.device
    g_rw = (
        torch.zeros(B, L, Hq, K, dtype=torch.bfloat16, device=dev)
        if grad_remote is None else grad_remote.to(torch.bfloat16).contiguous()
    )
    g_lw = None if grad_local is None else grad_local.to(torch.bfloat16).reshape(B, L, Hq).contiguous()
    d_scores = torch.empty(B, L, Hq, K, dtype=torch.float32, device=dev)
    d_bias = torch.zeros(B, C, Hkv, G, dtype=torch.float32, device=dev)
    d_lse = torch.empty(B, L, Hq, dtype=torch.float32, device=dev)
    d_gate = torch.zeros(2, dtype=torch.float32, device=dev)
    st = _lib.call(
        "mrsa_route_weights_bwd",
        _lib.ptr(sc), _lib.ptr(idx), _lib.ptr(bias), _lib.ptr(lse), _lib.ptr(g_rw),
        None if g_lw is None else _lib.ptr(g_lw),
        B, L, C, Hkv, G, K, float(temperature),
        0 if gate_offset is None else 1, 0.0 if gate_offset is None else float(gate_offset),
        0 if gate_scale is None else 1, 1.0 if gate_scale is None else float(gate_scale),
        _lib.ptr(d_scores), _lib.ptr(d_bias), _lib.ptr(d_lse), _lib.ptr(d_gate),
        _lib.stream_of(sc),
    )
    _lib.check(st, "route_weights backward")
    return d_scores, d_bias, d_lse, d_gate


def _gate_grad(param, value):
    if not isinstance(param, torch.Tensor) or not param.requires_grad:
        return None
    return value.to(param.dtype).reshape(param.shape)


class _RouteWeights(torch.autograd.Function):
    # ops/hils_bidir_route_weights_tilelang.py:169-242 (plain form) and the
    # autograd of attention.py:126-235 (both forms)
    @staticmethod
    def forward(ctx, scores, indices, prior_bias, local_lse, gate_offset, gate_scale, temperature):
        off, scale = _scalar(gate_offset), _scalar(gate_scale)
        prepared = _prepared(scores, indices, prior_bias, local_lse)
        remote, local = route_weights_launch(
            *prepared, temperature=temperature, gate_offset=off, gate_scale=scale
        )
        ctx.save_for_backward(*prepared)
        ctx.opts = (temperature, off, scale)
        ctx.params = (gate_offset, gate_scale)
        ctx.dtypes = (scores.dtype, prior_bias.dtype, local_lse.dtype)
        return remote, local

    @staticmethod
    def backward(ctx, grad_remote, grad_local):
        sc, idx, bias, lse = ctx.saved_tensors
        temperature, off, scale = ctx.opts
        d_scores, d_bias, d_lse, d_gate = route_weights_backward(
            sc, idx, bias, lse, grad_remote, grad_local,
            temperature=temperature, gate_offset=off, gate_scale=scale,
        )
        s_dt, b_dt, l_dt = ctx.dtypes
        p_off, p_scale = ctx.params
        return (
            d_scores.to(s_dt), None, d_bias.to(b_dt), d_lse.to(l_dt),
            _gate_grad(p_off, d_gate[1]), _gate_grad(p_scale, d_gate[0]), None,
        )


def _needs_grad(*xs):
    return torch.is_grad_enabled() and any(
        isinstance(x, torch.Tensor) and x.requires_grad for x in xs
    )


def _validate(scores, indices, prior_bias, local_lse):
    # ops/hils_bidir_route_weights_tilelang.py:244-273
    if scores.device.type != "cuda":
        raise ValueError("route_weights requires CUDA tensors")
    if not (scores.device == indices.device == prior_bias.device == local_lse.device):
        raise ValueError("all route_weights tensors must share one CUDA device")
    if scores.ndim != 4 or indices.ndim != 4 or prior_bias.ndim != 4:
        raise ValueError("scores, indices, and prior_bias must be 4D")
    if local_lse.ndim != 3:
        raise ValueError("local_lse must be [B,L,Hq]")
    batch, seq_len, h_q, topk = scores.shape
    bias_batch, chunks, kv_heads, groups = prior_bias.shape
    if topk <= 0 or topk + 1 > 32:
        raise ValueError(f"route_weights requires 1 <= topk <= 31, got {topk}")
    if groups <= 0 or groups > 16 or h_q != kv_heads * groups:
        raise ValueError(
            f"invalid grouped-head layout Hq={h_q}, Hkv={kv_heads}, G={groups}"
        )
    if bias_batch != batch or chunks <= 0:
        raise ValueError(f"invalid prior_bias shape {tuple(prior_bias.shape)}")
    if indices.shape != (batch, seq_len, kv_heads, topk):
        raise ValueError(f"invalid indices shape {tuple(indices.shape)}")
    if local_lse.shape != (batch, seq_len, h_q):
        raise ValueError(f"invalid local_lse shape {tuple(local_lse.shape)}")
    if scores.dtype != torch.bfloat16:
        raise ValueError("route_weights requires BF16 scores")
    if prior_bias.dtype != torch.float32 or local_lse.dtype != torch.float32:
        raise ValueError("prior_bias and local_lse must be FP32")


def route_weights(scores, indices, prior_bias, local_lse):
    """33-way softmax of [score + bias, local_lse] (topk <= 31); bf16 outputs."""

    _validate(scores, indices, prior_bias, local_lse)
    if _needs_grad(scores, prior_bias, local_lse):
        return _RouteWeights.apply(scores, indices, prior_bias, local_lse, None, None, 1.0)
    return route_weights_launch(scores, indices, prior_bias, local_lse)


def _scalar(x):
    if x is None:
        return None
    if isinstance(x, torch.Tensor):
        return float(x.detach().float().reshape(()).item())
    return float(x)


def route_weights_torch(
    scores, indices, prior_bias, local_lse, *, temperature, selected_gumbel=None,
    value_bonus=None, return_gate_logit=False, gate_offset=None, gate_scale=None,
):
    """Same contract as attention.py:126-235 for the forward outputs.

    gate_scale selects the affine-sigmoid form.  The training-only inputs
    (selected_gumbel, value_bonus) and the gate-logit diagnostic are not
    produced by the forward kernel.
    """

    if temperature <= 0:
        raise ValueError(f"temperature must be positive, got {temperature}")
    if scores.ndim != 4 or indices.ndim != 4 or prior_bias.ndim != 4:
        raise ValueError("scores, indices, and prior_bias must be 4D")
    if local_lse.ndim != 3:
        raise ValueError("local_lse must be [B,L,Hq]")
    batch, seq_len, h_q, topk = scores.shape
    bias_batch, chunks, h_kv, groups = prior_bias.shape
    if chunks <= 0:
        raise ValueError("prior_bias must contain at least one chunk")
    if h_q != h_kv * groups:
        raise ValueError(f"invalid grouped-head layout Hq={h_q}, Hkv={h_kv}, G={groups}")
    if bias_batch != batch:
        raise ValueError(f"invalid prior_bias shape {tuple(prior_bias.shape)}")
    if indices.shape != (batch, seq_len, h_kv, topk):
        raise ValueError(f"invalid indices shape {tuple(indices.shape)}")
    if local_lse.shape != (batch, seq_len, h_q):
        raise ValueError(f"invalid local_lse shape {tuple(local_lse.shape)}")
    if selected_gumbel is not None or value_bonus is not None:
        raise ValueError("selected_gumbel / value_bonus are training-only inputs; not supported")
    if return_gate_logit:
        raise ValueError("return_gate_logit is a training diagnostic; not produced by the kernel")
    if scores.device.type != "cuda":
        raise ValueError("route_weights requires CUDA tensors")
    if _needs_grad(scores, prior_bias, local_lse, gate_offset, gate_scale):
        return _RouteWeights.apply(
            scores, indices, prior_bias, local_lse, gate_offset, gate_scale, float(temperature)
        )
    return route_weights_launch(
        scores, indices, prior_bias, local_lse, temperature=temperature,
        gate_offset=_scalar(gate_offset), gate_scale=_scalar(gate_scale),
    )
