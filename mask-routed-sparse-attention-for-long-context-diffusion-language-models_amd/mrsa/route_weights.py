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


def _gate_tensor(x, device):
    """A gate parameter as an fp32 device scalar the kernel reads in place.

    Tensors (the layer's nn.Parameters) are used where they live, without a
    host round trip; Python numbers become a device scalar through a fill
    kernel (no copy from host memory).  None stays None ("not given").
    """

    if x is None:
        return None
    if isinstance(x, torch.Tensor):
        if x.numel() != 1:
            raise ValueError(f"gate parameters must hold one value, got shape {tuple(x.shape)}")
        return x.detach().to(device=device, dtype=torch.float32).reshape(()).contiguous()
    if torch.compiler.is_compiling() or torch._guards.detect_fake_mode() is not None:
        # traced: a fill op in the graph (a cached tensor would be a fake one)
        return torch.full((), float(x), dtype=torch.float32, device=device)
    key = (float(x), device)
    t = _GATE_CONSTANTS.get(key)
    if t is None:
        if len(_GATE_CONSTANTS) > 64:
            _GATE_CONSTANTS.clear()
        t = _GATE_CONSTANTS[key] = torch.full((), float(x), dtype=torch.float32, device=device)
    return t


# Device scalars made for numeric gate values, reused across calls.
_GATE_CONSTANTS: dict = {}


def route_weights_launch(
    scores: torch.Tensor,
    indices: torch.Tensor,
    prior_bias: torch.Tensor,
    local_lse: torch.Tensor,
    *,
    temperature: float = 1.0,
    gate_offset=None,
    gate_scale=None,
    return_gate_logit: bool = False,
    value_bonus=None,
    selected_gumbel=None,
):
    """Forward kernel call.  gate_offset / gate_scale: None, a number or a
    one-element tensor; value_bonus / selected_gumbel: None or [B, L, Hq, K]
    terms added to the remote logits.  Returns (remote bf16, local bf16[,
    gate_logit fp32])."""

    dev = scores.device
    remote, local, gl = torch.ops.mrsa.route_weights(
        scores, indices, prior_bias, local_lse, float(temperature),
        _gate_tensor(gate_offset, dev), _gate_tensor(gate_scale, dev), bool(return_gate_logit),
        value_bonus, selected_gumbel)
    if return_gate_logit:
        return remote, local, gl
    return remote, local


def _extra(t, like):
    """An additive logit term as the kernels read it: fp32, contiguous."""
    return None if t is None else t.to(device=like.device, dtype=torch.float32).contiguous()


def _route_weights_impl(scores, indices, prior_bias, local_lse, temperature, off, scl,
                        return_gate_logit, value_bonus=None, selected_gumbel=None):
    """Kernel call; the gate-logit output is empty unless requested."""
    B, L, Hq, K = scores.shape
    _, C, Hkv, G = prior_bias.shape
    dev = scores.device
    sc = scores.to(torch.bfloat16).contiguous()
    idx = indices.to(torch.int32).contiguous()
    bias = prior_bias.to(torch.float32).contiguous()
    lse = local_lse.to(torch.float32).reshape(B, L, Hq).contiguous()
    remote = torch.empty(B, L, Hq, K, dtype=torch.bfloat16, device=dev)
    local = torch.empty(B, L, Hq, dtype=torch.bfloat16, device=dev)
    gl = torch.empty(B, L, Hq if return_gate_logit else 0, dtype=torch.float32, device=dev)
    vb, gn = _extra(value_bonus, sc), _extra(selected_gumbel, sc)
    if vb is None and gn is None:
        st = _lib.call(
            "mrsa_route_weights_fwd",
            _lib.ptr(sc), _lib.ptr(idx), _lib.ptr(bias), _lib.ptr(lse),
            B, L, C, Hkv, G, K, float(temperature), _lib.ptr(off), _lib.ptr(scl),
            _lib.ptr(remote), _lib.ptr(local), _lib.ptr(gl) if return_gate_logit else None,
            _lib.stream_of(sc),
        )
    else:
        st = _lib.call(
            "mrsa_route_weights_extra_fwd",
            _lib.ptr(sc), _lib.ptr(idx), _lib.ptr(bias), _lib.ptr(lse),
            B, L, C, Hkv, G, K, float(temperature), _lib.ptr(off), _lib.ptr(scl),
            _lib.ptr(vb), _lib.ptr(gn),
            _lib.ptr(remote), _lib.ptr(local), _lib.ptr(gl) if return_gate_logit else None,
            _lib.stream_of(sc),
        )
    _lib.check(st, "route_weights")
    return remote, local, gl


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
    temperature: float = 1.0, gate_offset=None, gate_scale=None, grad_gate_logit=None,
    value_bonus=None, selected_gumbel=None,
):
    """(d_scores fp32, d_bias fp32, d_local_lse fp32, d_gate fp32[2]) for the
    forward inputs and bf16 upstream gradients (grad_local and
    grad_gate_logit may be None).  d_gate = (d gate_scale, d gate_offset).
    The gradients of value_bonus and selected_gumbel equal d_scores."""

    dev = scores.device
    return torch.ops.mrsa.route_weights_bwd(
        scores, indices, prior_bias, local_lse, grad_remote, grad_local, grad_gate_logit,
        float(temperature), _gate_tensor(gate_offset, dev), _gate_tensor(gate_scale, dev),
        value_bonus, selected_gumbel)


def _route_weights_bwd_impl(scores, indices, prior_bias, local_lse, grad_remote, grad_local,
                            grad_gate_logit, temperature, off, scl, value_bonus=None,
                            selected_gumbel=None):
    sc, idx, bias, lse = _prepared(scores, indices, prior_bias, local_lse)
    B, L, Hq, K = sc.shape
    _, C, Hkv, G = bias.shape
    dev = sc.device
    g_rw = (
        torch.zeros(B, L, Hq, K, dtype=torch.bfloat16, device=dev)
        if grad_remote is None else grad_remote.to(torch.bfloat16).contiguous()
    )
    g_lw = None if grad_local is None else grad_local.to(torch.bfloat16).reshape(B, L, Hq).contiguous()
    g_gl = (None if grad_gate_logit is None
            else grad_gate_logit.to(torch.float32).reshape(B, L, Hq).contiguous())
    d_scores = torch.empty(B, L, Hq, K, dtype=torch.float32, device=dev)
    d_bias = torch.zeros(B, C, Hkv, G, dtype=torch.float32, device=dev)
    d_lse = torch.empty(B, L, Hq, dtype=torch.float32, device=dev)
    d_gate = torch.zeros(2, dtype=torch.float32, device=dev)
    vb, gn = _extra(value_bonus, sc), _extra(selected_gumbel, sc)
    st = _lib.call(
        "mrsa_route_weights_extra_bwd",
        _lib.ptr(sc), _lib.ptr(idx), _lib.ptr(bias), _lib.ptr(lse), _lib.ptr(g_rw),
        _lib.ptr(g_lw), _lib.ptr(g_gl),
        B, L, C, Hkv, G, K, float(temperature), _lib.ptr(off), _lib.ptr(scl),
        _lib.ptr(vb), _lib.ptr(gn),
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
    # autograd of attention.py:126-235 (both forms, gate logit included)
    @staticmethod
    def forward(ctx, scores, indices, prior_bias, local_lse, gate_offset, gate_scale,
                temperature, want_gate_logit, value_bonus=None, selected_gumbel=None):
        prepared = _prepared(scores, indices, prior_bias, local_lse)
        dev = scores.device
        off = _gate_tensor(gate_offset, dev)
        scl = _gate_tensor(gate_scale, dev)
        vb, gn = _extra(value_bonus, scores), _extra(selected_gumbel, scores)
        outs = route_weights_launch(
            *prepared, temperature=temperature, gate_offset=off, gate_scale=scl,
            return_gate_logit=want_gate_logit, value_bonus=vb, selected_gumbel=gn,
        )
        ctx.save_for_backward(*prepared)
        ctx.temperature = temperature
        ctx.gates = (off, scl)
        ctx.params = (gate_offset, gate_scale)
        ctx.extras = (vb, gn)
        ctx.extra_dtypes = tuple(None if t is None else t.dtype
                                 for t in (value_bonus, selected_gumbel))
        ctx.dtypes = (scores.dtype, prior_bias.dtype, local_lse.dtype)
        if want_gate_logit:
            return outs
        gl = torch.zeros(0, dtype=torch.float32, device=dev)
        ctx.mark_non_differentiable(gl)
        return outs[0], outs[1], gl

    @staticmethod
    def backward(ctx, grad_remote, grad_local, grad_gate_logit):
        sc, idx, bias, lse = ctx.saved_tensors
        off, scl = ctx.gates
        if grad_gate_logit is not None and grad_gate_logit.numel() == 0:
            grad_gate_logit = None
        vb, gn = ctx.extras
        d_scores, d_bias, d_lse, d_gate = route_weights_backward(
            sc, idx, bias, lse, grad_remote, grad_local, temperature=ctx.temperature,
            gate_offset=off, gate_scale=scl, grad_gate_logit=grad_gate_logit,
            value_bonus=vb, selected_gumbel=gn,
        )
        s_dt, b_dt, l_dt = ctx.dtypes
        p_off, p_scale = ctx.params
        # value_bonus and selected_gumbel enter the logits as the scores do
        n_in = len(ctx.needs_input_grad)
        d_extra = tuple(None if dt is None or 8 + i >= n_in or not ctx.needs_input_grad[8 + i]
                        else d_scores.to(dt) for i, dt in enumerate(ctx.extra_dtypes))
        return (
            d_scores.to(s_dt), None, d_bias.to(b_dt), d_lse.to(l_dt),
            _gate_grad(p_off, d_gate[1]), _gate_grad(p_scale, d_gate[0]), None, None,
        ) + d_extra[:n_in - 8]


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
        remote, local, _ = _RouteWeights.apply(scores, indices, prior_bias, local_lse, None, None,
                                               1.0, False)
        return remote, local
    return route_weights_launch(scores, indices, prior_bias, local_lse)


def route_weights_torch(
    scores, indices, prior_bias, local_lse, *, temperature, selected_gumbel=None,
    value_bonus=None, return_gate_logit=False, gate_offset=None, gate_scale=None,
):
    """Same contract as attention.py:126-235.

    gate_scale selects the affine-sigmoid form; gate_offset / gate_scale are
    read on the device (the layer's parameters, no host round trip).  With
    return_gate_logit the third output is the fp32 gate logit.
    value_bonus and selected_gumbel (attention.py:172-181: value-aware fusion
    and top-k-restricted Gumbel noise) are added to the remote logits after
    the bias, in that order; both are differentiable.
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
    if selected_gumbel is not None and selected_gumbel.shape != scores.shape:
        raise ValueError(f"invalid selected_gumbel shape {tuple(selected_gumbel.shape)}")
    if value_bonus is not None and value_bonus.shape != scores.shape:
        raise ValueError(f"invalid value_bonus shape {tuple(value_bonus.shape)}")
    if scores.device.type != "cuda":
        raise ValueError("route_weights requires CUDA tensors")
    if _needs_grad(scores, prior_bias, local_lse, gate_offset, gate_scale, value_bonus,
                   selected_gumbel):
        remote, local, gl = _RouteWeights.apply(
            scores, indices, prior_bias, local_lse, gate_offset, gate_scale, float(temperature),
            bool(return_gate_logit), value_bonus, selected_gumbel,
        )
        return (remote, local, gl) if return_gate_logit else (remote, local)
    return route_weights_launch(
        scores, indices, prior_bias, local_lse, temperature=temperature,
        gate_offset=gate_offset, gate_scale=gate_scale, return_gate_logit=return_gate_logit,
        value_bonus=value_bonus, selected_gumbel=selected_gumbel,
    )
