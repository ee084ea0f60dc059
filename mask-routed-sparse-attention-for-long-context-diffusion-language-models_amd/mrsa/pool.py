"""Landmark chunk-summary attention pool.

Drop-in for ``ops.chunk_attn_pool_gqa_tilelang.chunk_attn_pool_gqa``
(ops/chunk_attn_pool_gqa_tilelang.py:425-448).  Same arguments, validation
messages and outputs.  Under autograd the backward runs the gfx950 pool
backward kernel (mrsa_chunk_attn_pool_gqa_bwd): the fused kernel's gradient
(:183-325) for groups > 1, the autograd of the torch twin (:17-37) for
groups == 1, as the reference dispatches.
"""

from __future__ import annotations

import math

import torch

from . import _lib


def _validate(mu_q, k_chunked, key_valid):
    # ops/chunk_attn_pool_gqa_tilelang.py:404-422
    if mu_q.device.type != "cuda":
        raise ValueError("chunk_attn_pool_gqa requires CUDA tensors")
    if mu_q.dtype != torch.bfloat16 or k_chunked.dtype != torch.bfloat16:
        raise ValueError("chunk_attn_pool_gqa requires BF16 mu_q and K")
    if mu_q.ndim != 5 or k_chunked.ndim != 5:
        raise ValueError("mu_q and k_chunked must be 5D")
    batch, chunks, kv_heads, groups, head_dim = mu_q.shape
    expected_k = (batch, chunks, k_chunked.shape[2], kv_heads, head_dim)
    if k_chunked.shape != expected_k:
        raise ValueError(
            f"expected compact K shape {expected_k}, got {tuple(k_chunked.shape)}"
        )
    if key_valid.shape != (batch, chunks, k_chunked.shape[2]):
        raise ValueError(f"invalid key_valid shape {tuple(key_valid.shape)}")
    if groups > 16:
        raise ValueError(f"groups must be <= 16, got {groups}")


def _launch(mu_q, k_chunked, key_valid, sm_scale, bias_scale=None):
    if bias_scale is not None and bias_scale.numel() != mu_q.shape[2] * mu_q.shape[3]:
        raise ValueError(
            f"bias_scale must have {mu_q.shape[2] * mu_q.shape[3]} elements, "
            f"got {bias_scale.numel()}")
    lmk, entropy, prior = torch.ops.mrsa.chunk_attn_pool(mu_q, k_chunked, key_valid,
                                                         float(sm_scale), bias_scale)
    return lmk, entropy, (prior if bias_scale is not None else None)


def _mu_rows(mu_q):
    """(tensor, row stride) of the landmark query rows [B, C, Hkv, G, D].
    They are read in place when each row's [Hkv, G, D] is contiguous and
    batch and chunk fold into one row stride (e.g. the mask-token rows
    route_q[:, S - 1::S] of the route queries): no gather copy."""
    batch, chunks, kv_heads, groups, head_dim = mu_q.shape
    st_ = mu_q.stride()
    inner = st_[4] == 1 and st_[3] == head_dim and st_[2] == groups * head_dim
    folds = batch == 1 or st_[0] == chunks * st_[1]
    if inner and folds and st_[1] >= kv_heads * groups * head_dim and mu_q.dtype == torch.bfloat16:
        return mu_q, st_[1]
    return mu_q.contiguous(), kv_heads * groups * head_dim


def _kv_fragments_pool_impl(k, v, mu_q, key_valid, sm_scale, bias_scale):
    """K/V fragments of k, v [B, L, Hkv, 128] and the landmark pool of
    mu_q [B, L / 64, Hkv, G, 128] over the same chunks (fused semantics),
    in one kernel: (kv_frags, landmark_keys, entropy, prior_bias)."""
    B, L, H, D = k.shape
    _, C, _, G, _ = mu_q.shape
    kc, vc = k.contiguous(), v.contiguous()
    mu, row_stride = _mu_rows(mu_q)
    kv = key_valid.to(device=k.device, dtype=torch.bool).contiguous()
    frags = torch.empty(B, H, C, 16384, dtype=torch.bfloat16, device=k.device)
    lmk = torch.empty(mu_q.shape, dtype=torch.bfloat16, device=k.device)
    entropy = torch.empty(B, C, H, G, device=k.device, dtype=torch.float32)
    scale = bias_scale.to(device=k.device, dtype=torch.float32).contiguous()
    prior = torch.empty_like(entropy)
    st = _lib.call(
        "mrsa_kv_fragments_pool_fwd",
        _lib.ptr(kc), _lib.ptr(vc), _lib.ptr(mu), int(row_stride), _lib.ptr(kv),
        B, L, H, G, D, float(sm_scale), _lib.ptr(scale), _lib.ptr(frags), _lib.ptr(lmk),
        _lib.ptr(entropy), _lib.ptr(prior), _lib.stream_of(kc),
    )
    _lib.check(st, "kv_fragments_pool")
    return frags, lmk, entropy, prior


def kv_fragments_pool(k, v, mu_q, key_valid, entropy_bias_scale, sm_scale=None):
    """kv_fragments(k, v) and chunk_attn_pool_gqa_prior(mu_q, k chunked,
    key_valid chunked, entropy_bias_scale) in one pass over the keys (same
    bits).  k, v [B, L, Hkv, 128] bf16 with L a multiple of 64; mu_q
    [B, L / 64, Hkv, G, 128] bf16, 2 <= G <= 16; key_valid [B, L].
    Returns (kv_frags, landmark_keys, entropy, prior_bias); no autograd."""

    B, L, H, D = k.shape
    if v is None or v.shape != k.shape or D != 128 or L % 64:
        raise ValueError("kv_fragments_pool requires k, v [B, L, Hkv, 128] with L % 64 == 0")
    if mu_q.ndim != 5 or tuple(mu_q.shape[:3]) != (B, L // 64, H) or mu_q.shape[4] != D:
        raise ValueError(f"mu_q must be [B, L / 64, Hkv, G, 128], got {tuple(mu_q.shape)}")
    G = mu_q.shape[3]
    if not 2 <= G <= 16:
        raise ValueError(f"kv_fragments_pool needs 2 <= groups <= 16, got {G}")
    if tuple(key_valid.shape) != (B, L):
        raise ValueError(f"key_valid must be [B, L] = {(B, L)}, got {tuple(key_valid.shape)}")
    if entropy_bias_scale.numel() != H * G:
        raise ValueError(f"bias_scale must have {H * G} elements, got {entropy_bias_scale.numel()}")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    return torch.ops.mrsa.kv_fragments_pool(k, v, mu_q, key_valid, float(sm_scale),
                                            entropy_bias_scale)


def _pool_impl(mu_q, k_chunked, key_valid, sm_scale, bias_scale):
    """Kernel call; the prior output is empty without a bias scale."""
    batch, chunks, kv_heads, groups, head_dim = mu_q.shape
    chunk_size = k_chunked.shape[2]
    mu, row_stride = _mu_rows(mu_q)
    kc = k_chunked.contiguous()
    kv = key_valid.to(device=mu_q.device, dtype=torch.bool).contiguous()
    lmk = torch.empty(mu_q.shape, dtype=torch.bfloat16, device=mu_q.device)
    entropy = torch.empty(
        batch, chunks, kv_heads, groups, device=mu.device, dtype=torch.float32
    )
    prior = entropy.new_empty(0)
    scale = None
    if bias_scale is not None:
        scale = bias_scale.to(device=mu.device, dtype=torch.float32).contiguous()
        prior = torch.empty_like(entropy)
    st = _lib.call(
        "mrsa_chunk_attn_pool_gqa_strided_fwd",
        _lib.ptr(mu), int(row_stride), _lib.ptr(kc), _lib.ptr(kv),
        batch * chunks, chunk_size, kv_heads, groups, head_dim,
        float(sm_scale), 1 if groups == 1 else 0,
        _lib.ptr(scale), _lib.ptr(lmk), _lib.ptr(entropy),
        _lib.ptr(prior) if scale is not None else None, _lib.stream_of(mu),
    )
    _lib.check(st, "chunk_attn_pool_gqa")
    return lmk, entropy, prior


def chunk_attn_pool_gqa_backward(mu_q, k_chunked, key_valid, grad_landmark, grad_entropy,
                                 sm_scale):
    """(d_mu_q, d_k_chunked) in bf16 for the pool's upstream gradients
    (either may be None)."""

    return torch.ops.mrsa.chunk_attn_pool_bwd(mu_q, k_chunked, key_valid, grad_landmark,
                                              grad_entropy, float(sm_scale))


def _pool_bwd_impl(mu_q, k_chunked, key_valid, grad_landmark, grad_entropy, sm_scale):
    batch, chunks, kv_heads, groups, head_dim = mu_q.shape
    chunk_size = k_chunked.shape[2]
    mu = mu_q.contiguous()
    kc = k_chunked.contiguous()
    kv = key_valid.to(device=mu.device, dtype=torch.bool).contiguous()
    g_lmk = None if grad_landmark is None else grad_landmark.to(torch.bfloat16).contiguous()
    g_ent = None if grad_entropy is None else grad_entropy.to(torch.float32).contiguous()
    d_mu = torch.empty_like(mu)
    d_k = torch.empty_like(kc)
    st = _lib.call(
        "mrsa_chunk_attn_pool_gqa_bwd",
        _lib.ptr(mu), _lib.ptr(kc), _lib.ptr(kv), _lib.ptr(g_lmk), _lib.ptr(g_ent),
        batch * chunks, chunk_size, kv_heads, groups, head_dim, float(sm_scale),
        1 if groups == 1 else 0, _lib.ptr(d_mu), _lib.ptr(d_k), _lib.stream_of(mu),
    )
    _lib.check(st, "chunk_attn_pool_gqa backward")
    return d_mu, d_k


class _ChunkAttnPoolGQA(torch.autograd.Function):
    # ops/chunk_attn_pool_gqa_tilelang.py:328-394
    @staticmethod
    def forward(ctx, mu_q, k_chunked, key_valid, sm_scale):
        lmk, entropy, _ = _launch(mu_q, k_chunked, key_valid, sm_scale)
        ctx.save_for_backward(mu_q, k_chunked, key_valid)
        ctx.sm_scale = sm_scale
        return lmk, entropy

    @staticmethod
    def backward(ctx, grad_lmk, grad_entropy):
        mu, kc, kv = ctx.saved_tensors
        d_mu, d_k = chunk_attn_pool_gqa_backward(mu, kc, kv, grad_lmk, grad_entropy, ctx.sm_scale)
        return d_mu, d_k, None, None


class _ChunkAttnPoolPrior(torch.autograd.Function):
    # the pool plus prior_bias = entropy * entropy_bias_scale (attention.py:1425-1430)
    @staticmethod
    def forward(ctx, mu_q, k_chunked, key_valid, bias_scale, sm_scale):
        lmk, entropy, prior = _launch(mu_q, k_chunked, key_valid, sm_scale, bias_scale)
        ctx.save_for_backward(mu_q, k_chunked, key_valid, bias_scale, entropy)
        ctx.sm_scale = sm_scale
        return lmk, entropy, prior

    @staticmethod
    def backward(ctx, grad_lmk, grad_entropy, grad_prior):
        mu, kc, kv, scale, entropy = ctx.saved_tensors
        d_scale = None
        if grad_prior is not None:
            s = scale.to(torch.float32).reshape(entropy.shape[2:])
            extra = grad_prior.float() * s
            grad_entropy = extra if grad_entropy is None else grad_entropy.float() + extra
            if ctx.needs_input_grad[3]:
                d_scale = (grad_prior.float() * entropy).sum(dim=(0, 1)).reshape(scale.shape)
                d_scale = d_scale.to(scale.dtype)
        d_mu, d_k = chunk_attn_pool_gqa_backward(mu, kc, kv, grad_lmk, grad_entropy, ctx.sm_scale)
        return d_mu, d_k, None, d_scale, None


def _needs_grad(*xs):
    return torch.is_grad_enabled() and any(
        isinstance(x, torch.Tensor) and x.requires_grad for x in xs
    )


def chunk_attn_pool_gqa(
    mu_q: torch.Tensor,
    k_chunked: torch.Tensor,
    key_valid: torch.Tensor,
    sm_scale: float | None = None,
):
    """Pool compact per-KV-head chunks into per-query-head summaries.

    mu_q [B, C, Hkv, G, D] bf16, k_chunked [B, C, S, Hkv, D] bf16,
    key_valid [B, C, S] -> (landmark_keys [B, C, Hkv, G, D] bf16,
    entropy [B, C, Hkv, G] fp32).
    """

    _validate(mu_q, k_chunked, key_valid)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(mu_q.shape[-1])
    if _needs_grad(mu_q, k_chunked):
        return _ChunkAttnPoolGQA.apply(mu_q, k_chunked, key_valid, float(sm_scale))
    lmk, entropy, _ = _launch(mu_q, k_chunked, key_valid, sm_scale)
    return lmk, entropy


def chunk_attn_pool_gqa_prior(
    mu_q: torch.Tensor,
    k_chunked: torch.Tensor,
    key_valid: torch.Tensor,
    entropy_bias_scale: torch.Tensor,
    sm_scale: float | None = None,
):
    """chunk_attn_pool_gqa plus prior_bias = entropy * entropy_bias_scale.

    The product of attention.py:1425-1430 is written by the same kernel.
    Returns (landmark_keys, entropy, prior_bias).
    """

    _validate(mu_q, k_chunked, key_valid)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(mu_q.shape[-1])
    if _needs_grad(mu_q, k_chunked, entropy_bias_scale):
        return _ChunkAttnPoolPrior.apply(
            mu_q, k_chunked, key_valid, entropy_bias_scale, float(sm_scale)
        )
    return _launch(mu_q, k_chunked, key_valid, sm_scale, entropy_bias_scale)
