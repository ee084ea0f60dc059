"""Bidirectional window attention with natural-log LSE.

Drop-ins for ``bidir_local_attention`` and ``cached_local_attention``
(dream_dllm_hils/local_attention.py:110-200).  Where the reference zeroes K
and V of inert slots and calls flash-attn with window_size=(W, W), the gfx950
kernel applies the same zero-K / zero-V rule while it streams the keys.
"""

from __future__ import annotations

import math
from typing import Tuple

import torch

from . import _lib
from .sparse_attention import FRAG_ELEMS, kv_fragments, kv_fragments_cached


def _validate_layout(q, k, v, key_valid) -> None:
    # local_attention.py:15-32
    if q.device.type != "cuda":
        raise ValueError("local attention requires CUDA tensors")
    if q.dtype != torch.bfloat16 or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("local attention requires BF16 q, k, and v")
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, and v must have BLHD layout")
    batch, seq_len, h_q, dim = q.shape
    if k.shape[0] != batch or v.shape != k.shape:
        raise ValueError(f"q/k/v batch mismatch: {q.shape}, {k.shape}, {v.shape}")
    if k.shape[-1] != dim or h_q % k.shape[2] != 0:
        raise ValueError("query heads must be divisible by KV heads with equal head_dim")
    if key_valid.shape[0] != batch or key_valid.shape[-1] != k.shape[1]:
        raise ValueError(
            f"key_valid must have shape {(batch, k.shape[1])}, got {tuple(key_valid.shape)}"
        )


def _flash_window(window: int, skip_inert_slots: bool, chunk_size: int) -> int:
    # local_attention.py:57-64
    if skip_inert_slots:
        return int(window + chunk_size - 1)
    return int(window)


def key_parts(batch: int, q_len: int, kv_heads: int, kv_len: int, flash_window: int) -> int:
    """Workgroups per query block of the window attention.  Long
    sequences: one.  A short block (the cached block step: 32 queries, 4 KV
    heads -> 8 workgroups over ~11 key tiles) splits its key tiles so that
    about 64 workgroups run, at least one tile each."""

    blocks = -(-q_len // 16) * kv_heads * batch  # ~16 queries per workgroup (18 for G = 7)
    if blocks >= 128 or blocks == 0:
        return 1
    tiles = (min(q_len, kv_len) + 2 * flash_window) // 64 + 2
    return max(1, min(64, tiles, 64 // blocks, 65535 // max(batch, 1)))


def local_attention_launch(
    q: torch.Tensor,
    kv_frags: torch.Tensor,
    key_valid: torch.Tensor | None,
    flash_window: int,
    inert_chunk: int,
    *,
    kv_len: int | None = None,
    query_positions: torch.Tensor | None = None,
    sm_scale: float | None = None,
    parts: int | None = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """q [B, Lq, Hq, D]; kv_frags = kv_fragments(k, v) of the kv_len-row keys
    (default: key_valid's length, else every row of the fragments).
    ``parts`` splits each query block's key tiles over that many workgroups
    (merged by a second kernel); None picks it with key_parts."""

    B, Lq, Hq, D = q.shape
    if kv_frags.ndim != 4 or kv_frags.shape[0] != B or kv_frags.shape[3] != FRAG_ELEMS:
        raise ValueError(f"kv_frags {tuple(kv_frags.shape)} is not a kv_fragments layout")
    Hkv = kv_frags.shape[1]
    if kv_len is None:
        kv_len = key_valid.shape[-1] if key_valid is not None else kv_frags.shape[2] * 64
    Lk = int(kv_len)
    if not 0 < Lk <= kv_frags.shape[2] * 64 or (Lk + 63) // 64 != kv_frags.shape[2]:
        raise ValueError(f"kv_len {Lk} does not match kv_frags {tuple(kv_frags.shape)}")
    if sm_scale is None:
        sm_scale = D ** -0.5
    if parts is None:
        parts = key_parts(B, Lq, Hkv, Lk, flash_window)
    return torch.ops.mrsa.local_attention(q, kv_frags, key_valid, Lk, int(flash_window),
                                          int(inert_chunk), query_positions, float(sm_scale),
                                          int(parts))


def _local_attention_impl(q, kv_frags, key_valid, kv_len, flash_window, inert_chunk,
                          query_positions, sm_scale, parts):
    B, Lq, Hq, D = q.shape
    Hkv, Lk = kv_frags.shape[1], kv_len
    qc = q.contiguous()
    kf = kv_frags.contiguous()
    kv = None if key_valid is None else key_valid.to(device=q.device, dtype=torch.bool).contiguous()
    pos = None
    if query_positions is not None:
        pos = query_positions.to(device=q.device, dtype=torch.int64).contiguous()
    out = torch.empty(B, Lq, Hq, D, dtype=torch.bfloat16, device=q.device)
    lse = torch.empty(B, Lq, Hq, dtype=torch.float32, device=q.device)
    args = (_lib.ptr(qc), _lib.ptr(kf), _lib.ptr(kv), _lib.ptr(pos),
            B, Lq, Lk, Hq, Hkv, D, int(flash_window), int(inert_chunk), float(sm_scale))
    if parts == 1:
        st = _lib.call("mrsa_local_attention_fwd", *args, _lib.ptr(out), _lib.ptr(lse),
                       _lib.stream_of(qc))
    else:
        nbytes = _lib.call("mrsa_local_attention_workspace_bytes", B, Lq, Hq, parts)
        ws = torch.empty(max(nbytes, 0) // 4, dtype=torch.float32, device=q.device)
        st = _lib.call("mrsa_local_attention_split_fwd", *args, parts, _lib.ptr(ws), int(nbytes),
                       _lib.ptr(out), _lib.ptr(lse), _lib.stream_of(qc))
    _lib.check(st, "local_attention")
    return out, lse


def local_attention_qf_launch(q: torch.Tensor, kv_frags: torch.Tensor,
                              key_valid: torch.Tensor | None, flash_window: int,
                              inert_chunk: int, *, sm_scale: float | None = None):
    """local_attention_launch over every query row (no key split) that also
    returns q_fragments(q, Hkv), written by the window kernel from the Q
    operands it loads anyway: (out, lse, q_frags)."""

    B, Lq, Hq, D = q.shape
    if kv_frags.ndim != 4 or kv_frags.shape[0] != B or kv_frags.shape[3] != FRAG_ELEMS:
        raise ValueError(f"kv_frags {tuple(kv_frags.shape)} is not a kv_fragments layout")
    Lk = key_valid.shape[-1] if key_valid is not None else kv_frags.shape[2] * 64
    if (Lk + 63) // 64 != kv_frags.shape[2]:
        raise ValueError(f"kv_len {Lk} does not match kv_frags {tuple(kv_frags.shape)}")
    if sm_scale is None:
        sm_scale = D ** -0.5
    return torch.ops.mrsa.local_attention_qf(q, kv_frags, key_valid, int(Lk), int(flash_window),
                                             int(inert_chunk), float(sm_scale))


def _local_attention_qf_impl(q, kv_frags, key_valid, kv_len, flash_window, inert_chunk,
                             sm_scale):
    B, Lq, Hq, D = q.shape
    Hkv = kv_frags.shape[1]
    qc = q.contiguous()
    kf = kv_frags.contiguous()
    kv = None if key_valid is None else key_valid.to(device=q.device, dtype=torch.bool).contiguous()
    out = torch.empty(B, Lq, Hq, D, dtype=torch.bfloat16, device=q.device)
    lse = torch.empty(B, Lq, Hq, dtype=torch.float32, device=q.device)
    qf = torch.empty(B, Hkv, Lq, 1024, dtype=torch.bfloat16, device=q.device)
    st = _lib.call("mrsa_local_attention_qf_fwd", _lib.ptr(qc), _lib.ptr(kf), _lib.ptr(kv),
                   None, B, Lq, kv_len, Hq, Hkv, D, int(flash_window), int(inert_chunk),
                   float(sm_scale), _lib.ptr(qf), _lib.ptr(out), _lib.ptr(lse),
                   _lib.stream_of(qc))
    _lib.check(st, "local_attention_qf")
    return out, lse, qf


def local_attention_backward(q, k, v, key_valid, out, lse, grad_out, flash_window, inert_chunk,
                             *, sm_scale=None):
    """Gradients (dq, dk, dv; fp32) of the window attention of full sequences
    (local_attention_launch with kv_len = q_len and no query positions): the
    gradient flash-attn's flash_attn_func gives (local_attention.py:67-107),
    with zero dk / dv for inert keys (:50-54).  out and lse are the forward's
    outputs; the LSE carries no gradient."""

    B, L, Hq, D = q.shape
    Hkv = k.shape[2]
    if k.shape[1] != L or v.shape != k.shape or out.shape != q.shape or grad_out.shape != q.shape:
        raise ValueError("local attention backward requires equal Q/K lengths and matching shapes")
    if sm_scale is None:
        sm_scale = D ** -0.5
    qc = q.to(torch.bfloat16).contiguous()
    kc = k.to(torch.bfloat16).contiguous()
    vc = v.to(torch.bfloat16).contiguous()
    oc = out.to(torch.bfloat16).contiguous()
    go = grad_out.to(torch.bfloat16).contiguous()
    lc = lse.to(torch.float32).contiguous()
    kv = None if key_valid is None else key_valid.to(device=q.device, dtype=torch.bool).contiguous()
    dq = torch.empty(B, L, Hq, D, dtype=torch.float32, device=q.device)
    dk = torch.empty(B, L, Hkv, D, dtype=torch.float32, device=q.device)
    dv = torch.empty(B, L, Hkv, D, dtype=torch.float32, device=q.device)
    nbytes = int(_lib.call("mrsa_local_attention_bwd_workspace_bytes", B, L, Hq, Hkv))
    if nbytes < 0:
        raise ValueError(f"invalid local attention shapes q {tuple(q.shape)} k {tuple(k.shape)}")
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=q.device)
    st = _lib.call(
        "mrsa_local_attention_bwd",
        _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(vc), _lib.ptr(kv), _lib.ptr(oc), _lib.ptr(lc),
        _lib.ptr(go), B, L, Hq, Hkv, D, int(flash_window), int(inert_chunk), float(sm_scale),
        _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(ws), nbytes, _lib.stream_of(qc),
    )
    _lib.check(st, "local_attention backward")
    return dq, dk, dv


class _LocalAttention(torch.autograd.Function):
    # flash_attn_func's autograd as bidir_local_attention uses it: gradients
    # for q, k, v; the LSE output is not differentiable.
    @staticmethod
    def forward(ctx, q, k, v, key_valid, flash_window, inert_chunk):
        out, lse = local_attention_launch(q, kv_fragments_cached(k, v), key_valid, flash_window,
                                          inert_chunk, kv_len=k.shape[1])
        ctx.mark_non_differentiable(lse)
        ctx.save_for_backward(q, k, v, key_valid, out, lse)
        ctx.flash_window, ctx.inert_chunk = flash_window, inert_chunk
        return out, lse

    @staticmethod
    def backward(ctx, grad_out, grad_lse):
        q, k, v, key_valid, out, lse = ctx.saved_tensors
        dq, dk, dv = local_attention_backward(q, k, v, key_valid, out, lse, grad_out,
                                              ctx.flash_window, ctx.inert_chunk)
        return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), None, None, None


def local_attention_autograd(q, k, v, key_valid, flash_window, inert_chunk):
    """(out, lse) of the full-sequence window attention, differentiable in q,
    k and v when one of them requires grad."""

    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
        return _LocalAttention.apply(q, k, v, key_valid, int(flash_window), int(inert_chunk))
    return local_attention_launch(q, kv_fragments_cached(k, v), key_valid, flash_window,
                                  inert_chunk, kv_len=k.shape[1])


def bidir_local_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    key_valid: torch.Tensor,
    window: int,
    chunk_size: int,
    allowed_mask: torch.Tensor | None = None,
    skip_inert_slots: bool = False,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Bidirectional local GQA attention and natural-log LSE [B, L, Hq];
    differentiable in q, k and v (the LSE is not), as flash_attn_func is."""

    _validate_layout(q, k, v, key_valid)
    seq_len = q.shape[1]
    if k.shape[1] != seq_len:
        raise ValueError("prefill local attention requires equal Q/K lengths")
    if window < 0 or chunk_size <= 0 or seq_len % chunk_size != 0:
        raise ValueError(
            f"invalid window/chunk layout: L={seq_len}, W={window}, S={chunk_size}"
        )
    if allowed_mask is not None:
        raise ValueError(
            "bidir_local_attention only accepts 2D key_valid; "
            "do not pass a dense L×L allowed_mask"
        )
    return local_attention_autograd(
        q, k, v, key_valid, _flash_window(window, skip_inert_slots, chunk_size),
        chunk_size if skip_inert_slots else 0,
    )


def cached_local_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    key_valid: torch.Tensor,
    query_positions: torch.Tensor,
    window: int,
    chunk_size: int,
    skip_inert_slots: bool = False,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Fast-dLLM query rows against a windowed K/V cache (local_attention.py:147-200)."""

    _validate_layout(q, k, v, key_valid)
    batch, query_len, h_q, dim = q.shape
    seq_len = k.shape[1]
    if query_positions.shape != (query_len,):
        raise ValueError(
            f"query_positions must have shape {(query_len,)}, "
            f"got {tuple(query_positions.shape)}"
        )
    if query_positions.device != q.device or query_positions.dtype != torch.long:
        raise ValueError("query_positions must be CUDA torch.long")
    if query_len == 0:
        empty_lse = q.new_empty((batch, 0, h_q), dtype=torch.float32)
        return q.new_empty((batch, 0, h_q, dim)), empty_lse
    if torch.unique(query_positions).numel() != query_len:
        raise ValueError("query_positions must be unique")
    if bool(((query_positions < 0) | (query_positions >= seq_len)).any()):
        raise ValueError("query_positions must be in cache range")
    if window < 0 or chunk_size <= 0 or seq_len % chunk_size:
        raise ValueError(
            f"invalid window/chunk layout: L={seq_len}, W={window}, S={chunk_size}"
        )
    return local_attention_launch(
        q, kv_fragments_cached(k, v), key_valid,
        _flash_window(window, skip_inert_slots, chunk_size),
        chunk_size if skip_inert_slots else 0, kv_len=seq_len,
        query_positions=query_positions,
    )
