"""Candidate token scores inside routed chunks.

Drop-in for ``ops.hils_token_score_gqa_tilelang.candidate_token_scores_gqa``
(ops/hils_token_score_gqa_tilelang.py:174-208).
"""

from __future__ import annotations

import math

import torch

from . import _lib
from .sparse_attention import FRAG_ELEMS, kv_fragments, kv_fragments_cached


def _validate(q, k, indices, key_valid, chunk_size):
    # ops/hils_token_score_gqa_tilelang.py:117-171
    if q.device.type != "cuda":
        raise ValueError("candidate_token_scores_gqa requires CUDA tensors")
    if not (q.device == k.device == indices.device == key_valid.device):
        raise ValueError("all token-score tensors must share one CUDA device")
    if q.ndim != 4 or k.ndim != 4 or indices.ndim != 4:
        raise ValueError("q, k, and indices must be rank-four tensors")
    batch, query_len, query_heads, head_dim = q.shape
    if k.shape[0] != batch or k.shape[-1] != head_dim:
        raise ValueError(f"incompatible q/k shapes {tuple(q.shape)} and {tuple(k.shape)}")
    kv_len, kv_heads = k.shape[1:3]
    if query_heads % kv_heads:
        raise ValueError(f"query_heads={query_heads} must divide kv_heads={kv_heads}")
    selected = indices.shape[-1]
    if indices.shape != (batch, query_len, kv_heads, selected):
        raise ValueError(f"invalid indices shape {tuple(indices.shape)}")
    if key_valid.shape != (batch, kv_len):
        raise ValueError(f"invalid key_valid shape {tuple(key_valid.shape)}")
    if chunk_size < 16 or kv_len % chunk_size:
        raise ValueError(f"kv_len={kv_len} must be divisible by chunk_size >= 16")
    if head_dim > 256:
        raise ValueError(f"head_dim must be <= 256, got {head_dim}")
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16:
        raise ValueError("candidate_token_scores_gqa requires BF16 q and k")
    if indices.dtype != torch.int32:
        raise ValueError("indices must be int32")
    if not (q.is_contiguous() and k.is_contiguous() and indices.is_contiguous()
            and key_valid.is_contiguous()):
        raise ValueError("candidate_token_scores_gqa requires contiguous tensors")


def candidate_token_scores_gqa(q, k, indices, key_valid, chunk_size, *, kv_frags=None):
    """FP32 [B, Lq, Hkv, K, chunk_size] max-over-group scores of routed tokens.

    ``kv_frags`` (keyword, not in the reference signature): the
    ``kv_fragments`` layout of k when the caller already holds it; built
    from k otherwise."""

    _validate(q, k, indices, key_valid, chunk_size)
    if kv_frags is None:
        kv_frags = kv_fragments_cached(k)
    elif kv_frags.shape != (k.shape[0], k.shape[2], (k.shape[1] + 63) // 64, FRAG_ELEMS):
        raise ValueError("kv_frags must be the kv_fragments layout of k")
    return torch.ops.mrsa.candidate_token_scores(q, kv_frags, indices, key_valid,
                                                 int(chunk_size))


def _token_scores_impl(q, kv_frags, indices, key_valid, chunk_size):
    B, Lq, Hq, D = q.shape
    Hkv, Lk = kv_frags.shape[1], kv_frags.shape[2] * 64
    K = indices.shape[-1]
    kv = key_valid.to(torch.bool).contiguous()
    out = torch.empty(B, Lq, Hkv, K, chunk_size, dtype=torch.float32, device=q.device)
    st = _lib.call(
        "mrsa_candidate_token_scores_fwd",
        _lib.ptr(q), _lib.ptr(kv_frags), _lib.ptr(indices), _lib.ptr(kv),
        B, Lq, Lk, Hq, Hkv, D, K, int(chunk_size), 1.0 / math.sqrt(D),
        _lib.ptr(out), _lib.stream_of(q),
    )
    _lib.check(st, "candidate_token_scores_gqa")
    return out
