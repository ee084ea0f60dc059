"""Remote-token refinement: the "global_qk" and "entropy_adaptive" policies.

Drop-ins for ``select_global_token_keep`` and ``refine_remote_tokens_g7``
(dream_dllm_hils/token_refinement.py:112-148, :359-392): candidate token
scores inside the routed chunks (``candidate_token_scores_gqa``), then the
global top-``token_budget`` keep mask per (query, KV head) from the gfx950
token-keep kernel (mrsa_token_keep_fwd); and for ``allocate_entropy_token_budget``,
``gather_selected_chunk_entropy``, ``select_entropy_adaptive_token_keep`` and
``refine_remote_tokens_entropy_g7`` (:150-438): per-chunk token quotas from
the routed chunks' pool entropy and the per-chunk keep, one kernel
(mrsa_token_keep_entropy_fwd).  The routed attention consumes the mask
through ``token_keep``.
"""

from __future__ import annotations

import math

import torch

from . import _lib
from .token_score import candidate_token_scores_gqa

_MAX_ROW = 4096  # K * chunk_size entries per row the keep kernel holds


def _scores_with_gumbel(scores, *, training=True, use_gumbel=False, gumbel_scale=1.0):
    # token_refinement.py:95-109: Gumbel ranking noise, training only.
    if gumbel_scale < 0:
        raise ValueError(f"gumbel_scale must be non-negative, got {gumbel_scale}")
    if not (bool(training) and bool(use_gumbel) and gumbel_scale > 0):
        return scores
    eps = torch.finfo(torch.float32).eps
    uniform = torch.empty_like(scores, dtype=torch.float32).uniform_(eps, 1.0 - eps)
    noise = -torch.log(-torch.log(uniform)) * float(gumbel_scale)
    noisy = scores.float() + noise
    return noisy.masked_fill(~torch.isfinite(scores), float("-inf"))


def select_global_token_keep(
    scores: torch.Tensor,
    token_budget: int,
    *,
    training: bool = True,
    use_gumbel: bool = False,
    gumbel_scale: float = 1.0,
    _dtype: torch.dtype = torch.uint8,
) -> torch.Tensor:
    """uint8 keep mask [B, L, Hkv, K, S]: in each (b, l, h) row the
    min(budget, K * S) largest scores are kept when finite (ties to the lower
    flat index).  (``_dtype`` int8 gives the same 0/1 bytes as the routed
    kernel's keep mask without a conversion pass.)"""

    if scores.ndim != 5:
        raise ValueError(f"scores must have shape [B,L,Hkv,K,S], got {tuple(scores.shape)}")
    if token_budget <= 0:
        raise ValueError(f"token_budget must be positive, got {token_budget}")
    if scores.device.type != "cuda":
        raise ValueError("select_global_token_keep requires a CUDA tensor")
    ranking = _scores_with_gumbel(
        scores, training=training, use_gumbel=use_gumbel, gumbel_scale=gumbel_scale
    )
    B, L, H, K, S = scores.shape
    n = K * S
    if n > _MAX_ROW:
        raise ValueError(f"K * chunk_size must be <= {_MAX_ROW}, got {n}")
    return torch.ops.mrsa.token_keep(ranking, int(token_budget), _dtype == torch.int8)


def _token_keep_impl(ranking, token_budget, as_int8):
    B, L, H, K, S = ranking.shape
    flat = ranking.to(torch.float32).contiguous()
    keep = torch.empty(B, L, H, K, S, dtype=torch.int8 if as_int8 else torch.uint8,
                       device=ranking.device)
    st = _lib.call("mrsa_token_keep_fwd", _lib.ptr(flat), B * L * H, K * S, int(token_budget),
                   _lib.ptr(keep), _lib.stream_of(flat))
    _lib.check(st, "token_keep")
    return keep


def refine_remote_tokens_g7(
    q: torch.Tensor,
    k: torch.Tensor,
    indices: torch.Tensor,
    key_valid: torch.Tensor,
    chunk_size: int,
    token_budget: int,
    *,
    training: bool = True,
    use_gumbel: bool = False,
    gumbel_scale: float = 1.0,
    kv_frags: torch.Tensor | None = None,
) -> torch.Tensor:
    """int8 keep mask [B, Lq, Hkv, K, chunk_size] of the routed tokens
    (token_refinement.py:359-392).  ``kv_frags``: the ``kv_fragments``
    layout of k when the caller holds it."""

    if q.shape[2] != k.shape[2] * 7:
        raise ValueError("Dream token refinement requires seven query heads per KV head")
    with torch.no_grad():
        scores = candidate_token_scores_gqa(
            q.detach().contiguous(),
            k.detach().contiguous(),
            indices.to(torch.int32).contiguous(),
            key_valid.contiguous(),
            chunk_size,
            kv_frags=kv_frags,
        )
        return select_global_token_keep(
            scores, token_budget, training=training, use_gumbel=use_gumbel,
            gumbel_scale=gumbel_scale, _dtype=torch.int8,
        )


# -- entropy_adaptive ---------------------------------------------------------
def _check_budget(chunk_count, token_budget, min_tokens_per_chunk):
    # token_refinement.py:170-187
    if token_budget <= 0:
        raise ValueError(f"token_budget must be positive, got {token_budget}")
    if min_tokens_per_chunk < 0:
        raise ValueError(
            f"min_tokens_per_chunk must be non-negative, got {min_tokens_per_chunk}")
    if token_budget < chunk_count * min_tokens_per_chunk:
        raise ValueError(
            "token_budget must cover the per-chunk minimum for every candidate: "
            f"{token_budget} < {chunk_count * min_tokens_per_chunk}")


def allocate_entropy_token_budget(entropy: torch.Tensor, capacity: torch.Tensor,
                                  token_budget: int, min_tokens_per_chunk: int = 1
                                  ) -> torch.Tensor:
    """int64 per-chunk token quotas (token_refinement.py:150-241): the capped
    largest-remainder apportionment of min(sum capacity, token_budget) by the
    entropy effective support exp(entropy), over the last dimension."""

    if entropy.shape != capacity.shape:
        raise ValueError(
            f"entropy and capacity shapes differ: {tuple(entropy.shape)} "
            f"and {tuple(capacity.shape)}")
    if entropy.ndim < 1:
        raise ValueError("entropy and capacity must have a chunk dimension")
    _check_budget(capacity.shape[-1], token_budget, min_tokens_per_chunk)
    if entropy.device.type != "cuda":
        raise ValueError("allocate_entropy_token_budget requires CUDA tensors")
    K = capacity.shape[-1]
    ent = entropy.to(torch.float32).reshape(-1, K).contiguous()
    cap = capacity.to(device=entropy.device, dtype=torch.int64).reshape(-1, K).contiguous()
    alloc = torch.empty_like(cap)
    rows = ent.shape[0]
    st = _lib.call("mrsa_token_keep_entropy_fwd", None, _lib.ptr(cap), _lib.ptr(ent), None, None,
                   1, rows, 1, 1, 1, K, 64, int(token_budget), int(min_tokens_per_chunk),
                   None, _lib.ptr(alloc), _lib.stream_of(ent))
    _lib.check(st, "allocate_entropy_token_budget")
    return alloc.reshape(capacity.shape)


def gather_selected_chunk_entropy(entropy: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """fp32 [B, L, Hkv, K]: the group mean of entropy [B, C, Hkv, G] at the
    routed chunks, 0 at negative indices (token_refinement.py:244-284)."""

    if entropy.ndim != 4 or indices.ndim != 4:
        raise ValueError("expected entropy [B,C,Hkv,G] and indices [B,L,Hkv,K]")
    B, C, Hkv, G = entropy.shape
    if indices.shape[0] != B or indices.shape[2] != Hkv:
        raise ValueError(
            f"incompatible entropy/indices shapes {tuple(entropy.shape)} "
            f"and {tuple(indices.shape)}")
    return torch.ops.mrsa.gather_selected_chunk_entropy(entropy, indices)


def _gather_entropy_impl(entropy, indices):
    B, C, Hkv, G = entropy.shape
    L, K = indices.shape[1], indices.shape[-1]
    ent = entropy.to(torch.float32).contiguous()
    idx = indices.to(device=entropy.device, dtype=torch.int32).contiguous()
    out = torch.empty(B, L, Hkv, K, dtype=torch.float32, device=entropy.device)
    st = _lib.call("mrsa_gather_selected_chunk_entropy", _lib.ptr(ent), _lib.ptr(idx), B, L, C,
                   Hkv, G, K, _lib.ptr(out), _lib.stream_of(ent))
    _lib.check(st, "gather_selected_chunk_entropy")
    return out


def _token_keep_entropy_impl(ranking, selected_entropy, entropy, indices, token_budget,
                             min_tokens_per_chunk, as_int8):
    B, L, H, K, S = ranking.shape
    sc = ranking.to(torch.float32).contiguous()
    sel = None if selected_entropy is None else \
        selected_entropy.to(device=sc.device, dtype=torch.float32).contiguous()
    ent = None if entropy is None else entropy.to(device=sc.device, dtype=torch.float32).contiguous()
    idx = None if indices is None else indices.to(device=sc.device, dtype=torch.int32).contiguous()
    C, G = (1, 1) if ent is None else (ent.shape[1], ent.shape[3])
    keep = torch.empty(B, L, H, K, S, dtype=torch.int8 if as_int8 else torch.uint8, device=sc.device)
    alloc = torch.empty(B, L, H, K, dtype=torch.int64, device=sc.device)
    st = _lib.call("mrsa_token_keep_entropy_fwd", _lib.ptr(sc), None, _lib.ptr(sel), _lib.ptr(ent),
                   _lib.ptr(idx), B, L, H, G, C, K, S, int(token_budget),
                   int(min_tokens_per_chunk), _lib.ptr(keep), _lib.ptr(alloc),
                   _lib.stream_of(sc))
    _lib.check(st, "entropy token keep")
    return keep, alloc


def select_entropy_adaptive_token_keep(
    scores: torch.Tensor,
    selected_entropy: torch.Tensor,
    token_budget: int,
    min_tokens_per_chunk: int = 1,
    *,
    training: bool = True,
    use_gumbel: bool = False,
    gumbel_scale: float = 1.0,
    _dtype: torch.dtype = torch.uint8,
) -> tuple[torch.Tensor, torch.Tensor]:
    """(keep uint8 [B, L, Hkv, K, S], allocation int64 [B, L, Hkv, K])
    (token_refinement.py:287-333): each chunk keeps its allocation's largest
    (noisy, when training with Gumbel) finite scores, ties to the lower key."""

    if scores.ndim != 5:
        raise ValueError(f"scores must have shape [B,L,Hkv,K,S], got {tuple(scores.shape)}")
    if selected_entropy.shape != scores.shape[:-1]:
        raise ValueError(
            f"selected_entropy shape {tuple(selected_entropy.shape)} must "
            f"equal {tuple(scores.shape[:-1])}")
    _check_budget(scores.shape[3], token_budget, min_tokens_per_chunk)
    if scores.device.type != "cuda":
        raise ValueError("select_entropy_adaptive_token_keep requires a CUDA tensor")
    ranking = _scores_with_gumbel(
        scores, training=training, use_gumbel=use_gumbel, gumbel_scale=gumbel_scale)
    return torch.ops.mrsa.token_keep_entropy(ranking, selected_entropy, None, None,
                                             int(token_budget), int(min_tokens_per_chunk),
                                             _dtype == torch.int8)


def refine_remote_tokens_entropy_g7(
    q: torch.Tensor,
    k: torch.Tensor,
    indices: torch.Tensor,
    key_valid: torch.Tensor,
    entropy: torch.Tensor,
    chunk_size: int,
    token_budget: int,
    min_tokens_per_chunk: int = 1,
    *,
    training: bool = True,
    use_gumbel: bool = False,
    gumbel_scale: float = 1.0,
    kv_frags: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """(int8 keep mask [B, Lq, Hkv, K, chunk_size], int64 allocation
    [B, Lq, Hkv, K]) of the entropy-adaptive policy (token_refinement.py:396-438):
    candidate scores, then per-chunk quotas from the routed chunks' entropy
    [B, C, Hkv, G] gathered inside the keep kernel."""

    if q.shape[2] != k.shape[2] * 7:
        raise ValueError("Dream token refinement requires seven query heads per KV head")
    if entropy.ndim != 4 or indices.ndim != 4:
        raise ValueError("expected entropy [B,C,Hkv,G] and indices [B,L,Hkv,K]")
    _check_budget(indices.shape[-1], token_budget, min_tokens_per_chunk)
    with torch.no_grad():
        scores = candidate_token_scores_gqa(
            q.detach().contiguous(),
            k.detach().contiguous(),
            indices.to(torch.int32).contiguous(),
            key_valid.contiguous(),
            chunk_size,
            kv_frags=kv_frags,
        )
        ranking = _scores_with_gumbel(
            scores, training=training, use_gumbel=use_gumbel, gumbel_scale=gumbel_scale)
        return torch.ops.mrsa.token_keep_entropy(ranking, None, entropy.detach(), indices,
                                                 int(token_budget), int(min_tokens_per_chunk),
                                                 True)
