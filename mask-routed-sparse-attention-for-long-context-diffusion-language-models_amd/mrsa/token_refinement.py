"""Remote-token refinement ("global_qk" policy).

Drop-ins for ``select_global_token_keep`` and ``refine_remote_tokens_g7``
(dream_dllm_hils/token_refinement.py:112-148, :359-392): candidate token
scores inside the routed chunks (``candidate_token_scores_gqa``), then the
global top-``token_budget`` keep mask per (query, KV head) from the gfx950
token-keep kernel (mrsa_token_keep_fwd).  The routed attention consumes the
mask through ``token_keep``.
"""

from __future__ import annotations

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
