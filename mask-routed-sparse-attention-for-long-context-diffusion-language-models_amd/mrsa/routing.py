"""Dream G=7 routing adapters.

Drop-ins for dream_dllm_hils/routing.py: ``route_topk_g7`` (:52-302),
``selected_attention_g7`` (:305-328) and ``selected_attention_g7_cached``
(:331-353).  The gfx950 kernels take the logical G=7 head layout directly,
so the physical-G=8 padding of the reference is not needed.
"""

from __future__ import annotations

import torch

from .sparse_attention import (kv_fragments, kv_fragments_cached, selected_attention_autograd,
                               selected_attention_launch)
from .topk import route_topk_launch

_LOGICAL_G = 7


def route_topk_g7(
    q: torch.Tensor,
    lmks: torch.Tensor,
    local_lse: torch.Tensor,
    prior_bias: torch.Tensor,
    drop_mask: torch.Tensor,
    topk: int,
    chunk_size: int,
    window: int,
    *,
    training: bool = True,
    use_gumbel: bool = False,
    gumbel_scale: float = 1.0,
    return_selected_gumbel: bool = False,
    selection_mode: str = "post_softmax",
):
    """Route logical G=7 query heads; same validation and outputs as the reference.

    Returns (indices [B, L, Hkv, topk], scores [B, L, Hq, topk] bf16), plus the
    selected Gumbel noise [B, L, Hq, topk] (or None) with
    return_selected_gumbel.  As in the reference, inference (training=False)
    indices are int64 and training indices int32; in training with
    use_gumbel the per-(head, chunk) noise joins the prior bias in the
    selection and the route LSE (routing.py:96-131, :232-302).
    """

    if q.ndim != 4 or lmks.ndim != 5:
        raise ValueError(
            f"expected q [B,L,Hq,D] and lmks [B,C,Hkv,7,D], got "
            f"{tuple(q.shape)} and {tuple(lmks.shape)}"
        )
    batch, seq_len, h_q, dim = q.shape
    if lmks.shape[0] != batch or lmks.shape[3:] != (_LOGICAL_G, dim):
        raise ValueError(f"invalid landmark shape {tuple(lmks.shape)} for q {tuple(q.shape)}")
    chunks, h_kv = lmks.shape[1:3]
    if h_q != h_kv * _LOGICAL_G:
        raise ValueError(f"expected {h_kv * _LOGICAL_G} query heads, got {h_q}")
    if local_lse.shape != (batch, seq_len, h_kv, _LOGICAL_G):
        raise ValueError(f"invalid local_lse shape {tuple(local_lse.shape)}")
    if prior_bias.shape != (batch, chunks, h_kv, _LOGICAL_G):
        raise ValueError(f"invalid prior_bias shape {tuple(prior_bias.shape)}")
    if drop_mask.shape != (batch, seq_len, chunks):
        raise ValueError(f"invalid drop_mask shape {tuple(drop_mask.shape)}")
    if topk <= 0:
        raise ValueError(f"topk must be positive, got {topk}")
    if gumbel_scale < 0:
        raise ValueError(f"gumbel_scale must be non-negative, got {gumbel_scale}")
    if selection_mode not in {"post_softmax", "pre_softmax"}:
        raise ValueError(f"unsupported selection_mode={selection_mode}")
    bias = prior_bias
    noise = None
    if bool(use_gumbel) and bool(training) and gumbel_scale > 0:
        # routing.py:98-103 / :232-245: uniform(eps, 1 - eps) -> -log(-log(u))
        # * gumbel_scale per (head, chunk), drawn in the reference's shapes
        # (pre-softmax: [1, 1, h_q, C]; post-softmax: the physical G=8 heads
        # and max(C, topk) chunks, of which the logical heads and the first C
        # chunks are used), so the same generator state gives the same noise.
        eps = torch.finfo(torch.float32).eps
        if selection_mode == "pre_softmax":
            uniform = torch.empty(1, 1, h_q, chunks, device=q.device,
                                  dtype=torch.float32).uniform_(eps, 1.0 - eps)
            noise = (-torch.log(-torch.log(uniform)) * float(gumbel_scale)).reshape(
                h_kv, _LOGICAL_G, chunks)
        else:
            uniform = torch.empty(1, 1, h_kv * 8, max(chunks, topk), device=q.device,
                                  dtype=torch.float32).uniform_(eps, 1.0 - eps)
            noise = (-torch.log(-torch.log(uniform)) * float(gumbel_scale)).reshape(
                h_kv, 8, -1)[:, :_LOGICAL_G, :chunks]
        bias = (prior_bias.float() + noise.permute(2, 0, 1)[None]).contiguous()

    indices, scores = route_topk_launch(
        q.reshape(batch, seq_len, h_kv, _LOGICAL_G, dim),
        lmks.reshape(batch, chunks, h_q, dim),
        local_lse,
        topk,
        chunk_size,
        bias4=bias,
        drop_mask=drop_mask,
        selection_mode=selection_mode,
    )
    scores = scores.reshape(batch, seq_len, h_q, topk).to(q.dtype)
    if not training:
        indices = indices.to(torch.int64)
    if not return_selected_gumbel:
        return indices, scores
    selected = None
    if noise is not None:
        # the noise of each head at its routed chunks, 0 at -1 slots
        idx = indices.long()
        safe = idx.clamp(0, chunks - 1)
        nz = noise.reshape(1, 1, h_kv, _LOGICAL_G, chunks).expand(batch, seq_len, -1, -1, -1)
        selected = torch.gather(nz, -1, safe[:, :, :, None, :].expand(-1, -1, -1, _LOGICAL_G, -1))
        selected = selected.masked_fill((idx < 0)[:, :, :, None, :], 0.0)
        selected = selected.reshape(batch, seq_len, h_q, topk)
    return indices, scores, selected


def _validate_selected(q, k, v, weights, indices, key_valid, chunk_size, token_keep):
    # dream_dllm_hils/routing.py:368-425
    if q.ndim != 4 or k.ndim != 4:
        raise ValueError(
            f"q and k must be BLHD tensors, got {tuple(q.shape)} and {tuple(k.shape)}"
        )
    batch, query_len, h_q, dim = q.shape
    if k.shape[0] != batch or k.shape[-1] != dim:
        raise ValueError(f"incompatible q/k shapes {tuple(q.shape)} and {tuple(k.shape)}")
    kv_len, h_kv = k.shape[1:3]
    if h_q != h_kv * _LOGICAL_G:
        raise ValueError(f"Dream G7 requires h_q == 7 * h_kv, got h_q={h_q}, h_kv={h_kv}")
    if v.shape != k.shape:
        raise ValueError(f"v shape {tuple(v.shape)} must match k shape {tuple(k.shape)}")
    selected = indices.shape[-1]
    if indices.shape != (batch, query_len, h_kv, selected):
        raise ValueError(f"invalid indices shape {tuple(indices.shape)}")
    if weights.shape != (batch, query_len, h_q, selected):
        raise ValueError(f"invalid weights shape {tuple(weights.shape)}")
    if key_valid.shape != (batch, kv_len):
        raise ValueError(f"invalid key_valid shape {tuple(key_valid.shape)}")
    if token_keep is not None and token_keep.shape != (
        batch, query_len, h_kv, selected, chunk_size
    ):
        raise ValueError(
            "token_keep must have shape "
            f"{(batch, query_len, h_kv, selected, chunk_size)}, got "
            f"{tuple(token_keep.shape)}"
        )
    if kv_len % chunk_size != 0:
        raise ValueError(f"cache length {kv_len} must be divisible by chunk_size={chunk_size}")
    if q.dtype != torch.bfloat16 or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("selected attention requires BF16 q, k, and v")
    if q.device != k.device or v.device != q.device:
        raise ValueError("q, k, and v must share a device")
    if weights.device != q.device or indices.device != q.device:
        raise ValueError("weights and indices must share the q device")
    if key_valid.device != q.device:
        raise ValueError("key_valid must share the q device")
    if token_keep is not None and token_keep.device != q.device:
        raise ValueError("token_keep must share the q device")
    if selected <= 0:
        raise ValueError("selected attention requires at least one chunk slot")


def selected_attention_g7(q, k, v, weights, indices, key_valid, chunk_size, training,
                          token_keep=None):
    """Selected-chunk attention with compact KV (routing.py:305-328), with
    autograd when an input requires grad."""

    _validate_selected(q, k, v, weights, indices, key_valid, chunk_size, token_keep)
    return selected_attention_autograd(q, k, v, weights, indices, key_valid, chunk_size,
                                       mask_last_token=True, token_keep=token_keep)


def selected_attention_g7_cached(q, k, v, weights, indices, key_valid, chunk_size,
                                 token_keep=None):
    """Partial queries against a full compact-GQA cache (routing.py:331-353)."""

    _validate_selected(q, k, v, weights, indices, key_valid, chunk_size, token_keep)
    return selected_attention_launch(
        q, kv_fragments_cached(k, v), weights, indices, key_valid, chunk_size, mask_last_token=True,
        token_keep=token_keep,
    )
