"""``torch.ops.mrsa.*``: the library's kernels as PyTorch custom operators.

Each operator has a schema (Tensor / scalar arguments, fresh output
tensors), a CUDA implementation that launches the gfx950 kernel through the
C ABI (include/mrsa.h) on the current stream, and a fake implementation that
gives output shapes and dtypes without running anything, so ``torch.compile``
(``fullgraph=True``) and ``torch.export`` trace through the ops the way the
reference traces its torch pool twin (ops/chunk_attn_pool_gqa_tilelang.py:40-44).

The Python drop-ins (``chunk_attn_pool_gqa``, ``route_topk_g7``,
``HiLS_block_M_head``, ...) validate their arguments with the reference's
ValueError messages and then call these operators.  There is no CPU
implementation: a CPU tensor reaching an operator raises.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from .fusion import _fuse_bwd_impl, _fuse_impl
from .kernel_utils import _drop_mask_impl, _drop_mask_rows_impl
from .local_attention import _local_attention_impl
from .pool import _kv_fragments_pool_impl, _pool_bwd_impl, _pool_impl
from .route_weights import _route_weights_bwd_impl, _route_weights_impl
from .local_attention import _local_attention_qf_impl
from .sparse_attention import (FRAG_ELEMS, _kv_fragments_impl, _kv_fragments_rows_impl,
                               _q_fragments_impl, _selected_attention_impl,
                               _selected_attention_bwd_impl)
from .token_refinement import _gather_entropy_impl, _token_keep_entropy_impl, _token_keep_impl
from .token_score import _token_scores_impl
from .topk import _route_score_bwd_impl, _route_topk_impl

_CUDA = "cuda"


def _op(name, mutates_args=()):
    return torch.library.custom_op(f"mrsa::{name}", mutates_args=mutates_args,
                                   device_types=_CUDA)


# -- K / V fragments --------------------------------------------------------
@_op("kv_fragments")
def kv_fragments(k: Tensor, v: Optional[Tensor]) -> Tensor:
    return _kv_fragments_impl(k, v)


@kv_fragments.register_fake
def _(k, v):
    B, L, H, _ = k.shape
    return k.new_empty(B, H, (L + 63) // 64, FRAG_ELEMS, dtype=torch.bfloat16)


@_op("kv_fragments_rows_", mutates_args=("kv_frags",))
def kv_fragments_rows_(k: Tensor, v: Tensor, kv_frags: Tensor, positions: Tensor) -> None:
    _kv_fragments_rows_impl(k, v, kv_frags, positions)


@kv_fragments_rows_.register_fake
def _(k, v, kv_frags, positions):
    return None


@_op("q_fragments")
def q_fragments(q: Tensor, kv_heads: int) -> Tensor:
    return _q_fragments_impl(q, kv_heads)


@q_fragments.register_fake
def _(q, kv_heads):
    B, L, _, _ = q.shape
    return q.new_empty(B, kv_heads, L, 1024, dtype=torch.bfloat16)


# -- window attention -----------------------------------------------------
@_op("local_attention")
def local_attention(q: Tensor, kv_frags: Tensor, key_valid: Optional[Tensor], kv_len: int,
                    flash_window: int, inert_chunk: int, query_positions: Optional[Tensor],
                    sm_scale: float, parts: int) -> tuple[Tensor, Tensor]:
    return _local_attention_impl(q, kv_frags, key_valid, kv_len, flash_window, inert_chunk,
                                 query_positions, sm_scale, parts)


@local_attention.register_fake
def _(q, kv_frags, key_valid, kv_len, flash_window, inert_chunk, query_positions, sm_scale,
      parts):
    B, Lq, Hq, D = q.shape
    return (q.new_empty(B, Lq, Hq, D, dtype=torch.bfloat16),
            q.new_empty(B, Lq, Hq, dtype=torch.float32))


@_op("local_attention_qf")
def local_attention_qf(q: Tensor, kv_frags: Tensor, key_valid: Optional[Tensor], kv_len: int,
                       flash_window: int, inert_chunk: int, sm_scale: float
                       ) -> tuple[Tensor, Tensor, Tensor]:
    return _local_attention_qf_impl(q, kv_frags, key_valid, kv_len, flash_window, inert_chunk,
                                    sm_scale)


@local_attention_qf.register_fake
def _(q, kv_frags, key_valid, kv_len, flash_window, inert_chunk, sm_scale):
    B, Lq, Hq, D = q.shape
    Hkv = kv_frags.shape[1]
    return (q.new_empty(B, Lq, Hq, D, dtype=torch.bfloat16),
            q.new_empty(B, Lq, Hq, dtype=torch.float32),
            q.new_empty(B, Hkv, Lq, 1024, dtype=torch.bfloat16))


# -- landmark pool --------------------------------------------------------
@_op("chunk_attn_pool")
def chunk_attn_pool(mu_q: Tensor, k_chunked: Tensor, key_valid: Tensor, sm_scale: float,
                    bias_scale: Optional[Tensor]) -> tuple[Tensor, Tensor, Tensor]:
    return _pool_impl(mu_q, k_chunked, key_valid, sm_scale, bias_scale)


@chunk_attn_pool.register_fake
def _(mu_q, k_chunked, key_valid, sm_scale, bias_scale):
    B, C, H, G, _ = mu_q.shape
    entropy = mu_q.new_empty(B, C, H, G, dtype=torch.float32)
    prior = (entropy.new_empty(B, C, H, G) if bias_scale is not None
             else entropy.new_empty(0))
    return mu_q.new_empty(mu_q.shape, dtype=torch.bfloat16), entropy, prior


@_op("kv_fragments_pool")
def kv_fragments_pool(k: Tensor, v: Tensor, mu_q: Tensor, key_valid: Tensor, sm_scale: float,
                      bias_scale: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    return _kv_fragments_pool_impl(k, v, mu_q, key_valid, sm_scale, bias_scale)


@kv_fragments_pool.register_fake
def _(k, v, mu_q, key_valid, sm_scale, bias_scale):
    B, L, H, _ = k.shape
    _, C, _, G, _ = mu_q.shape
    entropy = mu_q.new_empty(B, C, H, G, dtype=torch.float32)
    return (k.new_empty(B, H, (L + 63) // 64, FRAG_ELEMS, dtype=torch.bfloat16),
            mu_q.new_empty(mu_q.shape, dtype=torch.bfloat16), entropy,
            entropy.new_empty(B, C, H, G))


@_op("chunk_attn_pool_bwd")
def chunk_attn_pool_bwd(mu_q: Tensor, k_chunked: Tensor, key_valid: Tensor,
                        grad_landmark: Optional[Tensor], grad_entropy: Optional[Tensor],
                        sm_scale: float) -> tuple[Tensor, Tensor]:
    return _pool_bwd_impl(mu_q, k_chunked, key_valid, grad_landmark, grad_entropy, sm_scale)


@chunk_attn_pool_bwd.register_fake
def _(mu_q, k_chunked, key_valid, grad_landmark, grad_entropy, sm_scale):
    return (torch.empty_like(mu_q, memory_format=torch.contiguous_format),
            torch.empty_like(k_chunked, memory_format=torch.contiguous_format))


# -- route score + top-k --------------------------------------------------
@_op("route_topk")
def route_topk(q5: Tensor, lmks: Tensor, lse4: Optional[Tensor], bias4: Optional[Tensor],
               drop_mask: Optional[Tensor], key_valid: Optional[Tensor], topk: int,
               block_size: int, derive_window: int, is_causal: bool, window_size: int,
               q_offset: int, pre_softmax: bool, sm_scale: float, scores_fp32: bool,
               use_workspace: int) -> tuple[Tensor, Tensor]:
    return _route_topk_impl(q5, lmks, lse4, bias4, drop_mask, key_valid, topk, block_size,
                            derive_window, is_causal, window_size, q_offset, pre_softmax,
                            sm_scale, scores_fp32, use_workspace)


@route_topk.register_fake
def _(q5, lmks, lse4, bias4, drop_mask, key_valid, topk, block_size, derive_window, is_causal,
      window_size, q_offset, pre_softmax, sm_scale, scores_fp32, use_workspace):
    B, L, H, G, _ = q5.shape
    return (q5.new_empty(B, L, H, topk, dtype=torch.int32),
            q5.new_empty(B, L, H, G, topk,
                         dtype=torch.float32 if scores_fp32 else torch.bfloat16))


@_op("route_score_bwd")
def route_score_bwd(q5: Tensor, lmks: Tensor, indices: Tensor, grad_scores: Tensor,
                    sm_scale: float) -> tuple[Tensor, Tensor]:
    return _route_score_bwd_impl(q5, lmks, indices, grad_scores, sm_scale)


@route_score_bwd.register_fake
def _(q5, lmks, indices, grad_scores, sm_scale):
    return (q5.new_empty(q5.shape, dtype=torch.bfloat16),
            lmks.new_empty(lmks.shape, dtype=torch.bfloat16))


# -- route weights --------------------------------------------------------
@_op("route_weights")
def route_weights(scores: Tensor, indices: Tensor, prior_bias: Tensor, local_lse: Tensor,
                  temperature: float, gate_offset: Optional[Tensor],
                  gate_scale: Optional[Tensor], return_gate_logit: bool,
                  value_bonus: Optional[Tensor] = None,
                  selected_gumbel: Optional[Tensor] = None) -> tuple[Tensor, Tensor, Tensor]:
    return _route_weights_impl(scores, indices, prior_bias, local_lse, temperature, gate_offset,
                               gate_scale, return_gate_logit, value_bonus, selected_gumbel)


@route_weights.register_fake
def _(scores, indices, prior_bias, local_lse, temperature, gate_offset, gate_scale,
      return_gate_logit, value_bonus=None, selected_gumbel=None):
    B, L, Hq, K = scores.shape
    return (scores.new_empty(B, L, Hq, K, dtype=torch.bfloat16),
            scores.new_empty(B, L, Hq, dtype=torch.bfloat16),
            scores.new_empty(B, L, Hq if return_gate_logit else 0, dtype=torch.float32))


@_op("route_weights_bwd")
def route_weights_bwd(scores: Tensor, indices: Tensor, prior_bias: Tensor, local_lse: Tensor,
                      grad_remote: Optional[Tensor], grad_local: Optional[Tensor],
                      grad_gate_logit: Optional[Tensor], temperature: float,
                      gate_offset: Optional[Tensor], gate_scale: Optional[Tensor],
                      value_bonus: Optional[Tensor] = None,
                      selected_gumbel: Optional[Tensor] = None,
                      ) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    return _route_weights_bwd_impl(scores, indices, prior_bias, local_lse, grad_remote,
                                   grad_local, grad_gate_logit, temperature, gate_offset,
                                   gate_scale, value_bonus, selected_gumbel)


@route_weights_bwd.register_fake
def _(scores, indices, prior_bias, local_lse, grad_remote, grad_local, grad_gate_logit,
      temperature, gate_offset, gate_scale, value_bonus=None, selected_gumbel=None):
    B, L, Hq, K = scores.shape
    return (scores.new_empty(B, L, Hq, K, dtype=torch.float32),
            prior_bias.new_empty(prior_bias.shape, dtype=torch.float32),
            scores.new_empty(B, L, Hq, dtype=torch.float32),
            scores.new_empty(2, dtype=torch.float32))


# -- routed chunk attention -----------------------------------------------
@_op("selected_attention")
def selected_attention(q: Tensor, kv_frags: Tensor, weights: Tensor, indices: Tensor,
                       key_valid: Optional[Tensor], chunk_size: int, mask_last_token: bool,
                       sm_scale: float, parts: int, token_keep: Optional[Tensor],
                       fuse_local: Optional[Tensor], fuse_weight: Optional[Tensor],
                       q_frags: Optional[Tensor] = None, deterministic: bool = False) -> Tensor:
    return _selected_attention_impl(q, kv_frags, weights, indices, key_valid, chunk_size,
                                    mask_last_token, sm_scale, parts, token_keep, fuse_local,
                                    fuse_weight, q_frags, deterministic)


@selected_attention.register_fake
def _(q, kv_frags, weights, indices, key_valid, chunk_size, mask_last_token, sm_scale, parts,
      token_keep, fuse_local, fuse_weight, q_frags=None, deterministic=False):
    return q.new_empty(q.shape, dtype=torch.bfloat16)


# -- output fusion --------------------------------------------------------
@_op("fuse_hils_outputs")
def fuse_hils_outputs(remote_output: Tensor, local_output: Tensor,
                      local_weight: Tensor) -> Tensor:
    return _fuse_impl(remote_output, local_output, local_weight)


@fuse_hils_outputs.register_fake
def _(remote_output, local_output, local_weight):
    return torch.empty_like(remote_output)


@_op("selected_attention_bwd")
def selected_attention_bwd(q: Tensor, kv_frags: Tensor, kv_frags_bwd: Tensor, weights: Tensor,
                           indices: Tensor, key_valid: Optional[Tensor], grad_output: Tensor,
                           chunk_size: int, mask_last_token: bool, sm_scale: float,
                           token_keep: Optional[Tensor], kv_len: int
                           ) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    return _selected_attention_bwd_impl(q, kv_frags, kv_frags_bwd, weights, indices, key_valid,
                                        grad_output, chunk_size, mask_last_token, sm_scale,
                                        token_keep, kv_len)


@selected_attention_bwd.register_fake
def _(q, kv_frags, kv_frags_bwd, weights, indices, key_valid, grad_output, chunk_size,
      mask_last_token, sm_scale, token_keep, kv_len):
    B, Lq, Hq, D = q.shape
    Hkv = kv_frags.shape[1]
    return (q.new_empty(B, Lq, Hq, D, dtype=torch.float32),
            q.new_empty(B, kv_len, Hkv, D, dtype=torch.float32),
            q.new_empty(B, kv_len, Hkv, D, dtype=torch.float32),
            q.new_empty(B, Lq, Hq, indices.shape[-1], dtype=torch.bfloat16))


@_op("fuse_hils_outputs_bwd")
def fuse_hils_outputs_bwd(local_output: Tensor, local_weight: Tensor,
                          grad_output: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    return _fuse_bwd_impl(local_output, local_weight, grad_output)


@fuse_hils_outputs_bwd.register_fake
def _(local_output, local_weight, grad_output):
    return (torch.empty_like(local_output), torch.empty_like(local_output),
            torch.empty_like(local_weight))


# -- drop mask ------------------------------------------------------------
@_op("remote_drop_mask")
def remote_drop_mask(valid_mask: Tensor, allowed_mask: Optional[Tensor], window: int,
                     chunk_size: int) -> Tensor:
    return _drop_mask_impl(valid_mask, allowed_mask, window, chunk_size)


@remote_drop_mask.register_fake
def _(valid_mask, allowed_mask, window, chunk_size):
    B, L = valid_mask.shape
    return valid_mask.new_empty(B, L, L // chunk_size, dtype=torch.int32)


@_op("remote_drop_mask_rows")
def remote_drop_mask_rows(valid_mask: Tensor, query_positions: Tensor, window: int,
                          chunk_size: int) -> Tensor:
    return _drop_mask_rows_impl(valid_mask, query_positions, window, chunk_size)


@remote_drop_mask_rows.register_fake
def _(valid_mask, query_positions, window, chunk_size):
    B, L = valid_mask.shape
    return valid_mask.new_empty(B, query_positions.shape[0], L // chunk_size, dtype=torch.int32)


# -- remote-token refinement ----------------------------------------------
@_op("candidate_token_scores")
def candidate_token_scores(q: Tensor, kv_frags: Tensor, indices: Tensor, key_valid: Tensor,
                           chunk_size: int) -> Tensor:
    return _token_scores_impl(q, kv_frags, indices, key_valid, chunk_size)


@candidate_token_scores.register_fake
def _(q, kv_frags, indices, key_valid, chunk_size):
    B, Lq, Hkv, K = indices.shape
    return q.new_empty(B, Lq, Hkv, K, chunk_size, dtype=torch.float32)


@_op("token_keep")
def token_keep(ranking: Tensor, token_budget: int, as_int8: bool) -> Tensor:
    return _token_keep_impl(ranking, token_budget, as_int8)


@token_keep.register_fake
def _(ranking, token_budget, as_int8):
    return ranking.new_empty(ranking.shape, dtype=torch.int8 if as_int8 else torch.uint8)



@_op("token_keep_entropy")
def token_keep_entropy(ranking: Tensor, selected_entropy: Optional[Tensor], entropy: Optional[Tensor],
                       indices: Optional[Tensor], token_budget: int, min_tokens_per_chunk: int,
                       as_int8: bool) -> tuple[Tensor, Tensor]:
    return _token_keep_entropy_impl(ranking, selected_entropy, entropy, indices, token_budget,
                                    min_tokens_per_chunk, as_int8)


@token_keep_entropy.register_fake
def _(ranking, selected_entropy, entropy, indices, token_budget, min_tokens_per_chunk, as_int8):
    B, L, H, K, S = ranking.shape
    return (ranking.new_empty(ranking.shape, dtype=torch.int8 if as_int8 else torch.uint8),
            ranking.new_empty(B, L, H, K, dtype=torch.int64))


@_op("gather_selected_chunk_entropy")
def gather_selected_chunk_entropy(entropy: Tensor, indices: Tensor) -> Tensor:
    return _gather_entropy_impl(entropy, indices)


@gather_selected_chunk_entropy.register_fake
def _(entropy, indices):
    B, L, H, K = indices.shape
    return entropy.new_empty(B, L, H, K, dtype=torch.float32)

OPERATORS = (
    "kv_fragments", "kv_fragments_rows_", "q_fragments", "local_attention",
    "local_attention_qf", "chunk_attn_pool", "kv_fragments_pool",
    "chunk_attn_pool_bwd", "route_topk", "route_score_bwd", "route_weights", "route_weights_bwd",
    "selected_attention", "selected_attention_bwd", "fuse_hils_outputs", "fuse_hils_outputs_bwd",
    "remote_drop_mask",
    "remote_drop_mask_rows", "candidate_token_scores", "token_keep", "token_keep_entropy",
    "gather_selected_chunk_entropy",
)
