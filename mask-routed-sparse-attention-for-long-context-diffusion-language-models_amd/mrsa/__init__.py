"""MI355X (gfx950) mask-routed sparse attention.

Forward-path drop-ins for the MRSA reference's attention ops, backed by the
hand-written HIP kernels in ../csrc (C ABI: include/mrsa.h).  Module map:

    pool.py             chunk_attn_pool_gqa             (ops/chunk_attn_pool_gqa_tilelang.py)
    topk.py             ref_softmax_topk_max_pooling,
                        online_softmax_topk_head        (ops/topk_head_softmax.py)
    routing.py          route_topk_g7, selected_attention_g7[_cached]
                                                        (dream_dllm_hils/routing.py)
    sparse_attention.py HiLS_block_M_head, kv_fragments   (ops/hils_fwd_bwd_head.py)
    local_attention.py  bidir_local_attention, cached_local_attention
                                                        (dream_dllm_hils/local_attention.py)
    route_weights.py    route_weights, route_weights_torch
                        (ops/hils_bidir_route_weights_tilelang.py, attention.py:126-235)
    fusion.py           fuse_hils_outputs               (ops/hils_bidir_output_fusion_tilelang.py)
    token_score.py      candidate_token_scores_gqa      (ops/hils_token_score_gqa_tilelang.py)
    token_refinement.py global_qk / entropy_adaptive token keep
                                                        (dream_dllm_hils/token_refinement.py)
    kernel_utils.py     remote_drop_mask(_rows), chunk_aligned_local_bounds, group_pad_to/unpad
    route_layer.py      route_attention, swa_attention  (attention.py route / SWA layers),
                        cached_route_attention + LayerKVCache (fastdllm_attention.py cached step)
    ops.py              torch.ops.mrsa.* custom operators (schemas, CUDA and fake kernels)
"""

from .fusion import fuse_hils_outputs
from .kernel_utils import (
    chunk_aligned_local_bounds,
    group_pad_to,
    group_unpad,
    remote_drop_mask,
    remote_drop_mask_rows,
)
from .local_attention import bidir_local_attention, cached_local_attention
from .pool import (chunk_attn_pool_gqa, chunk_attn_pool_gqa_backward, chunk_attn_pool_gqa_prior,
                   kv_fragments_pool)
from .route_layer import (
    CachedBlockStep,
    LayerKVCache,
    RouteLayerConfig,
    cached_route_attention,
    route_attention,
    swa_attention,
)
from .route_weights import route_weights, route_weights_torch
from .routing import route_topk_g7, selected_attention_g7, selected_attention_g7_cached
from .sparse_attention import (HiLS_block_M_head, RoutedLockTimeout, check_routed_locks,
                               kv_fragments, q_fragments, routed_lock_giveups,
                               set_routed_lock_spin_limit)
from .token_score import candidate_token_scores_gqa
from .token_refinement import (
    allocate_entropy_token_budget,
    gather_selected_chunk_entropy,
    refine_remote_tokens_entropy_g7,
    refine_remote_tokens_g7,
    select_entropy_adaptive_token_keep,
    select_global_token_keep,
)
from .topk import online_softmax_topk_head, ref_softmax_topk_max_pooling
from ._lib import LIB_PATH, MrsaLibraryError, load as load_library
from . import ops  # registers torch.ops.mrsa.* (after every module it wraps)

__all__ = [
    "HiLS_block_M_head",
    "LIB_PATH",
    "MrsaLibraryError",
    "CachedBlockStep",
    "LayerKVCache",
    "RouteLayerConfig",
    "cached_route_attention",
    "bidir_local_attention",
    "cached_local_attention",
    "candidate_token_scores_gqa",
    "refine_remote_tokens_g7",
    "select_global_token_keep",
    "allocate_entropy_token_budget",
    "gather_selected_chunk_entropy",
    "refine_remote_tokens_entropy_g7",
    "select_entropy_adaptive_token_keep",
    "chunk_aligned_local_bounds",
    "chunk_attn_pool_gqa",
    "chunk_attn_pool_gqa_backward",
    "chunk_attn_pool_gqa_prior",
    "fuse_hils_outputs",
    "group_pad_to",
    "group_unpad",
    "load_library",
    "online_softmax_topk_head",
    "ref_softmax_topk_max_pooling",
    "remote_drop_mask",
    "remote_drop_mask_rows",
    "route_attention",
    "route_topk_g7",
    "route_weights",
    "route_weights_torch",
    "selected_attention_g7",
    "selected_attention_g7_cached",
    "swa_attention",
    "kv_fragments",
    "q_fragments",
    "kv_fragments_pool",
    "RoutedLockTimeout",
    "check_routed_locks",
    "routed_lock_giveups",
    "set_routed_lock_spin_limit",
]
