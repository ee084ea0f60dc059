"""The MRSA route-layer and SWA-layer attention cores on gfx950.

``route_attention`` is the part of ``KernelDreamFullHiLSAttention.forward``
(dream_dllm_hils/attention.py:1380-1774) between the q/k/v projections and
o_proj, for the inference configuration the layer ships with (no Gumbel, no
token budget, fusion weights from the affine gate at topk >= 32):

    local branch   bidir_local_attention(window W + S - 1, landmark K/V zeroed)
    landmarks      chunk_attn_pool_gqa on the routing query at each landmark slot
    prior          entropy * entropy_bias_scale
    routing        route_topk_g7 with remote_drop_mask(key_valid, W, S)
    weights        _route_weights_torch (layer temperature, affine fusion gate) at
                   topk >= 32; the plain route_weights (temperature 1, no
                   gate) below that (attention.py:1571-1578, :1643-1648)
    remote branch  selected_attention_g7
    output         fuse_hils_outputs(remote, local, local_weight), folded into
                   the routed-attention epilogue (same bits)

``swa_attention`` is ``KernelDreamSlidingWindowAttention.forward``
(attention.py:1168-1220) between projections and o_proj.

``cached_route_attention`` is the Fast-dLLM cached block step of a route layer
(``cached_attention_forward``, fastdllm_attention.py:203-382) after the
projections and the K/V cache update: a block of query rows against the
layer's cache, with the landmark summaries of the affected chunks refreshed
in place.

Everything runs on the library's kernels on the current stream; the drop mask
is derived inside the route kernel instead of being materialised, and V is
re-laid out once for both attention kernels.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import _lib
from .kernel_utils import drop_mask_rows_launch
from .local_attention import (key_parts, local_attention_autograd, local_attention_launch,
                              local_attention_qf_launch)
from .pool import _needs_grad, chunk_attn_pool_gqa_prior, kv_fragments_pool
from .route_weights import route_weights_launch
from .sparse_attention import (FRAG_ELEMS, kv_fragments, kv_fragments_cached, kv_fragments_rows,
                               selected_attention_launch)
from .token_refinement import refine_remote_tokens_entropy_g7, refine_remote_tokens_g7
from .topk import route_topk_launch


@dataclass
class RouteLayerConfig:
    """Route-layer hyper-parameters (canonical values of
    configs/from_dense16k/hils-s2-qcal-rmsnorm-rand-s1000-jingneng.json)."""

    local_window: int = 256
    chunk_size: int = 64
    topk: int = 32
    temperature: float = 1.0
    # fusion_gate_offset / fusion_gate_scale (attention.py:913-914): numbers,
    # or the layer's one-element parameter tensors (read on the device)
    gate_offset: float | torch.Tensor | None = 0.0
    gate_scale: float | torch.Tensor | None = 1.0
    skip_inert_slots: bool = True     # attention.py:902
    # Remote-token refinement (attention.py:1729-1759): with token_budget > 0
    # each (query, KV head) keeps only its budget of routed tokens -- the
    # highest-scoring ones overall ("global_qk") or per chunk under quotas
    # from the chunks' pool entropy ("entropy_adaptive", at least
    # min_tokens_per_chunk per non-empty chunk).
    token_budget: int = 0
    token_policy: str = "global_qk"
    min_tokens_per_chunk: int = 1
    # Routed attention adds each output row's chunk terms in ascending chunk
    # order (the same bits on every launch, eager or graph-captured) instead
    # of in the order the waves reach the row.  None: on for the cached block
    # step (where it costs nothing measurable), off for the full-sequence
    # layer (where the waves then wait for each other's rows: ~1.6x the
    # routed kernel's time at configuration 2).
    deterministic: bool | None = None


def _check_qkv(q, k, v, route_q):
    if q.device.type != "cuda":
        raise ValueError("route attention requires CUDA tensors")
    for name, t in (("q", q), ("k", k), ("v", v), ("route_q", route_q)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be bf16")
        if t.ndim != 4:
            raise ValueError(f"{name} must be [B, L, H, D]")
    if route_q.shape != q.shape:
        raise ValueError("route_q must have the shape of q")
    if k.shape != v.shape or k.shape[:2] != q.shape[:2] or k.shape[-1] != q.shape[-1]:
        raise ValueError(f"incompatible q/k/v shapes {q.shape}, {k.shape}, {v.shape}")
    if q.shape[2] % k.shape[2]:
        raise ValueError("query heads must be a multiple of KV heads")


def route_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    route_q: torch.Tensor,
    entropy_bias_scale: torch.Tensor,
    key_valid: torch.Tensor | None = None,
    cfg: RouteLayerConfig = RouteLayerConfig(),
    return_intermediates: bool = False,
    mark=None,
):
    """Route-layer attention: q, route_q [B, L, Hq, D], k, v [B, L, Hkv, D] bf16.

    Returns the fused output [B, L, Hq, D] bf16 (and a dict of the stage
    outputs when return_intermediates).  ``mark(stage)``, when given, is
    called after each stage is enqueued (stage timing with stream events).
    """

    def _mark(name):
        if mark is not None:
            mark(name)


    _check_qkv(q, k, v, route_q)
    _check_token_budget(cfg)
    B, L, Hq, D = q.shape
    Hkv = k.shape[2]
    G = Hq // Hkv
    S = cfg.chunk_size
    if L % S:
        raise ValueError(f"sequence length {L} must be divisible by chunk_size={S}")
    C = L // S
    if key_valid is None:
        kv_bool = torch.ones(B, L, dtype=torch.bool, device=q.device)
    else:
        kv_bool = key_valid.to(device=q.device, dtype=torch.bool).contiguous()

    _mark("start")
    q_lmk = route_q[:, S - 1 :: S].reshape(B, C, Hkv, G, D)
    # K/V fragments and the landmark pool in one pass over the keys when the
    # pool takes the fused semantics (G >= 2) and no gradient is asked for
    fused_pool = (S == 64 and D == 128 and 2 <= G <= 16
                  and not _needs_grad(route_q, k, entropy_bias_scale))
    if fused_pool:
        frags, lmk, entropy, prior = kv_fragments_pool(k, v, q_lmk, kv_bool, entropy_bias_scale)
    else:
        frags = kv_fragments(k, v)
    _mark("kv_fragments")
    flash_window = cfg.local_window + S - 1 if cfg.skip_inert_slots else cfg.local_window
    q_frags = None
    if G <= 8 and key_parts(B, L, Hkv, L, flash_window) == 1:
        # the window kernel also writes the routed attention's Q operand
        # images (read as whole cache lines by the routed kernel)
        local_out, local_lse, q_frags = local_attention_qf_launch(
            q, frags, kv_bool, flash_window, S if cfg.skip_inert_slots else 0)
    else:
        local_out, local_lse = local_attention_launch(
            q, frags, kv_bool, flash_window, S if cfg.skip_inert_slots else 0
        )
    _mark("local_attention")
    if not fused_pool:
        k_chunked = k.reshape(B, C, S, Hkv, D)
        lmk, entropy, prior = chunk_attn_pool_gqa_prior(
            q_lmk, k_chunked, kv_bool.reshape(B, C, S), entropy_bias_scale
        )
    _mark("pool")
    indices, scores = route_topk_launch(
        route_q.reshape(B, L, Hkv, G, D),
        lmk.reshape(B, C, Hq, D),
        local_lse.reshape(B, L, Hkv, G),
        cfg.topk,
        S,
        bias4=prior,
        derive_window=cfg.local_window,
        key_valid=kv_bool,
    )
    scores = scores.reshape(B, L, Hq, cfg.topk)
    _mark("route_topk")
    if cfg.topk >= 32:
        # attention.py:1571-1621: _route_weights_torch with the route
        # temperature and the fusion gate parameters
        remote_w, local_w = route_weights_launch(
            scores, indices, prior, local_lse, temperature=cfg.temperature,
            gate_offset=cfg.gate_offset, gate_scale=cfg.gate_scale,
        )
    else:
        # attention.py:1643-1648: route_weights, the plain 33-way softmax
        remote_w, local_w = route_weights_launch(scores, indices, prior, local_lse)
    _mark("route_weights")
    token_keep = None
    if cfg.token_budget > 0:
        token_keep = _token_keep(cfg, q, k, indices, kv_bool, entropy, frags)
        _mark("token_refinement")
    # Routed attention with the output fusion in its epilogue:
    # fuse_hils_outputs(remote, local_out, local_w) without materialising remote.
    out = selected_attention_launch(q, frags, remote_w, indices, kv_bool, S,
                                    token_keep=token_keep, fuse_local=local_out,
                                    fuse_weight=local_w, q_frags=q_frags,
                                    deterministic=bool(cfg.deterministic))
    _mark("selected_attention")
    if not return_intermediates:
        return out
    remote_out = selected_attention_launch(q, frags, remote_w, indices, kv_bool, S,
                                           token_keep=token_keep,
                                           deterministic=bool(cfg.deterministic))
    return out, {
        "local_output": local_out, "local_lse": local_lse, "landmark_keys": lmk,
        "entropy": entropy, "prior_bias": prior, "indices": indices, "scores": scores,
        "remote_weights": remote_w, "local_weight": local_w, "remote_output": remote_out,
        "token_keep": token_keep,
    }


def _check_token_budget(cfg):
    # attention.py:1264-1289
    if cfg.token_budget < 0:
        raise ValueError(f"token_budget must be >= 0, got {cfg.token_budget}")
    if cfg.token_budget > cfg.topk * cfg.chunk_size:
        raise ValueError(
            f"token_budget={cfg.token_budget} exceeds routed capacity "
            f"{cfg.topk * cfg.chunk_size}")
    if cfg.token_policy not in {"global_qk", "entropy_adaptive"}:
        raise ValueError(f"unsupported token_policy={cfg.token_policy}")
    if cfg.min_tokens_per_chunk < 0:
        raise ValueError("min_tokens_per_chunk must be non-negative")
    if cfg.token_budget > 0 and cfg.token_budget < cfg.topk * cfg.min_tokens_per_chunk:
        raise ValueError("token_budget must cover the minimum for every routed chunk")


def _token_keep(cfg, q, k, indices, key_valid, entropy, kv_frags):
    """The token keep mask of cfg.token_policy (attention.py:1729-1759,
    fastdllm_attention.py:330-361), inference mode."""
    if cfg.token_policy == "global_qk":
        return refine_remote_tokens_g7(q, k, indices, key_valid, cfg.chunk_size,
                                       cfg.token_budget, training=False, kv_frags=kv_frags)
    keep, _ = refine_remote_tokens_entropy_g7(
        q, k, indices, key_valid, entropy, cfg.chunk_size, cfg.token_budget,
        cfg.min_tokens_per_chunk, training=False, kv_frags=kv_frags)
    return keep


def swa_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    key_valid: torch.Tensor | None = None,
    window: int = 1280,
    chunk_size: int = 64,
    skip_inert_slots: bool = False,
) -> torch.Tensor:
    """Sliding-window layer attention (radius ``window``); [B, L, Hq, D] bf16."""

    if q.device.type != "cuda" or q.dtype != torch.bfloat16:
        raise ValueError("swa_attention requires CUDA bf16 tensors")
    flash_window = window + chunk_size - 1 if skip_inert_slots else window
    out, _ = local_attention_autograd(q, k, v, key_valid, flash_window,
                                      chunk_size if skip_inert_slots else 0)
    return out


@dataclass
class LayerKVCache:
    """The cache fields a cached route layer reads and refreshes
    (dream_dllm_hils/fastdllm_cache.py:10-161): key, value bf16 [1, L, Hkv, D],
    key_valid bool [1, L], landmark_keys bf16 [1, C, Hkv, G, D] and prior_bias
    fp32 [1, C, Hkv, G] (the last two refreshed in place).

    ``kv_frags`` (the ``kv_fragments`` layout of key and value both attention
    kernels read) is built on first use.  ``replace`` keeps it in step with
    the rows it writes; after writing ``key`` or ``value`` any other way,
    set it to None.
    """

    key: torch.Tensor
    value: torch.Tensor
    key_valid: torch.Tensor
    landmark_keys: torch.Tensor
    prior_bias: torch.Tensor
    kv_frags: torch.Tensor | None = field(default=None, repr=False)

    @property
    def physical_length(self) -> int:
        return int(self.key.shape[1])

    def replace(self, positions: torch.Tensor, key: torch.Tensor, value: torch.Tensor) -> None:
        """Write K/V rows at ``positions`` (fastdllm_cache.py:94-125, same checks
        and errors; the two position checks share one device round trip)."""

        positions = positions.to(device=self.key.device, dtype=torch.long)
        if positions.ndim != 1:
            raise ValueError("cache update positions must be one-dimensional")
        if positions.numel():
            srt = positions.sort().values
            flags = torch.stack([
                (srt[1:] == srt[:-1]).any(),
                ((positions < 0) | (positions >= self.physical_length)).any(),
            ]).tolist()
            if flags[0]:
                raise ValueError("cache update positions must be unique")
            if flags[1]:
                raise ValueError("cache update positions must be in range")
        expected = (self.key.shape[0], positions.numel(), self.key.shape[2], self.key.shape[3])
        if key.shape != expected or value.shape != expected:
            raise ValueError(
                f"replacement K/V shape must be {expected}, got "
                f"{tuple(key.shape)} and {tuple(value.shape)}"
            )
        if key.dtype != self.key.dtype or value.dtype != self.value.dtype:
            raise ValueError("replacement K/V dtype must match the cache")
        if key.device != self.key.device or value.device != self.value.device:
            raise ValueError("replacement K/V device must match the cache")
        _write_rows(self, positions, key, value)

    def __post_init__(self) -> None:
        # fastdllm_cache.py:20-80 (the checks this path depends on)
        if self.key.ndim != 4 or self.value.shape != self.key.shape:
            raise ValueError("key and value must have identical [B,L,Hkv,D] shape")
        if self.key.shape[0] != 1:
            raise ValueError("Fast-dLLM cache currently requires batch size one")
        if self.key_valid.shape != self.key.shape[:2]:
            raise ValueError("key_valid shape must match the cache batch and sequence")
        if self.key_valid.dtype != torch.bool:
            raise ValueError("key_valid must be boolean")
        batch, _, hkv, dim = self.key.shape
        lm = self.landmark_keys.shape
        if self.landmark_keys.ndim != 5 or lm[0] != batch or lm[2] != hkv or lm[4] != dim:
            raise ValueError(f"landmark_keys must have shape [B,C,{hkv},G,D]")
        if self.prior_bias.shape != lm[:-1]:
            raise ValueError(f"prior_bias must have shape {tuple(lm[:-1])}")
        if self.kv_frags is not None and self.kv_frags.shape != (
                batch, hkv, (self.key.shape[1] + 63) // 64, FRAG_ELEMS):
            raise ValueError("kv_frags must be kv_fragments(key, value)")


def _write_rows(cache: LayerKVCache, positions: torch.Tensor, key: torch.Tensor,
                value: torch.Tensor) -> None:
    """The row writes of LayerKVCache.replace (fastdllm_cache.py:126-127) and
    the fragment entries of those rows, as one launch (mrsa_kv_replace_rows)
    for a contiguous bf16 head_dim-128 cache; otherwise index_copy_ followed
    by kv_fragments_rows.  Arguments already checked."""

    c = cache
    if (c.key.device.type == "cuda" and c.key.dtype == torch.bfloat16 and c.key.shape[3] == 128
            and c.key.is_contiguous() and c.value.is_contiguous()):
        B, L, H, D = c.key.shape
        kr, vr, pos = key.contiguous(), value.contiguous(), positions.contiguous()
        st = _lib.call("mrsa_kv_replace_rows", _lib.ptr(kr), _lib.ptr(vr), _lib.ptr(pos),
                       pos.numel(), B, L, H, D, _lib.ptr(c.key), _lib.ptr(c.value),
                       _lib.ptr(c.kv_frags), _lib.stream_of(kr))
        _lib.check(st, "kv_replace_rows")
        return
    c.key.index_copy_(1, positions, key)
    c.value.index_copy_(1, positions, value)
    if c.kv_frags is not None:
        kv_fragments_rows(c.key, c.value, c.kv_frags, positions)


def _refresh_landmarks(route_q, cache, query_positions, affected_chunks, entropy_bias_scale,
                       chunk_size):
    """Landmark keys and prior bias of the affected chunks, refreshed in place
    (fastdllm_attention.py:236-292).  One launch (mrsa_pool_cached_chunks_fwd)
    reads the landmark query rows, the chunks' key rows and valid bytes where
    they lie; other shapes gather the rows and pool them with torch ops
    around chunk_attn_pool_gqa_prior.  Arguments already checked."""

    c = cache
    B, Lq, Hq, D = route_q.shape
    L, Hkv = c.key.shape[1], c.key.shape[2]
    G, S, n = Hq // Hkv, chunk_size, affected_chunks.numel()
    scale = entropy_bias_scale.to(device=route_q.device, dtype=torch.float32).contiguous()
    fused = (S == 64 and D == 128 and G <= 16 and L % 64 == 0 and c.key.is_contiguous()
             and c.landmark_keys.is_contiguous() and c.prior_bias.is_contiguous()
             and c.prior_bias.dtype == torch.float32 and c.key_valid.dtype == torch.bool
             and scale.numel() == Hq and not _needs_grad(route_q, c.key, entropy_bias_scale))
    if fused:
        rq, qp = route_q.contiguous(), query_positions.contiguous()
        ac, kv = affected_chunks.contiguous(), c.key_valid.contiguous()
        st = _lib.call("mrsa_pool_cached_chunks_fwd", _lib.ptr(rq), _lib.ptr(qp), Lq,
                       _lib.ptr(c.key), _lib.ptr(kv), B, L, _lib.ptr(ac), n, Hkv, G, D, S,
                       1.0 / D ** 0.5, _lib.ptr(scale), _lib.ptr(c.landmark_keys),
                       _lib.ptr(c.prior_bias), _lib.stream_of(rq))
        _lib.check(st, "pool_cached_chunks")
        return
    landmark_rows = torch.searchsorted(query_positions, affected_chunks * S + (S - 1))
    q_lmk = route_q.index_select(1, landmark_rows).reshape(1, n, Hkv, G, D)
    chunk_positions = (
        affected_chunks[:, None] * S + torch.arange(S, device=route_q.device)[None, :]
    ).reshape(-1)
    chunk_keys = c.key.index_select(1, chunk_positions).reshape(1, n, S, Hkv, D)
    chunk_valid = c.key_valid.index_select(1, chunk_positions).reshape(1, n, S)
    lmk, _, prior = chunk_attn_pool_gqa_prior(
        q_lmk.contiguous(), chunk_keys.contiguous(), chunk_valid.contiguous(),
        entropy_bias_scale,
    )
    c.landmark_keys.index_copy_(1, affected_chunks, lmk.reshape(1, n, Hkv, G, D))
    c.prior_bias.index_copy_(1, affected_chunks, prior.reshape(1, n, Hkv, G))


def cached_route_attention(
    q: torch.Tensor,
    route_q: torch.Tensor,
    cache: LayerKVCache,
    query_positions: torch.Tensor,
    affected_chunks: torch.Tensor,
    entropy_bias_scale: torch.Tensor,
    cfg: RouteLayerConfig = RouteLayerConfig(),
    return_intermediates: bool = False,
):
    """Route-layer attention of a query block against a K/V cache
    (fastdllm_attention.py:203-382 for KernelDreamFullHiLSAttention):

        local branch   cached_local_attention(cache, query_positions, skip_inert_slots)
        landmarks      chunk_attn_pool_gqa of each affected chunk from route_q at its
                       landmark row; cache.landmark_keys / prior_bias refreshed in place
        routing        route_topk_g7 with remote_drop_mask(key_valid, W, S) rows
        weights        _route_weights_torch(temperature=1.0): the plain 33-way
                       softmax (this path passes no fusion gate, :315-323)
        remote branch  selected_attention_g7_cached
        output         fuse_hils_outputs

    q, route_q: bf16 [1, Lq, Hq, D]; query_positions: sorted unique torch.long
    [Lq]; affected_chunks: torch.long [n] whose landmark positions are query
    positions.  Returns the fused output [1, Lq, Hq, D] bf16.
    """

    _check_cached_args(q, route_q, cache, query_positions, affected_chunks, cfg)
    return _cached_route_body(q, route_q, cache, query_positions, affected_chunks,
                              entropy_bias_scale, cfg, return_intermediates)


def _raise_cached_flags(flags, n, C):
    """The errors of the device-side checks (mrsa_cached_step_checks flags),
    in the order the reference raises them."""
    if flags[0]:
        raise ValueError("query_positions must be sorted and unique")
    if flags[1]:
        raise ValueError("query_positions must be in cache range")
    if n and flags[2]:
        raise ValueError(f"affected_chunks must be in [0, {C})")
    if n and flags[3]:
        raise ValueError("all owned positions must also be query positions")


def _check_cached_args(q, route_q, cache, query_positions, affected_chunks, cfg,
                       device_checks=True, defer=False):
    """cached_route_attention's argument checks; the ones that read device
    values run as one kernel and one round trip (skipped with
    device_checks=False).  With defer=True the kernel is only launched and
    (flags, n, C) is returned for _raise_cached_flags after the caller's own
    launches (None when there is nothing to read)."""

    _check_token_budget(cfg)
    if q.device.type != "cuda":
        raise ValueError("cached route attention requires CUDA tensors")
    for name, t in (("q", q), ("route_q", route_q)):
        if t.dtype != torch.bfloat16 or t.ndim != 4:
            raise ValueError(f"{name} must be bf16 [1, Lq, H, D]")
    if route_q.shape != q.shape:
        raise ValueError("route_q must have the shape of q")
    B, Lq, Hq, D = q.shape
    L, Hkv = cache.key.shape[1], cache.key.shape[2]
    if B != 1 or cache.key.shape[3] != D or Hq % Hkv:
        raise ValueError(f"incompatible q {tuple(q.shape)} and cache {tuple(cache.key.shape)}")
    G = Hq // Hkv
    S = cfg.chunk_size
    if L % S:
        raise ValueError(f"cache length {L} must be divisible by chunk_size={S}")
    C = L // S
    if cache.landmark_keys.shape[1] != C or cache.landmark_keys.shape[3] != G:
        raise ValueError(f"landmark_keys must have shape [1, {C}, {Hkv}, {G}, {D}]")
    if query_positions.shape != (Lq,) or query_positions.dtype != torch.long:
        raise ValueError(f"query_positions must be torch.long of shape {(Lq,)}")
    if query_positions.device != q.device or affected_chunks.device != q.device:
        raise ValueError("query_positions and affected_chunks must be on the device of q")
    if affected_chunks.ndim != 1 or affected_chunks.dtype != torch.long:
        raise ValueError("affected_chunks must be a 1-D torch.long tensor")
    n = affected_chunks.numel()
    if Lq and device_checks:
        # Every argument check that needs device values, in one kernel and
        # one round trip: sorted unique positions in range, affected chunks
        # in range, and each affected chunk's landmark row among the query
        # positions (fastdllm_attention.py:54-66, :84-118).
        qp = query_positions.contiguous()
        ac = affected_chunks.contiguous()
        flags = torch.empty(4, dtype=torch.int32, device=q.device)
        st = _lib.call("mrsa_cached_step_checks", _lib.ptr(qp), Lq, _lib.ptr(ac), n, L, S,
                       _lib.ptr(flags), _lib.stream_of(qp))
        _lib.check(st, "cached step checks")
        if defer:
            return flags, n, C
        _raise_cached_flags(flags.tolist(), n, C)
    elif n:
        raise ValueError("all owned positions must also be query positions")
    return None


def _cached_route_body(q, route_q, cache, query_positions, affected_chunks, entropy_bias_scale,
                       cfg, return_intermediates=False):
    """The cached step's launches, with no host synchronisation (arguments
    already checked); landmark rows located on the device."""

    B, Lq, Hq, D = q.shape
    L, Hkv = cache.key.shape[1], cache.key.shape[2]
    G, S = Hq // Hkv, cfg.chunk_size
    C = L // S
    n = affected_chunks.numel()
    if cache.kv_frags is None:
        cache.kv_frags = kv_fragments(cache.key, cache.value)
    flash_window = cfg.local_window + S - 1 if cfg.skip_inert_slots else cfg.local_window
    local_out, local_lse = local_attention_launch(
        q, cache.kv_frags, cache.key_valid, flash_window, S if cfg.skip_inert_slots else 0,
        query_positions=query_positions,
    )
    if n:
        _refresh_landmarks(route_q, cache, query_positions, affected_chunks, entropy_bias_scale, S)
    drop = drop_mask_rows_launch(cache.key_valid, cfg.local_window, S, query_positions)
    indices, scores = route_topk_launch(
        route_q.reshape(1, Lq, Hkv, G, D),
        cache.landmark_keys.reshape(1, C, Hq, D),
        local_lse.reshape(1, Lq, Hkv, G),
        cfg.topk,
        S,
        bias4=cache.prior_bias,
        drop_mask=drop,
    )
    scores = scores.reshape(1, Lq, Hq, cfg.topk)
    remote_w, local_w = route_weights_launch(
        scores, indices, cache.prior_bias, local_lse, temperature=1.0
    )
    token_keep = None
    if cfg.token_budget > 0:
        # fastdllm_attention.py:330-361; the entropy policy reads the entropy
        # back from the cached prior bias (:345-350)
        entropy = None
        if cfg.token_policy != "global_qk":
            entropy = cache.prior_bias / entropy_bias_scale.to(
                device=q.device, dtype=torch.float32).view(1, 1, Hkv, G)
        token_keep = _token_keep(cfg, q, cache.key, indices, cache.key_valid, entropy,
                                 cache.kv_frags)
    # the fixed accumulation order is the default of the cached step
    det = True if cfg.deterministic is None else bool(cfg.deterministic)
    out = selected_attention_launch(q, cache.kv_frags, remote_w, indices, cache.key_valid, S,
                                    token_keep=token_keep, fuse_local=local_out,
                                    fuse_weight=local_w, deterministic=det)
    if not return_intermediates:
        return out
    remote_out = selected_attention_launch(q, cache.kv_frags, remote_w, indices,
                                           cache.key_valid, S, token_keep=token_keep,
                                           deterministic=det)
    return out, {
        "local_output": local_out, "local_lse": local_lse, "indices": indices,
        "scores": scores, "remote_weights": remote_w, "local_weight": local_w,
        "remote_output": remote_out, "drop_mask": drop, "token_keep": token_keep,
    }


class CachedBlockStep:
    """One route layer's Fast-dLLM cached block step -- the block's K/V rows
    written into the cache (LayerKVCache.replace, fastdllm_cache.py:94-125)
    followed by cached_route_attention (fastdllm_attention.py:203-382) --
    captured once as a HIP graph and replayed for every block.

    A graph is specific to the block length (fixed here) and to the number of
    affected chunks (one graph per count, captured on first use).  Each call
    runs the argument checks of replace and cached_route_attention (one
    device round trip), copies its inputs into the graph's buffers and
    replays.  The returned tensor is the graph's output buffer, overwritten
    by the next call with the same affected-chunk count.
    """

    def __init__(self, cache: LayerKVCache, entropy_bias_scale: torch.Tensor,
                 cfg: RouteLayerConfig = RouteLayerConfig(), block_len: int = 32):
        if cache.key.device.type != "cuda":
            raise ValueError("CachedBlockStep requires a CUDA cache")
        self.cache, self.cfg, self.block_len = cache, cfg, int(block_len)
        dev = cache.key.device
        _, _, hkv, dim = cache.key.shape
        hq = hkv * cache.landmark_keys.shape[3]
        self.scale = entropy_bias_scale.to(device=dev, dtype=torch.float32).contiguous()
        self.q = torch.zeros(1, block_len, hq, dim, dtype=torch.bfloat16, device=dev)
        self.route_q = torch.zeros_like(self.q)
        self.k_rows = torch.zeros(1, block_len, hkv, dim, dtype=cache.key.dtype, device=dev)
        self.v_rows = torch.zeros_like(self.k_rows)
        self.positions = torch.zeros(block_len, dtype=torch.long, device=dev)
        self._graphs = {}  # affected count -> (graph, affected buffer, output)
        if cache.kv_frags is None:
            cache.kv_frags = kv_fragments(cache.key, cache.value)

    def _body(self, affected):
        c = self.cache
        _write_rows(c, self.positions, self.k_rows, self.v_rows)
        return _cached_route_body(self.q, self.route_q, c, self.positions, affected, self.scale,
                                  self.cfg)

    def __call__(self, q, route_q, k_rows, v_rows, query_positions, affected_chunks):
        if q.shape != self.q.shape or route_q.shape != self.q.shape:
            raise ValueError(f"q and route_q must have shape {tuple(self.q.shape)}")
        if k_rows.shape != self.k_rows.shape or v_rows.shape != self.k_rows.shape:
            raise ValueError(
                f"replacement K/V shape must be {tuple(self.k_rows.shape)}, got "
                f"{tuple(k_rows.shape)} and {tuple(v_rows.shape)}")
        if k_rows.dtype != self.k_rows.dtype or v_rows.dtype != self.k_rows.dtype:
            raise ValueError("replacement K/V dtype must match the cache")
        # Sorted unique in-range query positions also make the K/V rows'
        # positions unique and in range (replace's checks).  The device
        # checks run first and are read after the input copies are queued
        # (the copies fill the graph's own buffers only).
        pending = _check_cached_args(q, route_q, self.cache, query_positions, affected_chunks,
                                     self.cfg, defer=True)
        n = affected_chunks.numel()
        entry = self._graphs.get(n)
        # the inputs into the graph's buffers, in one launch
        dst = [self.q, self.route_q, self.k_rows, self.v_rows, self.positions]
        src = [q, route_q, k_rows, v_rows, query_positions]
        if entry is not None:
            dst.append(entry[1])
            src.append(affected_chunks)
        _lib.copy_buffers(dst, [t.contiguous() for t in src])
        if pending is not None:
            flags, nf, C = pending
            _raise_cached_flags(flags.tolist(), nf, C)
        if entry is None:
            affected = affected_chunks.clone()
            # One eager pass first (the step is idempotent: the same rows and
            # landmark refresh are written again by the replay), then capture.
            side = torch.cuda.Stream(device=self.q.device)
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                self._body(affected)
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                out = self._body(affected)
            entry = self._graphs[n] = (graph, affected, out)
        graph, _, out = entry
        graph.replay()
        return out
