"""GPU parity of the Fast-dLLM cached block step of a route layer
(dream_dllm_hils/fastdllm_attention.py:203-382) against the CPU oracle.

Tolerances as in test_gpu_parity.py: outputs within max-abs 2e-2 and mean-abs
2e-3; routing rows identical except near ties; drop rows bit-exact.
"""

import pytest
import torch

import mrsa
from oracle import mrsa_oracle as O
from routing_check import assert_nearly_identical, classify_routing

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _note(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g) * scale


def _planted_kv(L, Hkv, D, seed, sigma=0.3):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(1, L, Hkv, D, generator=g)
    shift = sigma * torch.randn(L // 64, Hkv, D, generator=g)
    k = k + shift.repeat_interleave(64, dim=0)[None]
    v = torch.randn(1, L, Hkv, D, generator=g)
    return k.bfloat16(), v.bfloat16()


def _close(actual, expected, what, max_abs=2e-2, mean_abs=2e-3):
    err = (actual.float().cpu() - expected.float()).abs()
    print(f"{what}: max_abs={err.max():.3e} mean_abs={err.mean():.3e}", flush=True)
    assert float(err.max()) <= max_abs, what
    assert float(err.mean()) <= mean_abs, what


def test_drop_mask_rows_bit_exact():
    _note("drop mask rows")
    L, S, W = 4096, 64, 256
    valid = torch.rand(1, L, generator=torch.Generator().manual_seed(3)) > 0.02
    valid[0, 64 * 7 : 64 * 7 + 63] = False  # an invalid chunk (landmark slot alone is valid)
    pos = torch.tensor([0, 1, 63, 64, 1000, 2047, 2048, 3000, 4095], dtype=torch.long)
    got = mrsa.remote_drop_mask_rows(valid.to(DEV), W, S, pos.to(DEV))
    ref = O.remote_drop_mask(valid, W, S)[:, pos]
    assert torch.equal(got.cpu(), ref)
    with pytest.raises(ValueError):
        mrsa.remote_drop_mask_rows(valid.to(DEV), W, S, torch.tensor([L], device=DEV))


def _cache_inputs(L, Hq, Hkv, D, seed):
    q = _rand((1, L, Hq, D), seed).bfloat16()
    rq = _rand((1, L, Hq, D), seed + 1).bfloat16()
    k, v = _planted_kv(L, Hkv, D, seed + 2)
    return q, rq, k, v


def test_cached_route_attention_vs_oracle():
    _note("cached route layer L=4096 block=chunk 31")
    L, Hq, Hkv, D, S = 4096, 28, 4, 128, 64
    C, G = L // S, Hq // Hkv
    q, rq, k, v = _cache_inputs(L, Hq, Hkv, D, 70)
    valid = torch.ones(1, L, dtype=torch.bool)
    valid[0, 900:905] = False
    scale = torch.rand(Hq, generator=torch.Generator().manual_seed(74)) + 0.5
    g = torch.Generator().manual_seed(75)
    lmk0 = torch.randn(1, C, Hkv, G, D, generator=g).bfloat16()
    prior0 = torch.rand(1, C, Hkv, G, generator=g) * 0.5
    chunk = 31
    rows = torch.arange(chunk * S, (chunk + 1) * S)
    aff = torch.tensor([chunk])
    cache = mrsa.LayerKVCache(k.to(DEV), v.to(DEV), valid.to(DEV), lmk0.clone().to(DEV),
                              prior0.clone().to(DEV))
    out, mid = mrsa.cached_route_attention(
        q[:, rows].to(DEV), rq[:, rows].to(DEV), cache, rows.to(DEV), aff.to(DEV),
        scale.to(DEV), return_intermediates=True)
    ref, rlmk, rprior, rmid = O.cached_route_layer(
        q[:, rows], rq[:, rows], k, v, valid, lmk0, prior0, rows, aff, scale)
    _close(cache.landmark_keys, rlmk, "refreshed landmark keys")
    torch.testing.assert_close(cache.prior_bias.cpu(), rprior, atol=1e-3, rtol=1e-3)
    others = torch.arange(C) != chunk
    assert torch.equal(cache.landmark_keys.cpu()[:, others], lmk0[:, others])
    assert torch.equal(mid["drop_mask"].cpu(), rmid["drop_mask"])
    classify_routing(mid["indices"], rmid["indices"], rq[:, rows], cache.landmark_keys,
                     mid["local_lse"], cache.prior_bias,
                     lambda r: O.remote_drop_mask_rows(valid, 256, S, rows[r]), 32, S,
                     "cached route layer L=4096")
    _close(mid["local_output"], rmid["local_output"], "cached local branch")
    _close(out, ref, "cached route layer")


def test_cached_refresh_matches_prefill():
    # Port of unittests/test_qcal.py:124-157: prefill, change the last chunk's
    # rows, refresh it through the cached step; the output rows and the
    # refreshed landmark match a new prefill of the changed inputs.
    _note("cached refresh vs prefill L=2048")
    L, Hq, Hkv, D, S = 2048, 28, 4, 128, 64
    q, rq, k, v = _cache_inputs(L, Hq, Hkv, D, 80)
    valid = torch.ones(1, L, dtype=torch.bool, device=DEV)
    scale = (torch.rand(Hq, generator=torch.Generator().manual_seed(84)) + 0.5).to(DEV)
    cfg = mrsa.RouteLayerConfig(gate_offset=None, gate_scale=None)  # the decode path's weights
    q, rq, k, v = (t.to(DEV) for t in (q, rq, k, v))
    _, mid = mrsa.route_attention(q, k, v, rq, scale, valid, cfg, return_intermediates=True)
    original_lmk = mid["landmark_keys"].clone()
    rows = torch.arange(L - S, L, device=DEV)
    g = torch.Generator().manual_seed(85)
    bump = lambda t: t.index_add(1, rows, (torch.randn(t[:, rows].shape, generator=g) * 0.1)
                                 .to(DEV, torch.bfloat16))
    q2, rq2, k2, v2 = bump(q), bump(rq), bump(k), bump(v)
    cache = mrsa.LayerKVCache(k2.clone(), v2.clone(), valid.clone(),
                              mid["landmark_keys"].clone(), mid["prior_bias"].clone())
    actual = mrsa.cached_route_attention(q2[:, rows], rq2[:, rows], cache, rows,
                                         torch.tensor([L // S - 1], device=DEV), scale, cfg)
    expected, emid = mrsa.route_attention(q2, k2, v2, rq2, scale, valid, cfg,
                                          return_intermediates=True)
    expected = expected[:, rows]
    torch.cuda.synchronize()
    assert torch.equal(cache.landmark_keys[:, :-1], original_lmk[:, :-1])
    torch.testing.assert_close(cache.landmark_keys.float(), emid["landmark_keys"].float(),
                               atol=0.01, rtol=0.03)
    error = (actual.float() - expected.float()).norm() / expected.float().norm()
    print(f"cached refresh vs prefill: rel error {float(error):.3e}", flush=True)
    assert float(error) < 0.03


def test_kv_fragments_rows_bit_exact():
    _note("kv fragments rows")
    L, Hkv, D = 1000, 4, 128   # last chunk partial
    g = torch.Generator().manual_seed(93)
    k = torch.randn(1, L, Hkv, D, generator=g).bfloat16().to(DEV)
    v = torch.randn(1, L, Hkv, D, generator=g).bfloat16().to(DEV)
    f = mrsa.kv_fragments(k, v)
    pos = torch.tensor([0, 5, 15, 16, 31, 32, 63, 64, 500, 999], device=DEV)
    k.index_copy_(1, pos, torch.randn(1, pos.numel(), Hkv, D, generator=g).bfloat16().to(DEV))
    v.index_copy_(1, pos, torch.randn(1, pos.numel(), Hkv, D, generator=g).bfloat16().to(DEV))
    mrsa.sparse_attention.kv_fragments_rows(k, v, f, pos)
    assert torch.equal(f, mrsa.kv_fragments(k, v))


def test_kv_replace_rows_equals_index_copy_and_fragment_rebuild():
    # mrsa_kv_replace_rows: the rows of LayerKVCache.replace
    # (fastdllm_cache.py:126-127) and their fragment entries in one launch.
    _note("kv replace rows")
    L, Hkv, D = 1000, 4, 128   # last chunk partial
    g = torch.Generator().manual_seed(94)
    k = torch.randn(1, L, Hkv, D, generator=g).bfloat16().to(DEV)
    v = torch.randn(1, L, Hkv, D, generator=g).bfloat16().to(DEV)
    valid = torch.ones(1, L, dtype=torch.bool, device=DEV)
    cache = mrsa.LayerKVCache(k.clone(), v.clone(), valid, torch.zeros(1, 15, Hkv, 7, D,
                              dtype=torch.bfloat16, device=DEV),
                              torch.zeros(1, 15, Hkv, 7, device=DEV))
    cache.kv_frags = mrsa.kv_fragments(cache.key, cache.value)
    pos = torch.tensor([999, 0, 5, 16, 31, 32, 63, 64, 500], device=DEV)
    kr = torch.randn(1, pos.numel(), Hkv, D, generator=g).bfloat16().to(DEV)
    vr = torch.randn(1, pos.numel(), Hkv, D, generator=g).bfloat16().to(DEV)
    cache.replace(pos, kr, vr)
    k.index_copy_(1, pos, kr)
    v.index_copy_(1, pos, vr)
    assert torch.equal(cache.key, k) and torch.equal(cache.value, v)
    assert torch.equal(cache.kv_frags, mrsa.kv_fragments(k, v))
    # without fragments only the rows are written
    bare = mrsa.LayerKVCache(cache.key.clone(), cache.value.clone(), valid,
                             cache.landmark_keys, cache.prior_bias)
    kr2 = torch.randn(1, 2, Hkv, D, generator=g).bfloat16().to(DEV)
    bare.replace(torch.tensor([7, 8], device=DEV), kr2, kr2)
    k.index_copy_(1, torch.tensor([7, 8], device=DEV), kr2)
    assert bare.kv_frags is None and torch.equal(bare.key, k)


def test_copy_buffers_copies_every_pair():
    # mrsa_copy_buffers: the graph step's input copies in one launch (16-byte
    # and 8-byte units; an unaligned pair falls back to copy_).
    _note("copy buffers")
    from mrsa import _lib
    g = torch.Generator().manual_seed(97)
    src = [torch.randn(1, 32, 28, 128, generator=g).bfloat16().to(DEV),
           torch.randn(1, 32, 4, 128, generator=g).bfloat16().to(DEV),
           torch.arange(32, device=DEV), torch.tensor([7], device=DEV),
           torch.empty(0, dtype=torch.long, device=DEV),
           torch.randn(3, 5, generator=g).to(DEV)]            # 60 bytes: unaligned size
    dst = [torch.zeros_like(t) for t in src]
    _lib.copy_buffers(dst[:5], src[:5])
    for d, s in zip(dst[:5], src[:5]):
        assert torch.equal(d, s)
    _lib.copy_buffers(dst, src)
    for d, s in zip(dst, src):
        assert torch.equal(d, s)
    with pytest.raises(ValueError):
        _lib.check(_lib.call("mrsa_copy_buffers", 9, None, None, None, _lib.stream_of(src[0])),
                   "copy_buffers")


def test_pool_cached_chunks_equals_the_gathered_pool():
    # mrsa_pool_cached_chunks_fwd: the landmark refresh of the cached step
    # (fastdllm_attention.py:236-292) read in place, against the gathered
    # rows through chunk_attn_pool_gqa_prior and index_copy_ (same bits).
    L, Hq, Hkv, D, S = 4096, 28, 4, 128, 64
    C, G = L // S, Hq // Hkv
    g = torch.Generator().manual_seed(95)
    k, _ = _planted_kv(L, Hkv, D, 96)
    k = k.to(DEV)
    valid = torch.rand(1, L, generator=g) > 0.05
    valid[0, 64 * 20 : 64 * 21 - 1] = False        # chunk 20: only its landmark slot valid
    valid = valid.to(DEV)
    scale = (torch.rand(Hq, generator=g) + 0.5).to(DEV)
    lmk0 = torch.randn(1, C, Hkv, G, D, generator=g).bfloat16().to(DEV)
    prior0 = torch.rand(1, C, Hkv, G, generator=g).to(DEV)
    for rows_lo, affected in ((64 * 19 + 32, [19, 20]), (64 * 40, [40]), (0, [0])):
        _note(f"pool cached chunks rows {rows_lo}.. affected {affected}")
        pos = torch.arange(rows_lo, rows_lo + 96, device=DEV)
        rq = torch.randn(1, pos.numel(), Hq, D, generator=g).bfloat16().to(DEV)
        aff = torch.tensor(affected, device=DEV)
        cache = mrsa.LayerKVCache(k, k, valid, lmk0.clone(), prior0.clone())
        mrsa.route_layer._refresh_landmarks(rq, cache, pos, aff, scale, S)
        rows = torch.searchsorted(pos, aff * S + (S - 1))
        chunk_pos = (aff[:, None] * S + torch.arange(S, device=DEV)[None]).reshape(-1)
        lmk, _, prior = mrsa.chunk_attn_pool_gqa_prior(
            rq.index_select(1, rows).reshape(1, -1, Hkv, G, D).contiguous(),
            k.index_select(1, chunk_pos).reshape(1, -1, S, Hkv, D).contiguous(),
            valid.index_select(1, chunk_pos).reshape(1, -1, S).contiguous(), scale)
        want_lmk, want_prior = lmk0.clone(), prior0.clone()
        want_lmk.index_copy_(1, aff, lmk)
        want_prior.index_copy_(1, aff, prior)
        assert torch.equal(cache.landmark_keys, want_lmk)
        assert torch.equal(cache.prior_bias, want_prior)
    # a chunk out of range, or whose landmark row is not a query position,
    # is left as it is
    _note("pool cached chunks: skipped chunks")
    cache = mrsa.LayerKVCache(k, k, valid, lmk0.clone(), prior0.clone())
    pos = torch.arange(64 * 5, 64 * 5 + 32, device=DEV)
    rq = torch.randn(1, 32, Hq, D, generator=g).bfloat16().to(DEV)
    mrsa.route_layer._refresh_landmarks(rq, cache, pos, torch.tensor([5, C, -1], device=DEV),
                                        scale, S)
    assert torch.equal(cache.landmark_keys, lmk0) and torch.equal(cache.prior_bias, prior0)


def test_cache_replace_keeps_tiles_and_checks_arguments():
    # LayerKVCache.replace (fastdllm_cache.py:94-125): rows written, the tiled
    # V copy kept in step (the next cached step equals one on a fresh cache),
    # duplicate / out-of-range positions rejected.
    _note("cache replace")
    L, Hq, Hkv, D, S = 2048, 28, 4, 128, 64
    q, rq, k, v = _cache_inputs(L, Hq, Hkv, D, 91)
    valid = torch.ones(1, L, dtype=torch.bool, device=DEV)
    scale = torch.ones(Hq, device=DEV)
    g = torch.Generator().manual_seed(92)
    lmk = torch.randn(1, L // S, Hkv, Hq // Hkv, D, generator=g).bfloat16().to(DEV)
    prior = (torch.rand(1, L // S, Hkv, Hq // Hkv, generator=g) * 0.5).to(DEV)
    k, v = k.to(DEV), v.to(DEV)
    cache = mrsa.LayerKVCache(k.clone(), v.clone(), valid, lmk.clone(), prior.clone())
    rows = torch.arange(L - 2 * S, L - S, device=DEV)
    empty = torch.empty(0, dtype=torch.long, device=DEV)
    qb, rqb = q[:, rows.cpu()].to(DEV), rq[:, rows.cpu()].to(DEV)
    mrsa.cached_route_attention(qb, rqb, cache, rows, empty, scale)   # builds the fragments
    assert cache.kv_frags is not None
    kb = torch.randn(1, S, Hkv, D, generator=g).bfloat16().to(DEV)
    vb = torch.randn(1, S, Hkv, D, generator=g).bfloat16().to(DEV)
    cache.replace(rows, kb, vb)
    got = mrsa.cached_route_attention(qb, rqb, cache, rows, empty, scale)
    fresh = mrsa.LayerKVCache(cache.key.clone(), cache.value.clone(), valid, lmk.clone(),
                              prior.clone())
    want = mrsa.cached_route_attention(qb, rqb, fresh, rows, empty, scale)
    assert torch.equal(cache.kv_frags, fresh.kv_frags)
    assert_nearly_identical(got, want, "replaced cache vs fresh cache", atol=0.03)
    with pytest.raises(ValueError, match="unique"):
        cache.replace(torch.tensor([3, 3], device=DEV), kb[:, :2], vb[:, :2])
    with pytest.raises(ValueError, match="range"):
        cache.replace(torch.tensor([L], device=DEV), kb[:, :1], vb[:, :1])


def test_cached_route_attention_argument_errors():
    _note("cached route errors")
    L, Hq, Hkv, D, S = 1024, 28, 4, 128, 64
    q, rq, k, v = _cache_inputs(L, Hq, Hkv, D, 93)
    valid = torch.ones(1, L, dtype=torch.bool, device=DEV)
    lmk = torch.zeros(1, L // S, Hkv, Hq // Hkv, D, dtype=torch.bfloat16, device=DEV)
    prior = torch.zeros(1, L // S, Hkv, Hq // Hkv, device=DEV)
    cache = mrsa.LayerKVCache(k.to(DEV), v.to(DEV), valid, lmk, prior)
    scale = torch.ones(Hq, device=DEV)
    qb, rqb = q[:, :4].to(DEV), rq[:, :4].to(DEV)
    ok = torch.tensor([60, 61, 62, 63], device=DEV)
    none = torch.empty(0, dtype=torch.long, device=DEV)
    with pytest.raises(ValueError, match="sorted"):
        mrsa.cached_route_attention(qb, rqb, cache, ok.flip(0), none, scale)
    with pytest.raises(ValueError, match="range"):
        mrsa.cached_route_attention(qb, rqb, cache, ok + L, none, scale)
    with pytest.raises(ValueError, match="affected_chunks"):
        mrsa.cached_route_attention(qb, rqb, cache, ok, torch.tensor([L // S], device=DEV), scale)
    with pytest.raises(ValueError, match="owned positions"):
        mrsa.cached_route_attention(qb, rqb, cache, ok, torch.tensor([1], device=DEV), scale)
    out = mrsa.cached_route_attention(qb, rqb, cache, ok, torch.tensor([0], device=DEV), scale)
    assert bool(torch.isfinite(out.float()).all())


def test_cached_block_step_argument_errors_leave_the_cache_alone():
    # CachedBlockStep reads its device checks (one kernel) after queueing the
    # input copies: a bad call raises the reference's errors and changes no
    # cache row; the next good call runs normally.
    _note("cached block step errors")
    L, Hq, Hkv, D, S, bs = 1024, 28, 4, 128, 64, 4
    q, rq, k, v = _cache_inputs(L, Hq, Hkv, D, 94)
    valid = torch.ones(1, L, dtype=torch.bool, device=DEV)
    lmk = torch.zeros(1, L // S, Hkv, Hq // Hkv, D, dtype=torch.bfloat16, device=DEV)
    prior = torch.zeros(1, L // S, Hkv, Hq // Hkv, device=DEV)
    cache = mrsa.LayerKVCache(k.to(DEV), v.to(DEV), valid, lmk, prior)
    step = mrsa.CachedBlockStep(cache, torch.ones(Hq, device=DEV), block_len=bs)
    qb, rqb = q[:, :bs].to(DEV), rq[:, :bs].to(DEV)
    kb = (torch.randn(1, bs, Hkv, D, generator=torch.Generator().manual_seed(95))).bfloat16().to(DEV)
    ok = torch.tensor([60, 61, 62, 63], device=DEV)
    none = torch.empty(0, dtype=torch.long, device=DEV)
    key0 = cache.key.clone()
    for pos, aff, msg in ((ok.flip(0), none, "sorted"), (ok + L, none, "range"),
                          (ok, torch.tensor([L // S], device=DEV), "affected_chunks"),
                          (ok, torch.tensor([1], device=DEV), "owned positions")):
        with pytest.raises(ValueError, match=msg):
            step(qb, rqb, kb, kb, pos, aff)
        torch.cuda.synchronize()
        assert torch.equal(cache.key, key0), msg
    out = step(qb, rqb, kb, kb, ok, torch.tensor([0], device=DEV))
    assert bool(torch.isfinite(out.float()).all())
    assert torch.equal(cache.key[:, 60:64], kb)


@pytest.mark.parametrize("policy", [None, "entropy_adaptive"])
def test_cached_block_step_graph_replays_match_eager(policy):
    # CachedBlockStep (HIP graph of the K/V row write + cached route layer)
    # against the eager replace + cached_route_attention on a twin cache,
    # block after block: graphs for 0 and 1 affected chunks, each replayed
    # several times with eager work and synchronisation in between; the caches
    # (keys, values, tiles, landmarks) equal, every replay's output equal up
    # to the routed attention's varying fp32 summation order.
    _note(f"cached block step graph token policy={policy}")
    cfg = mrsa.RouteLayerConfig() if policy is None else mrsa.RouteLayerConfig(
        token_budget=256, token_policy=policy)
    L, Hq, Hkv, D, S, bs = 4096, 28, 4, 128, 64, 32
    G = Hq // Hkv
    g = torch.Generator().manual_seed(95)
    k, v = _planted_kv(L, Hkv, D, 96)
    k, v = k.to(DEV), v.to(DEV)
    valid = torch.ones(1, L, dtype=torch.bool, device=DEV)
    valid[0, 1000:1003] = False
    scale = (torch.rand(Hq, generator=g) + 0.5).to(DEV)
    lmk = torch.randn(1, L // S, Hkv, G, D, generator=g).bfloat16().to(DEV)
    prior = (torch.rand(1, L // S, Hkv, G, generator=g) * 0.5).to(DEV)
    twin = lambda: mrsa.LayerKVCache(k.clone(), v.clone(), valid.clone(), lmk.clone(),
                                     prior.clone())
    graphed, eager = twin(), twin()
    step = mrsa.CachedBlockStep(graphed, scale, cfg, block_len=bs)
    start = L - 8 * bs
    for i in list(range(8)) + [1, 0]:
        pos = torch.arange(start + i * bs, start + (i + 1) * bs, device=DEV)
        aff = pos[(pos + 1) % S == 0] // S
        rnd = lambda *shape: torch.randn(*shape, generator=g).bfloat16().to(DEV)
        q, rq, kb, vb = rnd(1, bs, Hq, D), rnd(1, bs, Hq, D), rnd(1, bs, Hkv, D), rnd(1, bs, Hkv, D)
        got = step(q, rq, kb, vb, pos, aff).clone()
        eager.replace(pos, kb, vb)
        want = mrsa.cached_route_attention(q, rq, eager, pos, aff, scale, cfg)
        torch.cuda.synchronize()
        assert_nearly_identical(got, want, f"block {i}: graph vs eager", atol=0.03)
    for name in ("key", "value", "kv_frags", "landmark_keys", "prior_bias"):
        assert torch.equal(getattr(graphed, name), getattr(eager, name)), name
    with pytest.raises(ValueError, match="sorted"):
        step(q, rq, kb, vb, pos.flip(0), aff)
