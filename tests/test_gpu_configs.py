"""BASELINE configurations 3 and 5 at their full size, against the oracle on
sampled rows (configuration 2 is in test_gpu_parity.py, 4 in
test_gpu_dream.py).  The oracle's rows depend only on their own inputs, so
a full-size GPU run is checked row by row without running the oracle over
every row.

Tolerances (the build target): attention outputs within max-abs 2e-2 and
mean-abs 2e-3, the natural-log LSE within 2e-3; routing lists identical
except near ties (routing_check.py); drop rows bit-exact.
"""

import pytest
import torch

import mrsa
from mrsa.local_attention import local_attention_launch
from oracle import dream_oracle as DO
from oracle import mrsa_oracle as O
from routing_check import assert_nearly_identical, classify_routing

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _note(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _close(actual, expected, what, max_abs=2e-2, mean_abs=2e-3):
    err = (actual.float().cpu() - expected.float()).abs()
    print(f"{what}: max_abs={err.max():.3e} mean_abs={err.mean():.3e}", flush=True)
    assert float(err.max()) <= max_abs, what
    assert float(err.mean()) <= mean_abs, what


def _yarn_rotate(x):
    # YaRN factor 8 (theta 1e6, original context 2048) applied in fp32 over
    # positions 0..L-1, from the oracle's frequencies
    inv, af = DO.yarn_inv_freq(128, 1e6, 8.0, 2048)
    L = x.shape[1]
    ang = torch.outer(torch.arange(L, dtype=torch.float64), inv)
    c = (ang.cos() * af).float()[None, :, None, :]
    s = (ang.sin() * af).float()[None, :, None, :]
    x1, x2 = x[..., :64], x[..., 64:]
    return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s), dim=-1)


def test_config3_swa_full_size_sampled_rows():
    # SWA-1280 layer at L=16384, 28/4 heads: rows at both clipped edges, the
    # first and last rows with the full 2561-key window, tile boundaries of
    # the 16-query blocks and random interior rows.
    L, Hq, Hkv, D, W = 16384, 28, 4, 128, 1280
    _note(f"config 3 SWA L={L} W={W} full size")
    g = torch.Generator().manual_seed(300)
    q = _yarn_rotate(torch.randn(1, L, Hq, D, generator=g)).bfloat16()
    k = _yarn_rotate(torch.randn(1, L, Hkv, D, generator=g)).bfloat16()
    v = torch.randn(1, L, Hkv, D, generator=g).bfloat16()
    dq, dk, dv = q.to(DEV), k.to(DEV), v.to(DEV)
    out, lse = local_attention_launch(dq, mrsa.kv_fragments(dk, dv), None, W, 0)
    swa = mrsa.swa_attention(dq, dk, dv, None, W, 64)
    torch.cuda.synchronize()
    assert torch.equal(swa.view(torch.int16), out.view(torch.int16))
    rnd = torch.randint(W + 1, L - W - 1, (24,), generator=g).tolist()
    rows = sorted(set([0, 1, 15, 16, 63, 64, 640, W - 1, W, W + 1, 8191, 8192,
                       L - W - 2, L - W - 1, L - W, L - 65, L - 64, L - 17, L - 16, L - 2,
                       L - 1] + rnd))
    rows = torch.tensor(rows)
    full = ((rows >= W) & (rows <= L - 1 - W)).sum()
    assert int(full) >= 20       # rows whose window holds all 2561 keys
    ro, rl = O.local_attention(q[:, rows], k, v, None, W, 0, query_positions=rows,
                               query_block=1)
    _close(out.cpu()[:, rows], ro, f"config 3 rows ({rows.numel()}, {int(full)} full windows)")
    torch.testing.assert_close(lse.cpu()[:, rows], rl, atol=2e-3, rtol=1e-4)


def _cache(L, seed):
    S, Hq, Hkv, D = 64, 28, 4, 128
    C, G = L // S, Hq // Hkv
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(1, L, Hkv, D, generator=g)
    k = (k + 0.3 * torch.randn(C, Hkv, D, generator=g).repeat_interleave(S, 0)[None])
    v = torch.randn(1, L, Hkv, D, generator=g)
    k, v = k.bfloat16(), v.bfloat16()
    q_lmk = torch.randn(1, C, Hkv, G, D, generator=g).bfloat16()
    scale = torch.rand(Hq, generator=g) + 0.5
    return k, v, q_lmk, scale, g


def test_config5_cached_block_step_at_128k():
    # The cached block step (K/V rows written, landmark refresh of the
    # affected chunk, window + routing over all 2048 landmarks + routed
    # attention, one HIP graph) at a 131072-token cache: two successive
    # 32-token blocks at the tail, the second holding chunk 2047's landmark.
    L, S, Hq, Hkv, D, bs = 131072, 64, 28, 4, 128, 32
    C = L // S
    _note(f"config 5 cached block step cache={L}")
    k, v, q_lmk, scale, g = _cache(L, 500)
    valid = torch.ones(1, L, dtype=torch.bool)
    dk, dv, dvalid = k.to(DEV), v.to(DEV), valid.to(DEV)
    lmk, _, prior = mrsa.chunk_attn_pool_gqa_prior(q_lmk.to(DEV), dk.reshape(1, C, S, Hkv, D),
                                                   dvalid.reshape(1, C, S), scale.to(DEV))
    cache = mrsa.LayerKVCache(dk.clone(), dv.clone(), dvalid, lmk.contiguous(),
                              prior.contiguous())
    cfg = mrsa.RouteLayerConfig()
    step = mrsa.CachedBlockStep(cache, scale.to(DEV), cfg, bs)
    kc, vc = k.clone(), v.clone()
    for start, aff in ((L - 2 * bs, []), (L - bs, [C - 1])):
        pos = torch.arange(start, start + bs)
        q = torch.randn(1, bs, Hq, D, generator=g).bfloat16()
        rq = torch.randn(1, bs, Hq, D, generator=g).bfloat16()
        kb = torch.randn(1, bs, Hkv, D, generator=g).bfloat16()
        vb = torch.randn(1, bs, Hkv, D, generator=g).bfloat16()
        affected = torch.tensor(aff, dtype=torch.long)
        lmk_before = cache.landmark_keys.cpu()
        prior_before = cache.prior_bias.cpu()
        out = step(q.to(DEV), rq.to(DEV), kb.to(DEV), vb.to(DEV), pos.to(DEV),
                   affected.to(DEV)).clone()
        # the same state through the eager path, for the stage outputs (the
        # rows are written again and the refresh recomputes the same values)
        eager, mid = mrsa.cached_route_attention(q.to(DEV), rq.to(DEV), cache, pos.to(DEV),
                                                 affected.to(DEV), scale.to(DEV), cfg,
                                                 return_intermediates=True)
        torch.cuda.synchronize()
        assert_nearly_identical(out, eager, f"block {start}: graph vs eager", atol=0.03)
        kc[:, pos] = kb
        vc[:, pos] = vb
        ref, rlmk, rprior, rmid = O.cached_route_layer(
            q, rq, kc, vc, valid, lmk_before, prior_before, pos, affected, scale)
        assert torch.equal(mid["drop_mask"].cpu(), rmid["drop_mask"])
        others = torch.ones(C, dtype=torch.bool)
        others[aff] = False
        assert torch.equal(cache.landmark_keys.cpu()[:, others], lmk_before[:, others])
        _close(cache.landmark_keys.cpu(), rlmk, f"block {start}: landmarks")
        torch.testing.assert_close(cache.prior_bias.cpu(), rprior, atol=1e-3, rtol=1e-3)
        classify_routing(mid["indices"], rmid["indices"], rq, cache.landmark_keys,
                         mid["local_lse"], cache.prior_bias,
                         lambda r: O.remote_drop_mask_rows(valid, 256, S, pos[r]), 32, S,
                         f"config 5 block {start}")
        _close(mid["local_output"], rmid["local_output"], f"block {start}: local branch")
        _close(out, ref, f"block {start}: step output")
