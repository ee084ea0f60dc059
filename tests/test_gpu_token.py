"""GPU parity of the remote-token refinement ("global_qk" policy,
dream_dllm_hils/token_refinement.py:112-148, :359-392; attention.py:1729-1769)
against the CPU oracle, through the C-ABI.

Keep masks are bit-exact (ties at the budget threshold go to the lower flat
index on both sides); attention outputs within max-abs 2e-2 / mean-abs 2e-3.
"""

import math

import pytest
import torch

import mrsa
from mrsa.sparse_attention import selected_attention_launch
from oracle import mrsa_oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _note(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _close(actual, expected, what, max_abs=2e-2, mean_abs=2e-3):
    err = (actual.float().cpu() - expected.float()).abs()
    print(f"{what}: max_abs={err.max():.3e} mean_abs={err.mean():.3e}", flush=True)
    assert float(err.max()) <= max_abs, what
    assert float(err.mean()) <= mean_abs, what


@pytest.mark.parametrize("budget,ties", [(1, False), (512, False), (2048, False), (5000, False),
                                         (300, True)])
def test_token_keep_bit_exact(budget, ties):
    _note(f"token keep budget={budget} ties={ties}")
    g = torch.Generator().manual_seed(100 + budget)
    scores = torch.randn(1, 37, 4, 32, 64, generator=g)
    if ties:
        scores = scores.round(decimals=1)
    scores[..., -1] = float("-inf")                       # landmark slots
    scores[0, 3, :, 20:] = float("-inf")                  # -1 slots
    scores[0, 5, 1] = float("-inf")                       # nothing routed
    keep = mrsa.select_global_token_keep(scores.to(DEV), budget, training=False)
    assert keep.dtype == torch.uint8
    assert torch.equal(keep.cpu(), O.select_global_token_keep(scores, budget))


def _route_inputs(Lq, Lk, K, seed, Hkv=4, G=7, D=128):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, Lq, Hkv * G, D, generator=g).bfloat16()
    k = torch.randn(1, Lk, Hkv, D, generator=g).bfloat16()
    v = torch.randn(1, Lk, Hkv, D, generator=g).bfloat16()
    C = Lk // 64
    idx = torch.stack([torch.randperm(C, generator=g)[:K] for _ in range(Lq * Hkv)])
    idx = idx.sort(-1).values.reshape(1, Lq, Hkv, K).int()
    idx[0, 0, :, K // 2:] = -1
    w = torch.softmax(torch.randn(1, Lq, Hkv * G, K, generator=g), -1).bfloat16()
    valid = torch.rand(1, Lk, generator=g) > 0.03
    return q, k, v, idx, w, valid


def test_refine_remote_tokens_vs_oracle():
    _note("refine remote tokens")
    q, k, v, idx, w, valid = _route_inputs(50, 4096, 32, 110)
    keep = mrsa.refine_remote_tokens_g7(q.to(DEV), k.to(DEV), idx.to(DEV), valid.to(DEV), 64, 512,
                                        training=False)
    assert keep.dtype == torch.int8 and keep.shape == (1, 50, 4, 32, 64)
    ref = O.select_global_token_keep(O.candidate_token_scores(q, k, idx, valid, 64), 512)
    differ = (keep.cpu().to(torch.uint8) != ref).reshape(50 * 4, -1).any(-1)
    print(f"refine: rows whose keep mask differs: {int(differ.sum())} of {differ.numel()}",
          flush=True)
    assert int(differ.sum()) <= 2   # fp32 sum-order differences at the budget boundary only


@pytest.mark.parametrize("Lq,Lk,parts", [(300, 4096, 1), (777, 2048, 1), (32, 16384, 7)])
def test_selected_attention_token_keep_vs_oracle(Lq, Lk, parts):
    _note(f"selected keep Lq={Lq} Lk={Lk} parts={parts}")
    q, k, v, idx, w, valid = _route_inputs(Lq, Lk, 32, 120 + Lq)
    g = torch.Generator().manual_seed(130)
    keep = (torch.rand(1, Lq, 4, 32, 64, generator=g) > 0.4).to(torch.int8)
    keep[0, 1, 2, 5] = 0                                  # a slot with nothing kept
    out = selected_attention_launch(q.to(DEV), mrsa.kv_fragments(k.to(DEV), v.to(DEV)),
                                    w.to(DEV), idx.to(DEV), valid.to(DEV), 64, parts=parts,
                                    token_keep=keep.to(DEV))
    ref = O.selected_attention(q, k, v, w, idx, valid, 64, token_keep=keep)
    _close(out, ref, f"selected keep Lq={Lq}")


def test_selected_attention_reference_kat_filtered():
    # test_hils_non_power_two_topk.py:95-142 with filtered=True (token_keep),
    # cached and uncached shapes.
    for query_len in (35, 2048):
        _note(f"selected KAT filtered q={query_len}")
        g = torch.Generator().manual_seed(79)
        kv_len, h_kv, grp, dim, topk, size = 2048, 4, 7, 128, 31, 64
        q = torch.randn(1, query_len, h_kv * grp, dim, generator=g).bfloat16()
        k = torch.randn(1, kv_len, h_kv, dim, generator=g).bfloat16()
        v = torch.randn(1, kv_len, h_kv, dim, generator=g).bfloat16()
        indices = torch.arange(topk, dtype=torch.int32).expand(1, query_len, h_kv, -1).clone()
        indices[:, 0] = -1
        weights = torch.randn(1, query_len, h_kv * grp, topk, generator=g).softmax(-1).bfloat16()
        weights[:, 0] = 0
        valid = torch.ones(1, kv_len, dtype=torch.bool)
        valid[:, ::97] = False
        keep = torch.rand(1, query_len, h_kv, topk, size, generator=g) > 0.4
        args = [t.to(DEV) for t in (q, k, v, weights, indices, valid)]
        kd = keep.to(DEV)
        actual = (mrsa.selected_attention_g7_cached(*args, size, token_keep=kd) if query_len == 35
                  else mrsa.selected_attention_g7(*args, size, training=False, token_keep=kd))
        assert actual.shape == q.shape and bool(torch.isfinite(actual).all())
        assert torch.equal(actual[:, 0].cpu(), torch.zeros_like(actual[:, 0].cpu()))
        rows = torch.tensor([1, query_len // 2, query_len - 1])
        qs = q[0, rows].float().reshape(-1, h_kv, grp, dim)
        expected = torch.zeros_like(qs)
        ws = weights[0, rows].float().reshape(-1, h_kv, grp, topk)
        for chunk in range(topk):
            start = chunk * size
            ks, vs = k[0, start:start + size].float(), v[0, start:start + size].float()
            logits = torch.einsum("rhgd,shd->rhgs", qs, ks) / math.sqrt(dim)
            allowed = valid[0, start:start + size].expand(rows.numel(), h_kv, -1).clone()
            allowed[..., -1] = False
            allowed &= keep[0, rows, :, chunk]
            probs = logits.masked_fill(~allowed[:, :, None], float("-inf")).softmax(-1)
            expected += torch.einsum("rhgs,shd->rhgd", probs, vs) * ws[..., chunk, None]
        observed = actual.cpu()[0, rows].float().reshape_as(expected)
        assert float((observed - expected).norm() / expected.norm()) < 0.02
        torch.testing.assert_close(observed, expected, atol=0.01, rtol=0.025)
        assert torch.equal(kd.cpu(), keep)


def test_route_layer_with_token_budget_vs_oracle():
    _note("route layer token budget 512")
    L, Hq, Hkv, D = 2048, 28, 4, 128
    g = torch.Generator().manual_seed(140)
    q = torch.randn(1, L, Hq, D, generator=g).bfloat16()
    rq = torch.randn(1, L, Hq, D, generator=g).bfloat16()
    k = torch.randn(1, L, Hkv, D, generator=g)
    k = (k + 0.3 * torch.randn(L // 64, Hkv, D, generator=g).repeat_interleave(64, 0)[None])
    k = k.bfloat16()
    v = torch.randn(1, L, Hkv, D, generator=g).bfloat16()
    scale = torch.rand(Hq, generator=g) + 0.5
    valid = torch.ones(1, L, dtype=torch.bool)
    cfg = mrsa.RouteLayerConfig(token_budget=512)
    out, mid = mrsa.route_attention(q.to(DEV), k.to(DEV), v.to(DEV), rq.to(DEV), scale.to(DEV),
                                    valid.to(DEV), cfg, return_intermediates=True)
    ref, rmid = O.route_layer(q, k, v, rq, scale, valid, token_budget=512)
    same_routes = (mid["indices"].cpu().long() == rmid["indices"]).all(-1)
    same_keep = (mid["token_keep"].cpu().to(torch.uint8) == rmid["token_keep"]).all(-1).all(-1)
    rows = (same_routes & same_keep)[..., None].expand(-1, -1, -1, Hq // Hkv).reshape(1, L, Hq)
    print(f"route layer budget: rows with identical routes and keep masks: "
          f"{float(rows.float().mean()):.4f}", flush=True)
    assert float(rows.float().mean()) > 0.97
    _close(out.cpu()[rows], ref[rows], "route layer with token budget")
    with pytest.raises(ValueError, match="exceeds"):
        mrsa.route_attention(q.to(DEV), k.to(DEV), v.to(DEV), rq.to(DEV), scale.to(DEV),
                             valid.to(DEV), mrsa.RouteLayerConfig(token_budget=4096))


# -- entropy_adaptive (token_refinement.py:150-438) ----------------------------
@pytest.mark.parametrize("budget,mn,ties", [(256, 1, False), (64, 2, False), (2048, 0, False),
                                            (100, 1, True)])
def test_entropy_token_keep_bit_exact(budget, mn, ties):
    _note(f"entropy token keep budget={budget} min={mn} ties={ties}")
    g = torch.Generator().manual_seed(200 + budget)
    B, L, H, K, S = 1, 37, 4, 32, 64
    scores = torch.randn(B, L, H, K, S, generator=g)
    if ties:
        scores = scores.round(decimals=1)
    scores[..., -1] = float("-inf")                       # landmark slots
    scores[0, 3, :, 20:] = float("-inf")                  # -1 slots
    scores[0, 5, 1] = float("-inf")                       # nothing routed
    scores[0, 6, 2, :, 5:] = float("-inf")                # capacities of 5
    ent = torch.rand(B, L, H, K, generator=g) * 4 - 0.5
    ent[0, 7, 0, :4] = torch.tensor([float("nan"), float("inf"), float("-inf"), 9.0])
    keep, alloc = mrsa.select_entropy_adaptive_token_keep(scores.to(DEV), ent.to(DEV), budget, mn,
                                                          training=False)
    rkeep, ralloc = O.select_entropy_adaptive_token_keep(scores, ent, budget, mn)
    assert keep.dtype == torch.uint8 and alloc.dtype == torch.int64
    assert torch.equal(alloc.cpu(), ralloc)
    assert torch.equal(keep.cpu(), rkeep)
    # the allocation-only entry and the gather agree with the oracle too
    cap = torch.isfinite(scores).sum(-1)
    a2 = mrsa.allocate_entropy_token_budget(ent.to(DEV), cap.to(DEV), budget, mn)
    assert torch.equal(a2.cpu(), ralloc)


def test_gather_selected_chunk_entropy_vs_oracle():
    _note("gather selected chunk entropy")
    g = torch.Generator().manual_seed(210)
    ent = torch.rand(2, 40, 4, 7, generator=g) * 3
    idx = torch.randint(-1, 43, (2, 33, 4, 32), generator=g).int()
    got = mrsa.gather_selected_chunk_entropy(ent.to(DEV), idx.to(DEV))
    torch.testing.assert_close(got.cpu(), O.gather_selected_chunk_entropy(ent, idx),
                               atol=1e-6, rtol=1e-6)
    with pytest.raises(ValueError, match="per-chunk minimum"):
        mrsa.allocate_entropy_token_budget(ent[0, :, 0].to(DEV), torch.ones(40, 7, device=DEV),
                                           10, 2)


def test_refine_remote_tokens_entropy_vs_oracle():
    _note("refine remote tokens entropy")
    q, k, v, idx, w, valid = _route_inputs(50, 4096, 32, 220)
    g = torch.Generator().manual_seed(221)
    ent = torch.rand(1, 64, 4, 7, generator=g) * 3
    keep, alloc = mrsa.refine_remote_tokens_entropy_g7(
        q.to(DEV), k.to(DEV), idx.to(DEV), valid.to(DEV), ent.to(DEV), 64, 512, 1,
        training=False)
    assert keep.dtype == torch.int8 and keep.shape == (1, 50, 4, 32, 64)
    scores = O.candidate_token_scores(q, k, idx, valid, 64)
    rkeep, ralloc = O.select_entropy_adaptive_token_keep(
        scores, O.gather_selected_chunk_entropy(ent, idx), 512, 1)
    assert torch.equal(alloc.cpu(), ralloc)  # capacities are exact, so quotas match
    differ = (keep.cpu().to(torch.uint8) != rkeep).reshape(50 * 4, -1).any(-1)
    print(f"refine entropy: rows whose keep mask differs: {int(differ.sum())} of "
          f"{differ.numel()}", flush=True)
    assert int(differ.sum()) <= 2   # fp32 score differences at a chunk's quota boundary only


def test_route_layer_entropy_policy_vs_oracle():
    _note("route layer entropy policy budget 512")
    L, Hq, Hkv, D = 2048, 28, 4, 128
    g = torch.Generator().manual_seed(230)
    q = torch.randn(1, L, Hq, D, generator=g).bfloat16()
    rq = torch.randn(1, L, Hq, D, generator=g).bfloat16()
    k = torch.randn(1, L, Hkv, D, generator=g)
    k = (k + 0.3 * torch.randn(L // 64, Hkv, D, generator=g).repeat_interleave(64, 0)[None])
    k = k.bfloat16()
    v = torch.randn(1, L, Hkv, D, generator=g).bfloat16()
    scale = torch.rand(Hq, generator=g) + 0.5
    valid = torch.ones(1, L, dtype=torch.bool)
    cfg = mrsa.RouteLayerConfig(token_budget=512, token_policy="entropy_adaptive",
                                min_tokens_per_chunk=2)
    out, mid = mrsa.route_attention(q.to(DEV), k.to(DEV), v.to(DEV), rq.to(DEV), scale.to(DEV),
                                    valid.to(DEV), cfg, return_intermediates=True)
    ref, rmid = O.route_layer(q, k, v, rq, scale, valid, token_budget=512,
                              token_policy="entropy_adaptive", min_tokens_per_chunk=2)
    same_routes = (mid["indices"].cpu().long() == rmid["indices"]).all(-1)
    same_keep = (mid["token_keep"].cpu().to(torch.uint8) == rmid["token_keep"]).all(-1).all(-1)
    rows = (same_routes & same_keep)[..., None].expand(-1, -1, -1, Hq // Hkv).reshape(1, L, Hq)
    print(f"route layer entropy policy: rows with identical routes and keep masks: "
          f"{float(rows.float().mean()):.4f}", flush=True)
    assert float(rows.float().mean()) > 0.97
    _close(out.cpu()[rows], ref[rows], "route layer with entropy token policy")
    with pytest.raises(ValueError, match="cover the minimum"):
        mrsa.route_attention(q.to(DEV), k.to(DEV), v.to(DEV), rq.to(DEV), scale.to(DEV),
                             valid.to(DEV), mrsa.RouteLayerConfig(
                                 token_budget=40, token_policy="entropy_adaptive",
                                 min_tokens_per_chunk=2))


@pytest.mark.parametrize("policy", ["global_qk", "entropy_adaptive"])
def test_cached_route_attention_token_budget_vs_oracle(policy):
    _note(f"cached route layer token budget policy={policy}")
    L, Hq, Hkv, D, S = 4096, 28, 4, 128, 64
    C, G = L // S, Hq // Hkv
    g = torch.Generator().manual_seed(240)
    q = torch.randn(1, L, Hq, D, generator=g).bfloat16()
    rq = torch.randn(1, L, Hq, D, generator=g).bfloat16()
    k = torch.randn(1, L, Hkv, D, generator=g)
    k = (k + 0.3 * torch.randn(C, Hkv, D, generator=g).repeat_interleave(64, 0)[None]).bfloat16()
    v = torch.randn(1, L, Hkv, D, generator=g).bfloat16()
    valid = torch.ones(1, L, dtype=torch.bool)
    scale = torch.rand(Hq, generator=g) + 0.5
    lmk0 = torch.randn(1, C, Hkv, G, D, generator=g).bfloat16()
    prior0 = torch.rand(1, C, Hkv, G, generator=g) * 0.5
    chunk = 31
    rows = torch.arange(chunk * S, (chunk + 1) * S)
    aff = torch.tensor([chunk])
    cache = mrsa.LayerKVCache(k.to(DEV), v.to(DEV), valid.to(DEV), lmk0.clone().to(DEV),
                              prior0.clone().to(DEV))
    cfg = mrsa.RouteLayerConfig(token_budget=256, token_policy=policy)
    out, mid = mrsa.cached_route_attention(
        q[:, rows].to(DEV), rq[:, rows].to(DEV), cache, rows.to(DEV), aff.to(DEV),
        scale.to(DEV), cfg, return_intermediates=True)
    ref, _, _, rmid = O.cached_route_layer(
        q[:, rows], rq[:, rows], k, v, valid, lmk0, prior0, rows, aff, scale,
        token_budget=256, token_policy=policy)
    same_routes = (mid["indices"].cpu().long() == rmid["indices"]).all(-1)
    same_keep = (mid["token_keep"].cpu().to(torch.uint8) == rmid["token_keep"]).all(-1).all(-1)
    ok = (same_routes & same_keep)[..., None].expand(-1, -1, -1, G).reshape(1, S, Hq)
    print(f"cached {policy}: rows with identical routes and keep masks: "
          f"{float(ok.float().mean()):.4f}", flush=True)
    assert float(ok.float().mean()) > 0.95
    _close(out.cpu()[ok], ref[ok], f"cached route layer, {policy} token budget")
