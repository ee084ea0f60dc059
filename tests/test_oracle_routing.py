"""Pins the oracle's route scoring / top-k and route weights (CPU)."""

import math

import pytest
import torch

from oracle import mrsa_oracle as O


def _brute_route(q5, lmk, lse4, bias4, drop, topk):
    """Explicit loops: selection score, top-k with lower-index tie rule."""

    B, L, H, G, D = q5.shape
    C = lmk.shape[1]
    idx = torch.full((B, L, H, topk), -1, dtype=torch.int64)
    for b in range(B):
        for i in range(L):
            for h in range(H):
                sel = []
                for c in range(C):
                    best = -math.inf
                    for g in range(G):
                        xs = []
                        for cc in range(C):
                            s = sum(float(q5[b, i, h, g, d]) * float(lmk[b, cc, h * G + g, d])
                                    for d in range(D)) / math.sqrt(D)
                            xs.append(s + float(bias4[b, cc, h, g]))
                        m = max(xs)
                        lse_h = m + math.log(sum(math.exp(x - m) for x in xs))
                        a = float(lse4[b, i, h, g])
                        mm = max(a, lse_h)
                        tot = mm + math.log(math.exp(a - mm) + math.exp(lse_h - mm))
                        best = max(best, xs[c] - tot)
                    if drop[b, i, c]:
                        best = -math.inf
                    sel.append(best)
                order = sorted(range(C), key=lambda c: (-sel[c], c))[:topk]
                picks = sorted(c for c in order if sel[c] != -math.inf)
                for j, c in enumerate(picks):
                    idx[b, i, h, j] = c
    return idx


def _inputs(seed, B=1, L=6, H=2, G=3, D=8, C=9):
    g = torch.Generator().manual_seed(seed)
    q5 = torch.randn(B, L, H, G, D, generator=g).bfloat16()
    lmk = torch.randn(B, C, H * G, D, generator=g).bfloat16()
    lse4 = torch.randn(B, L, H, G, generator=g)
    bias4 = torch.rand(B, C, H, G, generator=g)
    drop = torch.rand(B, L, C, generator=g) < 0.25
    return q5, lmk, lse4, bias4, drop


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_route_topk_matches_brute_force(seed):
    q5, lmk, lse4, bias4, drop = _inputs(seed)
    idx, scores, _ = O.route_topk(q5, lmk, lse4, 4, 64, drop_mask=drop.int(), bias4=bias4)
    assert torch.equal(idx, _brute_route(q5, lmk, lse4, bias4, drop, 4))


def test_route_topk_reference_properties():
    # test_hils_non_power_two_topk.py:30-48: ascending picks, in range, raw scores.
    g = torch.Generator().manual_seed(73)
    q = torch.randn(1, 35, 28, 128, generator=g).bfloat16()
    lm = torch.randn(1, 64, 4, 7, 128, generator=g).bfloat16()
    idx, scores, _ = O.route_topk(
        q.reshape(1, 35, 4, 7, 128), lm.reshape(1, 64, 28, 128),
        torch.zeros(1, 35, 4, 7), 31, 64, drop_mask=torch.zeros(1, 35, 64, dtype=torch.int32),
        bias4=torch.zeros(1, 64, 4, 7),
    )
    assert bool((idx >= 0).all()) and bool((idx < 64).all())
    assert bool((idx[..., 1:] > idx[..., :-1]).all())
    raw = torch.einsum("bqhgd,bchgd->bqhgc", q.float().reshape(1, 35, 4, 7, 128), lm.float()) / math.sqrt(128)
    expect = torch.gather(raw, -1, idx[:, :, :, None, :].expand(-1, -1, -1, 7, -1))
    torch.testing.assert_close(scores, expect, atol=1e-5, rtol=1e-5)


def test_route_topk_drops_and_padding():
    q5, lmk, lse4, bias4, _ = _inputs(5, C=6)
    drop = torch.zeros(1, 6, 6, dtype=torch.int32)
    drop[:, :, :4] = 1                       # only 2 chunks routable
    idx, scores, _ = O.route_topk(q5, lmk, lse4, 4, 64, drop_mask=drop, bias4=bias4)
    assert bool((idx[..., :2] >= 4).all()) and bool((idx[..., 2:] == -1).all())
    assert bool(torch.isneginf(scores[..., 2:]).all())
    idx8, _, _ = O.route_topk(q5, lmk, lse4, 8, 64, drop_mask=drop, bias4=bias4)   # topk > C
    assert idx8.shape[-1] == 8 and bool((idx8[..., 2:] == -1).all())


def test_route_topk_planted_chunk_and_pre_softmax():
    q5, lmk, lse4, bias4, _ = _inputs(6, C=12)
    bias4 = bias4.clone()
    bias4[:, 7] = 50.0                       # chunk 7 dominates every head
    idx, _, _ = O.route_topk(q5, lmk, lse4, 1, 64, bias4=bias4)
    assert bool((idx == 7).all())
    # pre_softmax with zero bias picks argmax_c max_g q.k
    idx_pre, _, _ = O.route_topk(q5, lmk, None, 1, 64, selection_mode="pre_softmax")
    raw = torch.einsum("blhgd,bchgd->blhgc", q5.float(), lmk.float().reshape(1, 12, 2, 3, 8))
    assert torch.equal(idx_pre[..., 0], raw.max(dim=3).values.argmax(-1))


def test_route_topk_tie_goes_to_lower_index():
    q5 = torch.zeros(1, 2, 1, 2, 8).bfloat16()
    lmk = torch.zeros(1, 10, 2, 8).bfloat16()       # every chunk scores the same
    idx, _, sel = O.route_topk(q5, lmk, torch.zeros(1, 2, 1, 2), 3, 64)
    assert idx[0, 0, 0].tolist() == [0, 1, 2]
    assert bool((O.boundary_gap(sel, 3) == 0).all())


def test_route_weights_sum_and_forms_agree():
    g = torch.Generator().manual_seed(9)
    B, L, H, G, K, C = 1, 5, 2, 7, 8, 20
    scores = torch.randn(B, L, H * G, K, generator=g).bfloat16()
    idx = torch.randint(0, C, (B, L, H, K), generator=g)
    idx[0, 1, 0, 5:] = -1
    bias = torch.rand(B, C, H, G, generator=g)
    lse = torch.randn(B, L, H * G, generator=g)
    rw, lw = O.route_weights(scores, idx, bias, lse)
    # test_value_aware_fusion.py:13-29 -- total mass is one.
    torch.testing.assert_close(rw.sum(-1) + lw, torch.ones_like(lw), atol=1e-5, rtol=0)
    # test_force_remote.py:299-327 -- affine gate at scale 1, offset 0 equals the softmax.
    rw2, lw2 = O.route_weights(scores, idx, bias, lse, gate_offset=0.0, gate_scale=1.0)
    torch.testing.assert_close(rw, rw2, atol=1e-6, rtol=1e-5)
    torch.testing.assert_close(lw, lw2, atol=1e-6, rtol=1e-5)
    assert bool((rw[0, 1, :G, 5:] == 0).all())     # -1 slots carry no weight


def test_route_weights_closed_form_and_all_masked():
    scores = torch.tensor([[[[0.5, 0.0]]]]).bfloat16()        # [1,1,1,2]
    idx = torch.tensor([[[[3, -1]]]])
    bias = torch.zeros(1, 5, 1, 1)
    bias[0, 3] = 0.25
    lse = torch.tensor([[[1.0]]])
    rw, lw = O.route_weights(scores, idx, bias, lse)
    expect_local = 1.0 / (1.0 + math.exp(0.75 - 1.0))
    assert abs(float(lw) - expect_local) < 1e-6 and float(rw[..., 1]) == 0.0
    rw0, lw0 = O.route_weights(scores, torch.full_like(idx, -1), bias,
                               torch.full((1, 1, 1), float("-inf")))
    assert float(rw0.abs().sum()) == 0.0 and float(lw0) == 0.0


def test_route_weights_gate_logit_closed_forms():
    # attention.py:196-235: the gate logit is the log-odds of the remote mass.
    g = torch.Generator().manual_seed(21)
    B, L, H, G, K, C = 1, 6, 2, 7, 8, 20
    scores = torch.randn(B, L, H * G, K, generator=g).bfloat16()
    idx = torch.randint(0, C, (B, L, H, K), generator=g)
    idx[0, 2, 1, 3:] = -1
    bias = torch.rand(B, C, H, G, generator=g)
    lse = torch.randn(B, L, H * G, generator=g)
    # plain form with an offset and a temperature: log(sum remote) - log(local)
    rw, lw, gl = O.route_weights(scores, idx, bias, lse, temperature=0.7, gate_offset=0.3,
                                 return_gate_logit=True)
    torch.testing.assert_close(gl, rw.sum(-1).log() - lw.log(), atol=1e-5, rtol=1e-5)
    # affine form: sigmoid(gate logit) is the remote mass, scale and offset included
    rw, lw, gl = O.route_weights(scores, idx, bias, lse, temperature=1.3, gate_offset=-0.4,
                                 gate_scale=1.7, return_gate_logit=True)
    torch.testing.assert_close(torch.sigmoid(gl), rw.sum(-1), atol=1e-6, rtol=1e-5)
    torch.testing.assert_close(torch.sigmoid(-gl), lw, atol=1e-6, rtol=1e-5)
    # one row by hand: a single remote chunk c=3 (score 0.5, bias 0.25), local 1.0
    s1 = torch.tensor([[[[0.5, 0.0]]]]).bfloat16()
    i1 = torch.tensor([[[[3, -1]]]])
    b1 = torch.zeros(1, 5, 1, 1)
    b1[0, 3] = 0.25
    l1 = torch.tensor([[[1.0]]])
    _, _, g_plain = O.route_weights(s1, i1, b1, l1, gate_offset=0.5, return_gate_logit=True)
    assert abs(float(g_plain) - (0.75 - (1.0 - 0.5))) < 1e-6
    _, _, g_aff = O.route_weights(s1, i1, b1, l1, gate_offset=0.5, gate_scale=2.0,
                                  return_gate_logit=True)
    assert abs(float(g_aff) - (2.0 * (0.75 - 1.0) + 0.5)) < 1e-6
    # every logit masked -> 0; only the remote ones masked -> -inf
    _, _, g0 = O.route_weights(s1, torch.full_like(i1, -1), b1,
                               torch.full((1, 1, 1), float("-inf")), return_gate_logit=True)
    assert float(g0) == 0.0
    _, _, g1 = O.route_weights(s1, torch.full_like(i1, -1), b1, l1, gate_scale=1.5,
                               return_gate_logit=True)
    assert float(g1) == float("-inf")


def test_remote_drop_mask_rows_equal_full_mask_rows():
    g = torch.Generator().manual_seed(5)
    L, S, W = 1024, 64, 256
    valid = torch.rand(2, L, generator=g) > 0.2
    valid[1, 128:192] = False
    pos = torch.tensor([0, 1, 63, 64, 300, 511, 512, 700, 1000, 1023])
    torch.testing.assert_close(O.remote_drop_mask_rows(valid, W, S, pos),
                               O.remote_drop_mask(valid, W, S)[:, pos], rtol=0, atol=0)


def test_route_weights_temperature_closed_form():
    # Two remote chunks and the local branch, by hand: in both forms the two
    # remote weights stand in the ratio exp((x1 - x2) / T) (x = score + bias);
    # the plain form is the 3-way softmax of (x1, x2, lse) / T, the affine
    # form gives the local branch 1 - sigmoid(scale (logsumexp(x / T) -
    # lse / T) + offset).  A missing / T anywhere breaks one of these.
    s = torch.tensor([[[[0.5, -0.25]]]]).bfloat16()
    idx = torch.tensor([[[[1, 3]]]])
    bias = torch.zeros(1, 5, 1, 1)
    bias[0, 1] = 0.125
    bias[0, 3] = -0.375
    lse = torch.tensor([[[0.75]]])
    x1, x2, l = 0.5 + 0.125, -0.25 - 0.375, 0.75
    for T in (0.5, 1.0, 2.5):
        rw, lw = O.route_weights(s, idx, bias, lse, temperature=T)
        e1, e2, el = math.exp(x1 / T), math.exp(x2 / T), math.exp(l / T)
        tot = e1 + e2 + el
        torch.testing.assert_close(rw.flatten(), torch.tensor([e1 / tot, e2 / tot]),
                                   atol=1e-6, rtol=1e-6)
        assert abs(float(lw) - el / tot) < 1e-6
        for off, sc in ((0.3, 1.7), (-0.4, 0.6)):
            rw, lw = O.route_weights(s, idx, bias, lse, temperature=T, gate_offset=off,
                                     gate_scale=sc)
            assert abs(float(rw[..., 0] / rw[..., 1]) - math.exp((x1 - x2) / T)) < 1e-5
            gate = sc * (math.log(e1 + e2) - l / T) + off
            local = 1.0 - 1.0 / (1.0 + math.exp(-gate))
            assert abs(float(lw) - local) < 1e-6
            assert abs(float(rw.sum() + lw) - 1.0) < 1e-6


def test_route_weights_additive_terms_enter_the_remote_logits():
    # attention.py:172-181: value_bonus and selected_gumbel are added to the
    # remote logits after the bias, before the temperature.  With integer
    # values every sum is exact, so a call with the terms equals the call
    # whose bf16 scores already hold them -- in both forms, at T != 1, with
    # masked slots staying masked.  A term added after the temperature, to
    # the local logit, or to a masked slot breaks the equality.
    g = torch.Generator().manual_seed(31)
    B, L, H, G, K, C = 1, 4, 2, 3, 8, 12
    scores = torch.randint(-4, 5, (B, L, H * G, K), generator=g).float()
    vb = torch.randint(-3, 4, scores.shape, generator=g).float()
    gn = torch.randint(-2, 3, scores.shape, generator=g).float()
    idx = torch.randint(0, C, (B, L, H, K), generator=g)
    idx[0, 1, 0, 5:] = -1
    idx[0, 2, 1, 0] = C + 3
    bias = torch.randint(-2, 3, (B, C, H, G), generator=g).float()
    lse = torch.randint(-2, 3, (B, L, H * G), generator=g).float()
    for kw in (dict(temperature=0.5), dict(temperature=2.0, gate_offset=0.25, gate_scale=1.5),
               dict(temperature=1.0, gate_offset=-0.5, return_gate_logit=True)):
        got = O.route_weights(scores.bfloat16(), idx, bias, lse, value_bonus=vb,
                              selected_gumbel=gn, **kw)
        want = O.route_weights((scores + vb + gn).bfloat16(), idx, bias, lse, **kw)
        for a, b in zip(got, want):
            assert torch.equal(a, b)
        one = O.route_weights(scores.bfloat16(), idx, bias, lse, value_bonus=vb, **kw)
        want1 = O.route_weights((scores + vb).bfloat16(), idx, bias, lse, **kw)
        for a, b in zip(one, want1):
            assert torch.equal(a, b)
    assert not torch.equal(got[0], O.route_weights(scores.bfloat16(), idx, bias, lse,
                                                   temperature=1.0, gate_offset=-0.5)[0])
