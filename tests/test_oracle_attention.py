"""Pins the oracle's window attention, routed-chunk attention, fusion and
token scores (CPU)."""

import math

import torch

from oracle import mrsa_oracle as O


def _dense_window_attention(q, k, v, valid, window):
    """Independent dense L x L formulation (full score matrix, then mask)."""

    B, L, Hq, D = q.shape
    Hkv = k.shape[2]
    G = Hq // Hkv
    kz = k.float() * valid[:, :, None, None]
    vz = v.float() * valid[:, :, None, None]
    kr = kz.repeat_interleave(G, dim=2)
    vr = vz.repeat_interleave(G, dim=2)
    s = torch.einsum("bihd,bjhd->bhij", q.float(), kr) / math.sqrt(D)
    i = torch.arange(L)
    mask = (i[:, None] - i[None, :]).abs() <= window
    s = s.masked_fill(~mask, float("-inf"))
    lse = torch.logsumexp(s, dim=-1).permute(0, 2, 1)
    o = torch.einsum("bhij,bjhd->bihd", torch.softmax(s, dim=-1), vr)
    return o, lse


def test_local_attention_matches_dense_formulation():
    g = torch.Generator().manual_seed(11)
    B, L, Hkv, G, D = 1, 256, 2, 3, 32
    q = torch.randn(B, L, Hkv * G, D, generator=g).bfloat16()
    k = torch.randn(B, L, Hkv, D, generator=g).bfloat16()
    v = torch.randn(B, L, Hkv, D, generator=g).bfloat16()
    valid = torch.rand(B, L, generator=g) > 0.1
    inert = valid & ((torch.arange(L) + 1) % 64 != 0)[None]
    for window, chunk in ((37, 64), (300, 0)):
        eff_valid = inert if chunk else valid
        out, lse = O.local_attention(q, k, v, valid, window, chunk, query_block=48)
        ref_o, ref_l = _dense_window_attention(q, k, v, eff_valid, window)
        torch.testing.assert_close(out, ref_o, atol=2e-5, rtol=1e-4)
        torch.testing.assert_close(lse, ref_l, atol=2e-5, rtol=1e-5)


def test_local_attention_inert_keys_stay_in_denominator():
    # Two keys in reach; key 1 is a landmark slot (zero K/V): lse = log(e^s0 + e^0).
    q = torch.zeros(1, 2, 1, 4)
    q[0, 0, 0, 0] = 2.0
    k = torch.zeros(1, 2, 1, 4)
    k[0, 0, 0, 0] = 1.0
    k[0, 1, 0, 0] = 5.0            # ignored: zeroed as inert
    v = torch.ones(1, 2, 1, 4)
    out, lse = O.local_attention(q.bfloat16(), k.bfloat16(), v.bfloat16(), None, 1, 2)
    s0 = 2.0 * 1.0 / math.sqrt(4)
    assert abs(float(lse[0, 0, 0]) - math.log(math.exp(s0) + 1.0)) < 1e-6
    p0 = math.exp(s0) / (math.exp(s0) + 1.0)
    torch.testing.assert_close(out[0, 0, 0], torch.full((4,), p0), atol=1e-6, rtol=0)


def test_local_attention_positions_select_rows():
    g = torch.Generator().manual_seed(12)
    q = torch.randn(1, 128, 2, 16, generator=g).bfloat16()
    k = torch.randn(1, 128, 1, 16, generator=g).bfloat16()
    v = torch.randn(1, 128, 1, 16, generator=g).bfloat16()
    full_o, full_l = O.local_attention(q, k, v, None, 20, 16)
    pos = torch.tensor([3, 64, 99, 127])
    o, l = O.local_attention(q[:, pos], k, v, None, 20, 16, query_positions=pos)
    torch.testing.assert_close(o, full_o[:, pos], atol=1e-6, rtol=1e-6)
    torch.testing.assert_close(l, full_l[:, pos], atol=1e-6, rtol=1e-6)


def test_selected_attention_reference_kat():
    # Restates test_hils_non_power_two_topk.py:95-142 (uncached, unfiltered).
    g = torch.Generator().manual_seed(79)
    query_len, kv_len, h_kv, grp, dim, topk, size = 64, 2048, 4, 7, 128, 31, 64
    q = torch.randn(1, query_len, h_kv * grp, dim, generator=g).bfloat16()
    k = torch.randn(1, kv_len, h_kv, dim, generator=g).bfloat16()
    v = torch.randn(1, kv_len, h_kv, dim, generator=g).bfloat16()
    indices = torch.arange(topk, dtype=torch.int32).expand(1, query_len, h_kv, -1).clone()
    indices[:, 0] = -1
    weights = torch.randn(1, query_len, h_kv * grp, topk, generator=g).softmax(-1).bfloat16()
    weights[:, 0] = 0
    valid = torch.ones(1, kv_len, dtype=torch.bool)
    valid[:, ::97] = False
    actual = O.selected_attention(q, k, v, weights, indices, valid, size)
    assert torch.equal(actual[:, 0], torch.zeros_like(actual[:, 0]))
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
        probs = logits.masked_fill(~allowed[:, :, None], float("-inf")).softmax(-1)
        expected += torch.einsum("rhgs,shd->rhgd", probs, vs) * ws[..., chunk, None]
    observed = actual[0, rows].reshape_as(expected)
    torch.testing.assert_close(observed, expected, atol=1e-5, rtol=1e-4)


def test_selected_attention_identical_chunks_and_list_end():
    g = torch.Generator().manual_seed(13)
    chunk_k = torch.randn(64, 1, 16, generator=g)
    chunk_v = torch.randn(64, 1, 16, generator=g)
    k = chunk_k.repeat(4, 1, 1)[None].bfloat16()     # 4 identical chunks
    v = chunk_v.repeat(4, 1, 1)[None].bfloat16()
    q = torch.randn(1, 3, 2, 16, generator=g).bfloat16()
    idx = torch.tensor([[[[0, 2, 3]], [[1, -1, 3]], [[-1, 0, 1]]]], dtype=torch.int32)
    w = torch.full((1, 3, 2, 3), 0.25).bfloat16()
    out = O.selected_attention(q, k, v, w, idx, None, 64)
    single = O.selected_attention(q, k, v, torch.ones(1, 3, 2, 1).bfloat16(),
                                  torch.zeros(1, 3, 1, 1, dtype=torch.int32), None, 64)
    torch.testing.assert_close(out[0, 0], 0.75 * single[0, 0], atol=1e-6, rtol=1e-5)
    # A list ends at its first negative entry (hils_fwd_bwd_head.py:352-361).
    torch.testing.assert_close(out[0, 1], 0.25 * single[0, 1], atol=1e-6, rtol=1e-5)
    assert torch.equal(out[0, 2], torch.zeros_like(out[0, 2]))


def test_fuse_outputs_closed_form():
    g = torch.Generator().manual_seed(14)
    r = torch.randn(2, 8, 3, 16, generator=g).bfloat16()
    lo = torch.randn(2, 8, 3, 16, generator=g).bfloat16()
    w = torch.rand(2, 8, 3, generator=g).bfloat16()
    out = O.fuse_outputs(r, lo, w)
    expect = (r.double() + w.double()[..., None] * lo.double()).float().bfloat16()
    assert (out.float() - expect.float()).abs().max() <= 2 ** -7 * expect.float().abs().max()


def test_candidate_token_scores_closed_form():
    g = torch.Generator().manual_seed(15)
    q = torch.randn(1, 3, 6, 16, generator=g).bfloat16()
    k = torch.randn(1, 256, 2, 16, generator=g).bfloat16()
    idx = torch.tensor([[[[1, -1], [3, 0]]] * 3], dtype=torch.int32).reshape(1, 3, 2, 2)
    valid = torch.ones(1, 256, dtype=torch.bool)
    valid[0, 64 + 5] = False
    s = O.candidate_token_scores(q, k, idx, valid, 64)
    assert bool(torch.isneginf(s[:, :, 0, 1]).all())          # -1 chunk
    assert bool(torch.isneginf(s[..., 63]).all())              # landmark slot
    assert bool(torch.isneginf(s[0, :, 0, 0, 5]).all())        # invalid key
    qq = q[0, 1].float().reshape(2, 3, 16)
    kk = k[0, 3 * 64 + 7, 1].float()
    assert abs(float(s[0, 1, 1, 0, 7]) - float((qq[1] @ kk).max() / 4.0)) < 1e-5


def test_selected_attention_alibi_closed_form():
    # q = 0 leaves only the ALiBi term: chunk key s has logit
    # -slope[head] * max(0, 62 - s) * scale (hils_torch_ref :68-78: bias
    # before the scale, the last key masked), and one-hot values e_s make the
    # output the softmax itself.  Distinct slopes per head pin the head order;
    # scale = 1/8 (D = 64) separates "bias then scale" from "scale then bias".
    D, S, Hkv, G = 64, 64, 2, 2
    slope = torch.tensor([0.5, 0.125, 1.0, 0.03125])
    q = torch.zeros(1, 1, Hkv * G, D).bfloat16()
    k = torch.randn(1, S, Hkv, D, generator=torch.Generator().manual_seed(21)).bfloat16()
    v = torch.eye(S, D)[None, :, None, :].repeat(1, 1, Hkv, 1).bfloat16()
    idx = torch.zeros(1, 1, Hkv, 1, dtype=torch.int32)
    w = torch.ones(1, 1, Hkv * G, 1).bfloat16()
    out = O.selected_attention(q, k, v, w, idx, None, S, slope=slope)
    s = torch.arange(S, dtype=torch.float64)
    for h in range(Hkv * G):
        logit = -slope[h].double() * (62 - s).clamp(min=0) / math.sqrt(D)
        logit[-1] = float("-inf")
        expect = torch.softmax(logit, dim=0)
        torch.testing.assert_close(out[0, 0, h].double(), expect, atol=1e-6, rtol=1e-5)
    # with the last key visible, keys 62 and 63 both sit at distance 0 (a
    # shifted distance would only move the visible logits together above)
    out = O.selected_attention(q, k, v, w, idx, None, S, mask_last_token=False, slope=slope)
    for h in range(Hkv * G):
        logit = -slope[h].double() * (62 - s).clamp(min=0) / math.sqrt(D)
        torch.testing.assert_close(out[0, 0, h].double(), torch.softmax(logit, dim=0),
                                   atol=1e-6, rtol=1e-5)
    # slope 0 is the plain attention, bit for bit
    q2 = torch.randn(1, 3, Hkv * G, D, generator=torch.Generator().manual_seed(22)).bfloat16()
    plain = O.selected_attention(q2, k, v, w.repeat(1, 3, 1, 1), idx.repeat(1, 3, 1, 1), None, S)
    zero = O.selected_attention(q2, k, v, w.repeat(1, 3, 1, 1), idx.repeat(1, 3, 1, 1), None, S,
                                slope=torch.zeros(Hkv * G))
    assert torch.equal(plain, zero)
