"""Pins the oracle's token-level refinement (CPU): the global token-keep
selection and the keep mask of the routed chunk attention."""

import torch

from oracle import mrsa_oracle as O


def _brute_keep(row, budget):
    # Python sort by (value descending, index ascending); keep the finite ones.
    order = sorted(range(len(row)), key=lambda i: (-row[i], i))[:budget]
    keep = [0] * len(row)
    for i in order:
        if row[i] != float("-inf"):
            keep[i] = 1
    return keep


def test_select_global_token_keep_brute_force_and_ties():
    g = torch.Generator().manual_seed(1)
    B, L, H, K, S = 1, 3, 2, 4, 8
    scores = torch.randn(B, L, H, K, S, generator=g).round(decimals=1)  # many exact ties
    scores[0, 0, 0, :, -1] = float("-inf")
    scores[0, 1, 1] = float("-inf")                                   # nothing finite
    scores[0, 2, 0, 1:] = float("-inf")                               # fewer finite than budget
    for budget in (1, 5, 12, 40):
        keep = O.select_global_token_keep(scores, budget)
        assert keep.dtype == torch.uint8
        for l in range(L):
            for h in range(H):
                row = scores[0, l, h].reshape(-1).tolist()
                want = _brute_keep(row, min(budget, K * S))
                assert keep[0, l, h].reshape(-1).tolist() == want, (budget, l, h)
                nfin = sum(v != float("-inf") for v in row)
                assert int(keep[0, l, h].sum()) == min(budget, nfin)


def _inputs(Lq, Lk, Hkv, G, D, K, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, Lq, Hkv * G, D, generator=g).bfloat16()
    k = torch.randn(1, Lk, Hkv, D, generator=g).bfloat16()
    v = torch.randn(1, Lk, Hkv, D, generator=g).bfloat16()
    C = Lk // 64
    idx = torch.stack([torch.randperm(C, generator=g)[:K] for _ in range(Lq * Hkv)])
    idx = idx.sort(-1).values.reshape(1, Lq, Hkv, K).int()
    w = torch.softmax(torch.randn(1, Lq, Hkv * G, K, generator=g), -1).bfloat16()
    return q, k, v, idx, w


def test_selected_attention_keep_all_is_identity_and_zero_slot_is_weight_zero():
    q, k, v, idx, w = _inputs(5, 512, 2, 3, 16, 4, 2)
    valid = torch.rand(1, 512, generator=torch.Generator().manual_seed(3)) > 0.1
    base = O.selected_attention(q, k, v, w, idx, valid, 64)
    ones = torch.ones(1, 5, 2, 4, 64, dtype=torch.uint8)
    assert torch.equal(O.selected_attention(q, k, v, w, idx, valid, 64, token_keep=ones), base)
    keep = ones.clone()
    keep[0, 2, 1, 3] = 0                      # query 2, KV head 1, slot 3: nothing kept
    w0 = w.clone()
    w0[0, 2, 3:6, 3] = 0                      # the same slot's weights for that head group
    torch.testing.assert_close(O.selected_attention(q, k, v, w, idx, valid, 64, token_keep=keep),
                               O.selected_attention(q, k, v, w0, idx, valid, 64), atol=1e-6,
                               rtol=0)


def test_selected_attention_one_kept_key_per_slot_closed_form():
    # One kept key per (query, slot): each chunk softmax is 1 on that key, so
    # out[q, h] = sum_k w[q, h, k] * v[c_k * 64 + j_k].
    Lq, Lk, Hkv, G, D, K = 3, 512, 2, 3, 16, 4
    q, k, v, idx, w = _inputs(Lq, Lk, Hkv, G, D, K, 4)
    g = torch.Generator().manual_seed(5)
    pick = torch.randint(0, 63, (1, Lq, Hkv, K), generator=g)       # never the landmark slot
    keep = torch.zeros(1, Lq, Hkv, K, 64, dtype=torch.uint8)
    keep.scatter_(-1, pick[..., None], 1)
    out = O.selected_attention(q, k, v, w, idx, None, 64, token_keep=keep)
    want = torch.zeros(1, Lq, Hkv * G, D)
    for l in range(Lq):
        for h in range(Hkv):
            for s in range(K):
                row = int(idx[0, l, h, s]) * 64 + int(pick[0, l, h, s])
                for gg in range(G):
                    want[0, l, h * G + gg] += float(w[0, l, h * G + gg, s]) * v[0, row, h].float()
    torch.testing.assert_close(out, want, atol=1e-5, rtol=1e-5)
