"""Pins of the oracle's entropy-adaptive token policy
(dream_dllm_hils/token_refinement.py:150-333) on the CPU.

The reference has no unit test for this policy.  The allocation is pinned by
its invariants, by Hamilton's largest-remainder method computed in exact
rational arithmetic (which the capped procedure reduces to when no capacity
binds), by the uniform-support closed form and by a capped case; the keep
mask by a brute-force sort; the entropy gather by loops.
"""

import math
from fractions import Fraction

import torch

from oracle import mrsa_oracle as O


def test_gather_selected_chunk_entropy_brute_force():
    g = torch.Generator().manual_seed(1)
    B, C, H, G, L, K = 2, 9, 3, 7, 4, 5
    ent = torch.rand(B, C, H, G, generator=g) * 3
    idx = torch.randint(-1, C + 2, (B, L, H, K), generator=g)
    got = O.gather_selected_chunk_entropy(ent, idx)
    for b in range(B):
        for l in range(L):
            for h in range(H):
                for k in range(K):
                    c = int(idx[b, l, h, k])
                    exp = 0.0 if c < 0 else float(ent[b, min(c, C - 1), h].mean())
                    assert abs(float(got[b, l, h, k]) - exp) < 1e-6


def _rows(seed, R=200, K=8, cap_lo=1, cap_hi=64):
    g = torch.Generator().manual_seed(seed)
    ent = torch.rand(R, K, generator=g) * 4 - 0.5
    cap = torch.randint(cap_lo, cap_hi + 1, (R, K), generator=g)
    return ent, cap


def test_allocation_invariants():
    for budget, mn in ((40, 1), (100, 2), (500, 0), (8, 1)):
        ent, cap = _rows(2)
        cap[::7, 3] = 0  # empty chunks
        alloc = O.allocate_entropy_token_budget(ent, cap, budget, mn)
        target = cap.sum(-1).clamp_max(budget)
        assert torch.equal(alloc.sum(-1), target)
        assert bool((alloc <= cap).all())
        assert bool((alloc >= torch.minimum(cap, torch.full_like(cap, mn))).all())


def _hamilton(support, baseline, R):
    """Largest remainder in exact rationals: floor(R s_k / sum s) plus one
    for the largest fractional parts (ties to the lower index)."""
    tot = sum(support)
    quota = [Fraction(R) * s / tot for s in support]
    base = [math.floor(x) for x in quota]
    frac = [x - b for x, b in zip(quota, base)]
    left = R - sum(base)
    order = sorted(range(len(support)), key=lambda k: (-frac[k], k))
    out = [b0 + b for b0, b in zip(baseline, base)]
    for k in order[:left]:
        out[k] += 1
    near = min(min(abs(x - round(x)) for x in quota), 1)
    return out, near


def test_allocation_is_largest_remainder_when_no_capacity_binds():
    budget, mn, K = 96, 1, 8
    ent, _ = _rows(3, R=300, K=K)
    cap = torch.full((300, K), 1000)  # above any quota: no capacity binds
    alloc = O.allocate_entropy_token_budget(ent, cap, budget, mn)
    max_e = math.log(budget)
    checked = 0
    for r in range(ent.shape[0]):
        sup = [Fraction(float(torch.exp(torch.tensor(min(max(float(e), 0.0), max_e))))) for e in ent[r]]
        exp, near = _hamilton(sup, [mn] * K, budget - K * mn)
        if near < Fraction(1, 10 ** 4):
            continue  # fp32 quota within rounding of an integer
        assert alloc[r].tolist() == exp, r
        checked += 1
    assert checked > 250


def test_allocation_uniform_support_closed_form():
    # equal supports (entropy 0 -> support exactly 1): every chunk gets
    # floor(R / K) and the first R mod K chunks one more
    K, budget, mn = 6, 40, 2
    ent = torch.zeros(3, K)
    cap = torch.full((3, K), 64)
    alloc = O.allocate_entropy_token_budget(ent, cap, budget, mn)
    R = budget - K * mn
    exp = [mn + R // K + (1 if k < R % K else 0) for k in range(K)]
    assert alloc.tolist() == [exp] * 3


def test_allocation_capped_chunk_is_filled_and_rest_redistributed():
    K, budget = 4, 60
    ent = torch.tensor([[5.0, 0.0, 0.0, 0.0]])  # chunk 0 wants most slots
    cap = torch.tensor([[3, 64, 64, 64]])
    alloc = O.allocate_entropy_token_budget(ent, cap, budget, 1)
    assert int(alloc[0, 0]) == 3
    assert int(alloc.sum()) == budget
    # the other three have equal support: 57 slots split 19 each
    assert alloc[0, 1:].tolist() == [19, 19, 19]


def test_allocation_nonfinite_entropy():
    budget = 32
    ent = torch.tensor([[float("nan"), float("inf"), float("-inf"), 0.0]])
    cap = torch.full((1, 4), 64)
    alloc = O.allocate_entropy_token_budget(ent, cap, budget, 0)
    # supports 1, budget, 1, 1: quotas 32 * [1, 32, 1, 1] / 35
    sup = [Fraction(1), Fraction(float(torch.exp(torch.tensor(math.log(budget))))), Fraction(1),
           Fraction(1)]
    exp, _ = _hamilton(sup, [0] * 4, budget)
    assert alloc[0].tolist() == exp


def test_entropy_keep_is_top_allocation_per_chunk():
    g = torch.Generator().manual_seed(5)
    B, L, H, K, S = 1, 6, 2, 5, 64
    scores = torch.randn(B, L, H, K, S, generator=g)
    scores[torch.rand(B, L, H, K, S, generator=g) < 0.3] = float("-inf")
    scores[0, 0, 0, 1, 10:20] = 0.25  # ties: lower key first
    ent = torch.rand(B, L, H, K, generator=g) * 3
    keep, alloc = O.select_entropy_adaptive_token_keep(scores, ent, 100, 1)
    for l in range(L):
        for h in range(H):
            for k in range(K):
                row = scores[0, l, h, k].tolist()
                order = sorted(range(S), key=lambda s: (-row[s], s))
                a = int(alloc[0, l, h, k])
                want = set(s for s in order[:a] if math.isfinite(row[s]))
                got = set(torch.nonzero(keep[0, l, h, k]).flatten().tolist())
                assert got == want, (l, h, k)
                assert a <= sum(math.isfinite(x) for x in row)
