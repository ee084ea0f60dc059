"""Pins the oracle's landmark pool and drop mask (CPU).

Each check is independent of the oracle's vectorised formula: closed forms,
invariants, special cases and brute-force loops on tiny inputs.
"""

import math

import pytest
import torch

from oracle import mrsa_oracle as O


def _brute_pool(mu_q, k, valid, scale, dense):
    """Pure-Python loops over one tiny problem (no einsum, no torch.softmax)."""

    B, C, H, G, D = mu_q.shape
    S = k.shape[2]
    lmk = torch.zeros(B, C, H, G, D)
    ent = torch.zeros(B, C, H, G)
    for b in range(B):
        for c in range(C):
            real = [bool(valid[b, c, s]) and s < S - 1 for s in range(S)]
            chunk_ok = any(real)
            for h in range(H):
                for g in range(G):
                    logits = []
                    for s in range(S):
                        dot = sum(float(mu_q[b, c, h, g, d]) * float(k[b, c, s, h, d]) for d in range(D))
                        if dense:
                            logits.append(dot * scale if real[s] else -math.inf)
                        elif real[s] and chunk_ok:
                            logits.append(dot * scale)
                        else:
                            logits.append(0.0 if s == 0 else -math.inf)
                    m = max(logits)
                    if m == -math.inf:
                        p = [0.0] * S
                    else:
                        e = [math.exp(x - m) if x != -math.inf else 0.0 for x in logits]
                        tot = sum(e)
                        p = [x / tot for x in e]
                    if not dense and not chunk_ok:
                        continue
                    ent[b, c, h, g] = -sum(x * math.log(x) for x in p if x > 0)
                    for d in range(D):
                        acc = 0.0
                        for s in range(S):
                            w = p[s] if dense else float(torch.tensor(p[s]).to(torch.bfloat16).float())
                            acc += w * float(k[b, c, s, h, d])
                        lmk[b, c, h, g, d] = acc
    return lmk, ent


@pytest.mark.parametrize("dense", [False, True])
def test_pool_matches_brute_force(dense):
    g = torch.Generator().manual_seed(3)
    B, C, H, G, S, D = 1, 3, 2, (1 if dense else 3), 8, 4
    mu = torch.randn(B, C, H, G, D, generator=g).bfloat16()
    k = torch.randn(B, C, S, H, D, generator=g).bfloat16()
    valid = torch.rand(B, C, S, generator=g) > 0.3
    valid[0, 1, :] = False          # fully invalid chunk
    valid[0, 2, 0] = False          # masked slot 0 in a valid chunk (logit-0 quirk)
    valid[0, 2, 1] = True
    lmk, ent = O.chunk_attn_pool(mu, k, valid, 0.5, dense=dense)
    bl, be = _brute_pool(mu, k, valid, 0.5, dense)
    torch.testing.assert_close(lmk, bl, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(ent, be, atol=1e-5, rtol=1e-5)


def test_pool_uniform_logits_closed_form():
    # mu_q = 0 -> every real logit is 0 -> p = 1/63 over slots 0..62.
    g = torch.Generator().manual_seed(0)
    mu = torch.zeros(1, 2, 4, 7, 128).bfloat16()
    k = torch.randn(1, 2, 64, 4, 128, generator=g).bfloat16()
    valid = torch.ones(1, 2, 64, dtype=torch.bool)
    lmk, ent = O.chunk_attn_pool(mu, k, valid)
    p = torch.tensor(1.0 / 63).to(torch.bfloat16).float()
    expect = p * k.float()[:, :, :63].sum(dim=2)        # [1, 2, 4, 128]
    torch.testing.assert_close(lmk, expect[:, :, :, None].expand_as(lmk), atol=1e-4, rtol=1e-5)
    torch.testing.assert_close(ent, torch.full_like(ent, math.log(63)), atol=1e-5, rtol=0)


def test_pool_ignores_landmark_slot_and_bounds_entropy():
    g = torch.Generator().manual_seed(1)
    mu = torch.randn(1, 4, 4, 7, 128, generator=g).bfloat16()
    k = torch.randn(1, 4, 64, 4, 128, generator=g).bfloat16()
    valid = torch.ones(1, 4, 64, dtype=torch.bool)
    lmk1, ent1 = O.chunk_attn_pool(mu, k, valid)
    k2 = k.clone()
    k2[:, :, 63] = 100.0          # slot 63 must carry zero weight
    lmk2, ent2 = O.chunk_attn_pool(mu, k2, valid)
    assert torch.equal(lmk1, lmk2) and torch.equal(ent1, ent2)
    assert bool((ent1 >= 0).all()) and bool((ent1 <= math.log(63) + 1e-5).all())


def test_pool_invalid_chunk_is_zero_and_quirk_slot0():
    g = torch.Generator().manual_seed(2)
    mu = torch.randn(1, 2, 1, 2, 16, generator=g).bfloat16()
    k = torch.randn(1, 2, 8, 1, 16, generator=g).bfloat16()
    valid = torch.ones(1, 2, 8, dtype=torch.bool)
    valid[0, 0, :7] = False       # only the landmark slot valid -> chunk invalid
    valid[0, 1, 0] = False        # slot 0 masked but chunk valid -> logit 0 at slot 0
    lmk, ent = O.chunk_attn_pool(mu, k, valid, 1.0)
    assert torch.equal(lmk[0, 0], torch.zeros_like(lmk[0, 0]))
    assert torch.equal(ent[0, 0], torch.zeros_like(ent[0, 0]))
    # Kernel quirk: slot 0 keeps logit 0 instead of -inf.
    q = mu[0, 1, 0].float()
    kk = k[0, 1, :, 0].float()
    logits = torch.cat([torch.zeros(2, 1), (q @ kk[1:7].T)], dim=1)
    p = torch.softmax(logits, dim=1)
    expect = (p.bfloat16().float() @ kk[:7])
    torch.testing.assert_close(lmk[0, 1, 0], expect, atol=1e-5, rtol=1e-5)


def test_pool_single_head_matches_softmax_attention():
    # G == 1 (dense torch twin): plain masked softmax attention over real keys.
    g = torch.Generator().manual_seed(4)
    mu = torch.randn(1, 3, 2, 1, 32, generator=g).bfloat16()
    k = torch.randn(1, 3, 16, 2, 32, generator=g).bfloat16()
    valid = torch.ones(1, 3, 16, dtype=torch.bool)
    lmk, _ = O.chunk_attn_pool(mu, k, valid, 0.25)
    for c in range(3):
        for h in range(2):
            kk = k[0, c, :15, h].float()
            p = torch.softmax(0.25 * (kk @ mu[0, c, h, 0].float()), dim=0)
            torch.testing.assert_close(lmk[0, c, h, 0], p @ kk, atol=1e-5, rtol=1e-5)


def _brute_drop(valid, W, S):
    B, L = valid.shape
    C = L // S
    out = torch.zeros(B, L, C, dtype=torch.int32)
    for b in range(B):
        chunk_ok = [any(bool(valid[b, c * S + s]) for s in range(S - 1)) for c in range(C)]
        for i in range(L):
            left = (max(i - W, 0) // S) * S
            right = min(((min(i + W, L - 1) // S) + 1) * S, L)
            for c in range(C):
                overlap = max(c * S, left) < min((c + 1) * S, right)
                out[b, i, c] = int(overlap or not chunk_ok[c])
    return out


def test_drop_mask_brute_force_and_nine_local_chunks():
    L, S, W = 1024, 64, 256
    valid = torch.ones(1, L, dtype=torch.bool)
    valid[0, 3 * 64: 3 * 64 + 63] = False      # chunk 3: only its landmark slot valid
    drop = O.remote_drop_mask(valid, W, S)
    assert torch.equal(drop, _brute_drop(valid, W, S))
    # Interior queries always drop exactly 9 chunk-aligned local chunks.
    local_count = O.remote_drop_mask(torch.ones(1, L, dtype=torch.bool), W, S)[0].sum(-1)
    assert bool((local_count[W + 64: L - W - 64] == 9).all())
    assert bool((drop[0, :, 3] == 1).all())


def test_drop_mask_allowed_mask():
    L, S = 256, 64
    valid = torch.ones(1, L, dtype=torch.bool)
    allowed = torch.ones(1, L, L, dtype=torch.bool)
    allowed[0, 10, 3 * 64 + 63] = False       # query 10 may not see chunk 3's landmark
    drop = O.remote_drop_mask(valid, 0, S, allowed)
    assert drop[0, 10, 3] == 1 and drop[0, 11, 3] == 0
