"""Pins the oracle's cached route-layer step (CPU).

A query block decoded against a cache that holds the full inputs must
reproduce the oracle's prefill rows for that block: the same window
attention, routing and weights, once the stale landmark summary of the
block's chunk has been refreshed.  A wrong row <-> position mapping, drop-row
selection or refresh fails it.  Both sides use the plain 33-way weights (no
fusion gate), as the reference decode path does
(dream_dllm_hils/fastdllm_attention.py:315-323).
"""

import torch

from oracle import mrsa_oracle as O


def _inputs(L, Hq, Hkv, D, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, L, Hq, D, generator=g).bfloat16()
    rq = torch.randn(1, L, Hq, D, generator=g).bfloat16()
    k = torch.randn(1, L, Hkv, D, generator=g)
    shift = 0.3 * torch.randn(L // 64, Hkv, D, generator=g)
    k = (k + shift.repeat_interleave(64, dim=0)[None]).bfloat16()
    v = torch.randn(1, L, Hkv, D, generator=g).bfloat16()
    return q, rq, k, v


def _prefill(q, k, v, rq, scale, valid, W, S, K):
    return O.route_layer(q, k, v, rq, scale, valid, local_window=W, chunk_size=S, topk=K,
                         gate_offset=None, gate_scale=None)


def test_cached_block_reproduces_prefill_rows_after_refresh():
    L, Hq, Hkv, D, S, W, K = 1024, 14, 2, 32, 64, 64, 4
    q, rq, k, v = _inputs(L, Hq, Hkv, D, 5)
    valid = torch.ones(1, L, dtype=torch.bool)
    valid[0, 100:103] = False
    scale = torch.rand(Hq, generator=torch.Generator().manual_seed(6)) + 0.5
    ref, mid = _prefill(q, k, v, rq, scale, valid, W, S, K)
    chunk = 8
    rows = torch.arange(chunk * S, (chunk + 1) * S)
    stale_lmk = mid["landmark_keys"].clone()
    stale_prior = mid["prior_bias"].clone()
    stale_lmk[:, chunk] = 0
    stale_prior[:, chunk] = 0
    out, lmk, prior, cmid = O.cached_route_layer(
        q[:, rows], rq[:, rows], k, v, valid, stale_lmk, stale_prior, rows,
        torch.tensor([chunk]), scale, local_window=W, chunk_size=S, topk=K)
    # Refreshed chunk equals the prefill's summary; the others are untouched.
    torch.testing.assert_close(lmk.float(), mid["landmark_keys"].float(), atol=1e-2, rtol=0)
    torch.testing.assert_close(prior, mid["prior_bias"], atol=1e-4, rtol=1e-4)
    others = torch.arange(L // S) != chunk
    assert torch.equal(lmk[:, others], stale_lmk[:, others])
    agree = (cmid["indices"] == mid["indices"][:, rows]).all(-1).float().mean()
    assert float(agree) >= 0.98
    err = (out.float() - ref[:, rows].float()).abs()
    assert float(err.max()) <= 2e-2 and float(err.mean()) <= 1e-3


def test_cached_block_drop_rows_follow_positions():
    # Unaligned, non-contiguous query positions: the drop rows are the full
    # mask's rows at those positions, and no landmark changes without
    # affected chunks.
    L, Hq, Hkv, D, S, W, K = 768, 7, 1, 32, 64, 64, 3
    q, rq, k, v = _inputs(L, Hq, Hkv, D, 9)
    valid = torch.ones(1, L, dtype=torch.bool)
    scale = torch.ones(Hq)
    ref, mid = _prefill(q, k, v, rq, scale, valid, W, S, K)
    rows = torch.tensor([5, 130, 131, 400, 767])
    out, lmk, prior, cmid = O.cached_route_layer(
        q[:, rows], rq[:, rows], k, v, valid, mid["landmark_keys"], mid["prior_bias"], rows,
        torch.tensor([], dtype=torch.long), scale, local_window=W, chunk_size=S, topk=K)
    assert torch.equal(cmid["drop_mask"], O.remote_drop_mask(valid, W, S)[:, rows])
    assert torch.equal(lmk, mid["landmark_keys"])
    assert torch.equal(cmid["indices"], mid["indices"][:, rows])
    err = (out.float() - ref[:, rows].float()).abs()
    assert float(err.max()) <= 2e-2
