"""GPU parity: every gfx950 kernel against the CPU oracle on seeded inputs.

Tolerances (from the build target): routing indices bit-exact except rows
whose oracle top-k boundary gap is below 1e-5 (reported); attention outputs
within max-abs 2e-2 and mean-abs 2e-3 (bf16 in, fp32 accumulate).
"""

import math
import os

import pytest
import torch

import mrsa
from mrsa import _lib
from mrsa.local_attention import local_attention_launch
from mrsa.route_weights import route_weights_launch
from mrsa.sparse_attention import selected_attention_launch
from mrsa.topk import route_topk_launch
from oracle import mrsa_oracle as O
from routing_check import assert_nearly_identical, classify_routing

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
NEAR_TIE = 1e-5


def _note(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g) * scale


def _planted_kv(L, Hkv, D, seed, sigma=0.3):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(1, L, Hkv, D, generator=g)
    shift = sigma * torch.randn(-(-L // 64), Hkv, D, generator=g)
    k = k + shift.repeat_interleave(64, dim=0)[None, :L]
    v = torch.randn(1, L, Hkv, D, generator=g)
    return k.bfloat16(), v.bfloat16()


def _assert_close_attn(actual, expected, what):
    err = (actual.float().cpu() - expected.float()).abs()
    print(f"{what}: max_abs={err.max():.3e} mean_abs={err.mean():.3e}", flush=True)
    assert float(err.max()) <= 2e-2, what
    assert float(err.mean()) <= 2e-3, what


def _assert_lmk_close(actual, expected, what):
    # Landmark keys are bf16 outputs of a pool that weights the keys with
    # bf16-rounded probabilities (ops/chunk_attn_pool_gqa_tilelang.py:151-158):
    # a probability at a rounding midpoint can round the other way, so a rare
    # element moves by more than one output step.  Bound as test_pool_vs_oracle
    # does (1e-2 abs / rel, mean below 1e-4) and require 99% of the elements
    # to equal the oracle's value after its bf16 rounding.
    a = actual.float().cpu()
    er = expected.float().bfloat16().float()
    err = (a - er).abs()
    frac_same = float((err == 0).float().mean())
    print(f"{what}: max_abs={err.max():.3e} mean_abs={err.mean():.3e} "
          f"same_after_rounding={frac_same:.4f}", flush=True)
    torch.testing.assert_close(a, er, atol=1e-2, rtol=1e-2, msg=what)
    assert float(err.mean()) <= 1e-4, what
    assert frac_same > 0.99, what


def test_mfma_lane_layout():
    _note("mfma layout")
    a = _rand((16, 32), 1).bfloat16()
    b = _rand((32, 16), 2).bfloat16()
    c = torch.empty(16, 16, device=DEV)
    ad, bd = a.to(DEV), b.to(DEV)
    _lib.check(_lib.call("mrsa_selftest_mfma_layout", ad.data_ptr(), bd.data_ptr(),
                         c.data_ptr(), _lib.stream_of(c)), "selftest")
    torch.cuda.synchronize()
    torch.testing.assert_close(c.cpu(), a.float() @ b.float(), atol=1e-4, rtol=1e-4)


def test_fusion_bit_exact():
    _note("fusion")
    r = _rand((1, 300, 28, 128), 3).bfloat16()
    lo = _rand((1, 300, 28, 128), 4).bfloat16()
    w = torch.rand(1, 300, 28).bfloat16()
    out = mrsa.fuse_hils_outputs(r.to(DEV), lo.to(DEV), w.to(DEV))
    assert torch.equal(out.cpu(), O.fuse_outputs(r, lo, w))
    out2 = mrsa.fuse_hils_outputs(r[..., :100].contiguous().to(DEV), lo[..., :100].contiguous().to(DEV),
                                  w.to(DEV))   # scalar path (head_dim % 8 != 0)
    assert torch.equal(out2.cpu(), O.fuse_outputs(r[..., :100], lo[..., :100], w))


def test_drop_mask_bit_exact():
    _note("drop mask")
    L = 2048
    valid = torch.rand(2, L) > 0.02
    valid[1, 5 * 64: 5 * 64 + 63] = False
    allowed = torch.rand(2, L, L) > 0.001
    for W, al in ((256, None), (100, allowed)):
        got = mrsa.remote_drop_mask(valid.to(DEV), W, 64, None if al is None else al.to(DEV))
        assert torch.equal(got.cpu(), O.remote_drop_mask(valid, W, 64, al))


def _fragments_expected(k, v):
    # The operand images written out from their definition: K part
    # f[4 mt + ks][16 grp + j][e] = K[16 mt + j][32 ks + 8 grp + e]; V part
    # f[2 nt + ks][16 grp + j][4 b + e'] = V[32 ks + 16 b + 4 grp + e'][16 nt + j].
    B, L, H, D = k.shape
    C = (L + 63) // 64
    kp = torch.zeros(B, C * 64, H, D, dtype=k.dtype)
    vp = torch.zeros(B, C * 64, H, D, dtype=k.dtype)
    kp[:, :L] = k
    if v is not None:
        vp[:, :L] = v
    kc = kp.reshape(B, C, 64, H, D).permute(0, 3, 1, 2, 4)       # [B, H, C, key, dim]
    vc = vp.reshape(B, C, 64, H, D).permute(0, 3, 1, 2, 4)
    kf = kc.reshape(B, H, C, 4, 16, 4, 4, 8).permute(0, 1, 2, 3, 5, 6, 4, 7)
    vf = vc.reshape(B, H, C, 2, 2, 4, 4, 8, 16).permute(0, 1, 2, 7, 3, 5, 8, 4, 6)
    return torch.cat([kf.reshape(B, H, C, 8192), vf.reshape(B, H, C, 8192)], dim=-1)


def test_kv_fragments_layout():
    # Keys past the end (L = 200: the last chunk has 8 real keys) are zero,
    # and without v the V half is zero.
    _note("kv fragments")
    k = _rand((2, 200, 3, 128), 8).bfloat16()
    v = _rand((2, 200, 3, 128), 9).bfloat16()
    got = mrsa.kv_fragments(k.to(DEV), v.to(DEV)).cpu()
    assert torch.equal(got.view(torch.int16), _fragments_expected(k, v).view(torch.int16))
    got = mrsa.kv_fragments(k.to(DEV)).cpu()
    assert torch.equal(got.view(torch.int16), _fragments_expected(k, None).view(torch.int16))


@pytest.mark.parametrize("G,dense", [(7, False), (1, True), (3, False)])
def test_pool_vs_oracle(G, dense):
    _note(f"pool G={G}")
    B, C, H, S, D = 2, 40, 4, 64, 128
    mu = _rand((B, C, H, G, D), 6).bfloat16()
    k = _rand((B, C, S, H, D), 7).bfloat16()
    valid = torch.rand(B, C, S) > 0.1
    valid[0, 3] = False
    valid[1, 4, :63] = False
    valid[1, 5, 0] = False
    scale = torch.rand(H * G) + 0.5
    lmk, ent, prior = mrsa.chunk_attn_pool_gqa_prior(mu.to(DEV), k.to(DEV), valid.to(DEV), scale.to(DEV))
    rl, re = O.chunk_attn_pool(mu, k, valid)
    torch.testing.assert_close(lmk.cpu().float(), rl.bfloat16().float(), atol=1e-2, rtol=1e-2)
    assert (lmk.cpu().float() - rl.bfloat16().float()).abs().mean() < 1e-4
    torch.testing.assert_close(ent.cpu(), re, atol=2e-5, rtol=1e-5)
    torch.testing.assert_close(prior.cpu(), re * scale.view(1, 1, H, G), atol=5e-5, rtol=1e-5)
    lmk2, ent2 = mrsa.chunk_attn_pool_gqa(mu.to(DEV), k.to(DEV), valid.to(DEV))
    assert torch.equal(lmk2, lmk) and torch.equal(ent2, ent)


@pytest.mark.parametrize("B,L,H,G", [(1, 2048, 4, 7), (2, 640, 3, 16), (1, 320, 2, 2),
                                     (2, 1024, 1, 8)])
def test_kv_fragments_pool_equals_the_two_ops(B, L, H, G):
    # One pass over the keys: the same fragments and the same pool outputs,
    # bit for bit, as kv_fragments + chunk_attn_pool_gqa_prior, with the
    # landmark query rows read in place from the route queries; invalid keys,
    # a fully invalid chunk and an invalid landmark slot included.
    _note(f"kv fragments + pool in one pass B={B} L={L} H={H} G={G}")
    from mrsa.pool import kv_fragments_pool
    D, C = 128, L // 64
    k = _rand((B, L, H, D), 11).bfloat16().to(DEV)
    v = _rand((B, L, H, D), 12).bfloat16().to(DEV)
    route_q = _rand((B, L, H * G, D), 13).bfloat16().to(DEV)
    valid = torch.rand(B, L, generator=torch.Generator().manual_seed(14)) > 0.1
    valid[0, 64:128] = False
    valid[-1, 63] = False
    valid = valid.to(DEV)
    scale = (torch.rand(H * G) + 0.5).to(DEV)
    mu = route_q[:, 63::64].reshape(B, C, H, G, D)
    frags, lmk, ent, prior = kv_fragments_pool(k, v, mu, valid, scale)
    lmk2, ent2, prior2 = mrsa.chunk_attn_pool_gqa_prior(mu, k.reshape(B, C, 64, H, D),
                                                        valid.reshape(B, C, 64), scale)
    assert torch.equal(frags.view(torch.int16), mrsa.kv_fragments(k, v).view(torch.int16))
    assert torch.equal(lmk.view(torch.int16), lmk2.view(torch.int16))
    assert torch.equal(ent, ent2) and torch.equal(prior, prior2)
    assert float(lmk[0, 1].abs().max()) == 0.0 and float(ent[0, 1].abs().max()) == 0.0


def _route_case(L, C, G, Hkv, seed, derive=False, drop_frac=0.2):
    D = 128
    q5 = _rand((1, L, Hkv, G, D), seed).bfloat16()
    lmk = (_rand((1, C, Hkv * G, D), seed + 1) * 0.5).bfloat16()
    lse4 = _rand((1, L, Hkv, G), seed + 2) + 3.0
    bias4 = torch.rand(1, C, Hkv, G) * 0.5 + 3.5
    if derive:
        valid = torch.rand(1, L) > 0.01
        drop = O.remote_drop_mask(valid, 256, L // C)
    else:
        valid = None
        drop = (torch.rand(1, L, C) < drop_frac).to(torch.int32)
    return q5, lmk, lse4, bias4, drop, valid


def _check_route(idx_gpu, sc_gpu, q5, lmk, lse4, bias4, drop, topk, what, **opts):
    ridx, rsc, sel = O.route_topk(q5, lmk, lse4, topk, 64, drop_mask=drop, bias4=bias4, **opts)
    gap = O.boundary_gap(sel, topk)
    near = gap < NEAR_TIE
    idx = idx_gpu.cpu().long()
    rows_bad = (idx != ridx).any(-1)
    mism = rows_bad & ~near
    print(f"{what}: rows={rows_bad.numel()} near_ties={int(near.sum())} "
          f"mismatched_near_tie_rows={int((rows_bad & near).sum())} other_mismatches={int(mism.sum())}",
          flush=True)
    assert int(mism.sum()) == 0, f"{what}: {int(mism.sum())} non-tie rows differ"
    ok = ~rows_bad
    sc = sc_gpu.cpu().float()
    expect = rsc.bfloat16().float()
    okx = ok[:, :, :, None, None].expand_as(sc)
    torch.testing.assert_close(sc[okx], expect[okx], atol=0.02, rtol=0.01)


@pytest.mark.parametrize("L,C,G,topk", [(512, 256, 7, 32), (640, 200, 7, 31), (256, 300, 3, 16)])
def test_route_topk_vs_oracle(L, C, G, topk):
    _note(f"route topk L={L} C={C} G={G} K={topk}")
    q5, lmk, lse4, bias4, drop, _ = _route_case(L, C, G, 4, 10 + L)
    idx, sc = route_topk_launch(q5.to(DEV), lmk.to(DEV), lse4.to(DEV), topk, 64,
                                          bias4=bias4.to(DEV), drop_mask=drop.to(DEV))
    torch.cuda.synchronize()
    _check_route(idx, sc, q5, lmk, lse4, bias4, drop, topk, f"route L={L} C={C} G={G}")


@pytest.mark.parametrize("L,C,G,topk", [(300, 256, 7, 32), (1000, 130, 8, 20)])
def test_route_topk_exact_ties_go_to_the_lower_chunk(L, C, G, topk):
    # 64 chunks with identical landmarks and bias score exactly alike for
    # every query: with 10 distinct chunks above them, the picks are those 10
    # plus the lowest topk - 10 of the tied group (the stable order of the
    # reference's selection).  Partial last workgroup (L % 128 != 0); two
    # launches are identical.
    _note(f"route ties L={L} C={C} G={G} K={topk}")
    Hkv, D = 4, 128
    q5, lmk, lse4, bias4, _, _ = _route_case(L, C, G, Hkv, 60 + L)
    lmk5 = lmk.reshape(1, C, Hkv, G, D)
    lo, hi = 40, 104
    lmk5[:, lo:hi] = lmk5[:, 7:8]
    bias4[:, lo:hi] = 9.0
    bias4[:, C - 12:C - 2] = 20.0 + torch.arange(10.0).view(1, 10, 1, 1)
    lmk = lmk5.reshape(1, C, Hkv * G, D).contiguous()
    drop = torch.zeros(1, L, C, dtype=torch.int32)
    args = (q5.to(DEV), lmk.to(DEV), lse4.to(DEV), topk, 64)
    kw = dict(bias4=bias4.to(DEV), drop_mask=drop.to(DEV))
    i1, s1 = route_topk_launch(*args, **kw)
    i2, s2 = route_topk_launch(*args, **kw)
    torch.cuda.synchronize()
    assert torch.equal(i1, i2) and torch.equal(s1.view(torch.int16), s2.view(torch.int16))
    expect = torch.cat([torch.arange(lo, lo + topk - 10), torch.arange(C - 12, C - 2)])
    assert torch.equal(i1.cpu().long(), expect.expand(1, L, Hkv, topk))
    ridx, rsc, _ = O.route_topk(q5, lmk, lse4, topk, 64, drop_mask=drop, bias4=bias4)
    assert torch.equal(i1.cpu().long(), ridx)
    torch.testing.assert_close(s1.cpu().float(), rsc.bfloat16().float(), atol=0.02, rtol=0.01)


@pytest.mark.parametrize("L,C,G,topk,mode,causal,fp32,shared", [
    (32, 2048, 7, 32, "post_softmax", False, False, False),   # the cached block step
    (40, 1000, 8, 20, "pre_softmax", False, True, False),
    (33, 700, 4, 64, "post_softmax", True, True, True),
    (5, 4096, 7, 32, "post_softmax", False, False, False),
    # >= 4096 (token, KV head) rows: one selection wave per row
    (1024, 1024, 7, 32, "post_softmax", False, False, False),
    (1100, 512, 8, 32, "pre_softmax", True, True, False),
    (1024, 2048, 7, 32, "post_softmax", False, False, True),
    (1030, 1000, 7, 64, "post_softmax", False, True, False),
])
def test_route_topk_short_block_vs_oracle(L, C, G, topk, mode, causal, fp32, shared):
    # The logits-workspace path (matrix-core logits, then one selection
    # workgroup per row for short blocks or one selection wave per row for
    # long sequences): selection modes, the causal chunk mask with a query
    # offset, shared landmarks, fp32 scores, and up to 4096 chunks.
    _note(f"route short block L={L} C={C} G={G} K={topk} {mode} causal={causal}")
    Hkv = 4
    q5, lmk, lse4, bias4, drop, _ = _route_case(L, C, G, Hkv, 300 + L, drop_frac=0.1)
    if shared:
        lmk = lmk.reshape(1, C, Hkv, G, 128)[:, :, :, 0].contiguous()
    opts = dict(selection_mode=mode, is_causal=causal, q_offset=20000 if causal else 0)
    args = (q5.to(DEV), lmk.to(DEV), lse4.to(DEV), topk, 64)
    kw = dict(bias4=bias4.to(DEV), drop_mask=drop.to(DEV), scores_fp32=fp32, **opts)
    idx, sc = route_topk_launch(*args, use_workspace=True, **kw)
    torch.cuda.synchronize()
    _check_route(idx, sc, q5, lmk, lse4, bias4, drop, topk, f"route block L={L} C={C}", **opts)
    if C <= 2048:  # same selection as the general kernel away from near ties
        gidx, _ = route_topk_launch(*args, use_workspace=False, **kw)
        _, _, sel = O.route_topk(q5, lmk, lse4, topk, 64, drop_mask=drop, bias4=bias4, **opts)
        near = O.boundary_gap(sel, topk) < NEAR_TIE
        differ = (idx.cpu() != gidx.cpu()).any(-1)
        assert int((differ & ~near).sum()) == 0


@pytest.mark.parametrize("C,topk", [(2048, 32), (4096, 64), (700, 20)])
def test_route_topk_short_block_exact_ties_to_the_lower_chunk(C, topk):
    # The short-block selection (one workgroup per row: each wave's own K
    # largest, then one wave over the candidates) breaks exact ties at the
    # threshold by chunk index, like the reference's fused kernel
    # (topk_head_softmax.py:614-626).  20 chunks score highest; 40 chunks
    # spread over every wave's range tie below them; the rest score lowest:
    # the picks are the 20 and the lowest-indexed of the 40.
    _note(f"route short block exact ties C={C} K={topk}")
    L, Hkv, G, D = 4, 4, 7, 128
    g = torch.Generator().manual_seed(401)
    q5 = torch.randn(1, L, Hkv, G, D, generator=g).bfloat16()
    hi = torch.randn(Hkv * G, D, generator=g).bfloat16()
    tie = torch.randn(Hkv * G, D, generator=g).bfloat16()
    low = torch.randn(Hkv * G, D, generator=g).bfloat16()
    perm = torch.randperm(C, generator=g)
    top_set, tie_set = perm[:20], perm[20:60]
    lmk = low.expand(1, C, Hkv * G, D).clone()
    lmk[0, top_set] = hi
    lmk[0, tie_set] = tie
    # make the three groups' scores ordered hi > tie > low for every row
    q5 = (q5.float() * 0 + (hi.float() - low.float()).reshape(Hkv, G, D) * 0.05
          + (tie.float() - low.float()).reshape(Hkv, G, D) * 0.05).bfloat16().expand(1, L, Hkv, G, D).contiguous()
    lse4 = torch.zeros(1, L, Hkv, G)
    bias4 = torch.zeros(1, C, Hkv, G)
    drop = torch.zeros(1, L, C, dtype=torch.int32)
    idx, sc = route_topk_launch(q5.to(DEV), lmk.to(DEV), lse4.to(DEV), topk, 64,
                                bias4=bias4.to(DEV), drop_mask=drop.to(DEV), use_workspace=True)
    ridx, rsc, sel = O.route_topk(q5, lmk, lse4, topk, 64, drop_mask=drop, bias4=bias4)
    # the groups are ordered and the tie group really ties
    s0 = sel[0, 0, 0]
    assert float(s0[top_set].min()) > float(s0[tie_set].max())
    assert float(s0[tie_set].max()) == float(s0[tie_set].min())
    assert float(s0[tie_set].max()) > float(s0[perm[60:]].max())
    assert torch.equal(idx.cpu().long(), ridx)
    torch.testing.assert_close(sc.cpu().float(), rsc.bfloat16().float(), atol=0.02, rtol=0.01)


def test_route_topk_derived_drop_equals_explicit():
    _note("route derived drop")
    L = 16384 // 8
    C = L // 64
    q5, lmk, lse4, bias4, drop, valid = _route_case(L, C, 7, 4, 77, derive=True)
    a = route_topk_launch(q5.to(DEV), lmk.to(DEV), lse4.to(DEV), 8, 64,
                                    bias4=bias4.to(DEV), drop_mask=drop.to(DEV))
    b = route_topk_launch(q5.to(DEV), lmk.to(DEV), lse4.to(DEV), 8, 64,
                                    bias4=bias4.to(DEV), derive_window=256, key_valid=valid.to(DEV))
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    _check_route(a[0], a[1], q5, lmk, lse4, bias4, drop, 8, "route derived")


def test_route_topk_g7_api_and_determinism():
    _note("route_topk_g7 api")
    L, C = 1031, 40   # test_hils_non_power_two_topk.py:51-92 shape
    g = torch.Generator().manual_seed(74)
    q = torch.randn(1, L, 28, 128, generator=g).bfloat16().to(DEV)
    lm = torch.randn(1, C, 4, 7, 128, generator=g).bfloat16().to(DEV)
    lse = torch.randn(1, L, 4, 7, generator=g).to(DEV)
    bias = torch.randn(1, C, 4, 7, generator=g).to(DEV)
    dropped = torch.zeros(1, L, C, dtype=torch.int32, device=DEV)
    dropped[:, ::11, 3] = 1
    first = mrsa.route_topk_g7(q, lm, lse, bias, dropped, 32, 64, 512, training=False)
    second = mrsa.route_topk_g7(q, lm, lse, bias, dropped, 32, 64, 512, training=False)
    assert torch.equal(first[0], second[0]) and torch.equal(first[1], second[1])
    ri, rs = mrsa.ref_softmax_topk_max_pooling(q.reshape(1, L, 4, 7, 128), lm.reshape(1, C, 28, 128),
                                               lse, 32, 64, 512, drop_mask=dropped, bias=bias)
    assert torch.equal(first[0], ri)
    torch.testing.assert_close(first[1].float(), rs.reshape(1, L, 28, 32), atol=0.02, rtol=0.01)
    _check_route(first[0], first[1].reshape(1, L, 4, 7, 32), q.cpu().reshape(1, L, 4, 7, 128),
                 lm.cpu().reshape(1, C, 28, 128), lse.cpu(), bias.cpu(), dropped.cpu(), 32, "g7 api")


@pytest.mark.parametrize("affine,K", [(True, 32), (False, 32), (False, 64), (True, 8), (True, 20),
                                      (False, 24), (True, 40)])
def test_route_weights_vs_oracle(affine, K):
    _note(f"route weights affine={affine} K={K}")
    B, L, Hkv, G, C = 1, 700, 4, 7, 256
    scores = _rand((B, L, Hkv * G, K), 20).bfloat16()
    idx = torch.randint(0, C, (B, L, Hkv, K), generator=torch.Generator().manual_seed(21)).int()
    idx[0, 3, 1, K // 2:] = -1
    idx[0, 4, 2, :] = -1
    idx[0, 6, 0, 1] = C + 7       # out of range: masked like -1
    bias = torch.rand(B, C, Hkv, G) + 3.5
    lse = _rand((B, L, Hkv * G), 22) + 5.0
    lse[0, 5, 3] = float("-inf")
    kw = dict(gate_offset=0.0, gate_scale=1.0) if affine else {}
    rw, lw = route_weights_launch(scores.to(DEV), idx.to(DEV), bias.to(DEV),
                                                     lse.to(DEV), **kw)
    er, el = O.route_weights(scores, idx, bias, lse, **kw)
    torch.testing.assert_close(rw.cpu().float(), er.bfloat16().float(), atol=2e-3, rtol=1e-2)
    torch.testing.assert_close(lw.cpu().float(), el.bfloat16().float(), atol=2e-3, rtol=1e-2)
    if not affine and K == 32:
        torch.testing.assert_close(
            mrsa.route_weights(scores[:, :, :, :31].contiguous().to(DEV), idx[..., :31].contiguous().to(DEV),
                               bias.to(DEV), lse.to(DEV))[1].cpu().float(),
            O.route_weights(scores[..., :31], idx[..., :31], bias, lse)[1].bfloat16().float(),
            atol=2e-3, rtol=1e-2)


@pytest.mark.parametrize("L,W,inert,G", [(1024, 319, 64, 7), (2048, 1280, 0, 7), (512, 100, 64, 8),
                                         (1000, 200, 0, 7), (1000, 150, 48, 7), (1000, 319, 64, 3),
                                         (700, 200, 64, 5), (650, 150, 0, 6), (300, 100, 64, 2)])
def test_local_attention_vs_oracle(L, W, inert, G):
    _note(f"local attention L={L} W={W} inert={inert} G={G}")
    Hkv, D = 4, 128
    q = _rand((1, L, Hkv * G, D), 30).bfloat16()
    k, v = _planted_kv(L, Hkv, D, 31)
    valid = torch.rand(1, L) > 0.05
    # L = 1000: the last fragment tile is partial (keys past L are not keys)
    out, lse = local_attention_launch(
        q.to(DEV), mrsa.kv_fragments(k.to(DEV), v.to(DEV)), valid.to(DEV), W, inert)
    ro, rl = O.local_attention(q, k, v, valid, W, inert)
    _assert_close_attn(out, ro, f"local L={L} W={W}")
    torch.testing.assert_close(lse.cpu(), rl, atol=2e-3, rtol=1e-4)


@pytest.mark.parametrize("W,inert", [(319, 64), (1280, 0)])
def test_local_attention_stabiliser_recompute_and_determinism(W, inert):
    # Queries share a direction e (q + 10 e) and the keys of two later tiles
    # carry 80 e: their logits sit ~70 natural units above everything else
    # (lane sums of p beyond 2^64 against each column's first-tile anchor),
    # so those tiles take the exact recompute path, while the spread inside
    # them stays ordinary (no single key dominates).  The kernel has no
    # atomics: two launches must agree bit for bit.
    _note(f"local attention stabiliser recompute W={W} inert={inert}")
    L, Hkv, G, D = 3072, 4, 7, 128
    e = torch.ones(D) / D ** 0.5
    q = (_rand((1, L, Hkv * G, D), 40) + 10.0 * e).bfloat16()
    k, v = _planted_kv(L, Hkv, D, 41)
    k = k.float()
    k[:, 640:704] += 80.0 * e
    k[:, 1984:2048] += 80.0 * e
    k = k.bfloat16()
    valid = torch.rand(1, L, generator=torch.Generator().manual_seed(42)) > 0.02
    frags = mrsa.kv_fragments(k.to(DEV), v.to(DEV))
    out, lse = local_attention_launch(q.to(DEV), frags, valid.to(DEV), W, inert)
    out2, lse2 = local_attention_launch(q.to(DEV), frags, valid.to(DEV), W, inert)
    torch.cuda.synchronize()
    assert torch.equal(out, out2) and torch.equal(lse, lse2), "local attention is not deterministic"
    ro, rl = O.local_attention(q, k, v, valid, W, inert)
    _assert_close_attn(out, ro, f"local recompute W={W}")
    torch.testing.assert_close(lse.cpu(), rl, atol=2e-3, rtol=1e-4)


@pytest.mark.parametrize("parts,first", [(1, 8000), (3, 8000), (12, 8160), (40, 0), (5, 100)])
def test_local_attention_key_split(parts, first):
    # Key tiles of each 32-query block split over `parts` workgroups and
    # merged (cached block shape: 32 positions, window 319 with inert landmark
    # slots, invalid keys); more parts than tiles leaves some empty.  Blocks
    # at both sequence ends clip the window.
    _note(f"local key split parts={parts} first={first}")
    L, Hkv, G, D, W = 8192, 4, 7, 128, 319
    pos = torch.arange(first, min(L, first + 32))
    Lq = pos.numel()
    q = _rand((1, Lq, Hkv * G, D), 33).bfloat16()
    k, v = _planted_kv(L, Hkv, D, 34)
    valid = torch.rand(1, L, generator=torch.Generator().manual_seed(35)) > 0.05
    out, lse = local_attention_launch(
        q.to(DEV), mrsa.kv_fragments(k.to(DEV), v.to(DEV)), valid.to(DEV), W, 64,
        query_positions=pos.to(DEV), parts=parts)
    ro, rl = O.local_attention(q, k, v, valid, W, 64, query_positions=pos)
    _assert_close_attn(out, ro, f"local split parts={parts}")
    torch.testing.assert_close(lse.cpu(), rl, atol=2e-3, rtol=1e-4)


def test_bidir_and_cached_local_attention_api():
    _note("local attention api")
    L = 1024
    q = _rand((1, L, 28, 128), 32).bfloat16().to(DEV)
    k, v = _planted_kv(L, 4, 128, 33)
    k, v = k.to(DEV), v.to(DEV)
    valid = torch.ones(1, L, dtype=torch.bool, device=DEV)
    o, l = mrsa.bidir_local_attention(q, k, v, valid, 256, 64, skip_inert_slots=True)
    pos = torch.tensor([0, 5, 63, 400, 401, 1023], device=DEV)
    oc, lc = mrsa.cached_local_attention(q[:, pos], k, v, valid, pos, 256, 64, skip_inert_slots=True)
    torch.testing.assert_close(oc.float(), o[:, pos].float(), atol=1e-2, rtol=0)
    torch.testing.assert_close(lc, l[:, pos], atol=1e-4, rtol=0)


def _sorted_routes(Lq, Hkv, K, C, seed, neg_rows=()):
    g = torch.Generator().manual_seed(seed)
    idx = torch.stack([torch.randperm(C, generator=g)[:K] for _ in range(Lq * Hkv)])
    idx = idx.sort(-1).values.reshape(1, Lq, Hkv, K).int()
    for r in neg_rows:
        idx[0, r, :, K // 2:] = -1
    return idx


@pytest.mark.parametrize("Lq,Lk,K,unsorted", [(1024, 1024, 8, False), (777, 2048, 32, False),
                                               (300, 4096, 32, True)])
def test_selected_attention_vs_oracle(Lq, Lk, K, unsorted):
    _note(f"selected Lq={Lq} Lk={Lk} K={K} unsorted={unsorted}")
    Hkv, G, D, C = 4, 7, 128, Lk // 64
    q = _rand((1, Lq, Hkv * G, D), 40).bfloat16()
    k, v = _planted_kv(Lk, Hkv, D, 41)
    idx = _sorted_routes(Lq, Hkv, K, C, 42, neg_rows=(0, 5))
    if unsorted:
        perm = torch.randperm(K, generator=torch.Generator().manual_seed(43))
        idx = idx[..., perm].contiguous()
        idx[0, 7, 0, 3] = C + 5          # out of range -> skipped
    w = torch.softmax(_rand((1, Lq, Hkv * G, K), 44), -1).bfloat16()
    valid = torch.rand(1, Lk) > 0.03
    out = selected_attention_launch(
        q.to(DEV), mrsa.kv_fragments(k.to(DEV), v.to(DEV)), w.to(DEV), idx.to(DEV), valid.to(DEV), 64)
    ref = O.selected_attention(q, k, v, w, idx, valid, 64)
    _assert_close_attn(out, ref, f"selected Lq={Lq}")


@pytest.mark.parametrize("Lq,Lk,K,parts", [(32, 16384, 32, 7), (32, 16384, 32, 64),
                                             (50, 4096, 16, 5), (3, 4096, 4, 40)])
def test_selected_attention_walk_split(Lq, Lk, K, parts):
    # The walk split over `parts` workgroups (fp32 partials summed in a second
    # kernel) against the oracle and the unsplit kernel: unsorted rows with a
    # duplicate chunk, -1 tails, an out-of-range id and invalid keys.  The last
    # case has more parts than walk steps (empty parts contribute zeros).
    _note(f"selected split Lq={Lq} Lk={Lk} K={K} parts={parts}")
    Hkv, G, D, C = 4, 7, 128, Lk // 64
    q = _rand((1, Lq, Hkv * G, D), 45).bfloat16()
    k, v = _planted_kv(Lk, Hkv, D, 46)
    idx = _sorted_routes(Lq, Hkv, K, C, 47, neg_rows=(0,))
    perm = torch.randperm(K, generator=torch.Generator().manual_seed(48))
    idx = idx[..., perm].contiguous()
    idx[0, Lq - 1, :, 1] = idx[0, Lq - 1, :, 0]   # duplicate -> weights summed
    idx[0, Lq // 2, 0, 0] = C + 3                  # out of range -> skipped
    w = torch.softmax(_rand((1, Lq, Hkv * G, K), 49), -1).bfloat16()
    valid = torch.rand(1, Lk, generator=torch.Generator().manual_seed(50)) > 0.03
    args = (q.to(DEV), mrsa.kv_fragments(k.to(DEV), v.to(DEV)), w.to(DEV), idx.to(DEV),
            valid.to(DEV), 64)
    out = selected_attention_launch(*args, parts=parts)
    whole = selected_attention_launch(*args, parts=1)
    ref = O.selected_attention(q, k, v, w, idx, valid, 64)
    _assert_close_attn(out, ref, f"selected split parts={parts}")
    # Same terms, different fp32 summation order: within one bf16 step.
    torch.testing.assert_close(out.float(), whole.float(), atol=8e-3, rtol=8e-3)


@pytest.mark.parametrize("Lq,Lk,K,parts,keep", [(700, 2048, 32, 1, False), (32, 8192, 32, 9, False),
                                                  (200, 2048, 16, 1, True), (40, 4096, 8, 3, True),
                                                  (700, 2048, 1, 1, False), (32, 8192, 1, 9, False),
                                                  (200, 2048, 1, 1, True)])
def test_selected_attention_fused_output_equals_fusion(Lq, Lk, K, parts, keep):
    # The output fusion folded into the routed-attention epilogue (parts == 1)
    # or into the part sum (parts > 1) gives the bits of the routed output
    # followed by fuse_hils_outputs.  With one routed chunk per query every
    # output row is a single term, so two launches agree bit for bit; with
    # more, the fp32 sum's order varies between launches (rare one-step
    # flips).
    _note(f"selected fused Lq={Lq} Lk={Lk} K={K} parts={parts} keep={keep}")
    Hkv, G, D, C = 4, 7, 128, Lk // 64
    q = _rand((1, Lq, Hkv * G, D), 80).bfloat16()
    k, v = _planted_kv(Lk, Hkv, D, 81)
    idx = _sorted_routes(Lq, Hkv, K, C, 82, neg_rows=(0,))
    w = torch.softmax(_rand((1, Lq, Hkv * G, K), 83), -1).bfloat16()
    valid = torch.rand(1, Lk, generator=torch.Generator().manual_seed(84)) > 0.03
    local = _rand((1, Lq, Hkv * G, D), 85).bfloat16().to(DEV)
    lw = torch.rand(1, Lq, Hkv * G, generator=torch.Generator().manual_seed(86)).bfloat16().to(DEV)
    tk = None
    if keep:
        tk = (torch.rand(1, Lq, Hkv, K, 64, generator=torch.Generator().manual_seed(87)) > 0.5)
        tk = tk.to(torch.int8).to(DEV)
    args = (q.to(DEV), mrsa.kv_fragments(k.to(DEV), v.to(DEV)), w.to(DEV), idx.to(DEV),
            valid.to(DEV), 64)
    remote = selected_attention_launch(*args, parts=parts, token_keep=tk)
    fused = selected_attention_launch(*args, parts=parts, token_keep=tk, fuse_local=local,
                                      fuse_weight=lw)
    expect = mrsa.fuse_hils_outputs(remote, local, lw)
    torch.cuda.synchronize()
    if K == 1:
        assert torch.equal(fused.view(torch.int16), expect.view(torch.int16))
    else:
        assert_nearly_identical(fused, expect, f"fused vs fusion K={K}", atol=0.03)


@pytest.mark.parametrize("Lq,K,keep", [(4, 32, False), (4, 32, True), (8, 16, True)])
def test_selected_attention_contended_lock_repeats(Lq, K, keep):
    # Few queries that all route to the same chunks: every step of a walk
    # has the same owners, so the eight waves of a workgroup keep asking for
    # the same lock bits.  Waits that set momentary bits on a failed try can
    # lock two such waves in step until one gives up and adds without the
    # lock over another's read-modify-write (lost updates of whole rows).
    # Every repeat must match the oracle.
    _note(f"selected contended Lq={Lq} K={K} keep={keep}")
    Hkv, G, D, Lk = 4, 7, 128, 2048
    C = Lk // 64
    q = _rand((1, Lq, Hkv * G, D), 90).bfloat16()
    k, v = _planted_kv(Lk, Hkv, D, 91)
    idx = _sorted_routes(Lq, Hkv, K, C, 92)
    w = torch.softmax(_rand((1, Lq, Hkv * G, K), 93), -1).bfloat16()
    valid = torch.rand(1, Lk, generator=torch.Generator().manual_seed(94)) > 0.03
    tk = None
    if keep:
        tk = (torch.rand(1, Lq, Hkv, K, 64, generator=torch.Generator().manual_seed(95)) > 0.5)
        tk = tk.to(torch.int8)
    ref = O.selected_attention(q, k, v, w, idx, valid, 64, token_keep=tk)
    args = (q.to(DEV), mrsa.kv_fragments(k.to(DEV), v.to(DEV)), w.to(DEV), idx.to(DEV),
            valid.to(DEV), 64)
    tkd = None if tk is None else tk.to(DEV)
    outs = [selected_attention_launch(*args, parts=1, token_keep=tkd) for _ in range(40)]
    torch.cuda.synchronize()
    errs = [float((out.float().cpu() - ref.float()).abs().max()) for out in outs]
    print(f"contended repeats: max_abs worst {max(errs):.3e} median {sorted(errs)[20]:.3e}",
          flush=True)
    assert max(errs) <= 2e-2, errs


def test_selected_attention_reference_kat():
    # test_hils_non_power_two_topk.py:95-142 (cached and uncached shapes).
    for query_len in (35, 2048):
        _note(f"selected KAT q={query_len}")
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
        args = [t.to(DEV) for t in (q, k, v, weights, indices, valid)]
        actual = (mrsa.selected_attention_g7_cached(*args, size) if query_len == 35 else
                  mrsa.selected_attention_g7(*args, size, training=False))
        assert actual.shape == q.shape and bool(torch.isfinite(actual).all())
        assert torch.equal(actual[:, 0].cpu(), torch.zeros_like(actual[:, 0].cpu()))
        rows = torch.tensor([1, query_len // 2, query_len - 1])
        ref = O.selected_attention(q[:, rows], k, v, weights[:, rows], indices[:, rows], valid, size)
        observed = actual.cpu()[:, rows].float()
        assert float((observed - ref).norm() / ref.norm()) < 0.02
        torch.testing.assert_close(observed, ref, atol=0.01, rtol=0.025)
        for value, original in zip(args[3:], (weights, indices, valid)):
            assert torch.equal(value.cpu(), original)


def test_candidate_token_scores_vs_oracle():
    _note("token scores")
    Lq, Lk, K = 200, 2048, 8
    q = _rand((1, Lq, 28, 128), 50).bfloat16()
    k, _ = _planted_kv(Lk, 4, 128, 51)
    idx = _sorted_routes(Lq, 4, K, Lk // 64, 52, neg_rows=(3,))
    valid = torch.rand(1, Lk) > 0.05
    got = mrsa.candidate_token_scores_gqa(q.to(DEV), k.to(DEV), idx.to(DEV), valid.to(DEV), 64).cpu()
    ref = O.candidate_token_scores(q, k, idx, valid, 64)
    fin = torch.isfinite(ref)
    assert torch.equal(fin, torch.isfinite(got))
    torch.testing.assert_close(got[fin], ref[fin], atol=1e-3, rtol=1e-3)


def test_route_layer_config2_full_size_every_row():
    # BASELINE configuration 2 at its full size (L=16384, 28/4 heads, 256
    # chunks, planted per-chunk key shift).  Routing: the stage-fed oracle
    # (the GPU's landmarks, local LSE and prior) over all 16384 rows in
    # 512-row blocks; every (row, KV head) list must be identical except near
    # ties (boundary gap below 1e-5), which are counted and reported.  The
    # other stages are checked on 1024 rows (sequence ends, chunk edges,
    # random rows), each oracle stage fed that stage's GPU inputs.
    _note("route layer config 2, full size, every routing row")
    L, Hq, Hkv, D, S, G, K = 16384, 28, 4, 128, 64, 7, 32
    C = L // S
    cfg = mrsa.RouteLayerConfig()
    q = _rand((1, L, Hq, D), 90).bfloat16()
    k, v = _planted_kv(L, Hkv, D, 91)
    scale = torch.ones(Hq)
    valid = torch.ones(1, L, dtype=torch.bool)
    out, mid = mrsa.route_attention(q.to(DEV), k.to(DEV), v.to(DEV), q.to(DEV), scale.to(DEV),
                                    valid.to(DEV), cfg, return_intermediates=True)
    torch.cuda.synchronize()
    mid = {n: (t.cpu() if torch.is_tensor(t) else t) for n, t in mid.items()}
    out = out.cpu()
    # Landmark pool and prior over all 256 chunks.
    lmk, ent = O.chunk_attn_pool(q[:, S - 1 :: S].reshape(1, C, Hkv, G, D),
                                 k.reshape(1, C, S, Hkv, D), valid.reshape(1, C, S))
    _assert_lmk_close(mid["landmark_keys"].reshape(lmk.shape), lmk, "cfg2 landmarks")
    torch.testing.assert_close(mid["prior_bias"].float().reshape(ent.shape), ent, atol=1e-3,
                               rtol=1e-3)
    # Routing of every row.
    drop = O.remote_drop_mask(valid, cfg.local_window, S)
    ridx, rsc, sel = O.route_topk(
        q.reshape(1, L, Hkv, G, D), mid["landmark_keys"].reshape(1, C, Hq, D),
        mid["local_lse"].reshape(1, L, Hkv, G), K, S, drop_mask=drop,
        bias4=mid["prior_bias"].reshape(1, C, Hkv, G), query_block=512)
    gap = O.boundary_gap(sel, K)
    near = gap < NEAR_TIE
    gidx = mid["indices"].long()
    bad = (gidx != ridx).any(-1)
    lists = L * Hkv
    n_near, n_bad = int(near.sum()), int(bad.sum())
    n_flip = int((bad & near).sum())
    worst = torch.sort(gap[bad].flatten()).values[:10].tolist() if n_bad else []
    smallest = torch.sort(gap.flatten()).values[:5].tolist()
    lines = [
        f"lists (row, KV head): {lists}",
        f"near ties (boundary gap < {NEAR_TIE:g}): {n_near}",
        f"lists that differ from the oracle: {n_bad} (all near ties: {n_flip == n_bad})",
        f"gaps of the differing lists: {[f'{x:.3g}' for x in worst]}",
        f"smallest boundary gaps of all lists: {[f'{x:.3g}' for x in smallest]}",
    ]
    print("cfg2 routing, every row:\n  " + "\n  ".join(lines), flush=True)
    outdir = os.path.join(os.environ.get("GRAFT_REPO_ROOT", ""), "gpurun_out")
    if os.environ.get("GRAFT_REPO_ROOT") and os.path.isdir(outdir):
        with open(os.path.join(outdir, "cfg2_routing_parity.txt"), "w") as f:
            f.write("\n".join(lines) + "\n")
    assert int((bad & ~near).sum()) == 0, lines
    ok = (~bad)[..., None, None].expand(1, L, Hkv, G, K)
    gsc = mid["scores"].float().reshape(1, L, Hkv, G, K)
    torch.testing.assert_close(gsc[ok], rsc.bfloat16().float()[ok], atol=0.02, rtol=0.01)
    del sel, rsc, gsc, ok
    # The other stages on 1024 rows: sequence ends, both sides of every
    # 16th chunk edge, random rows.
    edges = [c * S + d for c in range(0, C, 16) for d in (-1, 0) if 0 <= c * S + d < L]
    rnd = torch.randint(0, L, (1024,), generator=torch.Generator().manual_seed(92)).tolist()
    base = sorted(set([0, 1, 2, 318, 319, 320, L - 321, L - 320, L - 3, L - 2, L - 1] + edges))
    rows = torch.tensor(sorted(set(base + rnd))[:1024])
    n = rows.numel()
    lo, ll = O.local_attention(q[:, rows], k, v, valid, cfg.local_window + S - 1, S,
                               query_positions=rows, query_block=1)
    _assert_close_attn(mid["local_output"][:, rows], lo, "cfg2 local rows")
    torch.testing.assert_close(mid["local_lse"][:, rows], ll, atol=2e-3, rtol=1e-4)
    rw, lw = O.route_weights(mid["scores"][:, rows], mid["indices"][:, rows].long(),
                             mid["prior_bias"], mid["local_lse"][:, rows],
                             temperature=cfg.temperature, gate_offset=cfg.gate_offset,
                             gate_scale=cfg.gate_scale)
    torch.testing.assert_close(mid["remote_weights"][:, rows].float(), rw, atol=1e-2, rtol=1e-2)
    torch.testing.assert_close(mid["local_weight"][:, rows].float(), lw, atol=1e-2, rtol=1e-2)
    remote = O.selected_attention(q[:, rows], k, v, mid["remote_weights"][:, rows],
                                  mid["indices"][:, rows], valid, S)
    _assert_close_attn(mid["remote_output"][:, rows], remote, f"cfg2 routed, {n} rows")
    fused = O.fuse_outputs(mid["remote_output"][:, rows], mid["local_output"][:, rows],
                           mid["local_weight"][:, rows])
    assert_nearly_identical(out[:, rows], fused, f"cfg2 fused output, {n} rows", atol=0.03)


def test_route_layer_vs_oracle():
    _note("route layer L=2048")
    L, Hq, Hkv, D = 2048, 28, 4, 128
    q = _rand((1, L, Hq, D), 60).bfloat16()
    rq = _rand((1, L, Hq, D), 61).bfloat16()
    k, v = _planted_kv(L, Hkv, D, 62)
    scale = torch.rand(Hq) + 0.5
    valid = torch.ones(1, L, dtype=torch.bool)
    valid[0, 700:705] = False
    out, mid = mrsa.route_attention(q.to(DEV), k.to(DEV), v.to(DEV), rq.to(DEV), scale.to(DEV),
                                    valid.to(DEV), return_intermediates=True)
    ref, rmid = O.route_layer(q, k, v, rq, scale, valid)
    _assert_close_attn(out, ref, "route layer")
    classify_routing(mid["indices"], rmid["indices"], rq, mid["landmark_keys"], mid["local_lse"],
                     mid["prior_bias"], lambda r: O.remote_drop_mask(valid, 256, 64)[:, r],
                     32, 64, "route layer L=2048")


# -- Gumbel route sampling (training): ops/topk_head_softmax.py:99-105, routing.py:96-302
def test_route_topk_gumbel_noise_vs_oracle():
    _note("route topk with explicit gumbel noise")
    B, L, Hkv, G, D, C, K = 1, 256, 2, 7, 128, 64, 16
    g = torch.Generator().manual_seed(300)
    q = torch.randn(B, L, Hkv * G, D, generator=g).bfloat16()
    lm = torch.randn(B, C, Hkv * G, D, generator=g).bfloat16()
    lse = torch.randn(B, L, Hkv * G, generator=g) + 3
    bias = torch.rand(B, C, Hkv, G, generator=g)
    noise = -torch.log(-torch.log(torch.rand(1, 1, Hkv * G, C, generator=g).clamp(1e-6, 1 - 1e-6)))
    idx, sc = mrsa.online_softmax_topk_head(q.to(DEV), lm.to(DEV), lse.to(DEV), K, 64, 0,
                                            is_causal=False, bias=bias.to(DEV),
                                            gumbel_noise=noise.to(DEV), G=G)
    ridx, rsc, sel = O.route_topk(q.reshape(B, L, Hkv, G, D), lm, lse.reshape(B, L, Hkv, G), K, 64,
                                  bias4=bias, gumbel_noise=noise)
    gap = O.boundary_gap(sel, K)
    same = (idx.cpu().long() == ridx).all(-1)
    assert bool((same | (gap < 1e-5)).all()), "index mismatch away from a near tie"
    # scores stay raw q.k * scale (no bias, no noise)
    ok = same[:, :, :, None].expand(-1, -1, -1, G).reshape(B, L, Hkv * G)
    # (one bf16 ulp: the fp32 dot products are summed in different orders)
    torch.testing.assert_close(sc.float().cpu()[ok], rsc.reshape(B, L, Hkv * G, K)[ok].bfloat16().float(),
                               rtol=2 ** -7, atol=1e-3)
    # the noise changes the routing
    nidx, _ = mrsa.online_softmax_topk_head(q.to(DEV), lm.to(DEV), lse.to(DEV), K, 64, 0,
                                            is_causal=False, bias=bias.to(DEV), G=G)
    assert not torch.equal(nidx.cpu(), idx.cpu())
    with pytest.raises(AssertionError, match="training"):
        mrsa.online_softmax_topk_head(q.to(DEV), lm.to(DEV), lse.to(DEV), K, 64, 0,
                                      is_causal=False, is_training=False,
                                      gumbel_noise=noise.to(DEV), G=G)


def test_route_topk_g7_gumbel_sampling_vs_oracle():
    _note("route_topk_g7 gumbel sampling")
    B, L, Hkv, G, D, C, K = 1, 128, 2, 7, 128, 48, 16
    g = torch.Generator().manual_seed(310)
    q = torch.randn(B, L, Hkv * G, D, generator=g).bfloat16().to(DEV)
    lm = torch.randn(B, C, Hkv, G, D, generator=g).bfloat16().to(DEV)
    lse = (torch.randn(B, L, Hkv, G, generator=g) + 3).to(DEV)
    prior = torch.rand(B, C, Hkv, G, generator=g).to(DEV)
    drop = torch.zeros(B, L, C, dtype=torch.int32, device=DEV)
    drop[:, :, 5] = 1
    torch.cuda.manual_seed(1234)
    idx, sc, selg = mrsa.route_topk_g7(q, lm, lse, prior, drop, K, 64, 256, training=True,
                                       use_gumbel=True, gumbel_scale=0.5,
                                       return_selected_gumbel=True)
    # the same draw, in the reference's physical shape
    torch.cuda.manual_seed(1234)
    eps = torch.finfo(torch.float32).eps
    u = torch.empty(1, 1, Hkv * 8, max(C, K), device=DEV).uniform_(eps, 1.0 - eps)
    noise = (-torch.log(-torch.log(u)) * 0.5).reshape(Hkv, 8, -1)[:, :7, :C].cpu()
    ridx, _, sel = O.route_topk(q.cpu().reshape(B, L, Hkv, G, D), lm.cpu().reshape(B, C, Hkv * G, D),
                                lse.cpu(), K, 64, drop_mask=drop.cpu(), bias4=prior.cpu(),
                                gumbel_noise=noise.reshape(1, 1, Hkv * G, C))
    gap = O.boundary_gap(sel, K)
    same = (idx.cpu().long() == ridx).all(-1)
    print(f"gumbel routing: identical lists {float(same.float().mean()):.4f}, "
          f"near ties among the rest {int(((~same) & (gap < 1e-5)).sum())}", flush=True)
    assert bool((same | (gap < 1e-5)).all())
    assert idx.dtype == torch.int32
    # selected noise: the head's noise at each routed chunk, 0 at -1 slots
    ii = idx.cpu().long()
    exp = torch.gather(noise[None, None].expand(B, L, Hkv, G, C), -1,
                       ii.clamp(min=0)[:, :, :, None, :].expand(-1, -1, -1, G, -1))
    exp = exp.masked_fill((ii < 0)[:, :, :, None, :], 0.0).reshape(B, L, Hkv * G, K)
    assert torch.equal(selg.cpu(), exp)


def test_routed_lock_giveups_are_reported_and_exact():
    # The bounded lock wait is forced from the host: with one try per tile,
    # contended tiles give up, are deferred and replayed after the walk (no
    # fault or hang, no lost terms), and the status word reports them.  With
    # the default bound the contended shape reports none.  A limit of 0
    # defers every tile.  Each output matches the oracle.
    _note("routed lock give-ups deferred, exact and reported")
    Lq, K, Hkv, G, D, Lk = 4, 32, 4, 7, 128, 2048
    q = _rand((1, Lq, Hkv * G, D), 96).bfloat16()
    k, v = _planted_kv(Lk, Hkv, D, 97)
    idx = _sorted_routes(Lq, Hkv, K, Lk // 64, 98)
    w = torch.softmax(_rand((1, Lq, Hkv * G, K), 99), -1).bfloat16()
    valid = torch.ones(1, Lk, dtype=torch.bool)
    args = (q.to(DEV), mrsa.kv_fragments(k.to(DEV), v.to(DEV)), w.to(DEV), idx.to(DEV),
            valid.to(DEV), 64)
    ref = O.selected_attention(q, k, v, w, idx, valid)
    mrsa.routed_lock_giveups(reset=True)
    for _ in range(10):
        _assert_close_attn(selected_attention_launch(*args, parts=1), ref, "default bound")
    assert mrsa.routed_lock_giveups(reset=True) == 0
    try:
        for limit in (1, 0):
            mrsa.set_routed_lock_spin_limit(limit)
            for _ in range(10):
                _assert_close_attn(selected_attention_launch(*args, parts=1), ref,
                                   f"spin limit {limit}")
            n = mrsa.routed_lock_giveups(reset=False)
            print(f"spin limit {limit}: {n} deferred tiles", flush=True)
            assert n > 0
            with pytest.raises(mrsa.RoutedLockTimeout):
                mrsa.check_routed_locks()
            assert mrsa.routed_lock_giveups(reset=True) == 0  # cleared by the check
        # every tile deferred, with token keep rows, and with the fusion
        # reading Q fragments
        mrsa.set_routed_lock_spin_limit(0)
        keep = (torch.rand(1, Lq, Hkv, K, 64, generator=torch.Generator().manual_seed(95))
                < 0.7).to(torch.int8)
        rk = O.selected_attention(q, k, v, w, idx, valid, token_keep=keep)
        _assert_close_attn(selected_attention_launch(*args, parts=1, token_keep=keep.to(DEV)),
                           rk, "spin limit 0, token keep")
        loc = _rand((1, Lq, Hkv * G, D), 94).bfloat16()
        lw = torch.rand(1, Lq, Hkv * G).bfloat16()
        fused = selected_attention_launch(*args, parts=1, fuse_local=loc.to(DEV),
                                          fuse_weight=lw.to(DEV),
                                          q_frags=mrsa.q_fragments(q.to(DEV), Hkv))
        _assert_close_attn(fused, O.fuse_outputs(ref, loc, lw), "spin limit 0, fused, Q fragments")
        assert mrsa.routed_lock_giveups(reset=True) > 0
    finally:
        mrsa.set_routed_lock_spin_limit(65536)


# -- Q fragments: the routed attention's Q^T operand images ----------------
def test_q_fragments_layout_bit_exact():
    _note("q fragments layout")
    for B, L, Hkv, G in ((1, 100, 4, 7), (2, 64, 2, 8), (1, 33, 3, 4)):
        q = _rand((B, L, Hkv * G, 128), 77).bfloat16()
        qf = mrsa.q_fragments(q.to(DEV), Hkv).cpu().reshape(B, Hkv, L, 4, 4, 8, 8)
        exp = torch.zeros(B, Hkv, L, 4, 4, 8, 8, dtype=torch.bfloat16)  # ks, grp, head, e
        exp[:, :, :, :, :, :G] = q.reshape(B, L, Hkv, G, 4, 4, 8).permute(0, 2, 1, 4, 5, 3, 6)
        assert torch.equal(qf, exp), (B, L, Hkv, G)


@pytest.mark.parametrize("G", [7, 4, 3, 6])
def test_local_attention_qf_same_outputs_and_q_fragments(G):
    # The window kernel's Q-fragment by-product changes nothing else, and the
    # images equal the standalone layout kernel's, zero head slots included
    # (G = 3, 6, 7 take the packed column layout, G = 4 the power-of-two one).
    _note(f"local attention with Q fragments G={G}")
    from mrsa.local_attention import local_attention_qf_launch
    L, Hkv, D = 1000, 2, 128
    q = _rand((1, L, Hkv * G, D), 81).bfloat16().to(DEV)
    k, v = _planted_kv(1024, Hkv, D, 82)
    valid = torch.ones(1, L, dtype=torch.bool)
    valid[0, 300:310] = False
    valid = valid.to(DEV)
    frags = mrsa.kv_fragments(k[:, :L].contiguous().to(DEV), v[:, :L].contiguous().to(DEV))
    o1, l1 = local_attention_launch(q, frags, valid, 319, 64, parts=1)
    o2, l2, qf = local_attention_qf_launch(q, frags, valid, 319, 64)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    assert torch.equal(qf, mrsa.q_fragments(q, Hkv))


def test_selected_attention_fused_with_q_fragments_matches():
    _note("fused routed attention reading Q fragments")
    Lq, Lk, Hkv, G, D, K = 300, 2048, 4, 7, 128, 32
    q = _rand((1, Lq, Hkv * G, D), 85).bfloat16()
    k, v = _planted_kv(Lk, Hkv, D, 86)
    idx = _sorted_routes(Lq, Hkv, K, Lk // 64, 87)
    w = torch.softmax(_rand((1, Lq, Hkv * G, K), 88), -1).bfloat16()
    valid = torch.ones(1, Lk, dtype=torch.bool)
    valid[0, 1000:1003] = False
    loc = _rand((1, Lq, Hkv * G, D), 89).bfloat16()
    lw = torch.rand(1, Lq, Hkv * G).bfloat16()
    args = (q.to(DEV), mrsa.kv_fragments(k.to(DEV), v.to(DEV)), w.to(DEV), idx.to(DEV),
            valid.to(DEV), 64)
    kw = dict(fuse_local=loc.to(DEV), fuse_weight=lw.to(DEV))
    qf = mrsa.q_fragments(q.to(DEV), Hkv)
    for parts in (1, 3):
        a = selected_attention_launch(*args, parts=parts, **kw)
        b = selected_attention_launch(*args, parts=parts, q_frags=qf, **kw)
        assert_nearly_identical(a, b, f"fused with Q fragments, parts={parts}", atol=0.03)
    ref = O.fuse_outputs(O.selected_attention(q, k, v, w, idx, valid), loc, lw)
    _assert_close_attn(b, ref, "fused with Q fragments vs oracle")
    with pytest.raises(ValueError):
        selected_attention_launch(*args, q_frags=qf)  # Q fragments need the fusion


# -- fixed-order (deterministic) routed attention -------------------------
def test_selected_attention_fixed_order_is_deterministic():
    # Every output row adds its chunk terms in ascending chunk order: twenty
    # launches of the contended shape (every query routes to every chunk, so
    # the waves always share rows) give the same bits, with walk splits,
    # keep rows, the fusion reading Q fragments and lists that are not
    # ascending (a duplicated chunk, an entry past the chunks, a -1 end).
    # With the bounded wait forced to one try, the deferred tiles replay in
    # step order: the same bits again.
    _note("fixed-order routed attention")
    Lq, K, Hkv, G, D, Lk = 40, 32, 4, 7, 128, 2048
    q = _rand((1, Lq, Hkv * G, D), 196).bfloat16()
    k, v = _planted_kv(Lk, Hkv, D, 197)
    idx = _sorted_routes(Lq, Hkv, K, Lk // 64, 198)
    w = torch.softmax(_rand((1, Lq, Hkv * G, K), 199), -1).bfloat16()
    valid = torch.ones(1, Lk, dtype=torch.bool)
    valid[0, 900:903] = False
    kf = mrsa.kv_fragments(k.to(DEV), v.to(DEV))
    args = (q.to(DEV), kf, w.to(DEV), idx.to(DEV), valid.to(DEV), 64)
    ref = O.selected_attention(q, k, v, w, idx, valid)
    keep = (torch.rand(1, Lq, Hkv, K, 64, generator=torch.Generator().manual_seed(194))
            < 0.8).to(torch.int8)
    loc = _rand((1, Lq, Hkv * G, D), 193).bfloat16()
    lw = torch.rand(1, Lq, Hkv * G).bfloat16()
    qf = mrsa.q_fragments(q.to(DEV), Hkv)
    cases = {
        "plain": dict(parts=1),
        "walk split": dict(parts=3),
        "keep": dict(parts=1, token_keep=keep.to(DEV)),
        "fused, Q fragments": dict(parts=1, fuse_local=loc.to(DEV), fuse_weight=lw.to(DEV),
                                   q_frags=qf),
    }
    firsts = {}
    for name, kw in cases.items():
        outs = [selected_attention_launch(*args, deterministic=True, **kw) for _ in range(20)]
        firsts[name] = outs[0]
        for o in outs[1:]:
            assert torch.equal(o, outs[0]), name
    _assert_close_attn(firsts["plain"], ref, "fixed order vs oracle")
    _assert_close_attn(firsts["walk split"], ref, "fixed order, walk split vs oracle")
    assert_nearly_identical(firsts["plain"], selected_attention_launch(*args, parts=1),
                            "fixed order vs locked order")
    # lists that are not ascending
    idx2 = idx.clone()
    idx2[0, :, :, 5] = idx2[0, :, :, 9]          # a duplicated chunk
    idx2[0, 3, :, 0] = Lk // 64 + 7              # an entry past the chunks
    idx2[0, 4, :, 20:] = -1                      # a list that ends early
    args2 = (q.to(DEV), kf, w.to(DEV), idx2.to(DEV), valid.to(DEV), 64)
    o2 = [selected_attention_launch(*args2, parts=1, deterministic=True) for _ in range(10)]
    for o in o2[1:]:
        assert torch.equal(o, o2[0])
    _assert_close_attn(o2[0], O.selected_attention(q, k, v, w, idx2, valid), "unsorted lists")
    # deferred tiles replay in step order: the same bits
    try:
        mrsa.set_routed_lock_spin_limit(1)
        for name in ("plain", "walk split"):
            o = selected_attention_launch(*args, deterministic=True, **cases[name])
            assert torch.equal(o, firsts[name]), f"{name} with deferred tiles"
        mrsa.routed_lock_giveups(reset=True)
    finally:
        mrsa.set_routed_lock_spin_limit(65536)


def test_selected_attention_fixed_order_graph_replays_match_eager():
    _note("fixed-order routed attention in a HIP graph")
    Lq, K, Hkv, G, D, Lk = 64, 32, 4, 7, 128, 4096
    q = _rand((1, Lq, Hkv * G, D), 296).bfloat16().to(DEV)
    k, v = _planted_kv(Lk, Hkv, D, 297)
    idx = _sorted_routes(Lq, Hkv, K, Lk // 64, 298).to(DEV)
    w = torch.softmax(_rand((1, Lq, Hkv * G, K), 299), -1).bfloat16().to(DEV)
    valid = torch.ones(1, Lk, dtype=torch.bool, device=DEV)
    kf = mrsa.kv_fragments(k.to(DEV), v.to(DEV))
    eager = selected_attention_launch(q, kf, w, idx, valid, 64, parts=4, deterministic=True)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        selected_attention_launch(q, kf, w, idx, valid, 64, parts=4, deterministic=True)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gout = selected_attention_launch(q, kf, w, idx, valid, 64, parts=4, deterministic=True)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout, eager)
        again = selected_attention_launch(q, kf, w, idx, valid, 64, parts=4, deterministic=True)
        torch.cuda.synchronize()
        assert torch.equal(again, eager)


def test_route_layer_config2_fixed_order_twice_same_bits():
    _note("route layer config 2, fixed order, two runs")
    L, Hq, Hkv, D = 16384, 28, 4, 128
    q = _rand((1, L, Hq, D), 390).bfloat16().to(DEV)
    k, v = _planted_kv(L, Hkv, D, 391)
    k, v = k.to(DEV), v.to(DEV)
    cfg = mrsa.RouteLayerConfig(deterministic=True)
    scale = torch.ones(Hq, device=DEV)
    a = mrsa.route_attention(q, k, v, q, scale, cfg=cfg)
    b = mrsa.route_attention(q, k, v, q, scale, cfg=cfg)
    assert torch.equal(a, b)
    c = mrsa.route_attention(q, k, v, q, scale)   # the default (lock) order
    assert_nearly_identical(a, c, "config 2: fixed order vs lock order", atol=0.03)
