"""GPU parity of the backward kernels against the oracle's autograd.

Route weights: the kernel recomputes the row probabilities in fp32, as the
oracle's forward does, so gradients agree to fp32 rounding (plus the order of
the atomic bias sums); d_scores is returned in bf16 like the reference's
``d_scores.to(score_dtype)``.  Fusion: d_remote and d_local bit-exact, d_weight
within one bf16 rounding of the fp32 sum.
"""

import pytest
import torch

import mrsa
from mrsa.fusion import fuse_hils_outputs_backward
from mrsa.route_weights import route_weights_backward
from oracle import mrsa_oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _note(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _case(seed, B, L, Hkv, G, K, C):
    g = torch.Generator().manual_seed(seed)
    scores = (torch.randn(B, L, Hkv * G, K, generator=g) * 2).bfloat16()
    idx = torch.randint(0, C, (B, L, Hkv, K), generator=g).int()
    idx[0, 3, 1 % Hkv, K // 2:] = -1
    idx[0, 4, 0, 0] = C + 5
    bias = torch.rand(B, C, Hkv, G, generator=g) + 1.0
    lse = torch.randn(B, L, Hkv * G, generator=g) + 2.0
    g_rw = torch.randn(B, L, Hkv * G, K, generator=g).bfloat16()
    g_lw = torch.randn(B, L, Hkv * G, generator=g).bfloat16()
    return scores, idx, bias, lse, g_rw, g_lw


def _oracle_grads(scores, idx, bias, lse, g_rw, g_lw, gate_offset=None, gate_scale=None, T=1.0):
    s = scores.float().requires_grad_(True)
    b = bias.clone().requires_grad_(True)
    l = lse.clone().requires_grad_(True)
    go = None if gate_offset is None else torch.tensor(gate_offset, requires_grad=True)
    gs = None if gate_scale is None else torch.tensor(gate_scale, requires_grad=True)
    rw, lw = O.route_weights(s, idx, b, l, temperature=T, gate_offset=go, gate_scale=gs)
    (rw * g_rw.float()).sum().add_((lw * g_lw.float()).sum()).backward()
    return (s.grad, b.grad, l.grad, None if gs is None else gs.grad,
            None if go is None else go.grad)


def _close(got, exp, what, atol=1e-5, rtol=1e-4):
    torch.testing.assert_close(got.cpu().float(), exp.float(), atol=atol, rtol=rtol, msg=what)


@pytest.mark.parametrize("form,K,T", [("plain", 31, 1.0), ("plain", 32, 0.7), ("offset", 32, 1.0),
                                      ("affine", 32, 1.0), ("affine", 20, 1.4), ("affine", 64, 0.8)])
def test_route_weights_backward_vs_oracle(form, K, T):
    _note(f"route weights bwd form={form} K={K} T={T}")
    B, L, Hkv, G, C = 1, 300, 4, 7, 96
    scores, idx, bias, lse, g_rw, g_lw = _case(40 + K, B, L, Hkv, G, K, C)
    off = {"plain": None, "offset": 0.35, "affine": -0.25}[form]
    scale = 0.9 if form == "affine" else None
    d_s, d_b, d_l, d_g = route_weights_backward(
        scores.to(DEV), idx.to(DEV), bias.to(DEV), lse.to(DEV), g_rw.to(DEV), g_lw.to(DEV),
        temperature=T, gate_offset=off, gate_scale=scale)
    e_s, e_b, e_l, e_gs, e_go = _oracle_grads(scores, idx, bias, lse, g_rw, g_lw, off, scale, T)
    _close(d_s, e_s, "d_scores")
    _close(d_b, e_b, "d_bias", atol=5e-5, rtol=2e-4)
    _close(d_l, e_l, "d_local_lse")
    if scale is not None:
        assert abs(float(d_g[0]) - float(e_gs)) <= 1e-3 * max(1.0, abs(float(e_gs)))
    if off is not None:
        assert abs(float(d_g[1]) - float(e_go)) <= 1e-3 * max(1.0, abs(float(e_go)))


def test_route_weights_backward_masked_rows_are_zero():
    _note("route weights bwd masked rows")
    B, L, Hkv, G, K, C = 1, 8, 2, 7, 8, 16
    scores, idx, bias, lse, g_rw, g_lw = _case(77, B, L, Hkv, G, K, C)
    idx[0, 2, 0, :] = -1                       # no valid chunk: affine rows constant
    lse[0, 2, :G] = float("-inf")              # and the plain rows fully masked
    idx[0, 5, 1, :] = -1                       # no valid chunk, finite local
    for kw in (dict(), dict(gate_offset=0.1, gate_scale=1.1)):
        d_s, d_b, d_l, _ = route_weights_backward(
            scores.to(DEV), idx.to(DEV), bias.to(DEV), lse.to(DEV), g_rw.to(DEV), g_lw.to(DEV),
            **kw)
        assert torch.isfinite(d_s).all() and torch.isfinite(d_l).all()
        assert float(d_s[0, 2, :G].abs().sum()) == 0.0 and float(d_l[0, 2, :G].abs().sum()) == 0.0
        assert float(d_s[0, 5, G:].abs().sum()) == 0.0
        e_s, e_b, e_l, _, _ = _oracle_grads(scores, idx, bias, lse, g_rw, g_lw,
                                            kw.get("gate_offset"), kw.get("gate_scale"))
        _close(d_s, torch.nan_to_num(e_s), "d_scores")
        _close(d_l, torch.nan_to_num(e_l), "d_local_lse")
        _close(d_b, e_b, "d_bias", atol=5e-5, rtol=2e-4)


@pytest.mark.parametrize("affine", [False, True])
def test_route_weights_autograd_api(affine):
    _note(f"route weights autograd affine={affine}")
    B, L, Hkv, G, K, C = 1, 64, 2, 7, 31 if not affine else 32, 40
    scores, idx, bias, lse, g_rw, g_lw = _case(90, B, L, Hkv, G, K, C)
    s = scores.to(DEV).requires_grad_(True)
    b = bias.to(DEV).requires_grad_(True)
    l = lse.to(DEV).requires_grad_(True)
    if affine:
        gs = torch.tensor(0.8, device=DEV, requires_grad=True)
        go = torch.tensor(0.2, device=DEV, requires_grad=True)
        rw, lw = mrsa.route_weights_torch(s, idx.to(DEV), b, l, temperature=1.0,
                                          gate_offset=go, gate_scale=gs)
    else:
        rw, lw = mrsa.route_weights(s, idx.to(DEV), b, l)
    (rw.float() * g_rw.to(DEV).float()).sum().add_((lw.float() * g_lw.to(DEV).float()).sum()).backward()
    e_s, e_b, e_l, e_gs, e_go = _oracle_grads(scores, idx, bias, lse, g_rw, g_lw,
                                              0.2 if affine else None, 0.8 if affine else None)
    assert s.grad.dtype == torch.bfloat16 and b.grad.dtype == torch.float32
    _close(s.grad, e_s.bfloat16(), "scores.grad", atol=1e-5, rtol=8e-3)
    _close(b.grad, e_b, "prior_bias.grad", atol=5e-5, rtol=2e-4)
    _close(l.grad, e_l, "local_lse.grad")
    if affine:
        assert abs(float(gs.grad) - float(e_gs)) <= 1e-3 * max(1.0, abs(float(e_gs)))
        assert abs(float(go.grad) - float(e_go)) <= 1e-3 * max(1.0, abs(float(e_go)))


@pytest.mark.parametrize("D", [128, 64, 256, 40])
def test_fusion_backward_vs_oracle(D):
    _note(f"fusion bwd D={D}")
    g = torch.Generator().manual_seed(D)
    shape = (2, 97, 5, D)
    r = torch.randn(*shape, generator=g).bfloat16()
    lo = torch.randn(*shape, generator=g).bfloat16()
    w = torch.rand(*shape[:-1], generator=g).bfloat16()
    go = torch.randn(*shape, generator=g).bfloat16()
    rr, ll, ww = (x.clone().requires_grad_(True) for x in (r, lo, w))
    O.fuse_outputs(rr, ll, ww).backward(go)
    d_r, d_l, d_w = fuse_hils_outputs_backward(lo.to(DEV), w.to(DEV), go.to(DEV))
    assert torch.equal(d_r.cpu(), rr.grad)
    assert torch.equal(d_l.cpu(), ll.grad)
    torch.testing.assert_close(d_w.cpu().float(), ww.grad.float(), atol=1e-6, rtol=8e-3)
    # Through the autograd API.
    a, b_, c = (x.to(DEV).requires_grad_(True) for x in (r, lo, w))
    mrsa.fuse_hils_outputs(a, b_, c).backward(go.to(DEV))
    assert torch.equal(a.grad.cpu(), rr.grad) and torch.equal(b_.grad.cpu(), ll.grad)
    torch.testing.assert_close(c.grad.cpu().float(), ww.grad.float(), atol=1e-6, rtol=8e-3)


def _pool_inputs(seed, C, S, H, G, D):
    g = torch.Generator().manual_seed(seed)
    mu = torch.randn(1, C, H, G, D, generator=g).bfloat16()
    k = torch.randn(1, C, S, H, D, generator=g).bfloat16()
    valid = torch.rand(1, C, S, generator=g) > 0.1
    valid[0, 1, 0] = False            # masked slot 0
    valid[0, 2, :-1] = False          # invalid chunk
    g_lmk = torch.randn(1, C, H, G, D, generator=g).bfloat16()
    g_ent = torch.randn(1, C, H, G, generator=g)
    return mu, k, valid, g_lmk, g_ent


def _rel(a, b):
    return float((a.float() - b.float()).norm() / b.float().norm().clamp_min(1e-12))


@pytest.mark.parametrize("C,S,H,G,D", [(37, 64, 4, 7, 128), (9, 128, 2, 16, 256), (11, 32, 3, 5, 64)])
def test_pool_backward_vs_oracle(C, S, H, G, D):
    _note(f"pool bwd C={C} S={S} H={H} G={G} D={D}")
    mu, k, valid, g_lmk, g_ent = _pool_inputs(C + S, C, S, H, G, D)
    scale = D ** -0.5
    d_mu, d_k = mrsa.chunk_attn_pool_gqa_backward(mu.to(DEV), k.to(DEV), valid.to(DEV),
                                                  g_lmk.to(DEV), g_ent.to(DEV), scale)
    e_mu, e_k = O.chunk_attn_pool_bwd(mu, k, valid, g_lmk, g_ent, scale)
    assert _rel(d_mu.cpu(), e_mu) < 5e-3 and _rel(d_k.cpu(), e_k) < 5e-3
    torch.testing.assert_close(d_mu.cpu().float(), e_mu.float(), atol=2e-2, rtol=2e-2)
    torch.testing.assert_close(d_k.cpu().float(), e_k.float(), atol=2e-2, rtol=2e-2)
    assert float(d_mu[0, 2].abs().sum()) == 0 and float(d_k[0, 2].abs().sum()) == 0
    # autograd API, with and without the entropy gradient
    m = mu.to(DEV).requires_grad_(True)
    kk = k.to(DEV).requires_grad_(True)
    lmk, ent = mrsa.chunk_attn_pool_gqa(m, kk, valid.to(DEV), scale)
    torch.autograd.backward([lmk, ent], [g_lmk.to(DEV), g_ent.to(DEV)])
    assert torch.equal(m.grad, d_mu) and torch.equal(kk.grad, d_k)
    m.grad = None
    lmk, _ = mrsa.chunk_attn_pool_gqa(m, k.to(DEV), valid.to(DEV), scale)
    lmk.backward(g_lmk.to(DEV))
    e_mu0, _ = O.chunk_attn_pool_bwd(mu, k, valid, g_lmk, None, scale)
    assert _rel(m.grad.cpu(), e_mu0) < 5e-3


def test_pool_backward_dense_groups1_vs_autograd():
    _note("pool bwd dense G=1")
    C, S, H, G, D = 13, 64, 4, 1, 128
    mu, k, valid, g_lmk, g_ent = _pool_inputs(5, C, S, H, G, D)
    valid[0, 3, :] = False            # fully masked chunk
    scale = D ** -0.5
    d_mu, d_k = mrsa.chunk_attn_pool_gqa_backward(mu.to(DEV), k.to(DEV), valid.to(DEV),
                                                  g_lmk.to(DEV), g_ent.to(DEV), scale)
    m = mu.float().requires_grad_(True)
    kk = k.float().requires_grad_(True)
    lmk, ent = O.chunk_attn_pool(m, kk, valid, scale, dense=True)
    (lmk * g_lmk.float()).sum().add_((ent * g_ent).sum()).backward()
    assert _rel(d_mu.cpu(), m.grad) < 5e-3 and _rel(d_k.cpu(), kk.grad) < 5e-3
    torch.testing.assert_close(d_k.cpu().float(), kk.grad, atol=2e-2, rtol=2e-2)


def test_pool_prior_backward():
    _note("pool prior bwd")
    C, S, H, G, D = 21, 64, 4, 7, 128
    mu, k, valid, g_lmk, g_ent = _pool_inputs(6, C, S, H, G, D)
    scale_t = torch.rand(H * G) + 0.5
    g_prior = torch.randn(1, C, H, G)
    m = mu.to(DEV).requires_grad_(True)
    bs = scale_t.to(DEV).requires_grad_(True)
    lmk, ent, prior = mrsa.chunk_attn_pool_gqa_prior(m, k.to(DEV), valid.to(DEV), bs)
    torch.autograd.backward([lmk, prior], [g_lmk.to(DEV), g_prior.to(DEV)])
    _, e_ent = O.chunk_attn_pool(mu, k, valid)
    e_scale = (g_prior * e_ent).sum(dim=(0, 1)).reshape(-1)
    torch.testing.assert_close(bs.grad.cpu(), e_scale, atol=1e-3, rtol=1e-3)
    e_mu, _ = O.chunk_attn_pool_bwd(mu, k, valid, g_lmk, g_prior * scale_t.reshape(H, G), D ** -0.5)
    assert _rel(m.grad.cpu(), e_mu) < 5e-3


# ---------------------------------------------------------------------------
# Routed (selected-chunk) attention backward (ops/hils_fwd_bwd_head.py:573-910)
# against the oracle's autograd.  The kernel rounds P, bf16(w dO) and dS to
# bf16 where the reference does and returns bf16 gradients, so each gradient
# is compared by its relative norm error (the reference test's measure for
# this op, test_hils_non_power_two_topk.py:139-142: rel. norm < 0.02).
# ---------------------------------------------------------------------------
def _rel_err(a, b):
    a = a.float().cpu()
    b = b.float().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-12))


@pytest.mark.parametrize("keep", [False, True])
def test_selected_attention_backward_vs_oracle(keep):
    _note(f"selected attention backward keep={keep}")
    B, Lq, Hkv, G, D, C, K = 1, 192, 4, 7, 128, 16, 8
    Lk = C * 64
    g = torch.Generator().manual_seed(70 + keep)
    q = (torch.randn(B, Lq, Hkv * G, D, generator=g) * 0.5).bfloat16()
    k = (torch.randn(B, Lk, Hkv, D, generator=g) * 0.5).bfloat16()
    v = torch.randn(B, Lk, Hkv, D, generator=g).bfloat16()
    w = torch.rand(B, Lq, Hkv * G, K, generator=g).bfloat16()
    idx = torch.stack([torch.randperm(C, generator=g)[:K] for _ in range(B * Lq * Hkv)])
    idx = idx.reshape(B, Lq, Hkv, K).int()
    idx[0, 5, 1, 5:] = -1              # list end
    idx[0, 6, 2, 3] = idx[0, 6, 2, 1]  # a chunk listed twice
    idx[0, 7, 0, 2] = C + 3            # out of range: skipped
    valid = torch.rand(B, Lk, generator=g) > 0.05
    token_keep = None
    if keep:
        token_keep = (torch.rand(B, Lq, Hkv, K, 64, generator=g) > 0.3).to(torch.int8)
    dout = torch.randn(B, Lq, Hkv * G, D, generator=g).bfloat16()

    tq, tk, tv, tw = (t.to(DEV).requires_grad_(True) for t in (q, k, v, w))
    out = mrsa.HiLS_block_M_head(tq, tk, tv, tw, idx.to(DEV), key_valid=valid.to(DEV),
                                 token_keep=None if token_keep is None else token_keep.to(DEV))
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()

    rq, rk, rv, rw = (t.float().requires_grad_(True) for t in (q, k, v, w))
    ref = O.selected_attention(rq, rk, rv, rw, idx, valid, token_keep=token_keep)
    (ref * dout.float()).sum().backward()
    for name, got, exp in (("dq", tq.grad, rq.grad), ("dk", tk.grad, rk.grad),
                           ("dv", tv.grad, rv.grad), ("dw", tw.grad, rw.grad)):
        assert got.dtype == torch.bfloat16, name
        err = _rel_err(got, exp)
        print(f"  {name}: rel-norm error {err:.3e}", flush=True)
        assert err < 2e-2, (name, err)
    # slots past a list's end or out of range get zero weight gradient
    assert float(tw.grad[0, 5, 7:14, 5:].abs().max()) == 0.0
    assert float(tw.grad[0, 7, 0:7, 2].abs().max()) == 0.0


@pytest.mark.parametrize("keep", [False, True])
def test_selected_attention_alibi_forward_backward_vs_oracle(keep):
    # HiLS_block_M_head(slope=...): the ALiBi bias -slope[head] max(0, 62 - s)
    # on the raw logits (ops/hils_fwd_bwd_head.py:445-451, :755-760), forward
    # and backward against the oracle's autograd.  Slopes of the usual ALiBi
    # scale (2^-k) and one large one, so the bias moves the softmax.
    _note(f"selected attention with ALiBi slopes keep={keep}")
    B, Lq, Hkv, G, D, C, K = 1, 160, 4, 7, 128, 16, 8
    Lk = C * 64
    g = torch.Generator().manual_seed(170 + keep)
    q = (torch.randn(B, Lq, Hkv * G, D, generator=g) * 0.5).bfloat16()
    k = (torch.randn(B, Lk, Hkv, D, generator=g) * 0.5).bfloat16()
    v = torch.randn(B, Lk, Hkv, D, generator=g).bfloat16()
    w = torch.rand(B, Lq, Hkv * G, K, generator=g).bfloat16()
    idx = torch.stack([torch.randperm(C, generator=g)[:K] for _ in range(B * Lq * Hkv)])
    idx = idx.reshape(B, Lq, Hkv, K).int()
    idx[0, 5, 1, 5:] = -1
    valid = torch.rand(B, Lk, generator=g) > 0.05
    slope = torch.tensor([2.0 ** -(1 + h % 8) for h in range(Hkv * G)])
    slope[3] = 1.5
    token_keep = None
    if keep:
        token_keep = (torch.rand(B, Lq, Hkv, K, 64, generator=g) > 0.3).to(torch.int8)
    dout = torch.randn(B, Lq, Hkv * G, D, generator=g).bfloat16()

    tq, tk, tv, tw = (t.to(DEV).requires_grad_(True) for t in (q, k, v, w))
    out = mrsa.HiLS_block_M_head(tq, tk, tv, tw, idx.to(DEV), key_valid=valid.to(DEV),
                                 slope=slope.to(DEV),
                                 token_keep=None if token_keep is None else token_keep.to(DEV))
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()

    rq, rk, rv, rw = (t.float().requires_grad_(True) for t in (q, k, v, w))
    ref = O.selected_attention(rq, rk, rv, rw, idx, valid, token_keep=token_keep, slope=slope)
    (ref * dout.float()).sum().backward()
    plain = O.selected_attention(q, k, v, w, idx, valid, token_keep=token_keep)
    assert _rel_err(plain, ref.detach()) > 0.05  # the slopes matter at this size
    err = _rel_err(out.detach(), ref.detach())
    print(f"  out: rel-norm error {err:.3e}", flush=True)
    assert err < 1e-2, err
    for name, got, exp in (("dq", tq.grad, rq.grad), ("dk", tk.grad, rk.grad),
                           ("dv", tv.grad, rv.grad), ("dw", tw.grad, rw.grad)):
        err = _rel_err(got, exp)
        print(f"  {name}: rel-norm error {err:.3e}", flush=True)
        assert err < 2e-2, (name, err)


def test_selected_attention_alibi_walk_split_and_fixed_order():
    # The ALiBi instances of the walk split (partials summed by the second
    # kernel) and of the fixed accumulation order give the one-launch result;
    # the fixed order twice gives the same bits.
    _note("selected attention with ALiBi: walk split and fixed order")
    from mrsa.sparse_attention import kv_fragments, selected_attention_alibi_launch
    B, Lq, Hkv, G, D, C, K = 1, 64, 4, 7, 128, 32, 16
    Lk = C * 64
    g = torch.Generator().manual_seed(181)
    q = (torch.randn(B, Lq, Hkv * G, D, generator=g) * 0.5).bfloat16().to(DEV)
    k = (torch.randn(B, Lk, Hkv, D, generator=g) * 0.5).bfloat16().to(DEV)
    v = torch.randn(B, Lk, Hkv, D, generator=g).bfloat16().to(DEV)
    w = torch.rand(B, Lq, Hkv * G, K, generator=g).bfloat16().to(DEV)
    idx = torch.stack([torch.randperm(C, generator=g)[:K].sort().values
                       for _ in range(B * Lq * Hkv)]).reshape(B, Lq, Hkv, K).int().to(DEV)
    slope = torch.tensor([0.25 * (1 + h % 3) for h in range(Hkv * G)], device=DEV)
    frags = kv_fragments(k, v)
    one = selected_attention_alibi_launch(q, frags, w, idx, None, 64, slope, parts=1)
    split = selected_attention_alibi_launch(q, frags, w, idx, None, 64, slope, parts=8)
    det1 = selected_attention_alibi_launch(q, frags, w, idx, None, 64, slope, parts=1,
                                           deterministic=True)
    det2 = selected_attention_alibi_launch(q, frags, w, idx, None, 64, slope, parts=1,
                                           deterministic=True)
    torch.cuda.synchronize()
    assert torch.equal(det1, det2)
    ref = O.selected_attention(q.cpu(), k.cpu(), v.cpu(), w.cpu(), idx.cpu(), None,
                               slope=slope.cpu())
    for name, got in (("one", one), ("split", split), ("det", det1)):
        err = _rel_err(got, ref)
        print(f"  {name}: rel-norm error {err:.3e}", flush=True)
        assert err < 1e-2, (name, err)


@pytest.mark.parametrize("L,W,inert,G,Hkv", [(1024, 319, 64, 7, 4), (1024, 1280, 0, 7, 2),
                                              (512, 100, 64, 4, 2), (640, 200, 0, 8, 2),
                                              (448, 150, 64, 3, 3), (256, 40, 0, 1, 2)])
def test_local_attention_backward_vs_oracle(L, W, inert, G, Hkv):
    # The window attention's gradient (flash_attn_func's, as
    # bidir_local_attention uses it) against autograd of the oracle: dq, dk,
    # dv; inert keys (failed key_valid, landmark slots) get exactly zero dk / dv.
    _note(f"local attention backward L={L} W={W} inert={inert} G={G} Hkv={Hkv}")
    from mrsa.local_attention import local_attention_autograd
    D = 128
    g = torch.Generator().manual_seed(300 + L + W + G)
    q = (torch.randn(1, L, Hkv * G, D, generator=g) * 0.5).bfloat16()
    k = (torch.randn(1, L, Hkv, D, generator=g) * 0.5).bfloat16()
    v = torch.randn(1, L, Hkv, D, generator=g).bfloat16()
    valid = torch.rand(1, L, generator=g) > 0.05
    dout = torch.randn(1, L, Hkv * G, D, generator=g).bfloat16()

    tq, tk, tv = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    out, lse = local_attention_autograd(tq, tk, tv, valid.to(DEV), W, inert)
    assert not lse.requires_grad
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()

    rq, rk, rv = (t.float().requires_grad_(True) for t in (q, k, v))
    ref, _ = O.local_attention(rq, rk, rv, valid, W, inert)
    (ref * dout.float()).sum().backward()
    for name, got, exp in (("dq", tq.grad, rq.grad), ("dk", tk.grad, rk.grad),
                           ("dv", tv.grad, rv.grad)):
        assert got.dtype == torch.bfloat16, name
        err = _rel_err(got, exp)
        print(f"  {name}: rel-norm error {err:.3e}", flush=True)
        assert err < 2e-2, (name, err)
    dead = ~valid[0]
    if inert:
        dead |= (torch.arange(L) + 1) % inert == 0
    assert float(tk.grad[0, dead.to(DEV)].abs().max()) == 0.0
    assert float(tv.grad[0, dead.to(DEV)].abs().max()) == 0.0


def test_bidir_local_attention_and_swa_are_differentiable():
    # The drop-ins carry the gradient through the public API: the route
    # layer's window (skip_inert_slots: radius 256 + 63, landmark slots inert)
    # and the SWA layer's.
    _note("bidir_local_attention / swa_attention backward")
    from mrsa.route_layer import swa_attention
    L, Hkv, G, D = 512, 2, 7, 128
    g = torch.Generator().manual_seed(321)
    q = (torch.randn(1, L, Hkv * G, D, generator=g) * 0.5).bfloat16()
    k = (torch.randn(1, L, Hkv, D, generator=g) * 0.5).bfloat16()
    v = torch.randn(1, L, Hkv, D, generator=g).bfloat16()
    valid = torch.ones(1, L, dtype=torch.bool)
    dout = torch.randn(1, L, Hkv * G, D, generator=g).bfloat16()
    for name, fn, W, inert in (
            ("bidir", lambda a, b, c: mrsa.bidir_local_attention(
                a, b, c, valid.to(DEV), 256, 64, skip_inert_slots=True)[0], 319, 64),
            ("swa", lambda a, b, c: swa_attention(a, b, c, valid.to(DEV), window=200), 200, 0)):
        tq, tk, tv = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
        fn(tq, tk, tv).backward(dout.to(DEV))
        rq, rk, rv = (t.float().requires_grad_(True) for t in (q, k, v))
        (O.local_attention(rq, rk, rv, valid, W, inert)[0] * dout.float()).sum().backward()
        for gname, got, exp in (("dq", tq.grad, rq.grad), ("dk", tk.grad, rk.grad),
                                ("dv", tv.grad, rv.grad)):
            err = _rel_err(got, exp)
            print(f"  {name} {gname}: rel-norm error {err:.3e}", flush=True)
            assert err < 2e-2, (name, gname, err)


def test_selected_attention_backward_two_runs_agree_within_rounding():
    # The routed backward is not bit-reproducible: each chunk's (query, slot)
    # pair list is filled in LDS-atomic order, dK/dV of multi-segment chunks
    # and dQ are fp32 atomic adds.  Two runs on the same inputs may therefore
    # differ where an fp32 sum in another order rounds to another bf16 value;
    # the differences stay at the bf16 rounding level of each gradient.
    _note("selected attention backward, two runs on the same inputs")
    B, Lq, Hkv, G, D, C, K = 1, 256, 4, 7, 128, 16, 8
    Lk = C * 64
    g = torch.Generator().manual_seed(91)
    q = (torch.randn(B, Lq, Hkv * G, D, generator=g) * 0.5).bfloat16().to(DEV)
    k = (torch.randn(B, Lk, Hkv, D, generator=g) * 0.5).bfloat16().to(DEV)
    v = torch.randn(B, Lk, Hkv, D, generator=g).bfloat16().to(DEV)
    w = torch.rand(B, Lq, Hkv * G, K, generator=g).bfloat16().to(DEV)
    idx = torch.stack([torch.randperm(C, generator=g)[:K].sort().values
                       for _ in range(B * Lq * Hkv)]).reshape(B, Lq, Hkv, K).int().to(DEV)
    dout = torch.randn(B, Lq, Hkv * G, D, generator=g).bfloat16().to(DEV)
    runs = []
    for _ in range(2):
        tq, tk, tv, tw = (t.clone().requires_grad_(True) for t in (q, k, v, w))
        mrsa.HiLS_block_M_head(tq, tk, tv, tw, idx).backward(dout)
        torch.cuda.synchronize()
        runs.append([t.grad.float().cpu() for t in (tq, tk, tv, tw)])
    for name, a, b in zip(("dq", "dk", "dv", "dw"), runs[0], runs[1]):
        diff = float((a - b).abs().max())
        rel = _rel_err(a, b)
        print(f"  {name}: run-to-run max diff {diff:.3e}, rel-norm {rel:.3e}", flush=True)
        assert rel < 2e-3, (name, rel)
        assert diff <= 2.0 ** -6 * float(b.abs().max()), (name, diff)


def test_selected_attention_backward_split_query_block():
    # A 32-query block against a longer cache (the cached step's shape): the
    # forward takes the walk split, the backward is the same kernel.
    _note("selected attention backward, 32 queries against 64 chunks")
    B, Lq, Hkv, G, D, C, K = 1, 32, 4, 7, 128, 64, 16
    Lk = C * 64
    g = torch.Generator().manual_seed(80)
    q = (torch.randn(B, Lq, Hkv * G, D, generator=g) * 0.5).bfloat16()
    k = (torch.randn(B, Lk, Hkv, D, generator=g) * 0.5).bfloat16()
    v = torch.randn(B, Lk, Hkv, D, generator=g).bfloat16()
    w = torch.rand(B, Lq, Hkv * G, K, generator=g).bfloat16()
    idx = torch.stack([torch.randperm(C, generator=g)[:K].sort().values
                       for _ in range(B * Lq * Hkv)]).reshape(B, Lq, Hkv, K).int()
    dout = torch.randn(B, Lq, Hkv * G, D, generator=g).bfloat16()
    tq, tk, tv, tw = (t.to(DEV).requires_grad_(True) for t in (q, k, v, w))
    valid = torch.ones(B, Lk, dtype=torch.bool)
    out = mrsa.selected_attention_g7(tq, tk, tv, tw, idx.to(DEV), valid.to(DEV), 64, True)
    out.backward(dout.to(DEV))
    rq, rk, rv, rw = (t.float().requires_grad_(True) for t in (q, k, v, w))
    ref = O.selected_attention(rq, rk, rv, rw, idx, valid)
    (ref * dout.float()).sum().backward()
    for name, got, exp in (("dq", tq.grad, rq.grad), ("dk", tk.grad, rk.grad),
                           ("dv", tv.grad, rv.grad), ("dw", tw.grad, rw.grad)):
        err = _rel_err(got, exp)
        print(f"  {name}: rel-norm error {err:.3e}", flush=True)
        assert err < 2e-2, (name, err)


# -- route-score backward (ops/topk_head_softmax.py:1074-1122) ---------------
def _score_case(seed, B, L, Hkv, G, K, C, per_head, D=128):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, L, Hkv, G, D, generator=g).bfloat16()
    lm = torch.randn(B, C, Hkv * G if per_head else Hkv, D, generator=g).bfloat16()
    keys = torch.rand(B * L * Hkv, C, generator=g)
    idx = keys.topk(min(K, C), dim=-1).indices.sort(dim=-1).values.int()
    if K > C:
        idx = torch.cat([idx, torch.full((idx.shape[0], K - C), -1, dtype=torch.int32)], -1)
    idx = idx.reshape(B, L, Hkv, K)
    idx[0, min(3, L - 1), 0, K // 2:] = -1
    idx[0, L - 1, Hkv - 1, 0] = C + 5
    gs = torch.randn(B, L, Hkv, G, K, generator=g).bfloat16()
    return q, lm, idx, gs


@pytest.mark.parametrize("B,L,Hkv,G,K,C,per_head,fp32", [
    (1, 100, 2, 7, 16, 64, True, False),
    (2, 77, 2, 3, 8, 40, False, False),
    (1, 70, 1, 7, 32, 300, True, False),     # two chunk blocks (fp32 grad_q path)
    (1, 1000, 4, 7, 32, 256, True, False),   # config-2 shape, fewer rows
    (1, 64, 2, 7, 32, 520, False, True),     # three blocks, shared, fp32 grads
])
def test_route_score_backward_vs_oracle(B, L, Hkv, G, K, C, per_head, fp32):
    _note(f"route_score_bwd B={B} L={L} Hkv={Hkv} G={G} K={K} C={C} per_head={per_head}")
    q, lm, idx, gs = _score_case(7 + C, B, L, Hkv, G, K, C, per_head)
    if fp32:
        gs = gs.float()
    scale = 128 ** -0.5
    eq, el = O.route_score_bwd(q, lm, idx, gs, scale)
    gq, gl = torch.ops.mrsa.route_score_bwd(q.to(DEV), lm.to(DEV), idx.to(DEV), gs.to(DEV),
                                             scale)
    gq2, gl2 = torch.ops.mrsa.route_score_bwd(q.to(DEV), lm.to(DEV), idx.to(DEV), gs.to(DEV),
                                               scale)
    torch.cuda.synchronize()
    assert gq.dtype == torch.bfloat16 and gl.dtype == torch.bfloat16
    assert torch.equal(gq, gq2) and torch.equal(gl, gl2), "not deterministic"
    for name, got, exp in (("grad_q", gq, eq), ("grad_lmks", gl, el)):
        got = got.float().cpu()
        err = _rel_err(got, exp)
        print(f"  {name}: rel-norm error {err:.3e}")
        assert err < 5e-3, name
        # one bf16 rounding of the fp32 result (plus fp32 order noise)
        assert ((got - exp).abs() <= exp.abs() * 2 ** -8 + 1e-3).all(), name


def test_route_score_autograd_through_online_softmax_topk_head():
    _note("route_score autograd via online_softmax_topk_head")
    B, L, Hkv, G, D, C, K = 1, 256, 2, 7, 128, 64, 16
    g = torch.Generator().manual_seed(5)
    q = torch.randn(B, L, Hkv * G, D, generator=g).bfloat16().to(DEV).requires_grad_(True)
    lm = torch.randn(B, C, Hkv * G, D, generator=g).bfloat16().to(DEV).requires_grad_(True)
    lse = (torch.randn(B, L, Hkv * G, generator=g) + 3).to(DEV)
    idx, sc = mrsa.online_softmax_topk_head(q, lm, lse, K, 64, 0, is_causal=False, G=G)
    assert idx.dtype == torch.int32 and sc.shape == (B, L, Hkv * G, K)
    assert not idx.requires_grad and sc.requires_grad
    gout = torch.randn(B, L, Hkv * G, K, generator=g).bfloat16().to(DEV)
    live = (idx >= 0)[:, :, :, None, :].expand(B, L, Hkv, G, K).reshape(B, L, Hkv * G, K)
    gout = torch.where(live, gout, torch.zeros_like(gout))
    (torch.where(live, sc.float(), torch.zeros_like(sc.float())) * gout.float()).sum().backward()
    eq, el = O.route_score_bwd(q.detach().cpu().reshape(B, L, Hkv, G, D), lm.detach().cpu(),
                               idx.cpu(), gout.cpu().reshape(B, L, Hkv, G, K), D ** -0.5)
    for name, got, exp in (("q", q.grad, eq.reshape(B, L, Hkv * G, D)), ("lmks", lm.grad, el)):
        err = _rel_err(got.float().cpu(), exp)
        print(f"  grad {name}: rel-norm error {err:.3e}")
        assert got.dtype == torch.bfloat16 and err < 5e-3, name


def test_selected_attention_backward_long_chunk_lists():
    # every query routes to chunk 3, so its pair list (1100 pairs per batch and
    # KV head) spans two work segments whose dK / dV sums are added; batch 2.
    _note("selected_attention_bwd long chunk lists B=2 Lq=1100")
    B, Lq, Lk, Hkv, G, D, K = 2, 1100, 1024, 2, 7, 128, 4
    C = Lk // 64
    g = torch.Generator().manual_seed(21)
    q = torch.randn(B, Lq, Hkv * G, D, generator=g).bfloat16()
    k = torch.randn(B, Lk, Hkv, D, generator=g).bfloat16()
    v = torch.randn(B, Lk, Hkv, D, generator=g).bfloat16()
    w = torch.rand(B, Lq, Hkv * G, K, generator=g).bfloat16()
    rest = torch.stack([torch.randperm(C - 1, generator=g)[:K - 1] for _ in range(B * Lq * Hkv)])
    rest = rest + (rest >= 3).long()  # chunks other than 3
    idx = torch.cat([torch.full((B * Lq * Hkv, 1), 3), rest], -1).sort(-1).values
    idx = idx.reshape(B, Lq, Hkv, K).int()
    valid = torch.rand(B, Lk, generator=g) > 0.05
    dout = torch.randn(B, Lq, Hkv * G, D, generator=g).bfloat16()
    tq, tk, tv, tw = (t.to(DEV).requires_grad_(True) for t in (q, k, v, w))
    out = mrsa.HiLS_block_M_head(tq, tk, tv, tw, idx.to(DEV), key_valid=valid.to(DEV))
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    rq, rk, rv, rw = (t.float().requires_grad_(True) for t in (q, k, v, w))
    ref = O.selected_attention(rq, rk, rv, rw, idx, valid)
    (ref * dout.float()).sum().backward()
    for name, got, exp in (("dq", tq.grad, rq.grad), ("dk", tk.grad, rk.grad),
                           ("dv", tv.grad, rv.grad), ("dw", tw.grad, rw.grad)):
        err = _rel_err(got, exp)
        print(f"  {name}: rel-norm error {err:.3e}")
        assert err < 2e-2, name


@pytest.mark.parametrize("affine,T", [(False, 0.8), (True, 1.3)])
def test_route_weights_value_bonus_and_gumbel_vs_oracle(affine, T):
    # _route_weights_torch(selected_gumbel=, value_bonus=) (attention.py:172-181):
    # forward against the oracle, and the two terms' gradients equal the
    # scores' (fp32) -- each enters the logit as the score does.
    _note(f"route weights extras affine={affine} T={T}")
    B, L, Hkv, G, K, C = 1, 96, 2, 7, 32, 50
    scores, idx, bias, lse, g_rw, g_lw = _case(123, B, L, Hkv, G, K, C)
    g = torch.Generator().manual_seed(124)
    vb = torch.randn(scores.shape, generator=g) * 0.5
    gn = -torch.log(-torch.log(torch.rand(scores.shape, generator=g).clamp(1e-6, 1 - 1e-6)))
    kw = dict(temperature=T, gate_offset=0.2 if affine else None,
              gate_scale=0.9 if affine else None)
    rw, lw = mrsa.route_weights_torch(scores.to(DEV), idx.to(DEV), bias.to(DEV), lse.to(DEV),
                                      value_bonus=vb.to(DEV), selected_gumbel=gn.to(DEV), **kw)
    erw, elw = O.route_weights(scores, idx, bias, lse, value_bonus=vb, selected_gumbel=gn, **kw)
    _close(rw, erw.bfloat16(), "remote weights", atol=1e-3, rtol=8e-3)
    _close(lw, elw.bfloat16(), "local weight", atol=1e-3, rtol=8e-3)
    # without the terms the weights differ (the terms reach the kernel)
    rw0, _ = mrsa.route_weights_torch(scores.to(DEV), idx.to(DEV), bias.to(DEV), lse.to(DEV),
                                      **kw)
    assert not torch.equal(rw0, rw)
    # gradients
    s = scores.to(DEV).float().requires_grad_(True)
    v = vb.to(DEV).requires_grad_(True)
    n = gn.to(DEV).requires_grad_(True)
    rw, lw = mrsa.route_weights_torch(s, idx.to(DEV), bias.to(DEV), lse.to(DEV),
                                      value_bonus=v, selected_gumbel=n, **kw)
    (rw.float() * g_rw.to(DEV).float()).sum().add_((lw.float() * g_lw.to(DEV).float()).sum()).backward()
    so = scores.float().requires_grad_(True)
    vo = vb.clone().requires_grad_(True)
    go = None if not affine else torch.tensor(0.2)
    gs = None if not affine else torch.tensor(0.9)
    erw, elw = O.route_weights(so, idx, bias, lse, temperature=T, gate_offset=go, gate_scale=gs,
                               value_bonus=vo, selected_gumbel=gn)
    (erw * g_rw.float()).sum().add_((elw * g_lw.float()).sum()).backward()
    _close(v.grad, vo.grad, "value_bonus.grad")
    _close(s.grad, so.grad, "scores.grad")
    assert torch.equal(v.grad, n.grad) and torch.equal(v.grad, s.grad)
