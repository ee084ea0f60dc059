"""Pins of the oracle's backward (its torch autograd) against closed forms.

The reference's route-weights backward kernel
(ops/hils_bidir_route_weights_tilelang.py:131-160) states the plain-form
gradient as d_logit = p * (g - sum_j p_j g_j), scattered into the bias by
chunk index; the fusion backward (ops/hils_bidir_output_fusion_tilelang.py:55-71)
as d_local = w g, d_weight = sum_d g l.  The affine form has no kernel in
the reference (its backward is autograd); it is pinned here by a
hand-derived chain rule and by central differences.
"""

import math

import torch

from oracle import mrsa_oracle as O


def _inputs(seed, B=1, L=4, H=2, G=3, K=5, C=9):
    g = torch.Generator().manual_seed(seed)
    scores = torch.randn(B, L, H * G, K, generator=g).bfloat16()
    idx = torch.randint(0, C, (B, L, H, K), generator=g)
    idx[0, 1, 0, 3:] = -1
    idx[0, L - 1, H - 1, 0] = C + 2  # out of range: masked like -1
    bias = torch.rand(B, C, H, G, generator=g)
    lse = torch.randn(B, L, H * G, generator=g)
    g_rw = torch.randn(B, L, H * G, K, generator=g)
    g_lw = torch.randn(B, L, H * G, generator=g)
    return scores, idx, bias, lse, g_rw, g_lw


def _autograd(scores, idx, bias, lse, g_rw, g_lw, **kw):
    s = scores.float().requires_grad_(True)
    b = bias.clone().requires_grad_(True)
    l = lse.clone().requires_grad_(True)
    rw, lw = O.route_weights(s, idx, b, l, **kw)
    (rw * g_rw).sum().add_((lw * g_lw).sum()).backward()
    return s.grad, b.grad, l.grad


def test_plain_backward_matches_reference_kernel_formula():
    T, off = 0.7, 0.3
    scores, idx, bias, lse, g_rw, g_lw = _inputs(3)
    ds, db, dl = _autograd(scores, idx, bias, lse, g_rw, g_lw, temperature=T, gate_offset=off)
    B, L, Hq, K = scores.shape
    _, C, H, G = bias.shape
    eds = torch.zeros(B, L, Hq, K, dtype=torch.float64)
    edb = torch.zeros(B, C, H, G, dtype=torch.float64)
    edl = torch.zeros(B, L, Hq, dtype=torch.float64)
    for b in range(B):
        for t in range(L):
            for hq in range(Hq):
                h, gg = divmod(hq, G)
                logit = []
                for j in range(K):
                    c = int(idx[b, t, h, j])
                    ok = 0 <= c < C
                    logit.append((float(scores[b, t, hq, j]) + float(bias[b, c, h, gg])) / T
                                 if ok else -math.inf)
                logit.append((float(lse[b, t, hq]) - off) / T)
                m = max(logit)
                e = [math.exp(x - m) if x > -math.inf else 0.0 for x in logit]
                p = [x / sum(e) for x in e]
                gr = [float(g_rw[b, t, hq, j]) for j in range(K)] + [float(g_lw[b, t, hq])]
                delta = sum(pi * gi for pi, gi in zip(p, gr))
                dlogit = [pi * (gi - delta) / T for pi, gi in zip(p, gr)]
                for j in range(K):
                    c = int(idx[b, t, h, j])
                    if 0 <= c < C:
                        eds[b, t, hq, j] = dlogit[j]
                        edb[b, c, h, gg] += dlogit[j]
                edl[b, t, hq] = dlogit[K]
    torch.testing.assert_close(ds.double(), eds, atol=2e-6, rtol=1e-5)
    torch.testing.assert_close(db.double(), edb, atol=2e-6, rtol=1e-5)
    torch.testing.assert_close(dl.double(), edl, atol=2e-6, rtol=1e-5)


def test_affine_backward_matches_chain_rule():
    T, sc, off = 1.3, 0.8, -0.2
    scores, idx, bias, lse, g_rw, g_lw = _inputs(5)
    gs = torch.tensor(sc, requires_grad=True)
    go = torch.tensor(off, requires_grad=True)
    s = scores.float().requires_grad_(True)
    b = bias.clone().requires_grad_(True)
    l = lse.clone().requires_grad_(True)
    rw, lw = O.route_weights(s, idx, b, l, temperature=T, gate_offset=go, gate_scale=gs)
    (rw * g_rw).sum().add_((lw * g_lw).sum()).backward()
    B, L, Hq, K = scores.shape
    _, C, H, G = bias.shape
    eds = torch.zeros(B, L, Hq, K, dtype=torch.float64)
    edl = torch.zeros(B, L, Hq, dtype=torch.float64)
    dscale = doff = 0.0
    for t in range(L):
        for hq in range(Hq):
            h, gg = divmod(hq, G)
            x = []
            for j in range(K):
                c = int(idx[0, t, h, j])
                x.append((float(scores[0, t, hq, j]) + float(bias[0, c, h, gg])) / T
                         if 0 <= c < C else -math.inf)
            loc = float(lse[0, t, hq]) / T
            m = max(x)
            e = [math.exp(v - m) if v > -math.inf else 0.0 for v in x]
            q = [v / sum(e) for v in e]
            rl = m + math.log(sum(e))
            mass = 1.0 / (1.0 + math.exp(-(sc * (rl - loc) + off)))
            gr = [float(g_rw[0, t, hq, j]) for j in range(K)]
            dm = sum(qi * gi for qi, gi in zip(q, gr)) - float(g_lw[0, t, hq])
            dgate = dm * mass * (1 - mass)
            dq = [gi * mass for gi in gr]
            qdq = sum(qi * di for qi, di in zip(q, dq))
            for j in range(K):
                eds[0, t, hq, j] = (q[j] * (dq[j] - qdq) + dgate * sc * q[j]) / T
            edl[0, t, hq] = -dgate * sc / T
            dscale += dgate * (rl - loc)
            doff += dgate
    torch.testing.assert_close(s.grad.double(), eds, atol=2e-6, rtol=1e-5)
    torch.testing.assert_close(l.grad.double(), edl, atol=2e-6, rtol=1e-5)
    assert abs(float(gs.grad) - dscale) < 1e-4 * max(1.0, abs(dscale))
    assert abs(float(go.grad) - doff) < 1e-4 * max(1.0, abs(doff))


def test_affine_backward_central_differences():
    scores, idx, bias, lse, g_rw, g_lw = _inputs(8, L=2, H=1, G=2, K=4, C=6)

    def loss(bias_, lse_, gs_, go_):
        rw, lw = O.route_weights(scores, idx, bias_, lse_, temperature=0.9,
                                 gate_offset=go_, gate_scale=gs_)
        return float((rw.double() * g_rw).sum() + (lw.double() * g_lw).sum())

    b = bias.clone().requires_grad_(True)
    l = lse.clone().requires_grad_(True)
    gs = torch.tensor(1.2, requires_grad=True)
    go = torch.tensor(0.4, requires_grad=True)
    rw, lw = O.route_weights(scores, idx, b, l, temperature=0.9, gate_offset=go, gate_scale=gs)
    (rw * g_rw).sum().add_((lw * g_lw).sum()).backward()
    eps = 1e-2
    for flat in range(bias.numel()):
        bp, bm = bias.clone(), bias.clone()
        bp.view(-1)[flat] += eps
        bm.view(-1)[flat] -= eps
        fd = (loss(bp, lse, 1.2, 0.4) - loss(bm, lse, 1.2, 0.4)) / (2 * eps)
        assert abs(fd - float(b.grad.view(-1)[flat])) < 2e-3, flat
    for flat in range(lse.numel()):
        lp, lm = lse.clone(), lse.clone()
        lp.view(-1)[flat] += eps
        lm.view(-1)[flat] -= eps
        fd = (loss(bias, lp, 1.2, 0.4) - loss(bias, lm, 1.2, 0.4)) / (2 * eps)
        assert abs(fd - float(l.grad.view(-1)[flat])) < 2e-3, flat
    fd = (loss(bias, lse, 1.2 + eps, 0.4) - loss(bias, lse, 1.2 - eps, 0.4)) / (2 * eps)
    assert abs(fd - float(gs.grad)) < 2e-3
    fd = (loss(bias, lse, 1.2, 0.4 + eps) - loss(bias, lse, 1.2, 0.4 - eps)) / (2 * eps)
    assert abs(fd - float(go.grad)) < 2e-3


def test_fusion_backward_matches_reference_kernel_formula():
    g = torch.Generator().manual_seed(2)
    r = torch.randn(2, 3, 4, 16, generator=g).bfloat16()
    lo = torch.randn(2, 3, 4, 16, generator=g).bfloat16()
    w = torch.rand(2, 3, 4, generator=g).bfloat16()
    go = torch.randn(2, 3, 4, 16, generator=g).bfloat16()
    rr, ll, ww = (x.clone().requires_grad_(True) for x in (r, lo, w))
    O.fuse_outputs(rr, ll, ww).backward(go)
    assert torch.equal(rr.grad, go)
    assert torch.equal(ll.grad, (go.float() * w.float()[..., None]).bfloat16())
    torch.testing.assert_close(ww.grad.float(),
                               (go.float() * lo.float()).sum(-1).bfloat16().float(),
                               atol=0, rtol=8e-3)


def _pool_case(seed, B=1, C=3, S=16, H=2, G=3, D=8):
    g = torch.Generator().manual_seed(seed)
    mu = torch.randn(B, C, H, G, D, generator=g).bfloat16()
    k = torch.randn(B, C, S, H, D, generator=g).bfloat16()
    valid = torch.rand(B, C, S, generator=g) > 0.2
    valid[..., 0] = True
    g_lmk = torch.randn(B, C, H, G, D, generator=g).bfloat16()
    g_ent = torch.randn(B, C, H, G, generator=g)
    return mu, k, valid, g_lmk, g_ent


def _pool_autograd(mu, k, valid, g_lmk, g_ent, dense):
    m = mu.float().requires_grad_(True)
    kk = k.float().requires_grad_(True)
    lmk, ent = O.chunk_attn_pool(m, kk, valid, 0.4, dense=dense)
    (lmk * g_lmk.float()).sum().add_((ent * g_ent).sum()).backward()
    return m.grad, kk.grad


def _rel(a, b):
    return float((a.float() - b.float()).norm() / b.float().norm().clamp_min(1e-12))


def test_pool_backward_formula_matches_autograd():
    # _pool_gqa_bwd's logit gradient p((dP - sum p dP) - g_H (ln p + H)) is the
    # softmax/entropy chain rule; with slot 0 valid in every chunk the oracle's
    # kernel restatement equals autograd of the fused forward up to bf16 rounding.
    mu, k, valid, g_lmk, g_ent = _pool_case(11)
    d_mu, d_k = O.chunk_attn_pool_bwd(mu, k, valid, g_lmk, g_ent, 0.4)
    a_mu, a_k = _pool_autograd(mu, k, valid, g_lmk, g_ent, dense=False)
    assert _rel(d_mu, a_mu) < 1.5e-2 and _rel(d_k, a_k) < 1.5e-2


def test_pool_backward_masked_slot0_and_invalid_chunk():
    mu, k, valid, g_lmk, g_ent = _pool_case(12)
    valid[0, 1, 0] = False                 # masked slot 0: constant logit 0
    valid[0, 2, :-1] = False               # invalid chunk: zero gradients
    d_mu, d_k = O.chunk_attn_pool_bwd(mu, k, valid, g_lmk, g_ent, 0.4)
    a_mu, a_k = _pool_autograd(mu, k, valid, g_lmk, g_ent, dense=False)
    assert float(d_mu[0, 2].abs().sum()) == 0 and float(d_k[0, 2].abs().sum()) == 0
    assert _rel(d_k[0, 1, 1:], a_k[0, 1, 1:]) < 1.5e-2
    # the kernel's extra term: d_k[slot 0] picks up dlogit[:, 0] * mu, d_mu picks up
    # dlogit[:, 0] * k[0]; autograd has neither (the logit there is a constant)
    extra_k = (d_k[0, 1, 0].float() - a_k[0, 1, 0]).abs().sum()
    assert float(extra_k) > 1e-3
    assert _rel(d_mu[0, 0], a_mu[0, 0]) < 1.5e-2


def test_pool_dense_backward_is_torch_twin_autograd():
    # groups == 1: the reference differentiates _compact_pool_torch; central
    # differences pin the oracle's dense forward gradient.
    mu, k, valid, g_lmk, g_ent = _pool_case(13, G=1, S=8, D=4, C=2, H=1)
    valid[0, 1, :] = False                 # fully masked chunk: zero
    a_mu, a_k = _pool_autograd(mu, k, valid, g_lmk, g_ent, dense=True)
    assert float(a_mu[0, 1].abs().sum()) == 0

    def loss(m):
        lmk, ent = O.chunk_attn_pool(m, k.float(), valid, 0.4, dense=True)
        return float((lmk.double() * g_lmk.double()).sum() + (ent.double() * g_ent).sum())

    eps = 1e-2
    for flat in range(mu.numel()):
        mp, mm = mu.float().clone(), mu.float().clone()
        mp.view(-1)[flat] += eps
        mm.view(-1)[flat] -= eps
        fd = (loss(mp) - loss(mm)) / (2 * eps)
        assert abs(fd - float(a_mu.view(-1)[flat])) < 3e-3, flat


# ---------------------------------------------------------------------------
# Routed (selected-chunk) attention backward: the reference kernel
# (ops/hils_fwd_bwd_head.py:573-910) computes the softmax-attention chain rule
#   dV += P^T (w dO),  dW = sum_s P (dO . V_s),
#   dS = scale w P (dO . V - dW),  dQ = dS K,  dK = dS^T Q;
# the oracle's backward is torch autograd of its forward restatement.
# ---------------------------------------------------------------------------
def _sel_inputs(seed, B=1, Lq=3, Hkv=2, G=3, D=128, C=3, K=2):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Lq, Hkv * G, D, generator=g) * 0.3
    k = torch.randn(B, C * 64, Hkv, D, generator=g) * 0.3
    v = torch.randn(B, C * 64, Hkv, D, generator=g)
    w = torch.rand(B, Lq, Hkv * G, K, generator=g)
    idx = torch.randint(0, C, (B, Lq, Hkv, K), generator=g)
    idx[0, 0, 1, 1] = -1
    valid = torch.ones(B, C * 64, dtype=torch.bool)
    valid[0, 5] = False
    dout = torch.randn(B, Lq, Hkv * G, D, generator=g)
    return q, k, v, w, idx, valid, dout


def _sel_grads(q, k, v, w, idx, valid, dout):
    ts = [t.clone().requires_grad_(True) for t in (q, k, v, w)]
    out = O.selected_attention(ts[0], ts[1], ts[2], ts[3], idx, valid)
    (out * dout).sum().backward()
    return [t.grad for t in ts]


def test_oracle_selected_attention_grad_closed_form_uniform_softmax():
    # q = 0: every visible key of a chunk has p = 1 / n, so out = w mean(V)
    # and dV_s = w dO / n, dW = dO . mean(V), dK = 0 (dS^T q = 0), and
    # dQ = scale w / n sum_s (dO . V_s - dW) K_s.
    B, Lq, Hkv, G, D, C = 1, 1, 1, 1, 128, 2
    g = torch.Generator().manual_seed(3)
    q = torch.zeros(B, Lq, Hkv * G, D)
    k = torch.randn(B, C * 64, Hkv, D, generator=g)
    v = torch.randn(B, C * 64, Hkv, D, generator=g)
    w = torch.full((B, Lq, Hkv * G, 1), 0.7)
    idx = torch.tensor([[[[1]]]])
    valid = torch.ones(B, C * 64, dtype=torch.bool)
    dout = torch.randn(B, Lq, Hkv * G, D, generator=g)
    dq, dk, dv, dw = _sel_grads(q, k, v, w, idx, valid, dout)
    keys = torch.arange(64, 127)  # chunk 1 without its landmark slot
    vs, ks = v[0, keys, 0], k[0, keys, 0]
    n = keys.numel()
    do = dout[0, 0, 0]
    torch.testing.assert_close(dv[0, keys, 0], (0.7 / n) * do.expand(n, D), atol=1e-6, rtol=1e-5)
    assert float(dv[0, 127].abs().max()) == 0.0 and float(dv[0, :64].abs().max()) == 0.0
    torch.testing.assert_close(dw[0, 0, 0, 0], (do * vs.mean(0)).sum(), atol=1e-5, rtol=1e-5)
    assert float(dk.abs().max()) == 0.0
    dp = vs @ do
    ref_dq = (1.0 / math.sqrt(D)) * 0.7 / n * ((dp - dp.mean())[:, None] * ks).sum(0)
    torch.testing.assert_close(dq[0, 0, 0], ref_dq, atol=1e-5, rtol=1e-4)


def test_oracle_selected_attention_grad_central_differences():
    q, k, v, w, idx, valid, dout = _sel_inputs(11)
    dq, dk, dv, dw = _sel_grads(q, k, v, w, idx, valid, dout)

    def f(q_, k_, v_, w_):
        return float((O.selected_attention(q_, k_, v_, w_, idx, valid) * dout).sum())

    g = torch.Generator().manual_seed(12)
    eps = 1e-2
    for which, grad in ((0, dq), (1, dk), (2, dv), (3, dw)):
        base = [q, k, v, w]
        t = base[which]
        # a random direction through the tensor
        d = torch.randn(t.shape, generator=g)
        plus = [x.clone() for x in base]
        minus = [x.clone() for x in base]
        plus[which] = t + eps * d
        minus[which] = t - eps * d
        num = (f(*plus) - f(*minus)) / (2 * eps)
        ana = float((grad * d).sum())
        assert abs(num - ana) <= 2e-2 * max(1.0, abs(ana)), (which, num, ana)


# -- route-score backward (ops/topk_head_softmax.py:1074-1122) ---------------
def _score_inputs(seed, B=2, L=5, H=2, G=3, K=4, C=7, D=16, per_head=True):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, L, H, G, D, generator=g).bfloat16()
    lm = torch.randn(B, C, H * G if per_head else H, D, generator=g).bfloat16()
    idx = torch.stack([torch.randperm(C, generator=g)[:K] for _ in range(B * L * H)])
    idx = idx.reshape(B, L, H, K)
    idx[0, 1, 0, 2:] = -1
    idx[1, L - 1, H - 1, 0] = C + 3  # out of range: contributes nothing
    gs = torch.randn(B, L, H, G, K, generator=g).bfloat16()
    return q, lm, idx, gs


def _score_autograd(q, lm, idx, gs, scale):
    """Autograd of the forward score = scale * q . lmk[idx] (gathered rows)."""
    B, L, H, G, D = q.shape
    C = lm.shape[1]
    qf = q.float().requires_grad_(True)
    lf = lm.float().requires_grad_(True)
    per_head = lm.shape[2] == H * G
    rows = lf.reshape(B, C, H, G, D) if per_head else lf[:, :, :, None, :].expand(B, C, H, G, D)
    ok = (idx >= 0) & (idx < C)
    safe = idx.clamp(0, C - 1)
    # picked[b, l, h, g, k, :] = rows[b, idx[b, l, h, k], h, g, :]
    bi = torch.arange(B)[:, None, None, None]
    hi = torch.arange(H)[None, None, :, None]
    picked = rows[bi, safe, hi]  # [B, L, H, K, G, D]
    s = scale * torch.einsum("blhgd,blhkgd->blhgk", qf, picked)
    s = torch.where(ok[:, :, :, None, :], s, torch.zeros_like(s))
    (s * gs.float()).sum().backward()
    return qf.grad, lf.grad


def test_oracle_route_score_bwd_matches_autograd_power_of_two_scale():
    # scale 2^-3: grad * scale is exact in bf16, so the oracle must equal the
    # autograd of the forward definition up to fp32 summation order.
    for per_head in (True, False):
        q, lm, idx, gs = _score_inputs(11, per_head=per_head)
        gq, gl = O.route_score_bwd(q, lm, idx, gs, 0.125)
        aq, al = _score_autograd(q, lm, idx, gs, 0.125)
        torch.testing.assert_close(gq, aq, atol=1e-5, rtol=1e-5)
        torch.testing.assert_close(gl, al, atol=1e-5, rtol=1e-5)


def test_oracle_route_score_bwd_rounds_scaled_gradient_to_bf16():
    # With scale 1/sqrt(D) the gradient is bf16(g * scale): equal to the
    # scale-1 autograd fed the pre-rounded upstream gradient.
    q, lm, idx, gs = _score_inputs(12)
    scale = 1.0 / math.sqrt(q.shape[-1] * 1.7)
    gq, gl = O.route_score_bwd(q, lm, idx, gs, scale)
    pre = (gs.float() * scale).bfloat16()
    aq, al = _score_autograd(q, lm, idx, pre, 1.0)
    torch.testing.assert_close(gq, aq, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(gl, al, atol=1e-5, rtol=1e-5)
    # ... and differs from the unrounded product by more than fp32 noise
    uq, _ = _score_autograd(q, lm, idx, gs, scale)
    assert (gq - uq).abs().max() > 1e-4


def test_oracle_route_score_bwd_ignores_invalid_slots_and_sums_shared_heads():
    q, lm, idx, gs = _score_inputs(13)
    gs2 = gs.clone()
    bad = (idx < 0) | (idx >= lm.shape[1])
    gs2.masked_fill_(bad[:, :, :, None, :], 7.0)
    a = O.route_score_bwd(q, lm, idx, gs)
    b = O.route_score_bwd(q, lm, idx, gs2)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    # shared landmarks = per-head landmarks that repeat over the group, with
    # the per-head gradient summed over the group
    B, L, H, G, D = q.shape
    shared = lm.reshape(B, -1, H, G, D)[:, :, :, 0]
    rep = shared[:, :, :, None, :].expand(B, -1, H, G, D).reshape(B, -1, H * G, D)
    sq, sl = O.route_score_bwd(q, shared, idx, gs)
    pq, pl = O.route_score_bwd(q, rep.contiguous(), idx, gs)
    torch.testing.assert_close(sq, pq, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(sl, pl.reshape(B, -1, H, G, D).sum(3), atol=1e-5, rtol=1e-5)


# -- window attention backward (flash_attn_func's gradient) -----------------
def test_oracle_local_attention_grad_central_differences_and_inert_keys():
    # The window-attention gradient checked by the GPU kernels is autograd of
    # the oracle's forward (itself pinned against a dense formulation).  Pin
    # that gradient numerically along random directions, and check the
    # masking rule: inert keys (failed key_valid, landmark slots) get zero
    # dk / dv because the forward uses k * m, v * m (local_attention.py:50-54).
    g = torch.Generator().manual_seed(31)
    B, L, Hkv, G, D, W, inert = 1, 24, 2, 3, 16, 5, 8
    q = torch.randn(B, L, Hkv * G, D, generator=g)
    k = torch.randn(B, L, Hkv, D, generator=g)
    v = torch.randn(B, L, Hkv, D, generator=g)
    valid = torch.rand(B, L, generator=g) > 0.2
    dout = torch.randn(B, L, Hkv * G, D, generator=g)
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (q, k, v))
    out, _ = O.local_attention(qr, kr, vr, valid, W, inert)
    (out * dout).sum().backward()
    dead = ~valid[0] | ((torch.arange(L) + 1) % inert == 0)
    assert bool(dead.any()) and bool((~dead).any())
    assert float(kr.grad[0, dead].abs().max()) == 0.0
    assert float(vr.grad[0, dead].abs().max()) == 0.0
    assert float(kr.grad[0, ~dead].abs().max()) > 0.0

    def f(q_, k_, v_):
        return float((O.local_attention(q_, k_, v_, valid, W, inert)[0].double() * dout).sum())

    eps = 1e-2
    for which, grad in ((0, qr.grad), (1, kr.grad), (2, vr.grad)):
        base = [q, k, v]
        d = torch.randn(base[which].shape, generator=g)
        plus = [x.clone() for x in base]
        minus = [x.clone() for x in base]
        plus[which] = base[which] + eps * d
        minus[which] = base[which] - eps * d
        num = (f(*plus) - f(*minus)) / (2 * eps)
        ana = float((grad * d).sum())
        assert abs(num - ana) <= 2e-2 * max(1.0, abs(ana)), (which, num, ana)
