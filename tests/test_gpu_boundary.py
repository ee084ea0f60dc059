"""The drop-in boundary on the GPU: the reference's own call forms, no host
synchronisation, and the torch.ops.mrsa layer under torch.compile.

Tolerances: bf16 weights within 2e-3 abs / 1e-2 rel of the oracle's
rounded values; the fp32 gate logit within 1e-4 abs / 1e-5 rel; gradients
within 1e-3 abs / 1e-2 rel; route-layer outputs max-abs 2e-2 / mean-abs 2e-3;
routing lists identical except near ties (routing_check.py).
"""

import pytest
import torch

import mrsa
from oracle import mrsa_oracle as O
from routing_check import assert_nearly_identical, classify_routing

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _note(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _weights_inputs(seed, B=1, L=600, Hkv=4, G=7, K=32, C=256, masked=True):
    g = torch.Generator().manual_seed(seed)
    scores = torch.randn(B, L, Hkv * G, K, generator=g).bfloat16()
    idx = torch.randint(0, C, (B, L, Hkv, K), generator=g).int()
    idx[0, 3, 1, K // 2:] = -1
    bias = torch.rand(B, C, Hkv, G, generator=g) + 3.5
    lse = torch.randn(B, L, Hkv * G, generator=g) + 5.0
    if masked:
        idx[0, 4, 2, :] = -1
        lse[0, 4, 14:21] = float("-inf")    # row 4, KV head 2: every logit masked
        lse[0, 5, 3] = float("-inf")        # a masked local logit: gate logit +inf
    return scores, idx, bias, lse


class _Layer(torch.nn.Module):
    """The parameters KernelDreamFullHiLSAttention owns (attention.py:913-914)."""

    def __init__(self, offset, scale):
        super().__init__()
        self.fusion_gate_offset = torch.nn.Parameter(torch.tensor(offset, dtype=torch.float32))
        self.fusion_gate_scale = torch.nn.Parameter(torch.tensor(scale, dtype=torch.float32))


@pytest.mark.parametrize("affine", [True, False])
def test_route_weights_torch_as_the_route_layer_calls_it(affine):
    # attention.py:1609-1622: tensors on the device, the layer's parameters
    # as gates, return_gate_logit=True; the call must not synchronise.
    _note(f"route_weights_torch reference call affine={affine}")
    scores, idx, bias, lse = _weights_inputs(1)
    layer = _Layer(0.3, 1.4).to(DEV)
    T = 0.8
    gate_scale = layer.fusion_gate_scale if affine else None
    args = [t.to(DEV) for t in (scores, idx, bias, lse)]
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        with torch.no_grad():
            routed = mrsa.route_weights_torch(
                args[0], args[1], args[2].contiguous(), args[3].float().contiguous(),
                temperature=T, selected_gumbel=None, value_bonus=None, return_gate_logit=True,
                gate_offset=getattr(layer, "fusion_gate_offset", None), gate_scale=gate_scale)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    remote_weights, local_weight, gate_logit = routed
    er, el, eg = O.route_weights(scores, idx, bias, lse, temperature=T, gate_offset=0.3,
                                 gate_scale=1.4 if affine else None, return_gate_logit=True)
    torch.testing.assert_close(remote_weights.cpu().float(), er.bfloat16().float(), atol=2e-3,
                               rtol=1e-2)
    torch.testing.assert_close(local_weight.cpu().float(), el.bfloat16().float(), atol=2e-3,
                               rtol=1e-2)
    assert gate_logit.dtype == torch.float32 and gate_logit.shape == lse.shape
    torch.testing.assert_close(gate_logit.cpu(), eg, atol=1e-4, rtol=1e-5)
    assert bool((gate_logit[0, 4, 14:21] == 0).all())   # every logit masked -> 0


@pytest.mark.parametrize("affine", [True, False])
def test_route_weights_torch_backward_with_gate_logit(affine):
    # Gradients of all three outputs (gate logit included) into scores,
    # prior_bias, local_lse and both gate parameters, against the oracle's
    # autograd (the reference's backward for this function is its autograd).
    # Fully masked rows are left out: their gradients are zero here
    # (test_gpu_backward.py covers them), while autograd of the torch
    # formulation gives NaN through the softmax of an all -inf row.
    _note(f"route_weights_torch backward affine={affine}")
    scores, idx, bias, lse = _weights_inputs(2, L=300, masked=False)
    g = torch.Generator().manual_seed(3)
    g_rw = torch.randn(scores.shape, generator=g).bfloat16()
    g_lw = torch.randn(lse.shape, generator=g).bfloat16()
    g_gl = torch.randn(lse.shape, generator=g)
    T = 1.3
    layer = _Layer(-0.2, 0.7).to(DEV)
    s_d = scores.to(DEV).requires_grad_()
    b_d = bias.to(DEV).requires_grad_()
    l_d = lse.to(DEV).requires_grad_()
    rw, lw, gl = mrsa.route_weights_torch(
        s_d, idx.to(DEV), b_d, l_d, temperature=T, return_gate_logit=True,
        gate_offset=layer.fusion_gate_offset, gate_scale=layer.fusion_gate_scale if affine else None)
    torch.autograd.backward([rw, lw, gl], [g_rw.to(DEV), g_lw.to(DEV), g_gl.to(DEV)])
    s_c = scores.float().requires_grad_()
    b_c = bias.clone().requires_grad_()
    l_c = lse.clone().requires_grad_()
    go = torch.tensor(-0.2, requires_grad=True)
    gs = torch.tensor(0.7, requires_grad=True) if affine else None
    er, el, eg = O.route_weights(s_c, idx, b_c, l_c, temperature=T, gate_offset=go,
                                 gate_scale=gs, return_gate_logit=True)
    torch.autograd.backward([er, el, eg], [g_rw.float(), g_lw.float(), g_gl])
    for name, got, ref in (("scores", s_d.grad, s_c.grad), ("bias", b_d.grad, b_c.grad),
                           ("lse", l_d.grad, l_c.grad)):
        torch.testing.assert_close(got.cpu().float(), ref, atol=1e-3, rtol=1e-2, msg=name)
    torch.testing.assert_close(layer.fusion_gate_offset.grad.cpu(), go.grad, atol=1e-2, rtol=1e-3)
    if affine:
        torch.testing.assert_close(layer.fusion_gate_scale.grad.cpu(), gs.grad, atol=1e-2,
                                   rtol=1e-3)


def test_torch_compile_fullgraph_pool():
    # The reference compiles its pool twin with fullgraph=True
    # (ops/chunk_attn_pool_gqa_tilelang.py:40-44); the gfx950 op must trace.
    _note("torch.compile fullgraph chunk_attn_pool_gqa")
    g = torch.Generator().manual_seed(4)
    B, C, S, Hkv, G, D = 1, 64, 64, 4, 7, 128
    mu = torch.randn(B, C, Hkv, G, D, generator=g).bfloat16().to(DEV)
    kc = torch.randn(B, C, S, Hkv, D, generator=g).bfloat16().to(DEV)
    kv = (torch.rand(B, C, S, generator=g) > 0.1).to(DEV)
    torch._dynamo.reset()
    compiled = torch.compile(mrsa.chunk_attn_pool_gqa, fullgraph=True, dynamic=False)
    lmk_c, ent_c = compiled(mu, kc, kv)
    lmk_e, ent_e = mrsa.chunk_attn_pool_gqa(mu, kc, kv)
    torch.cuda.synchronize()
    assert torch.equal(lmk_c.view(torch.int16), lmk_e.view(torch.int16))
    assert torch.equal(ent_c, ent_e)


def _layer_inputs(L, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, L, 28, 128, generator=g).bfloat16()
    rq = torch.randn(1, L, 28, 128, generator=g).bfloat16()
    k = torch.randn(1, L, 4, 128, generator=g)
    shift = 0.3 * torch.randn(L // 64, 4, 128, generator=g)
    k = (k + shift.repeat_interleave(64, dim=0)[None]).bfloat16()
    v = torch.randn(1, L, 4, 128, generator=g).bfloat16()
    scale = torch.rand(28, generator=g) + 0.5
    return q, rq, k, v, scale


def test_torch_compile_fullgraph_route_layer():
    # The whole route layer as one graph (no break) through torch.ops.mrsa,
    # with the results of the eager call.
    _note("torch.compile fullgraph route layer L=1024")
    q, rq, k, v, scale = (t.to(DEV) for t in _layer_inputs(1024, 5))
    layer = _Layer(0.1, 1.2).to(DEV)
    cfg = mrsa.RouteLayerConfig(gate_offset=layer.fusion_gate_offset,
                                gate_scale=layer.fusion_gate_scale)

    def f(q, k, v, rq, scale):
        return mrsa.route_attention(q, k, v, rq, scale, cfg=cfg)

    torch._dynamo.reset()
    with torch.no_grad():
        got = torch.compile(f, fullgraph=True, backend="aot_eager")(q, k, v, rq, scale)
        ref = f(q, k, v, rq, scale)
    torch.cuda.synchronize()
    assert_nearly_identical(got, ref, "compiled vs eager route layer", atol=0.03)


@pytest.mark.parametrize("topk,temperature", [(32, 0.8), (16, 0.8)])
def test_route_layer_weight_form_by_topk(topk, temperature):
    # attention.py:1571-1578 / 1643-1648: topk >= 32 takes the layer's
    # temperature and fusion gate, topk < 32 the plain 33-way softmax at
    # temperature 1 with no gate.  Non-trivial gate values tell them apart.
    # Also: the route layer never synchronises with the host.
    _note(f"route layer topk={topk} T={temperature} gates (0.4, 1.6)")
    L = 2048
    q, rq, k, v, scale = _layer_inputs(L, 6)
    valid = torch.ones(1, L, dtype=torch.bool)
    layer = _Layer(0.4, 1.6).to(DEV)
    cfg = mrsa.RouteLayerConfig(topk=topk, temperature=temperature,
                                gate_offset=layer.fusion_gate_offset,
                                gate_scale=layer.fusion_gate_scale)
    dq, dk, dv, drq, ds, dvalid = (t.to(DEV) for t in (q, k, v, rq, scale, valid))
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        with torch.no_grad():
            out, mid = mrsa.route_attention(dq, dk, dv, drq, ds, dvalid, cfg,
                                            return_intermediates=True)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    ref, rmid = O.route_layer(q, k, v, rq, scale, valid, topk=topk, temperature=temperature,
                              gate_offset=0.4, gate_scale=1.6)
    err = (out.float().cpu() - ref.float()).abs()
    print(f"route layer topk={topk}: max_abs={err.max():.3e} mean_abs={err.mean():.3e}",
          flush=True)
    assert float(err.max()) <= 2e-2 and float(err.mean()) <= 2e-3
    classify_routing(mid["indices"], rmid["indices"], rq, mid["landmark_keys"],
                     mid["local_lse"], mid["prior_bias"],
                     lambda r: O.remote_drop_mask(valid, 256, 64)[:, r], topk, 64,
                     f"route layer topk={topk}")
    # the weights of the GPU's own routing against the oracle's formula
    if topk >= 32:
        kw = dict(temperature=temperature, gate_offset=0.4, gate_scale=1.6)
    else:
        kw = {}
    rw, lw = O.route_weights(mid["scores"].cpu(), mid["indices"].cpu().long(),
                             mid["prior_bias"].cpu(), mid["local_lse"].cpu(), **kw)
    torch.testing.assert_close(mid["remote_weights"].cpu().float(), rw.bfloat16().float(),
                               atol=2e-3, rtol=1e-2)
    torch.testing.assert_close(mid["local_weight"].cpu().float(), lw.bfloat16().float(),
                               atol=2e-3, rtol=1e-2)


def test_per_op_drop_ins_reuse_the_kv_layout(monkeypatch):
    # A layer that runs the per-op drop-ins on the same k / v (the window
    # branch, then the routed attention; a decode loop against an unchanged
    # cache) lays K / V out once; an in-place write to the cache (version
    # bump) lays it out again.  Results equal the uncached path.
    import mrsa.sparse_attention as SA

    calls = []
    real = SA.kv_fragments
    monkeypatch.setattr(SA, "kv_fragments", lambda k, v=None: calls.append(1) or real(k, v))
    SA._FRAG_CACHE.clear()
    B, L, Hkv, G, D, K, S = 1, 1024, 4, 7, 128, 8, 64
    g = torch.Generator().manual_seed(5)
    q = torch.randn(B, 32, Hkv * G, D, generator=g).bfloat16().to(DEV)
    k = torch.randn(B, L, Hkv, D, generator=g).bfloat16().to(DEV)
    v = torch.randn(B, L, Hkv, D, generator=g).bfloat16().to(DEV)
    valid = torch.ones(B, L, dtype=torch.bool, device=DEV)
    idx = torch.stack([torch.randperm(L // S, generator=g)[:K] for _ in range(32 * Hkv)])
    idx = idx.sort(-1).values.reshape(B, 32, Hkv, K).int().to(DEV)
    w = torch.softmax(torch.randn(B, 32, Hkv * G, K, generator=g), -1).bfloat16().to(DEV)
    pos = torch.arange(L - 32, L, device=DEV)
    loc1 = mrsa.cached_local_attention(q, k, v, valid, pos, 319, S)
    out1 = mrsa.selected_attention_g7_cached(q, k, v, w, idx, valid, S)
    out2 = mrsa.selected_attention_g7_cached(q, k, v, w, idx, valid, S)
    assert len(calls) == 1
    assert torch.equal(SA.kv_fragments_cached(k, v), real(k, v))  # the layout itself
    fresh = SA.selected_attention_launch(q, real(k, v), w, idx, valid, S, deterministic=True)

    def close(a, b, what):
        err = (a.float() - b.float()).abs()
        print(f"{what}: max {float(err.max()):.3e} mean {float(err.mean()):.3e}", flush=True)
        assert float(err.max()) <= 2e-3 and float(err.mean()) <= 1e-5, what

    close(out1, fresh, "cached layout vs fresh")
    close(out2, fresh, "cached layout, second call")
    k[:, -1] += 1.0   # the cache is written in place: the layout is rebuilt
    out3 = mrsa.selected_attention_g7_cached(q, k, v, w, idx, valid, S)
    assert len(calls) == 2
    assert torch.equal(SA.kv_fragments_cached(k, v), real(k, v))
    close(out3, SA.selected_attention_launch(q, real(k, v), w, idx, valid, S, deterministic=True),
          "layout after an in-place write")
    del loc1
    SA._FRAG_CACHE.clear()
