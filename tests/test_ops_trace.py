"""The torch.ops.mrsa layer: schemas, fake kernels and full-graph tracing.

Runs without a GPU: fake CUDA tensors carry shapes and dtypes through the
operators' fake implementations, and a strict (dynamo) torch.export of the
whole route layer must produce one graph with no break, the property
``torch.compile(fullgraph=True)`` needs.  The GPU side (real kernels under
torch.compile) is in test_gpu_boundary.py.
"""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import mrsa
from mrsa import ops


def test_every_operator_is_registered():
    for name in ops.OPERATORS:
        assert hasattr(torch.ops.mrsa, name), name


def _fake_layer_inputs(L=1024, Hq=28, Hkv=4, D=128):
    q = torch.empty(1, L, Hq, D, dtype=torch.bfloat16, device="cuda")
    k = torch.empty(1, L, Hkv, D, dtype=torch.bfloat16, device="cuda")
    v = torch.empty_like(k)
    scale = torch.empty(Hq, device="cuda")
    return q, k, v, q.clone(), scale


class _RouteLayer(torch.nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.cfg = cfg

    def forward(self, q, k, v, route_q, scale):
        return mrsa.route_attention(q, k, v, route_q, scale, cfg=self.cfg)


@pytest.mark.parametrize("topk", [32, 16])
def test_route_layer_exports_as_one_graph(topk):
    cfg = mrsa.RouteLayerConfig(topk=topk)
    with FakeTensorMode(allow_non_fake_inputs=True):
        args = _fake_layer_inputs()
        ep = torch.export.export(_RouteLayer(cfg), args, strict=True)
    called = {n.target for n in ep.graph.nodes if n.op == "call_function"}
    names = {str(t) for t in called}
    for op in ("route_topk", "route_weights", "selected_attention"):
        assert f"mrsa.{op}.default" in names, (op, sorted(names))
    # K/V fragments and the landmark pool: one pass, or the two ops
    assert ("mrsa.kv_fragments_pool.default" in names
            or {"mrsa.kv_fragments.default", "mrsa.chunk_attn_pool.default"} <= names), sorted(names)
    # the window attention, with its Q-fragment by-product when it runs unsplit
    assert names & {"mrsa.local_attention.default", "mrsa.local_attention_qf.default"}
    out = [n for n in ep.graph.nodes if n.op == "output"][0]
    val = out.args[0][0].meta["val"]
    assert tuple(val.shape) == (1, 1024, 28, 128) and val.dtype == torch.bfloat16


def test_fake_kernels_match_the_reference_contracts():
    with FakeTensorMode():
        B, L, C, Hkv, G, D, K = 1, 512, 8, 4, 7, 128, 32
        mu = torch.empty(B, C, Hkv, G, D, dtype=torch.bfloat16, device="cuda")
        kc = torch.empty(B, C, 64, Hkv, D, dtype=torch.bfloat16, device="cuda")
        kv = torch.empty(B, C, 64, dtype=torch.bool, device="cuda")
        lmk, ent = mrsa.chunk_attn_pool_gqa(mu, kc, kv)
        assert lmk.shape == mu.shape and lmk.dtype == torch.bfloat16
        assert ent.shape == (B, C, Hkv, G) and ent.dtype == torch.float32
        scores = torch.empty(B, L, Hkv * G, K, dtype=torch.bfloat16, device="cuda")
        idx = torch.empty(B, L, Hkv, K, dtype=torch.int32, device="cuda")
        bias = torch.empty(B, C, Hkv, G, device="cuda")
        lse = torch.empty(B, L, Hkv * G, device="cuda")
        off = torch.zeros((), device="cuda")
        rw, lw, gl = mrsa.route_weights_torch(scores, idx, bias, lse, temperature=1.0,
                                              return_gate_logit=True, gate_offset=off,
                                              gate_scale=off + 1)
        assert rw.shape == scores.shape and rw.dtype == torch.bfloat16
        assert lw.shape == (B, L, Hkv * G) and gl.shape == (B, L, Hkv * G)
        assert gl.dtype == torch.float32
        q = torch.empty(B, L, Hkv * G, D, dtype=torch.bfloat16, device="cuda")
        k = torch.empty(B, L, Hkv, D, dtype=torch.bfloat16, device="cuda")
        o = mrsa.HiLS_block_M_head(q, k, k, rw, idx, key_valid=torch.ones(
            B, L, dtype=torch.bool, device="cuda"))
        assert o.shape == q.shape and o.dtype == torch.bfloat16
        o2, lse2 = mrsa.bidir_local_attention(q, k, k, torch.ones(B, L, dtype=torch.bool,
                                                                   device="cuda"), 256, 64)
        assert o2.shape == q.shape and lse2.shape == (B, L, Hkv * G)
        drop = mrsa.remote_drop_mask(torch.ones(B, L, dtype=torch.bool, device="cuda"), 256, 64)
        assert drop.shape == (B, L, C) and drop.dtype == torch.int32
