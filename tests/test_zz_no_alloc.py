"""The no-allocation route entry point (mrsa_route_topk_noalloc_fwd) against
the workspace entry point (mrsa_route_topk_ws_fwd) through the C ABI:
identical indices and scores (bit for bit) on two calls in a row, the second
smaller, for the short-block path (the static scratch holds the logits) and
the matrix-core path (no workspace needed); a problem beyond the static
buffer is rejected before any launch."""

import math

import pytest
import torch

from mrsa import _lib

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
SCRATCH_BYTES = 16 << 20


def _inputs(rows, chunks, seed, Hkv=4, G=7, D=128):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, rows, Hkv, G, D, generator=g).bfloat16().to(DEV)
    lmk = torch.randn(1, chunks, Hkv * G, D, generator=g).bfloat16().to(DEV)
    lse = (torch.randn(1, rows, Hkv, G, generator=g) + 4.0).to(DEV)
    bias = torch.rand(1, chunks, Hkv, G, generator=g).to(DEV)
    drop = (torch.rand(1, rows, chunks, generator=g) < 0.05).int().to(DEV)
    return q, lmk, lse, bias, drop


def _call(name, q, lmk, lse, bias, drop, topk=32, ws=None):
    _, rows, Hkv, G, D = q.shape
    chunks = lmk.shape[1]
    idx = torch.full((1, rows, Hkv, topk), -7, dtype=torch.int32, device=DEV)
    scores = torch.zeros(1, rows, Hkv, G, topk, dtype=torch.bfloat16, device=DEV)
    args = [_lib.ptr(q), _lib.ptr(lmk), _lib.ptr(lse), _lib.ptr(bias), _lib.ptr(drop), None, -1,
            1, rows, chunks, Hkv, G, D, topk, 64, 1, 0, 0, 0, 0, 1.0 / math.sqrt(D),
            _lib.ptr(idx), _lib.ptr(scores), 0]
    if ws is not None:
        args += [_lib.ptr(ws), ws.numel() * ws.element_size()]
    st = _lib.call(name, *args, _lib.stream_of(q))
    return st, idx, scores


def _workspace(rows, chunks, Hkv=4, G=7):
    n = rows * Hkv * G * chunks * 4
    return torch.empty((n + 3) // 4, dtype=torch.float32, device=DEV)


@pytest.mark.parametrize("shapes", [((32, 2048), (16, 1024)), ((1024, 256), (300, 128))])
def test_no_alloc_route_topk_equals_workspace_entry(shapes):
    for n, (rows, chunks) in enumerate(shapes):
        print(f"[gpu-case] no-alloc route topk call {n}: rows={rows} chunks={chunks}",
              flush=True)
        inp = _inputs(rows, chunks, 100 + n)
        st, idx, sc = _call("mrsa_route_topk_noalloc_fwd", *inp)
        assert st == 0, _lib.status_string(st)
        st, ridx, rsc = _call("mrsa_route_topk_ws_fwd", *inp, ws=_workspace(rows, chunks))
        assert st == 0, _lib.status_string(st)
        torch.cuda.synchronize()
        assert int((idx == -7).sum()) == 0
        assert torch.equal(idx, ridx)
        assert torch.equal(sc.view(torch.int16), rsc.view(torch.int16))


def test_no_alloc_route_topk_rejects_oversize():
    # 64 rows x 4 x 7 x 4096 chunks x 4 bytes = 29 MiB > the 16 MiB buffer:
    # rejected on the host, nothing launched.
    rows, chunks = 64, 4096
    assert rows * 4 * 7 * chunks * 4 > SCRATCH_BYTES
    st, idx, _ = _call("mrsa_route_topk_noalloc_fwd", *_inputs(rows, chunks, 7))
    assert st == _lib.MRSA_ERR_SCRATCH
    assert "scratch" in _lib.status_string(st)
    torch.cuda.synchronize()
    assert int((idx == -7).sum()) == idx.numel()


def _unaligned(t):
    # the same values at a data pointer 2 bytes off 16-byte alignment
    buf = torch.empty(t.numel() + 8, dtype=t.dtype, device=t.device)
    v = buf[1:1 + t.numel()].view(t.shape)
    v.copy_(t)
    return v


@pytest.mark.parametrize("case", ["topk80", "unaligned"])
def test_no_alloc_route_topk_off_the_matrix_core_path(case):
    # Shapes the one-pass kernel does not take although they have <= 256
    # chunks: more than 64 picks, or q / landmarks not 16-byte aligned.  The
    # no-allocation entry then hands its static buffer to the same dispatch
    # as the workspace entry: same results, bit for bit.
    rows, chunks, topk = (512, 200, 80) if case == "topk80" else (96, 128, 32)
    print(f"[gpu-case] no-alloc route topk {case}: rows={rows} chunks={chunks} topk={topk}",
          flush=True)
    q, lmk, lse, bias, drop = _inputs(rows, chunks, 11)
    if case == "unaligned":
        q, lmk = _unaligned(q), _unaligned(lmk)
    for n in range(2):
        st, idx, sc = _call("mrsa_route_topk_noalloc_fwd", q, lmk, lse, bias, drop, topk=topk)
        assert st == 0, _lib.status_string(st)
        st, ridx, rsc = _call("mrsa_route_topk_ws_fwd", q, lmk, lse, bias, drop, topk=topk,
                              ws=_workspace(rows, chunks))
        assert st == 0, _lib.status_string(st)
        torch.cuda.synchronize()
        assert int((idx == -7).sum()) == 0
        assert torch.equal(idx, ridx)
        assert torch.equal(sc.view(torch.int16), rsc.view(torch.int16))
        rows = rows // 2  # the second call smaller
        q, lse, drop = q[:, :rows], lse[:, :rows].contiguous(), drop[:, :rows].contiguous()
