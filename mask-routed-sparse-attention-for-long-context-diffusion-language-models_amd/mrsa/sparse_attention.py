"""Routed chunk attention and the K / V layout both attention kernels read.

Drop-in for ``ops.hils_fwd_bwd_head.HiLS_block_M_head``
(ops/hils_fwd_bwd_head.py:1113-1150) in its forward role, plus
``kv_fragments`` (the per-chunk operand images the routed and window
attention kernels read).
"""

from __future__ import annotations

import math

import torch

from . import _lib


FRAG_ELEMS = 16384  # bf16 per (batch, KV head, 64-key chunk)
_ROUTED_FIXED_ORDER = 1  # MRSA_ROUTED_FIXED_ORDER


def kv_fragments(k: torch.Tensor, v: torch.Tensor | None = None) -> torch.Tensor:
    """K, V [B, L, Hkv, 128] bf16 -> per-chunk fragments [B, Hkv, ceil(L/64), 16384] bf16.

    For each 64-key chunk, the register images of the routed attention's 32
    matrix-core operand loads (lane l = 16 grp + j, elements e = 0..7):
    f[512 i + 8 l + e] = K[16 mt + j][32 ks + 8 grp + e] for i = 4 mt + ks, and
    f[8192 + 512 i + 8 l + e] = V[32 ks + 16 (e >> 2) + 4 grp + (e & 3)][16 nt + j]
    for i = 2 nt + ks.  Keys past L are zero; without ``v`` the V half is zero
    (candidate token scores read only K).
    """

    if k.device.type != "cuda" or k.dtype != torch.bfloat16 or k.ndim != 4 or k.shape[3] != 128:
        raise ValueError("kv_fragments requires a CUDA BF16 [B, L, Hkv, 128] key tensor")
    if v is not None and (v.shape != k.shape or v.dtype != k.dtype or v.device != k.device):
        raise ValueError("kv_fragments requires v shaped, typed and placed like k")
    return torch.ops.mrsa.kv_fragments(k, v)


def _kv_fragments_impl(k: torch.Tensor, v: torch.Tensor | None) -> torch.Tensor:
    B, L, H, D = k.shape
    kc = k.contiguous()
    vc = None if v is None else v.contiguous()
    out = torch.empty(B, H, (L + 63) // 64, FRAG_ELEMS, dtype=torch.bfloat16, device=k.device)
    st = _lib.call("mrsa_kv_fragments", _lib.ptr(kc), _lib.ptr(vc), B, L, H, D, _lib.ptr(out),
                   _lib.stream_of(kc))
    _lib.check(st, "kv_fragments")
    return out


# Fragment layouts of recent (k, v) pairs, most recent last:
# (key, weakref(k), weakref(v) or None, fragments).
_FRAG_CACHE: list = []
_FRAG_CACHE_SIZE = 4


def _frag_key(t):
    return (t.data_ptr(), tuple(t.shape), tuple(t.stride()), t.dtype, t.device, t._version)


def kv_fragments_cached(k: torch.Tensor, v: torch.Tensor | None = None) -> torch.Tensor:
    """kv_fragments(k, v), reusing the layout last built for the same k and v
    tensor objects while neither has been written since (storage, shape,
    strides and version counter unchanged: an in-place update such as
    LayerKVCache.replace bumps the version).  The per-op drop-ins use it, so
    a layer that calls bidir_local_attention and then selected_attention_g7
    on the same k / v, or a decode loop that calls the cached ops against an
    unchanged cache, lays K / V out once.  The four most recent layouts are
    kept (each holds its source tensors only weakly); under torch.compile
    tracing the layout is built every time."""

    if torch.compiler.is_compiling() or k.device.type != "cuda":
        return kv_fragments(k, v)
    key = (_frag_key(k), None if v is None else _frag_key(v))
    alive = []
    hit = None
    for entry in _FRAG_CACHE:
        ek, wk, wv, frags = entry
        tk = wk()
        tv = None if wv is None else wv()
        if tk is None or (wv is not None and tv is None):
            continue  # a source tensor is gone
        alive.append(entry)
        if hit is None and ek == key and tk is k and tv is v:
            hit = entry
    _FRAG_CACHE[:] = alive
    if hit is not None:
        _FRAG_CACHE.remove(hit)
        _FRAG_CACHE.append(hit)
        return hit[3]
    frags = kv_fragments(k, v)
    import weakref

    _FRAG_CACHE.append((key, weakref.ref(k), None if v is None else weakref.ref(v), frags))
    del _FRAG_CACHE[:-_FRAG_CACHE_SIZE]
    return frags


def q_fragments(q: torch.Tensor, kv_heads: int) -> torch.Tensor:
    """q [B, L, Hq, 128] bf16 -> Q operand images [B, Hkv, L, 1024] bf16.

    Per (batch, KV head, query) the 2 KB register image of the routed
    attention's Q^T operand for the query's G = Hq / Hkv head columns:
    f[256 ks + 64 grp + 8 g + e] = q[h G + g][32 ks + 8 grp + e] (zeros for
    heads g >= G, up to 8), so the routed kernel reads each lane group's 8
    head columns as one 128-byte line.
    """

    if q.device.type != "cuda" or q.dtype != torch.bfloat16 or q.ndim != 4 or q.shape[3] != 128:
        raise ValueError("q_fragments requires a CUDA BF16 [B, L, Hq, 128] query tensor")
    if kv_heads <= 0 or q.shape[2] % kv_heads or q.shape[2] // kv_heads > 8:
        raise ValueError(f"q_fragments: {q.shape[2]} query heads over {kv_heads} KV heads "
                         "(at most 8 per group)")
    return torch.ops.mrsa.q_fragments(q, int(kv_heads))


def _q_fragments_impl(q: torch.Tensor, kv_heads: int) -> torch.Tensor:
    B, L, Hq, D = q.shape
    qc = q.contiguous()
    out = torch.empty(B, kv_heads, L, 1024, dtype=torch.bfloat16, device=q.device)
    st = _lib.call("mrsa_q_fragments", _lib.ptr(qc), B, L, Hq, kv_heads, D, _lib.ptr(out),
                   _lib.stream_of(qc))
    _lib.check(st, "q_fragments")
    return out


def kv_fragments_rows(k: torch.Tensor, v: torch.Tensor, kv_frags: torch.Tensor,
                      positions: torch.Tensor) -> None:
    """Rewrite the fragments of rows ``positions`` of k and v in ``kv_frags``
    (in place), after those rows were replaced.  Positions outside [0, L)
    are ignored."""

    if k.device.type != "cuda" or k.dtype != torch.bfloat16 or k.ndim != 4 or k.shape[3] != 128:
        raise ValueError("kv_fragments_rows requires a CUDA BF16 [B, L, Hkv, 128] key tensor")
    if v.shape != k.shape or v.dtype != k.dtype:
        raise ValueError("kv_fragments_rows requires v shaped and typed like k")
    B, L, H, _ = k.shape
    if kv_frags.shape != (B, H, (L + 63) // 64, FRAG_ELEMS) or not kv_frags.is_contiguous():
        raise ValueError("kv_frags must be the contiguous kv_fragments(k, v) layout")
    torch.ops.mrsa.kv_fragments_rows_(k, v, kv_frags, positions)


def _kv_fragments_rows_impl(k, v, kv_frags, positions) -> None:
    B, L, H, D = k.shape
    kc, vc = k.contiguous(), v.contiguous()
    pos = positions.to(device=k.device, dtype=torch.long).contiguous()
    st = _lib.call("mrsa_kv_fragments_rows", _lib.ptr(kc), _lib.ptr(vc), B, L, H, D,
                   _lib.ptr(pos), pos.numel(), _lib.ptr(kv_frags), _lib.stream_of(kc))
    _lib.check(st, "kv_fragments_rows")


# Queries per routed-attention workgroup (the kernel picks up to 32).
_SEL_TILE_QUERIES = 32
_SEL_MAX_PARTS = 64


def walk_parts(batch: int, q_len: int, kv_heads: int, kv_len: int, topk: int,
               chunk_size: int = 64) -> int:
    """Workgroups per (query tile, KV head) walk of the routed attention.

    Long sequences fill the chip with one workgroup per walk.  A short query
    block (the cached block step: 32 queries, 4 KV heads -> 4 walks of up to
    1024 chunks) splits each walk into parts of >= 32 steps (at most 512
    workgroups).  Every part builds the whole walk in its prologue and
    writes a partial output that the part sum reads back, so more, shorter
    parts stop paying off: at the cached block step 32 parts take 0.144 ms
    per block, 16 parts 0.149 ms, 64 parts 0.168 ms.
    """

    walks = -(-q_len // _SEL_TILE_QUERIES) * kv_heads * batch
    if walks >= 128 or walks == 0:
        return 1
    steps = min(kv_len // chunk_size, min(_SEL_TILE_QUERIES, q_len) * topk)
    parts = min(_SEL_MAX_PARTS, 512 // walks, steps // 32, 65535 // max(batch, 1))
    return max(1, parts)


class RoutedLockTimeout(RuntimeError):
    """Routed-attention tiles ran out of their bounded lock wait.  They were
    deferred and replayed after their workgroup's walk (the outputs are
    exact), but at the default bound this never happens in a healthy run."""


def routed_lock_giveups(reset: bool = True) -> int:
    """Number of routed-attention tiles on the current device whose bounded
    lock wait ran out since the last reset.  Each such tile is deferred and
    replayed onto its rows after the workgroup's walk, so outputs stay exact;
    the count reports that slow path.  One counter per device, shared by all
    streams; reading it waits for the device's queued work, so it cannot run
    under graph capture."""

    import ctypes

    count = ctypes.c_uint64(0)
    _lib.check(_lib.call("mrsa_routed_lock_giveups", ctypes.byref(count), 1 if reset else 0),
               "mrsa_routed_lock_giveups")
    return int(count.value)


def check_routed_locks(reset: bool = True) -> None:
    """Raise RoutedLockTimeout when any routed-attention tile gave up its lock
    wait since the last reset."""

    n = routed_lock_giveups(reset)
    if n:
        raise RoutedLockTimeout(
            f"{n} routed-attention tile(s) ran out of the bounded lock wait and were replayed "
            "after their walk (outputs exact; a lowered spin limit, or lock contention "
            "that should not occur)")


def set_routed_lock_spin_limit(limit: int = 65536) -> None:
    """Test hook: lock tries of the routed-attention kernels before a tile is
    deferred (process-wide, read at each launch; <= 0 defers every tile)."""

    _lib.check(_lib.call("mrsa_set_routed_lock_spin_limit", int(limit)),
               "mrsa_set_routed_lock_spin_limit")


def selected_attention_launch(
    q: torch.Tensor,
    kv_frags: torch.Tensor,
    weights: torch.Tensor,
    indices: torch.Tensor,
    key_valid: torch.Tensor | None,
    chunk_size: int,
    *,
    mask_last_token: bool = True,
    sm_scale: float | None = None,
    parts: int | None = None,
    token_keep: torch.Tensor | None = None,
    fuse_local: torch.Tensor | None = None,
    fuse_weight: torch.Tensor | None = None,
    q_frags: torch.Tensor | None = None,
    deterministic: bool = False,
) -> torch.Tensor:
    """q [B, Lq, Hq, D], kv_frags = kv_fragments(k, v) of the Lk-row cache,
    weights [B, Lq, Hq, K] -> [B, Lq, Hq, D] bf16.

    ``parts`` splits each walk over that many workgroups (fp32 partial
    outputs summed by a second kernel); None picks it with ``walk_parts``.
    ``token_keep`` [B, Lq, Hkv, K, chunk_size] (nonzero = kept) additionally
    masks the keys of each query's slot k.  ``fuse_local`` [B, Lq, Hq, D] and
    ``fuse_weight`` [B, Lq, Hq] (bf16, both or neither) fold the output
    fusion in: the result is fuse_hils_outputs(routed, fuse_local,
    fuse_weight), bit for bit, without materialising the routed output.
    ``q_frags`` = q_fragments(q, Hkv) (with the fusion only) makes the kernel
    read the queries from their operand images: the same result.
    ``deterministic`` adds every output row's chunk terms in ascending chunk
    order (per-query tickets instead of the row lock): the same bits on every
    launch, eager or graph-captured.
    """

    B, Lq, Hq, D = q.shape
    if kv_frags.ndim != 4 or kv_frags.shape[0] != B or kv_frags.shape[3] != FRAG_ELEMS:
        raise ValueError(f"kv_frags {tuple(kv_frags.shape)} is not a kv_fragments layout")
    Hkv, Lk = kv_frags.shape[1], kv_frags.shape[2] * 64
    K = indices.shape[-1]
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    if parts is None:
        parts = walk_parts(B, Lq, Hkv, Lk, K, chunk_size)
    parts = int(parts)
    if not 1 <= parts <= _SEL_MAX_PARTS:
        raise ValueError(f"parts must be in [1, {_SEL_MAX_PARTS}], got {parts}")
    if (fuse_local is None) != (fuse_weight is None):
        raise ValueError("fuse_local and fuse_weight go together")
    if fuse_local is not None and (fuse_local.shape != (B, Lq, Hq, D)
                                   or fuse_weight.shape != (B, Lq, Hq)):
        raise ValueError(
            f"fusion shapes {tuple(fuse_local.shape)} / {tuple(fuse_weight.shape)} do not "
            f"match the output [{B}, {Lq}, {Hq}, {D}]")
    if q_frags is not None:
        if fuse_local is None:
            raise ValueError("q_frags is read by the fused routed attention only")
        if q_frags.shape != (B, Hkv, Lq, 1024) or q_frags.dtype != torch.bfloat16:
            raise ValueError(f"q_frags {tuple(q_frags.shape)} is not q_fragments(q, {Hkv})")
    return torch.ops.mrsa.selected_attention(
        q, kv_frags, weights, indices, key_valid, int(chunk_size), bool(mask_last_token),
        float(sm_scale), parts, token_keep, fuse_local, fuse_weight, q_frags, bool(deterministic))


def _selected_attention_impl(q, kv_frags, weights, indices, key_valid, chunk_size,
                             mask_last_token, sm_scale, parts, token_keep, fuse_local,
                             fuse_weight, q_frags=None, deterministic=False):
    B, Lq, Hq, D = q.shape
    Hkv, Lk = kv_frags.shape[1], kv_frags.shape[2] * 64
    K = indices.shape[-1]
    qc = q.contiguous()
    kf = kv_frags.contiguous()
    w = weights.to(torch.bfloat16).contiguous()
    idx = indices.to(torch.int32).contiguous()
    kv = None if key_valid is None else key_valid.to(device=q.device, dtype=torch.bool).contiguous()
    out = torch.empty(B, Lq, Hq, D, dtype=torch.bfloat16, device=q.device)
    if deterministic:
        lo = lw = keep = partial = qf = None
        if fuse_local is not None:
            lo = fuse_local.to(torch.bfloat16).contiguous()
            lw = fuse_weight.to(torch.bfloat16).contiguous()
        if token_keep is not None:
            keep = token_keep.to(device=q.device, dtype=torch.int8).contiguous()
        if parts > 1:
            partial = torch.empty(parts, B, Lq, Hq, D, dtype=torch.float32, device=q.device)
        if q_frags is not None:
            qf = q_frags.contiguous()
        st = _lib.call(
            "mrsa_selected_attention_ex_fwd",
            _lib.ptr(qc), _lib.ptr(qf), _lib.ptr(kf), _lib.ptr(w), _lib.ptr(idx), _lib.ptr(kv),
            _lib.ptr(keep), _lib.ptr(lo), _lib.ptr(lw), B, Lq, Lk, Hq, Hkv, D, K,
            int(chunk_size), 1 if mask_last_token else 0, float(sm_scale), parts,
            _lib.ptr(partial), _ROUTED_FIXED_ORDER, _lib.ptr(out), _lib.stream_of(qc),
        )
        _lib.check(st, "selected_attention")
        return out
    if fuse_local is not None:
        lo = fuse_local.to(torch.bfloat16).contiguous()
        lw = fuse_weight.to(torch.bfloat16).contiguous()
        keep = None
        if token_keep is not None:
            keep = token_keep.to(device=q.device, dtype=torch.int8).contiguous()
        partial = None
        if parts > 1:
            partial = torch.empty(parts, B, Lq, Hq, D, dtype=torch.float32, device=q.device)
        if q_frags is not None:
            st = _lib.call(
                "mrsa_selected_attention_fused_qf_fwd",
                _lib.ptr(qc), _lib.ptr(q_frags.contiguous()), _lib.ptr(kf), _lib.ptr(w),
                _lib.ptr(idx), _lib.ptr(kv), _lib.ptr(keep), _lib.ptr(lo), _lib.ptr(lw),
                B, Lq, Lk, Hq, Hkv, D, K, int(chunk_size), 1 if mask_last_token else 0,
                float(sm_scale), parts, _lib.ptr(partial), _lib.ptr(out), _lib.stream_of(qc),
            )
        else:
            st = _lib.call(
                "mrsa_selected_attention_fused_fwd",
                _lib.ptr(qc), _lib.ptr(kf), _lib.ptr(w), _lib.ptr(idx),
                _lib.ptr(kv), _lib.ptr(keep), _lib.ptr(lo), _lib.ptr(lw), B, Lq, Lk, Hq, Hkv, D,
                K, int(chunk_size), 1 if mask_last_token else 0, float(sm_scale), parts,
                _lib.ptr(partial), _lib.ptr(out), _lib.stream_of(qc),
            )
    elif token_keep is not None:
        keep = token_keep.to(device=q.device, dtype=torch.int8).contiguous()
        partial = None
        if parts > 1:
            partial = torch.empty(parts, B, Lq, Hq, D, dtype=torch.float32, device=q.device)
        st = _lib.call(
            "mrsa_selected_attention_keep_fwd",
            _lib.ptr(qc), _lib.ptr(kf), _lib.ptr(w), _lib.ptr(idx),
            _lib.ptr(kv), _lib.ptr(keep), B, Lq, Lk, Hq, Hkv, D, K, int(chunk_size),
            1 if mask_last_token else 0, float(sm_scale), parts, _lib.ptr(partial),
            _lib.ptr(out), _lib.stream_of(qc),
        )
    elif parts == 1:
        st = _lib.call(
            "mrsa_selected_attention_fwd",
            _lib.ptr(qc), _lib.ptr(kf), _lib.ptr(w), _lib.ptr(idx),
            _lib.ptr(kv), B, Lq, Lk, Hq, Hkv, D, K, int(chunk_size),
            1 if mask_last_token else 0, float(sm_scale), _lib.ptr(out), _lib.stream_of(qc),
        )
    else:
        partial = torch.empty(parts, B, Lq, Hq, D, dtype=torch.float32, device=q.device)
        st = _lib.call(
            "mrsa_selected_attention_split_fwd",
            _lib.ptr(qc), _lib.ptr(kf), _lib.ptr(w), _lib.ptr(idx),
            _lib.ptr(kv), B, Lq, Lk, Hq, Hkv, D, K, int(chunk_size),
            1 if mask_last_token else 0, float(sm_scale), parts, _lib.ptr(partial),
            _lib.ptr(out), _lib.stream_of(qc),
        )
    _lib.check(st, "selected_attention")
    return out


def selected_attention_backward(q, k, v, weights, indices, key_valid, chunk_size, grad_output,
                                *, mask_last_token=True, sm_scale=None, token_keep=None):
    """Gradients (dq, dk, dv, dweights) of the routed attention, in the input
    dtypes (ops/hils_fwd_bwd_head.py:1050-1098: fp32 accumulation, cast at
    the end).  The fragment layouts of (k, v) and of (v, k) are built here."""

    return torch.ops.mrsa.selected_attention_bwd(
        q, kv_fragments_cached(k, v), kv_fragments_cached(v, k), weights, indices, key_valid,
        grad_output, int(chunk_size), bool(mask_last_token),
        float(sm_scale if sm_scale is not None else 1.0 / math.sqrt(q.shape[-1])), token_keep,
        int(k.shape[1]))


def _selected_attention_bwd_impl(q, kv_frags, kv_frags_bwd, weights, indices, key_valid,
                                 grad_output, chunk_size, mask_last_token, sm_scale,
                                 token_keep, kv_len):
    B, Lq, Hq, D = q.shape
    Hkv = kv_frags.shape[1]
    K = indices.shape[-1]
    qc = q.to(torch.bfloat16).contiguous()
    go = grad_output.to(torch.bfloat16).contiguous()
    w = weights.to(torch.bfloat16).contiguous()
    idx = indices.to(torch.int32).contiguous()
    kv = None if key_valid is None else key_valid.to(device=q.device, dtype=torch.bool).contiguous()
    keep = None if token_keep is None else token_keep.to(device=q.device, dtype=torch.int8).contiguous()
    dq = torch.zeros(B, Lq, Hq, D, dtype=torch.float32, device=q.device)
    dk = torch.zeros(B, kv_len, Hkv, D, dtype=torch.float32, device=q.device)
    dv = torch.zeros(B, kv_len, Hkv, D, dtype=torch.float32, device=q.device)
    dw = torch.zeros(B, Lq, Hq, K, dtype=torch.bfloat16, device=q.device)
    nbytes = int(_lib.call("mrsa_selected_attention_bwd_workspace_bytes", B, Lq, kv_len, Hq, Hkv, K))
    if nbytes < 0:
        raise ValueError(f"invalid routed attention shapes q {tuple(q.shape)} kv_len {kv_len}")
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=q.device)
    st = _lib.call(
        "mrsa_selected_attention_bwd",
        _lib.ptr(qc), _lib.ptr(go), _lib.ptr(kv_frags.contiguous()),
        _lib.ptr(kv_frags_bwd.contiguous()), _lib.ptr(w), _lib.ptr(idx), _lib.ptr(kv),
        _lib.ptr(keep), B, Lq, kv_len, Hq, Hkv, D, K, int(chunk_size),
        1 if mask_last_token else 0, float(sm_scale), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv),
        _lib.ptr(dw), _lib.ptr(ws), nbytes, _lib.stream_of(qc),
    )
    _lib.check(st, "selected_attention backward")
    return dq, dk, dv, dw


def selected_attention_alibi_launch(q, kv_frags, weights, indices, key_valid, chunk_size, slope,
                                   *, mask_last_token=True, sm_scale=None, parts=None,
                                   token_keep=None, deterministic=False):
    """selected_attention_launch with ALiBi slopes (fp32 [Hq]): before the
    scale, key s of a chunk gets -slope[head] * max(0, 62 - s) on its raw
    logit (ops/hils_fwd_bwd_head.py:445-451, hils_torch_ref :68-76)."""

    B, Lq, Hq, D = q.shape
    if kv_frags.ndim != 4 or kv_frags.shape[0] != B or kv_frags.shape[3] != FRAG_ELEMS:
        raise ValueError(f"kv_frags {tuple(kv_frags.shape)} is not a kv_fragments layout")
    if slope.shape != (Hq,):
        raise ValueError(f"slope must be 1-D with shape ({Hq},), got {tuple(slope.shape)}")
    Hkv, Lk = kv_frags.shape[1], kv_frags.shape[2] * 64
    K = indices.shape[-1]
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    if parts is None:
        parts = walk_parts(B, Lq, Hkv, Lk, K, chunk_size)
    parts = int(parts)
    if not 1 <= parts <= _SEL_MAX_PARTS:
        raise ValueError(f"parts must be in [1, {_SEL_MAX_PARTS}], got {parts}")
    qc = q.contiguous()
    w = weights.to(torch.bfloat16).contiguous()
    idx = indices.to(torch.int32).contiguous()
    kv = None if key_valid is None else key_valid.to(device=q.device, dtype=torch.bool).contiguous()
    keep = None if token_keep is None else token_keep.to(device=q.device, dtype=torch.int8).contiguous()
    sl = slope.to(device=q.device, dtype=torch.float32).contiguous()
    out = torch.empty(B, Lq, Hq, D, dtype=torch.bfloat16, device=q.device)
    partial = None
    if parts > 1:
        partial = torch.empty(parts, B, Lq, Hq, D, dtype=torch.float32, device=q.device)
    st = _lib.call(
        "mrsa_selected_attention_alibi_fwd",
        _lib.ptr(qc), None, _lib.ptr(kv_frags.contiguous()), _lib.ptr(w), _lib.ptr(idx),
        _lib.ptr(kv), _lib.ptr(keep), None, None, _lib.ptr(sl), B, Lq, Lk, Hq, Hkv, D, K,
        int(chunk_size), 1 if mask_last_token else 0, float(sm_scale), parts, _lib.ptr(partial),
        _ROUTED_FIXED_ORDER if deterministic else 0, _lib.ptr(out), _lib.stream_of(qc),
    )
    _lib.check(st, "selected_attention (ALiBi)")
    return out


def selected_attention_alibi_backward(q, k, v, weights, indices, key_valid, chunk_size,
                                      grad_output, slope, *, mask_last_token=True,
                                      sm_scale=None, token_keep=None):
    """Gradients (dq, dk, dv, dweights) of selected_attention_alibi_launch, fp32
    (ops/hils_fwd_bwd_head.py:755-760: the backward's bias term).  No
    gradient flows to the slopes."""

    B, Lq, Hq, D = q.shape
    Lk, Hkv = k.shape[1], k.shape[2]
    K = indices.shape[-1]
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    qc = q.to(torch.bfloat16).contiguous()
    go = grad_output.to(torch.bfloat16).contiguous()
    w = weights.to(torch.bfloat16).contiguous()
    idx = indices.to(torch.int32).contiguous()
    kv = None if key_valid is None else key_valid.to(device=q.device, dtype=torch.bool).contiguous()
    keep = None if token_keep is None else token_keep.to(device=q.device, dtype=torch.int8).contiguous()
    sl = slope.to(device=q.device, dtype=torch.float32).contiguous()
    dq = torch.zeros(B, Lq, Hq, D, dtype=torch.float32, device=q.device)
    dk = torch.zeros(B, Lk, Hkv, D, dtype=torch.float32, device=q.device)
    dv = torch.zeros(B, Lk, Hkv, D, dtype=torch.float32, device=q.device)
    dw = torch.zeros(B, Lq, Hq, K, dtype=torch.bfloat16, device=q.device)
    nbytes = int(_lib.call("mrsa_selected_attention_bwd_workspace_bytes", B, Lq, Lk, Hq, Hkv, K))
    if nbytes < 0:
        raise ValueError(f"invalid routed attention shapes q {tuple(q.shape)} kv_len {Lk}")
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=q.device)
    st = _lib.call(
        "mrsa_selected_attention_alibi_bwd",
        _lib.ptr(qc), _lib.ptr(go), _lib.ptr(kv_fragments_cached(k, v)),
        _lib.ptr(kv_fragments_cached(v, k)), _lib.ptr(w), _lib.ptr(idx), _lib.ptr(kv),
        _lib.ptr(keep), _lib.ptr(sl), B, Lq, Lk, Hq, Hkv, D, K, int(chunk_size),
        1 if mask_last_token else 0, float(sm_scale), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv),
        _lib.ptr(dw), _lib.ptr(ws), nbytes, _lib.stream_of(qc),
    )
    _lib.check(st, "selected_attention backward (ALiBi)")
    return dq, dk, dv, dw


def _routed_forward(q, k, v, weights, indices, key_valid, chunk_size, mask_last_token,
                    sm_scale, token_keep, slope):
    if slope is not None:
        return selected_attention_alibi_launch(
            q, kv_fragments_cached(k, v), weights, indices, key_valid, chunk_size, slope,
            mask_last_token=mask_last_token, sm_scale=sm_scale, token_keep=token_keep)
    return selected_attention_launch(
        q, kv_fragments_cached(k, v), weights, indices, key_valid, chunk_size,
        mask_last_token=mask_last_token, sm_scale=sm_scale, token_keep=token_keep)


class _SelectedAttention(torch.autograd.Function):
    # ops/hils_fwd_bwd_head.py:915-1098 (_hils_block_M_attention_inverse):
    # the forward saves its inputs; the backward recomputes each chunk's
    # softmax and casts the fp32 gradients to the input dtypes.  The ALiBi
    # slopes get no gradient (the reference returns none for them).
    @staticmethod
    def forward(ctx, q, k, v, weights, indices, key_valid, chunk_size, mask_last_token,
                sm_scale, token_keep, slope=None):
        ctx.save_for_backward(q, k, v, weights, indices, key_valid, token_keep, slope)
        ctx.chunk_size, ctx.mask_last_token, ctx.sm_scale = chunk_size, mask_last_token, sm_scale
        return _routed_forward(q, k, v, weights, indices, key_valid, chunk_size, mask_last_token,
                               sm_scale, token_keep, slope)

    @staticmethod
    def backward(ctx, grad_output):
        q, k, v, weights, indices, key_valid, token_keep, slope = ctx.saved_tensors
        if slope is not None:
            dq, dk, dv, dw = selected_attention_alibi_backward(
                q, k, v, weights, indices, key_valid, ctx.chunk_size, grad_output, slope,
                mask_last_token=ctx.mask_last_token, sm_scale=ctx.sm_scale,
                token_keep=token_keep)
        else:
            dq, dk, dv, dw = selected_attention_backward(
                q, k, v, weights, indices, key_valid, ctx.chunk_size, grad_output,
                mask_last_token=ctx.mask_last_token, sm_scale=ctx.sm_scale,
                token_keep=token_keep)
        grads = (dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dw.to(weights.dtype),
                 None, None, None, None, None, None, None)
        return grads[:len(ctx.needs_input_grad)]


def selected_attention_autograd(q, k, v, weights, indices, key_valid, chunk_size, *,
                                mask_last_token=True, sm_scale=None, token_keep=None,
                                slope=None):
    """Routed attention with autograd when an input requires grad (gfx950
    forward and backward kernels), else the plain forward.  ``slope`` (fp32
    [Hq]) adds the reference's ALiBi bias."""

    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v, weights)):
        return _SelectedAttention.apply(q, k, v, weights, indices, key_valid, chunk_size,
                                        mask_last_token, sm_scale, token_keep, slope)
    return _routed_forward(q, k, v, weights, indices, key_valid, chunk_size, mask_last_token,
                           sm_scale, token_keep, slope)


def HiLS_block_M_head(
    q, k, v, weights, indices,
    block_size=64, sm_scale=None, block_M=None,
    mask_last_token=True, dtype="bfloat16", accum_dtype="float",
    num_threads=None, num_threads_fwd=None, num_threads_bwd=None,
    is_training=True, slope=None, key_valid=None, token_keep=None,
):
    """Same arguments as ops/hils_fwd_bwd_head.py:1113-1150, with autograd
    (the backward of ops/hils_fwd_bwd_head.py:573-910) when an input requires
    grad.

    Tiling knobs (block_M, num_threads*) are accepted and ignored: the gfx950
    kernels pick their own tiling.  ``slope`` (shape (HQ,)) adds the ALiBi
    bias -slope[head] * max(0, block_size - 2 - s) to the raw logit of chunk
    key s (ops/hils_fwd_bwd_head.py:971-978, :445-451).
    """

    B, L, HQ, D = q.shape
    _, L_kv, H, Dk = k.shape
    assert D == Dk, f"Q head_dim ({D}) must equal K head_dim ({Dk})"
    assert HQ % H == 0, f"HQ={HQ} must be divisible by H={H}"
    if slope is not None:
        assert tuple(slope.shape) == (HQ,), (
            f"slope must be 1-D with shape ({HQ},), got {tuple(slope.shape)}"
        )
        slope = slope.to(dtype=torch.float32, device=q.device).contiguous()
    if token_keep is not None:
        expected_keep_shape = (B, L, H, indices.shape[-1], block_size)
        if token_keep.shape != expected_keep_shape:
            raise ValueError(
                "token_keep must have shape "
                f"{expected_keep_shape}, got {tuple(token_keep.shape)}"
            )
    if dtype != "bfloat16" or accum_dtype != "float":
        raise ValueError("only bf16 inputs with fp32 accumulation are supported")
    if key_valid is not None and key_valid.shape != (B, L_kv):
        raise ValueError(f"key_valid must have shape {(B, L_kv)}, got {tuple(key_valid.shape)}")
    return selected_attention_autograd(
        q, k, v, weights, indices, key_valid, block_size,
        mask_last_token=mask_last_token, sm_scale=sm_scale, token_keep=token_keep, slope=slope,
    )
