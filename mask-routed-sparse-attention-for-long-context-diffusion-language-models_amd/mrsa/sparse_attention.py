"""Routed chunk attention (and the tiled V layout it reads).

Drop-in for ``ops.hils_fwd_bwd_head.HiLS_block_M_head``
(ops/hils_fwd_bwd_head.py:1113-1150) in its forward role, plus
``value_tiles``, the V re-layout both attention kernels consume.
"""

from __future__ import annotations

import math

import torch

from . import _lib


def value_tiles(v: torch.Tensor) -> torch.Tensor:
    """V [B, L, Hkv, D] bf16 -> 64-key tiles stored transposed [B, Hkv, ceil(L/64), D, 64].

    Inside a tile row, key 32a + 16b + 4c + e (a, b in {0,1}; c, e in 0..3) sits
    at position 32a + 8c + 4b + e, the order the matrix-core kernels read it in.
    """

    if v.device.type != "cuda" or v.dtype != torch.bfloat16 or v.ndim != 4:
        raise ValueError("value_tiles requires a CUDA BF16 [B, L, Hkv, D] tensor")
    return torch.ops.mrsa.value_tiles(v)


def _value_tiles_impl(v: torch.Tensor) -> torch.Tensor:
    B, L, H, D = v.shape
    vc = v.contiguous()
    out = torch.empty(B, H, (L + 63) // 64, D, 64, dtype=torch.bfloat16, device=v.device)
    st = _lib.call("mrsa_value_tiles", _lib.ptr(vc), B, L, H, D, _lib.ptr(out), _lib.stream_of(vc))
    _lib.check(st, "value_tiles")
    return out


# Queries per routed-attention workgroup (12 waves x 2 column tiles x 2).
_SEL_TILE_QUERIES = 48
_SEL_MAX_PARTS = 64


def walk_parts(batch: int, q_len: int, kv_heads: int, kv_len: int, topk: int,
               chunk_size: int = 64) -> int:
    """Workgroups per (query tile, KV head) walk of the routed attention.

    Long sequences fill the chip with one workgroup per walk.  A short query
    block (the cached block step: 32 queries, 4 KV heads -> 4 walks of up to
    1024 chunks) splits each walk into parts of >= 16 steps so that about 512
    workgroups run.
    """

    walks = -(-q_len // _SEL_TILE_QUERIES) * kv_heads * batch
    if walks >= 128 or walks == 0:
        return 1
    steps = min(kv_len // chunk_size, min(_SEL_TILE_QUERIES, q_len) * topk)
    parts = min(_SEL_MAX_PARTS, 512 // walks, steps // 16, 65535 // max(batch, 1))
    return max(1, parts)


def value_tiles_rows(v: torch.Tensor, v_tiles: torch.Tensor, positions: torch.Tensor) -> None:
    """Rewrite the tiles of rows ``positions`` of v in ``v_tiles`` (in place),
    after those rows of v were replaced.  Positions outside [0, L) are ignored."""

    if v.device.type != "cuda" or v.dtype != torch.bfloat16 or v.ndim != 4:
        raise ValueError("value_tiles_rows requires a CUDA BF16 [B, L, Hkv, D] tensor")
    B, L, H, D = v.shape
    if v_tiles.shape != (B, H, (L + 63) // 64, D, 64) or not v_tiles.is_contiguous():
        raise ValueError("v_tiles must be the contiguous value_tiles(v) layout")
    torch.ops.mrsa.value_tiles_rows_(v, v_tiles, positions)


def _value_tiles_rows_impl(v: torch.Tensor, v_tiles: torch.Tensor, positions: torch.Tensor) -> None:
    B, L, H, D = v.shape
    vc = v.contiguous()
    pos = positions.to(device=v.device, dtype=torch.long).contiguous()
    st = _lib.call("mrsa_value_tiles_rows", _lib.ptr(vc), B, L, H, D, _lib.ptr(pos),
                   pos.numel(), _lib.ptr(v_tiles), _lib.stream_of(vc))
    _lib.check(st, "value_tiles_rows")


def selected_attention_launch(
    q: torch.Tensor,
    k: torch.Tensor,
    v_tiles: torch.Tensor,
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
) -> torch.Tensor:
    """q [B, Lq, Hq, D], k [B, Lk, Hkv, D], weights [B, Lq, Hq, K] -> [B, Lq, Hq, D] bf16.

    ``parts`` splits each walk over that many workgroups (fp32 partial
    outputs summed by a second kernel); None picks it with ``walk_parts``.
    ``token_keep`` [B, Lq, Hkv, K, chunk_size] (nonzero = kept) additionally
    masks the keys of each query's slot k.  ``fuse_local`` [B, Lq, Hq, D] and
    ``fuse_weight`` [B, Lq, Hq] (bf16, both or neither) fold the output
    fusion in: the result is fuse_hils_outputs(routed, fuse_local,
    fuse_weight), bit for bit, without materialising the routed output.
    """

    B, Lq, Hq, D = q.shape
    Lk, Hkv = k.shape[1], k.shape[2]
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
    return torch.ops.mrsa.selected_attention(
        q, k, v_tiles, weights, indices, key_valid, int(chunk_size), bool(mask_last_token),
        float(sm_scale), parts, token_keep, fuse_local, fuse_weight)


def _selected_attention_impl(q, k, v_tiles, weights, indices, key_valid, chunk_size,
                             mask_last_token, sm_scale, parts, token_keep, fuse_local,
                             fuse_weight):
    B, Lq, Hq, D = q.shape
    Lk, Hkv = k.shape[1], k.shape[2]
    K = indices.shape[-1]
    qc = q.contiguous()
    kc = k.contiguous()
    w = weights.to(torch.bfloat16).contiguous()
    idx = indices.to(torch.int32).contiguous()
    kv = None if key_valid is None else key_valid.to(device=q.device, dtype=torch.bool).contiguous()
    out = torch.empty(B, Lq, Hq, D, dtype=torch.bfloat16, device=q.device)
    if fuse_local is not None:
        lo = fuse_local.to(torch.bfloat16).contiguous()
        lw = fuse_weight.to(torch.bfloat16).contiguous()
        keep = None
        if token_keep is not None:
            keep = token_keep.to(device=q.device, dtype=torch.int8).contiguous()
        partial = None
        if parts > 1:
            partial = torch.empty(parts, B, Lq, Hq, D, dtype=torch.float32, device=q.device)
        st = _lib.call(
            "mrsa_selected_attention_fused_fwd",
            _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(v_tiles), _lib.ptr(w), _lib.ptr(idx),
            _lib.ptr(kv), _lib.ptr(keep), _lib.ptr(lo), _lib.ptr(lw), B, Lq, Lk, Hq, Hkv, D, K,
            int(chunk_size), 1 if mask_last_token else 0, float(sm_scale), parts,
            _lib.ptr(partial), _lib.ptr(out), _lib.stream_of(qc),
        )
    elif token_keep is not None:
        keep = token_keep.to(device=q.device, dtype=torch.int8).contiguous()
        partial = None
        if parts > 1:
            partial = torch.empty(parts, B, Lq, Hq, D, dtype=torch.float32, device=q.device)
        st = _lib.call(
            "mrsa_selected_attention_keep_fwd",
            _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(v_tiles), _lib.ptr(w), _lib.ptr(idx),
            _lib.ptr(kv), _lib.ptr(keep), B, Lq, Lk, Hq, Hkv, D, K, int(chunk_size),
            1 if mask_last_token else 0, float(sm_scale), parts, _lib.ptr(partial),
            _lib.ptr(out), _lib.stream_of(qc),
        )
    elif parts == 1:
        st = _lib.call(
            "mrsa_selected_attention_fwd",
            _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(v_tiles), _lib.ptr(w), _lib.ptr(idx),
            _lib.ptr(kv), B, Lq, Lk, Hq, Hkv, D, K, int(chunk_size),
            1 if mask_last_token else 0, float(sm_scale), _lib.ptr(out), _lib.stream_of(qc),
        )
    else:
        partial = torch.empty(parts, B, Lq, Hq, D, dtype=torch.float32, device=q.device)
        st = _lib.call(
            "mrsa_selected_attention_split_fwd",
            _lib.ptr(qc), _lib.ptr(kc), _lib.ptr(v_tiles), _lib.ptr(w), _lib.ptr(idx),
            _lib.ptr(kv), B, Lq, Lk, Hq, Hkv, D, K, int(chunk_size),
            1 if mask_last_token else 0, float(sm_scale), parts, _lib.ptr(partial),
            _lib.ptr(out), _lib.stream_of(qc),
        )
    _lib.check(st, "selected_attention")
    return out


def HiLS_block_M_head(
    q, k, v, weights, indices,
    block_size=64, sm_scale=None, block_M=None,
    mask_last_token=True, dtype="bfloat16", accum_dtype="float",
    num_threads=None, num_threads_fwd=None, num_threads_bwd=None,
    is_training=True, slope=None, key_valid=None, token_keep=None,
):
    """Same arguments as ops/hils_fwd_bwd_head.py:1113-1150, forward only.

    Tiling knobs (block_M, num_threads*) are accepted and ignored: the gfx950
    kernel picks its own tiling.  ALiBi slopes are not supported.
    """

    B, L, HQ, D = q.shape
    _, L_kv, H, Dk = k.shape
    assert D == Dk, f"Q head_dim ({D}) must equal K head_dim ({Dk})"
    assert HQ % H == 0, f"HQ={HQ} must be divisible by H={H}"
    if slope is not None:
        raise ValueError("ALiBi slopes are not supported by the gfx950 routed-attention kernel")
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
    if any(t.requires_grad for t in (q, k, v, weights)) and torch.is_grad_enabled():
        raise ValueError("HiLS_block_M_head on gfx950 is forward-only (no autograd)")
    return selected_attention_launch(
        q, k, value_tiles(v), weights, indices, key_valid, block_size,
        mask_last_token=mask_last_token, sm_scale=sm_scale, token_keep=token_keep,
    )
