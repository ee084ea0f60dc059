"""ctypes binding of libmrsa.so, the gfx950 C-ABI library (include/mrsa.h).

The library is loaded lazily, from this directory only.  If it is missing or
cannot be loaded every op raises immediately: there is no CPU fallback.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmrsa.so")

MRSA_OK = 0
MRSA_ERR_INVALID_ARGUMENT = 1
MRSA_ERR_UNSUPPORTED = 2
MRSA_ERR_LAUNCH = 3
MRSA_ERR_SCRATCH = 4

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float

# name -> (restype, argtypes); mirrors include/mrsa.h exactly.
SIGNATURES = {
    "mrsa_status_string": (ctypes.c_char_p, [_I]),
    "mrsa_abi_version": (_I, []),
    "mrsa_fuse_hils_outputs_fwd": (_I, [_P, _P, _P, _P, _I64, _I64, _P]),
    "mrsa_add_rms_norm_fwd": (_I, [_P, _P, _P, _I64, _I64, _F, _P, _P, _P]),
    "mrsa_rope_qkv_fwd": (
        _I, [_P, _P, _P, _P, _P, _F, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P],
    ),
    "mrsa_swiglu_fwd": (_I, [_P, _I64, _I64, _P, _P]),
    "mrsa_fuse_hils_outputs_bwd": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _P]),
    "mrsa_chunk_attn_pool_gqa_fwd": (
        _I,
        [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _I, _P, _P, _P, _P, _P],
    ),
    "mrsa_chunk_attn_pool_gqa_strided_fwd": (
        _I,
        [_P, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _I, _P, _P, _P, _P, _P],
    ),
    "mrsa_chunk_attn_pool_gqa_bwd": (
        _I,
        [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _I, _P, _P, _P],
    ),
    "mrsa_remote_drop_mask": (_I, [_P, _P, _I64, _I64, _I64, _I64, _P, _P]),
    "mrsa_remote_drop_mask_rows": (_I, [_P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P]),
    "mrsa_route_topk_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
         _I64, _I, _I, _I64, _I64, _I, _F, _P, _P, _I, _P],
    ),
    "mrsa_route_topk_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64, _I64]),
    "mrsa_route_topk_ws_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
         _I64, _I, _I, _I64, _I64, _I, _F, _P, _P, _I, _P, _I64, _P],
    ),
    "mrsa_route_topk_noalloc_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
         _I64, _I, _I, _I64, _I64, _I, _F, _P, _P, _I, _P],
    ),
    "mrsa_route_score_bwd_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64, _I64, _I]),
    "mrsa_route_score_bwd": (
        _I,
        [_P, _P, _P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I, _F, _P, _P, _P,
         _I64, _P],
    ),
    "mrsa_route_weights_fwd": (
        _I,
        [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P, _P,
         _P, _P, _P, _P],
    ),
    "mrsa_route_weights_extra_fwd": (
        _I,
        [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P, _P,
         _P, _P, _P, _P, _P, _P],
    ),
    "mrsa_route_weights_extra_bwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P, _P,
         _P, _P, _P, _P, _P, _P, _P],
    ),
    "mrsa_route_weights_bwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P, _P,
         _P, _P, _P, _P, _P],
    ),
    "mrsa_kv_fragments_bytes": (_I64, [_I64, _I64, _I64, _I64]),
    "mrsa_kv_fragments": (_I, [_P, _P, _I64, _I64, _I64, _I64, _P, _P]),
    "mrsa_kv_fragments_rows": (_I, [_P, _P, _I64, _I64, _I64, _I64, _P, _I64, _P, _P]),
    "mrsa_cached_step_checks": (_I, [_P, _I64, _P, _I64, _I64, _I64, _P, _P]),
    "mrsa_copy_buffers": (_I, [_I, _P, _P, _P, _P]),
    "mrsa_kv_replace_rows": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P]),
    "mrsa_pool_cached_chunks_fwd": (
        _I,
        [_P, _P, _I64, _P, _P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _I64, _F, _P, _P, _P,
         _P],
    ),
    "mrsa_kv_fragments_pool_fwd": (
        _I,
        [_P, _P, _P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _F, _P, _P, _P, _P, _P, _P],
    ),
    "mrsa_q_fragments_bytes": (_I64, [_I64, _I64, _I64, _I64]),
    "mrsa_q_fragments": (_I, [_P, _I64, _I64, _I64, _I64, _I64, _P, _P]),
    "mrsa_local_attention_fwd": (
        _I,
        [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F,
         _P, _P, _P],
    ),
    "mrsa_local_attention_qf_fwd": (
        _I,
        [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F,
         _P, _P, _P, _P],
    ),
    "mrsa_local_attention_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64]),
    "mrsa_local_attention_split_fwd": (
        _I,
        [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F,
         _I64, _P, _I64, _P, _P, _P],
    ),
    "mrsa_selected_attention_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
         _I, _F, _P, _P],
    ),
    "mrsa_selected_attention_split_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
         _I, _F, _I64, _P, _P, _P],
    ),
    "mrsa_selected_attention_keep_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
         _I, _F, _I64, _P, _P, _P],
    ),
    "mrsa_selected_attention_fused_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
         _I, _F, _I64, _P, _P, _P],
    ),
    "mrsa_selected_attention_fused_qf_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
         _I, _F, _I64, _P, _P, _P],
    ),
    "mrsa_selected_attention_ex_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
         _I, _F, _I64, _P, _I, _P, _P],
    ),
    "mrsa_selected_attention_alibi_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
         _I64, _I, _F, _I64, _P, _I, _P, _P],
    ),
    "mrsa_local_attention_bwd_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64]),
    "mrsa_local_attention_bwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P, _P, _P,
         _P, _I64, _P],
    ),
    "mrsa_routed_lock_giveups": (_I, [_P, _I]),
    "mrsa_set_routed_lock_spin_limit": (_I, [_I]),
    "mrsa_selected_attention_bwd_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "mrsa_selected_attention_bwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
         _I, _F, _P, _P, _P, _P, _P, _I64, _P],
    ),
    "mrsa_selected_attention_alibi_bwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
         _I, _F, _P, _P, _P, _P, _P, _I64, _P],
    ),
    "mrsa_token_keep_entropy_fwd": (
        _I,
        [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _P],
    ),
    "mrsa_gather_selected_chunk_entropy": (
        _I, [_P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P],
    ),
    "mrsa_token_keep_fwd": (_I, [_P, _I64, _I64, _I64, _P, _P]),
    "mrsa_candidate_token_scores_fwd": (
        _I,
        [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P, _P],
    ),
    "mrsa_selftest_mfma_layout": (_I, [_P, _P, _P, _P]),
}

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None


class MrsaLibraryError(RuntimeError):
    """libmrsa.so is missing or unusable."""


def load() -> ctypes.CDLL:
    """Load libmrsa.so (once) and attach the C signatures."""

    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise MrsaLibraryError(
                f"{LIB_PATH} not found: build it first (python -c "
                "'import __graft_entry__ as g; g.build()' from the repository root)"
            )
        try:
            lib = ctypes.CDLL(LIB_PATH)
        except OSError as exc:  # pragma: no cover - environment failure
            raise MrsaLibraryError(f"cannot load {LIB_PATH}: {exc}") from exc
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


def status_string(status: int) -> str:
    return load().mrsa_status_string(int(status)).decode()


def check(status: int, op: str) -> None:
    """Map a C status to the reference's Python exception convention."""

    if status == MRSA_OK:
        return
    msg = f"{op}: {status_string(status)} (status {status})"
    if status in (MRSA_ERR_INVALID_ARGUMENT, MRSA_ERR_UNSUPPORTED, MRSA_ERR_SCRATCH):
        raise ValueError(msg)
    raise RuntimeError(msg)


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    """Handle of the current HIP stream of the tensor's device."""

    return torch.cuda.current_stream(t.device).cuda_stream


def call(name: str, *args) -> int:
    return getattr(load(), name)(*args)


def copy_buffers(dst: list, src: list) -> None:
    """dst[i].copy_(src[i]) for same-shape, same-dtype contiguous CUDA
    tensors, in one launch (mrsa_copy_buffers; at most 8 pairs) when every
    size and address is a multiple of 8 bytes, else one copy_ per pair."""

    n = len(dst)
    if any((t.data_ptr() | t.numel() * t.element_size()) % 8 for t in list(src) + list(dst)):
        for d, s_ in zip(dst, src):
            d.copy_(s_)
        return
    srcs = (ctypes.c_void_p * max(n, 1))(*[t.data_ptr() for t in src])
    dsts = (ctypes.c_void_p * max(n, 1))(*[t.data_ptr() for t in dst])
    sizes = (ctypes.c_int64 * max(n, 1))(*[t.numel() * t.element_size() for t in src])
    st = call("mrsa_copy_buffers", n, ctypes.addressof(srcs), ctypes.addressof(dsts),
              ctypes.addressof(sizes), stream_of(dst[0]))
    check(st, "copy_buffers")
