"""The C-ABI library loads, exports every declared entry point and rejects bad
arguments on the host (no GPU needed: nothing here launches a kernel)."""

import ctypes
import os
import re

import pytest

from conftest import PKG_DIR, ROOT

HEADER = os.path.join(ROOT, "include", "mrsa.h")
LIB = os.path.join(PKG_DIR, "mrsa", "libmrsa.so")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mrsa_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} missing: run __graft_entry__.build() first")
    return ctypes.CDLL(LIB)


def test_header_lists_expected_entry_points():
    names = _declared()
    for expected in (
        "mrsa_chunk_attn_pool_gqa_fwd", "mrsa_remote_drop_mask", "mrsa_route_topk_fwd",
        "mrsa_route_weights_fwd", "mrsa_local_attention_fwd", "mrsa_selected_attention_fwd",
        "mrsa_fuse_hils_outputs_fwd", "mrsa_candidate_token_scores_fwd",
        "mrsa_kv_fragments", "mrsa_kv_fragments_rows",
    ):
        assert expected in names


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_python_binding_matches_header():
    import mrsa._lib as L

    assert sorted(L.SIGNATURES) == _declared()


def test_status_strings_and_version(lib):
    lib.mrsa_status_string.restype = ctypes.c_char_p
    assert lib.mrsa_status_string(0) == b"ok"
    assert b"invalid" in lib.mrsa_status_string(1)
    assert lib.mrsa_abi_version() >= 3


def test_host_side_argument_errors(lib):
    import mrsa._lib as L

    L.load()
    # Negative sizes and NULL pointers are rejected before any launch.
    assert L.call("mrsa_fuse_hils_outputs_fwd", None, None, None, None, -1, 128, None) == 1
    assert L.call("mrsa_fuse_hils_outputs_fwd", None, None, None, None, 4, 128, None) == 1
    assert L.call("mrsa_remote_drop_mask", None, None, 1, 100, 256, 64, None, None) == 1
    assert L.call("mrsa_chunk_attn_pool_gqa_fwd", None, None, None, 4, 64, 4, 17, 128,
                  1.0, 0, None, None, None, None, None) == 1
    assert L.call("mrsa_local_attention_fwd", 16, 16, None, None, 1, 64, 64, 28, 4, 96,
                  256, 0, 1.0, 16, 16, None) == 2          # head_dim 96 unsupported
    assert L.call("mrsa_selected_attention_fwd", 16, 16, 16, 16, None, 1, 64, 128, 28, 4,
                  128, 32, 32, 1, 1.0, 16, None) == 2      # chunk_size 32 unsupported
    assert L.call("mrsa_route_weights_fwd", 16, 16, 16, 16, 1, 4, 4, 4, 7, 65, 1.0, None,
                  None, 16, 16, None, None) == 2           # topk > 64
    assert L.call("mrsa_route_weights_fwd", 16, 16, 16, 16, 1, 4, 4, 4, 7, 32, 0.0, None,
                  None, 16, 16, None, None) == 1           # temperature <= 0
    assert L.call("mrsa_route_weights_bwd", 16, 16, 16, 16, 16, None, None, 1, 4, 4, 4, 7, 32,
                  1.0, 16, None, 16, 16, 16, None, None) == 1  # gate given, no d_gate
    # Walk split: parts outside 1..64, or a missing workspace, are rejected.
    assert L.call("mrsa_selected_attention_split_fwd", 16, 16, 16, 16, None, 1, 64, 128,
                  28, 4, 128, 32, 64, 1, 1.0, 0, 16, 16, None) == 1
    assert L.call("mrsa_selected_attention_split_fwd", 16, 16, 16, 16, None, 1, 64, 128,
                  28, 4, 128, 32, 64, 1, 1.0, 65, 16, 16, None) == 1
    assert L.call("mrsa_selected_attention_split_fwd", 16, 16, 16, 16, None, 1, 64, 128,
                  28, 4, 128, 32, 64, 1, 1.0, 4, None, 16, None) == 1
    assert L.call("mrsa_selected_attention_split_fwd", 16, 16, 16, 16, None, 2000, 64,
                  128, 28, 4, 128, 32, 64, 1, 1.0, 40, 16, 16, None) == 2  # batch * parts
    assert L.call("mrsa_kv_fragments_bytes", 2, 65, 4, 128) == 2 * 4 * 2 * 16384 * 2
    assert L.call("mrsa_kv_fragments_bytes", 1, 64, 4, 96) == -1
    assert L.call("mrsa_kv_fragments", 16, None, 1, 64, 4, 96, 16, None) == 2  # head_dim 96
    assert L.call("mrsa_kv_fragments", None, None, 1, 64, 4, 128, 16, None) == 1
    # Empty problems are a successful no-op.
    assert L.call("mrsa_fuse_hils_outputs_fwd", None, None, None, None, 0, 128, None) == 0


def test_key_parts_heuristic():
    from mrsa.local_attention import key_parts

    assert key_parts(1, 16384, 4, 16384, 319) == 1
    # Cached block step: 32 queries (8 workgroups), window 319 -> 8 parts.
    assert key_parts(1, 32, 4, 131072, 319) == 8
    assert key_parts(1, 32, 4, 131072, 0) == 2
    assert key_parts(0, 32, 4, 4096, 319) == 1


def test_walk_parts_heuristic():
    from mrsa.sparse_attention import walk_parts

    # Long sequences: one workgroup per walk.
    assert walk_parts(1, 16384, 4, 16384, 32) == 1
    # The cached block step (32 queries, 4 KV heads, 2048 chunks): 32 parts.
    assert walk_parts(1, 32, 4, 131072, 32) == 32
    # Parts keep >= 32 steps each: 3 queries x 4 chunks -> 12 steps -> 1.
    assert walk_parts(1, 3, 4, 131072, 4) == 1
    assert walk_parts(1, 32, 4, 4096, 32) == 2
    assert walk_parts(0, 32, 4, 4096, 32) == 1


def test_layer_cache_replace_on_host_tensors():
    # fastdllm_cache.py:94-125 on CPU tensors (no tiled copy yet): rows land,
    # errors as in the reference.
    import torch

    import mrsa

    k = torch.zeros(1, 256, 4, 8, dtype=torch.bfloat16)
    v = torch.zeros_like(k)
    cache = mrsa.LayerKVCache(k, v, torch.ones(1, 256, dtype=torch.bool),
                              torch.zeros(1, 4, 4, 7, 8, dtype=torch.bfloat16),
                              torch.zeros(1, 4, 4, 7))
    pos = torch.tensor([7, 3])
    cache.replace(pos, torch.ones(1, 2, 4, 8, dtype=torch.bfloat16),
                  torch.full((1, 2, 4, 8), 2.0, dtype=torch.bfloat16))
    assert float(cache.key[0, 3].float().sum()) == 32 and float(cache.value[0, 7, 0, 0]) == 2
    assert cache.physical_length == 256
    with pytest.raises(ValueError, match="unique"):
        cache.replace(torch.tensor([1, 1]), k[:, :2], v[:, :2])
    with pytest.raises(ValueError, match="range"):
        cache.replace(torch.tensor([256]), k[:, :1], v[:, :1])
    with pytest.raises(ValueError, match="shape"):
        cache.replace(torch.tensor([1]), k[:, :2], v[:, :2])
