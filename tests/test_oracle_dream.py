"""Pins of the Dream-forward oracle's glue (YaRN tables, RMSNorm, rotary,
SwiGLU) against closed forms and library routines, and the product's YaRN
tables against the oracle's."""

import math

import torch
import torch.nn.functional as F

from mrsa.dream import DreamShape, yarn_tables
from oracle import dream_oracle as DO


def test_route_layer_indices():
    assert DreamShape().route_layers() == [3, 7, 11, 15, 19, 23, 27]


def test_yarn_reduces_to_rope_and_blends_by_parts():
    inv1, af1 = DO.yarn_inv_freq(128, 1e6, 1.0, 2048)
    plain = torch.tensor([1e6 ** (-2 * i / 128) for i in range(64)], dtype=torch.float64)
    assert af1 == 1.0 and torch.allclose(inv1, plain, rtol=1e-12, atol=0)
    inv8, af8 = DO.yarn_inv_freq(128, 1e6, 8.0, 2048)
    assert abs(af8 - (0.1 * math.log(8) + 1)) < 1e-12
    # high-frequency dims (many turns over 2048 tokens) keep their frequency,
    # low-frequency dims (less than one turn) are interpolated by the factor
    turns = 2048 * plain / (2 * math.pi)
    assert torch.allclose(inv8[turns > 32], plain[turns > 32], rtol=1e-12, atol=0)
    assert torch.allclose(inv8[turns < 1], plain[turns < 1] / 8, rtol=1e-12, atol=0)
    mid = (turns >= 1) & (turns <= 32)
    assert bool(((inv8[mid] <= plain[mid]) & (inv8[mid] >= plain[mid] / 8)).all())


def test_product_yarn_tables_match_oracle():
    s = DreamShape()
    cos, sin = yarn_tables(3000, s, "cpu")
    ecos, esin = DO.yarn_tables(3000, 128, 1e6, 8.0, 2048)
    assert torch.equal(cos, ecos) and torch.equal(sin, esin)


def test_rms_norm_rope_swiglu_pins():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(17, 256, generator=g).bfloat16()
    w = (1 + 0.1 * torch.randn(256, generator=g)).bfloat16()
    ref = F.rms_norm(x.float(), (256,), eps=1e-6).bfloat16().float() * w.float()
    assert torch.equal(DO.rms_norm(x, w, 1e-6), ref.bfloat16())
    q = torch.randn(5, 3, 128, generator=g).bfloat16()
    ang = torch.rand(5, 64, generator=g) * 6.0
    cos, sin = ang.cos(), ang.sin()
    z = torch.complex(q.float()[..., :64], q.float()[..., 64:]) * torch.polar(
        torch.ones_like(ang), ang)[:, None, :]
    torch.testing.assert_close(DO.rope(q, cos, sin).float(),
                               torch.cat((z.real, z.imag), -1).bfloat16().float(),
                               atol=1e-2, rtol=1e-2)
    gu = torch.randn(9, 64, generator=g).bfloat16()
    ref = (F.silu(gu[:, :32].float()).bfloat16().float() * gu[:, 32:].float()).bfloat16()
    assert torch.equal(DO.swiglu(gu), ref)


def test_landmark_layout_positions():
    # data.py:999-1010 by hand for chunk_size 4: text slots 0, 1, 2 | 3, 4, 5 | ...,
    # each landmark one past its chunk's last text position.
    assert DO.landmark_positions(12, 4).tolist() == [0, 1, 2, 3, 3, 4, 5, 6, 6, 7, 8, 9]
    from mrsa.dream import landmark_layout, landmark_positions
    from mrsa.route_layer import RouteLayerConfig

    s = DreamShape(route=RouteLayerConfig(chunk_size=4))
    text = torch.arange(100, 109)[None]
    ids, pos = landmark_layout(text, s)
    assert ids.tolist() == [[100, 101, 102, s.mask_token_id, 103, 104, 105, s.mask_token_id,
                             106, 107, 108, s.mask_token_id]]
    assert pos.tolist() == DO.landmark_positions(12, 4).tolist()
    s64 = DreamShape()
    assert torch.equal(landmark_positions(4096, s64, "cpu"), DO.landmark_positions(4096, 64))


def test_yarn_factor8_matches_transformers_yarn():
    # transformers' own YaRN initialiser (ROPE_INIT_FUNCTIONS["yarn"], the
    # routine Dream's configuration reaches through train_fulltext.py:2820-2856)
    # at the configuration-3/4 parameters: theta 1e6, head_dim 128, factor 8,
    # original context 2048.  transformers computes in float32.
    import pytest

    rope_utils = pytest.importorskip("transformers.modeling_rope_utils")
    from transformers import PretrainedConfig

    def hf(factor, original):
        cfg = PretrainedConfig()
        cfg.hidden_size, cfg.num_attention_heads, cfg.head_dim = 3584, 28, 128
        cfg.max_position_embeddings = 131072
        cfg.rope_theta = 1e6
        cfg.rope_parameters = {"rope_type": "yarn", "factor": factor, "rope_theta": 1e6,
                               "original_max_position_embeddings": original}
        inv, af = rope_utils.ROPE_INIT_FUNCTIONS["yarn"](cfg, "cpu")
        return inv.double(), af

    inv, af = hf(8.0, 2048)
    inv8, af8 = DO.yarn_inv_freq(128, 1e6, 8.0, 2048)
    assert abs(af - af8) < 1e-12
    assert float(((inv - inv8).abs() / inv8).max()) < 1e-6
    # the comparison is sensitive to the parameters it pins
    inv_o, _ = hf(8.0, 4096)
    assert float(((inv_o - inv8).abs() / inv8).max()) > 1e-2
    inv4, af4 = hf(4.0, 2048)
    assert float(((inv4 - inv8).abs() / inv8).max()) > 1e-2 and af4 != af8
