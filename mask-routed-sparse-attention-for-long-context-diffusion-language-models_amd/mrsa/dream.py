"""Dream-7B-shaped denoising forward over the MRSA attention path.

The decoder follows the reference's layer loop (dream_dllm_hils/fastdllm_v1.py:
375-403, a Qwen2 decoder):

    h = embed(ids) (+ the landmark type embedding on each chunk's last slot,
        train_fulltext.py:2336-2350)
    per layer: a = attn(rms_norm(h)); h = h + o_proj(a);
               h = h + down(swiglu(gate_up(rms_norm(h))))
    logits = lm_head(rms_norm(h))

Layers ``i % interleave == interleave - 1`` are MRSA route layers
(``hils_layer_indices``, attention.py:1823-1826) with the Q-Cal routing query
(qcal.py:40-60, attention.py:460-511); the others are bidirectional
sliding-window layers.  GEMMs run on hipBLASLt through ``torch.nn.functional
.linear``; the attention stages and the elementwise glue run on the gfx950
kernels of libmrsa (``mrsa_add_rms_norm_fwd``, ``mrsa_rope_qkv_fwd``,
``mrsa_swiglu_fwd``).  Weights are random-initialised (no checkpoint).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

from . import _lib
from .route_layer import RouteLayerConfig, route_attention, swa_attention


@dataclass(frozen=True)
class DreamShape:
    """Dream-v0-Base-7B dimensions and the route-layer settings of the
    configuration the reference trains (configs/from_dense16k/*.json)."""

    layers: int = 28
    hidden: int = 3584
    intermediate: int = 18944
    q_heads: int = 28
    kv_heads: int = 4
    head_dim: int = 128
    vocab: int = 152064
    rope_theta: float = 1.0e6
    yarn_factor: float = 8.0
    yarn_original_max: int = 2048
    rms_eps: float = 1e-6
    interleave: int = 4
    swa_window: int = 1280
    qcal_rank: int = 64
    qcal_eps: float = 1e-6
    mask_token_id: int = 151666
    route: RouteLayerConfig = field(default_factory=RouteLayerConfig)

    def route_layers(self) -> list[int]:
        # attention.py:1823-1826
        if self.interleave <= 0:
            return list(range(self.layers))
        return [i for i in range(self.layers) if i % self.interleave == self.interleave - 1]


def yarn_tables(seq_len: int, shape: DreamShape, device) -> tuple[torch.Tensor, torch.Tensor]:
    """YaRN rotary tables (Peng et al. 2023, "YaRN: Efficient Context Window
    Extension of Large Language Models"; the rope_type "yarn" of the model
    config): per-frequency blend of interpolated (theta_i / factor) and
    original frequencies over the correction range of beta_fast = 32,
    beta_slow = 1 rotations, and cos/sin scaled by 0.1 ln(factor) + 1.
    Returns fp32 [seq_len, head_dim / 2] tables holding bf16 values (the model
    hands cos/sin to the rotary op in bf16)."""

    inv_freq, attn_factor = yarn_inv_freq(shape)
    t = torch.arange(seq_len, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    cos = (freqs.cos() * attn_factor).to(torch.bfloat16).to(torch.float32)
    sin = (freqs.sin() * attn_factor).to(torch.bfloat16).to(torch.float32)
    return cos.to(device).contiguous(), sin.to(device).contiguous()


def yarn_inv_freq(shape: DreamShape) -> tuple[torch.Tensor, float]:
    """fp32 YaRN frequencies [head_dim / 2] and the attention factor."""

    dim = shape.head_dim
    base = shape.rope_theta
    factor = shape.yarn_factor
    half = dim // 2
    pos_freqs = base ** (torch.arange(0, dim, 2, dtype=torch.float64) / dim)
    inv_extra = 1.0 / pos_freqs
    if factor == 1.0:
        inv_freq = inv_extra
        attn_factor = 1.0
    else:
        inv_inter = 1.0 / (factor * pos_freqs)

        def correction_dim(rotations):
            return (dim * math.log(shape.yarn_original_max / (rotations * 2 * math.pi))) / (
                2 * math.log(base))

        low = max(math.floor(correction_dim(32.0)), 0)
        high = min(math.ceil(correction_dim(1.0)), dim - 1)
        if low == high:
            high += 0.001
        ramp = ((torch.arange(half, dtype=torch.float64) - low) / (high - low)).clamp(0, 1)
        extra_weight = 1.0 - ramp
        inv_freq = inv_inter * (1 - extra_weight) + inv_extra * extra_weight
        attn_factor = 0.1 * math.log(factor) + 1.0
    return inv_freq.to(torch.float32), attn_factor


def yarn_rotate_fp32(x: torch.Tensor, shape: DreamShape) -> torch.Tensor:
    """x [B, L, heads, D] rotated in fp32 at positions 0..L-1 with fp32 YaRN
    cos/sin (BASELINE configuration 3's input preparation); fp32 result."""

    inv_freq, attn_factor = yarn_inv_freq(shape)
    L, half = x.shape[1], x.shape[-1] // 2
    ang = torch.outer(torch.arange(L, dtype=torch.float32), inv_freq).to(x.device)
    c = (ang.cos() * attn_factor)[None, :, None, :]
    s = (ang.sin() * attn_factor)[None, :, None, :]
    xf = x.float()
    x1, x2 = xf[..., :half], xf[..., half:]
    return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s), dim=-1)


@dataclass
class DreamLayerWeights:
    input_norm: torch.Tensor          # bf16 [hidden]
    qkv_weight: torch.Tensor          # bf16 [(Hq + 2 Hkv) * D, hidden]
    qkv_bias: torch.Tensor            # bf16 [(Hq + 2 Hkv) * D]
    o_weight: torch.Tensor            # bf16 [hidden, Hq * D]
    post_norm: torch.Tensor           # bf16 [hidden]
    gate_up_weight: torch.Tensor      # bf16 [2 * intermediate, hidden]
    down_weight: torch.Tensor         # bf16 [hidden, intermediate]
    qcal_down: torch.Tensor | None = None      # bf16 [rank, hidden]
    qcal_up: torch.Tensor | None = None        # bf16 [Hq * D, rank]
    qcal_norm: torch.Tensor | None = None      # fp32 [D]
    entropy_bias_scale: torch.Tensor | None = None  # fp32 [Hq]


@dataclass
class DreamWeights:
    shape: DreamShape
    embed: torch.Tensor               # bf16 [vocab, hidden]
    lmk_type: torch.Tensor            # bf16 [hidden]
    final_norm: torch.Tensor          # bf16 [hidden]
    lm_head: torch.Tensor             # bf16 [vocab, hidden]
    layers: list[DreamLayerWeights]

    @classmethod
    def random(cls, shape: DreamShape, device, seed: int = 0, std: float = 0.02) -> "DreamWeights":
        """Normal(0, std) matrices (the initializer_range of the config),
        RMSNorm weights near one, Q-Cal as install_qcal draws it
        (qcal.py:40-60), entropy_bias_scale ones (attention.py:737-739)."""

        g = torch.Generator(device=device)
        g.manual_seed(seed)
        H, I, D = shape.hidden, shape.intermediate, shape.head_dim
        P = (shape.q_heads + 2 * shape.kv_heads) * D

        def mat(*size, s=std):
            return torch.empty(*size, dtype=torch.bfloat16, device=device).normal_(0.0, s, generator=g)

        def norm_w(n):
            return (1.0 + 0.1 * torch.randn(n, generator=g, device=device)).to(torch.bfloat16)

        route = set(shape.route_layers())
        layers = []
        for i in range(shape.layers):
            lw = DreamLayerWeights(
                input_norm=norm_w(H), qkv_weight=mat(P, H), qkv_bias=mat(P, s=0.1),
                o_weight=mat(H, shape.q_heads * D), post_norm=norm_w(H),
                gate_up_weight=mat(2 * I, H), down_weight=mat(H, I),
            )
            if i in route:
                lw.qcal_down = mat(shape.qcal_rank, H)
                lw.qcal_up = mat(shape.q_heads * D, shape.qcal_rank)
                lw.qcal_norm = torch.ones(D, dtype=torch.float32, device=device)
                lw.entropy_bias_scale = torch.ones(shape.q_heads, dtype=torch.float32, device=device)
            layers.append(lw)
        return cls(shape=shape, embed=mat(shape.vocab, H), lmk_type=mat(H, s=0.5),
                   final_norm=norm_w(H), lm_head=mat(shape.vocab, H), layers=layers)


def add_rms_norm(x, residual, weight, eps):
    """(bf16(x + residual) or None, RMSNorm of it) on the glue kernel."""

    rows, hidden = x.shape
    out = torch.empty_like(x)
    total = None if residual is None else torch.empty_like(x)
    st = _lib.call("mrsa_add_rms_norm_fwd", _lib.ptr(x), _lib.ptr(residual), _lib.ptr(weight),
                   rows, hidden, float(eps), _lib.ptr(total), _lib.ptr(out), _lib.stream_of(x))
    _lib.check(st, "add_rms_norm")
    return total, out


def rope_qkv(qkv, cos, sin, shape: DreamShape, qcal_delta=None, qcal_norm=None):
    """Split and rotate the fused projection; with qcal_delta also the Q-Cal
    routing query.  Returns (q, k, v, route_q or None) as [1, L, heads, D]."""

    L = qkv.shape[0]
    D = shape.head_dim
    q = torch.empty(1, L, shape.q_heads, D, dtype=torch.bfloat16, device=qkv.device)
    k = torch.empty(1, L, shape.kv_heads, D, dtype=torch.bfloat16, device=qkv.device)
    v = torch.empty_like(k)
    rq = None if qcal_delta is None else torch.empty_like(q)
    st = _lib.call("mrsa_rope_qkv_fwd", _lib.ptr(qkv), _lib.ptr(cos), _lib.ptr(sin),
                   _lib.ptr(qcal_delta), _lib.ptr(qcal_norm), float(shape.qcal_eps), L,
                   shape.q_heads, shape.kv_heads, D, _lib.ptr(q), _lib.ptr(k), _lib.ptr(v),
                   _lib.ptr(rq), _lib.stream_of(qkv))
    _lib.check(st, "rope_qkv")
    return q, k, v, rq


def swiglu(gate_up):
    rows, two_i = gate_up.shape
    out = torch.empty(rows, two_i // 2, dtype=torch.bfloat16, device=gate_up.device)
    st = _lib.call("mrsa_swiglu_fwd", _lib.ptr(gate_up), rows, two_i // 2, _lib.ptr(out),
                   _lib.stream_of(gate_up))
    _lib.check(st, "swiglu")
    return out


def landmark_layout(text_ids: torch.Tensor, shape: DreamShape):
    """The physical sequence of the "mask_type" landmark mode for one
    all-valid document (dream_dllm_hils/data.py:970-1010): every chunk is
    chunk_size - 1 text tokens followed by a landmark slot holding the mask
    token; text tokens are numbered 0, 1, ... in order (landmarks skipped)
    and each landmark takes the position after its chunk's last text token.

    text_ids int64 [1, C * (chunk_size - 1)] -> (input_ids [1, C * chunk_size],
    position_ids int64 [C * chunk_size]) on text_ids' device."""

    S = shape.route.chunk_size
    if text_ids.ndim != 2 or text_ids.shape[0] != 1 or text_ids.shape[1] % (S - 1):
        raise ValueError(f"text_ids must be [1, C * {S - 1}], got {tuple(text_ids.shape)}")
    C = text_ids.shape[1] // (S - 1)
    dev = text_ids.device
    ids = torch.cat([text_ids.reshape(C, S - 1),
                     torch.full((C, 1), shape.mask_token_id, dtype=text_ids.dtype, device=dev)],
                    dim=1).reshape(1, C * S)
    return ids, landmark_positions(C * S, shape, dev)


def landmark_positions(seq_len: int, shape: DreamShape, device) -> torch.Tensor:
    """position_ids of landmark_layout for seq_len physical slots: slot j of
    chunk c holds text position c (S - 1) + j, the landmark (j = S - 1) the
    position after its chunk's last text token (data.py:999-1010)."""

    S = shape.route.chunk_size
    slot = torch.arange(seq_len, device=device)
    return (slot // S) * (S - 1) + slot % S


def rope_tables(position_ids: torch.Tensor, shape: DreamShape):
    """The YaRN tables of yarn_tables, one row per position id."""

    cos, sin = yarn_tables(int(position_ids.max()) + 1, shape, position_ids.device)
    return cos[position_ids].contiguous(), sin[position_ids].contiguous()


def embed_tokens(w: DreamWeights, input_ids: torch.Tensor) -> torch.Tensor:
    """Token embeddings plus the landmark type offset on every chunk's last
    slot, which holds the mask token (the "mask_type" landmark mode,
    train_fulltext.py:2305-2350; ValueError as there when a landmark slot
    holds another token)."""

    S = w.shape.route.chunk_size
    if bool((input_ids.reshape(-1)[S - 1 :: S] != w.shape.mask_token_id).any()):
        raise ValueError("landmark_mask marks positions that are not LMK tokens")
    h = F.embedding(input_ids.reshape(-1), w.embed)
    h[S - 1 :: S] = h[S - 1 :: S] + w.lmk_type
    return h


@torch.no_grad()
def dream_forward(w: DreamWeights, input_ids: torch.Tensor, *, position_ids=None, tables=None,
                  return_hidden: bool = False) -> torch.Tensor:
    """Denoising forward of one sequence: input_ids int64 [1, L] in the
    landmark layout (landmark_layout) -> logits bf16 [L, vocab] (or the final
    normed hidden [L, hidden]).  position_ids default to the layout's
    (landmark_positions); tables = (cos, sin) rows per slot, if precomputed."""

    shape = w.shape
    if input_ids.ndim != 2 or input_ids.shape[0] != 1:
        raise ValueError("dream_forward takes input_ids of shape [1, L]")
    L = input_ids.shape[1]
    if L % shape.route.chunk_size:
        raise ValueError(f"sequence length {L} must be a multiple of {shape.route.chunk_size}")
    if input_ids.device.type != "cuda":
        raise ValueError("dream_forward requires CUDA tensors")
    if tables is None:
        if position_ids is None:
            position_ids = landmark_positions(L, shape, input_ids.device)
        tables = rope_tables(position_ids, shape)
    cos, sin = tables
    route = set(shape.route_layers())
    Hq, D = shape.q_heads, shape.head_dim
    h = embed_tokens(w, input_ids)
    _, x = add_rms_norm(h, None, w.layers[0].input_norm, shape.rms_eps)
    for i, lw in enumerate(w.layers):
        qkv = F.linear(x, lw.qkv_weight, lw.qkv_bias)
        if i in route:
            delta = F.linear(F.linear(x, lw.qcal_down), lw.qcal_up)
            q, k, v, rq = rope_qkv(qkv, cos, sin, shape, delta, lw.qcal_norm)
            a = route_attention(q, k, v, rq, lw.entropy_bias_scale, None, shape.route)
        else:
            q, k, v, _ = rope_qkv(qkv, cos, sin, shape)
            a = swa_attention(q, k, v, None, shape.swa_window, shape.route.chunk_size)
        o = F.linear(a.reshape(L, Hq * D), lw.o_weight)
        h, x = add_rms_norm(o, h, lw.post_norm, shape.rms_eps)
        m = F.linear(swiglu(F.linear(x, lw.gate_up_weight)), lw.down_weight)
        nxt = w.layers[i + 1].input_norm if i + 1 < len(w.layers) else w.final_norm
        h, x = add_rms_norm(m, h, nxt, shape.rms_eps)
    if return_hidden:
        return x
    return F.linear(x, w.lm_head)


def dream_flops(shape: DreamShape, seq_len: int) -> float:
    """Matrix FLOPs of one forward: the projections and lm_head, plus the
    attention products (route layers: local window, pool, routing and the
    routed chunks; SWA layers: the clipped window)."""

    H, I, D = shape.hidden, shape.intermediate, shape.head_dim
    Hq, Hkv = shape.q_heads, shape.kv_heads
    L = seq_len
    per_layer = 2 * L * H * ((Hq + 2 * Hkv) * D + Hq * D + 3 * I)
    n_route = len(shape.route_layers())
    flops = shape.layers * per_layer + n_route * 2 * L * H * shape.qcal_rank * 2
    flops += n_route * 2 * L * shape.qcal_rank * Hq * D
    flops += 2 * L * H * shape.vocab
    S, K, R = shape.route.chunk_size, shape.route.topk, shape.route.local_window
    W = shape.swa_window
    sum_swa = sum(min(L - 1, p + W) - max(0, p - W) + 1 for p in range(0, L, 64)) * 64
    flops += (shape.layers - n_route) * 4 * Hq * D * sum_swa
    route_keys = (2 * (R + S - 1) + 1) + K * S + L // S
    flops += n_route * 4 * Hq * D * L * route_keys
    return float(flops)
