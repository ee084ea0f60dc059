"""CPU restatement of the Dream-7B-shaped denoising forward -- TEST INFRASTRUCTURE.

Only tests/ may import this module, as the checker of mrsa.dream.  The layer
loop follows dream_dllm_hils/fastdllm_v1.py:375-403 (a Qwen2 decoder); the
attention of route layers is mrsa_oracle.route_layer, of the other layers
mrsa_oracle.local_attention (radius ``swa_window``).  Every tensor that the
reference stores in bf16 between ops is rounded to bf16 here at the same
point; arithmetic is fp32.
"""

from __future__ import annotations

import math

import torch

from oracle import mrsa_oracle as O


def yarn_inv_freq(dim, base, factor, original_max, beta_fast=32.0, beta_slow=1.0):
    """YaRN frequencies and attention factor (Peng et al. 2023, section 3:
    "NTK-by-parts" interpolation with the ramp between the dimensions that
    complete beta_fast and beta_slow rotations over the original context,
    plus the sqrt(1/t) = 0.1 ln(s) + 1 attention scale)."""

    theta = base ** (-torch.arange(0, dim, 2, dtype=torch.float64) / dim)
    if factor == 1.0:
        return theta, 1.0

    def dim_of(rot):  # dimension index whose wavelength fits `rot` turns in original_max
        return dim * math.log(original_max / (rot * 2 * math.pi)) / (2 * math.log(base))

    lo = max(math.floor(dim_of(beta_fast)), 0)
    hi = min(math.ceil(dim_of(beta_slow)), dim - 1)
    if lo == hi:
        hi += 0.001
    gamma = 1.0 - ((torch.arange(dim // 2, dtype=torch.float64) - lo) / (hi - lo)).clamp(0, 1)
    inv = theta / factor * (1 - gamma) + theta * gamma
    return inv, 0.1 * math.log(factor) + 1.0


def yarn_tables(seq_len, dim, base, factor, original_max):
    inv, af = yarn_inv_freq(dim, base, factor, original_max)
    freqs = torch.outer(torch.arange(seq_len, dtype=torch.float32), inv.to(torch.float32))
    cos = O.bf16_round(freqs.cos() * af)
    sin = O.bf16_round(freqs.sin() * af)
    return cos, sin


def rms_norm(x, weight, eps):
    """Qwen2RMSNorm: bf16(weight * bf16(x * rsqrt(mean(x^2) + eps)))."""

    xf = x.float()
    n = O.bf16_round(xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps))
    return (weight.float() * n).to(torch.bfloat16)


def rope(x, cos, sin):
    """x [L, heads, D] bf16 rotated with fp32 cos/sin [L, D/2] (the fp32 form of
    ops/rope_tilelang_fp32.py:19-94); one bf16 rounding."""

    xf = x.float()
    h = xf.shape[-1] // 2
    x1, x2 = xf[..., :h], xf[..., h:]
    c, s = cos[:, None, :], sin[:, None, :]
    return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s), dim=-1).to(torch.bfloat16)


def qcal_route_q(q_unrot, delta, norm_weight, cos, sin, eps):
    """attention.py:477-502 and qcal.py:22-26: rope(rms_norm(q + delta) * w)."""

    comb = (q_unrot.float() + delta.float()).to(torch.bfloat16).float()
    n = comb * torch.rsqrt(comb.square().mean(-1, keepdim=True) + eps)
    return rope((norm_weight.float() * n).to(torch.bfloat16), cos, sin)


def swiglu(gate_up):
    i = gate_up.shape[-1] // 2
    g, u = gate_up[..., :i].float(), gate_up[..., i:].float()
    return (O.bf16_round(g * torch.sigmoid(g)) * u).to(torch.bfloat16)


def linear(x, w, b=None):
    y = x.float() @ w.float().t()
    if b is not None:
        y = y + b.float()
    return y.to(torch.bfloat16)


def landmark_positions(seq_len, chunk_size):
    """position_ids of the "mask_type" landmark layout of one all-valid
    document (dream_dllm_hils/data.py:999-1010): text slots numbered in
    order with landmarks skipped; a landmark takes the position after its
    chunk's last text token."""

    pos = torch.zeros(seq_len, dtype=torch.long)
    nxt = 0
    for j in range(seq_len):
        if (j + 1) % chunk_size:
            pos[j] = nxt
            nxt += 1
        else:
            pos[j] = pos[j - 1] + 1
    return pos


def dream_forward(w, input_ids, return_hidden=False, position_ids=None):
    """w: mrsa.dream.DreamWeights with every tensor on the CPU; input_ids in
    the landmark layout (every chunk's last slot holds the mask token)."""

    s = w.shape
    L = input_ids.shape[1]
    S = s.route.chunk_size
    D, Hq, Hkv = s.head_dim, s.q_heads, s.kv_heads
    pos = landmark_positions(L, S) if position_ids is None else position_ids.long().cpu()
    cos, sin = yarn_tables(int(pos.max()) + 1, D, s.rope_theta, s.yarn_factor,
                           s.yarn_original_max)
    cos, sin = cos[pos], sin[pos]
    assert bool((input_ids.reshape(-1)[S - 1 :: S] == s.mask_token_id).all())
    h = w.embed[input_ids.reshape(-1)].clone()
    h[S - 1 :: S] = (h[S - 1 :: S].float() + w.lmk_type.float()).to(torch.bfloat16)
    route = set(s.route_layers())
    for i, lw in enumerate(w.layers):
        x = rms_norm(h, lw.input_norm, s.rms_eps)
        qkv = linear(x, lw.qkv_weight, lw.qkv_bias)
        qp = qkv[:, : Hq * D].reshape(L, Hq, D)
        kp = qkv[:, Hq * D : (Hq + Hkv) * D].reshape(L, Hkv, D)
        v = qkv[:, (Hq + Hkv) * D :].reshape(1, L, Hkv, D)
        q = rope(qp, cos, sin)[None]
        k = rope(kp, cos, sin)[None]
        if i in route:
            delta = linear(linear(x, lw.qcal_down), lw.qcal_up).reshape(L, Hq, D)
            rq = qcal_route_q(qp, delta, lw.qcal_norm, cos, sin, s.qcal_eps)[None]
            r = s.route
            a, _ = O.route_layer(q, k, v, rq, lw.entropy_bias_scale, None,
                                 local_window=r.local_window, chunk_size=S, topk=r.topk,
                                 temperature=r.temperature, gate_offset=r.gate_offset,
                                 gate_scale=r.gate_scale, skip_inert_slots=r.skip_inert_slots)
        else:
            a, _ = O.local_attention(q, k, v, None, s.swa_window, 0)
            a = a.to(torch.bfloat16)
        o = linear(a.reshape(L, Hq * D), lw.o_weight)
        h = (h.float() + o.float()).to(torch.bfloat16)
        x = rms_norm(h, lw.post_norm, s.rms_eps)
        m = linear(swiglu(linear(x, lw.gate_up_weight)), lw.down_weight)
        h = (h.float() + m.float()).to(torch.bfloat16)
    x = rms_norm(h, w.final_norm, s.rms_eps)
    if return_hidden:
        return x
    return linear(x, w.lm_head)
