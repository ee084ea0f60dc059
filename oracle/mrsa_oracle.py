"""CPU fp32 restatement of the MRSA route-layer forward -- TEST INFRASTRUCTURE.

This module is the parity oracle.  Only tests/, __graft_entry__.smoke() and
bench.py's CPU-baseline leg may import it, and only as the checker (or as the
timed CPU baseline).  The product path (the ``mrsa`` package) never calls it.

Every function restates one stage of the reference
(NRHLYM/Mask-Routed-Sparse-Attention-for-Long-Context-Diffusion-Language-Models)
in plain torch on the CPU, in fp32, at the bf16 rounding points the reference
has between stages.  Citations are file:line in that repository.

Conventions: bf16 tensors in, fp32 math; functions return fp32 unless noted.
Ties in the route selection are broken toward the lower chunk index (the rule
of the reference's fused selection kernel, ops/topk_head_softmax.py:614-626;
its torch path uses torch.topk, whose tie order is implementation-defined).
"""

from __future__ import annotations

import math
from typing import Optional

import torch

NEG_INF = float("-inf")


def bf16_round(x: torch.Tensor) -> torch.Tensor:
    """Round to bf16 (nearest-even) and widen back to fp32."""

    return x.to(torch.bfloat16).to(torch.float32)


# ---------------------------------------------------------------------------
# a4: landmark pool
# ---------------------------------------------------------------------------
def chunk_attn_pool(mu_q, k_chunked, key_valid, sm_scale=None, *, dense=None):
    """Landmark keys and entropy of ops/chunk_attn_pool_gqa_tilelang.py.

    mu_q [B, C, Hkv, G, D], k_chunked [B, C, S, Hkv, D], key_valid [B, C, S].
    dense=None picks what chunk_attn_pool_gqa dispatches to: the compiled torch
    twin _compact_pool_torch (:17-37) for G == 1, else the fused kernel
    semantics of _pool_gqa_fwd (:47-180):
      * chunk valid iff any of its first S-1 keys is valid (:94-99);
      * masked slot -> -inf, except slot 0 -> logit 0 (:118-129);
      * pooling uses the probabilities rounded to bf16 (:151-158);
      * entropy from the fp32 probabilities (:142-149);
      * invalid chunk -> zero key and zero entropy (:161-178).
    Returns (landmark_keys fp32 before the final bf16 rounding, entropy fp32).
    """

    B, C, H, G, D = mu_q.shape
    S = k_chunked.shape[2]
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    if dense is None:
        dense = G == 1
    q = mu_q.float()
    k = k_chunked.float()
    real = key_valid.bool().clone()
    real[..., -1] = False
    logits = torch.einsum("bchgd,bcshd->bchgs", q, k) * sm_scale
    if dense:
        logits = logits.masked_fill(~real[:, :, None, None, :], NEG_INF)
        probs = torch.nan_to_num(torch.softmax(logits, dim=-1), nan=0.0)
        chunk_ok = torch.ones(B, C, dtype=torch.bool)
        p_pool = probs
    else:
        chunk_ok = real.any(dim=-1)
        ok = real & chunk_ok[..., None]
        fill = torch.full((S,), NEG_INF)
        fill[0] = 0.0
        logits = torch.where(ok[:, :, None, None, :], logits, fill)
        probs = torch.softmax(logits, dim=-1)
        p_pool = bf16_round(probs)
    lmk = torch.einsum("bchgs,bcshd->bchgd", p_pool, k)
    logp = torch.where(probs > 0, probs.clamp_min(1e-30).log(), torch.zeros_like(probs))
    entropy = -(probs * logp).sum(dim=-1)
    zero = ~chunk_ok[:, :, None, None]
    lmk = lmk.masked_fill(zero[..., None], 0.0)
    entropy = entropy.masked_fill(zero, 0.0)
    return lmk, entropy


def chunk_attn_pool_bwd(mu_q, k_chunked, key_valid, grad_lmk, grad_entropy, sm_scale=None):
    """Backward of the fused pool kernel, _pool_gqa_bwd
    (ops/chunk_attn_pool_gqa_tilelang.py:183-325), as _ChunkAttnPoolGQA.backward
    (:355-394) runs it for groups > 1.  Returns (d_mu_q, d_k_chunked) in bf16.

    The kernel's rounding points are kept: the saved probabilities are zero
    for an invalid chunk (:164-169) and enter as bf16 (:241-246); the logit
    gradient p * ((dP - sum p dP) - g_H * (ln p + H)) (:264-283) is rounded to
    bf16 after the sm_scale factor; d_mu and d_k are bf16 roundings of fp32
    sums (:286-312).  Like the kernel, a masked slot 0 (whose logit is the
    constant 0) still receives the logit gradient.  For groups == 1 the
    reference differentiates _compact_pool_torch instead: autograd of
    chunk_attn_pool(..., dense=True) is that backward.
    """

    B, C, H, G, D = mu_q.shape
    S = k_chunked.shape[2]
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    q = mu_q.float()
    k = k_chunked.float()
    real = key_valid.bool().clone()
    real[..., -1] = False
    chunk_ok = real.any(dim=-1)
    ok = real & chunk_ok[..., None]
    fill = torch.full((S,), NEG_INF)
    fill[0] = 0.0
    logits = torch.einsum("bchgd,bcshd->bchgs", q, k) * sm_scale
    probs = torch.softmax(torch.where(ok[:, :, None, None, :], logits, fill), dim=-1)
    logp = torch.where(probs > 0, probs.clamp_min(1e-30).log(), torch.zeros_like(probs))
    entropy = (-(probs * logp).sum(dim=-1)).masked_fill(~chunk_ok[:, :, None, None], 0.0)
    pb = bf16_round(probs.masked_fill(~chunk_ok[:, :, None, None, None], 0.0))
    gk = (torch.zeros_like(q) if grad_lmk is None else grad_lmk).bfloat16().float()
    gb = torch.zeros(B, C, H, G) if grad_entropy is None else grad_entropy.float()
    dP = torch.einsum("bchgd,bcshd->bchgs", gk, k)
    delta = (pb * dP).sum(dim=-1, keepdim=True)
    lpb = torch.where(pb > 0, pb.clamp_min(1e-30).log(), torch.zeros_like(pb))
    dlogit = torch.where(
        pb > 0, pb * ((dP - delta) - gb[..., None] * (lpb + entropy[..., None])),
        torch.zeros_like(pb))
    dl = bf16_round(dlogit * sm_scale)
    d_mu = torch.einsum("bchgs,bcshd->bchgd", dl, k)
    d_k = torch.einsum("bchgs,bchgd->bcshd", dl, q) + torch.einsum("bchgs,bchgd->bcshd", pb, gk)
    return d_mu.bfloat16(), d_k.bfloat16()


# ---------------------------------------------------------------------------
# a1: drop mask
# ---------------------------------------------------------------------------
def chunk_aligned_local_bounds(seq_len, window, chunk_size):
    """dream_dllm_hils/kernel_utils.py:75-99."""

    pos = torch.arange(seq_len)
    left = (pos - window).clamp_min(0).div(chunk_size, rounding_mode="floor") * chunk_size
    right = ((pos + window).clamp_max(seq_len - 1).div(chunk_size, rounding_mode="floor") + 1) * chunk_size
    return left, right.clamp_max(seq_len)


def remote_drop_mask(valid_mask, window, chunk_size, allowed_mask=None):
    """dream_dllm_hils/kernel_utils.py:102-161; int32 [B, L, L/S]."""

    B, L = valid_mask.shape
    C = L // chunk_size
    pos = torch.arange(L)
    real = (pos + 1).remainder(chunk_size) != 0
    chunk_valid = (valid_mask.bool() & real[None]).reshape(B, C, chunk_size).any(-1)
    left, right = chunk_aligned_local_bounds(L, window, chunk_size)
    lc = left.div(chunk_size, rounding_mode="floor")
    rc = (right - 1).div(chunk_size, rounding_mode="floor")
    ids = torch.arange(C)
    local = (ids[None, :] >= lc[:, None]) & (ids[None, :] <= rc[:, None])
    drop = local[None] | ~chunk_valid[:, None, :]
    if allowed_mask is not None:
        lmk_pos = torch.arange(chunk_size - 1, L, chunk_size)
        drop = drop | ~allowed_mask.bool().index_select(-1, lmk_pos)
    return drop.to(torch.int32)


def remote_drop_mask_rows(valid_mask, window, chunk_size, positions):
    """Rows ``positions`` of remote_drop_mask (kernel_utils.py:102-161, no
    allowed mask), built without the full [B, L, L/S] mask: the cached block
    step reads only its query rows (fastdllm_attention.py:295-299).
    int32 [B, len(positions), L/S]."""

    B, L = valid_mask.shape
    C = L // chunk_size
    pos = torch.as_tensor(positions).long()
    real = (torch.arange(L) + 1).remainder(chunk_size) != 0
    chunk_valid = (valid_mask.bool() & real[None]).reshape(B, C, chunk_size).any(-1)
    left = (pos - window).clamp_min(0).div(chunk_size, rounding_mode="floor")
    right = (pos + window).clamp_max(L - 1).div(chunk_size, rounding_mode="floor")
    ids = torch.arange(C)
    local = (ids[None, :] >= left[:, None]) & (ids[None, :] <= right[:, None])
    return (local[None] | ~chunk_valid[:, None, :]).to(torch.int32)


# ---------------------------------------------------------------------------
# a5: route scoring + top-k
# ---------------------------------------------------------------------------
def route_topk(q5, lmks, lse4, topk, block_size, *, drop_mask=None, bias4=None,
               selection_mode="post_softmax", is_causal=False, window_size=0, q_offset=0,
               query_block=512, gumbel_noise=None):
    """ref_softmax_topk_max_pooling (ops/topk_head_softmax.py:15-156).

    q5 [B, L, Hkv, G, D]; lmks [B, C, Hkv*G, D] or [B, C, Hkv, D];
    lse4 [B, L, Hkv, G]; bias4 [B, C, Hkv, G]; drop_mask [B, L, C];
    gumbel_noise [1, 1, Hkv * G, C], added after the bias to the selection
    logits and the route LSE (:99-105).
    Returns indices [B, L, Hkv, topk] int64 (ascending, -1 last), scores
    [B, L, Hkv, G, topk] fp32 (raw scaled q.k at the picks, -inf at -1) and
    the selection scores [B, L, Hkv, C] (max over G after the drop mask) used
    to find near ties.
    """

    B, L, H, G, D = q5.shape
    C = lmks.shape[1]
    per_head = lmks.shape[2] == H * G
    lm = lmks.float().reshape(B, C, H, G, D) if per_head else lmks.float()
    scale = 1.0 / math.sqrt(D)
    idx_out = torch.empty(B, L, H, topk, dtype=torch.int64)
    sc_out = torch.empty(B, L, H, G, topk)
    sel_out = torch.empty(B, L, H, C)
    kk = min(topk, C)
    for l0 in range(0, L, query_block):
        l1 = min(L, l0 + query_block)
        q = q5[:, l0:l1].float()
        if per_head:
            logits = torch.einsum("blhgd,bchgd->blhgc", q, lm)
        else:
            logits = torch.einsum("blhgd,bchd->blhgc", q, lm)
        logits = logits * scale
        if is_causal:
            i = torch.arange(l0, l1)[:, None] + q_offset
            j = torch.arange(C)[None, :]
            thr = (i - window_size + 1).div(block_size, rounding_mode="floor") if window_size > 0 \
                else i.div(block_size, rounding_mode="floor")
            cm = (j >= thr).view(1, l1 - l0, 1, 1, C)
            logits = logits.masked_fill(cm, NEG_INF)
        x = logits
        if bias4 is not None:
            x = x + bias4.float().permute(0, 2, 3, 1)[:, None]
        if gumbel_noise is not None:
            x = x + gumbel_noise.float().reshape(1, 1, H, G, C)
        if selection_mode == "pre_softmax":
            y = x
        else:
            lse_h = torch.logsumexp(x, dim=-1)
            tot = torch.logaddexp(lse4[:, l0:l1].float(), lse_h)
            y = x - tot[..., None]
        sel = y.max(dim=3).values
        if drop_mask is not None:
            sel = sel.masked_fill(drop_mask[:, l0:l1].bool()[:, :, None, :], NEG_INF)
        sel_out[:, l0:l1] = sel
        order = torch.sort(sel, dim=-1, descending=True, stable=True).indices[..., :kk]
        topv = torch.gather(sel, -1, order)
        order = order.masked_fill(topv == NEG_INF, -1)
        if kk < topk:
            pad = torch.full((*order.shape[:-1], topk - kk), -1, dtype=order.dtype)
            order = torch.cat([order, pad], dim=-1)
        key = order.masked_fill(order < 0, C + 1000)
        idx = torch.sort(key, dim=-1).values
        idx = idx.masked_fill(idx >= C, -1)
        safe = idx.clamp_min(0)[:, :, :, None, :].expand(-1, -1, -1, G, -1)
        sc = torch.gather(logits, -1, safe)
        sc = sc.masked_fill(idx[:, :, :, None, :] < 0, NEG_INF)
        idx_out[:, l0:l1] = idx
        sc_out[:, l0:l1] = sc
    return idx_out, sc_out, sel_out


def boundary_gap(sel, topk):
    """Gap between the topk-th and (topk+1)-th selection scores per row (inf if undefined)."""

    vals = torch.sort(sel, dim=-1, descending=True).values
    if vals.shape[-1] <= topk:
        return torch.full(vals.shape[:-1], float("inf"))
    a = vals[..., topk - 1]
    b = vals[..., topk]
    gap = a - b
    return torch.where(torch.isfinite(a) & torch.isfinite(b), gap, torch.full_like(gap, float("inf")))


def route_score_bwd(q5, lmks, indices, grad_scores, sm_scale=None):
    """SoftmaxTopKMaxPoolingFusedFn.backward (ops/topk_head_softmax.py:1074-1122).

    q5 [B, L, Hkv, G, D]; lmks [B, C, Hkv*G, D] (per head) or [B, C, Hkv, D]
    (shared); indices [B, L, Hkv, K]; grad_scores [B, L, Hkv, G, K].  The
    gradient times sm_scale is rounded to bf16 (the reference's mul_ in the
    bf16 gradient dtype, :1090-1091) and scattered into a dense [L, C] matrix
    per (h, g); slots outside [0, C) are zeroed (:1084-1092).  Returns fp32
    grad_q (bmm with the landmarks, :1107-1108) and grad_lmks (bmm with q,
    :1110-1121; summed over g for shared landmarks).
    """

    B, L, H, G, D = q5.shape
    C = lmks.shape[1]
    K = indices.shape[-1]
    per_head = lmks.shape[2] == H * G
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    idx = indices.long()[:, :, :, None, :].expand(B, L, H, G, K)
    valid = (idx >= 0) & (idx < C)
    val = bf16_round(grad_scores.float().reshape(B, L, H, G, K) * sm_scale)
    val = torch.where(valid, val, torch.zeros_like(val))
    dense = torch.zeros(B, L, H, G, C)
    # Valid slots of one list hold distinct chunks in the reference's
    # forward, so the scatter is a plain sum over the slots.
    dense.scatter_add_(4, idx.clamp(0, C - 1), val)
    q = q5.float()
    if per_head:
        lm = lmks.float().reshape(B, C, H, G, D)
        grad_q = torch.einsum("blhgc,bchgd->blhgd", dense, lm)
        grad_l = torch.einsum("blhgc,blhgd->bchgd", dense, q).reshape(B, C, H * G, D)
    else:
        lm = lmks.float()
        grad_q = torch.einsum("blhgc,bchd->blhgd", dense, lm)
        grad_l = torch.einsum("blhgc,blhgd->bchd", dense, q)
    return grad_q, grad_l


# ---------------------------------------------------------------------------
# a7: route weights
# ---------------------------------------------------------------------------
def route_weights(scores, indices, prior_bias, local_lse, *, temperature=1.0,
                  gate_offset=None, gate_scale=None, return_gate_logit=False,
                  value_bonus=None, selected_gumbel=None):
    """_route_weights_torch (dream_dllm_hils/attention.py:126-235), fp32 outputs.

    value_bonus and selected_gumbel ([B, L, Hq, K], optional) are added to the
    remote logits after the bias, in that order (:172-181).

    scores [B, L, Hq, K] (bf16 values), indices [B, L, Hkv, K], prior_bias
    [B, C, Hkv, G], local_lse [B, L, Hq].  Returns (remote [B, L, Hq, K],
    local [B, L, Hq]) before the bf16 rounding, plus the fp32 gate logit
    [B, L, Hq] with return_gate_logit (:196-235: lse of the remote logits
    minus the local logit, affine-transformed in the gate form, 0 where every
    logit is masked).  Differentiable: gate_offset and gate_scale may be 0-d
    tensors, whose gradients autograd then forms (the reference's own
    backward for this function is its autograd).
    """

    def gate_value(x):
        return x.float().reshape(()) if isinstance(x, torch.Tensor) else float(x)

    B, L, Hq, K = scores.shape
    _, C, Hkv, G = prior_bias.shape
    idx = indices.long().repeat_interleave(G, dim=2)
    valid = (idx >= 0) & (idx < C)
    safe = idx.clamp(0, C - 1)
    bias_by_head = prior_bias.float().reshape(B, C, Hq).permute(0, 2, 1)
    sel_bias = torch.gather(bias_by_head[:, None].expand(B, L, Hq, C), -1, safe)
    remote_logits = scores.float() + sel_bias
    if value_bonus is not None:
        remote_logits = remote_logits + value_bonus.float()
    if selected_gumbel is not None:
        remote_logits = remote_logits + selected_gumbel.float()
    remote_logits = remote_logits.masked_fill(~valid, NEG_INF)
    local_logits = local_lse.float()[..., None]
    affine = gate_scale is not None
    if gate_offset is not None and not affine:
        local_logits = local_logits - gate_value(gate_offset)
    logits = torch.cat((remote_logits, local_logits), dim=-1) / float(temperature)
    all_masked = torch.isneginf(logits).all(dim=-1, keepdim=True)
    logits = torch.where(all_masked, torch.zeros_like(logits), logits)
    remote_lse = torch.logsumexp(logits[..., :K], dim=-1)
    gate = remote_lse - logits[..., K]
    if affine:
        gate = gate_value(gate_scale) * gate + (
            gate_value(gate_offset) if gate_offset is not None else 0.0)
    gate_logit = torch.where(all_masked[..., 0], torch.zeros_like(gate), gate)
    if affine:
        mass = torch.sigmoid(gate)
        internal = torch.softmax(remote_logits / float(temperature), dim=-1)
        internal = torch.where((~valid).all(dim=-1, keepdim=True), torch.zeros_like(internal), internal)
        remote = internal * mass[..., None]
        local = 1.0 - mass
        remote = torch.where(all_masked, torch.zeros_like(remote), remote)
        local = torch.where(all_masked[..., 0], torch.zeros_like(local), local)
        return (remote, local, gate_logit) if return_gate_logit else (remote, local)
    probs = torch.softmax(logits, dim=-1)
    probs = torch.where(all_masked, torch.zeros_like(probs), probs)
    if return_gate_logit:
        return probs[..., :K], probs[..., K], gate_logit
    return probs[..., :K], probs[..., K]


# ---------------------------------------------------------------------------
# a2 / a3: window attention
# ---------------------------------------------------------------------------
def local_attention(q, k, v, key_valid, window, inert_chunk=0, query_positions=None,
                    query_block=256):
    """Window attention with the zero-K/V inert rule (local_attention.py:35-107).

    Key j visible to the query at position p iff |p - j| <= window; keys that
    fail key_valid (and landmark slots when inert_chunk > 0) have K = V = 0.
    Returns (out fp32 [B, Lq, Hq, D], lse fp32 [B, Lq, Hq]).
    """

    B, Lq, Hq, D = q.shape
    Lk, Hkv = k.shape[1], k.shape[2]
    G = Hq // Hkv
    scale = D ** -0.5
    valid = torch.ones(B, Lk, dtype=torch.bool) if key_valid is None else key_valid.bool().clone()
    if inert_chunk > 0:
        valid &= ((torch.arange(Lk) + 1) % inert_chunk != 0)[None]
    kz = k.float() * valid[:, :, None, None]
    vz = v.float() * valid[:, :, None, None]
    pos = torch.arange(Lq) if query_positions is None else query_positions.long().cpu()
    out = torch.zeros(B, Lq, Hq, D)
    lse = torch.zeros(B, Lq, Hq)
    for i0 in range(0, Lq, query_block):
        i1 = min(Lq, i0 + query_block)
        p = pos[i0:i1]
        lo = max(int(p.min()) - window, 0)
        hi = min(int(p.max()) + window + 1, Lk)
        if hi <= lo:
            lse[:, i0:i1] = NEG_INF
            continue
        qb = q[:, i0:i1].float().reshape(B, i1 - i0, Hkv, G, D)
        s = torch.einsum("bqhgd,bkhd->bqhgk", qb, kz[:, lo:hi]) * scale
        j = torch.arange(lo, hi)
        vis = (j[None, :] - p[:, None]).abs() <= window
        s = s.masked_fill(~vis[None, :, None, None, :], NEG_INF)
        l = torch.logsumexp(s, dim=-1)
        pr = torch.softmax(s, dim=-1)
        o = torch.einsum("bqhgk,bkhd->bqhgd", pr, vz[:, lo:hi])
        out[:, i0:i1] = o.reshape(B, i1 - i0, Hq, D)
        lse[:, i0:i1] = l.reshape(B, i1 - i0, Hq)
    return out, lse


# ---------------------------------------------------------------------------
# a8: routed chunk attention
# ---------------------------------------------------------------------------
def selected_attention(q, k, v, weights, indices, key_valid, chunk_size=64,
                       mask_last_token=True, query_block=256, token_keep=None, slope=None):
    """Weighted sum of per-chunk softmax attentions.

    Formula of the reference test test_hils_non_power_two_topk.py:122-138 and
    hils_torch_ref (ops/hils_fwd_bwd_head.py:21-93), with the kernel's key_valid
    masking (:479-486) and index-list reading (:352-361: a list ends at its
    first negative entry).  Entries >= kv_len / chunk_size are skipped.
    q [B, Lq, Hq, D], k/v [B, Lk, Hkv, D], weights [B, Lq, Hq, K],
    indices [B, Lq, Hkv, K].  token_keep [B, Lq, Hkv, K, S] (nonzero = keep)
    additionally masks the keys of slot k of each query (:457-486, the
    TokenKeep[b, q, h, slot, key] term).  slope [Hq] adds the ALiBi bias
    -slope[head] * max(0, (S - 2) - s) to the raw logit of chunk key s before
    the scale (hils_torch_ref :68-76).  Returns fp32 [B, Lq, Hq, D].
    """

    B, Lq, Hq, D = q.shape
    Lk, Hkv = k.shape[1], k.shape[2]
    G = Hq // Hkv
    S = chunk_size
    C = Lk // S
    K = indices.shape[-1]
    scale = 1.0 / math.sqrt(D)
    kc = k.float().reshape(B, C, S, Hkv, D)
    vc = v.float().reshape(B, C, S, Hkv, D)
    allowed = torch.ones(B, C, S, dtype=torch.bool) if key_valid is None else \
        key_valid.bool().reshape(B, C, S).clone()
    if mask_last_token:
        allowed[..., -1] = False
    idx = indices.long()
    neg = idx < 0
    before_neg = torch.cumsum(neg.int(), dim=-1) == 0
    ok = before_neg & (idx >= 0) & (idx < C)
    safe = idx.clamp(0, C - 1)
    alibi = None
    if slope is not None:
        dist = ((S - 2) - torch.arange(S, dtype=torch.float32)).clamp(min=0)
        alibi = -slope.float().reshape(Hkv, G)[:, :, None] * dist        # [Hkv, G, S]
    out = torch.zeros(B, Lq, Hq, D)
    bidx = torch.arange(B)[:, None, None]
    hidx = torch.arange(Hkv)[None, None, :]
    for i0 in range(0, Lq, query_block):
        i1 = min(Lq, i0 + query_block)
        qb = q[:, i0:i1].float().reshape(B, i1 - i0, Hkv, G, D)
        wb = weights[:, i0:i1].float().reshape(B, i1 - i0, Hkv, G, K)
        acc = torch.zeros(B, i1 - i0, Hkv, G, D)
        for kk in range(K):
            c = safe[:, i0:i1, :, kk]                       # [B, l, Hkv]
            kg = kc[bidx, c, :, hidx]                       # [B, l, Hkv, S, D]
            vg = vc[bidx, c, :, hidx]
            al = allowed[bidx, c]                           # [B, l, Hkv, S]
            if token_keep is not None:
                al = al & (token_keep[:, i0:i1, :, kk] != 0)
            s = torch.einsum("blhgd,blhsd->blhgs", qb, kg)
            if alibi is not None:
                s = s + alibi
            s = s * scale
            s = s.masked_fill(~al[:, :, :, None, :], NEG_INF)
            p = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0)
            o = torch.einsum("blhgs,blhsd->blhgd", p, vg)
            w = wb[..., kk] * ok[:, i0:i1, :, kk][..., None].float()
            acc += o * w[..., None]
        out[:, i0:i1] = acc.reshape(B, i1 - i0, Hq, D)
    return out


# ---------------------------------------------------------------------------
# a9: fusion
# ---------------------------------------------------------------------------
def fuse_outputs(remote_output, local_output, local_weight):
    """ops/hils_bidir_output_fusion_tilelang.py:28-35; returns bf16."""

    r = remote_output.float()
    lw = local_weight.float()[..., None]
    lo = local_output.float()
    return (r + lw * lo).to(torch.bfloat16)


# ---------------------------------------------------------------------------
# a6: candidate token scores
# ---------------------------------------------------------------------------
def select_global_token_keep(scores, token_budget):
    """select_global_token_keep (dream_dllm_hils/token_refinement.py:112-148)
    without training noise: in each (b, l, h) row the min(budget, K * S)
    largest of the flattened [K * S] scores are kept when finite.  Ties at the
    threshold go to the lower flat index (the reference's torch.topk
    (sorted=False) leaves their order to the device).  uint8 [B, L, Hkv, K, S].
    """

    B, L, H, K, S = scores.shape
    flat = scores.float().reshape(B, L, H, K * S)
    budget = min(int(token_budget), K * S)
    order = torch.sort(flat, dim=-1, descending=True, stable=True).indices[..., :budget]
    picked = torch.gather(flat, -1, order)
    keep = torch.zeros(B, L, H, K * S, dtype=torch.uint8)
    keep.scatter_(-1, order, torch.isfinite(picked).to(torch.uint8))
    return keep.reshape(B, L, H, K, S)


def candidate_token_scores(q, k, indices, key_valid, chunk_size):
    """candidate_token_scores_reference (dream_dllm_hils/token_refinement.py:10-92)."""

    B, Lq, Hq, D = q.shape
    Lk, Hkv = k.shape[1], k.shape[2]
    G = Hq // Hkv
    C = Lk // chunk_size
    K = indices.shape[-1]
    kc = k.float().reshape(B, C, chunk_size, Hkv, D)
    idx = indices.long()
    safe = idx.clamp(0, max(C - 1, 0))
    bidx = torch.arange(B)[:, None, None, None]
    hidx = torch.arange(Hkv)[None, None, :, None]
    kg = kc[bidx, safe, :, hidx]                           # [B, Lq, Hkv, K, S, D]
    qg = q.float().reshape(B, Lq, Hkv, G, D)
    s = torch.einsum("blhgd,blhksd->blhkgs", qg, kg).amax(dim=-2) / math.sqrt(D)
    valid_chunk = (idx >= 0) & (idx < C)
    kv = torch.ones(B, Lk, dtype=torch.bool) if key_valid is None else key_valid.bool()
    sel_valid = kv.reshape(B, C, chunk_size)[torch.arange(B)[:, None, None, None], safe]
    sel_valid = sel_valid & valid_chunk[..., None]
    sel_valid[..., -1] = False
    return s.masked_fill(~sel_valid, NEG_INF)


def gather_selected_chunk_entropy(entropy, indices):
    """gather_selected_chunk_entropy (dream_dllm_hils/token_refinement.py:244-284):
    the group mean of entropy [B, C, Hkv, G] at each routed chunk (indices
    clamped to [0, C - 1]), 0 where the index is negative.  [B, L, Hkv, K]."""

    B, C, H, G = entropy.shape
    idx = indices.long()
    safe = idx.clamp(0, max(C - 1, 0))
    ent = entropy.float()
    bi = torch.arange(B)[:, None, None, None]
    hi = torch.arange(H)[None, None, :, None]
    gathered = ent[bi, safe, hi].mean(dim=-1)  # [B, L, H, K]
    return gathered.masked_fill(idx < 0, 0.0)


def allocate_entropy_token_budget(entropy, capacity, token_budget, min_tokens_per_chunk=1):
    """allocate_entropy_token_budget (dream_dllm_hils/token_refinement.py:150-241):
    min(sum capacity, token_budget) token slots per row over the last
    dimension: baseline min(capacity, min_tokens_per_chunk), then K + 1
    rounds of capped largest-remainder apportionment by the effective
    support exp(clamp(entropy, 0, ln budget)) (0 for empty chunks); ties in
    the fractional parts go to the lower chunk (stable sort).  int64."""

    capacity = capacity.long()
    K = capacity.shape[-1]
    target = capacity.sum(dim=-1).clamp_max(token_budget)
    alloc = torch.minimum(capacity, torch.full_like(capacity, min_tokens_per_chunk))
    remaining = target - alloc.sum(dim=-1)
    max_entropy = math.log(max(token_budget, 1))
    support = torch.exp(torch.nan_to_num(entropy.float(), nan=0.0, posinf=max_entropy,
                                         neginf=0.0).clamp(min=0.0, max=max_entropy))
    support = support.masked_fill(capacity <= 0, 0.0)
    rank = torch.arange(K).view(*([1] * (capacity.ndim - 1)), K)
    for _ in range(K + 1):
        active = alloc < capacity
        act_sup = support * active
        den = act_sup.sum(dim=-1, keepdim=True)
        quota = torch.where(den > 0, remaining[..., None].float() * act_sup / den.clamp_min(1e-12),
                            torch.zeros_like(act_sup))
        alloc = alloc + torch.minimum(torch.floor(quota).long(), capacity - alloc)
        remaining = target - alloc.sum(dim=-1)
        active = alloc < capacity
        bonus_count = torch.minimum(remaining, active.sum(dim=-1))
        frac = (quota - torch.floor(quota)).masked_fill(~active, float("-inf"))
        order = torch.argsort(frac, dim=-1, descending=True, stable=True)
        bonus = torch.zeros_like(alloc)
        bonus.scatter_(-1, order, (rank < bonus_count[..., None]).long())
        alloc = torch.minimum(alloc + bonus, capacity)
        remaining = target - alloc.sum(dim=-1)
    return alloc


def select_entropy_adaptive_token_keep(scores, selected_entropy, token_budget,
                                       min_tokens_per_chunk=1):
    """select_entropy_adaptive_token_keep (dream_dllm_hils/token_refinement.py:
    287-333) without training noise: per chunk, the allocation's largest
    finite scores (stable descending order: ties to the lower key).
    Returns (keep uint8 [B, L, H, K, S], allocation int64 [B, L, H, K])."""

    sc = scores.float()
    capacity = torch.isfinite(sc).sum(dim=-1)
    alloc = allocate_entropy_token_budget(selected_entropy, capacity, token_budget,
                                          min_tokens_per_chunk)
    order = torch.argsort(sc, dim=-1, descending=True, stable=True)
    S = sc.shape[-1]
    rank = torch.arange(S).view(*([1] * (sc.ndim - 1)), S)
    keep = torch.zeros_like(sc, dtype=torch.uint8)
    keep.scatter_(-1, order, (rank < alloc[..., None]).to(torch.uint8))
    return keep.masked_fill(~torch.isfinite(sc), 0), alloc


# ---------------------------------------------------------------------------
# a10: the route layer
# ---------------------------------------------------------------------------
def route_layer(q, k, v, route_q, entropy_bias_scale, key_valid=None, *, local_window=256,
                chunk_size=64, topk=32, temperature=1.0, gate_offset=0.0, gate_scale=1.0,
                skip_inert_slots=True, token_budget=0, token_policy="global_qk",
                min_tokens_per_chunk=1):
    """KernelDreamFullHiLSAttention.forward between projections and o_proj
    (dream_dllm_hils/attention.py:1380-1774), with the reference's bf16
    rounding between stages.  token_budget > 0 adds the token refinement
    (attention.py:1729-1769): candidate token scores of q in the routed
    chunks, the keep mask of the policy ("global_qk": global top budget;
    "entropy_adaptive": per-chunk quotas from the pool entropy), and the
    routed attention restricted to it.  Returns (out bf16, intermediates dict)."""

    B, L, Hq, D = q.shape
    Hkv = k.shape[2]
    G = Hq // Hkv
    S = chunk_size
    C = L // S
    kv = torch.ones(B, L, dtype=torch.bool) if key_valid is None else key_valid.bool()
    window = local_window + S - 1 if skip_inert_slots else local_window
    local_out, local_lse = local_attention(q, k, v, kv, window, S if skip_inert_slots else 0)
    local_out = local_out.to(torch.bfloat16)
    q_lmk = route_q[:, S - 1 :: S].reshape(B, C, Hkv, G, D)
    lmk, entropy = chunk_attn_pool(q_lmk, k.reshape(B, C, S, Hkv, D), kv.reshape(B, C, S))
    lmk = lmk.to(torch.bfloat16)
    prior = entropy * entropy_bias_scale.float().view(1, 1, Hkv, G)
    drop = remote_drop_mask(kv, local_window, S)
    idx, scores, sel = route_topk(
        route_q.reshape(B, L, Hkv, G, D), lmk.reshape(B, C, Hq, D),
        local_lse.reshape(B, L, Hkv, G), topk, S, drop_mask=drop, bias4=prior,
    )
    scores_bf = scores.reshape(B, L, Hq, topk).to(torch.bfloat16)
    if topk >= 32:
        # attention.py:1571-1621: _route_weights_torch with the layer's
        # temperature and fusion gate parameters
        rw, lw = route_weights(scores_bf, idx, prior, local_lse, temperature=temperature,
                               gate_offset=gate_offset, gate_scale=gate_scale)
    else:
        # attention.py:1643-1648: the TileLang route_weights, plain 33-way
        # softmax at temperature 1 with no gate
        rw, lw = route_weights(scores_bf, idx, prior, local_lse)
    rw = rw.to(torch.bfloat16)
    lw = lw.to(torch.bfloat16)
    keep = None
    if token_budget > 0:
        keep = _token_keep(q, k, idx, kv, S, token_budget, token_policy, entropy,
                           min_tokens_per_chunk)
    remote = selected_attention(q, k, v, rw, idx, kv, S, token_keep=keep).to(torch.bfloat16)
    out = fuse_outputs(remote, local_out, lw)
    return out, {
        "local_output": local_out, "local_lse": local_lse, "landmark_keys": lmk,
        "entropy": entropy, "prior_bias": prior, "indices": idx, "scores": scores_bf,
        "selection": sel, "remote_weights": rw, "local_weight": lw, "remote_output": remote,
        "token_keep": keep,
    }


def _token_keep(q, k, idx, kv, S, token_budget, token_policy, entropy, min_tokens_per_chunk):
    """The token keep mask of a policy (attention.py:1729-1759,
    fastdllm_attention.py:330-361)."""

    scores = candidate_token_scores(q, k, idx, kv, S)
    if token_policy == "global_qk":
        return select_global_token_keep(scores, token_budget)
    keep, _ = select_entropy_adaptive_token_keep(
        scores, gather_selected_chunk_entropy(entropy, idx), token_budget, min_tokens_per_chunk)
    return keep


def cached_route_layer(q, route_q, cache_key, cache_value, cache_valid, landmark_keys,
                       prior_bias, query_positions, affected_chunks, entropy_bias_scale, *,
                       local_window=256, chunk_size=64, topk=32, skip_inert_slots=True,
                       token_budget=0, token_policy="global_qk", min_tokens_per_chunk=1):
    """Cached block step of a route layer (dream_dllm_hils/fastdllm_attention.py:
    203-382) after the projections and the K/V update, with the reference's
    bf16 rounding between stages.  landmark_keys [1, C, Hkv, G, D] bf16 and
    prior_bias [1, C, Hkv, G] fp32 are refreshed for affected_chunks (copies
    are returned; the inputs are not modified).  Returns (out bf16,
    landmark_keys, prior_bias, intermediates dict)."""

    B, Lq, Hq, D = q.shape
    L, Hkv = cache_key.shape[1], cache_key.shape[2]
    G = Hq // Hkv
    S = chunk_size
    C = L // S
    kv = cache_valid.bool()
    pos = query_positions.long().cpu()
    window = local_window + S - 1 if skip_inert_slots else local_window
    local_out, local_lse = local_attention(q, cache_key, cache_value, kv, window,
                                           S if skip_inert_slots else 0, query_positions=pos)
    local_out = local_out.to(torch.bfloat16)
    lmk_all = landmark_keys.clone()
    prior_all = prior_bias.clone()
    aff = affected_chunks.long().cpu()
    if aff.numel():
        # fastdllm_attention.py:236-292 (_rows_for_positions: rows of the
        # landmark positions in the query block)
        rows = torch.searchsorted(pos, aff * S + (S - 1))
        q_lmk = route_q[:, rows].reshape(B, aff.numel(), Hkv, G, D)
        cpos = (aff[:, None] * S + torch.arange(S)[None]).reshape(-1)
        chunk_keys = cache_key[:, cpos].reshape(B, aff.numel(), S, Hkv, D)
        chunk_valid = kv[:, cpos].reshape(B, aff.numel(), S)
        lmk, entropy = chunk_attn_pool(q_lmk, chunk_keys, chunk_valid)
        lmk_all[:, aff] = lmk.to(torch.bfloat16)
        prior_all[:, aff] = entropy * entropy_bias_scale.float().view(1, 1, Hkv, G)
    drop = remote_drop_mask_rows(kv, local_window, S, pos)
    idx, scores, sel = route_topk(
        route_q.reshape(B, Lq, Hkv, G, D), lmk_all.reshape(B, C, Hq, D),
        local_lse.reshape(B, Lq, Hkv, G), topk, S, drop_mask=drop, bias4=prior_all,
    )
    scores_bf = scores.reshape(B, Lq, Hq, topk).to(torch.bfloat16)
    rw, lw = route_weights(scores_bf, idx, prior_all, local_lse, temperature=1.0)
    rw = rw.to(torch.bfloat16)
    lw = lw.to(torch.bfloat16)
    keep = None
    if token_budget > 0:
        # fastdllm_attention.py:345-350: the entropy of the cached prior bias
        entropy = prior_all / entropy_bias_scale.float().view(1, 1, Hkv, G)
        keep = _token_keep(q, cache_key, idx, kv, S, token_budget, token_policy, entropy,
                           min_tokens_per_chunk)
    remote = selected_attention(q, cache_key, cache_value, rw, idx, kv, S,
                                token_keep=keep).to(torch.bfloat16)
    out = fuse_outputs(remote, local_out, lw)
    return out, lmk_all, prior_all, {
        "local_output": local_out, "local_lse": local_lse, "indices": idx,
        "scores": scores_bf, "selection": sel, "remote_weights": rw, "local_weight": lw,
        "remote_output": remote, "drop_mask": drop, "token_keep": keep,
    }
