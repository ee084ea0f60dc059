"""Route scoring with per-KV-group top-k ("softmax then max pooling").

Drop-ins for ``ops.topk_head_softmax.ref_softmax_topk_max_pooling``
(ops/topk_head_softmax.py:15-156) and ``online_softmax_topk_head``
(:1242-1415).  Both run the gfx950 route kernel (mrsa_route_topk_fwd); when q or the
landmarks require grad the scores are differentiable through the route-score
backward kernel (mrsa_route_score_bwd).  Gumbel noise [1, 1, h_q, S] (training
only) is added, like the bias, to the selection logits and the route LSE and
not to the returned scores (ops/topk_head_softmax.py:99-105, :341-353,
:599-607): it enters the kernel folded into the per-chunk bias.
"""

from __future__ import annotations

import math

import torch

from . import _lib
from .kernel_utils import group_pad_to

# Largest fp32 logits workspace the workspace route path may take (a 64k-token
# Dream layer with 1024 chunks needs 7.5 GB of the 288 GB of HBM; the scalar
# general kernel it replaces is about 50x slower there).
_WORKSPACE_LIMIT = 16 << 30


def _fast_shape(C, G, D, topk, scores_fp32, is_causal):
    """Shapes of the matrix-core route kernel (up to 256 chunks, bf16 scores)."""
    return (not scores_fp32 and not is_causal and D == 128 and C <= 256 and topk <= 64
            and G in (7, 8))


def _workspace_bytes(B, L, C, Hkv, G, D, topk, scores_fp32, is_causal):
    """Bytes of the workspace the route kernels take, 0 for none.  The
    matrix-core kernel (up to 256 chunks) runs without one; beyond 256
    chunks, with head_dim 128, groups <= 8 and chunks <= 4096, the two-kernel
    path runs over an fp32 logits workspace [B, L, Hkv, G, C]."""
    if _fast_shape(C, G, D, topk, scores_fp32, is_causal):
        return 0
    if D != 128 or G > 8 or C > 4096:
        return 0
    n = B * L * Hkv * G * C * 4
    return n if n <= _WORKSPACE_LIMIT else 0


def route_topk_launch(
    q5: torch.Tensor,
    lmks: torch.Tensor,
    lse4: torch.Tensor | None,
    topk: int,
    block_size: int,
    *,
    bias4: torch.Tensor | None = None,
    drop_mask: torch.Tensor | None = None,
    derive_window: int = -1,
    key_valid: torch.Tensor | None = None,
    is_causal: bool = False,
    window_size: int = 0,
    q_offset: int = 0,
    selection_mode: str = "post_softmax",
    sm_scale: float | None = None,
    scores_fp32: bool = False,
    use_workspace: bool | None = None,
):
    """Run the route kernel.

    q5 [B, L, Hkv, G, D] bf16; lmks [B, C, Hkv*G, D] (per-head) or
    [B, C, Hkv, D] (shared) bf16; lse4 [B, L, Hkv, G] fp32; bias4
    [B, C, Hkv, G] fp32; drop_mask [B, L, C].  With derive_window >= 0 the
    drop mask of remote_drop_mask(key_valid, derive_window, block_size) is
    computed inside the kernel instead.
    Returns indices [B, L, Hkv, topk] int32 and scores [B, L, Hkv, G, topk].
    ``use_workspace`` (None: by shape) passes the kernels an fp32 logits
    workspace [B, L, Hkv, G, C] for the short-block path; the matrix-core
    kernel (up to 256 chunks) takes none.
    """

    if selection_mode not in {"post_softmax", "pre_softmax"}:
        raise ValueError(f"unsupported selection_mode={selection_mode}")
    if q5.device.type != "cuda":
        raise ValueError("route scoring requires CUDA tensors")
    B, L, Hkv, G, D = q5.shape
    C = lmks.shape[1]
    if lmks.shape[2] == Hkv * G:
        per_head = 1
    elif lmks.shape[2] == Hkv:
        per_head = 0
    else:
        raise AssertionError(
            f"k_lmks h dim ({lmks.shape[2]}) must be either h_kv ({Hkv}) or h_kv*G ({Hkv * G})"
        )
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    if selection_mode == "post_softmax" and lse4 is None:
        raise ValueError("post_softmax selection needs the local LSE")
    if drop_mask is not None and derive_window < 0 and drop_mask.shape != (B, L, C):
        raise ValueError(f"invalid drop_mask shape {tuple(drop_mask.shape)}")
    if selection_mode != "post_softmax":
        lse4 = None
    if derive_window >= 0:
        drop_mask = None
    else:
        key_valid = None
    args = (q5, lmks, lse4, bias4, drop_mask, key_valid, int(topk), int(block_size),
            int(derive_window), bool(is_causal), int(window_size), int(q_offset),
            selection_mode != "post_softmax", float(sm_scale), bool(scores_fp32),
            -1 if use_workspace is None else int(bool(use_workspace)))
    if torch.is_grad_enabled() and (q5.requires_grad or lmks.requires_grad):
        return _RouteTopK.apply(*args)
    return torch.ops.mrsa.route_topk(*args)


class _RouteTopK(torch.autograd.Function):
    """Route scoring with the scores differentiable in q and the landmarks
    (SoftmaxTopKMaxPoolingFusedFn, ops/topk_head_softmax.py:1004-1122): the
    indices, the local LSE, the bias and the drop mask get no gradient."""

    @staticmethod
    def forward(ctx, q5, lmks, lse4, bias4, drop_mask, key_valid, topk, block_size,
                derive_window, is_causal, window_size, q_offset, pre_softmax, sm_scale,
                scores_fp32, use_workspace):
        indices, scores = torch.ops.mrsa.route_topk(
            q5, lmks, lse4, bias4, drop_mask, key_valid, topk, block_size, derive_window,
            is_causal, window_size, q_offset, pre_softmax, sm_scale, scores_fp32,
            use_workspace)
        ctx.mark_non_differentiable(indices)
        ctx.save_for_backward(q5, lmks, indices)
        ctx.sm_scale = sm_scale
        return indices, scores

    @staticmethod
    def backward(ctx, grad_indices, grad_scores):
        q5, lmks, indices = ctx.saved_tensors
        none = (None,) * 14
        if grad_scores is None:
            return (None, None) + none
        grad_q, grad_lmks = torch.ops.mrsa.route_score_bwd(
            q5, lmks, indices, grad_scores, ctx.sm_scale)
        grad_q = grad_q.to(q5.dtype) if ctx.needs_input_grad[0] else None
        grad_lmks = grad_lmks.to(lmks.dtype) if ctx.needs_input_grad[1] else None
        return (grad_q, grad_lmks) + none


def _route_score_bwd_impl(q5, lmks, indices, grad_scores, sm_scale):
    """Gradients of the route scores in q [B, L, Hkv, G, D] and the landmarks
    [B, C, Hkv*G or Hkv, D] (bf16, the shapes of the inputs)."""
    B, L, Hkv, G, D = q5.shape
    C = lmks.shape[1]
    K = indices.shape[-1]
    per_head = 1 if lmks.shape[2] == Hkv * G else 0
    qc = q5.to(torch.bfloat16).contiguous()
    lc = lmks.to(torch.bfloat16).contiguous()
    idx = indices.to(device=q5.device, dtype=torch.int32).contiguous()
    gs = grad_scores.reshape(B, L, Hkv, G, K)
    if gs.dtype not in (torch.bfloat16, torch.float32):
        gs = gs.float()
    gs = gs.contiguous()
    grad_q = torch.empty_like(qc)
    grad_lmks = torch.empty_like(lc)
    nbytes = int(_lib.call("mrsa_route_score_bwd_workspace_bytes", B, L, C, Hkv, G, per_head))
    if nbytes < 0:
        raise ValueError(f"invalid route score shapes q {tuple(q5.shape)} lmks {tuple(lmks.shape)}")
    ws = torch.empty(max(nbytes, 16) // 4, dtype=torch.float32, device=q5.device)
    st = _lib.call(
        "mrsa_route_score_bwd", _lib.ptr(qc), _lib.ptr(lc), _lib.ptr(idx), _lib.ptr(gs),
        1 if gs.dtype == torch.float32 else 0, B, L, C, Hkv, G, D, K, per_head, float(sm_scale),
        _lib.ptr(grad_q), _lib.ptr(grad_lmks), _lib.ptr(ws), nbytes, _lib.stream_of(qc))
    _lib.check(st, "route_score_bwd")
    return grad_q, grad_lmks


def _route_topk_impl(q5, lmks, lse4, bias4, drop_mask, key_valid, topk, block_size,
                     derive_window, is_causal, window_size, q_offset, pre_softmax, sm_scale,
                     scores_fp32, use_workspace):
    B, L, Hkv, G, D = q5.shape
    C = lmks.shape[1]
    per_head = 1 if lmks.shape[2] == Hkv * G else 0
    selection_mode = "pre_softmax" if pre_softmax else "post_softmax"
    use_workspace = None if use_workspace < 0 else bool(use_workspace)
    qc = q5.to(torch.bfloat16).contiguous()
    lc = lmks.to(torch.bfloat16).contiguous()
    lse = None
    if lse4 is not None:
        lse = lse4.to(device=q5.device, dtype=torch.float32).reshape(B, L, Hkv, G).contiguous()
    bias = None
    if bias4 is not None:
        bias = bias4.to(device=q5.device, dtype=torch.float32).reshape(B, C, Hkv, G).contiguous()
    drop = None
    if drop_mask is not None:
        drop = drop_mask.to(device=q5.device, dtype=torch.int32).contiguous()
    kv = None
    if key_valid is not None:
        kv = key_valid.to(device=q5.device, dtype=torch.bool).contiguous()
    indices = torch.empty(B, L, Hkv, topk, dtype=torch.int32, device=q5.device)
    scores = torch.empty(
        B, L, Hkv, G, topk,
        dtype=torch.float32 if scores_fp32 else torch.bfloat16, device=q5.device,
    )
    args = (
        _lib.ptr(qc), _lib.ptr(lc), _lib.ptr(lse), _lib.ptr(bias), _lib.ptr(drop),
        _lib.ptr(kv), int(derive_window), B, L, C, Hkv, G, D, int(topk), int(block_size),
        per_head, 1 if is_causal else 0, int(window_size), int(q_offset),
        0 if selection_mode == "post_softmax" else 1, float(sm_scale),
        _lib.ptr(indices), _lib.ptr(scores), 1 if scores_fp32 else 0,
    )
    nbytes = _workspace_bytes(B, L, C, Hkv, G, D, topk, scores_fp32, is_causal)
    if use_workspace is None:
        use_workspace = nbytes > 0
    if use_workspace:
        if not _fast_shape(C, G, D, topk, scores_fp32, is_causal):
            nbytes = _lib.call("mrsa_route_topk_workspace_bytes", B, L, C, Hkv, G)
        nbytes = max(int(nbytes), 0)
        ws = torch.empty((nbytes + 3) // 4, dtype=torch.float32, device=q5.device)
        st = _lib.call("mrsa_route_topk_ws_fwd", *args, _lib.ptr(ws), nbytes,
                       _lib.stream_of(qc))
    else:
        st = _lib.call("mrsa_route_topk_fwd", *args, _lib.stream_of(qc))
    _lib.check(st, "route_topk")
    return indices, scores


def _fold_noise(bias4, noise, B, C, Hkv, G, device):
    """bias4 [B, C, Hkv, G] (or None) plus Gumbel noise [1, 1, Hkv * G, C]:
    both are added to the same selection logits and route LSE terms."""
    if noise is None:
        return bias4
    if tuple(noise.shape) != (1, 1, Hkv * G, C):
        raise AssertionError(
            f"gumbel_noise shape {tuple(noise.shape)} != ({1}, {1}, {Hkv * G}, {C})")
    nz = noise.detach().to(device=device, dtype=torch.float32).reshape(Hkv, G, C)
    nz = nz.permute(2, 0, 1)[None]
    if bias4 is None:
        return nz.expand(B, C, Hkv, G).contiguous()
    return (bias4.to(device=device, dtype=torch.float32) + nz).contiguous()


def _bias4(bias, B, C, Hkv, G):
    if bias is None:
        return None
    if bias.dim() == 3:
        assert bias.shape == (B, C, Hkv * G), (
            f"bias shape {tuple(bias.shape)} != ({B}, {C}, {Hkv * G})"
        )
    elif bias.dim() == 4:
        assert bias.shape == (B, C, Hkv, G), (
            f"bias shape {tuple(bias.shape)} != ({B}, {C}, {Hkv}, {G})"
        )
    else:
        raise AssertionError(
            f"bias must be [B, S, h_q] or [B, S, h_kv, G], got {tuple(bias.shape)}"
        )
    return bias.reshape(B, C, Hkv, G)


def ref_softmax_topk_max_pooling(
    q, k_lmks, lse_swa, topk, block_size, window_size, is_causal=False, q_offset=0,
    drop_mask=None, bias=None, gumbel_noise=None, selection_mode="post_softmax",
):
    """Same contract as ops/topk_head_softmax.py:15-156.

    q [B, L, h_kv, G, D]; k_lmks [B, S, h_kv, D] or [B, S, h_kv*G, D];
    lse_swa [B, L, h_q] or [B, L, h_kv, G]; gumbel_noise [1, 1, h_q, S] or
    None; returns indices [B, L, h_kv, topk] (int64, ascending, -1 last) and
    fp32 raw scores [B, L, h_kv, G, topk] (without bias or noise).
    """

    if selection_mode not in {"post_softmax", "pre_softmax"}:
        raise ValueError(f"unsupported selection_mode={selection_mode}")
    B, L, Hkv, G, D = q.shape
    C = k_lmks.shape[1]
    lse4 = None
    if selection_mode == "post_softmax":
        lse4 = lse_swa.reshape(B, L, Hkv, G)
    indices, scores = route_topk_launch(
        q, k_lmks, lse4, topk, block_size,
        bias4=_fold_noise(_bias4(bias, B, C, Hkv, G), gumbel_noise, B, C, Hkv, G, q.device),
        drop_mask=drop_mask,
        is_causal=is_causal, window_size=window_size, q_offset=q_offset,
        selection_mode=selection_mode, sm_scale=1.0 / math.sqrt(D), scores_fp32=True,
    )
    return indices.to(torch.int64), scores


def online_softmax_topk_head(
    q, lmks, lse_swa, topk, block_size, window_size, is_causal=True, q_offset=0,
    is_training=True, drop_mask=None, sm_scale=None, bias=None, use_gumbel=False,
    gumbel_noise=None, G=1,
):
    """Same contract as ops/topk_head_softmax.py:1242-1415.  The scores are
    differentiable in q and lmks when they require grad; use_gumbel (or a
    given gumbel_noise [1, 1, h_q, S]) adds Gumbel noise to the selection in
    training mode.

    Returns (indices [B, L, h_kv, topk] int32, scores [B, L, h_q, topk] bf16);
    for is_training=False with a logical group of 7 the scores come back in
    the reference's physical G=8 layout (pad slot -inf), as its inference
    branch does.
    """

    use_gumbel = bool(use_gumbel) or gumbel_noise is not None
    if use_gumbel and not is_training:
        raise AssertionError("gumbel_noise is only supported in training mode")
    if q.dim() == 4:
        B, L, h_q, D = q.shape
        lmks_h = lmks.shape[2]
        if lmks.shape[3] != D:
            ratio = lmks.shape[3] // D
            lmks = lmks.reshape(lmks.shape[0], lmks.shape[1], lmks_h * ratio, D)
            lmks_h *= ratio
        if G == 1:
            assert h_q % lmks_h == 0, f"h_q ({h_q}) must be divisible by lmks_h ({lmks_h})"
            h_kv = lmks_h
            g_eff = h_q // h_kv
        else:
            assert lmks_h == h_q, f"when G>1, lmks must have h_q ({h_q}) heads, got {lmks_h}"
            assert h_q % G == 0, f"h_q ({h_q}) must be divisible by G ({G})"
            h_kv = h_q // G
            g_eff = G
        q5 = q.reshape(B, L, h_kv, g_eff, D)
    else:
        B, L, h_kv, g_eff, D = q.shape
        h_q = h_kv * g_eff
        q5 = q
        if G > 1 and (h_q // G != h_kv or G != g_eff):
            h_kv, g_eff = h_q // G, G
            q5 = q.reshape(B, L, h_kv, g_eff, D)
    C = lmks.shape[1]
    lse4 = lse_swa.reshape(B, L, h_kv, g_eff)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    bias4 = _bias4(bias, B, C, h_kv, g_eff)
    if use_gumbel:
        if gumbel_noise is None:
            # ops/topk_head_softmax.py:1177-1180
            u = torch.rand(1, 1, h_kv * g_eff, C, device=q.device, dtype=torch.float32)
            u.clamp_(min=1e-20, max=1 - 1e-7)
            gumbel_noise = -torch.log(-torch.log(u))
        bias4 = _fold_noise(bias4, gumbel_noise, B, C, h_kv, g_eff, q.device)
    indices, scores = route_topk_launch(
        q5, lmks, lse4, topk, block_size,
        bias4=bias4, drop_mask=drop_mask,
        is_causal=is_causal, window_size=window_size, q_offset=q_offset,
        sm_scale=sm_scale if is_training else 1.0 / math.sqrt(D),
    )
    if not is_training and g_eff == 7:
        scores = group_pad_to(
            scores.reshape(B, L, h_kv * 7, topk), h_kv, 7, 8, value=float("-inf")
        )
        return indices.to(torch.int64), scores
    return indices, scores.reshape(B, L, h_kv * g_eff, topk)
