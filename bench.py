"""Benchmark: MRSA route-layer forward tokens/s at L=16384 on one MI355X.

One step = one route-layer attention forward (value tiles, local window
attention, landmark pool, route scoring + top-32, route weights, routed chunk
attention, output fusion) over B=1, L=16384, 28 query / 4 KV heads, d=128,
64-token chunks, local radius 256 on
synthetic seeded Gaussian Q/K/V with a per-chunk planted key shift (sigma 0.3).
Inputs are resident in HBM before timing starts.

Prints ONE JSON line (rank 0).  Besides the contract fields it carries:
  roofline      dominant kernel (routed chunk attention) against bf16 MFMA peak,
                its average duration from HIP events around each launch in the
                timed steps, HBM traffic per launch from profiles/pmc_traffic.json
  cpu_baseline  the CPU oracle's route layer at configuration 1 (L=4096, fp32)
                timed on this host's cores
  stages_us     average per-stage times from per-stage events, recorded in
                as many extra steps after the timed region (an event between
                dependent kernels costs a few microseconds of dispatch, so the
                timed steps record only the two around the routed attention)

``--workload backward`` times the backward of the routed attention, of the
route scores and of the window attention (radius 319, landmark slots inert)
at configuration 2's shapes, on the routing of the forward route layer
(training-side: no BASELINE number exists for it).

``--workload decode`` instead times the Fast-dLLM cached block step of one
route layer (SURVEY configuration 5): a K/V cache of L=131072 tokens (2048
chunks), 64 successive 32-token query blocks at its tail; each step writes the
block's K/V rows into the cache, refreshes the landmark summary of the chunk
whose landmark slot the block holds, and runs mrsa.cached_route_attention.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(
    ROOT, "mask-routed-sparse-attention-for-long-context-diffusion-language-models_amd"
)
for _p in (PKG_DIR, ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "MRSA route-layer fwd tokens/s @16k (Dream-7B heads); % MFMA/HBM roofline"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0

L_CFG2, HQ, HKV, D, CHUNK, TOPK, WINDOW = 16384, 28, 4, 128, 64, 32, 256


def selected_flops(L: int) -> float:
    """Algorithmic FLOPs of the routed chunk attention: QK^T + PV over every
    routed (query head, chunk) pair, the 63 real keys of each chunk (the
    landmark slot is excluded), 2 FLOP per MAC."""

    return 4.0 * D * HQ * L * TOPK * 63


def make_inputs(L: int, seed: int, device, dtype):
    import torch

    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, L, HQ, D, generator=g)
    k = torch.randn(1, L, HKV, D, generator=g)
    v = torch.randn(1, L, HKV, D, generator=g)
    shift = 0.3 * torch.randn(L // CHUNK, HKV, D, generator=g)
    k = k + shift.repeat_interleave(CHUNK, dim=0)[None]
    return q.to(device=device, dtype=dtype), k.to(device=device, dtype=dtype), \
        v.to(device=device, dtype=dtype)


def cpu_baseline(budget_s: float = 30.0):
    """Oracle route layer at BASELINE configuration 1 on the host CPU: one
    untimed warmup forward, then the median of 3 timed forwards (fewer only
    when the budget runs out)."""

    import torch

    from oracle import mrsa_oracle as O

    torch.set_num_threads(os.cpu_count() or 1)
    L = 4096
    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, L, HQ, D, generator=g)
    k = torch.randn(1, L, HKV, D, generator=g)
    v = torch.randn(1, L, HKV, D, generator=g)
    k[:, CHUNK - 1 :: CHUNK] += 0.5    # landmark role offset
    scale = torch.ones(HQ)
    runs = []
    t_end = time.perf_counter() + budget_s
    O.route_layer(q.bfloat16(), k.bfloat16(), v.bfloat16(), q.bfloat16(), scale)  # warmup
    while True:
        t0 = time.perf_counter()
        O.route_layer(q.bfloat16(), k.bfloat16(), v.bfloat16(), q.bfloat16(), scale)
        runs.append(time.perf_counter() - t0)
        if time.perf_counter() > t_end or len(runs) >= 3:
            break
    best = sorted(runs)[len(runs) // 2]
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": L / best,
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"1 warmup + {len(runs)} timed full route-layer forwards at L=4096 "
                  f"(config 1), fp32 CPU oracle, median {best:.2f} s; cpu={cpu_model}",
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # None: per workload.  The route and SWA steps take ~1-3 ms; their kernels
    # reach steady clocks only after a few dozen launches, so the default
    # warmup is long enough for the timed steps to see that state.
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--workload", choices=("route", "decode", "swa", "model", "backward"),
                    default="route")
    ap.add_argument("--token-budget", type=int, default=0,
                    help="route workload with the remote-token refinement (global_qk) at "
                         "this budget (0: off, the configuration-2 default)")
    ap.add_argument("--deterministic", action="store_true",
                    help="routed attention in the fixed accumulation order "
                         "(RouteLayerConfig.deterministic)")
    ap.add_argument("--decode-eager", action="store_true",
                    help="decode workload without the captured step graph")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run a plain 1 GiB device copy three times (reference "
                         "dispatch for scaling FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    short = args.workload in ("route", "swa", "backward")
    if args.steps is None:
        args.steps = 50 if short else 20
    if args.warmup is None:
        args.warmup = 30 if short else 5
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); "
              "the route layer shards by KV head / sequence as described in DESIGN.md",
              file=sys.stderr)
        return 2

    import torch

    import mrsa

    dev = torch.device("cuda:0")
    if args.workload == "decode":
        return decode_main(args, torch, mrsa, dev)
    if args.workload == "model":
        return model_main(args, torch, mrsa, dev)
    if args.workload == "swa":
        return swa_main(args, torch, mrsa, dev)
    if args.workload == "backward":
        return backward_main(args, torch, mrsa, dev)
    if args.copy_calibration:
        src = torch.empty(1 << 29, dtype=torch.int16, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    q, k, v = make_inputs(L_CFG2, 1234, dev, torch.bfloat16)
    route_q = q
    scale = torch.ones(HQ, device=dev)
    key_valid = torch.ones(1, L_CFG2, dtype=torch.bool, device=dev)
    cfg = mrsa.RouteLayerConfig(local_window=WINDOW, chunk_size=CHUNK, topk=TOPK,
                                token_budget=args.token_budget,
                                deterministic=args.deterministic)

    stream = torch.cuda.current_stream(dev)

    # Timed steps record two events each, around the routed attention (the
    # dominant kernel): an event between dependent kernels costs a few
    # microseconds of dispatch, so the per-stage events run in separate
    # steps after the timed region.
    def run(events):
        evs = []

        def mark(name):
            if events == "all" or name in ("route_weights", "token_refinement",
                                           "selected_attention"):
                e = torch.cuda.Event(enable_timing=True)
                e.record(stream)
                evs.append((name, e))
        out = mrsa.route_attention(q, k, v, route_q, scale, key_valid, cfg,
                                   mark=mark if events else None)
        return out, evs

    for _ in range(args.warmup):
        run(None)
    torch.cuda.synchronize()
    routed_events = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        routed_events.append(run("routed")[1])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = 1000.0 * elapsed / args.steps
    sel = [evs[-2][1].elapsed_time(evs[-1][1]) * 1000.0 for evs in routed_events]

    stage_events = [run("all")[1] for _ in range(args.steps)]
    torch.cuda.synchronize()
    stages = {}
    for evs in stage_events:
        for (_, a), (name, b) in zip(evs[:-1], evs[1:]):
            stages.setdefault(name, []).append(a.elapsed_time(b) * 1000.0)
    stages_us = {n: sum(x) / len(x) for n, x in stages.items()}

    sel_us = sum(sel) / len(sel)
    achieved = selected_flops(L_CFG2) / (sel_us * 1e-6) / 1e12
    # HBM bytes per launch cannot be counted from inside the run: they come
    # from the FETCH_SIZE / WRITE_SIZE counter passes of the committed profile
    # (rocprofv3 --pmc over this bench), labelled with the commit they were
    # measured at.
    traffic, traffic_src = None, None
    tpath = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    if os.path.exists(tpath):
        try:
            tj = json.load(open(tpath))
            traffic = tj.get("selected_attention_bytes_per_launch")
            traffic_src = f"{tj.get('source')} @ {tj.get('measured_at', '?')}"
        except (OSError, ValueError):
            traffic = None
    giveups = mrsa.routed_lock_giveups(reset=True)

    line = {
        "metric": METRIC,
        "value": L_CFG2 / (ms_per_step / 1000.0),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "MRSA route-layer attention forward (BASELINE config 2)",
            "global_batch": 1,
            "seq_len": L_CFG2,
            "q_heads": HQ,
            "kv_heads": HKV,
            "head_dim": D,
            "chunk_size": CHUNK,
            "topk": TOPK,
            "local_window": WINDOW,
            "token_budget": args.token_budget,
            "deterministic": args.deterministic,
            "parallelism": "single-gpu",
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "selected_attention (routed chunk attention)",
            "achieved": achieved,
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": achieved / PEAK_BF16_TFLOPS,
            "traffic": traffic,
            "traffic_source": traffic_src,
            "flops_per_launch": selected_flops(L_CFG2),
            "avg_launch_us": sel_us,
        },
        "stages_us": stages_us,
        "lock_giveups": giveups,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)
    if giveups:
        # a routed-attention tile ran out of its bounded lock wait at the
        # default bound: replayed exactly, but a sign of a broken lock
        print(f"bench.py: {giveups} routed-attention tiles ran out of the lock wait",
              file=sys.stderr)
        return 1
    return 0


def backward_flops(L: int) -> float:
    """Algorithmic FLOPs of the routed-attention backward: per (query head,
    routed slot) the five 63-key x 128 products S, dP, dQ, dK, dV (2 FLOP per
    MAC)."""
    return 5.0 * 2.0 * 63 * D * HQ * TOPK * L


def backward_main(args, torch, mrsa, dev) -> int:
    """Backward of the routed chunk attention (HiLS_block_M_head's backward:
    dQ, dK, dV, dW, K/V fragment layouts included) and of the route scores
    (grad_q, grad_lmk) at configuration 2, with indices, weights and
    landmarks from the forward route layer and seeded upstream gradients."""

    from mrsa.local_attention import local_attention_backward, local_attention_launch
    from mrsa.sparse_attention import kv_fragments, selected_attention_backward

    L, C, G = L_CFG2, L_CFG2 // CHUNK, HQ // HKV
    q, k, v = make_inputs(L, 1234, dev, torch.bfloat16)
    valid = torch.ones(1, L, dtype=torch.bool, device=dev)
    cfg = mrsa.RouteLayerConfig(local_window=WINDOW, chunk_size=CHUNK, topk=TOPK)
    _, mid = mrsa.route_attention(q, k, v, q, torch.ones(HQ, device=dev), valid, cfg,
                                  return_intermediates=True)
    idx, w, lmk = mid["indices"], mid["remote_weights"], mid["landmark_keys"]
    g = torch.Generator(device=dev).manual_seed(97)
    dout = torch.randn(1, L, HQ, D, generator=g, device=dev).bfloat16()
    dscore = torch.randn(1, L, HKV, G, TOPK, generator=g, device=dev).bfloat16()
    q5 = q.reshape(1, L, HKV, G, D)
    lmk4 = lmk.reshape(1, C, HQ, D)
    flash_window = WINDOW + CHUNK - 1
    local_out, local_lse = local_attention_launch(q, kv_fragments(k, v), valid, flash_window, CHUNK)
    stream = torch.cuda.current_stream(dev)
    times = []

    def run(record):
        e = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        e[0].record(stream)
        selected_attention_backward(q, k, v, w, idx, valid, CHUNK, dout)
        e[1].record(stream)
        torch.ops.mrsa.route_score_bwd(q5, lmk4, idx, dscore, D ** -0.5)
        e[2].record(stream)
        local_attention_backward(q, k, v, valid, local_out, local_lse, dout, flash_window, CHUNK)
        e[3].record(stream)
        if record:
            times.append(e)

    for _ in range(args.warmup):
        run(False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run(True)
    torch.cuda.synchronize()
    ms_per_step = 1000.0 * (time.perf_counter() - t0) / args.steps
    sel_us = sum(e[0].elapsed_time(e[1]) for e in times) * 1000.0 / len(times)
    score_us = sum(e[1].elapsed_time(e[2]) for e in times) * 1000.0 / len(times)
    window_us = sum(e[2].elapsed_time(e[3]) for e in times) * 1000.0 / len(times)
    flops = backward_flops(L)
    achieved = flops / (sel_us * 1e-6) / 1e12
    line = {
        "metric": "MRSA route-layer backward (routed attention + route scores + window) tokens/s @16k (config 2 shapes)",
        "value": L / (ms_per_step / 1000.0),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "routed attention + route score + window attention backward (config 2 shapes)",
                   "seq_len": L, "q_heads": HQ, "kv_heads": HKV, "head_dim": D,
                   "chunk_size": CHUNK, "topk": TOPK, "parallelism": "single-gpu"},
        "roofline": {"bound": "mfma", "kernel": "selected_attention backward (chunk-major)",
                     "achieved": achieved, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_BF16_TFLOPS, "traffic": None,
                     "flops_per_launch": flops, "avg_launch_us": sel_us},
        "stages_us": {"selected_attention_backward": sel_us, "route_score_backward": score_us,
                      "local_attention_backward": window_us},
    }
    print(json.dumps(line), flush=True)
    return 0


SWA_L, SWA_WINDOW = 16384, 1280


def swa_flops(L: int, W: int) -> float:
    """Algorithmic FLOPs of bidirectional window attention of radius W: QK^T
    + PV over every in-window (query head, key) pair (2 FLOP per MAC)."""
    pairs = L * (2 * W + 1) - W * (W + 1)
    return 4.0 * D * HQ * pairs


def swa_main(args, torch, mrsa, dev) -> int:
    """SWA-1280 layer attention (configuration 3): tokens/s of
    swa_attention (V re-layout + window kernel) at L=16384, 28/4 heads, d=128.
    Seeded N(0,1) q/k/v with YaRN factor-8 RoPE applied to q and k in fp32
    over positions 0..L-1 before the bf16 cast."""

    from mrsa.dream import DreamShape, yarn_rotate_fp32

    L, W = SWA_L, SWA_WINDOW
    g = torch.Generator().manual_seed(2468)
    shape = DreamShape()
    q = yarn_rotate_fp32(torch.randn(1, L, HQ, D, generator=g).to(dev), shape)
    k = yarn_rotate_fp32(torch.randn(1, L, HKV, D, generator=g).to(dev), shape)
    v = torch.randn(1, L, HKV, D, generator=g).to(dev)
    q, k, v = (t.to(torch.bfloat16) for t in (q, k, v))
    valid = torch.ones(1, L, dtype=torch.bool, device=dev)
    stream = torch.cuda.current_stream(dev)
    times = []

    def run(record):
        frags = mrsa.kv_fragments(k, v)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        out, _ = mrsa.local_attention.local_attention_launch(q, frags, valid, W, 0)
        e1.record(stream)
        if record:
            times.append((e0, e1))
        return out

    for _ in range(args.warmup):
        run(False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run(True)
    torch.cuda.synchronize()
    ms_per_step = 1000.0 * (time.perf_counter() - t0) / args.steps
    kern_us = sum(a.elapsed_time(b) for a, b in times) * 1000.0 / len(times)
    flops = swa_flops(L, W)
    achieved = flops / (kern_us * 1e-6) / 1e12
    line = {
        "metric": "SWA-1280 layer attention tokens/s @16k (config 3)",
        "value": L / (ms_per_step / 1000.0),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "bidirectional window attention, radius 1280 (config 3)",
                   "seq_len": L, "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "window": W,
                   "parallelism": "single-gpu"},
        "roofline": {"bound": "mfma", "kernel": "local_attention (window 1280)",
                     "achieved": achieved, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_BF16_TFLOPS, "traffic": None,
                     "flops_per_launch": flops, "avg_launch_us": kern_us},
    }
    print(json.dumps(line), flush=True)
    return 0


MODEL_L = 65536


def model_main(args, torch, mrsa, dev) -> int:
    """Full Dream-7B-shaped denoising forward (configuration 4): 28 layers
    (route layers 3, 7, ..., 27 with Q-Cal; SWA-1280 elsewhere), hidden 3584,
    MLP 18944, vocab 152064, L = 65536, random-init bf16 weights, uniform
    random token ids with 25% set to the mask token.  One step = embeddings to
    logits for every position."""

    from mrsa.dream import (DreamShape, DreamWeights, dream_flops, dream_forward,
                            landmark_layout, rope_tables)

    shape = DreamShape()
    L = MODEL_L
    w = DreamWeights.random(shape, dev, seed=7)
    g = torch.Generator().manual_seed(8)
    # uniform random text tokens, 25% replaced by the mask token, in the
    # landmark layout (mask-token landmark slot per chunk, text positions)
    S = shape.route.chunk_size
    text = torch.randint(0, shape.vocab, (1, L // S * (S - 1)), generator=g)
    text[torch.rand(text.shape, generator=g) < 0.25] = shape.mask_token_id
    ids, pos = landmark_layout(text, shape)
    ids = ids.to(dev)
    tables = rope_tables(pos.to(dev), shape)
    stream = torch.cuda.current_stream(dev)
    times = []

    def run(record):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        out = dream_forward(w, ids, tables=tables)
        e1.record(stream)
        if record:
            times.append((e0, e1))
        return out

    for _ in range(args.warmup):
        run(False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        logits = run(True)
    torch.cuda.synchronize()
    ms_per_step = 1000.0 * (time.perf_counter() - t0) / args.steps
    fwd_ms = sum(a.elapsed_time(b) for a, b in times) / len(times)
    assert bool(torch.isfinite(logits[:: 997].float()).all())
    flops = dream_flops(shape, L)
    achieved = flops / (fwd_ms * 1e-3) / 1e12
    line = {
        "metric": "Dream-7B-shaped denoising forward tokens/s @64k (config 4)",
        "value": L / (ms_per_step / 1000.0),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights, random token ids, 25% mask tokens)",
        "config": {"workload": "Dream-7B-shaped denoising forward (config 4)",
                   "seq_len": L, "layers": shape.layers, "route_layers": shape.route_layers(),
                   "hidden": shape.hidden, "intermediate": shape.intermediate,
                   "vocab": shape.vocab, "q_heads": shape.q_heads,
                   "kv_heads": shape.kv_heads, "swa_window": shape.swa_window,
                   "qcal_rank": shape.qcal_rank, "parallelism": "single-gpu"},
        "roofline": {"bound": "mfma", "kernel": "whole forward (GEMMs + attention)",
                     "achieved": achieved, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_BF16_TFLOPS, "traffic": None,
                     "flops_per_step": flops, "forward_ms": fwd_ms},
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)
    return 0


DECODE_L, DECODE_BLOCK, DECODE_BLOCKS = 131072, 32, 64


def decode_main(args, torch, mrsa, dev) -> int:
    """Cached block decode (configuration 5): tokens/s over DECODE_BLOCKS
    successive blocks of DECODE_BLOCK query tokens against a DECODE_L cache."""

    L, S, nb, bs = DECODE_L, CHUNK, DECODE_BLOCKS, DECODE_BLOCK
    C, G = L // S, HQ // HKV
    g = torch.Generator().manual_seed(4321)
    k = torch.randn(1, L, HKV, D, generator=g)
    k = k + 0.3 * torch.randn(C, HKV, D, generator=g).repeat_interleave(S, dim=0)[None]
    v = torch.randn(1, L, HKV, D, generator=g)
    k = k.to(device=dev, dtype=torch.bfloat16)
    v = v.to(device=dev, dtype=torch.bfloat16)
    valid = torch.ones(1, L, dtype=torch.bool, device=dev)
    scale = torch.ones(HQ, device=dev)
    # Landmark summaries of the whole cache (prefill state), not timed.
    q_lmk = torch.randn(1, C, HKV, G, D, generator=g).to(device=dev, dtype=torch.bfloat16)
    lmk, _, prior = mrsa.chunk_attn_pool_gqa_prior(q_lmk, k.reshape(1, C, S, HKV, D),
                                                   valid.reshape(1, C, S), scale)
    cache = mrsa.LayerKVCache(k, v, valid, lmk.contiguous(), prior.contiguous())
    cfg = mrsa.RouteLayerConfig(local_window=WINDOW, chunk_size=S, topk=TOPK,
                                deterministic=args.deterministic)
    start = L - nb * bs
    blocks = []
    for i in range(nb):
        pos = torch.arange(start + i * bs, start + (i + 1) * bs, device=dev)
        lm = pos[(pos + 1) % S == 0]
        blocks.append((
            torch.randn(1, bs, HQ, D, generator=g).to(device=dev, dtype=torch.bfloat16),
            torch.randn(1, bs, HQ, D, generator=g).to(device=dev, dtype=torch.bfloat16),
            torch.randn(1, bs, HKV, D, generator=g).to(device=dev, dtype=torch.bfloat16),
            torch.randn(1, bs, HKV, D, generator=g).to(device=dev, dtype=torch.bfloat16),
            pos, lm // S,
        ))

    graph_step = None if args.decode_eager else mrsa.CachedBlockStep(cache, scale, cfg, bs)

    def step(b):
        q, rq, kb, vb, pos, aff = b
        if graph_step is not None:   # K/V row write + route layer, one HIP graph replay
            return graph_step(q, rq, kb, vb, pos, aff)
        cache.replace(pos, kb, vb)             # the block's K/V rows (fastdllm_cache.py)
        return mrsa.cached_route_attention(q, rq, cache, pos, aff, scale, cfg)

    for b in blocks[: max(2, args.warmup)]:  # both affected-chunk counts captured
        step(b)
    torch.cuda.synchronize()
    reps = max(1, args.steps // 10)
    t0 = time.perf_counter()
    for _ in range(reps):
        for b in blocks:
            step(b)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_block = 1000.0 * elapsed / (reps * nb)
    line = {
        "metric": "MRSA route-layer cached block decode tokens/s @128k (config 5)",
        "value": bs / (ms_per_block / 1000.0),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": reps * nb,
        "warmup": max(2, args.warmup),
        "ms_per_step": ms_per_block,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "Fast-dLLM cached block step of one route layer (SURVEY config 5)",
            "cache_len": L, "block": bs, "blocks": nb, "q_heads": HQ, "kv_heads": HKV,
            "head_dim": D, "chunk_size": S, "topk": TOPK, "local_window": WINDOW,
            "parallelism": "single-gpu",
            "step": "eager" if args.decode_eager else "hip-graph",
        },
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
