"""Benchmark of the causal-chunk attention hot path on one MI355X.

Workload (one step = one chunk's attention cost across a full Wan-14B DiT forward):
  Wan-14B shape, 720p, 1 latent frame per chunk (45 x 80 patch grid = 3600 queries) over
  12 cached frames + the chunk (46800 keys), 40 heads x 128, 40 layers with distinct buffers,
  back to back on one stream. Per layer: fused q/k RMSNorm + 3-D RoPE (writing the chunk's
  K and V into its cache slot), then flash attention of the 3600 queries over the cache.
Synthetic N(0,1) inputs, random RMSNorm gammas. Metric: attention TFLOP/s (4 Lq Lk D H per
layer, softmax excluded) over the whole timed step, plus ms per chunk.

Usage: python bench.py [--steps K] [--warmup W] [--layers N] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "lingbot-world-v2_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_FP8_TFLOPS = 5000.0
PEAK_HBM_GBS = 8000.0

H, D = 40, 128
C = H * D
GRID = (1, 45, 80)
LQ = GRID[0] * GRID[1] * GRID[2]            # 3600
CACHED_FRAMES = 12
LK = LQ * (CACHED_FRAMES + 1)               # 46800
START_FRAME = CACHED_FRAMES
EPS = 1e-6


def attn_flops() -> float:
    return 4.0 * LQ * LK * D * H


def build_layers(n_layers, dev):
    import torch
    g = torch.Generator(device=dev).manual_seed(1234)
    layers = []
    for _ in range(n_layers):
        cache_k = torch.randn(1, LK, H, D, generator=g, device=dev).to(torch.bfloat16)
        cache_v = torch.randn(1, LK, H, D, generator=g, device=dev).to(torch.bfloat16)
        layers.append(dict(
            xq=torch.randn(LQ, C, generator=g, device=dev).to(torch.bfloat16),
            xk=torch.randn(LQ, C, generator=g, device=dev).to(torch.bfloat16),
            xv=torch.randn(LQ, C, generator=g, device=dev).to(torch.bfloat16),
            wq=(1 + 0.1 * torch.randn(C, generator=g, device=dev)).to(torch.bfloat16),
            wk=(1 + 0.1 * torch.randn(C, generator=g, device=dev)).to(torch.bfloat16),
            q=torch.empty(LQ, C, dtype=torch.bfloat16, device=dev),
            out=torch.empty(1, LQ, H, D, dtype=torch.bfloat16, device=dev),
            cache_k=cache_k, cache_v=cache_v))
    return layers


def run_layer(L, tabs, ev=None):
    from lbw_amd import attention_segments, qk_norm_rope_
    slot = slice(LK - LQ, LK)
    if ev is not None:
        ev[0].record()
    qk_norm_rope_(L["xq"], L["xk"], None, None, L["wq"], L["wk"], tabs, EPS, H, q_out=L["q"],
                  k_out=L["cache_k"][0, slot].view(LQ, C), v=L["xv"],
                  v_out=L["cache_v"][0, slot].view(LQ, C))
    if ev is not None:
        ev[1].record()
    attention_segments(L["q"].view(1, LQ, H, D), [(L["cache_k"], L["cache_v"])], out=L["out"])
    if ev is not None:
        ev[2].record()


def cpu_baseline(budget_s: float = 12.0):
    """The oracle on the host cores: fp32 attention of the same workload, one head at a time
    until the time budget is used, scaled to TFLOP/s."""
    import torch
    import oracle as O
    torch.set_num_threads(os.cpu_count() or 1)
    g = torch.Generator().manual_seed(7)
    heads = 0
    t0 = time.perf_counter()
    while heads < H:
        q = torch.randn(1, LQ, 1, D, generator=g).to(torch.bfloat16)
        k = torch.randn(1, LK, 1, D, generator=g).to(torch.bfloat16)
        v = torch.randn(1, LK, 1, D, generator=g).to(torch.bfloat16)
        O.attention_ref(q, k, v, q_block=600)
        heads += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    dt = time.perf_counter() - t0
    flops = 4.0 * LQ * LK * D * heads
    return {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"oracle fp32 attention, {heads} of {H} heads of one layer "
                      f"({LQ} q x {LK} k x {D}), {dt:.1f} s; "
                      f"ms per 40-layer chunk extrapolated: {dt / heads * H * 40 * 1e3:.0f}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=40)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this path has no multi-GPU leg (run with --gpus 1)",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from lbw_amd import causal_rope_tables, wan_rope_freqs

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    layers = build_layers(args.layers, dev)
    tabs = causal_rope_tables(wan_rope_freqs(D), GRID, START_FRAME, device=dev)
    torch.cuda.synchronize()

    for _ in range(args.warmup):
        for L in layers:
            run_layer(L, tabs)
    torch.cuda.synchronize()

    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)]
           for _ in range(args.steps * len(layers))]
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    i = 0
    for _ in range(args.steps):
        for L in layers:
            run_layer(L, tabs, evs[i])
            i += 1
        print(f"step {_ + 1}/{args.steps} issued", file=sys.stderr, flush=True)
    stop.record()
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(stop)
    ms_step = total_ms / args.steps
    qk_ms = sum(e[0].elapsed_time(e[1]) for e in evs) / len(evs)
    attn_ms = sum(e[1].elapsed_time(e[2]) for e in evs) / len(evs)
    flops_layer = attn_flops()
    value = flops_layer * len(layers) / (ms_step / 1e3) / 1e12
    achieved = flops_layer / (attn_ms / 1e3) / 1e12

    res = {
        "metric": "chunk self-attn TFLOP/s + ms/chunk (14B shape, 720p) and % of bf16 MFMA peak",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "wan14b_720p_causal_chunk_selfattn", "layers": len(layers),
                   "heads": H, "head_dim": D, "q_tokens": LQ, "kv_tokens": LK,
                   "grid": list(GRID), "start_frame": START_FRAME,
                   "per_layer": "qk_norm_rope(+KV commit) -> chunk_attn_fwd"},
        "ms_per_chunk": round(ms_step, 3),
        "ms_per_layer": round(ms_step / len(layers), 4),
        "attn_ms_per_layer": round(attn_ms, 4),
        "qk_norm_rope_ms_per_layer": round(qk_ms, 4),
        "pct_bf16_peak": round(100.0 * value / PEAK_BF16_TFLOPS, 2),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": None,
                     "kernel": "chunk attention call (attn_fwd_kernel + split merge)",
                     "flops_per_launch": flops_layer},
    }
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(args.cpu_budget)
    print(json.dumps(res))


if __name__ == "__main__":
    main()
