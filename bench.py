"""Benchmark of the causal-chunk attention hot path on one MI355X.

Workload (one step = one chunk's attention cost across a full Wan-14B DiT forward):
  Wan-14B shape, 720p, 1 latent frame per chunk (45 x 80 patch grid = 3600 queries) over
  12 cached frames + the chunk (46800 keys), 40 heads x 128, 40 layers with distinct buffers,
  back to back on one stream. Per layer: fused q/k RMSNorm + 3-D RoPE (writing the chunk's
  K and V into its cache slot), then flash attention of the 3600 queries over the cache.
Synthetic N(0,1) inputs, random RMSNorm gammas. Metric: attention TFLOP/s (4 Lq Lk D H per
layer, softmax excluded) over the whole timed step, plus ms per chunk.

Usage: python bench.py [--steps K] [--warmup W] [--layers N] [--no-cpu]

HBM traffic of the attention call (roofline.traffic) comes from two rocprofv3 --pmc passes
over ``bench.py --pmc-workload`` (FETCH_SIZE, then WRITE_SIZE), scaled by what the same counter
reads for a plain 1 GiB copy in the same program, and summarised by
``bench.py --pmc-summarize FETCH_DIR WRITE_DIR`` into profiles/; bench.py reports it when that
summary is present.
"""
from __future__ import annotations

import argparse
import csv
import glob
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
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "attn_fwd_bf16_wan14b_720p_traffic.txt")
COPY_BYTES = 1 << 30


def attn_flops() -> float:
    return 4.0 * LQ * LK * D * H


def attn_bytes() -> float:
    """Algorithmic HBM bytes of one attention call: Q and O [LQ, H, D] plus K and V [LK, H, D],
    bf16, each touched once."""
    return 2.0 * (2 * LQ + 2 * LK) * H * D


def qk_bytes() -> float:
    """Algorithmic HBM bytes of one fused q/k norm + RoPE call: q, k, v rows read, q', k', v
    written (bf16), plus the two gamma vectors and the RoPE tables (negligible)."""
    return 2.0 * 6 * LQ * C + 2 * 2 * C


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
    from lbw_amd import PRESCALED_SOFTMAX_SCALE, attention_segments, prescaled_q_scale, qk_norm_rope_
    slot = slice(LK - LQ, LK)
    if ev is not None:
        ev[0].record()
    qk_norm_rope_(L["xq"], L["xk"], None, None, L["wq"], L["wk"], tabs, EPS, H, q_out=L["q"],
                  k_out=L["cache_k"][0, slot].view(LQ, C), v=L["xv"],
                  v_out=L["cache_v"][0, slot].view(LQ, C), q_scale=prescaled_q_scale(D))
    if ev is not None:
        ev[1].record()
    # q carries log2(e)/sqrt(D) (the reference's pre-scaled q, model_fast.py:1233): folded softmax
    attention_segments(L["q"].view(1, LQ, H, D), [(L["cache_k"], L["cache_v"])], out=L["out"],
                       softmax_scale=PRESCALED_SOFTMAX_SCALE)
    if ev is not None:
        ev[2].record()


def _cpu_model() -> str:
    """The host CPU's model name (first /proc/cpuinfo entry) and its logical CPU count."""
    name = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return f"{name} ({os.cpu_count()} logical CPUs visible)"


def _cpu_attention_heads(g, heads, lq, lk, budget_s, fp8=False, valid=None):
    """The oracle's fp32 attention of `heads` heads (lq queries over lk keys, bf16 inputs), one
    head at a time until `budget_s` is used; with `fp8` the keys and values go through the
    oracle's e4m3 quantiser and are dequantised first (what the fp8 cache holds); `valid`
    masks the keys to a valid length (the masked cross-attention). Returns (heads done, s)."""
    import torch
    import oracle as O
    done, spent = 0, 0.0
    kl = None if valid is None else torch.tensor([valid], dtype=torch.int32)
    while done < heads:
        q = torch.randn(1, lq, 1, D, generator=g).to(torch.bfloat16)
        k = torch.randn(1, lk, 1, D, generator=g).to(torch.bfloat16)
        v = torch.randn(1, lk, 1, D, generator=g).to(torch.bfloat16)
        if fp8:   # (the quantiser is not timed: the attention reads the dequantised cache)
            k = O.dequantize_kv_fp8(*O.quantize_kv_fp8(k.float()))
            v = O.dequantize_kv_fp8(*O.quantize_kv_fp8(v.float()))
        t0 = time.perf_counter()
        O.attention_ref(q, k, v, k_lens=kl, q_block=600)
        spent += time.perf_counter() - t0
        done += 1
        if spent >= budget_s:
            break
    return done, spent


def _cpu_qk_norm_rope(g, lq, grid, start_frame, heads):
    """The oracle's q/k RMSNorm + 3-D RoPE (qk_post arithmetic) of one chunk, q and k, in
    seconds."""
    import torch
    import oracle as O
    C = heads * D
    xq = torch.randn(lq, C, generator=g).to(torch.bfloat16)
    xk = torch.randn(lq, C, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(C, generator=g)).to(torch.bfloat16)
    t0 = time.perf_counter()
    cos, sin = O.causal_rope_grids(O.wan_rope_freqs(D), *grid, start_frame=start_frame)
    O.qk_post_norm_rope(xq, None, w, cos, sin)
    O.qk_post_norm_rope(xk, None, w, cos, sin)
    return time.perf_counter() - t0


def _cpu_c1_layer(g):
    """One whole Wan-1.3B self-attention layer in fp32 on the host (the oracle's layer: QKV
    projections, RMSNorm, 3-D RoPE, attention over 2 cached frames + the chunk, o-projection),
    480p, one latent frame of 1560 tokens; seconds and FLOP."""
    import torch
    import oracle as O
    C1, H1, grid = 1536, 12, (1, 30, 52)
    L = grid[1] * grid[2]
    rn = lambda *s, sc=1.0: (sc * torch.randn(*s, generator=g))
    x, xc = rn(1, L, C1), rn(1, 2 * L, C1)
    w = [rn(C1, C1, sc=0.02) for _ in range(4)]
    b = [rn(C1, sc=0.02) for _ in range(4)]
    gq, gk = 1 + 0.1 * rn(C1), 1 + 0.1 * rn(C1)
    t0 = time.perf_counter()
    O.self_attention_layer_ref(x, xc, w[0], b[0], w[1], b[1], w[2], b[2], w[3], b[3], gq, gk,
                               heads=H1, grid=grid, cache_grid=(2, 30, 52), start_frame=2)
    dt = time.perf_counter() - t0
    flops = 2.0 * L * C1 * C1 * 4 + 2.0 * 2 * L * C1 * C1 * 2 + 4.0 * L * 3 * L * (C1 // H1) * H1
    return dt, flops


def cpu_baseline(budget_s: float = 12.0):
    """The oracle on the host cores: fp32 attention of the same workload (the 14B 720p chunk),
    one head at a time until the time budget is used, scaled to TFLOP/s; and, under
    ``per_config``, every other workload of the path on a bounded sample (whole c1 layer;
    attention and q/k norm + RoPE per layer at the 1.3B / 14B 480p chunks, the cross-attention
    and the fp8-cache long horizon), each extrapolated to one layer."""
    import torch
    torch.set_num_threads(os.cpu_count() or 1)
    g = torch.Generator().manual_seed(7)
    heads, dt = _cpu_attention_heads(g, H, LQ, LK, budget_s)
    flops = 4.0 * LQ * LK * D * heads
    res = {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": torch.get_num_threads(),
           "cpu_model": _cpu_model(), "kind": "port",
           "sample": f"oracle fp32 attention, {heads} of {H} heads of one layer "
                     f"({LQ} q x {LK} k x {D}), {dt:.1f} s; "
                     f"ms per 40-layer chunk extrapolated: {dt / heads * H * 40 * 1e3:.0f}"}
    per = {}
    t, fl = _cpu_c1_layer(g)
    per["wan13b_480p_1f_over_2f_full_layer"] = {
        "ms_per_layer": round(t * 1e3, 1), "TFLOP/s": round(fl / t / 1e12, 4),
        "sample": "whole layer (projections, norm, RoPE, attention, o-projection), fp32"}
    for name, h, lq, lk, grid, sf, kw in (
            ("wan13b_480p_3f_over_6f", 12, 4680, 14040, (3, 30, 52), 6, {}),
            ("wan14b_480p_3f_over_18f", 40, 4680, 32760, (3, 30, 52), 18, {}),
            ("wan14b_480p_cross_512ctx_300valid", 40, 4680, 512, None, 0, {"valid": 300}),
            ("wan14b_480p_cross_512ctx_unmasked", 40, 4680, 512, None, 0, {}),
            ("wan14b_720p_1f_over_24f_fp8kv", 40, 3600, 90000, (1, 45, 80), 24, {"fp8": True})):
        n, ta = _cpu_attention_heads(g, h, lq, lk, 1.5, **kw)
        nk = kw.get("valid", lk)
        fl = 4.0 * lq * nk * D * n
        ent = {"attention_ms_per_layer": round(ta / n * h * 1e3, 1),
               "attention_TFLOP/s": round(fl / ta / 1e12, 4),
               "sample": f"{n} of {h} heads, extrapolated"}
        if grid is not None:
            ent["qk_norm_rope_ms_per_layer"] = round(_cpu_qk_norm_rope(g, lq, grid, sf, h) * 1e3, 1)
        per[name] = ent
    res["per_config"] = per
    return res


_SLEEP_CYCLES_PER_MS = []


def _gpu_busy(ms: float):
    """Queue about ``ms`` of GPU spinning (torch.cuda._sleep, a bounded clock loop) on the
    current stream, calibrated once with events."""
    import torch
    if not _SLEEP_CYCLES_PER_MS:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        torch.cuda._sleep(1_000_000)
        e1.record()
        torch.cuda.synchronize()
        _SLEEP_CYCLES_PER_MS.append(1_000_000 / max(e0.elapsed_time(e1), 1e-3))
    torch.cuda._sleep(int(_SLEEP_CYCLES_PER_MS[0] * ms))


def _time_ms(fn, iters=10, warmup=2, reps=5):
    """GPU time per call of ``fn``: the median over ``reps`` repetitions of ``iters`` calls back
    to back (single 10-call averages of one shape spread by 5-10 % from one repetition to the
    next). The GPU is kept busy while the host queues each repetition's calls, so that the
    Python/ctypes time between launches of a short kernel is not counted."""
    import torch
    host_ms = 1.0
    for _ in range(max(warmup, 2)):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        host_ms = (time.perf_counter() - t0) * 1e3   # host time of one launch (the last one)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    per_call = []
    for _ in range(reps):
        _gpu_busy(min(2.0 + 2.0 * host_ms * iters, 500.0))
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        per_call.append(e0.elapsed_time(e1) / iters)
    per_call.sort()
    return per_call[len(per_call) // 2]


def other_configs(dev):
    """The other workload shapes of this path, timed once each after the headline step (not
    part of `value`): 1.3B 480p 3-frame chunk over 6 cached frames, 14B 480p 3-frame chunk over
    18 cached frames, its cross-attention to a 512-token context (300 valid), and the 14B 720p
    long-horizon chunk over an fp8-e4m3 cache of 24 frames + the chunk. The self-attention
    calls take q pre-scaled as the layer pipeline's fused q/k kernel writes it, with the
    plain-scaled call beside it."""
    import torch
    from lbw_amd import attention_fp8kv, attention_segments, cross_attention, quantize_kv_fp8
    g = torch.Generator(device=dev).manual_seed(99)
    rnd = lambda *s: torch.randn(*s, generator=g, device=dev).to(torch.bfloat16)
    out = {}
    # q pre-scaled as the fused q/k kernel writes it in the layer pipeline (the folded softmax,
    # as in the headline step), and the same call on a plain-scaled q
    from lbw_amd import PRESCALED_SOFTMAX_SCALE, prescaled_q_scale
    for name, h, lq, lc in (("wan13b_480p_3f_over_6f", 12, 4680, 9360),
                            ("wan14b_480p_3f_over_18f", 40, 4680, 28080)):
        q = rnd(1, lq, h, D)
        qs = (q.float() * prescaled_q_scale(D)).to(torch.bfloat16)
        kc, vc, kn, vn = rnd(1, lc, h, D), rnd(1, lc, h, D), rnd(1, lq, h, D), rnd(1, lq, h, D)
        o = torch.empty_like(q)
        ms = _time_ms(lambda: attention_segments(qs, [(kc, vc), (kn, vn)], out=o,
                                                 softmax_scale=PRESCALED_SOFTMAX_SCALE))
        ms_plain = _time_ms(lambda: attention_segments(q, [(kc, vc), (kn, vn)], out=o))
        fl = 4.0 * lq * (lc + lq) * D * h
        out[name] = {"ms": round(ms, 4), "TFLOP/s": round(fl / ms / 1e9, 1),
                     "pct_bf16_peak": round(fl / ms / 1e9 / PEAK_BF16_TFLOPS * 100, 2),
                     "ms_plain_scale_q": round(ms_plain, 4),
                     "pct_bf16_peak_plain_scale_q": round(fl / ms_plain / 1e9 / PEAK_BF16_TFLOPS * 100, 2)}
        del q, qs, kc, vc, kn, vn
    q = rnd(1, 4680, 40, D)
    kx, vx = rnd(1, 512, 40, D), rnd(1, 512, 40, D)
    kl = torch.tensor([300], dtype=torch.int32, device=dev)
    kx[:, 300:] = kx[:, 511:]   # identical padding rows, as the projected zero padding gives
    vx[:, 300:] = vx[:, 511:]
    for name, lens, nk, nd in (("wan14b_480p_cross_512ctx_300valid", kl, 300, None),
                               ("wan14b_480p_cross_512ctx_unmasked", None, 512, None),
                               ("wan14b_480p_cross_512ctx_unmasked_dedup", None, 512, 300)):
        ms = _time_ms(lambda: cross_attention(q, kx, vx, k_lens=lens, n_distinct=nd), iters=20)
        fl = 4.0 * 4680 * nk * D * 40
        by = 2.0 * (2 * 4680 + 2 * nk) * 40 * D
        out[name] = {"ms": round(ms, 4), "TFLOP/s": round(fl / ms / 1e9, 1),
                     "GB/s": round(by / ms / 1e6, 1),
                     "pct_bf16_peak": round(fl / ms / 1e9 / PEAK_BF16_TFLOPS * 100, 2),
                     "pct_hbm_peak": round(by / ms / 1e6 / PEAK_HBM_GBS * 100, 2)}
    del q, kx, vx
    # q pre-scaled as the fused q/k kernel writes it (the folded softmax), as in the headline
    # step; the same call on a plain-scaled q, and on a bf16 cache of the same keys
    q = rnd(1, 3600, 40, D)
    qs = (q.float() * prescaled_q_scale(D)).to(torch.bfloat16)
    lk = 3600 * 25
    kb, vb = rnd(1, lk, 40, D), rnd(1, lk, 40, D)
    k8, v8 = quantize_kv_fp8(kb), quantize_kv_fp8(vb)
    o = torch.empty_like(q)
    ms = _time_ms(lambda: attention_fp8kv(qs, [(k8, v8)], softmax_scale=PRESCALED_SOFTMAX_SCALE,
                                          out=o))
    ms_plain = _time_ms(lambda: attention_fp8kv(q, [(k8, v8)], out=o))
    ms_bf16 = _time_ms(lambda: attention_segments(qs, [(kb, vb)],
                                                  softmax_scale=PRESCALED_SOFTMAX_SCALE, out=o))
    fl = 4.0 * 3600 * lk * D * 40
    out["wan14b_720p_1f_over_24f_fp8kv"] = {
        "ms": round(ms, 4), "TFLOP/s": round(fl / ms / 1e9, 1),
        "pct_fp8_peak": round(fl / ms / 1e9 / PEAK_FP8_TFLOPS * 100, 2),
        "pct_bf16_peak": round(fl / ms / 1e9 / PEAK_BF16_TFLOPS * 100, 2),
        "ms_plain_scale_q": round(ms_plain, 4), "ms_bf16_cache_same_keys": round(ms_bf16, 4)}
    del q, qs, kb, vb, k8, v8
    # fused q/k norm + RoPE with head-major d-major outputs [H, D, L] (q scaled by 1/sqrt(D)),
    # 14B 720p chunk; four input/output sets in turn so that the MALL does not serve the reads
    from lbw_amd import causal_rope_tables, qk_norm_rope_, wan_rope_freqs
    tabs = causal_rope_tables(wan_rope_freqs(D), GRID, START_FRAME, device=dev)
    w = (1 + 0.1 * torch.randn(C, generator=g, device=dev)).to(torch.bfloat16)
    sets = [(rnd(LQ, C), rnd(LQ, C), torch.empty(H, D, LQ, dtype=torch.bfloat16, device=dev),
             torch.empty(H, D, LQ, dtype=torch.bfloat16, device=dev)) for _ in range(4)]
    turn = [0]

    def qk_t():
        xq, xk, oq, ok = sets[turn[0] % len(sets)]
        turn[0] += 1
        qk_norm_rope_(xq, xk, None, None, w, w, tabs, EPS, H, q_out=oq, k_out=ok,
                      q_scale=1.0 / math.sqrt(D), layout="dmajor")
    ms = _time_ms(qk_t, iters=40)
    by = 2.0 * 4 * LQ * C
    out["wan14b_720p_qk_norm_rope_t_dmajor"] = {
        "ms": round(ms, 4), "GB/s": round(by / ms / 1e6, 1),
        "pct_hbm_peak": round(by / ms / 1e6 / PEAK_HBM_GBS * 100, 2)}
    del sets
    # the whole self-attention of one 14B block at the 720p chunk: fused QKV GEMM (hipBLASLt,
    # V bias in its epilogue) -> fused q/k norm + RoPE + KV commit -> attention over the
    # 46800-token flat cache -> o-projection GEMM; random-init weights N(0, 0.02)
    from lbw_amd import FlatKVCache, WanSelfAttention
    wts = [(0.02 * torch.randn(C, C, generator=g, device=dev)).to(torch.bfloat16) for _ in range(4)]
    vec = lambda sc, off: (off + sc * torch.randn(C, generator=g, device=dev)).to(torch.bfloat16)
    layer = WanSelfAttention(wts[0], vec(0.02, 0), wts[1], vec(0.02, 0), wts[2], vec(0.02, 0),
                             wts[3], vec(0.02, 0), vec(0.1, 1.0), vec(0.1, 1.0), heads=H)
    cache = FlatKVCache(1, LK, H, D, device=dev, local_attn_size=-1)
    cache.k.copy_(rnd(1, LK, H, D))
    cache.v.copy_(rnd(1, LK, H, D))
    x = rnd(1, LQ, C)
    start = LK - LQ

    def layer_fwd():
        cache.global_end = cache.local_end = start
        layer.forward(x, GRID, START_FRAME, cache, start)
    ms = _time_ms(layer_fwd, iters=10)
    fl_proj = 4 * 2.0 * LQ * C * C
    fl = attn_flops() + fl_proj
    out["wan14b_720p_selfattn_layer_with_projections"] = {
        "ms": round(ms, 4), "TFLOP/s": round(fl / ms / 1e9, 1),
        "pct_bf16_peak": round(fl / ms / 1e9 / PEAK_BF16_TFLOPS * 100, 2),
        "projection_TFLOP": round(fl_proj / 1e12, 4)}
    return out


def boundary_costs(dev):
    """Host cost of the Python -> torch.ops.lbw -> C ABI boundary, without padding the GPU queue:
    ``host_us`` = host time to issue one call while the GPU is busy with earlier work (what the
    boundary adds on the CPU), ``eager_us`` = wall time per call of back-to-back calls from an idle
    GPU to the last one's end (what a caller waiting on each call sees), ``gpu_us`` = GPU time
    per call. For the c4 chunk attention, the same call through the no-alloc C entry point (whose
    fixed 64 MiB scratch holds no split partials at this size, so it runs one pass), and the 14B
    480p cross-attention (300-row mask)."""
    import ctypes
    import torch
    from lbw_amd import PRESCALED_SOFTMAX_SCALE, _lib, attention_segments, cross_attention
    g = torch.Generator(device=dev).manual_seed(3)
    rnd = lambda *s: torch.randn(*s, generator=g, device=dev).to(torch.bfloat16)
    q = rnd(1, LQ, H, D)
    kc, vc = rnd(1, LK, H, D), rnd(1, LK, H, D)
    out = torch.empty_like(q)
    qx = rnd(1, 4680, 40, D)
    kx, vx = rnd(1, 512, 40, D), rnd(1, 512, 40, D)
    kl = torch.tensor([300], dtype=torch.int32, device=dev)
    lib = _lib.load()
    p_na = _lib.attn_params(q, out, [(kc, vc)], softmax_scale=PRESCALED_SOFTMAX_SCALE)
    calls = {
        "chunk_attention_wan14b_720p": (lambda: attention_segments(
            q, [(kc, vc)], out=out, softmax_scale=PRESCALED_SOFTMAX_SCALE), 10),
        "chunk_attention_wan14b_720p_noalloc": (lambda: _lib.check(
            lib.lbw_attention_fwd_noalloc(ctypes.byref(p_na), _lib.stream_ptr()), "noalloc"), 10),
        "cross_attention_wan14b_480p_300valid": (lambda: cross_attention(qx, kx, vx, k_lens=kl), 50),
    }
    res = {}
    for name, (fn, n) in calls.items():
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        # host issue time: queue a long spin first, so no call waits on the GPU
        _gpu_busy(200.0)
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        host = (time.perf_counter() - t0) / n * 1e6
        torch.cuda.synchronize()
        # eager wall time from an idle GPU
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        eager = (time.perf_counter() - t0) / n * 1e6
        gpu = _time_ms(fn, iters=n) * 1e3
        res[name] = {"host_us": round(host, 1), "eager_us": round(eager, 1), "gpu_us": round(gpu, 1)}
    return res


def pmc_workload():
    """The program the --pmc passes profile: 3 layers' qk-norm/RoPE + attention calls of the
    workload, then 3 plain copies of COPY_BYTES (calibration of the byte counters)."""
    import torch
    from lbw_amd import causal_rope_tables, wan_rope_freqs
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    layers = build_layers(1, dev)
    tabs = causal_rope_tables(wan_rope_freqs(D), GRID, START_FRAME, device=dev)
    src = torch.empty(COPY_BYTES // 2, dtype=torch.bfloat16, device=dev).normal_()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        run_layer(layers[0], tabs)
    torch.cuda.synchronize()
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)     # the calibration copy: the last 3 dispatches
    torch.cuda.synchronize()
    print("pmc workload done", flush=True)


def counter_workload():
    """The program the SQ counter passes profile: 5 chunk attention calls at the workload's
    shape with q pre-scaled by log2(e)/sqrt(D) (the folded softmax), on seeded inputs."""
    import torch
    from lbw_amd import PRESCALED_SOFTMAX_SCALE, attention_segments, prescaled_q_scale
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    q = (torch.randn(1, LQ, H, D, generator=g, device=dev) * prescaled_q_scale(D)).to(torch.bfloat16)
    k = torch.randn(1, LK, H, D, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(1, LK, H, D, generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    for _ in range(5):
        attention_segments(q, [(k, v)], out=out, softmax_scale=PRESCALED_SOFTMAX_SCALE)
    torch.cuda.synchronize()
    print("counter workload done", flush=True)


def cross_workload():
    """The program the cross-attention profiles run: 5 calls each of the 14B 480p
    cross-attention (4680 q x 40 heads over a 512-row context, rows 300.. identical) masked to
    300 rows, unmasked (512 keys) and the exact dedup, on seeded inputs; then 5 calls of the
    unmasked context through the general chunk kernel (the path it took before the ring form),
    for comparison in the same trace."""
    import torch
    from lbw_amd import attention_segments, cross_attention, padding_start
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(1, 4680, 40, D, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(1, 512, 40, D, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(1, 512, 40, D, generator=g, device=dev).to(torch.bfloat16)
    k[:, 300:] = k[:, 511:]
    v[:, 300:] = v[:, 511:]
    kl = torch.tensor([300], dtype=torch.int32, device=dev)
    nd = padding_start(k, v)
    for _ in range(5):
        cross_attention(q, k, v, k_lens=kl)
    for _ in range(5):
        cross_attention(q, k, v)
    for _ in range(5):
        cross_attention(q, k, v, n_distinct=nd)
    for _ in range(5):
        attention_segments(q, [(k, v)], num_splits=1)
    torch.cuda.synchronize()
    print("cross workload done", flush=True)


def fp8_workload():
    """The program the fp8-cache profiles run: 5 calls of the 14B 720p long-horizon chunk
    (3600 q x 40 heads over 90000 keys) on an fp8-e4m3 cache, then 5 on the same keys as a bf16
    cache, on seeded inputs, q pre-scaled (the folded softmax, as in the headline step)."""
    import torch
    from lbw_amd import (PRESCALED_SOFTMAX_SCALE, attention_fp8kv, attention_segments,
                         prescaled_q_scale, quantize_kv_fp8)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(1, 3600, 40, D, generator=g, device=dev)
    q = (q * prescaled_q_scale(D)).to(torch.bfloat16)
    k = torch.randn(1, 90000, 40, D, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(1, 90000, 40, D, generator=g, device=dev).to(torch.bfloat16)
    k8, v8 = quantize_kv_fp8(k), quantize_kv_fp8(v)
    for _ in range(5):
        attention_fp8kv(q, [(k8, v8)], softmax_scale=PRESCALED_SOFTMAX_SCALE)
    for _ in range(5):
        attention_segments(q, [(k, v)], softmax_scale=PRESCALED_SOFTMAX_SCALE)
    torch.cuda.synchronize()
    print("fp8 workload done", flush=True)


def _pmc_rows(d, counter):
    """Per-dispatch values of `counter` from a rocprofv3 --pmc csv output directory."""
    files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {d}")
    rows = {}
    for f in files:
        for r in csv.DictReader(open(f)):
            if r["Counter_Name"] != counter:
                continue
            k = int(r["Dispatch_Id"])
            name, v = rows.get(k, (r["Kernel_Name"], 0.0))
            rows[k] = (name, v + float(r["Counter_Value"]))
    return [rows[k] for k in sorted(rows)]


def pmc_summarize(fetch_dir, write_dir, cmds):
    """Scale FETCH_SIZE / WRITE_SIZE (KiB per dispatch) by the calibration copy and write the
    traffic summary that bench.py reports as roofline.traffic."""
    out = {}
    for key, d, counter in (("fetch", fetch_dir, "FETCH_SIZE"), ("write", write_dir, "WRITE_SIZE")):
        rows = _pmc_rows(d, counter)
        copy = [v for _, v in rows[-3:]]
        factor = COPY_BYTES / (sum(copy) / len(copy) * 1024.0)
        out[key + "_factor"] = factor
        for tag, pat in (("attn_main", "attn_fwd_bf16"), ("attn_merge", "attn_merge"),
                         ("qk_norm_rope", "qk_norm_rope")):
            vals = [v for n, v in rows[:-3] if pat in n]
            out[f"{tag}_{key}_bytes"] = (sum(vals) / len(vals) * 1024.0 * factor) if vals else 0.0
            out[f"{tag}_dispatches"] = len(vals)
    attn = sum(out[f"attn_{p}_{k}_bytes"] for p in ("main", "merge") for k in ("fetch", "write"))
    qk = out["qk_norm_rope_fetch_bytes"] + out["qk_norm_rope_write_bytes"]
    lines = [
        "# HBM traffic per call, chunk attention at Wan-14B 720p (3600 q x 46800 k, 40 x 128, bf16)",
        "# counters: rocprofv3 --pmc FETCH_SIZE, then --pmc WRITE_SIZE, KiB per dispatch, each",
        "# scaled by (1 GiB / the counter's reading for a plain 1 GiB copy in the same program)",
        "# commands (from /tmp, TMPDIR=/tmp):",
        *[f"#   {c}" for c in cmds],
        f"fetch_factor = {out['fetch_factor']:.4f}",
        f"write_factor = {out['write_factor']:.4f}",
    ]
    for tag in ("attn_main", "attn_merge", "qk_norm_rope"):
        lines.append(f"{tag}_fetch_bytes = {out[tag + '_fetch_bytes']:.0f}")
        lines.append(f"{tag}_write_bytes = {out[tag + '_write_bytes']:.0f}")
    lines += [f"attn_algorithmic_bytes = {attn_bytes():.0f}",
              f"attn_traffic_bytes = {attn:.0f}",
              f"attn_traffic_over_algorithmic = {attn / attn_bytes():.3f}",
              f"qk_algorithmic_bytes = {qk_bytes():.0f}",
              f"qk_traffic_bytes = {qk:.0f}",
              f"qk_traffic_over_algorithmic = {qk / qk_bytes():.3f}"]
    os.makedirs(os.path.dirname(TRAFFIC_FILE), exist_ok=True)
    with open(TRAFFIC_FILE, "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))


def load_traffic():
    """key = value figures of the committed traffic summary, or None."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    vals = {}
    for line in open(TRAFFIC_FILE):
        if "=" in line and not line.startswith("#"):
            k, v = line.split("=", 1)
            vals[k.strip()] = float(v)
    return vals


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=40)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the timings of the other workload shapes")
    ap.add_argument("--counter-workload", action="store_true",
                    help="5 pre-scaled chunk attention calls (the program of the SQ counter passes)")
    ap.add_argument("--cross-workload", action="store_true",
                    help="5 calls each of the 14B 480p cross-attention, masked / unmasked / dedup")
    ap.add_argument("--fp8-workload", action="store_true",
                    help="5 calls of the 14B 720p long-horizon chunk on an fp8 cache, 5 on bf16")
    ap.add_argument("--pmc-workload", action="store_true",
                    help="run the program profiled by the FETCH_SIZE / WRITE_SIZE passes")
    ap.add_argument("--pmc-summarize", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="turn the two --pmc outputs into the committed traffic summary")
    ap.add_argument("--pmc-cmd", action="append", default=[],
                    help="command lines recorded in the summary (with --pmc-summarize)")
    args = ap.parse_args()
    if args.pmc_summarize:
        pmc_summarize(*args.pmc_summarize, args.pmc_cmd)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this path has no multi-GPU leg (run with --gpus 1)",
              file=sys.stderr)
        sys.exit(2)

    if args.counter_workload:
        counter_workload()
        return
    if args.pmc_workload:
        pmc_workload()
        return
    if args.cross_workload:
        cross_workload()
        return
    if args.fp8_workload:
        fp8_workload()
        return

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
    qk_all = sorted(e[0].elapsed_time(e[1]) for e in evs)
    attn_all = sorted(e[1].elapsed_time(e[2]) for e in evs)
    qk_ms = sum(qk_all) / len(qk_all)
    attn_ms = sum(attn_all) / len(attn_all)
    pct = lambda xs, f: xs[min(len(xs) - 1, int(f * len(xs)))]
    flops_layer = attn_flops()
    value = flops_layer * len(layers) / (ms_step / 1e3) / 1e12
    achieved = flops_layer / (attn_ms / 1e3) / 1e12
    tr = load_traffic()

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
                   "per_layer": "qk_norm_rope(+KV commit, q pre-scaled by log2(e)/sqrt(128)) -> chunk_attn_fwd (softmax scale ln 2: folded softmax)"},
        "ms_per_chunk": round(ms_step, 3),
        "ms_per_layer": round(ms_step / len(layers), 4),
        "attn_ms_per_layer": round(attn_ms, 4),
        "qk_norm_rope_ms_per_layer": round(qk_ms, 4),
        "attn_ms_p10_p50_p90": [round(pct(attn_all, f), 4) for f in (0.1, 0.5, 0.9)],
        "qk_norm_rope_ms_p10_p50_p90": [round(pct(qk_all, f), 4) for f in (0.1, 0.5, 0.9)],
        "pct_bf16_peak": round(100.0 * value / PEAK_BF16_TFLOPS, 2),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": round(tr["attn_traffic_bytes"]) if tr else None,
                     "kernel": "chunk attention call (queue reset + attn_fwd_bf16_kernel, split pieces merged in-kernel)",
                     "flops_per_launch": flops_layer,
                     "algorithmic_bytes_per_launch": attn_bytes()},
        "qk_norm_rope_roofline": {"bound": "hbm",
                                  "achieved": round(qk_bytes() / (qk_ms / 1e3) / 1e9, 1),
                                  "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                  "frac": round(qk_bytes() / (qk_ms / 1e3) / 1e9 / PEAK_HBM_GBS, 4),
                                  "traffic": round(tr["qk_traffic_bytes"]) if tr else None},
    }
    if not args.no_extra:
        del layers
        torch.cuda.empty_cache()
        res["other_configs"] = other_configs(dev)
        res["boundary_costs"] = boundary_costs(dev)
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(args.cpu_budget)
    print(json.dumps(res))


if __name__ == "__main__":
    main()
