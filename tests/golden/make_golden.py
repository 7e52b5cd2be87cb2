"""Writes the golden fixtures of the attention path (inputs and expected outputs) from the
oracle, plus the reference's published chunk-routing table.

    python tests/golden/make_golden.py        # rewrites tests/golden/*.npz, *.json

bf16 tensors are stored as their uint16 bit patterns (numpy has no bf16). Every fixture is
small (well under 1 MB) and loads with numpy's default ``allow_pickle=False``.
"""
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle as O  # noqa: E402

# wan/modules/chunked_kv_cache.py:54-59: window_size=12 / chunk_size=3 -> n_chunks=4
REFERENCE_ROUTING_TABLE = [
    [0, 0, []], [1, 1, [0]], [2, 2, [0, 1]], [3, 3, [0, 1, 2]], [4, 1, [0, 2, 3]],
    [5, 2, [0, 1, 3]],
]


def bits(t):
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def attention_fixture():
    g = torch.Generator().manual_seed(101)
    B, Lq, Lk, H, D = 1, 40, 150, 2, 128
    q = torch.randn(B, Lq, H, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Lk, H, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Lk, H, D, generator=g).to(torch.bfloat16)
    lo, hi = 13, 140
    out = O.attention_ref(q, k, v, kv_lo=lo, kv_hi=hi)
    # cross-attention form: two batches, per-batch valid key counts
    qc = torch.randn(2, 24, H, D, generator=g).to(torch.bfloat16)
    kc = torch.randn(2, 96, H, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(2, 96, H, D, generator=g).to(torch.bfloat16)
    k_lens = [70, 33]
    outc = O.attention_ref(qc, kc, vc, k_lens=k_lens)
    np.savez_compressed(os.path.join(HERE, "attention.npz"), q=bits(q), k=bits(k), v=bits(v),
                        kv_lo=lo, kv_hi=hi, out=out.numpy(), qc=bits(qc), kc=bits(kc),
                        vc=bits(vc), k_lens=np.array(k_lens, np.int32), outc=outc.numpy())


def qk_fixture():
    g = torch.Generator().manual_seed(102)
    grid, start_frame, heads, C = (2, 3, 4), 5, 2, 256
    L = grid[0] * grid[1] * grid[2] + 5                 # 5 rows past the grid: not rotated
    q = (torch.randn(L, C, generator=g) * 1.5).to(torch.bfloat16)
    k = (torch.randn(L, C, generator=g) * 1.5).to(torch.bfloat16)
    bq = (torch.randn(C, generator=g) * 0.2).to(torch.bfloat16)
    bk = (torch.randn(C, generator=g) * 0.2).to(torch.bfloat16)
    wq = (1 + 0.1 * torch.randn(C, generator=g)).to(torch.bfloat16)
    wk = (1 + 0.1 * torch.randn(C, generator=g)).to(torch.bfloat16)
    cos, sin = O.causal_rope_grids(O.wan_rope_freqs(C // heads), *grid, start_frame=start_frame)
    qo = O.qk_post_norm_rope(q, bq, wq, cos, sin, 1e-6, heads)
    ko = O.qk_post_norm_rope(k, bk, wk, cos, sin, 1e-6, heads)
    np.savez_compressed(os.path.join(HERE, "qk_norm_rope.npz"), q=bits(q), k=bits(k), bq=bits(bq),
                        bk=bits(bk), wq=bits(wq), wk=bits(wk), grid=np.array(grid, np.int32),
                        start_frame=start_frame, heads=heads, eps=np.float32(1e-6),
                        q_out=bits(qo), k_out=bits(ko))


def fp8_fixture():
    g = torch.Generator().manual_seed(103)
    x = torch.randn(1, 150, 2, 128, generator=g)
    m = torch.rand(x.shape, generator=g) < 0.01
    sgn = torch.where(torch.rand(x.shape, generator=g) < 0.5, -1.0, 1.0)
    x = torch.where(m, 8.0 * sgn, x).to(torch.bfloat16)
    codes, scales = O.quantize_kv_fp8(x)
    np.savez_compressed(os.path.join(HERE, "kv_quant_fp8.npz"), x=bits(x), codes=codes.numpy(),
                        scales=scales.numpy())


def cache_plans_fixture():
    routing = [[i, *O.chunk_routing(i, 4)] for i in range(12)]
    routing = [[i, d, list(lead)] for i, d, lead in routing]
    assert routing[:6] == REFERENCE_ROUTING_TABLE
    # a windowed flat cache: 4 frames of 60 tokens, a 1-frame sink, 9 chunks of one frame
    kv, sink, frame = 240, 60, 60
    ge = le = 0
    plans = []
    for c in range(9):
        p = O.flat_cache_write_plan(kv, ge, le, c * frame, frame, sink, kv)
        plans.append({"chunk": c, **{k: (list(v) if isinstance(v, tuple) else v)
                                      for k, v in p.items()}})
        ge, le = p["global_end"], p["local_end"]
    with open(os.path.join(HERE, "cache_plans.json"), "w") as f:
        json.dump({"reference_routing_table_n4": REFERENCE_ROUTING_TABLE,
                   "routing_n4": routing,
                   "flat_plan": {"kv_cache_size": kv, "sink_tokens": sink, "frame": frame,
                                 "plans": plans}}, f, indent=1)


if __name__ == "__main__":
    attention_fixture()
    qk_fixture()
    fp8_fixture()
    cache_plans_fixture()
    print("fixtures written to", HERE)
