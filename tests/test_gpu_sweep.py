"""A wide seeded sweep through the chunk and cross-attention kernels against the fp32 oracle:
200 random cases each, cheap enough to run in seconds.

Chunk kernel: batch 1-2, 1-4 heads, 1-777 queries (around the 32-query block and the 256-query
tile), 1-5 KV segments of 0-1500 keys (lengths around the 32-key sub-block and the 64-key tile,
empty ones included), random windows (empty ones included), per-batch k_lens, 0-7 KV splits,
both softmax forms (plain scale; q pre-scaled by log2(e)/sqrt(d) with scale ln 2), q gains
0.25-4. Cross kernel: 1-6 heads, 1-1000 queries, contexts of 1-700 rows (around the 32-key
sub-block and the 320-row resident chunk), random per-batch k_lens. V is scaled (by 1/4, 1/2) so
that |o| stays where the 1e-2 max-abs bar holds for a bf16 output. Each case prints what names
it before it runs."""
import math
import random

import pytest
import torch

import oracle as O
from parity import assert_parity

pytestmark = pytest.mark.gpu
DEV = "cuda"
N_CASES = 200


def _chunk_case(i):
    rng = random.Random(50000 + i)
    B = rng.choice([1, 1, 2])
    H = rng.randint(1, 4)
    Lq = rng.choice([1, 5, 31, 32, 33, 96, 255, 256, 257, 300, 511, 512, 513, 777])
    lens = [rng.choice([0, 1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 129, 200, 640, 1000, 1500])
            for _ in range(rng.randint(1, 5))]
    if sum(lens) == 0:
        lens[0] = 7
    tot = sum(lens)
    win = None
    if rng.random() < 0.5:
        lo = rng.randint(0, tot)
        win = (lo, rng.randint(lo, tot))
    splits = rng.choice([0, 1, 2, 3, 4, 7])
    pre = rng.random() < 0.5
    kl = [rng.randint(0, tot) for _ in range(B)] if rng.random() < 0.3 else None
    gain = rng.choice([0.25, 1.0, 4.0])
    return B, H, Lq, lens, win, splits, pre, kl, gain


def test_chunk_sweep_matches_oracle(lib):
    from lbw_amd import PRESCALED_SOFTMAX_SCALE, attention_segments, prescaled_q_scale
    for i in range(N_CASES):
        B, H, Lq, lens, win, splits, pre, kl, gain = _chunk_case(i)
        tag = (f"chunk case {i}: B={B} H={H} Lq={Lq} segs={lens} window={win} splits={splits} "
               f"prescaled={pre} k_lens={kl} gain={gain}")
        print(tag, flush=True)
        g = torch.Generator().manual_seed(i)
        q = torch.randn(B, Lq, H, 128, generator=g) * gain
        if pre:
            q = q * prescaled_q_scale(128)
        q = q.to(torch.bfloat16)
        ks = [torch.randn(B, L, H, 128, generator=g).to(torch.bfloat16) for L in lens]
        vs = [(0.25 * torch.randn(B, L, H, 128, generator=g)).to(torch.bfloat16) for L in lens]
        lo, hi = (None, None) if win is None else win
        klt = None if kl is None else torch.tensor(kl, dtype=torch.int32)
        out = attention_segments(q.to(DEV), [(k.to(DEV), v.to(DEV)) for k, v in zip(ks, vs)],
                                 kv_lo=lo, kv_hi=hi, num_splits=splits,
                                 k_lens=None if klt is None else klt.to(DEV),
                                 softmax_scale=PRESCALED_SOFTMAX_SCALE if pre else None)
        ref = O.attention_ref(q, torch.cat(ks, 1), torch.cat(vs, 1), kv_lo=lo, kv_hi=hi,
                              k_lens=klt, softmax_scale=math.log(2.0) if pre else None)
        assert_parity(out, ref, tag)


def test_cross_sweep_matches_oracle(lib):
    from lbw_amd import cross_attention
    for i in range(N_CASES):
        rng = random.Random(60000 + i)
        B = rng.choice([1, 1, 2])
        H = rng.randint(1, 6)
        Lq = rng.choice([1, 33, 255, 256, 257, 1000])
        L = rng.choice([1, 31, 32, 33, 300, 319, 320, 321, 512, 700])
        kl = None if rng.random() < 0.5 else [rng.randint(0, L) for _ in range(B)]
        tag = f"cross case {i}: B={B} H={H} Lq={Lq} L={L} k_lens={kl}"
        print(tag, flush=True)
        g = torch.Generator().manual_seed(i)
        q = torch.randn(B, Lq, H, 128, generator=g).to(torch.bfloat16)
        k = torch.randn(B, L, H, 128, generator=g).to(torch.bfloat16)
        v = (0.5 * torch.randn(B, L, H, 128, generator=g)).to(torch.bfloat16)
        klt = None if kl is None else torch.tensor(kl, dtype=torch.int32)
        out = cross_attention(q.to(DEV), k.to(DEV), v.to(DEV),
                              k_lens=None if klt is None else klt.to(DEV))
        ref = O.attention_ref(q, k, v, k_lens=klt)
        assert_parity(out, ref, tag)
