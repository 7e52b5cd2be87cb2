"""Seeded random shapes through the chunk attention kernel, both softmax pairings (plain scale:
the FMA form; q pre-scaled by log2(e)/sqrt(d) with scale ln 2: the folded form), against the fp32
oracle: batch 1-2, 1-5 heads, 1-700 queries, 1-4 ragged KV segments (empty ones included),
random windows (empty ones included), 0-5 KV splits, head gains 0.25-16. V is scaled by 1/4 so
that |o| stays below 1, where the 1e-2 max-abs bound holds for a kernel with bf16 P and a bf16
output (at |o| near 2 one output rounding alone costs up to 0.0078)."""
import math
import random

import pytest
import torch

import oracle as O
from parity import assert_parity

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _case(i):
    rng = random.Random(1000 + i)
    B = rng.choice([1, 1, 2])
    H = rng.randint(1, 5)
    Lq = rng.choice([1, 17, 100, 255, 256, 257, 513, 700])
    lens = [rng.choice([0, 1, 31, 64, 65, 200, 640, 900]) for _ in range(rng.randint(1, 4))]
    if sum(lens) == 0:
        lens[0] = 5
    tot = sum(lens)
    win = None
    if rng.random() < 0.4:
        lo = rng.randint(0, tot)
        win = (lo, rng.randint(lo, tot))
    splits = rng.choice([0, 1, 2, 3, 5])
    pre = i % 2 == 1
    gains = [rng.choice([0.25, 1.0, 4.0, 16.0]) for _ in range(H)]
    return B, H, Lq, lens, win, splits, pre, gains


@pytest.mark.parametrize("i", range(30))
def test_random_shape_matches_oracle(lib, i):
    from lbw_amd import PRESCALED_SOFTMAX_SCALE, attention_segments, prescaled_q_scale
    B, H, Lq, lens, win, splits, pre, gains = _case(i)
    g = torch.Generator().manual_seed(i)
    q = torch.randn(B, Lq, H, 128, generator=g) * torch.tensor(gains).view(1, 1, H, 1)
    if pre:
        q = q * prescaled_q_scale(128)
    q = q.to(torch.bfloat16)
    ks = [torch.randn(B, L, H, 128, generator=g).to(torch.bfloat16) for L in lens]
    vs = [(0.25 * torch.randn(B, L, H, 128, generator=g)).to(torch.bfloat16) for L in lens]
    lo, hi = (None, None) if win is None else win
    out = attention_segments(q.to(DEV), [(k.to(DEV), v.to(DEV)) for k, v in zip(ks, vs)],
                             kv_lo=lo, kv_hi=hi, num_splits=splits,
                             softmax_scale=PRESCALED_SOFTMAX_SCALE if pre else None)
    ref = O.attention_ref(q, torch.cat(ks, 1), torch.cat(vs, 1), kv_lo=lo, kv_hi=hi,
                          softmax_scale=math.log(2.0) if pre else None)
    assert_parity(out, ref, f"case {i}: B={B} H={H} Lq={Lq} segs={lens} window={win} "
                            f"splits={splits} prescaled={pre}")
