"""Seeded random shapes through the fp8-KV attention kernel (Q K^T on the fp8 matrix cores, V
staged and converted per wave): batch 1-2, 1-3 heads, 1-513 queries, 1-4 ragged fp8 segments
(lengths around the 32-key sub-block and the 64-token scale block), random windows (empty ones
included), 0-5 KV splits, q rows of magnitudes 2^-8 .. 2^2, V with 1 % outliers; every other
case with q pre-scaled by log2(e)/sqrt(128) and softmax scale ln 2 (the folded instances).

Against the oracle on the dequantised K/V: the fp32 output within the row bound its arithmetic
fixes (P's bf16 rounding plus the fp8 matrix cores' score error, see test_gpu_fp8), and the bf16
output equal to the round-to-nearest-even of the fp32 one (the same kernel, plan and merge; only
the output type differs)."""
import math
import random

import pytest
import torch

import oracle as O
from test_gpu_fp8 import _outliers, _row_bound, _score_err

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(i):
    rng = random.Random(2000 + i)
    B = rng.choice([1, 1, 2])
    H = rng.randint(1, 3)
    Lq = rng.choice([1, 17, 100, 255, 257, 513])
    lens = [rng.choice([1, 31, 33, 64, 65, 200, 640, 900]) for _ in range(rng.randint(1, 4))]
    tot = sum(lens)
    win = None
    if rng.random() < 0.4:
        lo = rng.randint(0, tot)
        win = (lo, rng.randint(lo, tot))
    splits = rng.choice([0, 1, 2, 3, 5])
    return B, H, Lq, lens, win, splits


@pytest.mark.parametrize("i", range(24))
def test_fp8_random_shape_within_kernel_bound(lib, i):
    from lbw_amd import attention_fp8kv, quantize_kv_fp8
    B, H, Lq, lens, win, splits = _case(i)
    print(f"case {i}: B={B} H={H} Lq={Lq} segs={lens} window={win} splits={splits}", flush=True)
    g = torch.Generator().manual_seed(3000 + i)
    q = torch.randn(B, Lq, H, 128, generator=g)
    q = (q * torch.exp2(torch.randint(-8, 3, (B, Lq, H, 1), generator=g).float())).to(torch.bfloat16)
    segs, kds, vds = [], [], []
    for L in lens:
        k = _outliers(torch.randn(B, L, H, 128, generator=g), g).to(torch.bfloat16)
        v = _outliers(torch.randn(B, L, H, 128, generator=g), g).to(torch.bfloat16)
        kq, vq = quantize_kv_fp8(k.to(DEV)), quantize_kv_fp8(v.to(DEV))
        segs.append((kq, vq))
        kds.append(O.dequantize_kv_fp8(kq.codes.cpu(), kq.scales.cpu()))
        vds.append(O.dequantize_kv_fp8(vq.codes.cpu(), vq.scales.cpu()))
    lo, hi = (None, None) if win is None else win
    scale, kw = 128 ** -0.5, {}
    if i % 2 == 1:
        from lbw_amd import PRESCALED_SOFTMAX_SCALE, prescaled_q_scale
        q = (q.float() * prescaled_q_scale(128)).to(torch.bfloat16)
        scale, kw = math.log(2.0), {"softmax_scale": PRESCALED_SOFTMAX_SCALE}
    qd = q.to(DEV)
    o32 = attention_fp8kv(qd, segs, kv_lo=lo, kv_hi=hi, num_splits=splits, out_dtype=torch.float32,
                          **kw)
    o16 = attention_fp8kv(qd, segs, kv_lo=lo, kv_hi=hi, num_splits=splits, **kw)
    torch.cuda.synchronize()
    kd, vd = torch.cat(kds, 1), torch.cat(vds, 1)
    ref = O.attention_ref(q, kd, vd, kv_lo=lo, kv_hi=hi, softmax_scale=scale)
    a, b = (0, sum(lens)) if win is None else win
    if b > a:
        bound = _row_bound(vd[:, a:b], _score_err(q, kd[:, a:b], scale))
    else:
        bound = torch.full((B, Lq, H), 1e-5)   # no keys: the output is exactly 0
    err = (o32.cpu() - ref).abs().amax(-1)
    print(f"  max err {float(err.max()):.3e}, worst err/bound {float((err / bound).max()):.3f}")
    assert bool((err <= bound).all())
    assert torch.equal(o16.cpu(), o32.cpu().to(torch.bfloat16))
