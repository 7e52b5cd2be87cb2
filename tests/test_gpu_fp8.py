"""GPU checks of the fp8-e4m3 KV path: the quantiser is bit-exact against the oracle (byte
output), and attention over the quantised cache reaches cosine >= 0.999 against the fp32
reference on the unquantised inputs (spec), plus a tighter check against the oracle run on
the dequantised K/V (the kernel's own arithmetic)."""
import pytest
import torch

import oracle as O
from parity import FP8_COSINE, cosine, metrics

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _outliers(x, g, frac=0.01, mag=8.0):
    m = torch.rand(x.shape, generator=g) < frac
    s = torch.where(torch.rand(x.shape, generator=g) < 0.5, -mag, mag)
    return torch.where(m, s, x)


@pytest.mark.parametrize("L,H", [(150, 3), (64, 1), (1000, 2)])
def test_quantizer_bit_exact(lib, L, H):
    from lbw_amd import quantize_kv_fp8
    g = torch.Generator().manual_seed(L)
    x = _outliers(torch.randn(1, L, H, 128, generator=g), g).to(torch.bfloat16)
    x[0, 3, 0, 5] = 0.0
    if L >= 128:
        x[0, 64:128, 0] = 0.0          # an all-zero block -> scale 1, codes 0
    q = quantize_kv_fp8(x.to(DEV))
    codes, scales = O.quantize_kv_fp8(x.float())
    assert torch.equal(q.scales.cpu(), scales)
    assert torch.equal(q.codes.cpu(), codes)


def test_quantizer_rounding_edges(lib):
    """Values on and next to e4m3 rounding ties, subnormals and the 448 saturation edge."""
    from lbw_amd import quantize_kv_fp8
    vals = torch.tensor([448.0, -448.0, 1.0, 1.0625, 1.125, 1.1875, 2.0 ** -6, 2.0 ** -7,
                         3 * 2.0 ** -10, 2.0 ** -10, 2.0 ** -9, 0.0, 13.0, 15.0, 17.0, 240.0,
                         232.0, 0.3, -0.3, 100.0], dtype=torch.float32)
    x = torch.zeros(1, 64, 1, 128)
    x.view(-1)[:vals.numel()] = vals
    x = x.to(torch.bfloat16)
    q = quantize_kv_fp8(x.to(DEV))
    codes, scales = O.quantize_kv_fp8(x.float())
    assert torch.equal(q.codes.cpu(), codes) and torch.equal(q.scales.cpu(), scales)


def test_quantizer_power_of_two_scale_edges(lib):
    """Block scales at their edges, bit-exact against the oracle: block maxima of exactly
    448 * 2^k (scale 2^k, code 448) and one bf16 step above (scale 2^(k+1)), mantissas at and
    past 1.75, a bf16 subnormal maximum (scale clamped to 2^-126), an all-zero block (scale 1);
    every scale a power of two."""
    from lbw_amd import quantize_kv_fp8
    maxima = [448.0, 448.0 * 2.0 ** -5, 1.75, 1.7578125, 1.0, 0.9921875, 3.0e4, 2.0 ** -130, 0.0,
              448.0 * 2.0 ** 3, 1.0e-3]
    x = torch.zeros(1, 64 * len(maxima), 2, 128)
    g = torch.Generator().manual_seed(3)
    for i, m in enumerate(maxima):
        blk = torch.rand(64, 2, 128, generator=g) * 2 - 1
        x[0, 64 * i:64 * (i + 1)] = blk * m * 0.99
        x[0, 64 * i + 5, :, 7] = m
    x = x.to(torch.bfloat16)
    q = quantize_kv_fp8(x.to(DEV))
    codes, scales = O.quantize_kv_fp8(x.float())
    assert torch.equal(q.scales.cpu(), scales) and torch.equal(q.codes.cpu(), codes)
    mant, _ = torch.frexp(scales)
    assert torch.all(mant == 0.5)
    assert float(scales[0, 0, 0]) == 1.0 and float(scales[0, 0, 1]) == 2.0 ** -5
    assert float(scales[0, 0, 7]) == 2.0 ** -126 and float(scales[0, 0, 8]) == 1.0


@pytest.mark.parametrize("Lq,H,lk,window", [(300, 2, 2000, None), (100, 3, 777, (13, 700))])
def test_fp8_attention_cosine(lib, Lq, H, lk, window):
    from lbw_amd import attention_fp8kv, quantize_kv_fp8
    g = torch.Generator().manual_seed(lk)
    q = torch.randn(1, Lq, H, 128, generator=g).to(torch.bfloat16)
    k = _outliers(torch.randn(1, lk, H, 128, generator=g), g).to(torch.bfloat16)
    v = _outliers(torch.randn(1, lk, H, 128, generator=g), g).to(torch.bfloat16)
    kq = quantize_kv_fp8(k.to(DEV))
    vq = quantize_kv_fp8(v.to(DEV))
    lo, hi = (None, None) if window is None else window
    out = attention_fp8kv(q.to(DEV), [(kq, vq)], kv_lo=lo, kv_hi=hi)
    ref = O.attention_ref(q, k, v, kv_lo=lo, kv_hi=hi)
    c = cosine(out, ref)
    m = metrics(out, ref)
    print(f"fp8 Lq={Lq} lk={lk}: cosine {c:.6f}", m)
    assert c >= FP8_COSINE and m["nonfinite"] == 0
    kd = O.dequantize_kv_fp8(kq.codes.cpu(), kq.scales.cpu())
    vd = O.dequantize_kv_fp8(vq.codes.cpu(), vq.scales.cpu())
    ref_d = O.attention_ref(q, kd, vd, kv_lo=lo, kv_hi=hi)
    assert cosine(out, ref_d) >= 0.9995


def test_fp8_attention_two_segments_unaligned(lib):
    """A cache segment plus a chunk whose length is not a multiple of the 64-token block."""
    from lbw_amd import attention_fp8kv, quantize_kv_fp8
    g = torch.Generator().manual_seed(99)
    H, Lq = 2, 200
    segs, ks, vs = [], [], []
    for L in (640, 130):
        k = torch.randn(1, L, H, 128, generator=g).to(torch.bfloat16)
        v = torch.randn(1, L, H, 128, generator=g).to(torch.bfloat16)
        ks.append(k)
        vs.append(v)
        segs.append((quantize_kv_fp8(k.to(DEV)), quantize_kv_fp8(v.to(DEV))))
    q = torch.randn(1, Lq, H, 128, generator=g).to(torch.bfloat16)
    out = attention_fp8kv(q.to(DEV), segs, kv_lo=100, kv_hi=700)
    ref = O.attention_ref(q, torch.cat(ks, 1), torch.cat(vs, 1), kv_lo=100, kv_hi=700)
    assert cosine(out, ref) >= FP8_COSINE


def test_fp8_full_size_long_horizon(lib):
    """14B 720p long horizon: 3600 q over 90000 keys (24 cached frames + 1), 40 heads, with
    1% +-8 outliers; parity on a subset of heads and rows."""
    from lbw_amd import attention_fp8kv, quantize_kv_fp8
    H, Lq, Lk = 40, 3600, 90000
    gd = torch.Generator(device=DEV).manual_seed(5)
    q = torch.randn(1, Lq, H, 128, generator=gd, device=DEV).to(torch.bfloat16)

    def kv():
        x = torch.randn(1, Lk, H, 128, generator=gd, device=DEV)
        m = torch.rand(x.shape, generator=gd, device=DEV) < 0.01
        s = torch.where(torch.rand(x.shape, generator=gd, device=DEV) < 0.5, -8.0, 8.0)
        return torch.where(m, s, x).to(torch.bfloat16)
    k, v = kv(), kv()
    kq, vq = quantize_kv_fp8(k), quantize_kv_fp8(v)
    out = attention_fp8kv(q, [(kq, vq)])
    torch.cuda.synchronize()
    sel = torch.randperm(Lq, generator=torch.Generator().manual_seed(1))[:128].sort().values
    for h in (0, 23):
        ref = O.attention_ref(q[:, sel, h:h + 1].cpu(), k[:, :, h:h + 1].cpu(), v[:, :, h:h + 1].cpu())
        c = cosine(out[:, sel, h:h + 1], ref)
        # max-abs beside the cosine: the quantised cache alone moves the output by what the
        # oracle on the dequantised K/V shows; the kernel may add its bf16 tolerance on top
        kd = O.dequantize_kv_fp8(kq.codes[:, :, h:h + 1].cpu(), kq.scales[:, h:h + 1].cpu())
        vd = O.dequantize_kv_fp8(vq.codes[:, :, h:h + 1].cpu(), vq.scales[:, h:h + 1].cpu())
        ref_d = O.attention_ref(q[:, sel, h:h + 1].cpu(), kd, vd)
        quant = float((ref_d - ref).abs().max())
        m = metrics(out[:, sel, h:h + 1], ref)
        md = metrics(out[:, sel, h:h + 1], ref_d)
        print(f"fp8 full size head {h}: cosine {c:.6f}, max-abs {m['max_abs']:.4f} vs the fp32 "
              f"reference (quantisation alone {quant:.4f}), {md['max_abs']:.4f} vs the "
              f"dequantised-cache reference")
        assert c >= FP8_COSINE
        assert md["max_abs"] <= 1e-2
        assert m["max_abs"] <= quant + 1e-2


def _wide_q(Lq, H, g):
    """q rows with magnitudes 2^-12 .. 2^2, row 0 all zero (uniform weights) and row 1 a
    single nonzero element: the per-query exponent of the fp8 query operands at its edges."""
    q = torch.randn(1, Lq, H, 128, generator=g)
    q = q * torch.exp2(torch.randint(-12, 3, (1, Lq, H, 1), generator=g).float())
    q[0, 0] = 0.0
    if Lq > 1:
        q[0, 1] = 0.0
        q[0, 1, :, 77] = 3.0
    return q.to(torch.bfloat16)


# The fp8 matrix cores sum each group of 8 consecutive products of an x64 MFMA in fixed point
# aligned to the group's largest product, dropping the bits more than 2^12 below it (measured on
# structured sums); the group sums then add in fp32. With the query split into hi and lo
# operands that hold its bf16 values, a score's error is below 7 * 2^-12 * (1 + 2^-4) per
# group's largest |q_d k_d|, i.e. below 2^-9 sum_d |q_d k_d|.
def _score_err(q, kd, scale):
    """Per query row: 2^-9 * scale * max over keys of sum_d |q_d k_d| ([B, Lq, H])."""
    qa, ka = q.float().abs(), kd.float().abs()
    s = torch.einsum("blhd,bkhd->blhk", qa, ka).amax(-1)
    return s * scale * 2.0 ** -9


def _row_bound(vd, delta):
    """|o - o_ref| per row: P's bf16 rounding (2^-8 max|V|) plus weights off by at most
    e^(2 delta) - 1 in total from the score errors."""
    return float(vd.abs().max()) * (2.0 ** -8 * 1.01 + torch.expm1(2 * delta)) + 1e-5


@pytest.mark.parametrize("Lq,H,lk,window,splits", [
    (1, 1, 1, None, 0),              # one key: a single partial tile
    (33, 2, 64, None, 0),            # exactly one tile
    (100, 2, 65, None, 0),           # a tile and one row
    (257, 3, 130, (3, 129), 0),      # partial first and last tiles, a partial wave
    (300, 2, 2000, None, 1),
    (300, 2, 2000, None, 3),         # split-KV partials and their merge
    (64, 5, 4096, (1000, 3001), 0),
])
def test_fp8_kernel_arithmetic_fp32(lib, Lq, H, lk, window, splits):
    """The kernel against the oracle run on the dequantised K/V, on the fp32 output, row by row
    within the bound its arithmetic fixes (P rounded to bf16, the fp8 cores' score error); and
    the relative L1 error against the same oracle stays at the level of P's bf16 rounding."""
    from lbw_amd import attention_fp8kv, quantize_kv_fp8
    g = torch.Generator().manual_seed(lk + Lq)
    q = _wide_q(Lq, H, g)
    k = _outliers(torch.randn(1, lk, H, 128, generator=g), g).to(torch.bfloat16)
    v = _outliers(torch.randn(1, lk, H, 128, generator=g), g).to(torch.bfloat16)
    kq, vq = quantize_kv_fp8(k.to(DEV)), quantize_kv_fp8(v.to(DEV))
    lo, hi = (None, None) if window is None else window
    print(f"case Lq={Lq} H={H} lk={lk} window={window} splits={splits}", flush=True)
    out = attention_fp8kv(q.to(DEV), [(kq, vq)], kv_lo=lo, kv_hi=hi, num_splits=splits,
                          out_dtype=torch.float32)
    kd = O.dequantize_kv_fp8(kq.codes.cpu(), kq.scales.cpu())
    vd = O.dequantize_kv_fp8(vq.codes.cpu(), vq.scales.cpu())
    ref = O.attention_ref(q, kd, vd, kv_lo=lo, kv_hi=hi)
    a, b = (0, lk) if window is None else window
    bound = _row_bound(vd[:, a:b], _score_err(q, kd[:, a:b], 128 ** -0.5))
    err = (out.cpu() - ref).abs().amax(-1)
    rel_l1 = float((out.cpu() - ref).abs().sum() / ref.abs().sum().clamp_min(1e-30))
    print(f"  max err {float(err.max()):.3e} (row bound min {float(bound.min()):.3e}), "
          f"rel_l1 {rel_l1:.3e}, worst err/bound {float((err / bound).max()):.3f}")
    assert bool((err <= bound).all())
    assert rel_l1 <= 4e-3


@pytest.mark.parametrize("n_segs,splits", [(1, 0), (1, 3), (2, 0), (2, 2)])
def test_fp8_prescaled_q_folded(lib, n_segs, splits):
    """A q pre-scaled by log2(e)/sqrt(d) with softmax scale ln 2 takes the folded fp8 instances
    (one segment: tile copies addressed by index; two: the general cursor): the fp32 output
    against the oracle on the dequantised K/V within the kernel's arithmetic bound, and within
    one bf16 step of the plain fp8 kernel on the same q."""
    import math
    from lbw_amd import (PRESCALED_SOFTMAX_SCALE, attention_fp8kv, prescaled_q_scale,
                         quantize_kv_fp8)
    g = torch.Generator().manual_seed(31 + n_segs + splits)
    H, Lq = 3, 290
    lens = (1300,) if n_segs == 1 else (640, 130)
    q = _wide_q(Lq, H, g)
    qs = (q.float() * prescaled_q_scale(128)).to(torch.bfloat16)
    segs, kds, vds = [], [], []
    for L in lens:
        k = _outliers(torch.randn(1, L, H, 128, generator=g), g).to(torch.bfloat16)
        v = _outliers(torch.randn(1, L, H, 128, generator=g), g).to(torch.bfloat16)
        kq, vq = quantize_kv_fp8(k.to(DEV)), quantize_kv_fp8(v.to(DEV))
        segs.append((kq, vq))
        kds.append(O.dequantize_kv_fp8(kq.codes.cpu(), kq.scales.cpu()))
        vds.append(O.dequantize_kv_fp8(vq.codes.cpu(), vq.scales.cpu()))
    kd, vd = torch.cat(kds, 1), torch.cat(vds, 1)
    print(f"case segs={lens} splits={splits}", flush=True)
    out = attention_fp8kv(qs.to(DEV), segs, softmax_scale=PRESCALED_SOFTMAX_SCALE,
                          num_splits=splits, out_dtype=torch.float32)
    plain = attention_fp8kv(qs.to(DEV), segs, softmax_scale=math.log(2.0) + 1e-7,
                            num_splits=splits, out_dtype=torch.float32)
    ref = O.attention_ref(qs, kd, vd, softmax_scale=math.log(2.0))
    bound = _row_bound(vd, _score_err(qs, kd, math.log(2.0)))
    err = (out.cpu() - ref).abs().amax(-1)
    print(f"  worst err/bound {float((err / bound).max()):.3f}")
    assert bool((err <= bound).all())
    d = (out - plain).abs().max().item()
    assert d <= 2.0 ** -7 * max(1.0, float(plain.abs().max())), d


def test_fp8_scales_not_powers_of_two_give_nan(lib):
    """The attention reads power-of-two block scales only: a tile whose K or V scale is not one
    turns the rows that read it into NaN instead of a silently wrong result."""
    from lbw_amd import attention_fp8kv, quantize_kv_fp8
    from lbw_amd.fp8 import Fp8KV
    g = torch.Generator().manual_seed(12)
    q = torch.randn(1, 70, 2, 128, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(1, 200, 2, 128, generator=g).to(torch.bfloat16).to(DEV)
    kq, vq = quantize_kv_fp8(k), quantize_kv_fp8(k)
    good = attention_fp8kv(q, [(kq, vq)])
    assert bool(torch.isfinite(good).all())
    for which in ("k", "v"):
        ks, vs = kq.scales.clone(), vq.scales.clone()
        (ks if which == "k" else vs)[0, 1, 2] *= 1.5      # head 1, block 2 (keys 128..191)
        out = attention_fp8kv(q, [(Fp8KV(kq.codes, ks), Fp8KV(vq.codes, vs))])
        torch.cuda.synchronize()
        assert bool(torch.isnan(out[:, :, 1]).all()), which
        assert torch.equal(out[:, :, 0], good[:, :, 0]), which


def test_fp8_partials_capi_match_oracle(lib):
    """The unnormalised partials (cte_partial contract: O and l relative to the row max m of the
    scaled scores) of the fp8 entry point, called through the C ABI, against the oracle on the
    dequantised K/V; two unaligned segments, a window. m within the score error bound, O / l
    within the output bound, l within e^(2 delta) - 1 relative."""
    from lbw_amd import _lib, quantize_kv_fp8
    g = torch.Generator().manual_seed(7)
    B, Lq, H = 1, 150, 2
    segs, kds, vds = [], [], []
    for L in (300, 190):
        k = _outliers(torch.randn(B, L, H, 128, generator=g), g).to(torch.bfloat16)
        v = _outliers(torch.randn(B, L, H, 128, generator=g), g).to(torch.bfloat16)
        kq, vq = quantize_kv_fp8(k.to(DEV)), quantize_kv_fp8(v.to(DEV))
        segs.append((kq.codes, vq.codes, kq.scales, vq.scales))
        kds.append(O.dequantize_kv_fp8(kq.codes.cpu(), kq.scales.cpu()))
        vds.append(O.dequantize_kv_fp8(vq.codes.cpu(), vq.scales.cpu()))
    q = _wide_q(Lq, H, g)
    qd = q.to(DEV)
    po = torch.empty(B, H, Lq, 128, device=DEV)
    pm = torch.empty(B, H, Lq, device=DEV)
    pl = torch.empty(B, H, Lq, device=DEV)
    p = _lib.attn_params(qd, None, segs, 40, 470, None, None, 0, parts=(po, pm, pl))
    L = _lib.load()
    ws_bytes = L.lbw_attention_fp8kv_workspace_size(p)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
    _lib.check(L.lbw_attention_fwd_fp8kv(p, ws.data_ptr(), ws_bytes, _lib.stream_ptr(DEV)),
               "lbw_attention_fwd_fp8kv")
    torch.cuda.synchronize()
    kd, vd = torch.cat(kds, 1)[:, 40:470], torch.cat(vds, 1)[:, 40:470]
    _, (ro, rm, rl) = O.attention_ref(q, kd, vd, return_partials=True)
    delta = _score_err(q, kd, 128 ** -0.5).permute(0, 2, 1)  # [B, H, Lq]
    assert bool(((pm.cpu() - rm).abs() <= delta + 1e-5 * rm.abs() + 1e-6).all())
    assert bool(((pl.cpu() - rl).abs() <= rl * (torch.expm1(2 * delta) + 1e-3)).all())
    o, r = po.cpu() / pl.cpu()[..., None], ro / rl[..., None]
    bound = _row_bound(vd, delta)[..., None]
    assert bool(((o - r).abs() <= bound).all())
