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
    out = attention_fp8kv(q, [(quantize_kv_fp8(k), quantize_kv_fp8(v))])
    torch.cuda.synchronize()
    sel = torch.randperm(Lq, generator=torch.Generator().manual_seed(1))[:128].sort().values
    for h in (0, 23):
        ref = O.attention_ref(q[:, sel, h:h + 1].cpu(), k[:, :, h:h + 1].cpu(), v[:, :, h:h + 1].cpu())
        c = cosine(out[:, sel, h:h + 1], ref)
        print(f"fp8 full size head {h}: cosine {c:.6f}")
        assert c >= FP8_COSINE
