"""GPU parity of the folded softmax: q pre-scaled by log2(e)/sqrt(d) with softmax scale ln 2
(scale * log2(e) == 1 in fp32), the pairing the fused q/k kernel and the Wan layers use. The
kernel then starts each QK chain from -m instead of scaling every score, and sets each row's
exponent reference from its first valid sub-block. Checked against the fp32 oracle on the same
pre-scaled bf16 q, over the shapes of the plain-scale tests: windows, ragged and empty segments,
rows with no keys, KV splits through the work queues, references that move mid-row, and
peaked heads."""
import math

import pytest
import torch

import oracle as O
from parity import assert_parity

pytestmark = pytest.mark.gpu

DEV = "cuda"
LN2 = math.log(2.0)


def _prescaled(q):
    from lbw_amd import prescaled_q_scale
    return (q.float() * prescaled_q_scale(q.shape[-1])).to(torch.bfloat16)


def _case(B, Lq, H, seg_lens, seed):
    g = torch.Generator().manual_seed(seed)
    gains = torch.tensor([0.25, 0.5, 1.0, 2.0, 4.0, 8.0, 16.0, 1.0])[torch.arange(H) % 8]
    q = (torch.randn(B, Lq, H, 128, generator=g) * gains.view(1, 1, H, 1)).to(torch.bfloat16)
    ks = [torch.randn(B, L, H, 128, generator=g).to(torch.bfloat16) for L in seg_lens]
    # V halved (exact): peaked heads copy single V rows, and |o| >= 4 would put one bf16
    # output rounding above the 1e-2 bound
    vs = [(torch.randn(B, L, H, 128, generator=g) * 0.5).to(torch.bfloat16) for L in seg_lens]
    return _prescaled(q), ks, vs


@pytest.mark.parametrize("B,Lq,H,seg_lens,window,splits", [
    (1, 300, 2, [1000], None, 0),
    (1, 37, 3, [64], None, 0),
    (1, 1, 1, [1], None, 0),
    (1, 257, 2, [65], None, 0),
    (2, 129, 2, [100, 37, 200, 5], (50, 300), 0),
    (1, 512, 7, [4096, 1560], (1000, 5656), 0),
    (1, 96, 2, [7, 0, 130], None, 0),
    (1, 96, 2, [300], (200, 100), 0),       # empty window: every row has no keys -> 0
    (1, 300, 7, [2000], None, 3),
    (3, 100, 7, [2000], None, 1),
    (2, 513, 3, [333], None, 5),
    (1, 256, 5, [130], None, 7),
])
def test_prescaled_matches_oracle(lib, B, Lq, H, seg_lens, window, splits):
    from lbw_amd import PRESCALED_SOFTMAX_SCALE, attention_segments
    q, ks, vs = _case(B, Lq, H, seg_lens, seed=Lq + H + splits)
    lo, hi = (None, None) if window is None else window
    out = attention_segments(q.to(DEV), [(k.to(DEV), v.to(DEV)) for k, v in zip(ks, vs)],
                             kv_lo=lo, kv_hi=hi, softmax_scale=PRESCALED_SOFTMAX_SCALE,
                             num_splits=splits)
    ref = O.attention_ref(q, torch.cat(ks, 1), torch.cat(vs, 1), kv_lo=lo, kv_hi=hi,
                          softmax_scale=LN2)
    assert_parity(out, ref, f"B={B} Lq={Lq} H={H} segs={seg_lens} window={window} splits={splits}")


def test_prescaled_window_starting_mid_tile(lib):
    """Keys from 100 on: the first tile's first sub-block is masked whole, so the reference stays
    unset through it and is set from the second."""
    from lbw_amd import PRESCALED_SOFTMAX_SCALE, attention_segments
    q, ks, vs = _case(1, 200, 4, [700], seed=5)
    for lo in (40, 100, 129):
        out = attention_segments(q.to(DEV), [(ks[0].to(DEV), vs[0].to(DEV))], kv_lo=lo,
                                 softmax_scale=PRESCALED_SOFTMAX_SCALE)
        ref = O.attention_ref(q, ks[0], vs[0], kv_lo=lo, softmax_scale=LN2)
        assert_parity(out, ref, f"lo={lo}")


@pytest.mark.parametrize("jump", [2.0, 12.0, 60.0])
def test_prescaled_reference_moves_mid_row(lib, jump):
    """Scores that rise by `jump` natural-log units per 64-key tile: the reference moves, and
    the next sub-block's S, started from the old -m in the same step, moves with it."""
    from lbw_amd import PRESCALED_SOFTMAX_SCALE, attention_segments
    g = torch.Generator().manual_seed(31)
    B, Lq, H, L = 1, 70, 2, 12 * 64 + 17
    u = torch.randn(128, generator=g)
    u = u / u.norm()
    q = (torch.randn(B, Lq, H, 128, generator=g) * 0.3 + 4.0 * u).to(torch.bfloat16)
    ramp = torch.arange(L, dtype=torch.float32).div(64).floor()
    gain = (ramp * jump * math.sqrt(128) / 4.0).view(1, L, 1, 1)
    k = (torch.randn(B, L, H, 128, generator=g) * 0.3 + gain * u).to(torch.bfloat16)
    v = (torch.randn(B, L, H, 128, generator=g) * 0.5).to(torch.bfloat16)
    qs = _prescaled(q)
    ref = O.attention_ref(qs, k, v, softmax_scale=LN2)
    for splits in (1, 3):
        out = attention_segments(qs.to(DEV), [(k.to(DEV), v.to(DEV))], num_splits=splits,
                                 softmax_scale=PRESCALED_SOFTMAX_SCALE)
        assert_parity(out, ref, f"jump {jump} splits {splits}")


def test_prescaled_equals_plain_kernel(lib):
    """The folded kernel and the plain one (scale ln 2 (1 + 2^-21): c != 1 in fp32, the FMA
    path) on the same pre-scaled q agree to bf16 rounding."""
    from lbw_amd import PRESCALED_SOFTMAX_SCALE, attention_segments
    q, ks, vs = _case(1, 400, 6, [1500], seed=77)
    segs = [(ks[0].to(DEV), vs[0].to(DEV))]
    fold = attention_segments(q.to(DEV), segs, softmax_scale=PRESCALED_SOFTMAX_SCALE)
    plain = attention_segments(q.to(DEV), segs, softmax_scale=LN2 * (1 + 2.0 ** -21))
    assert (fold.float() - plain.float()).abs().max() < 8e-3


def test_prescaled_cross_attention_masked_and_dedup(lib):
    """The folded kernel on the cross-attention paths: per-batch valid key counts (k_lens) and
    the exact dedup form, whose multiplicity bias ln(mult) / scale is log2(mult) when
    scale * log2(e) == 1."""
    from lbw_amd import PRESCALED_SOFTMAX_SCALE, attention_segments, padding_start
    g = torch.Generator().manual_seed(43)
    H, Lq, L, nv = 4, 333, 512, 300
    q = _prescaled(torch.randn(2, Lq, H, 128, generator=g).to(torch.bfloat16))
    k = torch.randn(2, L, H, 128, generator=g).to(torch.bfloat16)
    v = (0.5 * torch.randn(2, L, H, 128, generator=g)).to(torch.bfloat16)
    k_lens = torch.tensor([300, 512], dtype=torch.int32)
    out = attention_segments(q.to(DEV), [(k.to(DEV), v.to(DEV))], k_lens=k_lens.to(DEV),
                             cross=True, softmax_scale=PRESCALED_SOFTMAX_SCALE)
    ref = O.attention_ref(q, k, v, k_lens=k_lens, softmax_scale=LN2)
    assert_parity(out, ref, "masked")
    # dedup: rows nv.. of k/v identical (one batch)
    kd = torch.randn(1, L, H, 128, generator=g)
    vd = 0.5 * torch.randn(1, L, H, 128, generator=g)
    kd[:, nv:] = torch.randn(1, 1, H, 128, generator=g)
    vd[:, nv:] = 0.5 * torch.randn(1, 1, H, 128, generator=g)
    kd, vd = kd.to(torch.bfloat16), vd.to(torch.bfloat16)
    nd = padding_start(kd.to(DEV), vd.to(DEV))
    assert nd == nv
    out = attention_segments(q[:1].to(DEV), [(kd.to(DEV), vd.to(DEV))], cross=True, n_distinct=nd,
                             softmax_scale=PRESCALED_SOFTMAX_SCALE)
    assert_parity(out, O.attention_ref(q[:1], kd, vd, softmax_scale=LN2), "dedup")


@pytest.mark.parametrize("H,Lq,L,gain", [(40, 4680, 512, 4.0), (3, 9000, 448, 1.0), (2, 700, 330, 8.0)])
def test_prescaled_cross_ring(lib, H, Lq, L, gain):
    """The folded softmax in the cross ring form (an unmasked context over 320 keys): rounds that
    restart the exponent reference without rescaling the previous round's O, peaked queries that
    move it mid-round; fp32 output within the arithmetic bound on sampled rows of three heads, the
    bf16 output equal to it rounded once and within twice that bound (plus the bf16 rounding) of
    the plain-softmax kernel on the same inputs."""
    from lbw_amd import PRESCALED_SOFTMAX_SCALE, attention_segments
    g = torch.Generator().manual_seed(L + H)
    q = _prescaled((gain * torch.randn(1, Lq, H, 128, generator=g)).to(torch.bfloat16))
    k = torch.randn(1, L, H, 128, generator=g).to(torch.bfloat16)
    v = (0.5 * torch.randn(1, L, H, 128, generator=g)).to(torch.bfloat16)
    print(f"case H={H} Lq={Lq} L={L} gain={gain}", flush=True)
    dq, dk, dv = q.to(DEV), k.to(DEV), v.to(DEV)
    o32 = attention_segments(dq, [(dk, dv)], cross=True, softmax_scale=PRESCALED_SOFTMAX_SCALE,
                             out_dtype=torch.float32)
    o16 = attention_segments(dq, [(dk, dv)], cross=True, softmax_scale=PRESCALED_SOFTMAX_SCALE)
    plain = attention_segments(dq, [(dk, dv)], cross=True, softmax_scale=LN2 * (1 + 2.0 ** -21))
    torch.cuda.synchronize()
    assert torch.equal(o32.to(torch.bfloat16), o16)
    # (the two forms round p differently, each within the arithmetic bound of the exact result:
    # together within twice it, plus the bf16 rounding of both outputs)
    tol = 2 * float(v.float().abs().max()) * 2.0 ** -8 * 1.01 + 2.0 ** -8 * float(plain.float().abs().max())
    assert float((o16.float() - plain.float()).abs().max()) <= tol
    sel = torch.cat([torch.randperm(Lq, generator=torch.Generator().manual_seed(3))[:300],
                     torch.arange((Lq // 32) * 32, Lq)]).unique().sort().values
    oc = o32[:, sel].cpu()
    for h in sorted({0, H // 2, H - 1}):
        ref = O.attention_ref(q[:, sel][:, :, h:h + 1], k[:, :, h:h + 1], v[:, :, h:h + 1],
                              softmax_scale=LN2)
        err = float((oc[:, :, h:h + 1] - ref).abs().max())
        bound = float(v[:, :, h].float().abs().max()) * 2.0 ** -8 * 1.01 + 1e-5
        assert err <= bound, (h, err, bound)


def test_prescaled_partials_and_chain(lib):
    """The partials API (tracked row max, the FMA form with c = 1) under the pre-scaled pairing:
    m in scaled units (scale * s) as the oracle's partials, and a chain over key sets equal to
    attention over their union."""
    from lbw_amd import PRESCALED_SOFTMAX_SCALE, attention_chain, attention_partial
    g = torch.Generator().manual_seed(51)
    q = _prescaled(torch.randn(1, 150, 3, 128, generator=g).to(torch.bfloat16))
    ks = [torch.randn(1, n, 3, 128, generator=g).to(torch.bfloat16) for n in (500, 260)]
    vs = [(0.5 * torch.randn(1, n, 3, 128, generator=g)).to(torch.bfloat16) for n in (500, 260)]
    po, pm, pl = attention_partial(q.to(DEV), [(ks[0].to(DEV), vs[0].to(DEV))],
                                   softmax_scale=PRESCALED_SOFTMAX_SCALE)
    _, (ro, rm, rl) = O.attention_ref(q, ks[0], vs[0], softmax_scale=LN2, return_partials=True)
    assert torch.allclose(pm.cpu(), rm, rtol=1e-5, atol=1e-4)
    assert torch.allclose(pl.cpu(), rl, rtol=5e-3, atol=1e-3)
    segs = [(k.to(DEV), v.to(DEV)) for k, v in zip(ks, vs)]
    state = attention_chain(q.to(DEV), segs[:1], softmax_scale=PRESCALED_SOFTMAX_SCALE)
    state = attention_chain(q.to(DEV), segs[1:], state, softmax_scale=PRESCALED_SOFTMAX_SCALE)
    out = attention_chain(q.to(DEV), [], state, normalize=True)
    ref = O.attention_ref(q, torch.cat(ks, 1), torch.cat(vs, 1), softmax_scale=LN2)
    assert_parity(out, ref, "chain")
