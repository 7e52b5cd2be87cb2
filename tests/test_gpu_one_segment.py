"""The index-addressed kernel instances (a call over one KV segment, or two with the same row
strides, and no multiplicity bias: their tile copies are addressed by the tile index) against the
general segment cursor and the oracle.

The same keys passed as one segment, as two segments split at a multiple of 64, and as three
(the two and an empty one between them, which the index-addressed forms do not take) walk exactly
the same 64-key tiles in the same order, so all three must give the same output bit for bit; any
error in the index addressing (a tile off by one, a wrong partial-tile row range at the window's
ends, a piece of a split starting at the wrong tile, the wrong segment for a tile) breaks that
equality. The cases put the window's ends inside tiles, on tile boundaries and in one tile, split
the keys into 1-5 pieces that start mid-segment, and limit keys per batch with k_lens; both
softmax forms (plain and pre-scaled q)."""
import math

import pytest
import torch

import oracle as O
from parity import assert_parity

pytestmark = pytest.mark.gpu
DEV = "cuda"

# (B, H, Lq, L, window (lo, hi) or None, splits, pre-scaled q, k_lens or None, split point c)
CASES = [
    (1, 2, 300, 1500, None, 3, True, None, 640),
    (1, 2, 300, 1500, (77, 1433), 3, True, None, 704),
    (1, 2, 257, 1500, (77, 1433), 5, False, None, 128),
    (1, 1, 100, 1000, (130, 150), 2, True, None, 64),      # both ends in one tile
    (1, 1, 100, 1000, (128, 192), 1, False, None, 128),    # exactly one full tile
    (1, 3, 513, 2000, (0, 1984), 4, True, None, 1024),     # hi on a tile boundary
    (1, 2, 64, 777, (64, 700), 3, True, None, 320),        # lo on a tile boundary
    (2, 2, 200, 1200, None, 3, True, [1200, 333], 576),    # k_lens per batch
    (2, 2, 200, 1200, (10, 1100), 2, False, [900, 1150], 512),
    (1, 2, 33, 70, None, 1, True, None, 64),               # two tiles, the second partial
]


@pytest.mark.parametrize("i", range(len(CASES)))
def test_index_addressed_match_general_cursor_and_oracle(lib, i):
    from lbw_amd import PRESCALED_SOFTMAX_SCALE, attention_segments, prescaled_q_scale
    B, H, Lq, L, win, splits, pre, klens, c = CASES[i]
    print(f"case {i}: B={B} H={H} Lq={Lq} L={L} window={win} splits={splits} pre={pre} "
          f"k_lens={klens} split at {c}", flush=True)
    assert c % 64 == 0 and 0 < c < L
    g = torch.Generator().manual_seed(50 + i)
    q = torch.randn(B, Lq, H, 128, generator=g)
    if pre:
        q = q * prescaled_q_scale(128)
    q = q.to(torch.bfloat16)
    k = torch.randn(B, L, H, 128, generator=g).to(torch.bfloat16)
    v = (0.5 * torch.randn(B, L, H, 128, generator=g)).to(torch.bfloat16)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    lo, hi = (None, None) if win is None else win
    kl = None if klens is None else torch.tensor(klens, dtype=torch.int32, device=DEV)
    scale = PRESCALED_SOFTMAX_SCALE if pre else None
    one = attention_segments(qd, [(kd, vd)], kv_lo=lo, kv_hi=hi, k_lens=kl, num_splits=splits,
                             softmax_scale=scale)
    two = attention_segments(qd, [(kd[:, :c], vd[:, :c]), (kd[:, c:], vd[:, c:])], kv_lo=lo,
                             kv_hi=hi, k_lens=kl, num_splits=splits, softmax_scale=scale)
    three = attention_segments(qd, [(kd[:, :c], vd[:, :c]), (kd[:, c:c], vd[:, c:c]),
                                    (kd[:, c:], vd[:, c:])], kv_lo=lo, kv_hi=hi, k_lens=kl,
                               num_splits=splits, softmax_scale=scale)
    torch.cuda.synchronize()
    for name, x in (("one", one), ("two", two)):
        d = (x.float() - three.float()).abs()
        print(f"  {name} vs three segments: max diff {float(d.max()):.3e}, "
              f"differing {int((d > 0).sum())}")
    assert torch.equal(one, three) and torch.equal(two, three)
    kls = None if klens is None else torch.tensor(klens, dtype=torch.int32)
    ref = O.attention_ref(q, k, v, kv_lo=lo, kv_hi=hi, k_lens=kls,
                          softmax_scale=math.log(2.0) if pre else None)
    assert_parity(one, ref, f"case {i}")


FP8_CASES = [
    (1, 2, 300, 1500, None, 3, 640),
    (1, 2, 257, 1500, (77, 1433), 5, 128),
    (1, 1, 100, 1000, (130, 150), 2, 64),
    (2, 2, 200, 1200, (10, 1100), 2, 512),
]


@pytest.mark.parametrize("i", range(len(FP8_CASES)))
def test_fp8_one_segment_matches_general_cursor(lib, i):
    """The fp8-KV kernel's one-segment instance (K codes, V codes and block scales addressed by
    the tile index) against the general cursor over the same codes as two block-aligned
    segments (quantising the halves separately gives the whole cache's codes and scales)."""
    from lbw_amd import attention_fp8kv, quantize_kv_fp8
    B, H, Lq, L, win, splits, c = FP8_CASES[i]
    print(f"fp8 case {i}: B={B} H={H} Lq={Lq} L={L} window={win} splits={splits} split at {c}",
          flush=True)
    g = torch.Generator(device=DEV).manual_seed(70 + i)
    q = torch.randn(B, Lq, H, 128, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(B, L, H, 128, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(B, L, H, 128, generator=g, device=DEV).to(torch.bfloat16)
    whole = (quantize_kv_fp8(k), quantize_kv_fp8(v))
    halves = [(quantize_kv_fp8(k[:, :c]), quantize_kv_fp8(v[:, :c])),
              (quantize_kv_fp8(k[:, c:]), quantize_kv_fp8(v[:, c:]))]
    assert torch.equal(whole[0].codes[:, c:], halves[1][0].codes)
    lo, hi = (None, None) if win is None else win
    one = attention_fp8kv(q, [whole], kv_lo=lo, kv_hi=hi, num_splits=splits)
    two = attention_fp8kv(q, halves, kv_lo=lo, kv_hi=hi, num_splits=splits)
    torch.cuda.synchronize()
    d = (one.float() - two.float()).abs()
    print(f"  one vs two segments: max diff {float(d.max()):.3e}, differing {int((d > 0).sum())}")
    assert torch.equal(one, two)
