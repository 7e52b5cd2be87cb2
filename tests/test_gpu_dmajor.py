"""GPU parity of the chunk kernel reading K d-major: the reference's N-major K cache [N, D, L]
(wan/modules/chunked_kv_cache.py:118-148) and pre-transposed cross cache
(wan/modules/attention.py:494-499, 557-579), handed over as d-major views (token stride 1) and
read as they lie. Against the oracle, and against the same call on a token-major copy of K."""
import math

import pytest
import torch

import oracle as O
from parity import assert_parity, metrics

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _dmajor(k, cap=None):
    """A d-major view [B, L, N, D] (strides: token 1, d = capacity) of K, on the GPU."""
    B, L, H, D = k.shape
    cap = L if cap is None else cap
    buf = torch.zeros(B, H, D, cap, dtype=torch.bfloat16, device=DEV)
    buf[..., :L] = k.to(DEV).permute(0, 2, 3, 1)
    view = buf[..., :L].permute(0, 3, 1, 2)
    assert view.stride(1) == 1 and view.stride(3) == cap
    return view


def _case(B, Lq, H, lens, seed):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16)
    return r(B, Lq, H, 128), [r(B, L, H, 128) for L in lens], [r(B, L, H, 128) for L in lens]


@pytest.mark.parametrize("B,Lq,H,lens,window,splits", [
    (1, 300, 2, [1000], None, 0),
    (1, 37, 3, [64], None, 1),
    (2, 129, 2, [104, 40, 200, 8], (50, 300), 0),
    (1, 512, 4, [4096, 1560], (1000, 5656), 3),
    (1, 96, 2, [8, 0, 136], None, 2),
    (1, 260, 3, [2000], (7, 1999), 5),
])
def test_dmajor_k_matches_oracle(lib, B, Lq, H, lens, window, splits):
    from lbw_amd import attention_segments
    q, ks, vs = _case(B, Lq, H, lens, seed=Lq + H + len(lens))
    lo, hi = (None, None) if window is None else window
    segs_t = [(k.to(DEV), v.to(DEV)) for k, v in zip(ks, vs)]
    segs_d = [(_dmajor(k, cap=k.shape[1] + 24), v.to(DEV)) for k, v in zip(ks, vs)]
    out = attention_segments(q.to(DEV), segs_d, kv_lo=lo, kv_hi=hi, num_splits=splits)
    tok = attention_segments(q.to(DEV), segs_t, kv_lo=lo, kv_hi=hi, num_splits=splits)
    torch.cuda.synchronize()
    ref = O.attention_ref(q, torch.cat(ks, 1), torch.cat(vs, 1), kv_lo=lo, kv_hi=hi)
    m = metrics(out, ref)
    print(f"d-major B={B} Lq={Lq} H={H} lens={lens} window={window} splits={splits}", m)
    assert_parity(out, ref)
    # the same products summed in another order inside the MFMA: one bf16 step at most
    assert float((out.float() - tok.float()).abs().max()) <= 2.0 ** -6 * max(1.0, float(tok.float().abs().max()))


def test_dmajor_k_prescaled_and_partials(lib):
    """The folded softmax (q pre-scaled, scale ln 2) and the partials (tracked row max) over
    d-major K, against the oracle."""
    from lbw_amd import (PRESCALED_SOFTMAX_SCALE, attention_partial, attention_segments,
                         prescaled_q_scale)
    q, ks, vs = _case(1, 200, 3, [1200, 344], seed=8)
    qs = (q.float() * prescaled_q_scale(128)).to(torch.bfloat16)
    segs = [(_dmajor(k), v.to(DEV)) for k, v in zip(ks, vs)]
    kk, vv = torch.cat(ks, 1), torch.cat(vs, 1)
    out = attention_segments(qs.to(DEV), segs, softmax_scale=PRESCALED_SOFTMAX_SCALE)
    assert_parity(out, O.attention_ref(qs, kk, vv, softmax_scale=math.log(2.0)), "folded")
    po, pm, pl = attention_partial(q.to(DEV), segs)
    _, (ro, rm, rl) = O.attention_ref(q, kk, vv, return_partials=True)
    assert torch.allclose(pm.cpu(), rm, rtol=1e-5, atol=1e-4)
    assert torch.allclose(pl.cpu(), rl, rtol=5e-3, atol=1e-3)


def test_nmajor_cross_cache_dedup(lib):
    """The reference's N-major cross cache (K [N, D, 512], V [N, 512, D]) with zero-padded rows
    identical from row 300 on: the exact dedup and the masked call over the d-major cache equal
    the oracle."""
    from lbw_amd import cross_attention
    g = torch.Generator().manual_seed(4)
    H, Lq = 4, 700
    q = torch.randn(1, Lq, H, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 512, H, 128, generator=g).to(torch.bfloat16)
    # (V halved, exact in bf16: rows peaked on a few of 300 keys would otherwise put |o| where
    # one bf16 output step exceeds the 1e-2 bound)
    v = (0.5 * torch.randn(1, 512, H, 128, generator=g)).to(torch.bfloat16)
    k[:, 300:] = k[:, 511:]
    v[:, 300:] = v[:, 511:]
    k_nd = _dmajor(k)
    v_nld = v.to(DEV).permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)  # [N, L, D] storage
    out = cross_attention(q.to(DEV), k_nd, v_nld, n_distinct=300)
    assert_parity(out, O.attention_ref(q, k, v), "dedup")
    tok = cross_attention(q.to(DEV), k.to(DEV), v.to(DEV), n_distinct=300)
    assert float((out.float() - tok.float()).abs().max()) <= 2.0 ** -7
    kl = torch.tensor([300], dtype=torch.int32, device=DEV)
    out_m = cross_attention(q.to(DEV), k_nd, v_nld, k_lens=kl)
    assert_parity(out_m, O.attention_ref(q, k, v, k_lens=torch.tensor([300])), "masked")
    # the same cache as the 3-D N-major tensors the reference's cross path passes
    k3 = k[0].permute(1, 2, 0).contiguous().to(DEV)      # [N, D, L]
    v3 = v[0].permute(1, 0, 2).contiguous().to(DEV)      # [N, L, D]
    out3 = cross_attention(q.to(DEV), k3, v3)
    assert_parity(out3, O.attention_ref(q, k, v), "N-major 3-D")


def test_dmajor_cache_written_by_the_qk_kernel(lib):
    """The whole d-major path: the fused q/k kernel writes the chunk's K into a [N, D, capacity]
    cache slot (its d-major output), and the attention reads the cache's d-major K directly."""
    from lbw_amd import attention_segments, causal_rope_tables, qk_norm_rope_, wan_rope_freqs
    g = torch.Generator().manual_seed(6)
    H, D = 3, 128
    C = H * D
    grid = (1, 8, 10)
    L, Lc, cap = 80, 160, 256
    xq = torch.randn(L, C, generator=g).to(torch.bfloat16)
    xk = torch.randn(L, C, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(C, generator=g)).to(torch.bfloat16)
    kc = torch.randn(1, Lc, H, D, generator=g).to(torch.bfloat16)
    v = torch.randn(1, Lc + L, H, D, generator=g).to(torch.bfloat16)
    cache = torch.zeros(H, D, cap, dtype=torch.bfloat16, device=DEV)
    cache[:, :, :Lc] = kc[0].to(DEV).permute(1, 2, 0)
    tabs = causal_rope_tables(wan_rope_freqs(D), grid, 2, device=DEV)
    q_out = torch.empty(L, C, dtype=torch.bfloat16, device=DEV)
    # q in rows (what the attention reads), k d-major straight into the cache slot (one tensor
    # per call: the kernel's single-tensor form)
    qk_norm_rope_(xq.to(DEV), None, None, None, w.to(DEV), None, tabs, 1e-6, H, q_out=q_out,
                  k_out=None)
    qk_norm_rope_(xk.to(DEV), None, None, None, w.to(DEV), None, tabs, 1e-6, H,
                  q_out=cache[:, :, Lc:Lc + L], k_out=None, layout="dmajor")
    k_view = cache[:, :, :Lc + L].permute(2, 0, 1).unsqueeze(0)          # [1, Lc+L, H, D]
    out = attention_segments(q_out.view(1, L, H, D), [(k_view, v.to(DEV))])
    torch.cuda.synchronize()
    cos, sin = O.causal_rope_grids(O.wan_rope_freqs(D), *grid, start_frame=2)
    rq = O.qk_post_norm_rope(xq, None, w, cos, sin).view(1, L, H, D)
    rk = O.qk_post_norm_rope(xk, None, w, cos, sin).view(1, L, H, D)
    ref = O.attention_ref(rq, torch.cat([kc, rk], 1), v)
    assert_parity(out, ref, "d-major cache")


def test_exact_attention_chunks_nmajor(lib):
    """exact_attention_chunks over the reference's N-major chunk list (attention.py:1048-1058,
    993-1019): K [N, D, L] (pre-transposed) or [N, L, D], V [N, L, D], chunks of different
    lengths read where they lie; against the oracle over the concatenation."""
    from lbw_amd import exact_attention_chunks
    g = torch.Generator().manual_seed(12)
    H, D, Lq = 3, 128, 333
    lens = [1560, 64, 936]
    q = torch.randn(1, Lq, H, D, generator=g).to(torch.bfloat16)
    ks = [torch.randn(1, L, H, D, generator=g).to(torch.bfloat16) for L in lens]
    vs = [(0.5 * torch.randn(1, L, H, D, generator=g)).to(torch.bfloat16) for L in lens]
    ref = O.attention_ref(q, torch.cat(ks, 1), torch.cat(vs, 1))
    v_n = [v[0].permute(1, 0, 2).contiguous().to(DEV) for v in vs]          # [N, L, D]
    for k_layout in ("ndl", "nld"):
        if k_layout == "ndl":
            k_n = [k[0].permute(1, 2, 0).contiguous().to(DEV) for k in ks]  # [N, D, L]
        else:
            k_n = [k[0].permute(1, 0, 2).contiguous().to(DEV) for k in ks]  # [N, L, D]
        out = exact_attention_chunks(q.to(DEV), k_n, v_n)
        assert_parity(out, ref, f"N-major chunks, K {k_layout}")


def test_dmajor_refusals(lib):
    from lbw_amd import attention_fp8kv, attention_segments, quantize_kv_fp8
    q, ks, vs = _case(1, 64, 2, [100, 64], seed=1)
    with pytest.raises(RuntimeError, match="multiples of 8"):      # len 100: not a multiple of 8
        attention_segments(q.to(DEV), [(_dmajor(ks[0]), vs[0].to(DEV))])
    with pytest.raises(RuntimeError, match="d-major, or none"):    # mixed layouts
        attention_segments(q.to(DEV), [(_dmajor(ks[1]), vs[1].to(DEV)),
                                       (ks[1].to(DEV), vs[1].to(DEV))])
