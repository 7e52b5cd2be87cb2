"""GPU parity of the cross-attention kernel (cross_attn.hip, lbw_cross_attention_fwd and the
dedup entry point) against the fp32 oracle.

The kernel keeps a (batch, head)'s K/V rows resident in LDS when at most 320 keys are attended
and otherwise walks them in 320-key chunks, with persistent workgroups that run consecutive
256-query rounds; an unmasked context longer than 320 keys runs its ring form, which streams the
context through LDS in 64-key tiles and pipelines each round into the next. The cases cover both paths and their edges: key counts around the 32-key
sub-block and the 320-key chunk, per-batch valid lengths (k_lens) that put one batch on each
path, windows, query counts that leave partial 32-query blocks and rounds, head counts whose
rounds straddle workgroups, strided views, the bf16 bar and, on the fp32 output, the bound the
kernel's arithmetic fixes (P enters the PV product as bf16: |o - o_exact| <= 2^-8 max|V|)."""
import math

import pytest
import torch

import oracle as O
from parity import assert_parity

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _kernel_bound(v):
    return float(v.float().abs().max()) * 2.0 ** -8 * 1.01 + 1e-5


def _qkv(B, Lq, H, L, seed, qgain=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, Lq, H, 128, generator=g) * qgain).to(torch.bfloat16)
    k = torch.randn(B, L, H, 128, generator=g).to(torch.bfloat16)
    v = (0.5 * torch.randn(B, L, H, 128, generator=g)).to(torch.bfloat16)
    return q, k, v


@pytest.mark.parametrize("B,Lq,H,L,lens", [
    (1, 1, 1, 1, None),
    (1, 33, 2, 31, None),
    (1, 64, 1, 32, None),
    (1, 100, 3, 33, None),
    (1, 257, 2, 300, None),
    (1, 300, 2, 319, None),
    (1, 513, 2, 320, None),
    (1, 96, 2, 321, None),           # chunked: 320 + 1
    (1, 200, 3, 640, None),          # two full chunks
    (2, 130, 2, 700, [0, 700]),      # one batch with no keys (output 0), one chunked
    (2, 333, 4, 512, [300, 512]),    # resident and chunked batches in one call
    (3, 77, 5, 4096, [1, 4096, 333]),
])
def test_cross_matches_oracle(lib, B, Lq, H, L, lens):
    from lbw_amd import cross_attention
    q, k, v = _qkv(B, Lq, H, L, seed=Lq + L + H)
    kl = None if lens is None else torch.tensor(lens, dtype=torch.int32)
    print(f"case B={B} Lq={Lq} H={H} L={L} k_lens={lens}", flush=True)
    out = cross_attention(q.to(DEV), k.to(DEV), v.to(DEV),
                          k_lens=None if kl is None else kl.to(DEV))
    ref = O.attention_ref(q, k, v, k_lens=kl)
    assert_parity(out, ref, "cross")


@pytest.mark.parametrize("H,Lq", [(40, 4680), (7, 1000)])
def test_cross_rounds_across_workgroups_fp32(lib, H, Lq):
    """Many heads (rounds of one head spread over several workgroups, workgroups spanning two
    heads, the K/V reload at each switch) on the fp32 output, against the arithmetic bound;
    peaked queries (gain 4) so that the exponent reference moves. Sampled rows of every 5th
    head, including the partial last 32-query block."""
    from lbw_amd import attention_segments
    q, k, v = _qkv(1, Lq, H, 512, seed=H, qgain=4.0)
    kl = torch.tensor([300], dtype=torch.int32)
    out = attention_segments(q.to(DEV), [(k.to(DEV), v.to(DEV))], k_lens=kl.to(DEV), cross=True,
                             out_dtype=torch.float32)
    torch.cuda.synchronize()
    tail = torch.arange((Lq // 32) * 32, Lq)
    sel = torch.cat([torch.randperm(Lq, generator=torch.Generator().manual_seed(H))[:200], tail])
    sel = sel.unique().sort().values
    oc = out[:, sel].cpu()
    for h in range(0, H, 5):
        ref = O.attention_ref(q[:, sel][:, :, h:h + 1], k[:, :, h:h + 1], v[:, :, h:h + 1], k_lens=kl)
        err = float((oc[:, :, h:h + 1] - ref).abs().max())
        bound = _kernel_bound(v[:, :300, h])
        assert err <= bound, (h, err, bound)


@pytest.mark.parametrize("B,Lq,H,L,window", [
    (1, 256, 1, 321, None),
    (2, 300, 3, 384, None),
    (1, 513, 2, 385, None),
    (1, 64, 5, 512, None),
    (2, 1000, 3, 512, (20, 470)),    # a 450-key window
    (1, 100, 7, 450, None),
    (1, 333, 3, 1000, None),         # 16 tiles a round, the last 40 keys valid
    (1, 200, 2, 4096, None),         # the longest context: 64 tiles a round
])
def test_cross_long_unmasked_context(lib, B, Lq, H, L, window):
    """Unmasked contexts longer than the 320 resident keys (up to the reference's padded 512)
    run the ring form (the context streamed through LDS, rounds pipelined into each other):
    bf16 bar, and the fp32 output within the kernel's arithmetic bound and equal to the bf16
    output before its rounding."""
    from lbw_amd import attention_segments, cross_attention
    q, k, v = _qkv(B, Lq, H, L, seed=3 * Lq + L + H, qgain=2.0)
    lo, hi = (None, None) if window is None else window
    print(f"case B={B} Lq={Lq} H={H} L={L} window={window}", flush=True)
    if window is None:
        out = cross_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    else:
        out = attention_segments(q.to(DEV), [(k.to(DEV), v.to(DEV))], kv_lo=lo, kv_hi=hi,
                                 cross=True)
    ref = O.attention_ref(q, k, v, kv_lo=lo, kv_hi=hi)
    assert_parity(out, ref, "long context")
    o32 = attention_segments(q.to(DEV), [(k.to(DEV), v.to(DEV))], kv_lo=lo, kv_hi=hi, cross=True,
                             out_dtype=torch.float32)
    a, b = (0, L) if window is None else window
    err = float((o32.cpu() - ref).abs().max())
    assert err <= _kernel_bound(v[:, a:b]), err
    assert torch.equal(o32.to(torch.bfloat16), out)


@pytest.mark.parametrize("H,Lq,L", [(40, 4680, 512), (3, 25600, 448), (1, 200, 330)])
def test_cross_ring_rounds_fp32(lib, H, Lq, L):
    """The ring form over many rounds per workgroup (25600 queries of 3 heads: ~10 rounds each),
    rounds crossing heads, a workgroup with a single round (one head of 200 queries), and the
    round boundary at every stage of the ring (8 and 7 tiles per round): fp32 output against the
    arithmetic bound on sampled rows of several heads, including the partial last 32-query
    block, with peaked queries (gain 4) so that the exponent reference moves; bf16 output equal
    to the fp32 output rounded once."""
    from lbw_amd import attention_segments, cross_attention
    q, k, v = _qkv(1, Lq, H, L, seed=H + L, qgain=4.0)
    print(f"case H={H} Lq={Lq} L={L}", flush=True)
    dq, dk, dv = q.to(DEV), k.to(DEV), v.to(DEV)
    o32 = attention_segments(dq, [(dk, dv)], cross=True, out_dtype=torch.float32)
    o16 = cross_attention(dq, dk, dv)
    torch.cuda.synchronize()
    assert torch.equal(o32.to(torch.bfloat16), o16)
    tail = torch.arange((Lq // 32) * 32, Lq)
    sel = torch.cat([torch.randperm(Lq, generator=torch.Generator().manual_seed(L))[:300], tail])
    sel = sel.unique().sort().values
    oc = o32[:, sel].cpu()
    for h in sorted({0, H // 2, H - 1}):
        ref = O.attention_ref(q[:, sel][:, :, h:h + 1], k[:, :, h:h + 1], v[:, :, h:h + 1])
        err = float((oc[:, :, h:h + 1] - ref).abs().max())
        bound = _kernel_bound(v[:, :, h])
        assert err <= bound, (h, err, bound)


def test_cross_ring_rounds_restart_the_softmax(lib):
    """Each round of the ring form starts a fresh softmax: 256-query rounds alternate between
    queries scaled by 40 and by 1/40 (scores ~1e3 against ~1e-1), so a reference carried over
    from a large round would underflow the next round's probabilities to 0."""
    from lbw_amd import cross_attention
    q, k, v = _qkv(1, 2048, 2, 512, seed=91)
    gain = torch.where((torch.arange(2048) // 256) % 2 == 0, 40.0, 1.0 / 40.0)
    q = (q.float() * gain[None, :, None, None]).to(torch.bfloat16)
    out = cross_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    assert_parity(out, O.attention_ref(q, k, v), "alternating rounds")


def test_cross_ring_non_finite_value_stays_in_its_head(lib):
    """An infinite V entry in one head makes that head's outputs non-finite (as the reference's
    softmax(QK^T) V does) and leaves every other head's outputs exact: the round boundary adds
    only the previous round's own P V to the previous round's O."""
    from lbw_amd import cross_attention
    q, k, v = _qkv(1, 1024, 4, 512, seed=5)
    v[:, 77, 1, 5] = float("inf")
    out = cross_attention(q.to(DEV), k.to(DEV), v.to(DEV)).cpu()
    assert not torch.isfinite(out[:, :, 1, 5]).any()
    keep = [0, 2, 3]
    assert_parity(out[:, :, keep], O.attention_ref(q[:, :, keep], k[:, :, keep], v[:, :, keep]),
                  "other heads")


def test_cross_out_views(lib):
    """Both cross kernels (resident: 300 keys via k_lens; ring: all 512) writing into given
    outputs: a bf16 view whose rows start 8 bytes past a 16-byte boundary (the kernels' 8-byte
    store form) and an fp32 view; each equal to the call's own fresh output, and nothing written
    outside the view."""
    from lbw_amd import attention_segments
    q, k, v = _qkv(1, 700, 3, 512, seed=13)
    dq, dk, dv = q.to(DEV), k.to(DEV), v.to(DEV)
    for kl in (torch.tensor([300], dtype=torch.int32, device=DEV), None):
        ref16 = attention_segments(dq, [(dk, dv)], k_lens=kl, cross=True)
        ref32 = attention_segments(dq, [(dk, dv)], k_lens=kl, cross=True, out_dtype=torch.float32)
        big16 = torch.full((1, 700, 3, 136), 7.0, dtype=torch.bfloat16, device=DEV)
        big32 = torch.full((1, 700, 3, 136), 7.0, dtype=torch.float32, device=DEV)
        o16, o32 = big16[..., 4:132], big32[..., 4:132]
        attention_segments(dq, [(dk, dv)], k_lens=kl, cross=True, out=o16)
        attention_segments(dq, [(dk, dv)], k_lens=kl, cross=True, out=o32)
        torch.cuda.synchronize()
        assert torch.equal(o16, ref16) and torch.equal(o32, ref32), kl
        for big in (big16, big32):
            assert bool((big[..., :4] == 7).all()) and bool((big[..., 132:] == 7).all())


def test_cross_dedup_past_the_resident_keys(lib):
    """The exact dedup over a context whose distinct rows end past the resident chunk (400 of
    512: the distinct rows and the weighted identical ones up to their tile's end, 448 keys)
    equals the full-context oracle."""
    from lbw_amd import cross_attention
    q, k, v = _qkv(1, 700, 3, 512, seed=77)
    k[:, 400:] = k[:, 511:]
    v[:, 400:] = v[:, 511:]
    out = cross_attention(q.to(DEV), k.to(DEV), v.to(DEV), n_distinct=400)
    assert_parity(out, O.attention_ref(q, k, v), "dedup past 320")


def test_cross_window_and_strided_views(lib):
    """A key window [lo, hi) on a context held as column views of a fused [L, 2, H, D] buffer,
    q and out as strided views; bf16 output."""
    from lbw_amd import attention_segments
    g = torch.Generator().manual_seed(17)
    B, Lq, H, L = 2, 150, 3, 600
    kv = torch.randn(B, L, 2, H, 128, generator=g).to(torch.bfloat16)
    qx = torch.randn(B, Lq, 2, H, 128, generator=g).to(torch.bfloat16)
    q, k, v = qx[:, :, 0], kv[:, :, 0], kv[:, :, 1]
    d_kv, d_qx = kv.to(DEV), qx.to(DEV)
    for lo, hi in [(100, 400), (10, 600), (333, 334)]:
        out = attention_segments(d_qx[:, :, 0], [(d_kv[:, :, 0], d_kv[:, :, 1])], kv_lo=lo,
                                 kv_hi=hi, cross=True)
        assert_parity(out, O.attention_ref(q, k, v, kv_lo=lo, kv_hi=hi), f"window {lo}-{hi}")


def test_cross_full_size_wan14b_480p(lib):
    """The 14B 480p cross-attention at full size: 4680 queries x 40 heads over a 512-row context
    with rows 300.. identical (the projected zero padding); masked to 300 rows, unmasked, and
    the exact dedup, on sampled rows of 4 heads (bf16 bar), plus the dedup result against the
    unmasked one."""
    from lbw_amd import cross_attention, padding_start
    g = torch.Generator(device=DEV).manual_seed(23)
    H, Lq, L, nv = 40, 4680, 512, 300
    q = torch.randn(1, Lq, H, 128, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(1, L, H, 128, generator=g, device=DEV)
    v = 0.5 * torch.randn(1, L, H, 128, generator=g, device=DEV)
    k[:, nv:] = k[:, L - 1:]
    v[:, nv:] = v[:, L - 1:]
    k, v = k.to(torch.bfloat16), v.to(torch.bfloat16)
    kl = torch.tensor([nv], dtype=torch.int32, device=DEV)
    nd = padding_start(k, v)
    assert nd == nv
    outs = {"masked": cross_attention(q, k, v, k_lens=kl),
            "unmasked": cross_attention(q, k, v),
            "dedup": cross_attention(q, k, v, n_distinct=nd)}
    torch.cuda.synchronize()
    sel = torch.cat([torch.randperm(Lq, generator=torch.Generator().manual_seed(5))[:256],
                     torch.arange(4672, Lq)]).unique().sort().values
    qc, kc, vc = q[:, sel].cpu(), k.cpu(), v.cpu()
    for h in (0, 13, 26, 39):
        for name, out in outs.items():
            ref = O.attention_ref(qc[:, :, h:h + 1], kc[:, :, h:h + 1], vc[:, :, h:h + 1],
                                  k_lens=torch.tensor([nv]) if name == "masked" else None)
            m = assert_parity(out[:, sel][:, :, h:h + 1], ref, f"{name} head {h}")
            print(f"  {name} head {h}: {m}", flush=True)
    assert float((outs["dedup"].float() - outs["unmasked"].float()).abs().max()) <= 1e-2
