"""Pins the CPU oracle: closed forms, invariants, the reference's own known-answer table,
float64 brute force and torch's SDPA. Each check is chosen so that a plausible mistake in
the restatement (a dropped term, a wrong index or sign, a transposed operand) fails it."""
import math

import numpy as np
import pytest
import torch

import oracle as O


# ----------------------------------------------------------------------------- RoPE
def test_rope_freqs_closed_form():
    f = O.wan_rope_freqs(128)
    assert f.shape == (O.MAX_LATENT_FRAMES, 64)
    assert O.rope_axis_split(64) == (22, 21, 21)
    pos = torch.arange(O.MAX_LATENT_FRAMES).double()
    # column i of the t block: pos * 10000^(-2i/44); h and w blocks: 10000^(-2i/42)
    # columns: t = 0..21, h = 22..42, w = 43..63
    for col, (i, dim) in [(0, (0, 44)), (5, (5, 44)), (21, (21, 44)), (22, (0, 42)),
                          (30, (8, 42)), (42, (20, 42)), (43, (0, 42)), (63, (20, 42))]:
        want = pos * 10000.0 ** (-2.0 * i / dim)
        assert torch.allclose(f[:, col].double(), want, rtol=2e-6, atol=1e-6), col
    # pair 0 of every axis has inverse frequency 1: angle == position
    for col in (0, 22, 43):
        assert torch.equal(f[:, col], torch.arange(O.MAX_LATENT_FRAMES).float())


def test_rope_grid_token_order_and_identity():
    fr = O.wan_rope_freqs(128)
    f, h, w = 2, 3, 5
    cos, sin = O.causal_rope_grids(fr, f, h, w, start_frame=0)
    assert cos.shape == (f * h * w, 64)
    assert torch.all(cos[0] == 1) and torch.all(sin[0] == 0)          # position (0,0,0)
    # frame-major token order: token (fi, hi, wi) -> (fi*h + hi)*w + wi; pair 0 of each axis
    # carries that axis' position as its angle
    for fi in range(f):
        for hi in range(h):
            for wi in range(w):
                t = (fi * h + hi) * w + wi
                assert sin[t, 0] == math.sin(float(fi)) or abs(sin[t, 0] - math.sin(fi)) < 1e-6
                assert abs(sin[t, 22] - math.sin(hi)) < 1e-6
                assert abs(sin[t, 43] - math.sin(wi)) < 1e-6
    # start_frame shifts only the frame axis
    c2, s2 = O.causal_rope_grids(fr, f, h, w, start_frame=7)
    assert torch.equal(c2[:, 22:], cos[:, 22:])
    assert abs(s2[0, 0] - math.sin(7.0)) < 1e-6


def test_axis_tables_expand_to_grid_bitwise():
    fr = O.wan_rope_freqs(128)
    for (f, h, w, sf) in [(1, 45, 80, 12), (3, 30, 52, 6), (2, 3, 4, 2879 - 2)]:
        cos, sin = O.causal_rope_grids(fr, f, h, w, start_frame=sf)
        c2, s2 = O.expand_axis_tables(O.rope_axis_tables(fr, f, h, w, sf), f, h, w)
        assert torch.equal(cos, c2) and torch.equal(sin, s2)


def test_rope_rotation_norm_and_relative_position():
    torch.manual_seed(0)
    fr = O.wan_rope_freqs(128)
    H, D = 2, 128
    f, h, w = 3, 4, 5
    L = f * h * w
    x = torch.randn(L, H, D, dtype=torch.float64).float()
    cos, sin = O.causal_rope_grids(fr, f, h, w, start_frame=3)
    y = O.rope_apply_rotation(x, cos, sin)
    # rotation preserves every pair's norm
    n0 = x.view(L, H, 64, 2).norm(dim=-1)
    n1 = y.view(L, H, 64, 2).norm(dim=-1)
    assert torch.allclose(n0, n1, rtol=1e-5, atol=1e-5)
    # <R(p) q, R(p') k> depends only on p - p' per axis: shifting start_frame of both
    # leaves every dot product unchanged (a wrong sign or pair index breaks this)
    q = torch.randn(L, H, D)
    k = torch.randn(L, H, D)
    cA, sA = O.causal_rope_grids(fr, f, h, w, start_frame=0)
    cB, sB = O.causal_rope_grids(fr, f, h, w, start_frame=9)
    dA = torch.einsum("ihd,jhd->hij", O.rope_apply_rotation(q, cA, sA).double(),
                      O.rope_apply_rotation(k, cA, sA).double())
    dB = torch.einsum("ihd,jhd->hij", O.rope_apply_rotation(q, cB, sB).double(),
                      O.rope_apply_rotation(k, cB, sB).double())
    assert torch.allclose(dA, dB, rtol=1e-4, atol=2e-3)
    # the rotation direction: pair j at angle a maps (1, 0) to (cos a, sin a)
    e = torch.zeros(L, 1, D)
    e[:, :, 0] = 1.0
    r = O.rope_apply_rotation(e, cos, sin)
    assert torch.allclose(r[:, 0, 0], cos[:, 0]) and torch.allclose(r[:, 0, 1], sin[:, 0])


def test_rope_rows_past_grid_pass_through():
    fr = O.wan_rope_freqs(128)
    cos, sin = O.causal_rope_grids(fr, 1, 2, 3)
    x = torch.randn(10, 1, 128)
    y = O.rope_apply_rotation(x, cos, sin)
    assert torch.equal(y[6:], x[6:])


# ----------------------------------------------------------------------------- RMSNorm
def test_rms_norm_closed_forms():
    C = 64
    g = torch.linspace(0.5, 1.5, C)
    # constant row c -> sign(c) * g / sqrt(1 + eps / c^2); zero row -> 0
    for c in (3.0, -0.25, 1e-2):
        x = torch.full((1, C), c)
        y = O.rms_norm_module(x, g, eps=1e-6)
        want = math.copysign(1.0, c) / math.sqrt(1 + 1e-6 / c ** 2) * g
        assert torch.allclose(y[0], want, rtol=1e-6)
    assert torch.all(O.rms_norm_module(torch.zeros(1, C), g) == 0)
    # the statistic is a MEAN over the row: a row of (a, -a, a, -a ...) has rms |a|
    x = torch.tensor([[2.0, -2.0] * (C // 2)])
    assert torch.allclose(O.rms_norm_module(x, torch.ones(C), eps=0.0), x / 2.0)


def test_qk_post_sequence_closed_form():
    C, D = 256, 128
    fr = O.wan_rope_freqs(D)
    cos, sin = O.causal_rope_grids(fr, 1, 1, 3, start_frame=0)
    x = torch.full((3, C), 0.75).to(torch.bfloat16)
    b = torch.full((C,), 0.25).to(torch.bfloat16)
    w = torch.full((C,), 2.0)
    out = O.qk_post_norm_rope(x, b, w, cos, sin, eps=1e-6).float()
    # token 0 sits at position (0, 0, 0): identity rotation, every feature = 2/sqrt(1+eps)
    want = 2.0 / math.sqrt(1.0 + 1e-6)
    assert torch.allclose(out[0], torch.full((C,), want).to(torch.bfloat16).float())
    # token 2 (w = 2): pair 43 (w axis, inverse frequency 1) has (t, t) rotated by 2 rad
    t = 2.0
    re = t * math.cos(2.0) - t * math.sin(2.0)
    im = t * math.sin(2.0) + t * math.cos(2.0)
    assert abs(out[2, 86] - re) < 2e-2 and abs(out[2, 87] - im) < 2e-2
    # the sum of squares spans the whole row (all heads) and includes the bias
    ss = O.qk_post_ss(x, b)
    assert torch.allclose(ss, torch.full((3,), C * 1.0))


def test_qk_post_matches_module_sequence_within_one_rounding():
    torch.manual_seed(1)
    L, C, D = 40, 512, 128
    fr = O.wan_rope_freqs(D)
    cos, sin = O.causal_rope_grids(fr, 1, 5, 8, start_frame=2)
    x = torch.randn(L, C).to(torch.bfloat16)
    g = (1 + 0.1 * torch.randn(C)).to(torch.bfloat16)
    fused = O.qk_post_norm_rope(x, None, g, cos, sin).float()
    mod = O.rms_norm_module(x[None], g, 1e-6)[0]                     # bf16 x gamma rounding
    mod = O.rope_apply_rotation(mod.view(L, C // D, D), cos, sin).reshape(L, C)
    assert (fused - mod.float()).abs().max() < 3e-2
    assert (fused - mod.float()).abs().mean() < 2e-3


def _qk_post_t_inputs(L=2176, F=1280, SEQ=2160, seed=0):
    """perf/qk_post_t_test.py:18-29's inputs: q, k x1.5, bias x0.2, gamma 1 + 0.1 N, random
    angles for the first SEQ rows and identity rows after them."""
    g = torch.Generator().manual_seed(seed)
    C = 64
    q = (torch.randn(L, F, generator=g) * 1.5).to(torch.bfloat16)
    k = (torch.randn(L, F, generator=g) * 1.5).to(torch.bfloat16)
    bq = (torch.randn(F, generator=g) * 0.2).to(torch.bfloat16)
    bk = (torch.randn(F, generator=g) * 0.2).to(torch.bfloat16)
    wq = (1 + torch.randn(F, generator=g) * 0.1).to(torch.bfloat16)
    wk = (1 + torch.randn(F, generator=g) * 0.1).to(torch.bfloat16)
    ang = torch.rand(SEQ, C, generator=g) * 6.28
    return q, k, bq, bk, wq, wk, ang.cos(), ang.sin()


def test_qk_post_t_scale_rides_on_cos_sin():
    """The _t variants' q scale (qk_post.py:259-265): exact for a power of two (scaling
    commutes with every rounding), and against the reference test's own fp32 formula
    (perf/qk_post_t_test.py:32-41: rotate, then x 1/sqrt(D)) within bf16 rounding."""
    q, k, bq, bk, wq, wk, cos, sin = _qk_post_t_inputs()
    L, F = q.shape
    one = O.qk_post_norm_rope(q, bq, wq, cos, sin)
    quarter = O.qk_post_norm_rope(q, bq, wq, cos, sin, out_scale=0.25)
    assert torch.equal(quarter, (one.float() * 0.25).to(torch.bfloat16))
    qs = 1.0 / math.sqrt(128)
    got = O.qk_post_norm_rope(q, bq, wq, cos, sin, out_scale=qs).float()
    y = q.float() + bq.float()
    r = torch.rsqrt((y * y).sum(-1) / F + 1e-6)
    t = (y * r[:, None]).to(torch.bfloat16).float() * wq.float()
    t4 = t.view(L, F // 128, 64, 2)
    cb = torch.cat([cos, torch.ones(L - cos.shape[0], 64)])[:, None, :]
    sb = torch.cat([sin, torch.zeros(L - sin.shape[0], 64)])[:, None, :]
    want = torch.stack([t4[..., 0] * cb - t4[..., 1] * sb, t4[..., 0] * sb + t4[..., 1] * cb],
                       -1).reshape(L, F) * qs
    assert ((got - want).norm() / want.norm()).item() < 3e-3
    assert ((got - want).abs() <= want.abs() * 2.0 ** -7 + 1e-3).float().mean() > 0.999
    # rows past the grid are scaled only
    assert torch.allclose(got[2160:], (t[2160:] * qs).to(torch.bfloat16).float())


def test_qk_post_t_layout_is_head_major_d_major():
    q, k, bq, bk, wq, wk, cos, sin = _qk_post_t_inputs(L=40, F=384, SEQ=33)
    rows = O.qk_post_norm_rope(k, bk, wk, cos, sin)
    t = O.qk_post_norm_rope_t(k, bk, wk, cos, sin)
    assert t.shape == (3, 128, 40)
    for h, d, l in [(0, 0, 0), (1, 5, 7), (2, 127, 39), (2, 3, 35)]:
        assert t[h, d, l] == rows[l, 128 * h + d]
    assert torch.equal(t.permute(2, 0, 1).reshape(40, 384), rows)


# ----------------------------------------------------------------------------- attention
def _qkv(B, Lq, Lk, H, D, seed=0, gain=1.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Lq, H, D, generator=g) * gain
    k = torch.randn(B, Lk, H, D, generator=g)
    v = torch.randn(B, Lk, H, D, generator=g)
    return q, k, v


def test_attention_matches_sdpa_with_window():
    q, k, v = _qkv(2, 37, 91, 3, 64, seed=3, gain=2.0)
    for lo, hi in [(0, 91), (10, 70), (0, 1), (90, 91)]:
        ref = O.sdpa_ref(q, k, v, attn_mask=O.window_mask(91, lo, hi))
        got = O.attention_ref(q, k, v, kv_lo=lo, kv_hi=hi, q_block=16)
        assert torch.allclose(got, ref, atol=2e-6, rtol=1e-5), (lo, hi)


def test_attention_matches_f64_bruteforce():
    q, k, v = _qkv(1, 5, 23, 2, 16, seed=4, gain=3.0)
    ref = O.attention_brute_f64(q, k, v, lo=4, hi=19)
    got = O.attention_ref(q, k, v, kv_lo=4, kv_hi=19).double().numpy()
    assert np.abs(got - ref).max() < 1e-5


def test_attention_empty_window_is_zero_like_sdpa():
    q, k, v = _qkv(1, 4, 8, 1, 16)
    got = O.attention_ref(q, k, v, kv_lo=5, kv_hi=5)
    ref = O.sdpa_ref(q, k, v, attn_mask=O.window_mask(8, 5, 5))
    assert torch.all(got == 0) and torch.allclose(got, ref)


def test_attention_special_cases():
    q, k, v = _qkv(1, 6, 10, 2, 32, seed=5)
    # one key -> its value
    got = O.attention_ref(q, k, v, kv_lo=3, kv_hi=4)
    assert torch.allclose(got, v[:, 3:4].expand(1, 6, 2, 32), atol=1e-6)
    # identical keys -> the mean of their values
    kk = k.clone()
    kk[:, :] = k[:, :1]
    got = O.attention_ref(q, kk, v)
    assert torch.allclose(got, v.mean(1, keepdim=True).expand_as(got), atol=1e-5)
    # key permutation invariance (with matching V)
    perm = torch.randperm(10)
    a = O.attention_ref(q, k, v)
    b = O.attention_ref(q, k[:, perm], v[:, perm])
    assert torch.allclose(a, b, atol=1e-6)
    # a uniform shift of every score of a row changes nothing: add a multiple of the
    # query to... every key's component along a fixed direction orthogonal to nothing is
    # not uniform, so shift via an extra constant dimension instead
    q2 = torch.cat([q, torch.ones(1, 6, 2, 1)], -1)
    k2 = torch.cat([k, torch.zeros(1, 10, 2, 1)], -1)
    k3 = torch.cat([k, torch.full((1, 10, 2, 1), 5.0)], -1)
    assert torch.allclose(O.attention_ref(q2, k2, v, softmax_scale=0.2),
                          O.attention_ref(q2, k3, v, softmax_scale=0.2), atol=1e-5)


def test_k_lens_masks_per_batch():
    q, k, v = _qkv(2, 7, 30, 2, 32, seed=6)
    got = O.attention_ref(q, k, v, k_lens=[12, 30])
    ref0 = O.sdpa_ref(q[:1], k[:1, :12], v[:1, :12])
    ref1 = O.sdpa_ref(q[1:], k[1:], v[1:])
    assert torch.allclose(got[:1], ref0, atol=2e-6) and torch.allclose(got[1:], ref1, atol=2e-6)


def test_partials_merge_equals_full():
    q, k, v = _qkv(1, 33, 120, 2, 32, seed=7, gain=4.0)
    full = O.attention_ref(q, k, v)
    parts = []
    for lo, hi in [(0, 50), (50, 51), (51, 120)]:
        _, p = O.attention_ref(q, k[:, lo:hi], v[:, lo:hi], return_partials=True)
        parts.append(p)
    merged = O.merge_partials(parts)
    assert torch.allclose(merged, full, atol=2e-6)
    # a partial's m is the row max of the scaled scores
    _, (po, pm, pl) = O.attention_ref(q, k, v, return_partials=True)
    s = torch.einsum("qhd,khd->hqk", q[0], k[0]) / math.sqrt(32)
    assert torch.allclose(pm[0], s.max(-1).values, atol=1e-5)
    assert torch.allclose(pl[0], torch.exp(s - s.max(-1, keepdim=True).values).sum(-1), rtol=1e-5)


# ----------------------------------------------------------------------------- caches
def test_chunk_routing_reference_table():
    """chunked_kv_cache.py:54-59, window 12 / chunk 3 -> n_chunks 4."""
    n = O.num_chunks(12, 3)
    assert n == 4
    table = {0: (0, ()), 1: (1, (0,)), 2: (2, (0, 1)), 3: (3, (0, 1, 2)),
             4: (1, (0, 2, 3)), 5: (2, (0, 1, 3))}
    for i, want in table.items():
        assert O.chunk_routing(i, n) == want
    assert O.num_chunks(-1, 3) == 0 and O.chunk_routing(7, 1) == (0, ())


@pytest.mark.parametrize("n", [2, 3, 4, 6])
def test_ordered_chunks_sink_first_destination_last(n):
    """chunked_kv_cache.py:47-76, 172-177: simulate the chunked cache writing chunk i (its
    token ids) into the routed slot; the ordered buffers the attention then reads must be
    the sink chunk 0 first (once one more chunk exists), the chunk just written last (the
    destination: the entry the write goes to), and exactly the sink plus the most recent
    n - 1 chunks, each once. A destination placed first, a reversed leading order or a
    missing slot fails one of these."""
    slots = [None] * n
    for i in range(4 * n + 3):
        dest, lead = O.chunk_routing(i, n)
        slots[dest] = i
        order = O.ordered_chunks(slots, dest, lead)
        assert order[-1] == i
        if i >= 1:
            assert order[0] == 0
        recent = list(range(max(1, i - (n - 2)), i + 1)) if i >= 1 else [0]
        want = sorted(set([0] + recent))
        assert sorted(order) == want and len(order) == len(want)


def test_flat_cache_plan_keeps_sink_and_recent_window():
    """Simulate the windowed flat cache over many chunks with token ids: the sink frames
    stay at the front, the rest of the window holds the most recent tokens in order."""
    frame, sink_f, window_f, chunk_f = 4, 1, 6, 2
    size = window_f * frame
    cache = [-1] * size
    g_end = l_end = 0
    for c in range(8):
        start = c * chunk_f * frame
        n = chunk_f * frame
        p = O.flat_cache_write_plan(size, g_end, l_end, start, n, sink_f * frame,
                                    max_attention_size=size)
        if p["roll"] is not None:
            dst, src, ln = p["roll"]
            cache[dst:dst + ln] = cache[src:src + ln]
        s, e = p["write"]
        assert e - s == n and 0 <= s and e <= size
        cache[s:e] = list(range(start, start + n))
        g_end, l_end = p["global_end"], p["local_end"]
        win = cache[p["attn_lo"]:p["attn_hi"]]
        seen = start + n
        if seen <= size:
            assert win == list(range(seen))
        else:
            assert win[:sink_f * frame] == list(range(sink_f * frame))
            rest = size - sink_f * frame
            assert win[sink_f * frame:] == list(range(seen - rest, seen))


# ----------------------------------------------------------------------------- fp8
def test_fp8_decode_table_and_library_cast():
    codes = torch.arange(256, dtype=torch.int64).to(torch.uint8)
    ours = O.fp8_e4m3_decode(codes)
    lib = codes.view(torch.float8_e4m3fn).float()
    fin = ~torch.isnan(lib)
    assert torch.equal(torch.isnan(ours), torch.isnan(lib)) and torch.equal(ours[fin], lib[fin])
    assert ours[0x7E] == 448.0 and ours[0x38] == 1.0 and ours[0x08] == 2.0 ** -6
    assert ours[0x01] == 2.0 ** -9 and ours[0xFE] == -448.0 and int(torch.isnan(ours).sum()) == 2


def test_fp8_quantizer_round_trip_and_scale_layout():
    g = torch.Generator().manual_seed(8)
    x = torch.randn(1, 150, 3, 16, generator=g)
    x[0, 70, 1, 5] = 40.0                                       # an outlier in block 1, head 1
    codes, sc = O.quantize_kv_fp8(x, block=64)
    assert sc.shape == (1, 3, 3)
    # scales are the smallest powers of two with amax / scale <= 448: 40 -> 2^-3, 40 / 2^-3 =
    # 320 = 1.25 * 2^8, e4m3 code 0x7A (exponent field 15, mantissa 010)
    assert sc[0, 1, 1] == 0.125 and codes[0, 70, 1, 5] == 0x7A
    mant, _ = torch.frexp(sc)
    assert torch.all(mant == 0.5)                                # powers of two
    amax = x.abs().view(1, 150, 3, 16)
    amax = torch.cat([amax, torch.zeros(1, 42, 3, 16)], 1).view(1, 3, 64, 3, 16).amax(dim=(2, 4))
    ratio = amax.permute(0, 2, 1) / sc
    assert torch.all(ratio <= 448) and torch.all(ratio > 224)   # the smallest such power
    # the edges: amax = 448 * 2^k -> scale 2^k exactly; just above -> 2^(k+1)
    for v, want in ((448.0 * 2.0 ** -5, 2.0 ** -5), (448.0 * 2.0 ** -5 * (1 + 2.0 ** -20), 2.0 ** -4),
                    (448.0, 1.0), (1.0, 2.0 ** -8), (1.75, 2.0 ** -8), (1.75 * (1 + 2.0 ** -20), 2.0 ** -7)):
        _, s1 = O.quantize_kv_fp8(torch.full((1, 64, 1, 4), v))
        assert float(s1[0, 0, 0]) == want, (v, float(s1[0, 0, 0]), want)
    deq = O.dequantize_kv_fp8(codes, sc)
    s_tok = sc.permute(0, 2, 1).repeat_interleave(64, 1)[:, :150].unsqueeze(-1)
    # RNE error bound: half a step of 2^-3 relative for normals, 2^-10 * scale for subnormals
    bound = torch.maximum(x.abs() * 2.0 ** -4, s_tok * 2.0 ** -10) * 1.0001
    assert torch.all((deq - x).abs() <= bound)
    z = torch.zeros(1, 64, 1, 8)
    c0, s0 = O.quantize_kv_fp8(z)
    assert torch.all(c0 == 0) and torch.all(s0 == 1)


def test_layer_ref_zero_qk_weights_give_mean_of_values():
    """Zero q/k projections and biases: q = k = RMSNorm(0) = 0, every score is 0, so each
    output row is Wo (mean over all cached and chunk V rows) + bo."""
    g = torch.Generator().manual_seed(21)
    C, H = 256, 2
    x = torch.randn(1, 12, C, generator=g)
    xc = torch.randn(1, 24, C, generator=g)
    z = torch.zeros(C, C)
    zb = torch.zeros(C)
    wv, wo = torch.randn(C, C, generator=g) * 0.05, torch.randn(C, C, generator=g) * 0.05
    bv, bo = torch.randn(C, generator=g), torch.randn(C, generator=g)
    out = O.self_attention_layer_ref(x, xc, z, zb, z, zb, wv, bv, wo, bo, torch.ones(C),
                                     torch.ones(C), heads=H, grid=(1, 3, 4),
                                     cache_grid=(2, 3, 4), start_frame=2)
    vmean = (torch.cat([xc, x], 1)[0].double() @ wv.double().T + bv.double()).mean(0)
    ref = vmean @ wo.double().T + bo.double()
    assert torch.allclose(out[0].double(), ref.expand(12, C), atol=1e-5)


def test_layer_ref_shifting_all_frames_changes_nothing():
    """RoPE depends on position differences only: moving the chunk and the cached frames by
    the same number of frames leaves the layer output unchanged (a wrong start_frame in either
    the chunk's or the cache's grid breaks this)."""
    g = torch.Generator().manual_seed(22)
    C, H = 256, 2
    x = torch.randn(1, 12, C, generator=g)
    xc = torch.randn(1, 24, C, generator=g)
    ws = [torch.randn(C, C, generator=g) * 0.1 for _ in range(4)]
    bs = [torch.randn(C, generator=g) * 0.1 for _ in range(4)]
    gq, gk = 1 + 0.1 * torch.randn(C, generator=g), 1 + 0.1 * torch.randn(C, generator=g)
    args = (x, xc, ws[0], bs[0], ws[1], bs[1], ws[2], bs[2], ws[3], bs[3], gq, gk)
    a = O.self_attention_layer_ref(*args, heads=H, grid=(1, 3, 4), cache_grid=(2, 3, 4),
                                   start_frame=2, cache_start_frame=0)
    b = O.self_attention_layer_ref(*args, heads=H, grid=(1, 3, 4), cache_grid=(2, 3, 4),
                                   start_frame=9, cache_start_frame=7)
    c = O.self_attention_layer_ref(*args, heads=H, grid=(1, 3, 4), cache_grid=(2, 3, 4),
                                   start_frame=3, cache_start_frame=0)
    assert torch.allclose(a, b, atol=2e-5)
    assert not torch.allclose(a, c, atol=1e-3)


def _seq_weights(C, g):
    ws = [torch.randn(C, C, generator=g) * 0.1 for _ in range(4)]
    bs = [torch.randn(C, generator=g) * 0.1 for _ in range(4)]
    gq, gk = 1 + 0.1 * torch.randn(C, generator=g), 1 + 0.1 * torch.randn(C, generator=g)
    return (ws[0], bs[0], ws[1], bs[1], ws[2], bs[2], ws[3], bs[3], gq, gk)


def test_windowed_sequence_without_eviction_equals_layer_over_all_frames():
    """A cache large enough never to evict: chunk i attends frames 0..i, which is the layer
    reference over the i cached frames (contiguous grid from frame 0) plus the chunk."""
    g = torch.Generator().manual_seed(24)
    C, H, hw = 256, 2, (3, 4)
    xs = [torch.randn(1, 12, C, generator=g) for _ in range(4)]
    wts = _seq_weights(C, g)
    outs = O.windowed_layer_sequence_ref(xs, *wts, heads=H, frame_hw=hw, kv_cache_size=48,
                                         sink_tokens=12, max_attention_size=48)
    for i in range(1, 4):
        ref = O.self_attention_layer_ref(xs[i], torch.cat(xs[:i], 1), *wts, heads=H,
                                         grid=(1, *hw), cache_grid=(i, *hw), start_frame=i,
                                         cache_start_frame=0)
        assert torch.allclose(outs[i], ref, atol=2e-5), i


def test_windowed_sequence_with_eviction_attends_recent_frames():
    """Cache of 5 frames with a 1-frame sink and a 4-frame attention window: once the cache
    rolls, the window [end - 4 frames, end) holds exactly frames i-3..i (the sink sits before
    it), so chunk i equals the layer reference over frames max(0, i-3)..i-1 plus the chunk.
    A wrong roll (source, destination or length) puts other frames in the window."""
    g = torch.Generator().manual_seed(25)
    C, H, hw, F = 256, 2, (3, 4), 12
    xs = [torch.randn(1, F, C, generator=g) for _ in range(9)]
    wts = _seq_weights(C, g)
    outs = O.windowed_layer_sequence_ref(xs, *wts, heads=H, frame_hw=hw, kv_cache_size=5 * F,
                                         sink_tokens=F, max_attention_size=4 * F)
    for i in range(1, 9):
        f0 = max(0, i - 3)
        ref = O.self_attention_layer_ref(xs[i], torch.cat(xs[f0:i], 1), *wts, heads=H,
                                         grid=(1, *hw), cache_grid=(i - f0, *hw),
                                         start_frame=i, cache_start_frame=f0)
        assert torch.allclose(outs[i], ref, atol=2e-5), i


def test_cross_kv_ref_closed_forms():
    """K = RMSNorm(ctx Wk + bk) is scale invariant (bk = 0) and zero for a zero context;
    V = ctx Wv + bv is affine."""
    g = torch.Generator().manual_seed(23)
    C, H = 256, 2
    ctx = torch.randn(1, 10, C, generator=g)
    ctx[:, 7:] = 0
    wk, wv = torch.randn(C, C, generator=g) * 0.05, torch.randn(C, C, generator=g) * 0.05
    bv = torch.randn(C, generator=g)
    gk = 1 + 0.1 * torch.randn(C, generator=g)
    k1, v1 = O.cross_kv_ref(ctx, wk, torch.zeros(C), wv, bv, gk, H)
    k3, v3 = O.cross_kv_ref(3 * ctx, wk, torch.zeros(C), wv, bv, gk, H)
    assert torch.allclose(k1[:, :7], k3[:, :7], atol=1e-5)
    assert torch.all(k1[:, 7:] == 0)
    assert torch.allclose(v1[:, 7:], bv.view(1, 1, H, -1).expand(1, 3, H, C // H))
    assert torch.allclose((v3 - bv.view(H, -1)), 3 * (v1 - bv.view(H, -1)), atol=1e-4)
    # per-row RMS of K / gamma is 1 (the norm's defining property)
    kk = (k1[0, :7].reshape(7, C) / gk)
    assert torch.allclose(kk.pow(2).mean(-1), torch.ones(7), atol=1e-4)


def test_cross_dedup_forms_equal_full_attention():
    """attention.py:516-523: identical padding rows can share one softmax term weighted by their
    count. Full attention over all L rows == the reference's kc-row slice with the
    cross_dedup_bias == the minimal form (distinct rows + one padding row, bias log(m))."""
    g = torch.Generator().manual_seed(31)
    L, n_valid, H, D = 64, 23, 2, 16
    k = torch.randn(1, L, H, D, generator=g)
    v = torch.randn(1, L, H, D, generator=g)
    k[:, n_valid:] = torch.randn(1, 1, H, D, generator=g)    # padding rows: one repeated row
    v[:, n_valid:] = torch.randn(1, 1, H, D, generator=g)
    q = torch.randn(1, 9, H, D, generator=g)
    full = O.attention_ref(q, k, v)
    kc = 32
    bias = O.cross_dedup_bias(k[0], v[0], kc)
    assert int((bias != 0).sum()) == kc - n_valid
    ref_form = O.attention_key_bias_ref(q, k[:, :kc], v[:, :kc], bias)
    minimal_bias = torch.zeros(n_valid + 1)
    minimal_bias[-1] = math.log(L - n_valid)
    minimal = O.attention_key_bias_ref(q, k[:, :n_valid + 1], v[:, :n_valid + 1], minimal_bias)
    assert torch.allclose(ref_form, full, atol=1e-5) and torch.allclose(minimal, full, atol=1e-5)
