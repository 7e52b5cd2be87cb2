"""GPU parity of the chunk flash-attention kernel (lbw_attention_fwd / lbw_cross_attention_fwd)
against the fp32 CPU oracle, through the product wrappers over the C ABI."""
import math

import pytest
import torch

import oracle as O
from parity import assert_parity, metrics

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _rand(shape, g, scale=1.0):
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def _gains(H):
    base = torch.tensor([0.25, 0.5, 1.0, 2.0, 4.0, 8.0, 16.0, 1.0])
    return base[torch.arange(H) % len(base)]


def _case(B, Lq, H, seg_lens, seed, gain=True):
    g = torch.Generator().manual_seed(seed)
    q = _rand((B, Lq, H, 128), g)
    if gain:
        q = (q.float() * _gains(H).view(1, 1, H, 1)).to(torch.bfloat16)
    ks = [_rand((B, L, H, 128), g) for L in seg_lens]
    vs = [_rand((B, L, H, 128), g) for L in seg_lens]
    return q, ks, vs


@pytest.mark.parametrize("B,Lq,H,seg_lens,window", [
    (1, 300, 2, [1000], None),
    (1, 37, 3, [64], None),
    (1, 1, 1, [1], None),
    (1, 257, 2, [65], None),
    (2, 129, 2, [100, 37, 200, 5], (50, 300)),
    (1, 512, 4, [4096, 1560], (1000, 5656)),
    (1, 96, 2, [7, 0, 130], None),
])
def test_attention_matches_oracle(lib, B, Lq, H, seg_lens, window):
    from lbw_amd import attention_segments
    q, ks, vs = _case(B, Lq, H, seg_lens, seed=Lq + H)
    lo, hi = (None, None) if window is None else window
    out = attention_segments(q.to(DEV), [(k.to(DEV), v.to(DEV)) for k, v in zip(ks, vs)],
                             kv_lo=lo, kv_hi=hi)
    ref = O.attention_ref(q, torch.cat(ks, 1), torch.cat(vs, 1), kv_lo=lo, kv_hi=hi)
    print(f"case B={B} Lq={Lq} H={H} segs={seg_lens} window={window}", metrics(out, ref))
    assert_parity(out, ref)


def test_attention_dropin_signature_and_mask(lib):
    from lbw_amd import attention, flash_attention
    q, ks, vs = _case(1, 200, 2, [777], seed=5)
    k, v = ks[0], vs[0]
    mask = O.window_mask(777, 100, 650)
    ref = O.sdpa_ref(q, k, v, attn_mask=mask)
    out = attention(q.to(DEV), k.to(DEV), v.to(DEV), attn_mask=mask.to(DEV))
    assert out.shape == q.shape and out.dtype == torch.bfloat16
    assert_parity(out, ref, "attn_mask")
    out2 = flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), kv_lo=torch.tensor(100),
                           kv_hi=torch.tensor(650))
    assert torch.equal(out, out2)
    with pytest.raises(NotImplementedError):
        attention(q.to(DEV), k.to(DEV), v.to(DEV), causal=True)


def test_strided_views_from_fused_qkv(lib):
    from lbw_amd import attention_segments
    g = torch.Generator().manual_seed(11)
    B, L, H = 2, 333, 3
    qkv = _rand((B, L, 3, H, 128), g)
    q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
    out = attention_segments(q.to(DEV), [(k.to(DEV), v.to(DEV))])
    d = qkv.to(DEV)
    out_v = attention_segments(d[:, :, 0], [(d[:, :, 1], d[:, :, 2])])
    ref = O.attention_ref(q, k, v)
    assert_parity(out_v, ref, "strided")
    assert torch.equal(out, out_v)


def test_empty_window_gives_zero(lib):
    from lbw_amd import attention_segments
    q, ks, vs = _case(1, 70, 2, [300], seed=3)
    out = attention_segments(q.to(DEV), [(ks[0].to(DEV), vs[0].to(DEV))], kv_lo=120, kv_hi=120)
    assert torch.all(out == 0)


@pytest.mark.parametrize("splits", [2, 3, 7])
def test_split_kv_merge_matches_single_pass(lib, splits):
    from lbw_amd import attention_segments
    q, ks, vs = _case(1, 300, 2, [3000, 600], seed=splits)
    segs = [(k.to(DEV), v.to(DEV)) for k, v in zip(ks, vs)]
    one = attention_segments(q.to(DEV), segs, num_splits=1)
    many = attention_segments(q.to(DEV), segs, num_splits=splits)
    ref = O.attention_ref(q, torch.cat(ks, 1), torch.cat(vs, 1))
    assert_parity(one, ref, "single")
    assert_parity(many, ref, f"splits={splits}")
    assert (one.float() - many.float()).abs().max() < 4e-3


@pytest.mark.parametrize("B,Lq,H,Lk,splits", [
    (1, 40, 1, 700, 3),      # one unit: seven XCD queues empty, their workgroups take from XCD 0
    (1, 300, 3, 900, 2),     # six units, ragged last q-tile
    (2, 513, 3, 333, 5),     # batch 2, 18 units, pieces of 1-2 tiles
    (1, 256, 5, 130, 7),     # more pieces than tiles: empty pieces merge as nothing
    (3, 100, 7, 2000, 1),    # 21 units, single pass through the queues
])
def test_work_queue_covers_every_item(lib, B, Lq, H, Lk, splits):
    """The per-XCD work queues with stealing hand every (piece, batch, head, q-tile) item to
    exactly one workgroup for unit counts below, at and above the XCD count, with pieces that
    hold no tiles, and with batch > 1."""
    from lbw_amd import attention_segments
    q, ks, vs = _case(B, Lq, H, [Lk], seed=B * 1000 + Lq + splits)
    # V halved (exact in bf16): with a few hundred keys a peaked head copies single V rows, and
    # |o| >= 4 would put one bf16 output rounding above the 1e-2 bound
    v = (vs[0].float() * 0.5).to(torch.bfloat16)
    out = attention_segments(q.to(DEV), [(ks[0].to(DEV), v.to(DEV))], num_splits=splits)
    ref = O.attention_ref(q, ks[0], v)
    print(f"queue case B={B} Lq={Lq} H={H} Lk={Lk} splits={splits}", metrics(out, ref))
    assert_parity(out, ref, f"B={B} Lq={Lq} H={H} Lk={Lk} splits={splits}")


@pytest.mark.parametrize("jump", [2.0, 12.0, 60.0])
def test_exponent_reference_moves_mid_row(lib, jump):
    """Scores that rise tile after tile (by `jump` natural-log units per 64-key tile along one
    direction of q): the row maximum keeps moving, so the exponentials computed against the
    current reference outgrow 2^16 (jump 2.0: every few tiles; 12.0: every tile, and without a
    move they would pass fp32's range by the last tile; 60.0: they overflow to +inf at once) and
    the step must move the reference and redo them. Against the oracle, in the single-pass and
    the 3-split path, and through the partials (exact row max). With the redo switched off the
    12.0 and 60.0 cases fail."""
    from lbw_amd import attention_partial, attention_segments
    g = torch.Generator().manual_seed(31)
    B, Lq, H, L = 1, 70, 2, 12 * 64 + 17
    u = torch.randn(128, generator=g)
    u = u / u.norm()
    q = (torch.randn(B, Lq, H, 128, generator=g) * 0.3 + 4.0 * u).to(torch.bfloat16)
    ramp = torch.arange(L, dtype=torch.float32).div(64).floor()          # tile index per key
    # q . k gains ~ jump per tile in softmax units (scale 1/sqrt(128), |q . u| ~ 4)
    gain = (ramp * jump * math.sqrt(128) / 4.0).view(1, L, 1, 1)
    k = (torch.randn(B, L, H, 128, generator=g) * 0.3 + gain * u).to(torch.bfloat16)
    v = (torch.randn(B, L, H, 128, generator=g) * 0.5).to(torch.bfloat16)
    ref = O.attention_ref(q, k, v)
    for splits in (1, 3):
        out = attention_segments(q.to(DEV), [(k.to(DEV), v.to(DEV))], num_splits=splits)
        assert_parity(out, ref, f"jump {jump} splits {splits}")
    po, pm, pl = attention_partial(q.to(DEV), [(k.to(DEV), v.to(DEV))])
    _, (ro, rm, rl) = O.attention_ref(q, k, v, return_partials=True)
    assert torch.allclose(pm.cpu(), rm, rtol=1e-4, atol=1e-3)  # fp32 sums of ~1e4-sized scores


def test_partials_match_oracle_and_merge(lib):
    from lbw_amd import attention_merge, attention_partial
    q, ks, vs = _case(1, 150, 2, [500, 260], seed=21)
    parts_gpu = [attention_partial(q.to(DEV), [(k.to(DEV), v.to(DEV))]) for k, v in zip(ks, vs)]
    for (po, pm, pl), k, v in zip(parts_gpu, ks, vs):
        _, (ro, rm, rl) = O.attention_ref(q, k, v, return_partials=True)
        assert torch.allclose(pm.cpu(), rm, rtol=1e-5, atol=1e-4)
        assert torch.allclose(pl.cpu(), rl, rtol=5e-3, atol=1e-3)
        assert (po.cpu() - ro).abs().max() <= 1e-2 * max(1.0, float(rl.max()))
    merged = attention_merge(parts_gpu)
    ref = O.attention_ref(q, torch.cat(ks, 1), torch.cat(vs, 1))
    assert_parity(merged, ref, "merge")


def test_chain_over_key_sets_equals_union(lib):
    """cte_call's chain (attention.py:654-694): calls over the cached chunks, then the new
    chunk, continue one softmax; the normalizing call equals attention over all the keys."""
    from lbw_amd import attention_chain
    q, ks, vs = _case(1, 300, 3, [700, 450, 300], seed=11)
    segs = [(k.to(DEV), v.to(DEV)) for k, v in zip(ks, vs)]
    state = attention_chain(q.to(DEV), segs[:2])          # cached chunks (two segments)
    state = attention_chain(q.to(DEV), segs[2:3], state)  # the new chunk
    out = attention_chain(q.to(DEV), [], state, normalize=True)
    ref = O.attention_ref(q, torch.cat(ks, 1), torch.cat(vs, 1))
    assert_parity(out, ref, "chain")
    # the same keys in one call
    one = attention_chain(q.to(DEV), segs, normalize=True)
    assert (one.float() - out.float()).abs().max() < 4e-3


def test_cross_attention_masked_and_unmasked(lib):
    from lbw_amd import attention, cross_attention
    g = torch.Generator().manual_seed(7)
    B, Lq, H = 2, 333, 4
    q = _rand((B, Lq, H, 128), g)
    k = _rand((B, 512, H, 128), g)
    v = _rand((B, 512, H, 128), g)
    k_lens = torch.tensor([300, 512], dtype=torch.int32)
    out = cross_attention(q.to(DEV), k.to(DEV), v.to(DEV), k_lens=k_lens.to(DEV))
    ref = O.attention_ref(q, k, v, k_lens=k_lens)
    assert_parity(out, ref, "masked")
    out_u = attention(q.to(DEV), k.to(DEV), v.to(DEV), is_cross_attn=True)
    assert_parity(out_u, O.attention_ref(q, k, v), "unmasked")
    # peaked rows (query gain 4): outputs approach single V rows, |o| up to ~4, where one bf16
    # step is 2^-6; bound the error relative to the output's scale instead
    q4 = (q.float() * 4).to(torch.bfloat16)
    out4 = cross_attention(q4.to(DEV), k.to(DEV), v.to(DEV), k_lens=k_lens.to(DEV))
    ref4 = O.attention_ref(q4, k, v, k_lens=k_lens)
    d = (out4.float().cpu() - ref4).abs()
    assert bool(torch.all(d <= 1e-2 * ref4.abs().clamp_min(1.0))), float(d.max())


def test_deterministic_bitwise(lib):
    from lbw_amd import attention_segments
    q, ks, vs = _case(1, 700, 3, [2000, 400], seed=8)
    segs = [(k.to(DEV), v.to(DEV)) for k, v in zip(ks, vs)]
    a = attention_segments(q.to(DEV), segs, num_splits=3)
    b = attention_segments(q.to(DEV), segs, num_splits=3)
    assert torch.equal(a, b)


def test_errors_are_loud(lib):
    from lbw_amd import attention_segments
    q = torch.zeros(1, 4, 1, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="head_dim"):
        attention_segments(q, [(q, q)])


def test_torch_ops_refuse_wrong_types_and_shapes(lib):
    """The torch.ops.lbw operators, called directly (as a traced graph calls them, past the
    Python wrappers' checks), refuse K/V, scales, weights and outputs of the wrong type, device
    or shape with a RuntimeError before any kernel runs."""
    from lbw_amd import _lib
    _lib.ops()
    ops = torch.ops.lbw
    q = torch.zeros(1, 8, 2, 128, dtype=torch.bfloat16, device=DEV)
    k32 = torch.zeros(1, 16, 2, 128, device=DEV)
    with pytest.raises(RuntimeError, match="bf16"):
        ops.attention(q, [k32], [k32], 0, -1, None, 0.0, 0, False)
    kb = k32.to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="uint8"):
        ops.attention_fp8kv(q, [kb], [kb], [torch.ones(1, 2, 1, device=DEV)],
                            [torch.ones(1, 2, 1, device=DEV)], 0, -1, 0.0, 0, False)
    codes = torch.zeros(1, 16, 2, 128, dtype=torch.uint8, device=DEV)
    with pytest.raises(RuntimeError, match="scales"):
        ops.attention_fp8kv(q, [codes], [codes], [torch.ones(1, 2, 3, device=DEV)],
                            [torch.ones(1, 2, 3, device=DEV)], 0, -1, 0.0, 0, False)
    L, C = 8, 256
    x = torch.zeros(L, C, dtype=torch.bfloat16, device=DEV)
    w = torch.ones(C, dtype=torch.bfloat16, device=DEV)
    rope = torch.zeros(1, device=DEV)
    dims = [0, 0, 0, 22, 21]
    with pytest.raises(RuntimeError, match="wq"):
        ops.qk_norm_rope_(x, None, None, None, w.float(), None, rope, dims, 1e-6, 2, x.clone(),
                          None, None, None, 1.0, 1.0, 0)
    with pytest.raises(RuntimeError, match="v_out"):
        ops.qk_norm_rope_(x, None, None, None, w, None, rope, dims, 1e-6, 2, x.clone(), None,
                          x, x[:4], 1.0, 1.0, 0)
    with pytest.raises(RuntimeError, match="q_out"):
        ops.qk_norm_rope_(x, None, None, None, w, None, rope, dims, 1e-6, 2,
                          torch.zeros(2, 128, L, dtype=torch.bfloat16, device=DEV)[:, :, :4],
                          None, None, None, 1.0, 1.0, 1)
    # RoPE tables shorter than the grid's (f, h, w, s0, s1) need
    with pytest.raises(RuntimeError, match="rope holds"):
        ops.qk_norm_rope_(x, None, None, None, w, None, torch.zeros(100, device=DEV),
                          [1, 2, 4, 22, 21], 1e-6, 2, x.clone(), None, None, None, 1.0, 1.0, 0)
    # quantiser scales of the wrong size or device
    xq = torch.zeros(1, 130, 2, 128, dtype=torch.bfloat16, device=DEV)
    c8 = torch.zeros(1, 130, 2, 128, dtype=torch.uint8, device=DEV)
    with pytest.raises(RuntimeError, match="scales must be"):
        ops.kv_quant_fp8_(xq, c8, torch.zeros(1, 2, 2, device=DEV))
    with pytest.raises(RuntimeError, match="device"):
        ops.kv_quant_fp8_(xq, c8, torch.zeros(1, 2, 3))
    # merge partials whose (B, N) differ from O's, or that sit on another device
    po = torch.zeros(1, 2, 8, 128, device=DEV)
    pm = torch.zeros(1, 2, 8, device=DEV)
    ob = torch.zeros(1, 8, 2, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="differ in shape"):
        ops.attention_merge_out([po], [torch.zeros(1, 3, 8, device=DEV)],
                                [torch.zeros(1, 3, 8, device=DEV)], ob)
    with pytest.raises(RuntimeError, match="device"):
        ops.attention_merge_out([po], [pm.cpu()], [pm], ob)
    # device window bounds that are not one-element integer tensors on q's device
    kq = torch.zeros(1, 16, 2, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="kv_hi_dev"):
        ops.attention(q, [kq], [kq], 0, -1, None, 0.0, 0, False, None,
                      torch.tensor([3.0], device=DEV))
    with pytest.raises(RuntimeError, match="kv_lo_dev"):
        ops.attention(q, [kq], [kq], 0, -1, None, 0.0, 0, False,
                      torch.tensor([1, 2], device=DEV), None)
    torch.cuda.synchronize()


def test_two_streams_get_separate_workspaces(lib):
    """Two split-KV calls in flight on two streams at once: each call's workspace (work-queue
    counters and partials) comes from the caching allocator on its own stream, so neither call
    takes the other's items or overwrites its partials. Both outputs are checked against the
    oracle."""
    from lbw_amd import attention_segments
    cases = [_case(1, 700, 3, [3000], seed=s) for s in (31, 32)]
    dev_in = [(q.to(DEV), ks[0].to(DEV), vs[0].to(DEV)) for q, ks, vs in cases]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    cur = torch.cuda.current_stream()
    outs = []
    for st, (q, k, v) in zip(streams, dev_in):
        st.wait_stream(cur)
        with torch.cuda.stream(st):
            outs.append(attention_segments(q, [(k, v)], num_splits=4))
    for st in streams:
        cur.wait_stream(st)
    torch.cuda.synchronize()
    for out, (q, ks, vs) in zip(outs, cases):
        assert_parity(out, O.attention_ref(q, ks[0], vs[0]), "stream")


def _full_size_subset(H, Lq, lk_cache, lk_chunk, heads, rows, seed):
    from lbw_amd import attention_segments
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(1, Lq, H, 128, generator=g, device=DEV).to(torch.bfloat16)
    kc = torch.randn(1, lk_cache, H, 128, generator=g, device=DEV).to(torch.bfloat16)
    vc = torch.randn(1, lk_cache, H, 128, generator=g, device=DEV).to(torch.bfloat16)
    kn = torch.randn(1, lk_chunk, H, 128, generator=g, device=DEV).to(torch.bfloat16)
    vn = torch.randn(1, lk_chunk, H, 128, generator=g, device=DEV).to(torch.bfloat16)
    out = attention_segments(q, [(kc, vc), (kn, vn)])
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out.float()).all())
    sel = torch.randperm(Lq, generator=torch.Generator().manual_seed(seed))[:rows].sort().values
    for h in heads:
        qh = q[:, sel][:, :, h:h + 1].cpu()
        k = torch.cat([kc[:, :, h:h + 1], kn[:, :, h:h + 1]], 1).cpu()
        v = torch.cat([vc[:, :, h:h + 1], vn[:, :, h:h + 1]], 1).cpu()
        ref = O.attention_ref(qh, k, v)
        m = assert_parity(out[:, sel][:, :, h:h + 1], ref, f"head {h}")
        print(f"head {h}: {m}")


def test_full_size_wan13b_480p_chunk(lib):
    """1.3B 480p: 3-frame chunk (4680 q) over 6 cached frames + chunk (14040 keys), 12 heads."""
    _full_size_subset(12, 4680, 9360, 4680, heads=[0, 7, 11], rows=384, seed=1)


def test_full_size_wan14b_720p_chunk(lib):
    """14B 720p: 1-frame chunk (3600 q) over 12 cached frames + chunk (46800 keys), 40 heads."""
    _full_size_subset(40, 3600, 43200, 3600, heads=[0, 19, 39], rows=256, seed=2)


def test_full_size_wan14b_480p_chunk(lib):
    """14B 480p: 3-frame chunk (4680 q) over 18 cached frames + chunk (32760 keys), 40 heads."""
    _full_size_subset(40, 4680, 28080, 4680, heads=[0, 21, 39], rows=256, seed=3)


def test_cross_attention_dedup_matches_full_context():
    """Exact dedup (attention.py:493-554): a 512-row context whose rows 300.. are identical
    (the projected zero padding); the deduplicated call equals unmasked attention over all
    512 rows (oracle) and the plain unmasked kernel call."""
    from lbw_amd import cross_attention, padding_start
    g = torch.Generator().manual_seed(41)
    H, Lq, L, nv = 4, 333, 512, 300
    q = torch.randn(1, Lq, H, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(1, L, H, 128, generator=g)
    # V at half scale: the padding row carries 212/512 of the keys, so outputs follow it
    # closely; this keeps |o| < 2, where one bf16 output rounding stays within the 1e-2 bound
    v = 0.5 * torch.randn(1, L, H, 128, generator=g)
    k[:, nv:] = torch.randn(1, 1, H, 128, generator=g)
    v[:, nv:] = 0.5 * torch.randn(1, 1, H, 128, generator=g)
    k, v = k.to(torch.bfloat16), v.to(torch.bfloat16)
    kd, vd = k.to(DEV), v.to(DEV)
    nd = padding_start(kd, vd)
    assert nd == nv
    out = cross_attention(q.to(DEV), kd, vd, n_distinct=nd)
    ref = O.attention_ref(q, k, v)
    assert_parity(out, ref, "dedup")
    plain = cross_attention(q.to(DEV), kd, vd)
    assert float((out.float() - plain.float()).abs().max()) <= 1e-2
    # no padding at all: n_distinct = L - 1 (the last row counts once)
    k2 = torch.randn(1, 96, H, 128, generator=g).to(torch.bfloat16)
    v2 = torch.randn(1, 96, H, 128, generator=g).to(torch.bfloat16)
    nd2 = padding_start(k2.to(DEV), v2.to(DEV))
    assert nd2 == 95
    out2 = cross_attention(q.to(DEV), k2.to(DEV), v2.to(DEV), n_distinct=nd2)
    assert_parity(out2, O.attention_ref(q, k2, v2), "dedup, no padding")


@pytest.mark.parametrize("splits", [2, 3, 5, 8, 9, 12])
def test_split_pieces_merged_in_kernel(lib, splits):
    """Split calls of up to 8 pieces merge in the attention kernel (the last piece of each
    (batch, head, q-tile) unit to finish reads the others' partials at device scope); more
    pieces run the separate merge kernel. Many units spread over the XCDs: parity with the
    oracle, bf16 output = the fp32 output rounded once, and repeated calls bit for bit equal."""
    from lbw_amd import attention_segments
    q, ks, vs = _case(3, 1000, 16, [1500, 700], seed=splits, gain=False)
    segs = [(k.to(DEV), v.to(DEV)) for k, v in zip(ks, vs)]
    qd = q.to(DEV)
    runs = [attention_segments(qd, segs, num_splits=splits) for _ in range(3)]
    o32 = attention_segments(qd, segs, num_splits=splits, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = O.attention_ref(q, torch.cat(ks, 1), torch.cat(vs, 1))
    print(f"splits={splits}", metrics(runs[0], ref), flush=True)
    assert_parity(runs[0], ref)
    for r in runs[1:]:
        assert torch.equal(r, runs[0])
    assert torch.equal(o32.to(torch.bfloat16), runs[0])


def test_chain_state_is_one_running_triple(lib):
    """The chain state is one (O, m, l) triple merged call by call (the reference's running
    (O, -max, sum)): 20 calls -- more than one merge launch takes partials -- over 20 key
    sets, one of them empty, equal attention over their union; the state after the calls is
    the union's partials: m the row max of all scores, l and O relative to it."""
    from lbw_amd import attention_chain
    lens = [64 * (i % 5) + 17 * i for i in range(20)]
    q, ks, vs = _case(1, 150, 2, lens, seed=77, gain=False)
    qd = q.to(DEV)
    state = None
    for k, v in zip(ks, vs):
        state = attention_chain(qd, [(k.to(DEV), v.to(DEV))] if k.shape[1] else [], state)
        assert state is None or len(state) == 3
    out = attention_chain(qd, [], state, normalize=True)
    torch.cuda.synchronize()
    kk, vv = torch.cat(ks, 1), torch.cat(vs, 1)
    assert_parity(out, O.attention_ref(q, kk, vv), "20-call chain")
    _, (ro, rm, rl) = O.attention_ref(q, kk, vv, return_partials=True)
    po, pm, pl = state
    assert torch.allclose(pm.cpu(), rm, rtol=1e-5, atol=1e-4)
    assert torch.allclose(pl.cpu(), rl, rtol=5e-3, atol=1e-3)
    # O is relative to the row max (sums of up to hundreds of bf16 p): held as the normalised
    # rows and by its relative L1 error
    po, pl = po.cpu(), pl.cpu()
    assert torch.allclose(po / pl[..., None], ro / rl[..., None], atol=1e-2)
    assert float((po - ro).abs().mean() / ro.abs().mean()) <= 4e-3


def test_merge_partials_of_empty_rows(lib):
    """Rows with no keys in any partial (m = -inf, l = 0) merge to m = -inf, l = 0, O = 0, and
    normalise to 0, as SDPA's fully masked rows."""
    from lbw_amd import attention_merge, attention_merge_partials, attention_partial
    q, ks, vs = _case(1, 40, 2, [300], seed=3)
    segs = [(ks[0].to(DEV), vs[0].to(DEV))]
    a = attention_partial(q.to(DEV), segs, kv_lo=100, kv_hi=100)
    b = attention_partial(q.to(DEV), segs, kv_lo=0, kv_hi=0)
    po, pm, pl = attention_merge_partials([a, b])
    torch.cuda.synchronize()
    assert torch.all(torch.isneginf(pm)) and torch.all(pl == 0) and torch.all(po == 0)
    assert torch.all(attention_merge([(po, pm, pl)]) == 0)
