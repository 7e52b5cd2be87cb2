"""GPU checks of the Wan attention layers (the hot path's callers) against the fp32 oracle:
projections -> fused q/k norm + RoPE with the KV commit -> attention -> o-projection.

Tolerance: the layer rounds to bf16 after each stage (projections, norm, RoPE, attention,
o-projection), so it is held to relative-L1 <= 1e-2 and cosine >= 0.9999 against the fp32
oracle run on the same bf16 inputs and weights."""
import pytest
import torch

import oracle as O
from parity import cosine, metrics

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _w(g, *shape, std=0.02):
    return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)


def _weights(C, g, bias_std=0.0, gamma_std=0.0):
    ws = {}
    for n in ("q", "k", "v", "o"):
        ws["w" + n] = _w(g, C, C)
        ws["b" + n] = (torch.randn(C, generator=g) * bias_std).to(torch.bfloat16)
    ws["gq"] = (1 + torch.randn(C, generator=g) * gamma_std).to(torch.bfloat16)
    ws["gk"] = (1 + torch.randn(C, generator=g) * gamma_std).to(torch.bfloat16)
    return ws


def _layer(cls, ws, heads):
    d = {k: v.to(DEV) for k, v in ws.items()}
    return cls(d["wq"], d["bq"], d["wk"], d["bk"], d["wv"], d["bv"], d["wo"], d["bo"],
               d["gq"], d["gk"], heads=heads)


def _check(out, ref, what):
    m = metrics(out, ref)
    c = cosine(out, ref)
    print(what, f"cosine {c:.6f}", m)
    assert m["nonfinite"] == 0 and m["rel_l1"] <= 1e-2 and c >= 0.9999, (what, c, m)


@pytest.mark.parametrize("bias_std,gamma_std", [(0.0, 0.0), (0.05, 0.1)])
def test_wan13b_layer_over_flat_cache(lib, bias_std, gamma_std):
    """1.3B, 480p: one latent frame (30 x 52 = 1560 tokens) at start frame 2 over 2 cached
    frames (3120 tokens) plus itself; weights N(0, 0.02), bias 0 and gamma 1 as specified, and
    a second case with random bias and gamma."""
    from lbw_amd import FlatKVCache, WanSelfAttention
    g = torch.Generator().manual_seed(1)
    C, H = 1536, 12
    x_cache = torch.randn(1, 3120, C, generator=g).to(torch.bfloat16)
    x = torch.randn(1, 1560, C, generator=g).to(torch.bfloat16)
    ws = _weights(C, g, bias_std, gamma_std)
    layer = _layer(WanSelfAttention, ws, H)
    cache = FlatKVCache(1, 4680, H, 128, device=DEV)
    layer.prefill(x_cache.to(DEV), (2, 30, 52), 0, cache, current_start=0)
    out = layer.forward(x.to(DEV), (1, 30, 52), 2, cache, current_start=3120)
    f = {k: v.float() for k, v in ws.items()}
    ref = O.self_attention_layer_ref(x.float(), x_cache.float(), f["wq"], f["bq"], f["wk"], f["bk"],
                                     f["wv"], f["bv"], f["wo"], f["bo"], f["gq"], f["gk"], heads=H,
                                     grid=(1, 30, 52), cache_grid=(2, 30, 52), start_frame=2,
                                     cache_start_frame=0)
    _check(out, ref, "layer")


@pytest.mark.parametrize("max_att_frames", [5, 4])
def test_windowed_flat_cache_evicts_with_sink(lib, max_att_frames):
    """The windowed flat cache past capacity (model_fast.py:2510-2526): 5-frame cache with a
    1-frame sink, 9 one-frame chunks of 8 x 8 tokens, so the last 4 chunks each roll the
    cache (everything after the sink moves left by a frame) before their K/V are committed.
    With a 5-frame attention window the sink is attended; with 4 frames it falls outside.
    Every chunk's layer output is checked against the oracle's windowed sequence."""
    from lbw_amd import FlatKVCache, WanSelfAttention
    g = torch.Generator().manual_seed(8)
    C, H, F = 512, 4, 64
    ws = _weights(C, g, 0.02, 0.05)
    layer = _layer(WanSelfAttention, ws, H)
    xs = [torch.randn(1, F, C, generator=g).to(torch.bfloat16) for _ in range(9)]
    cache = FlatKVCache(1, 5 * F, H, 128, device=DEV, sink_tokens=F,
                        max_attention_size=max_att_frames * F)
    f = {k: v.float() for k, v in ws.items()}
    refs = O.windowed_layer_sequence_ref([x.float() for x in xs], f["wq"], f["bq"], f["wk"],
                                         f["bk"], f["wv"], f["bv"], f["wo"], f["bo"], f["gq"],
                                         f["gk"], heads=H, frame_hw=(8, 8), kv_cache_size=5 * F,
                                         sink_tokens=F, max_attention_size=max_att_frames * F)
    rolls = 0
    for i, x in enumerate(xs):
        rolls += cache.plan(i * F, F).roll is not None
        out = layer.forward(x.to(DEV), (1, 8, 8), i, cache, current_start=i * F)
        _check(out, refs[i], f"chunk {i} (rolls so far {rolls})")
    assert rolls == 4


def test_chunked_cache_path_equals_flat(lib):
    """The chunked cache (3 slots of one 8 x 8 frame each) gives the flat cache's result: the
    64-token chunks make both layouts walk the same key tiles in the same order; and each
    chunk's output against the oracle's layer over the frames the chunks hold."""
    from lbw_amd import FlatKVCache, WanSelfAttention, allocate_self_kv_chunks
    g = torch.Generator().manual_seed(2)
    C, H, F = 512, 4, 8 * 8
    ws = _weights(C, g, 0.02, 0.05)
    layer = _layer(WanSelfAttention, ws, H)
    frames = [torch.randn(1, F, C, generator=g).to(torch.bfloat16).to(DEV) for _ in range(3)]
    flat = FlatKVCache(1, 3 * F, H, 128, device=DEV)
    chunks = allocate_self_kv_chunks(1, 1, F, H, 128, 3, device=DEV)[0]
    f = {k: v.float() for k, v in ws.items()}
    for i, fr in enumerate(frames):
        a = layer.forward(fr, (1, 8, 8), i, flat, current_start=i * F)
        b = layer.forward_chunked(fr, (1, 8, 8), i, chunks, chunk_index=i)
        m = metrics(b, a)
        print(i, "identical" if torch.equal(a, b) else "differs", m)
        assert m["nonfinite"] == 0 and m["max_abs"] <= 1e-3, (i, m)
        if i == 0:
            continue
        # the chunks before this one are the cache: frames 0 .. i-1 at start frame 0
        xc = torch.cat([x.cpu() for x in frames[:i]], 1).float()
        ref = O.self_attention_layer_ref(fr.cpu().float(), xc, f["wq"], f["bq"], f["wk"],
                                         f["bk"], f["wv"], f["bv"], f["wo"], f["bo"], f["gq"],
                                         f["gk"], heads=H, grid=(1, 8, 8), cache_grid=(i, 8, 8),
                                         start_frame=i, cache_start_frame=0)
        _check(b, ref, f"chunked cache, chunk {i}")


def test_chunked_fp8_cache_path(lib):
    """The fp8 chunked cache: the routed slot holds exactly quantize_kv_fp8 of the chunk's
    roped K/V (the bf16 chunked cache's slot), and the layer output stays within the fp8
    tolerance (cosine >= 0.999) of the bf16 chunked path, over 4 chunks so that slot 1 is
    rewritten and the sink stays."""
    from lbw_amd import (WanSelfAttention, allocate_self_kv_chunks, allocate_self_kv_chunks_fp8,
                         quantize_kv_fp8)
    g = torch.Generator().manual_seed(4)
    C, H, F = 512, 4, 8 * 8
    ws = _weights(C, g, 0.02, 0.05)
    layer = _layer(WanSelfAttention, ws, H)
    frames = [torch.randn(1, F, C, generator=g).to(torch.bfloat16).to(DEV) for _ in range(4)]
    bf = allocate_self_kv_chunks(1, 1, F, H, 128, 3, device=DEV)[0]
    f8 = allocate_self_kv_chunks_fp8(1, 1, F, H, 128, 3, device=DEV)[0]
    from lbw_amd import chunk_routing
    for i, fr in enumerate(frames):
        a = layer.forward_chunked(fr, (1, 8, 8), i, bf, chunk_index=i)
        b = layer.forward_chunked_fp8(fr, (1, 8, 8), i, f8, chunk_index=i)
        dest, _ = chunk_routing(i, 3)
        for key in ("k", "v"):
            ref = quantize_kv_fp8(bf[key][dest])
            assert torch.equal(f8[key][dest].codes, ref.codes), (i, key)
            assert torch.equal(f8[key][dest].scales, ref.scales), (i, key)
        cs = cosine(b, a)
        print(i, dest, f"cos {cs:.6f}")
        assert torch.isfinite(b).all() and cs >= 0.999, (i, cs)


def test_wan14b_cross_attention_layer(lib):
    """14B cross-attention: 4680 chunk queries against a 512-token context of dim 4096
    (N(0,1), rows 300..511 zeroed) projected to 5120 by N(0, 0.02) weights; masked to the
    300 valid rows. Oracle on a subset of query rows."""
    from lbw_amd import WanCrossAttention
    g = torch.Generator().manual_seed(3)
    C, H, Lq = 5120, 40, 4680
    ctx_raw = torch.randn(1, 512, 4096, generator=g)
    ctx_raw[:, 300:] = 0
    w_text = _w(g, C, 4096)
    ctx = (ctx_raw.to(torch.bfloat16).float() @ w_text.float().T).to(torch.bfloat16)
    x = torch.randn(1, Lq, C, generator=g).to(torch.bfloat16)
    ws = _weights(C, g, 0.02, 0.05)
    layer = _layer(WanCrossAttention, ws, H)
    k_lens = torch.tensor([300], dtype=torch.int32, device=DEV)
    out = layer.forward(x.to(DEV), ctx.to(DEV), k_lens=k_lens)
    rows = torch.randperm(Lq, generator=g)[:256].sort().values
    f = {k: v.float() for k, v in ws.items()}
    q = O.rms_norm_module(x[:, rows].float() @ f["wq"].T + f["bq"], f["gq"])
    kk, vv = O.cross_kv_ref(ctx.float(), f["wk"], f["bk"], f["wv"], f["bv"], f["gk"], H)
    o = O.attention_ref(q.view(1, -1, H, 128), kk, vv, k_lens=[300])
    ref = o.reshape(1, -1, C) @ f["wo"].T + f["bo"]
    _check(out[:, rows], ref, "cross")


def test_wan14b_cross_attention_layer_dedup(lib):
    """The same 14B cross-attention with the reference's unmasked semantics (all 512 context
    rows attended) computed by the exact dedup: the 212 zero-padding rows project to identical
    K/V rows and are attended as one key of multiplicity 212."""
    from lbw_amd import WanCrossAttention
    g = torch.Generator().manual_seed(4)
    C, H, Lq = 5120, 40, 1560
    ctx_raw = torch.randn(1, 512, 4096, generator=g)
    ctx_raw[:, 300:] = 0
    w_text = _w(g, C, 4096)
    ctx = (ctx_raw.to(torch.bfloat16).float() @ w_text.float().T).to(torch.bfloat16)
    x = torch.randn(1, Lq, C, generator=g).to(torch.bfloat16)
    ws = _weights(C, g, 0.02, 0.05)
    d = {k: v.to(DEV) for k, v in ws.items()}
    layer = WanCrossAttention(d["wq"], d["bq"], d["wk"], d["bk"], d["wv"], d["bv"], d["wo"],
                              d["bo"], d["gq"], d["gk"], heads=H, dedup=True)
    out = layer.forward(x.to(DEV), ctx.to(DEV))
    assert layer.n_distinct == 300
    rows = torch.randperm(Lq, generator=g)[:192].sort().values
    f = {k: v.float() for k, v in ws.items()}
    q = O.rms_norm_module(x[:, rows].float() @ f["wq"].T + f["bq"], f["gq"])
    kk, vv = O.cross_kv_ref(ctx.float(), f["wk"], f["bk"], f["wv"], f["bv"], f["gk"], H)
    o = O.attention_ref(q.view(1, -1, H, 128), kk, vv)
    ref = o.reshape(1, -1, C) @ f["wo"].T + f["bo"]
    _check(out[:, rows], ref, "cross dedup")
