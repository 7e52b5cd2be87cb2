"""GPU parity of the fused q/k RMSNorm + Wan 3-D RoPE kernel (lbw_qk_norm_rope) against the
oracle's restatement of kernels/qk_post.py:88-141 and the grid of model_fast.py:878-931.

Tolerance: the kernel follows the oracle's rounding sequence op for op except the order of
the fp32 sum of squares (and so possibly the last bit of the rsqrt), so where the normalised
value sits on a bf16 rounding boundary one intermediate flips by one bf16 step; through the
rotation and the final rounding that is at most two bf16 steps of the rotated pair's
magnitude: |diff| <= 2^-5 * |pair| everywhere, and >= 99.9% of elements bit-identical."""
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _check(out, ref, what):
    o = out.float().cpu()
    r = ref.float().cpu()
    d = (o - r).abs()
    pair = r.view(*r.shape[:-1], -1, 2).norm(dim=-1, keepdim=True).expand(
        *r.shape[:-1], r.shape[-1] // 2, 2).reshape(r.shape)
    assert bool(torch.all(d <= pair * 2.0 ** -5 + 1e-6)), (what, float(d.max()))
    same = float((o == r).float().mean())
    assert same >= 0.999, (what, same)
    return same


@pytest.mark.parametrize("name,L,C,grid,start,bias,extra", [
    ("wan13b_480p_3f", 4680, 1536, (3, 30, 52), 6, False, 0),
    ("wan14b_720p_1f", 3600, 5120, (1, 45, 80), 12, True, 0),
    ("ragged_tail", 200, 512, (2, 7, 13), 2879 - 2, True, 18),
])
def test_qk_norm_rope_matches_oracle(lib, name, L, C, grid, start, bias, extra):
    from lbw_amd import causal_rope_tables, qk_norm_rope, wan_rope_freqs
    g = torch.Generator().manual_seed(L)
    f, h, w = grid
    assert L == f * h * w + extra
    q = (torch.randn(L, C, generator=g) * 1.5).to(torch.bfloat16)
    k = (torch.randn(L, C, generator=g) * 1.5).to(torch.bfloat16)
    bq = (torch.randn(C, generator=g) * 0.2).to(torch.bfloat16) if bias else None
    bk = (torch.randn(C, generator=g) * 0.2).to(torch.bfloat16) if bias else None
    wq = (1 + torch.randn(C, generator=g) * 0.1).to(torch.bfloat16)
    wk = (1 + torch.randn(C, generator=g) * 0.1).to(torch.bfloat16)
    freqs = wan_rope_freqs(128)
    tabs = causal_rope_tables(freqs, grid, start, device=DEV)
    qo, ko = qk_norm_rope(q.to(DEV), k.to(DEV), None if bq is None else bq.to(DEV),
                          None if bk is None else bk.to(DEV), wq.to(DEV), wk.to(DEV), tabs,
                          eps=1e-6)
    cos, sin = O.causal_rope_grids(O.wan_rope_freqs(128), f, h, w, start_frame=start)
    rq = O.qk_post_norm_rope(q, bq, wq, cos, sin, eps=1e-6)
    rk = O.qk_post_norm_rope(k, bk, wk, cos, sin, eps=1e-6)
    sq = _check(qo, rq, name + ":q")
    sk = _check(ko, rk, name + ":k")
    print(name, "bit-identical fraction q", sq, "k", sk)


def test_qk_norm_rope_writes_cache_slot_and_v(lib):
    """k_out/v_out as a slot of a [1, S, H, D] cache (the fused KV commit)."""
    from lbw_amd import causal_rope_tables, qk_norm_rope_, wan_rope_freqs
    g = torch.Generator().manual_seed(3)
    H, D = 4, 128
    C = H * D
    grid = (1, 6, 10)
    L = 60
    q = torch.randn(L, C, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(L, C, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(L, C, generator=g).to(torch.bfloat16).to(DEV)
    w = torch.ones(C, dtype=torch.bfloat16, device=DEV)
    cache_k = torch.zeros(1, 5 * L, H, D, dtype=torch.bfloat16, device=DEV)
    cache_v = torch.zeros_like(cache_k)
    qo = torch.empty_like(q)
    tabs = causal_rope_tables(wan_rope_freqs(128), grid, 4, device=DEV)
    qk_norm_rope_(q, k, None, None, w, w, tabs, 1e-6, H, q_out=qo,
                  k_out=cache_k[0, 2 * L:3 * L].view(L, C), v=v,
                  v_out=cache_v[0, 2 * L:3 * L].view(L, C))
    cos, sin = O.causal_rope_grids(O.wan_rope_freqs(128), *grid, start_frame=4)
    rk = O.qk_post_norm_rope(k.cpu(), None, w.cpu(), cos, sin)
    _check(cache_k[0, 2 * L:3 * L].reshape(L, C), rk, "cache slot")
    assert torch.equal(cache_v[0, 2 * L:3 * L].reshape(L, C), v)
    assert torch.all(cache_k[0, :2 * L] == 0) and torch.all(cache_k[0, 3 * L:] == 0)


def _inputs(L, C, seed, bias=True):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(L, C, generator=g) * 1.5).to(torch.bfloat16)
    k = (torch.randn(L, C, generator=g) * 1.5).to(torch.bfloat16)
    bq = (torch.randn(C, generator=g) * 0.2).to(torch.bfloat16) if bias else None
    bk = (torch.randn(C, generator=g) * 0.2).to(torch.bfloat16) if bias else None
    wq = (1 + torch.randn(C, generator=g) * 0.1).to(torch.bfloat16)
    wk = (1 + torch.randn(C, generator=g) * 0.1).to(torch.bfloat16)
    return q, k, bq, bk, wq, wk


def _dev(*ts):
    return [None if t is None else t.to(DEV) for t in ts]


def _rows_of(t):
    """[H, D, L] -> [L, H * D]"""
    H, D, L = t.shape
    return t.permute(2, 0, 1).reshape(L, H * D)


@pytest.mark.parametrize("name,L,C,grid,start", [
    ("qk_post_t_test_shape", 2176, 1280, (1, 40, 54), 3),   # perf/qk_post_t_test.py:11-16
    ("wan14b_720p_1f", 3600, 5120, (1, 45, 80), 12),
    ("ragged_tail", 200, 512, (2, 7, 13), 9),
])
def test_qk_norm_rope_t_matches_oracle(lib, name, L, C, grid, start):
    """kernels/qk_post.py:216-306: [H, D, L] outputs, q scaled by 1/sqrt(D) through cos/sin."""
    from lbw_amd import causal_rope_tables, qk_norm_rope_t, wan_rope_freqs
    q, k, bq, bk, wq, wk = _inputs(L, C, seed=L + 1)
    tabs = causal_rope_tables(wan_rope_freqs(128), grid, start, device=DEV)
    qt, kt = qk_norm_rope_t(*_dev(q, k, bq, bk, wq, wk), tabs, eps=1e-6)
    assert qt.shape == (C // 128, 128, L) and kt.shape == (C // 128, 128, L)
    cos, sin = O.causal_rope_grids(O.wan_rope_freqs(128), *grid, start_frame=start)
    rq = O.qk_post_norm_rope_t(q, bq, wq, cos, sin, out_scale=1.0 / 128 ** 0.5)
    rk = O.qk_post_norm_rope_t(k, bk, wk, cos, sin)
    sq = _check(_rows_of(qt), _rows_of(rq), name + ":q_t")
    sk = _check(_rows_of(kt), _rows_of(rk), name + ":k_t")
    print(name, "bit-identical fraction q_t", sq, "k_t", sk)


@pytest.mark.parametrize("offset", [16, 3])
def test_qk_norm_rope_t_into_cache_slot(lib, offset):
    """d-major outputs as a slot of a [H, D, capacity] cache (16-byte stores when the slot
    start is a multiple of 8 tokens, element stores otherwise); the rest stays untouched."""
    from lbw_amd import causal_rope_tables, qk_norm_rope_, wan_rope_freqs
    H, D, L, cap = 4, 128, 75, 200
    C = H * D
    grid = (1, 5, 15)
    q, k, bq, bk, wq, wk = _inputs(L, C, seed=offset)
    tabs = causal_rope_tables(wan_rope_freqs(128), grid, 1, device=DEV)
    cq = torch.zeros(H, D, cap, dtype=torch.bfloat16, device=DEV)
    ck = torch.zeros_like(cq)
    v = torch.randn(L, C).to(torch.bfloat16).to(DEV)
    v_out = torch.zeros(cap, C, dtype=torch.bfloat16, device=DEV)
    qk_norm_rope_(*_dev(q, k, bq, bk, wq, wk), tabs, 1e-6, H, q_out=cq[:, :, offset:offset + L],
                  k_out=ck[:, :, offset:offset + L], q_scale=0.5, layout="dmajor", v=v,
                  v_out=v_out[offset:offset + L])
    cos, sin = O.causal_rope_grids(O.wan_rope_freqs(128), *grid, start_frame=1)
    rq = O.qk_post_norm_rope_t(q, bq, wq, cos, sin, out_scale=0.5)
    rk = O.qk_post_norm_rope_t(k, bk, wk, cos, sin)
    _check(_rows_of(cq[:, :, offset:offset + L]), _rows_of(rq), "slot q")
    _check(_rows_of(ck[:, :, offset:offset + L]), _rows_of(rk), "slot k")
    for c in (cq, ck):
        assert torch.all(c[:, :, :offset] == 0) and torch.all(c[:, :, offset + L:] == 0)
    assert torch.equal(v_out[offset:offset + L], v)
    assert torch.all(v_out[:offset] == 0) and torch.all(v_out[offset + L:] == 0)


def test_single_tensor_and_fused_projection_forms(lib):
    """x_norm_rope (rows), x_norm_rope_t3 / qk_norm_rope3 / qk_norm_rope_t3 on the fused
    projection [L, 3C] (kernels/qk_post.py:81-86, 166-215, 221-225, 331-402), and the rows
    layout with an output scale."""
    from lbw_amd import (causal_rope_tables, qk_norm_rope, qk_norm_rope3, qk_norm_rope_t3,
                         wan_rope_freqs, x_norm_rope, x_norm_rope_t3)
    L, C, grid, start = 1560, 1536, (1, 30, 52), 4
    q, k, bq, bk, wq, wk = _inputs(L, C, seed=7)
    v = torch.randn(L, C).to(torch.bfloat16)
    qkv = torch.cat([q, k, v], dim=1).to(DEV)
    tabs = causal_rope_tables(wan_rope_freqs(128), grid, start, device=DEV)
    cos, sin = O.causal_rope_grids(O.wan_rope_freqs(128), *grid, start_frame=start)
    s = 1.0 / 128 ** 0.5
    rq = O.qk_post_norm_rope(q, bq, wq, cos, sin)
    rk = O.qk_post_norm_rope(k, bk, wk, cos, sin)
    rqs = O.qk_post_norm_rope(q, bq, wq, cos, sin, out_scale=s)
    bq_, bk_, wq_, wk_ = _dev(bq, bk, wq, wk)
    _check(x_norm_rope(qkv[:, :C], bq_, wq_, tabs), rq, "x_norm_rope q")
    _check(x_norm_rope(qkv[:, C:2 * C], bk_, wk_, tabs, scale=s),
           O.qk_post_norm_rope(k, bk, wk, cos, sin, out_scale=s), "x_norm_rope k scaled")
    _check(_rows_of(x_norm_rope_t3(qkv, 0, bq_, wq_, tabs, scale=s)), rqs, "x_norm_rope_t3 q")
    _check(_rows_of(x_norm_rope_t3(qkv, C, bk_, wk_, tabs)), rk, "x_norm_rope_t3 k")
    q3, k3 = qk_norm_rope3(qkv, bq_, bk_, wq_, wk_, tabs)
    _check(q3, rq, "qk_norm_rope3 q")
    _check(k3, rk, "qk_norm_rope3 k")
    qt3, kt3 = qk_norm_rope_t3(qkv, bq_, bk_, wq_, wk_, tabs)
    _check(_rows_of(qt3), rqs, "qk_norm_rope_t3 q")
    _check(_rows_of(kt3), rk, "qk_norm_rope_t3 k")
    qs_, _ = qk_norm_rope(qkv[:, :C], qkv[:, C:2 * C], bq_, bk_, wq_, wk_, tabs, q_scale=s)
    _check(qs_, rqs, "rows layout, scaled q")
