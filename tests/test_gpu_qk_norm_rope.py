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
