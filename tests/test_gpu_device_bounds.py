"""The flat cache's window handed over as device tensors, as the reference passes it
(model_fast.py:2538-2550: ``attn_lo`` / ``attn_hi`` are one-element int64 tensors on the device):
the kernel reads the bounds on the GPU, so ``attention(..., kv_lo=attn_lo, kv_hi=attn_hi)`` needs
no host synchronisation and traces under ``torch.compile(fullgraph=True)``. Results are checked
against the oracle and, bit for bit, against the same call with host bounds."""
import warnings

import pytest
import torch

import oracle as O
from parity import assert_parity, metrics

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _case(B, Lq, H, Lk, seed):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16)
    return r(B, Lq, H, 128), r(B, Lk, H, 128), r(B, Lk, H, 128)


def _dev(x, dtype=torch.int64):
    return torch.tensor([x], dtype=dtype, device=DEV)


@pytest.mark.parametrize("lo,hi", [(0, 3000), (700, 2900), (1234, 1235), (100, 100),
                                   (2000, 1000), (-50, 5000), (64, 192)])
def test_device_bounds_match_oracle(lib, lo, hi):
    """attention() with the window as device tensors equals the oracle over the clamped window
    (empty windows give 0, as SDPA's fully masked rows), and with the same split count the
    host-bound call bit for bit (the host plans splits for the whole cache when it does not
    know the window, so the drop-in's own split count may differ)."""
    from lbw_amd import attention, attention_segments
    q, k, v = _case(1, 300, 3, 3000, seed=lo % 97 + hi % 89)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    out = attention(qd, kd, vd, kv_lo=_dev(lo), kv_hi=_dev(hi))
    dev3 = attention_segments(qd, [(kd, vd)], kv_lo=_dev(lo), kv_hi=_dev(hi), num_splits=3)
    host = attention_segments(qd, [(kd, vd)], kv_lo=max(lo, 0), kv_hi=min(max(hi, 0), 3000),
                              num_splits=3)
    torch.cuda.synchronize()
    clo, chi = max(lo, 0), min(hi, 3000)
    ref = O.attention_ref(q, k, v, kv_lo=clo, kv_hi=max(chi, clo))
    print(f"window [{lo}, {hi}) ->", metrics(out, ref), flush=True)
    assert_parity(out, ref)
    assert torch.equal(dev3, host)


def test_device_and_host_bounds_intersect(lib):
    """Host and device bounds given together: the window is their intersection; int32 device
    bounds are converted on the device."""
    from lbw_amd import attention_segments
    q, k, v = _case(2, 260, 2, 2000, seed=11)
    ks = [(k[:, :900].to(DEV), v[:, :900].to(DEV)), (k[:, 900:].to(DEV), v[:, 900:].to(DEV))]
    out = attention_segments(q.to(DEV), ks, kv_lo=_dev(300, torch.int32), kv_hi=_dev(1800))
    both = attention_segments(q.to(DEV), ks, kv_lo=500, kv_hi=_dev(1800, torch.int32))
    both2 = attention_segments(q.to(DEV), ks, kv_lo=_dev(300), kv_hi=1500)
    torch.cuda.synchronize()
    assert_parity(out, O.attention_ref(q, k, v, kv_lo=300, kv_hi=1800))
    assert_parity(both, O.attention_ref(q, k, v, kv_lo=500, kv_hi=1800))
    assert_parity(both2, O.attention_ref(q, k, v, kv_lo=300, kv_hi=1500))


def test_device_bounds_fp8_and_partials(lib):
    """The fp8-KV kernel and the partials mode read device bounds too: bit for bit equal to the
    same calls (same split count) with host bounds."""
    from lbw_amd import attention_fp8kv, attention_partial, quantize_kv_fp8
    q, k, v = _case(1, 200, 2, 2500, seed=3)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    k8, v8 = quantize_kv_fp8(kd), quantize_kv_fp8(vd)
    a = attention_fp8kv(qd, [(k8, v8)], kv_lo=_dev(130), kv_hi=_dev(2222), num_splits=2)
    b = attention_fp8kv(qd, [(k8, v8)], kv_lo=130, kv_hi=2222, num_splits=2)
    pa = attention_partial(qd, [(kd, vd)], kv_lo=_dev(77), kv_hi=_dev(1999))
    pb = attention_partial(qd, [(kd, vd)], kv_lo=77, kv_hi=1999)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    for x, y in zip(pa, pb):
        assert torch.equal(x, y)


def test_device_bounds_need_no_host_sync(lib):
    """With torch's sync debug mode set to error, the drop-in call with device bounds runs (a
    host read of a bound, as .item(), raises in that mode: checked first)."""
    from lbw_amd import attention
    q, k, v = _case(1, 128, 2, 1000, seed=5)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    lo, hi = _dev(100), _dev(900)
    attention(qd, kd, vd, kv_lo=lo, kv_hi=hi)      # warm: library load and workspace pool
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        with pytest.raises(RuntimeError):
            int(hi.item())
        out = attention(qd, kd, vd, kv_lo=lo, kv_hi=hi)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
    assert_parity(out, O.attention_ref(q, k, v, kv_lo=100, kv_hi=900))


def test_compile_fullgraph_with_device_bounds(lib):
    """torch.compile(fullgraph=True) of the drop-in attention() with the window as device
    tensors (the reference's call, model_fast.py:2546-2550) gives one graph and the eager
    result."""
    from lbw_amd import attention
    q, k, v = _case(1, 300, 2, 1600, seed=9)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)

    def f(q, k, v, lo, hi):
        return attention(q, k, v, kv_lo=lo, kv_hi=hi).float() * 2.0

    torch._dynamo.reset()
    cf = torch.compile(f, backend="aot_eager", fullgraph=True)
    lo, hi = _dev(200), _dev(1500)
    got = cf(qd, kd, vd, lo, hi)
    want = f(qd, kd, vd, lo, hi)
    lo.fill_(0)                  # new window values, same graph
    hi.fill_(700)
    got2 = cf(qd, kd, vd, lo, hi)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert_parity(got2 / 2.0, O.attention_ref(q, k, v, kv_lo=0, kv_hi=700))


def test_q_scale_is_ignored_like_the_reference(lib):
    """The reference's attention() never applies q_scale (attention.py:1082-1143): the drop-in
    returns the same result, with a warning."""
    from lbw_amd import attention
    q, k, v = _case(1, 64, 2, 300, seed=2)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        a = attention(qd, kd, vd, q_scale=3.0)
    assert any("q_scale" in str(x.message) for x in w)
    b = attention(qd, kd, vd)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_softmax_scale_is_ignored_like_the_reference(lib):
    """The reference's attention() scales by 1/sqrt(head_dim) whatever softmax_scale says (its
    kernels and its SDPA fallback, attention.py:378, 439, 1127-1143): the drop-in returns the
    same result, with a warning, and equals the oracle at the default scale."""
    from lbw_amd import attention
    q, k, v = _case(1, 64, 2, 300, seed=4)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        a = attention(qd, kd, vd, softmax_scale=0.25)
    assert any("softmax_scale" in str(x.message) for x in w)
    b = attention(qd, kd, vd)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert_parity(a, O.attention_ref(q, k, v))


def test_cross_attention_refuses_device_bounds(lib):
    from lbw_amd import attention_segments
    q, k, v = _case(1, 64, 2, 300, seed=2)
    with pytest.raises(ValueError, match="device window"):
        attention_segments(q.to(DEV), [(k.to(DEV), v.to(DEV))], kv_hi=_dev(100), cross=True)
