"""lbw_attention_fwd_noalloc, the entry point for callers that cannot allocate: its work-queue
counters and split partials live in the library's static device scratch array. Checked through
the C ABI against lbw_attention_fwd (the allocating entry point, the same kernels) on two calls
in a row -- the second smaller, so that it runs over the first call's leftovers in the scratch
-- and against the oracle, to the bf16 bar of every parity test here."""
import ctypes

import pytest
import torch

import oracle as O
from parity import assert_parity

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(B, Lq, H, L, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Lq, H, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(B, L, H, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(B, L, H, 128, generator=g).to(torch.bfloat16)
    return q, k, v


def _noalloc(lib, q, k, v, splits):
    from lbw_amd import _lib
    out = torch.empty(q.shape, dtype=torch.bfloat16, device=DEV)
    p = _lib.attn_params(q, out, [(k, v)], None, None, None, None, splits)
    rc = lib.lbw_attention_fwd_noalloc(ctypes.byref(p), _lib.stream_ptr())
    _lib.check(rc, "lbw_attention_fwd_noalloc")
    return out


def test_noalloc_matches_allocating_entry_point(lib):
    from lbw_amd import attention_segments
    # (B, Lq, H, keys, splits): a split call whose partials fill 33 MB of the scratch, then a
    # smaller one with the host's own split choice
    for B, Lq, H, L, splits in [(1, 2000, 8, 6000, 4), (2, 700, 3, 3000, 0)]:
        q, k, v = _inputs(B, Lq, H, L, seed=Lq)
        qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
        print(f"case B={B} Lq={Lq} H={H} keys={L} splits={splits}", flush=True)
        out = _noalloc(lib, qd, kd, vd, splits)
        want = attention_segments(qd, [(kd, vd)], num_splits=splits)
        torch.cuda.synchronize()
        # same kernels, same plan: identical results
        assert torch.equal(out, want)
        assert_parity(out, O.attention_ref(q, k, v), "noalloc")


def test_noalloc_rejects_splits_beyond_its_scratch(lib):
    """An explicit split count whose partials exceed the scratch fails with a clear error (no
    launch); the host's own choice (num_splits = 0) is lowered to what fits instead."""
    from lbw_amd import _lib
    q = torch.empty(1, 3600, 40, 128, dtype=torch.bfloat16, device=DEV)
    k = torch.empty(1, 46800, 40, 128, dtype=torch.bfloat16, device=DEV)
    p = _lib.attn_params(q, q, [(k, k)], None, None, None, None, 3)
    rc = lib.lbw_attention_fwd_noalloc(ctypes.byref(p), _lib.stream_ptr())
    assert rc == 4 and b"scratch" in lib.lbw_last_error()
