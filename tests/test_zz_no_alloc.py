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


def test_noalloc_lowers_the_host_split_choice_to_what_fits(lib):
    """12 heads x 3600 queries over 46800 keys: the host's own choice is 4 pieces (90 MB of
    partials); without an explicit count the entry point lowers it to the most that fit its
    64 MiB scratch (2 pieces), bit for bit the allocating entry point's 2-piece call."""
    from lbw_amd import _lib, attention_segments
    g = torch.Generator(device=DEV).manual_seed(12)
    q = torch.randn(1, 3600, 12, 128, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(1, 46800, 12, 128, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(1, 46800, 12, 128, generator=g, device=DEV).to(torch.bfloat16)
    p = _lib.attn_params(q, q, [(k, v)])
    per = 3600 * 12 * 130 * 4
    assert lib.lbw_attention_workspace_size(ctypes.byref(p)) // per == 4
    out = _noalloc(lib, q, k, v, 0)
    want = attention_segments(q, [(k, v)], num_splits=2)
    other = attention_segments(q, [(k, v)], num_splits=4)
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    assert not torch.equal(out, other)


def test_noalloc_replays_in_a_hip_graph(lib):
    """The entry point captured in a HIP graph (its queue counters are cleared by a kernel, not
    a memset) and replayed with new inputs, every replay bitwise equal to an eager call of the
    allocating entry point, with eager work between the replays."""
    from lbw_amd import _lib, attention_segments
    g = torch.Generator(device=DEV).manual_seed(3)
    rnd = lambda *s: torch.randn(*s, generator=g, device=DEV).to(torch.bfloat16)
    q, k, v = rnd(1, 700, 6, 128), rnd(1, 4000, 6, 128), rnd(1, 4000, 6, 128)
    out = torch.empty_like(q)
    p = _lib.attn_params(q, out, [(k, v)], None, None, None, None, 3)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _lib.check(lib.lbw_attention_fwd_noalloc(ctypes.byref(p), _lib.stream_ptr()), "warm")
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _lib.check(lib.lbw_attention_fwd_noalloc(ctypes.byref(p), _lib.stream_ptr()), "capture")
    torch.cuda.synchronize()
    for rep in range(3):
        print(f"replay {rep}", flush=True)
        for t in (q, k, v):
            t.copy_(rnd(*t.shape))
        graph.replay()
        want = attention_segments(q, [(k, v)], num_splits=3)
        torch.cuda.synchronize()
        assert torch.equal(out, want), rep


_FIRST_CALL_UNDER_CAPTURE = r"""
import ctypes, sys, torch
sys.path[:0] = sys.argv[1:3]
from lbw_amd import _lib, attention_segments
lib = _lib.load()
g = torch.Generator(device="cuda").manual_seed(9)
q, k, v = (torch.randn(*s, generator=g, device="cuda").to(torch.bfloat16)
           for s in ((1, 300, 2, 128), (1, 2000, 2, 128), (1, 2000, 2, 128)))
out = torch.empty_like(q)
p = _lib.attn_params(q, out, [(k, v)], None, None, None, None, 2)
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):     # the device's first no-alloc call: its scratch lookup too
    _lib.check(lib.lbw_attention_fwd_noalloc(ctypes.byref(p), _lib.stream_ptr()), "capture")
graph.replay()
want = attention_segments(q, [(k, v)], num_splits=2)
torch.cuda.synchronize()
assert torch.equal(out, want)
print("first call under capture ok")
"""


def test_noalloc_first_call_under_capture(lib):
    """In a fresh process, the first no-alloc call on the device (which looks up the scratch
    address) made inside a graph capture: the capture and its replay work without a warm-up
    call."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_UNDER_CAPTURE, root,
                        os.path.join(root, "lingbot-world-v2_amd")],
                       capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr[-2000:])
    assert r.returncode == 0 and "first call under capture ok" in r.stdout
