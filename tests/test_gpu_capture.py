"""The hot path under the two ways a PyTorch program hands it to the runtime as a whole:

- HIP graphs: the per-layer chunk step (fused q/k RMSNorm + RoPE writing the pre-scaled q and the
  chunk's K/V into its cache slot, then the folded-softmax attention with split pieces, work
  queues and the merge) captured once and replayed with new inputs, with eager work and
  synchronisations between the replays; every replay is checked bitwise against an eager run of
  the same step (the kernels are deterministic: the work queues change which workgroup runs an
  item, not what it computes). The work-queue counters are cleared by a kernel, not a memset, so
  the captured graph stays correct on every replay.
- torch.compile: the `torch.ops.lbw` operators carry Meta implementations, so a function calling
  them traces as one graph (fullgraph=True fails on any graph break) and gives the eager results.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
H, D = 4, 128
C = H * D
GRID = (1, 20, 30)            # 600 tokens per chunk
LQ = GRID[0] * GRID[1] * GRID[2]
CACHED = 3                    # frames before the chunk
LK = LQ * (CACHED + 1)


def _step(bufs, tabs):
    from lbw_amd import PRESCALED_SOFTMAX_SCALE, attention_segments, prescaled_q_scale, qk_norm_rope_
    slot = slice(LK - LQ, LK)
    qk_norm_rope_(bufs["xq"], bufs["xk"], None, None, bufs["wq"], bufs["wk"], tabs, 1e-6, H,
                  q_out=bufs["q"], k_out=bufs["ck"][0, slot].view(LQ, C), v=bufs["xv"],
                  v_out=bufs["cv"][0, slot].view(LQ, C), q_scale=prescaled_q_scale(D))
    attention_segments(bufs["q"].view(1, LQ, H, D), [(bufs["ck"], bufs["cv"])], out=bufs["out"],
                       softmax_scale=PRESCALED_SOFTMAX_SCALE, num_splits=3)


def _buffers(g):
    rnd = lambda *s: torch.randn(*s, generator=g, device=DEV).to(torch.bfloat16)
    return dict(xq=rnd(LQ, C), xk=rnd(LQ, C), xv=rnd(LQ, C),
                wq=(1 + 0.1 * torch.randn(C, generator=g, device=DEV)).to(torch.bfloat16),
                wk=(1 + 0.1 * torch.randn(C, generator=g, device=DEV)).to(torch.bfloat16),
                q=torch.empty(LQ, C, dtype=torch.bfloat16, device=DEV),
                ck=rnd(1, LK, H, D), cv=rnd(1, LK, H, D),
                out=torch.empty(1, LQ, H, D, dtype=torch.bfloat16, device=DEV))


def test_hip_graph_replays_the_chunk_step(lib):
    from lbw_amd import causal_rope_tables, wan_rope_freqs
    g = torch.Generator(device=DEV).manual_seed(3)
    tabs = causal_rope_tables(wan_rope_freqs(D), GRID, CACHED, device=DEV)
    static = _buffers(g)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):   # warm-up off the capture stream, as torch requires
        _step(static, tabs)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _step(static, tabs)
    torch.cuda.synchronize()
    for rep in range(3):
        print(f"replay {rep}", flush=True)
        fresh = _buffers(g)
        for name in ("xq", "xk", "xv", "wq", "wk", "ck", "cv"):
            static[name].copy_(fresh[name])
        graph.replay()
        _step(fresh, tabs)                       # eager, same stream, between the replays
        torch.cuda.synchronize()
        for name in ("q", "ck", "cv", "out"):
            d = (static[name].float() - fresh[name].float()).abs()
            print(f"  {name}: max diff {float(d.max()):.3e}, differing {int((d > 0).sum())} of {d.numel()}")
        assert torch.equal(static["out"], fresh["out"]), rep
        assert torch.equal(static["q"], fresh["q"]), rep
        assert torch.equal(static["ck"], fresh["ck"]) and torch.equal(static["cv"], fresh["cv"]), rep
        assert float(static["out"].float().abs().sum()) > 0


def test_torch_compile_traces_the_ops_as_one_graph(lib):
    from lbw_amd import _lib
    _lib.ops()  # registers torch.ops.lbw
    g = torch.Generator(device=DEV).manual_seed(4)
    rnd = lambda *s: torch.randn(*s, generator=g, device=DEV).to(torch.bfloat16)
    q, k, v = rnd(1, 300, H, D), rnd(1, 1000, H, D), rnd(1, 1000, H, D)
    kc, vc = rnd(1, 512, H, D), rnd(1, 512, H, D)
    kl = torch.tensor([300], dtype=torch.int32, device=DEV)

    def f(q, k, v, kc, vc, kl):
        o = torch.ops.lbw.attention(q, [k[:, :600], k[:, 600:]], [v[:, :600], v[:, 600:]],
                                    10, 990, None, 0.0, 2, False)
        x = torch.ops.lbw.cross_attention(o, kc, vc, kl, -1, 0, -1, 0.0, False)
        return x.float().mul(2.0)

    torch._dynamo.reset()
    cf = torch.compile(f, backend="aot_eager", fullgraph=True)
    got = cf(q, k, v, kc, vc, kl)
    want = f(q, k, v, kc, vc, kl)
    torch.cuda.synchronize()
    assert got.shape == (1, 300, H, D)
    assert torch.equal(got, want)


def _xstep(b):
    """Cross-attention to a masked context, then the fp8-KV path: the quantiser and the fp8
    attention over 3 pieces (work queues and merge); returns both outputs."""
    from lbw_amd import attention_fp8kv, cross_attention, quantize_kv_fp8
    x = cross_attention(b["q"], b["kc"], b["vc"], k_lens=b["kl"])
    k8, v8 = quantize_kv_fp8(b["k"]), quantize_kv_fp8(b["v"])
    y = attention_fp8kv(b["q"], [(k8, v8)], kv_lo=10, num_splits=3)
    return x, y


def _xbuffers(g, valid):
    rnd = lambda *s: torch.randn(*s, generator=g, device=DEV).to(torch.bfloat16)
    return dict(q=rnd(1, LQ, H, D), kc=rnd(1, 512, H, D), vc=rnd(1, 512, H, D),
                kl=torch.tensor([valid], dtype=torch.int32, device=DEV),
                k=rnd(1, 1500, H, D), v=rnd(1, 1500, H, D))


def test_hip_graph_replays_cross_and_fp8(lib):
    """The cross-attention kernel and the fp8-KV path (quantiser, fp8 attention with split
    pieces, work queues, merge) captured once and replayed with new inputs -- a new valid
    context length read by the kernel from the device each replay included -- each replay
    bitwise equal to an eager run between the replays."""
    g = torch.Generator(device=DEV).manual_seed(5)
    static = _xbuffers(g, 300)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _xstep(static)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = _xstep(static)
    torch.cuda.synchronize()
    for rep, valid in enumerate((300, 77, 512)):
        print(f"replay {rep}: {valid} valid context rows", flush=True)
        fresh = _xbuffers(g, valid)
        for name in ("q", "kc", "vc", "kl", "k", "v"):
            static[name].copy_(fresh[name])
        graph.replay()
        want = _xstep(fresh)
        torch.cuda.synchronize()
        for what, got, ref in zip(("cross", "fp8"), outs, want):
            d = (got.float() - ref.float()).abs()
            print(f"  {what}: max diff {float(d.max()):.3e}, differing {int((d > 0).sum())}")
            assert torch.equal(got, ref), (rep, what)
            assert float(ref.float().abs().sum()) > 0
