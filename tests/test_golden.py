"""Committed golden fixtures (tests/golden/, written by make_golden.py from the oracle and the
reference's routing table): the oracle must still reproduce them on the CPU, and the HIP path
must match their expected outputs on the GPU."""
import json
import os

import numpy as np
import pytest
import torch

import oracle as O
from parity import assert_parity

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLDEN, name))


def bf16(a):
    return torch.from_numpy(a.astype(np.uint16).view(np.int16)).view(torch.bfloat16)


# ------------------------------------------------------------------ CPU: the oracle is unchanged

def test_oracle_reproduces_attention_fixture():
    z = _load("attention.npz")
    out = O.attention_ref(bf16(z["q"]), bf16(z["k"]), bf16(z["v"]), kv_lo=int(z["kv_lo"]),
                          kv_hi=int(z["kv_hi"]))
    assert torch.allclose(out, torch.from_numpy(z["out"]), atol=1e-6, rtol=1e-5)
    outc = O.attention_ref(bf16(z["qc"]), bf16(z["kc"]), bf16(z["vc"]),
                           k_lens=z["k_lens"].tolist())
    assert torch.allclose(outc, torch.from_numpy(z["outc"]), atol=1e-6, rtol=1e-5)


def test_oracle_reproduces_qk_fixture():
    z = _load("qk_norm_rope.npz")
    heads = int(z["heads"])
    C = z["q"].shape[1]
    cos, sin = O.causal_rope_grids(O.wan_rope_freqs(C // heads), *z["grid"].tolist(),
                                   start_frame=int(z["start_frame"]))
    for x, b, w, o in (("q", "bq", "wq", "q_out"), ("k", "bk", "wk", "k_out")):
        got = O.qk_post_norm_rope(bf16(z[x]), bf16(z[b]), bf16(z[w]), cos, sin, float(z["eps"]),
                                  heads)
        assert torch.equal(got, bf16(z[o])), x


def test_oracle_reproduces_fp8_fixture():
    z = _load("kv_quant_fp8.npz")
    codes, scales = O.quantize_kv_fp8(bf16(z["x"]))
    assert np.array_equal(codes.numpy(), z["codes"]) and np.array_equal(scales.numpy(), z["scales"])


def test_cache_plan_fixture():
    from lbw_amd.chunked_kv_cache import chunk_routing, plan_flat_write
    d = json.load(open(os.path.join(GOLDEN, "cache_plans.json")))
    for i, dest, lead in d["reference_routing_table_n4"] + d["routing_n4"]:
        assert O.chunk_routing(i, 4) == (dest, tuple(lead))
        assert chunk_routing(i, 4) == (dest, tuple(lead))
    fp = d["flat_plan"]
    ge = le = 0
    for p in fp["plans"]:
        c = p["chunk"]
        got = plan_flat_write(fp["kv_cache_size"], ge, le, c * fp["frame"], fp["frame"],
                              fp["sink_tokens"], fp["kv_cache_size"])
        assert got.write == tuple(p["write"]) and got.attn_lo == p["attn_lo"] \
            and got.attn_hi == p["attn_hi"] and got.global_end == p["global_end"] \
            and got.local_end == p["local_end"], c
        assert (got.roll is None and p["roll"] is None) or got.roll == tuple(p["roll"]), c
        ge, le = got.global_end, got.local_end


# ------------------------------------------------------------------ GPU: the HIP path matches

@pytest.mark.gpu
def test_hip_attention_matches_fixture(lib):
    from lbw_amd import attention_segments, cross_attention
    z = _load("attention.npz")
    out = attention_segments(bf16(z["q"]).cuda(), [(bf16(z["k"]).cuda(), bf16(z["v"]).cuda())],
                             kv_lo=int(z["kv_lo"]), kv_hi=int(z["kv_hi"]))
    assert_parity(out, torch.from_numpy(z["out"]), "window")
    k_lens = torch.from_numpy(z["k_lens"]).cuda()
    outc = cross_attention(bf16(z["qc"]).cuda(), bf16(z["kc"]).cuda(), bf16(z["vc"]).cuda(),
                           k_lens=k_lens)
    assert_parity(outc, torch.from_numpy(z["outc"]), "cross k_lens")


@pytest.mark.gpu
def test_hip_qk_norm_rope_matches_fixture(lib):
    from lbw_amd import causal_rope_tables, qk_norm_rope, wan_rope_freqs
    z = _load("qk_norm_rope.npz")
    heads = int(z["heads"])
    C = z["q"].shape[1]
    tabs = causal_rope_tables(wan_rope_freqs(C // heads), tuple(z["grid"].tolist()),
                              int(z["start_frame"]), device="cuda")
    qo, ko = qk_norm_rope(*(bf16(z[n]).cuda() for n in ("q", "k", "bq", "bk", "wq", "wk")),
                          tabs, float(z["eps"]), heads)
    for got, name in ((qo, "q_out"), (ko, "k_out")):
        ref = bf16(z[name]).float()
        d = (got.float().cpu() - ref).abs()
        # one bf16 rounding step of the pair's magnitude at most; almost all bitwise equal
        assert float(d.max()) <= 2.0 ** -5 * float(ref.abs().max()), name
        assert float((d == 0).float().mean()) >= 0.99, name


@pytest.mark.gpu
def test_hip_kv_quant_matches_fixture_bitwise(lib):
    from lbw_amd import quantize_kv_fp8
    z = _load("kv_quant_fp8.npz")
    q = quantize_kv_fp8(bf16(z["x"]).cuda())
    assert np.array_equal(q.codes.cpu().numpy(), z["codes"])
    assert np.array_equal(q.scales.cpu().numpy(), z["scales"])
