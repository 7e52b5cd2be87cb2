"""Host-side cache logic of the product (lbw_amd.chunked_kv_cache), checked on the CPU against
the reference's own known-answer table and the oracle's restatement of the flat-cache write."""
import pytest
import torch

import oracle as O
from lbw_amd import chunked_kv_cache as C


def test_chunk_routing_reference_table():
    """chunked_kv_cache.py:54-59 (window 12, chunk 3 -> 4 chunks)."""
    n = C.num_chunks(12, 3)
    assert n == 4
    table = {0: (0, ()), 1: (1, (0,)), 2: (2, (0, 1)), 3: (3, (0, 1, 2)),
             4: (1, (0, 2, 3)), 5: (2, (0, 1, 3))}
    for i, want in table.items():
        assert C.chunk_routing(i, n) == want


@pytest.mark.parametrize("n", [1, 2, 3, 5, 8])
def test_chunk_routing_matches_oracle_and_invariants(n):
    for i in range(40):
        d, lead = C.chunk_routing(i, n)
        assert (d, lead) == O.chunk_routing(i, n)
        if n > 1:
            assert d not in lead and len(lead) == min(i, n - 1)
            if i > 0:
                assert d != 0 and 0 in lead           # the sink is never overwritten


@pytest.mark.parametrize("sink_f,window_f,chunk_f,max_att", [(1, 6, 2, None), (0, 4, 1, None),
                                                              (2, 9, 3, 5), (1, 5, 2, 3)])
def test_flat_plan_matches_oracle(sink_f, window_f, chunk_f, max_att):
    frame = 7
    size = window_f * frame
    mas = size if max_att is None else max_att * frame
    ge = le = 0
    for c in range(12):
        start, n = c * chunk_f * frame, chunk_f * frame
        p = C.plan_flat_write(size, ge, le, start, n, sink_f * frame, mas)
        o = O.flat_cache_write_plan(size, ge, le, start, n, sink_f * frame, mas)
        assert p.roll == o["roll"] and p.write == o["write"]
        assert (p.attn_lo, p.attn_hi, p.global_end, p.local_end) == \
               (o["attn_lo"], o["attn_hi"], o["global_end"], o["local_end"])
        ge, le = p.global_end, p.local_end


def test_global_cache_writes_in_place():
    p = C.plan_flat_write(100, 30, 30, 30, 10, 0, 100, local_attn_size=-1)
    assert p.write == (30, 40) and p.roll is None and (p.attn_lo, p.attn_hi) == (0, 40)


def test_allocate_and_order_chunks():
    cache = C.allocate_self_kv_chunks(2, 1, 8, 2, 4, 4, device="cpu")
    assert len(cache) == 2 and len(cache[0]["k"]) == 4
    assert C.chunk_bytes(cache) == 2 * 2 * 4 * 8 * 2 * 4 * 2
    ks, vs = C.ordered_chunks(cache[0], 2, (0, 1, 3))
    assert ks[-1] is cache[0]["k"][2] and vs[0] is cache[0]["v"][0]


def test_allocate_fp8_chunks_layout():
    """fp8 chunk slots: uint8 codes in the token-major layout, one fp32 scale per (batch, head,
    64-token block of the slot), and one bf16 staging pair per layer."""
    cache = C.allocate_self_kv_chunks_fp8(2, 1, 100, 3, 128, 4, device="cpu")
    assert len(cache) == 2 and len(cache[0]["k"]) == 4 and len(cache[1]["v"]) == 4
    s = cache[0]["k"][1]
    assert s.codes.shape == (1, 100, 3, 128) and s.codes.dtype == torch.uint8
    assert s.scales.shape == (1, 3, 2) and bool((s.scales == 1).all())
    assert cache[0]["stage"]["v"].shape == (1, 100, 3, 128)
    assert cache[0]["stage"]["k"].dtype == torch.bfloat16

