"""GPU parity of a per-key additive score bias (cross_attention_dedup's bias,
wan/modules/attention.py:532-554): softmax(scale q k^T + bias) v against the oracle, for an
arbitrary bias, the reference's dedup bias (cross_dedup_bias) on token-major and N-major caches,
and with d-major K."""
import pytest
import torch

import oracle as O
from parity import assert_parity, metrics

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(B, Lq, H, L, seed, vscale=1.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Lq, H, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(B, L, H, 128, generator=g).to(torch.bfloat16)
    v = (vscale * torch.randn(B, L, H, 128, generator=g)).to(torch.bfloat16)
    bias = 2.0 * torch.randn(L, generator=g)
    return q, k, v, bias


@pytest.mark.parametrize("B,Lq,H,lens", [(1, 300, 2, [512]), (2, 77, 3, [100, 230, 64]),
                                         (1, 513, 4, [3000])])
def test_arbitrary_key_bias_matches_oracle(lib, B, Lq, H, lens):
    from lbw_amd import attention_segments
    q, k, v, bias = _case(B, Lq, H, sum(lens), seed=Lq, vscale=0.5)
    segs, o = [], 0
    for L in lens:
        segs.append((k[:, o:o + L].to(DEV), v[:, o:o + L].to(DEV)))
        o += L
    out = attention_segments(q.to(DEV), segs, key_bias=bias.to(DEV))
    ref = O.attention_key_bias_ref(q, k, v, bias)
    print(f"key bias B={B} Lq={Lq} H={H} lens={lens}", metrics(out, ref))
    assert_parity(out, ref)


def test_key_bias_with_window_and_dmajor_k(lib):
    """The bias is indexed by key position in the concatenation, the window cuts keys from it;
    with d-major K as well."""
    from lbw_amd import attention_segments
    q, k, v, bias = _case(1, 200, 2, 1024, seed=5, vscale=0.5)
    kd = torch.zeros(1, 2, 128, 1024, dtype=torch.bfloat16, device=DEV)
    kd[:] = k.to(DEV).permute(0, 2, 3, 1)
    out = attention_segments(q.to(DEV), [(kd.permute(0, 3, 1, 2), v.to(DEV))], kv_lo=100,
                             kv_hi=900, key_bias=bias.to(DEV))
    ref = O.attention_key_bias_ref(q, k[:, 100:900], v[:, 100:900], bias[100:900])
    assert_parity(out, ref)


def test_reference_dedup_bias_equals_full_context(lib):
    """cross_attention_dedup with the reference's cross_dedup_bias over the first kc rows equals
    attention over all 512 context rows (rows 300.. identical), on the token-major cache and on
    the N-major cache ([N, D, L] K, [N, L, D] V) as the reference passes it."""
    from lbw_amd import cross_attention_dedup
    g = torch.Generator().manual_seed(8)
    H, Lq, kc = 4, 600, 384
    q = torch.randn(1, Lq, H, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 512, H, 128, generator=g).to(torch.bfloat16)
    v = (0.5 * torch.randn(1, 512, H, 128, generator=g)).to(torch.bfloat16)
    k[:, 300:] = k[:, 511:]
    v[:, 300:] = v[:, 511:]
    bias = O.cross_dedup_bias(k[0], v[0], kc)
    full = O.attention_ref(q, k, v)
    out = cross_attention_dedup(q.to(DEV), k.to(DEV), v.to(DEV), bias.to(DEV), kc)
    assert_parity(out, full, "token-major")
    k_ndl = k[0].permute(1, 2, 0).contiguous().to(DEV)      # [N, D, L]
    v_nld = v[0].permute(1, 0, 2).contiguous().to(DEV)      # [N, L, D]
    out_n = cross_attention_dedup(q.to(DEV), k_ndl, v_nld, bias.to(DEV), kc)
    assert_parity(out_n, full, "N-major")
    assert_parity(out_n, O.attention_key_bias_ref(q, k[:, :kc], v[:, :kc], bias), "bias form")


def test_key_bias_refusals(lib):
    from lbw_amd import _lib, attention_segments
    q, k, v, bias = _case(1, 64, 2, 300, seed=1)
    with pytest.raises(RuntimeError, match="key_bias"):
        attention_segments(q.to(DEV), [(k.to(DEV), v.to(DEV))], key_bias=bias[:299].to(DEV))
    with pytest.raises(ValueError, match="n_distinct"):
        attention_segments(q.to(DEV), [(k.to(DEV), v.to(DEV))], key_bias=bias.to(DEV),
                           cross=True, n_distinct=200)
