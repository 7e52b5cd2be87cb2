"""fp8-e4m3 KV cache: quantiser and attention over quantised segments.

No reference counterpart (the reference keeps bf16 caches; its nearest relative is the
delayed fp8 K dequant of kernels/attention_cte_lb.py:645-647). Format: e4m3fn codes in the
cache's own ``[B, L, N, D]`` layout, plus fp32 scales ``[B, N, ceil(L/64)]`` per
(batch, head, 64-token block by index within the buffer): scale = the smallest power of two
>= amax/448 (1 for an all-zero block), code = round_to_nearest_even(x / scale). The attention
reads only power-of-two scales (rows that read any other come out NaN): K's scale is the
exponent scale of the fp8 matrix-core product and V's the scale of the codes' exact conversion
to bf16, so neither enters the softmax.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from .attention import _as_bf16, _bounds, _check_4d

__all__ = ["Fp8KV", "quantize_kv_fp8", "attention_fp8kv"]

BLOCK = _lib.FP8_BLOCK


@dataclass
class Fp8KV:
    """A quantised K or V buffer: codes uint8 ``[B, L, N, D]``, scales fp32 ``[B, N, nblk]``."""
    codes: torch.Tensor
    scales: torch.Tensor


def quantize_kv_fp8(x: torch.Tensor, out: Fp8KV | None = None) -> Fp8KV:
    """bf16 ``[B, L, N, 128]`` -> :class:`Fp8KV` (into ``out`` when given)."""
    ops = _lib.ops()
    _check_4d("x", x, x.device)
    x = _as_bf16(x)
    B, L, H, D = x.shape
    nblk = (L + BLOCK - 1) // BLOCK
    if out is None:
        out = Fp8KV(torch.empty(B, L, H, D, dtype=torch.uint8, device=x.device),
                    torch.empty(B, H, nblk, dtype=torch.float32, device=x.device))
    if out.codes.shape != (B, L, H, D) or not out.codes.is_contiguous():
        raise ValueError("codes must be contiguous [B, L, N, D] uint8")
    if out.scales.shape != (B, H, nblk) or not out.scales.is_contiguous():
        raise ValueError(f"scales must be contiguous [B, N, {nblk}] fp32")
    ops.kv_quant_fp8_(x, out.codes, out.scales)
    return out


def attention_fp8kv(q: torch.Tensor, segments, *, kv_lo=None, kv_hi=None, softmax_scale=None,
                    num_splits: int = 0, out: torch.Tensor | None = None,
                    out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Attention of bf16 q ``[B, Lq, N, 128]`` over fp8 segments ``[(Fp8KV k, Fp8KV v), ...]``.

    Q K^T runs on the fp8 matrix cores: the K codes go to LDS as they are, and each query is
    split into two e4m3 operands (hi + lo / 16, times a power of two per query) that hold its
    bf16 values, with K's block scale (a power of two) as the product's exponent scale. The V
    codes are converted exactly to bf16 at V's block scale and P V runs on the bf16 matrix
    cores. A q pre-scaled by ``prescaled_q_scale`` with ``softmax_scale=PRESCALED_SOFTMAX_SCALE``
    takes the folded softmax, as in ``attention_segments``.
    ``out_dtype=torch.float32`` returns the output before its bf16 rounding."""
    ops = _lib.ops()
    device = q.device
    _check_4d("q", q, device)
    q = _as_bf16(q)
    if not 1 <= len(segments) <= _lib.MAX_KV_SEGMENTS:
        raise ValueError(f"{len(segments)} KV segments: 1..{_lib.MAX_KV_SEGMENTS} supported")
    kc, vc, ksc, vsc = [], [], [], []
    for k, v in segments:
        for t in (k, v):
            if t.codes.dtype != torch.uint8 or t.codes.device != device:
                raise ValueError("fp8 segments hold uint8 codes on q's device")
        kc.append(k.codes)
        vc.append(v.codes)
        ksc.append(k.scales)
        vsc.append(v.scales)
    lo, hi, dlo, dhi = _bounds(kv_lo, kv_hi, device)
    scale = 0.0 if softmax_scale is None else float(softmax_scale)
    if out is None:
        return ops.attention_fp8kv(q, kc, vc, ksc, vsc, lo, hi, scale, int(num_splits),
                                   out_dtype == torch.float32, dlo, dhi)
    if out.dtype not in (torch.bfloat16, torch.float32) or out.shape != q.shape:
        raise ValueError("out must be a bf16 or fp32 tensor of q's shape")
    ops.attention_fp8kv_out(q, kc, vc, ksc, vsc, lo, hi, scale, int(num_splits), out, dlo, dhi)
    return out
