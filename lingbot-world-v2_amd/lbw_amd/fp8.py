"""fp8-e4m3 KV cache: quantiser and attention over quantised segments.

No reference counterpart (the reference keeps bf16 caches; its nearest relative is the
delayed fp8 K dequant of kernels/attention_cte_lb.py:645-647). Format: e4m3fn codes in the
cache's own ``[B, L, N, D]`` layout, plus fp32 scales ``[B, N, ceil(L/64)]`` per
(batch, head, 64-token block by index within the buffer): scale = amax/448 (1 for an
all-zero block), code = round_to_nearest_even(x / scale).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from .attention import _as_bf16, _check_4d, _params, _workspace, ctypes_ref

__all__ = ["Fp8KV", "quantize_kv_fp8", "attention_fp8kv"]

BLOCK = _lib.FP8_BLOCK


@dataclass
class Fp8KV:
    """A quantised K or V buffer: codes uint8 ``[B, L, N, D]``, scales fp32 ``[B, N, nblk]``."""
    codes: torch.Tensor
    scales: torch.Tensor


def quantize_kv_fp8(x: torch.Tensor, out: Fp8KV | None = None) -> Fp8KV:
    """bf16 ``[B, L, N, 128]`` -> :class:`Fp8KV` (into ``out`` when given)."""
    lib = _lib.load()
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
    with torch.cuda.device(x.device):
        _lib.check(lib.lbw_kv_quant_fp8(x.data_ptr(), B, L, H, D, x.stride(0), x.stride(1),
                                        x.stride(2), out.codes.data_ptr(), out.scales.data_ptr(),
                                        BLOCK, _lib.stream_ptr(x.device)), "lbw_kv_quant_fp8")
    return out


def attention_fp8kv(q: torch.Tensor, segments, *, kv_lo=None, kv_hi=None, softmax_scale=None,
                    num_splits: int = 0, out: torch.Tensor | None = None,
                    out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Attention of bf16 q ``[B, Lq, N, 128]`` over fp8 segments ``[(Fp8KV k, Fp8KV v), ...]``.

    The kernel converts each 64-token tile's codes exactly to bf16 on their way to LDS (every
    e4m3 value is a bf16 value) and runs the bf16 MFMA loop with q unquantised; the K block
    scale folds into the softmax exponent's multiplier and the V block scale into its addend
    (and out of the row sum). ``out_dtype=torch.float32`` returns the output before its bf16
    rounding."""
    lib = _lib.load()
    device = q.device
    _check_4d("q", q, device)
    q = _as_bf16(q)
    segs = []
    for k, v in segments:
        for t in (k, v):
            if t.codes.dtype != torch.uint8 or t.codes.device != device:
                raise ValueError("fp8 segments hold uint8 codes on q's device")
        segs.append((k.codes, v.codes, k.scales, v.scales))
    if out is None:
        out = torch.empty(q.shape, dtype=out_dtype, device=device)
    p = _params(q, out, segs, kv_lo, kv_hi, None, softmax_scale, num_splits)
    with torch.cuda.device(device):
        stream = _lib.stream_ptr(device)
        ws_bytes = lib.lbw_attention_fp8kv_workspace_size(ctypes_ref(p))
        ws = _workspace(device, stream, ws_bytes) if ws_bytes else None
        _lib.check(lib.lbw_attention_fwd_fp8kv(ctypes_ref(p), ws.data_ptr() if ws is not None else None,
                                               ws_bytes, stream),
                   "lbw_attention_fwd_fp8kv")
    return out
