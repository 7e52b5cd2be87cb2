"""Fused q/k post-processing: bias + RMSNorm + Wan 3-D RoPE in one gfx950 kernel.

Mirrors kernels/qk_post.py (exports at 404-413). The reference splits it into ``qk_ss``
(sums of squares), a TP all-reduce, and ``qk_norm_rope``; one GPU holds the whole row, so
``qk_norm_rope`` here computes the sums itself. The rounding sequence is the reference
kernel's (qk_post.py:88-141): y = x + b (fp32), r = rsqrt(sum(y^2)/C + eps),
t = bf16(y r) * gamma (fp32), RoPE in fp32, one bf16 rounding of the result.
"""
from __future__ import annotations

import torch

from . import _lib
from .attention import ctypes_ref
from .rope import RopeTables

__all__ = ["qk_norm_rope", "qk_norm_rope_"]


def _rows(name, t, C):
    if t.dim() != 2 or t.shape[1] != C or t.stride(1) != 1 or t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bf16 [L, {C}] with contiguous rows, got "
                         f"{tuple(t.shape)} {t.dtype} strides {t.stride()}")


def qk_norm_rope_(q, k, bq, bk, wq, wk, rope: RopeTables, eps: float, heads: int, *, q_out,
                  k_out, q_scale: float = 1.0, k_scale: float = 1.0, v=None, v_out=None):
    """Write-into form: q, k ``[L, C]`` bf16 rows -> q_out, k_out (row-strided views are fine,
    e.g. a KV-cache slot ``cache_k[0, s:e].view(L, C)``). Optionally copies v into v_out (the
    new chunk's V commit). ``bq``/``bk`` may be None."""
    lib = _lib.load()
    L, C = q.shape
    for name, t in (("q", q), ("k", k), ("q_out", q_out), ("k_out", k_out)):
        _rows(name, t, C)
        if t.shape[0] != L:
            raise ValueError(f"{name} has {t.shape[0]} rows, q has {L}")
    for name, t in (("wq", wq), ("wk", wk), ("bq", bq), ("bk", bk)):
        if t is not None and (t.numel() != C or t.dtype != torch.bfloat16 or not t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous bf16 [C] vector")
    p = _lib.QkNormRopeParams()
    p.tokens, p.dim, p.heads = L, C, heads
    p.q, p.q_stride = q.data_ptr(), q.stride(0)
    p.k, p.k_stride = k.data_ptr(), k.stride(0)
    p.bq = bq.data_ptr() if bq is not None else None
    p.bk = bk.data_ptr() if bk is not None else None
    p.wq, p.wk = wq.data_ptr(), wk.data_ptr()
    p.eps = float(eps)
    p.rope = rope.packed.data_ptr()
    p.grid_f, p.grid_h, p.grid_w, p.s0, p.s1 = rope.f, rope.h, rope.w, rope.s0, rope.s1
    p.q_out, p.q_out_stride = q_out.data_ptr(), q_out.stride(0)
    p.k_out, p.k_out_stride = k_out.data_ptr(), k_out.stride(0)
    p.q_out_scale, p.k_out_scale = float(q_scale), float(k_scale)
    if v is not None:
        _rows("v", v, C)
        _rows("v_out", v_out, C)
        p.v, p.v_stride = v.data_ptr(), v.stride(0)
        p.v_out, p.v_out_stride = v_out.data_ptr(), v_out.stride(0)
    if rope.packed.device != q.device:
        raise ValueError("rope tables are on another device")
    with torch.cuda.device(q.device):
        _lib.check(lib.lbw_qk_norm_rope(ctypes_ref(p), _lib.stream_ptr(q.device)), "lbw_qk_norm_rope")
    return q_out, k_out


def qk_norm_rope(q, k, bq, bk, wq, wk, rope: RopeTables, eps: float = 1e-6,
                 heads: int | None = None, q_scale: float = 1.0):
    """kernels/qk_post.py qk_norm_rope without the separate sums/all-reduce: returns new
    ``(q', k')`` bf16 ``[L, C]``."""
    L, C = q.shape
    D = 2 * (rope.s0 + 2 * rope.s1)
    heads = heads if heads is not None else C // D
    qo = torch.empty_like(q)
    ko = torch.empty_like(k)
    return qk_norm_rope_(q, k, bq, bk, wq, wk, rope, eps, heads, q_out=qo, k_out=ko,
                         q_scale=q_scale)
