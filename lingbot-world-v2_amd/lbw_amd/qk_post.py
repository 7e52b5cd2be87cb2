"""Fused q/k post-processing: bias + RMSNorm + Wan 3-D RoPE in one gfx950 kernel.

Mirrors kernels/qk_post.py (exports at 404-413). The reference splits it into ``qk_ss``
(sums of squares), a TP all-reduce, and ``qk_norm_rope``; one GPU holds the whole row, so
``qk_norm_rope`` here computes the sums itself. The rounding sequence is the reference
kernel's (qk_post.py:88-141): y = x + b (fp32), r = rsqrt(sum(y^2)/C + eps),
t = bf16(y r) * gamma (fp32), RoPE in fp32 with an output scale folded into cos/sin
(qk_post.py:259-265), one bf16 rounding of the result.

Variants, as in the reference:
- ``qk_norm_rope`` / ``qk_norm_rope3``: q' and k' as ``[L, C]`` rows;
- ``qk_norm_rope_t`` / ``qk_norm_rope_t3`` (qk_post.py:216-306): head-major, d-major
  ``[H, D, L]`` outputs, q pre-scaled (1/sqrt(D) by default);
- ``x_norm_rope`` / ``x_norm_rope_t3`` (qk_post.py:166-215, 331-402): one tensor alone.
The ``*3`` forms take the fused projection output ``[L, 3C]`` (q, k, v column blocks).
"""
from __future__ import annotations

import math

import torch

from . import _lib
from .rope import RopeTables

__all__ = ["qk_norm_rope", "qk_norm_rope_", "qk_norm_rope3", "qk_norm_rope_t", "qk_norm_rope_t3",
           "x_norm_rope", "x_norm_rope_t3"]

LAYOUT_ROWS = 0
LAYOUT_DMAJOR = 1


def _rows(name, t, C):
    if t.dim() != 2 or t.shape[1] != C or t.stride(1) != 1 or t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bf16 [L, {C}] with contiguous rows, got "
                         f"{tuple(t.shape)} {t.dtype} strides {t.stride()}")


def _dmajor(name, t, H, D, L):
    """[H, D, L] with token stride 1 and head stride D * (d stride); returns the d stride."""
    if (t.dim() != 3 or tuple(t.shape) != (H, D, L) or t.dtype != torch.bfloat16
            or t.stride(2) != 1 or t.stride(0) != D * t.stride(1)):
        raise ValueError(f"{name} must be bf16 [{H}, {D}, {L}] with strides (D*s, s, 1), got "
                         f"{tuple(t.shape)} {t.dtype} strides {t.stride()}")
    return t.stride(1)


def _head_dim(rope: RopeTables) -> int:
    return 2 * (rope.s0 + 2 * rope.s1)


def qk_norm_rope_(q, k, bq, bk, wq, wk, rope: RopeTables, eps: float, heads: int, *, q_out,
                  k_out, q_scale: float = 1.0, k_scale: float = 1.0, v=None, v_out=None,
                  layout: str = "rows"):
    """Write-into form: q, k ``[L, C]`` bf16 rows (row-strided views are fine, e.g. column
    blocks of a fused ``[L, 3C]`` projection) -> q_out, k_out.

    ``layout="rows"``: outputs ``[L, C]`` with contiguous rows, e.g. a KV-cache slot
    ``cache_k[0, s:e].view(L, C)``. ``layout="dmajor"``: outputs ``[H, D, L]`` with token
    stride 1, e.g. ``cache_kt[:, :, s:e]`` of a ``[H, D, capacity]`` cache.
    ``k=None`` processes q alone (``k_out``/``wk``/``bk`` ignored). Optionally copies v into
    v_out (rows; the new chunk's V commit). ``bq``/``bk`` may be None."""
    ops = _lib.ops()
    L, C = q.shape
    if layout not in ("rows", "dmajor"):
        raise ValueError(f"layout {layout!r}: 'rows' or 'dmajor'")
    D = C // heads
    has_k = k is not None
    _rows("q", q, C)
    if has_k:
        _rows("k", k, C)
        if k.shape[0] != L:
            raise ValueError(f"k has {k.shape[0]} rows, q has {L}")
    outs = (("q_out", q_out),) + ((("k_out", k_out),) if has_k else ())
    for name, t in outs:
        if layout == "rows":
            _rows(name, t, C)
            if t.shape[0] != L:
                raise ValueError(f"{name} has {t.shape[0]} rows, q has {L}")
        else:
            _dmajor(name, t, heads, D, L)
    vecs = (("wq", wq), ("bq", bq)) + ((("wk", wk), ("bk", bk)) if has_k else ())
    for name, t in vecs:
        if t is not None and (t.numel() != C or t.dtype != torch.bfloat16 or not t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous bf16 [C] vector")
    if v is not None:
        _rows("v", v, C)
        _rows("v_out", v_out, C)
    if rope.packed.device != q.device:
        raise ValueError("rope tables are on another device")
    ops.qk_norm_rope_(q, k, bq, bk if has_k else None, wq, wk if has_k else None, rope.packed,
                      [rope.f, rope.h, rope.w, rope.s0, rope.s1], float(eps), heads, q_out,
                      k_out if has_k else None, v, v_out if v is not None else None,
                      float(q_scale), float(k_scale),
                      LAYOUT_ROWS if layout == "rows" else LAYOUT_DMAJOR)
    return (q_out, k_out) if has_k else q_out


def qk_norm_rope(q, k, bq, bk, wq, wk, rope: RopeTables, eps: float = 1e-6,
                 heads: int | None = None, q_scale: float = 1.0):
    """kernels/qk_post.py qk_norm_rope without the separate sums/all-reduce: returns new
    ``(q', k')`` bf16 ``[L, C]``."""
    L, C = q.shape
    heads = heads if heads is not None else C // _head_dim(rope)
    qo = torch.empty_like(q)
    ko = torch.empty_like(k)
    return qk_norm_rope_(q, k, bq, bk, wq, wk, rope, eps, heads, q_out=qo, k_out=ko,
                         q_scale=q_scale)


def qk_norm_rope3(qkv, bq, bk, wq, wk, rope: RopeTables, eps: float = 1e-6,
                  heads: int | None = None):
    """kernels/qk_post.py:81-86: ``qk_norm_rope`` on the fused projection ``[L, 3C]``."""
    C = wq.numel()
    return qk_norm_rope(qkv[:, :C], qkv[:, C:2 * C], bq, bk, wq, wk, rope, eps, heads)


def qk_norm_rope_t(q, k, bq, bk, wq, wk, rope: RopeTables, eps: float = 1e-6,
                   heads: int | None = None, q_scale: float | None = None):
    """kernels/qk_post.py:216-306 (``qk_norm_rope_t``): new ``(q_t, k_t)`` bf16 ``[H, D, L]``,
    q_t scaled by ``q_scale`` (default 1/sqrt(D)) through cos/sin."""
    L, C = q.shape
    D = _head_dim(rope)
    heads = heads if heads is not None else C // D
    q_scale = 1.0 / math.sqrt(D) if q_scale is None else q_scale
    qt = torch.empty(heads, D, L, dtype=torch.bfloat16, device=q.device)
    kt = torch.empty(heads, D, L, dtype=torch.bfloat16, device=q.device)
    return qk_norm_rope_(q, k, bq, bk, wq, wk, rope, eps, heads, q_out=qt, k_out=kt,
                         q_scale=q_scale, layout="dmajor")


def qk_norm_rope_t3(qkv, bq, bk, wq, wk, rope: RopeTables, eps: float = 1e-6,
                    heads: int | None = None, q_scale: float | None = None):
    """kernels/qk_post.py:221-225: ``qk_norm_rope_t`` on the fused projection ``[L, 3C]``."""
    C = wq.numel()
    return qk_norm_rope_t(qkv[:, :C], qkv[:, C:2 * C], bq, bk, wq, wk, rope, eps, heads, q_scale)


def x_norm_rope(x, b, w, rope: RopeTables, eps: float = 1e-6, heads: int | None = None,
                scale: float = 1.0):
    """kernels/qk_post.py:166-215 (``x_norm_rope``): one tensor, new ``[L, C]`` rows."""
    L, C = x.shape
    heads = heads if heads is not None else C // _head_dim(rope)
    out = torch.empty_like(x)
    return qk_norm_rope_(x, None, b, None, w, None, rope, eps, heads, q_out=out, k_out=None,
                         q_scale=scale)


def x_norm_rope_t3(qkv, c0: int, b, w, rope: RopeTables, eps: float = 1e-6,
                   heads: int | None = None, scale: float = 1.0):
    """kernels/qk_post.py:331-402 (``x_norm_rope_t3``): columns ``c0 .. c0 + C`` of the fused
    projection, one tensor -> new ``[H, D, L]`` scaled by ``scale`` through cos/sin."""
    C = w.numel()
    x = qkv[:, c0:c0 + C]
    L = x.shape[0]
    D = _head_dim(rope)
    heads = heads if heads is not None else C // D
    out = torch.empty(heads, D, L, dtype=torch.bfloat16, device=x.device)
    return qk_norm_rope_(x, None, b, None, w, None, rope, eps, heads, q_out=out, k_out=None,
                         q_scale=scale, layout="dmajor")
