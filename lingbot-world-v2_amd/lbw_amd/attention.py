"""Drop-in attention entry points backed by the gfx950 kernels of liblbw_attn.so.

Mirrors wan/modules/attention.py: ``attention()`` keeps the reference signature
(attention.py:1082-1100) and its layout contract (q ``[B, Lq, N, D]``, k/v ``[B, Lk, N, D]``
-> ``[B, Lq, N, D]``), ``flash_attention`` is its alias (attention.py:1146),
``exact_attention`` / ``exact_attention_chunks`` take the chunked cache's chunk lists
without concatenating them (attention.py:1048-1079), and ``attention_partial`` /
``attention_merge`` carry the unnormalised (O, row max, row sum) contract of
``cte_partial`` / ``cte_merge`` (attention.py:617-645, 963-990).

Every call goes through the torch op set ``torch.ops.lbw`` (liblbw_torch.so, over the C ABI
of liblbw_attn.so), runs on the tensors' device on torch's current stream, and raises when a
library is missing or rejects the arguments: there is no CPU or SDPA fallback.
"""
from __future__ import annotations

import math
import warnings
from typing import Sequence

import torch

from . import _lib

__all__ = ["attention", "flash_attention", "exact_attention", "exact_attention_chunks",
           "cross_attention", "cross_attention_dedup", "attention_partial", "attention_merge", "attention_merge_partials",
           "attention_chain",
           "attention_segments", "window_from_mask", "PRESCALED_SOFTMAX_SCALE",
           "prescaled_q_scale"]


def _check_dtype(dtype):
    """The kernels compute in bf16 (bf16 MFMA, fp32 softmax and accumulators). The reference
    casts q/k/v to ``dtype`` and runs SDPA in it (attention.py:1134-1141): any other ``dtype``
    would silently get bf16 accuracy here, so it raises instead."""
    if dtype != torch.bfloat16:
        raise NotImplementedError(f"dtype={dtype}: this attention path computes in bfloat16 only")


def _as_bf16(t: torch.Tensor) -> torch.Tensor:
    t = t if t.dtype == torch.bfloat16 else t.to(torch.bfloat16)
    if t.stride(-1) != 1:
        t = t.contiguous()
    return t


def _as_bf16_k(t: torch.Tensor) -> torch.Tensor:
    """A K segment: token-major ``[B, L, N, D]`` with a contiguous head dim, or a d-major view
    of the reference's N-major K cache (``k_ndl.permute(2, 0, 1)[None]`` of an ``[N, D, L]``
    buffer: token stride 1), which the kernel reads as it lies."""
    if t.dtype == torch.bfloat16 and t.dim() == 4 and t.stride(-1) != 1 and t.stride(1) == 1:
        return t
    return _as_bf16(t)


def _check_4d(name, t, device):
    if t.dim() != 4:
        raise ValueError(f"{name} must be [B, L, N, D], got shape {tuple(t.shape)}")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, q on {device}")
    if t.device.type != "cuda":
        raise RuntimeError(f"{name} must be a GPU tensor (the path has no CPU implementation)")


def _bounds(kv_lo, kv_hi, device):
    """(host lo, host hi, device lo, device hi) of a window given as ints, host tensors or
    one-element integer tensors on ``device`` (read there by the kernel: no host sync)."""
    out = []
    for b, default in ((kv_lo, 0), (kv_hi, -1)):
        if b is None:
            out.append((default, None))
        elif torch.is_tensor(b) and b.device.type != "cpu":
            if b.device != device or b.numel() != 1 or b.dtype.is_floating_point or b.dtype == torch.bool:
                raise ValueError("a device window bound must be a one-element integer tensor "
                                 "on q's device")
            out.append((default, b.reshape(1)))
        else:
            out.append((int(b), None))
    (lo, dlo), (hi, dhi) = out
    return lo, hi, dlo, dhi


def attention_segments(q: torch.Tensor, segments: Sequence, *, kv_lo=None, kv_hi=None,
                       k_lens: torch.Tensor | None = None, softmax_scale=None,
                       num_splits: int = 0, out: torch.Tensor | None = None,
                       cross: bool = False, n_distinct: int | None = None,
                       out_dtype: torch.dtype = torch.bfloat16,
                       key_bias: torch.Tensor | None = None) -> torch.Tensor:
    """softmax(scale Q K^T) V over the windowed concatenation of KV ``segments``.

    q ``[B, Lq, N, 128]``; each segment is ``(k, v)`` with k/v ``[B, L_i, N, 128]`` (strided
    views are fine as long as the head dim is contiguous; K may instead be a d-major view, token
    stride 1, of the reference's N-major ``[N, D, L]`` K cache -- every segment's or none); the window ``[kv_lo, kv_hi)``
    indexes the concatenation (ints, or one-element integer tensors on q's device that the
    kernel reads there, so the call needs no host sync). ``k_lens`` (int32 ``[B]`` on the device) limits each batch's
    keys. With ``cross``, a single short segment; ``n_distinct`` (cross only) declares keys
    ``n_distinct..`` identical rows, attended as one key of that multiplicity (exact).
    Returns bf16 ``[B, Lq, N, 128]`` (into ``out`` when given). ``out_dtype=torch.float32``
    (or an fp32 ``out``) returns the normalised output before its bf16 rounding, from the same
    kernels and plan: a check of the kernels' own arithmetic. ``key_bias`` (fp32, one value per
    key of the concatenation, shared by batch and heads) is added to the scaled scores:
    softmax(scale Q K^T + bias) V."""
    ops = _lib.ops()
    device = q.device
    _check_4d("q", q, device)
    q = _as_bf16(q)
    ks, vs = _segments(segments, device)
    scale = 0.0 if softmax_scale is None else float(softmax_scale)
    lo, hi, dlo, dhi = _bounds(kv_lo, kv_hi, device)
    if out is not None:
        if out.dtype not in (torch.bfloat16, torch.float32) or out.shape != q.shape:
            raise ValueError("out must be a bf16 or fp32 tensor of q's shape")
    elif out_dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"out_dtype {out_dtype}: bfloat16 or float32")
    if k_lens is not None:
        k_lens = k_lens.to(device=device, dtype=torch.int32).contiguous()
    if key_bias is not None:
        key_bias = key_bias.to(device=device, dtype=torch.float32).contiguous()
        cross = False  # (the chunk kernel carries the bias; one pass for a short context)
        if n_distinct is not None:
            raise ValueError("n_distinct carries its own bias: pass one or the other")
    if cross:
        if len(ks) != 1:
            raise ValueError("cross-attention takes one KV segment")
        if dlo is not None or dhi is not None:
            raise ValueError("cross-attention takes no device window bounds")
        nd = -1 if n_distinct is None else int(n_distinct)
        if out is None:
            return ops.cross_attention(q, ks[0], vs[0], k_lens, nd, lo, hi, scale,
                                       out_dtype == torch.float32)
        ops.cross_attention_out(q, ks[0], vs[0], k_lens, nd, lo, hi, scale, out)
        return out
    if out is None:
        return ops.attention(q, ks, vs, lo, hi, k_lens, scale, int(num_splits),
                             out_dtype == torch.float32, dlo, dhi, key_bias)
    ops.attention_out(q, ks, vs, lo, hi, k_lens, scale, int(num_splits), out, dlo, dhi, key_bias)
    return out


def _segments(segments, device):
    """(k list, v list) of bf16 ``[B, L_i, N, D]`` segments on ``device``."""
    if not 1 <= len(segments) <= _lib.MAX_KV_SEGMENTS:
        raise ValueError(f"{len(segments)} KV segments: 1..{_lib.MAX_KV_SEGMENTS} supported")
    ks, vs = [], []
    for k, v in segments:
        _check_4d("k", k, device)
        _check_4d("v", v, device)
        ks.append(_as_bf16_k(k))
        vs.append(_as_bf16(v))
    return ks, vs


def window_from_mask(attn_mask: torch.Tensor, lk: int):
    """(lo, hi) of a KV-window mask as model_fast.py:2538-2545 builds it (bool, True =
    attend, broadcast over batch, heads and queries). Raises for any other mask."""
    if attn_mask.dtype != torch.bool:
        raise ValueError("only boolean KV-window masks are supported")
    m = attn_mask.reshape(-1, attn_mask.shape[-1])
    if attn_mask.shape[-1] != lk or not bool(torch.all(m == m[:1])):
        raise ValueError("attn_mask must be a [.., Lk] KV window shared by every query")
    idx = torch.nonzero(m[0]).flatten()
    if idx.numel() == 0:
        return 0, 0
    lo, hi = int(idx[0]), int(idx[-1]) + 1
    if idx.numel() != hi - lo:
        raise ValueError("attn_mask is not a contiguous KV window")
    return lo, hi


def attention(q, k, v, q_lens=None, k_lens=None, dropout_p=0., softmax_scale=None,
              q_scale=None, causal=False, window_size=(-1, -1), deterministic=False,
              dtype=torch.bfloat16, fa_version=None, attn_mask=None, is_cross_attn=False,
              kv_lo=None, kv_hi=None):
    """attention.py:1082-1143 with the reference's signature and layout.

    Differences from the reference's SDPA fallback, all loud: ``causal=True``,
    ``dropout_p > 0`` and masks that are not a KV window raise. ``kv_lo``/``kv_hi`` take
    precedence over ``attn_mask`` (they carry the same window, model_fast.py:2546-2550); as
    the reference passes them -- one-element tensors on the device (``attn_lo``,
    ``attn_hi``) -- the kernel reads them there and the call never synchronises the host.
    ``q_lens``/``k_lens`` are ignored with the reference's warning (attention.py:1128-1132);
    masked cross-attention is ``cross_attention``. ``q_scale`` and ``softmax_scale`` are
    ignored, as the reference ignores them on every path (attention.py:1082-1143: its kernels
    and its SDPA fallback use 1/sqrt(head_dim), attention.py:378, 439), with a warning; a caller
    that wants another scale, or the folded softmax of a pre-scaled q, calls
    ``attention_segments``. The kernels compute in
    bf16, so ``dtype`` must be ``torch.bfloat16`` (the reference computes in ``dtype``; any
    other value raises). Output: bf16 ``[B, Lq, N, D]``."""
    _check_dtype(dtype)
    if causal:
        raise NotImplementedError("causal masking is not part of this path (the chunked "
                                  "cache carries causality; attention.py:360-365)")
    if dropout_p:
        raise NotImplementedError("dropout is not supported")
    if window_size not in ((-1, -1), [-1, -1]):
        raise NotImplementedError("local window_size is not supported")
    if q_lens is not None or k_lens is not None:
        warnings.warn('Padding mask is disabled when using scaled_dot_product_attention. '
                      'It can have a significant impact on performance.')
    if q_scale is not None:
        warnings.warn("q_scale is ignored, as in the reference's attention() "
                      "(wan/modules/attention.py:1082-1143)")
    if softmax_scale is not None:
        warnings.warn("softmax_scale is ignored, as in the reference's attention(): the scale is "
                      "1/sqrt(head_dim) (wan/modules/attention.py:1082-1143); attention_segments "
                      "takes one")
    lo, hi = kv_lo, kv_hi
    if attn_mask is not None and lo is None and hi is None:
        lo, hi = window_from_mask(attn_mask, k.shape[1])
    on_dev = any(torch.is_tensor(b) and b.device.type != "cpu" for b in (lo, hi))
    out = attention_segments(q, [(k, v)], kv_lo=lo, kv_hi=hi,
                             cross=bool(is_cross_attn) and k.shape[1] <= 4096 and not on_dev)
    return out


flash_attention = attention


def exact_attention(q, k, v, dtype=torch.bfloat16):
    """attention.py:1061-1079: exact attention, streamed (no score matrix)."""
    return attention(q, k, v, dtype=dtype)


def _nmajor_chunk(kc, vc, d):
    """One N-major cache chunk as the reference passes it to its merged path
    (attention.py:1016-1019): K ``[N, D, L]`` (pre-transposed) or ``[N, L, D]`` (told apart as
    there: the last dim is D and the middle one is not), V ``[N, L, D]``; returned as
    ``[1, L, N, D]`` views of the same memory (K d-major in the first case)."""
    if kc.dim() != 3 or vc.dim() != 3:
        raise ValueError("N-major chunks are 3-D: K [N, D, L] or [N, L, D], V [N, L, D]")
    tp_k = int(kc.shape[-1]) == d and int(kc.shape[1]) != d
    k4 = kc.permute(1, 0, 2)[None] if tp_k else kc.permute(2, 0, 1)[None]
    return k4, vc.permute(1, 0, 2)[None]


def exact_attention_chunks(q, k_chunks, v_chunks, dtype=torch.bfloat16):
    """attention.py:1048-1058: attention over the concatenation of KV chunks, read in
    place as segments (no torch.cat, no padding copy). Chunks are ``[B, L_c, N, D]``, or, as
    the reference's merged path takes them, N-major 3-D chunks (K ``[N, D, L]`` or
    ``[N, L, D]``, V ``[N, L, D]``; q ``[1, Lq, N, D]``), read where they lie.
    ``dtype`` must be bf16, as for :func:`attention`."""
    _check_dtype(dtype)
    if len(k_chunks) != len(v_chunks):
        raise ValueError("k_chunks and v_chunks differ in length")
    pairs = list(zip(k_chunks, v_chunks))
    if pairs and pairs[0][0].dim() == 3:
        pairs = [_nmajor_chunk(kc, vc, q.shape[-1]) for kc, vc in pairs]
    return attention_segments(q, pairs)


def cross_attention(q, k, v, k_lens=None, dtype=torch.bfloat16, n_distinct=None):
    """Cross-attention to a short context (kernels/cross_attention.py:17 semantics), with the
    optional per-batch valid length ``k_lens`` masked (the reference attends all rows;
    ``k_lens=None`` reproduces that). ``n_distinct`` selects the exact deduplicated form of
    attention.py:493-554: rows ``n_distinct..`` of k/v are identical (the context's padding)
    and are attended as one key weighted by their count (see ``padding_start``).
    k / v are ``[B, L, N, D]`` or, for batch 1, the reference's N-major cross cache as
    cte_cross_attention_nmajor takes it (attention.py:557-579: K ``[N, D, L]``, V ``[N, L, D]``),
    read in place. ``dtype`` must be bf16, as for :func:`attention`."""
    _check_dtype(dtype)
    if n_distinct is not None and k_lens is not None:
        raise ValueError("dedup reproduces the unmasked attention: pass k_lens or n_distinct")
    if k.dim() == 3 and v.dim() == 3:
        k, v = _nmajor_chunk(k, v, q.shape[-1])
    return attention_segments(q, [(k, v)], k_lens=k_lens, cross=True, n_distinct=n_distinct)


def cross_attention_dedup(q, k, v, bias, kc, dtype=torch.bfloat16):
    """attention.py:532-554 ``cross_attention_dedup``: q ``[1, Lq, N, D]`` against the first
    ``kc`` keys of the cross cache with a per-key additive bias ``[kc]`` (natural log, the
    log-multiplicity of cross_dedup_bias or any other), softmax(q k^T / sqrt(D) + bias) v.
    k / v are ``[1, L, N, D]`` (token-major, or d-major K views) or the reference's N-major
    cache as it is passed there, K ``[N, D, L]`` and V ``[N, L, D]`` (read in place).
    ``dtype`` must be bf16, as for :func:`attention`."""
    _check_dtype(dtype)
    if k.dim() == 3 and v.dim() == 3:   # the reference's N-major cache itself: [N, D, L], [N, L, D]
        k, v = _nmajor_chunk(k, v, q.shape[-1])
    kc = int(kc)
    if bias.numel() != kc:
        raise ValueError(f"bias has {bias.numel()} values, kc = {kc}")
    return attention_segments(q, [(k[:, :kc], v[:, :kc])], key_bias=bias.reshape(kc))


def padding_start(k: torch.Tensor, v: torch.Tensor) -> int:
    """Index of the first of the trailing rows of a cross K/V cache ``[1, L, N, D]`` that equal
    its last row in both K and V (the projected zero padding of the context;
    cross_dedup_bias, attention.py:493-503, counts the same rows); L when there is none.
    One device sync: call it once per context (the cross cache is filled once per
    generation)."""
    if k.shape[0] != 1 or v.shape[0] != 1:
        raise ValueError("padding_start expects batch 1")
    same = ((k[0] == k[0, -1:]).flatten(1).all(dim=1) & (v[0] == v[0, -1:]).flatten(1).all(dim=1))
    L = same.shape[0]
    # length of the trailing run of identical rows
    idx = torch.arange(L, device=k.device)
    last_diff = torch.where(~same, idx, torch.full_like(idx, -1)).max()
    start = int(last_diff.item()) + 1
    return start if start < L else L


def attention_partial(q, segments, *, kv_lo=None, kv_hi=None, softmax_scale=None):
    """cte_partial (attention.py:617-645): unnormalised attention over ``segments``.

    Returns ``(O [B, N, Lq, D] fp32, m [B, N, Lq] fp32, l [B, N, Lq] fp32)`` with
    O = exp(s - m) V, m the row max of the scaled scores and l = sum exp(s - m)
    (m = -inf, l = 0 for rows with no keys)."""
    ops = _lib.ops()
    device = q.device
    _check_4d("q", q, device)
    q = _as_bf16(q)
    ks, vs = _segments(segments, device)
    lo, hi, dlo, dhi = _bounds(kv_lo, kv_hi, device)
    return ops.attention_partial(q, ks, vs, lo, hi,
                                 0.0 if softmax_scale is None else float(softmax_scale), dlo, dhi)


def attention_merge(parts, out: torch.Tensor | None = None) -> torch.Tensor:
    """cte_merge (attention.py:963-990): out = sum_c e^(m_c - M) O_c / sum_c e^(m_c - M) l_c
    over partials ``(O [B, N, Lq, D], m [B, N, Lq], l [B, N, Lq])`` -> bf16 ``[B, Lq, N, D]``."""
    ops = _lib.ops()
    if not 1 <= len(parts) <= 16:
        raise ValueError("1..16 partials")
    _check_parts(parts)
    os_, ms, ls = [p[0] for p in parts], [p[1] for p in parts], [p[2] for p in parts]
    if out is None:
        return ops.attention_merge(os_, ms, ls)
    ops.attention_merge_out(os_, ms, ls, out)
    return out


def _check_parts(parts):
    po0 = parts[0][0]
    B, H, Lq, D = po0.shape
    for o, m, l in parts:
        if o.shape != po0.shape or m.shape != (B, H, Lq) or l.shape != (B, H, Lq):
            raise ValueError("partials differ in shape")
        if not (o.is_contiguous() and m.is_contiguous() and l.is_contiguous()):
            raise ValueError("partials must be contiguous")
        if o.dtype != torch.float32 or m.dtype != torch.float32 or l.dtype != torch.float32:
            raise ValueError("partials must be float32")


def attention_merge_partials(parts):
    """The log-sum-exp merge of partials ``(O, m, l)`` into one partial triple (O relative to
    the merged row max M, m = M, l the merged row sum): the running state of cte_call's chain
    (attention.py:654-694). ``attention_merge`` of the result normalises it."""
    if not 1 <= len(parts) <= 16:
        raise ValueError("1..16 partials")
    _check_parts(parts)
    return _lib.ops().attention_merge_partials([p[0] for p in parts], [p[1] for p in parts],
                                               [p[2] for p in parts])


def attention_chain(q, segments, chain=None, normalize=False, *, kv_lo=None, kv_hi=None,
                    softmax_scale=None, out: torch.Tensor | None = None):
    """cte_call's chain contract (attention.py:654-694): a call over ``segments`` continues the
    online softmax of the earlier calls in ``chain`` (same q, other keys); the call with
    ``normalize=True`` returns the attention over the union of every call's keys, bf16
    ``[B, Lq, N, D]``. Without it the call returns the new chain state.

    The state is one running triple ``(O, m, l)`` as the reference's (O, -max, sum): each call's
    partials (attention_partial) are merged into it by ``attention_merge_partials``, so its size
    does not grow with the number of calls; the normalizing call divides it out."""
    state = chain
    if segments:
        part = attention_partial(q, segments, kv_lo=kv_lo, kv_hi=kv_hi,
                                 softmax_scale=softmax_scale)
        state = part if state is None else attention_merge_partials([state, part])
    if not normalize:
        return state
    if state is None:
        raise ValueError("a chain needs at least one call with keys")
    return attention_merge([state], out=out)


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)


LOG2E = 1.4426950408889634
# Softmax scale for a q that already carries log2(e)/sqrt(d) (``prescaled_q_scale``): then
# scale * log2(e) is exactly 1 in fp32 and the kernel takes its folded softmax, which needs no
# per-score scaling. The pre-scale is the reference's own (model_fast.py:1233, 2666-2676: q
# pre-scaled by 1/sqrt(d) in bf16 by the fused norm + RoPE kernel), with log2(e) folded in too.
PRESCALED_SOFTMAX_SCALE = math.log(2.0)


def prescaled_q_scale(head_dim: int) -> float:
    """The q scale for the fused q/k kernel's output that pairs with
    ``softmax_scale=PRESCALED_SOFTMAX_SCALE``: softmax(q k^T / sqrt(d)) unchanged, up to one bf16
    rounding of the scaled q."""
    return LOG2E / math.sqrt(head_dim)
