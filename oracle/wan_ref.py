"""fp32 CPU restatement of the reference's causal-chunk attention path (test infrastructure).

Every function cites the reference file:line it restates. Layout convention everywhere:
tokens-major ``[B, L, H, D]`` (the layout ``attention()`` receives, attention.py:1082-1100).
"""
from __future__ import annotations

import math

import numpy as np
import torch

__all__ = [
    "MAX_LATENT_FRAMES", "rope_params", "wan_rope_freqs", "rope_axis_split",
    "causal_rope_grids", "rope_axis_tables", "expand_axis_tables", "rope_apply_rotation",
    "rms_norm_module", "qk_post_norm_rope", "qk_post_norm_rope_t", "qk_post_ss", "attention_ref", "sdpa_ref",
    "attention_brute_f64", "merge_partials", "window_mask", "num_chunks", "chunk_routing",
    "ordered_chunks", "flat_cache_write_plan", "fp8_e4m3_encode", "fp8_e4m3_decode",
    "quantize_kv_fp8", "dequantize_kv_fp8", "self_attention_layer_ref", "cross_kv_ref",
    "cross_dedup_bias", "attention_key_bias_ref", "windowed_layer_sequence_ref",
]

# wan/modules/model.py:44 -- rows of the RoPE frequency tables (frame axis bound).
MAX_LATENT_FRAMES = 2880


# ----------------------------------------------------------------------------- RoPE
def rope_params(max_seq_len: int, dim: int, theta: float = 10000.0) -> torch.Tensor:
    """model.py:47-53: outer(arange(n), 1 / theta^(arange(0, dim, 2) / dim)) in fp32."""
    assert dim % 2 == 0
    return torch.outer(
        torch.arange(max_seq_len).float(),
        1.0 / torch.pow(theta, torch.arange(0, dim, 2).float().div(dim)))


def wan_rope_freqs(head_dim: int = 128, max_frames: int = MAX_LATENT_FRAMES) -> torch.Tensor:
    """model.py:480-487: [max_frames, head_dim/2] = cat(t: d-4(d//6), h: 2(d//6), w: 2(d//6))."""
    d = head_dim
    assert d % 2 == 0
    return torch.cat([
        rope_params(max_frames, d - 4 * (d // 6)),
        rope_params(max_frames, 2 * (d // 6)),
        rope_params(max_frames, 2 * (d // 6)),
    ], dim=1)


def rope_axis_split(c: int):
    """model_fast.py:889-891: (c - 2(c//3), c//3, c//3) columns for (frame, height, width)."""
    return c - 2 * (c // 3), c // 3, c // 3


def causal_rope_grids(freqs: torch.Tensor, f: int, h: int, w: int, start_frame: int = 0,
                      dtype=torch.float32):
    """model_fast.py:878-931 (no width shard): cos/sin ``[f*h*w, c]`` in frame-major token
    order, angles = cat(t[start_frame + fi], h[hi], w[wi]) computed in fp32 on the CPU."""
    c = freqs.size(1)
    s0, s1, _ = rope_axis_split(c)
    fs = freqs.float().split([s0, s1, s1], dim=1)
    ang = torch.cat([
        fs[0][start_frame:start_frame + f].view(f, 1, 1, -1).expand(f, h, w, -1),
        fs[1][:h].view(1, h, 1, -1).expand(f, h, w, -1),
        fs[2][:w].view(1, 1, w, -1).expand(f, h, w, -1),
    ], dim=-1).reshape(f * h * w, c)
    return torch.cos(ang).to(dtype), torch.sin(ang).to(dtype)


def rope_axis_tables(freqs: torch.Tensor, f: int, h: int, w: int, start_frame: int = 0):
    """Factorised form of causal_rope_grids: the per-axis cos/sin tables
    ``(cos_t [f, s0], sin_t, cos_h [h, s1], sin_h, cos_w [w, s1], sin_w)``.

    The grid of model_fast.py:893-928 is a column concatenation of per-axis angle rows,
    and cos/sin act elementwise, so the grid row of token (fi, hi, wi) equals
    cat(cos_t[fi], cos_h[hi], cos_w[wi]) bit for bit (expand_axis_tables)."""
    c = freqs.size(1)
    s0, s1, _ = rope_axis_split(c)
    fs = freqs.float().split([s0, s1, s1], dim=1)
    at = fs[0][start_frame:start_frame + f]
    ah, aw = fs[1][:h], fs[2][:w]
    return (torch.cos(at), torch.sin(at), torch.cos(ah), torch.sin(ah),
            torch.cos(aw), torch.sin(aw))


def expand_axis_tables(tables, f: int, h: int, w: int):
    """Per-axis tables -> full ``[f*h*w, c]`` cos/sin grids (frame-major token order)."""
    ct, st, ch, sh, cw, sw = tables

    def grid(a, b, cc):
        return torch.cat([
            a.view(f, 1, 1, -1).expand(f, h, w, -1),
            b.view(1, h, 1, -1).expand(f, h, w, -1),
            cc.view(1, 1, w, -1).expand(f, h, w, -1)], dim=-1).reshape(f * h * w, -1)
    return grid(ct, ch, cw), grid(st, sh, sw)


def rope_apply_rotation(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                        compute_dtype=torch.float32) -> torch.Tensor:
    """model_fast.py:933-979 for one sample: x ``[L, H, D]``, cos/sin ``[S, D/2]`` (S <= L).

    Interleaved pairs (x[2j], x[2j+1]) -> (re*c - im*s, re*s + im*c) in ``compute_dtype``;
    rows past S are passed through. Returns ``compute_dtype`` (caller casts)."""
    L, H, D = x.shape
    c = D // 2
    S = cos.shape[0]
    xs = x[:S].to(compute_dtype).reshape(S, H, c, 2)
    re, im = xs[..., 0], xs[..., 1]
    cg = cos.to(compute_dtype).view(S, 1, c)
    sg = sin.to(compute_dtype).view(S, 1, c)
    out = torch.stack([re * cg - im * sg, re * sg + im * cg], dim=-1).reshape(S, H, D)
    return torch.cat([out, x[S:].to(compute_dtype)], dim=0)


# ----------------------------------------------------------------------------- RMSNorm
def rms_norm_module(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """model.py:126-142 ``WanRMSNorm.forward``: ``_norm(x.float()).type_as(x) * weight``
    with ``_norm = x * rsqrt(mean(x^2, -1) + eps)``."""
    xf = x.float()
    n = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return n.type_as(x) * weight


def qk_post_ss(x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    """kernels/qk_post.py:49-73 (``_qk_ss_body``): per-row sum over features of (x + b)^2, fp32."""
    y = x.float() + (bias.float() if bias is not None else 0.0)
    return (y * y).sum(-1)


def qk_post_norm_rope(x: torch.Tensor, bias: torch.Tensor | None, weight: torch.Tensor,
                      cos: torch.Tensor, sin: torch.Tensor, eps: float = 1e-6,
                      heads: int | None = None, out_scale: float = 1.0) -> torch.Tensor:
    """kernels/qk_post.py:88-141 (``_qk_norm_rope_body``), the rounding sequence of the fused
    kernel this path replaces, on one tensor ``x [L, C]``:

        y  = x + b                                   (fp32)
        r  = rsqrt(sum(y^2) / C + eps)               (fp32, full-row sum)
        t  = bf16(y * r) * w                         (one bf16 rounding, x gamma in fp32)
        RoPE on interleaved pairs with cos/sin [L', D/2] fp32, the output scale s folded
        into them first (fp32 cos*s, sin*s); rows >= L' are t*s
        out = bf16(that)

    ``out_scale`` restates the ``_t`` variants' pre-scale of q by 1/sqrt(D), which rides on
    q's cos/sin (qk_post.py:259-265, 359-365). Returns bf16 ``[L, C]``."""
    L, C = x.shape
    y = x.float() + (bias.float() if bias is not None else 0.0)
    ss = (y * y).sum(-1)
    r = torch.rsqrt(ss * (1.0 / C) + eps)
    t = (y * r[:, None]).to(torch.bfloat16).float() * weight.float().view(1, C)
    D = 2 * cos.shape[1]
    H = heads if heads is not None else C // D
    S = cos.shape[0]
    s = torch.tensor(out_scale, dtype=torch.float32)
    out = rope_apply_rotation(t.view(L, H, D), cos.float() * s, sin.float() * s, torch.float32)
    out = out.reshape(L, C)
    if out_scale != 1.0:
        out = torch.cat([out[:S], out[S:] * s])
    return out.to(torch.bfloat16)


def qk_post_norm_rope_t(x: torch.Tensor, bias: torch.Tensor | None, weight: torch.Tensor,
                        cos: torch.Tensor, sin: torch.Tensor, eps: float = 1e-6,
                        heads: int | None = None, out_scale: float = 1.0) -> torch.Tensor:
    """kernels/qk_post.py:228-306 (``_qk_norm_rope_t_body``) and 331-402 (``_x_norm_rope_t3``):
    the same values as :func:`qk_post_norm_rope` written head-major, d-major: bf16
    ``[H, D, L]`` with element ``(h, d, l)`` = row ``l``'s feature ``h * D + d``."""
    L, C = x.shape
    D = 2 * cos.shape[1]
    H = heads if heads is not None else C // D
    rows = qk_post_norm_rope(x, bias, weight, cos, sin, eps, H, out_scale)
    return rows.view(L, H, D).permute(1, 2, 0).contiguous()


# ----------------------------------------------------------------------------- attention
def window_mask(kv_size: int, attn_lo: int, attn_hi: int) -> torch.Tensor:
    """model_fast.py:2538-2545: bool ``[1, 1, 1, kv_size]``, True on positions in [lo, hi)."""
    pos = torch.arange(kv_size)
    return ((pos >= attn_lo) & (pos < attn_hi)).view(1, 1, 1, kv_size)


def _key_range(lk: int, kv_lo, kv_hi, k_len):
    lo = 0 if kv_lo is None else max(0, int(kv_lo))
    hi = lk if kv_hi is None else min(lk, int(kv_hi))
    if k_len is not None:
        hi = min(hi, int(k_len))
    return lo, max(lo, hi)


def attention_ref(q, k, v, *, kv_lo=None, kv_hi=None, k_lens=None, softmax_scale=None,
                  q_block: int = 1024, return_partials: bool = False):
    """Exact attention in fp32, the SDPA fallback of attention() (attention.py:1127-1143)
    with the KV window of model_fast.py:2538-2545 and, for cross-attention, a per-batch
    valid key count ``k_lens`` (the masked mode; ``None`` attends every key as the
    reference's SDPA path does, attention.py:1128-1132).

    q ``[B, Lq, H, D]``, k/v ``[B, Lk, H, D]`` (any float dtype, upcast to fp32).
    Keys attended for batch b: ``[lo, hi)`` with lo = kv_lo, hi = min(kv_hi, k_lens[b]).
    A row with no keys returns 0 (what torch's SDPA returns for a fully masked row).

    Looped per (batch, head, query block): no ``[H, Lq, Lk]`` tensor is materialised.
    With ``return_partials`` also returns the cte_partial contract (attention.py:617-645):
    ``O_unnorm [B, H, Lq, D]`` = exp(s - m) @ V, ``m [B, H, Lq]`` = row max of the scaled
    scores, ``l [B, H, Lq]`` = row sum of exp(s - m)."""
    B, Lq, H, D = q.shape
    Lk = k.shape[1]
    scale = (1.0 / math.sqrt(D)) if softmax_scale is None else float(softmax_scale)
    Dv = v.shape[-1]
    out = torch.zeros(B, Lq, H, Dv, dtype=torch.float32)
    if return_partials:
        po = torch.zeros(B, H, Lq, Dv)
        pm = torch.full((B, H, Lq), float("-inf"))
        pl = torch.zeros(B, H, Lq)
    for b in range(B):
        kl = None if k_lens is None else int(k_lens[b])
        lo, hi = _key_range(Lk, kv_lo, kv_hi, kl)
        if hi <= lo:
            continue
        for hh in range(H):
            Kh = k[b, lo:hi, hh].float()
            Vh = v[b, lo:hi, hh].float()
            for q0 in range(0, Lq, q_block):
                Qb = q[b, q0:q0 + q_block, hh].float()
                s = (Qb @ Kh.T) * scale
                m = s.max(dim=-1, keepdim=True).values
                p = torch.exp(s - m)
                l = p.sum(dim=-1, keepdim=True)
                o = p @ Vh
                out[b, q0:q0 + q_block, hh] = o / l
                if return_partials:
                    po[b, hh, q0:q0 + q_block] = o
                    pm[b, hh, q0:q0 + q_block] = m[:, 0]
                    pl[b, hh, q0:q0 + q_block] = l[:, 0]
    if return_partials:
        return out, (po, pm, pl)
    return out


def sdpa_ref(q, k, v, attn_mask=None):
    """attention.py:1127-1143 with ``dtype=torch.float32``: transpose to [B, H, L, D],
    ``F.scaled_dot_product_attention``, transpose back. For small shapes only (the
    library materialises the scores)."""
    qt = q.transpose(1, 2).float()
    kt = k.transpose(1, 2).float()
    vt = v.transpose(1, 2).float()
    o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=attn_mask)
    return o.transpose(1, 2).contiguous()


def attention_brute_f64(q, k, v, lo: int = 0, hi: int | None = None, scale=None) -> np.ndarray:
    """Textbook softmax(QK^T * scale)V in float64 numpy with explicit loops over heads and
    queries: the brute-force pin for tiny shapes."""
    qn = q.double().numpy()
    kn = k.double().numpy()
    vn = v.double().numpy()
    B, Lq, H, D = qn.shape
    hi = kn.shape[1] if hi is None else hi
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    out = np.zeros((B, Lq, H, D))
    for b in range(B):
        for h in range(H):
            for i in range(Lq):
                s = np.array([np.dot(qn[b, i, h], kn[b, j, h]) * sc for j in range(lo, hi)])
                if s.size == 0:
                    continue
                w = np.exp(s - s.max())
                w /= w.sum()
                out[b, i, h] = (w[:, None] * vn[b, lo:hi, h]).sum(0)
    return out


def merge_partials(parts):
    """attention.py:963-990 (``cte_merge``): partials ``(O [B,H,Lq,D], m [B,H,Lq],
    l [B,H,Lq])`` over disjoint key sets -> ``[B, Lq, H, D]`` fp32:

        M = max_c m_c,  w_c = exp(m_c - M),  out = sum_c w_c O_c / sum_c w_c l_c
    """
    outs = [p[0].float() for p in parts]
    maxs = [p[1].float() for p in parts]
    sums = [p[2].float() for p in parts]
    if len(outs) == 1:
        lam = [1.0 / sums[0]]
    else:
        m_all = maxs[0]
        for m in maxs[1:]:
            m_all = torch.maximum(m_all, m)
        w = [torch.exp(m - m_all) for m in maxs]
        den = w[0] * sums[0]
        for wc, sc in zip(w[1:], sums[1:]):
            den = den + wc * sc
        inv = 1.0 / den
        lam = [wc * inv for wc in w]
    out = lam[0].unsqueeze(-1) * outs[0]
    for l_, o in zip(lam[1:], outs[1:]):
        out = out + l_.unsqueeze(-1) * o
    return out.permute(0, 2, 1, 3).contiguous()


# ----------------------------------------------------------------------------- KV caches
def num_chunks(local_attn_size, chunk_size) -> int:
    """chunked_kv_cache.py:36-44: window // chunk (latent frames); 0 for a global cache."""
    if local_attn_size is None or local_attn_size < 0:
        return 0
    return max(1, int(local_attn_size) // max(1, int(chunk_size)))


def chunk_routing(chunk_index: int, n_chunks: int):
    """chunked_kv_cache.py:47-76: ``(destination, leading)`` for the write about to happen.
    Chunk 0 is the pinned sink; slots 1..n-1 rotate round-robin; the destination is last
    in the attention order."""
    i = int(chunk_index)
    if n_chunks <= 1:
        return 0, ()
    dest = 0 if i == 0 else 1 + (i - 1) % (n_chunks - 1)
    written = min(i, n_chunks)
    return dest, tuple(j for j in range(written) if j != dest)


def ordered_chunks(chunks, destination, leading):
    """chunked_kv_cache.py:172-177: buffers in ``(leading..., destination)`` order."""
    return tuple(chunks[i] for i in (*leading, destination))


def flat_cache_write_plan(kv_cache_size: int, global_end: int, local_end: int,
                          current_start: int, num_new: int, sink_tokens: int,
                          max_attention_size: int, local_attn_size: int = 0):
    """model_fast.py:2436-2545, the eager branches of the flat (windowed) cache write.

    Returns ``dict(roll=(dst, src, len) or None, write=(start, end), global_end, local_end,
    attn_lo, attn_hi)``: the roll-with-sink eviction (``cache[dst:dst+len] =
    cache[src:src+len]``), the slot the new K/V go to, the updated indices and the
    attention window ``[attn_lo, attn_hi)``. ``local_attn_size == -1`` is the global cache
    fast path (write at [current_start, current_end))."""
    current_end = current_start + num_new
    roll = None
    if local_attn_size == -1:
        ls, le = current_start, current_end
    elif current_end > global_end and num_new + local_end > kv_cache_size:
        evicted = num_new + local_end - kv_cache_size
        rolled = local_end - evicted - sink_tokens
        roll = (sink_tokens, sink_tokens + evicted, rolled)
        le = local_end + current_end - global_end - evicted
        ls = le - num_new
    else:
        le = local_end + current_end - global_end
        ls = le - num_new
    attn_hi = le
    attn_lo = max(attn_hi - max_attention_size, 0)
    return dict(roll=roll, write=(ls, le), global_end=current_end, local_end=le,
                attn_lo=attn_lo, attn_hi=attn_hi)


# ----------------------------------------------------------------------------- fp8 KV
FP8_E4M3_MAX = 448.0


def fp8_e4m3_encode(x: torch.Tensor) -> torch.Tensor:
    """fp32 -> OCP e4m3fn codes (uint8), round to nearest even; the library cast
    ``torch.float8_e4m3fn`` (finite inputs within +-448 stay finite)."""
    return x.float().to(torch.float8_e4m3fn).view(torch.uint8)


def fp8_e4m3_decode(codes: torch.Tensor) -> torch.Tensor:
    """OCP e4m3fn decode written from the format definition (1 sign, 4 exponent bits with
    bias 7, 3 mantissa bits, no infinities, S.1111.111 = NaN)."""
    c = codes.to(torch.int64)
    s = torch.where((c >> 7) & 1 == 1, -1.0, 1.0).double()
    e = (c >> 3) & 0xF
    m = (c & 7).double()
    val = torch.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * torch.pow(2.0, (e - 7).double()))
    val = torch.where((e == 15) & (c & 7 == 7), torch.tensor(float("nan"), dtype=torch.float64), val)
    return (s * val).float()


def quantize_kv_fp8(x: torch.Tensor, block: int = 64):
    """fp8-e4m3 KV-cache quantiser (no reference counterpart; defined here).

    x ``[B, L, H, D]`` -> ``(codes uint8 [B, L, H, D], scales fp32 [B, H, ceil(L/block)])``.
    Per (batch, head, block of ``block`` tokens by absolute index within the buffer):

        amax  = max |x| over the block's tokens and all D   (fp32)
        scale = the smallest power of two 2^k >= amax / 448 (k >= -126), or 1 when amax == 0
        inv   = 1 / scale = 2^-k                            (exact)
        code  = e4m3fn_rne(x * inv)                         (exact multiply, then RNE)

    The scales are fp32 powers of two, so the block's largest magnitude maps into (224, 448]
    and a code times its scale is exact in bf16 and fp32 alike.
    """
    B, L, H, D = x.shape
    nb = (L + block - 1) // block
    xf = x.float()
    pad = nb * block - L
    xp = torch.cat([xf, torch.zeros(B, pad, H, D)], 1) if pad else xf
    amax = xp.abs().view(B, nb, block, H, D).amax(dim=(2, 4)).permute(0, 2, 1).contiguous()
    # amax = m 2^e with m in [1, 2) (frexp: mant = m / 2 in [0.5, 1), ex = e + 1):
    # m 2^(e - k) <= 1.75 * 2^8 holds from k = e - 8 on when m <= 1.75, else from k = e - 7
    mant, ex = torch.frexp(amax)
    k = torch.where(mant <= 0.875, ex - 9, ex - 8).clamp(min=-126)
    scale = torch.where(amax > 0, torch.ldexp(torch.ones_like(amax), k.float()), torch.ones_like(amax))
    inv = torch.tensor(1.0, dtype=torch.float32) / scale                    # [B, H, nb]
    inv_tok = inv.permute(0, 2, 1).repeat_interleave(block, dim=1)[:, :L]   # [B, L, H]
    codes = fp8_e4m3_encode(xf * inv_tok.unsqueeze(-1))
    return codes, scale


def dequantize_kv_fp8(codes: torch.Tensor, scales: torch.Tensor, block: int = 64):
    """codes ``[B, L, H, D]`` x scales ``[B, H, nb]`` -> fp32 ``[B, L, H, D]``."""
    B, L, H, D = codes.shape
    s_tok = scales.permute(0, 2, 1).repeat_interleave(block, dim=1)[:, :L]
    return fp8_e4m3_decode(codes) * s_tok.unsqueeze(-1)


# ----------------------------------------------------------------------------- layers
def self_attention_layer_ref(x, x_cache, wq, bq, wk, bk, wv, bv, wo, bo, gq, gk, *,
                             heads: int, grid, cache_grid, start_frame: int,
                             cache_start_frame: int = 0, eps: float = 1e-6,
                             freqs=None):
    """One Wan self-attention layer over a KV cache, fp32 on the CPU (model.py:158-212 with
    the causal grid of model_fast.py:1687-1906 and the flat-cache attention of 2436-2583):

      cached frames: k_c = RoPE(RMSNorm(x_cache Wk + bk)), v_c = x_cache Wv + bv at
                     ``cache_start_frame``;
      chunk:         q, k, v likewise at ``start_frame``;
      out = Wo attention(q, [k_c; k], [v_c; v]) + bo.

    x ``[1, L, C]``, x_cache ``[1, Lc, C]``; grid / cache_grid are (f, h, w). Everything in
    fp32 (the RMSNorm's type_as is then the identity)."""
    C = x.shape[-1]
    D = C // heads
    freqs = wan_rope_freqs(D) if freqs is None else freqs

    def proj(t, w, b):
        return t.float() @ w.float().T + b.float()

    def qk(t, w, b, g, grd, sf):
        y = rms_norm_module(proj(t, w, b), g.float(), eps)[0]
        cos, sin = causal_rope_grids(freqs, *grd, start_frame=sf)
        return rope_apply_rotation(y.view(-1, heads, D), cos, sin)

    q = qk(x, wq, bq, gq, grid, start_frame)
    k = qk(x, wk, bk, gk, grid, start_frame)
    v = proj(x, wv, bv)[0].view(-1, heads, D)
    kc = qk(x_cache, wk, bk, gk, cache_grid, cache_start_frame)
    vc = proj(x_cache, wv, bv)[0].view(-1, heads, D)
    kk = torch.cat([kc, k], 0)[None]
    vv = torch.cat([vc, v], 0)[None]
    o = attention_ref(q[None], kk, vv)
    return o.reshape(1, -1, C) @ wo.float().T + bo.float()


def windowed_layer_sequence_ref(xs, wq, bq, wk, bk, wv, bv, wo, bo, gq, gk, *, heads: int,
                                frame_hw, kv_cache_size: int, sink_tokens: int,
                                max_attention_size: int, eps: float = 1e-6, freqs=None):
    """A Wan self-attention layer run over consecutive one-frame chunks ``xs`` (each
    ``[1, h*w, C]``, chunk i at latent frame i) with the windowed flat KV cache of
    model_fast.py:2436-2583, fp32 on the CPU: per chunk, q/k/v as in
    :func:`self_attention_layer_ref` at start frame i; :func:`flat_cache_write_plan` gives the
    eviction roll (sink kept, the rest shifted left), the slot and the attention window
    ``[attn_lo, attn_hi)``; out_i = Wo attention(q_i, K[lo:hi], V[lo:hi]) + bo.
    Returns the list of outputs ``[1, h*w, C]``."""
    C = xs[0].shape[-1]
    D = C // heads
    freqs = wan_rope_freqs(D) if freqs is None else freqs
    h, w = frame_hw

    def proj(t, wt, b):
        return t.float() @ wt.float().T + b.float()

    def qk(t, wt, b, g, sf):
        y = rms_norm_module(proj(t, wt, b), g.float(), eps)[0]
        cos, sin = causal_rope_grids(freqs, 1, h, w, start_frame=sf)
        return rope_apply_rotation(y.view(-1, heads, D), cos, sin)

    kc = torch.zeros(kv_cache_size, heads, D)
    vc = torch.zeros(kv_cache_size, heads, D)
    g_end = l_end = 0
    outs = []
    for i, x in enumerate(xs):
        n = x.shape[1]
        plan = flat_cache_write_plan(kv_cache_size, g_end, l_end, i * n, n, sink_tokens,
                                     max_attention_size)
        if plan["roll"] is not None:
            dst, src, ln = plan["roll"]
            if ln > 0:
                kc[dst:dst + ln] = kc[src:src + ln].clone()
                vc[dst:dst + ln] = vc[src:src + ln].clone()
        s0, e0 = plan["write"]
        kc[s0:e0] = qk(x, wk, bk, gk, i)
        vc[s0:e0] = proj(x, wv, bv)[0].view(-1, heads, D)
        g_end, l_end = plan["global_end"], plan["local_end"]
        q = qk(x, wq, bq, gq, i)
        lo, hi = plan["attn_lo"], plan["attn_hi"]
        o = attention_ref(q[None], kc[None, lo:hi], vc[None, lo:hi])
        outs.append(o.reshape(1, -1, C) @ wo.float().T + bo.float())
    return outs


def cross_dedup_bias(k, v, kc: int):
    """attention.py:493-503 ``cross_dedup_bias``: over the first kc rows of K / V ``[L, n, d]``,
    log(m / r) on the r rows of the slice that equal the last row in both K and V (m such rows
    in all), 0 elsewhere (fp32 ``[kc]``)."""
    same = (k == k[-1:]).flatten(1).all(dim=1) & (v == v[-1:]).flatten(1).all(dim=1)
    s = same[:kc]
    m, r = same.sum().float(), s.sum().float()
    return torch.where(s, torch.log(m / r), torch.zeros((), dtype=torch.float32))


def attention_key_bias_ref(q, k, v, bias, softmax_scale=None):
    """softmax(scale q k^T + bias) v with a per-key additive bias (natural-log units), fp32,
    q ``[B, Lq, H, D]``, k/v ``[B, Lk, H, D]``, bias ``[Lk]`` (attention.py:546-554)."""
    D = q.shape[-1]
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(D)
    qh = q.float().permute(0, 2, 1, 3)
    kh = k.float().permute(0, 2, 3, 1)
    vh = v.float().permute(0, 2, 1, 3)
    p = torch.softmax(torch.matmul(qh, kh) * scale + bias.float(), dim=-1)
    return torch.matmul(p, vh).permute(0, 2, 1, 3)


def cross_kv_ref(context, wk, bk, wv, bv, gk, heads: int, eps: float = 1e-6):
    """model_fast.py:2784-2798 (first call per generation): K = RMSNorm(ctx Wk + bk),
    V = ctx Wv + bv, fp32, ``[1, Lc, H, D]`` each."""
    C = wk.shape[0]
    D = C // heads
    k = rms_norm_module(context.float() @ wk.float().T + bk.float(), gk.float(), eps)
    v = context.float() @ wv.float().T + bv.float()
    return k.view(1, -1, heads, D), v.view(1, -1, heads, D)
