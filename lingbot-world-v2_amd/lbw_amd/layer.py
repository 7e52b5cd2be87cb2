"""Wan attention layers on the gfx950 path: the callers of the hot path.

``WanSelfAttention`` mirrors CausalWanSelfAttention.forward (wan/modules/model_fast.py:1687-2594)
for one GPU: q/k/v projections (torch linear, bf16 on hipBLASLt), then ONE fused kernel for
bias + RMSNorm + 3-D RoPE of q and k that also commits the chunk's K and V into their cache
slot (model_fast.py:2398-2409, 2482-2483 write with copy_), then chunk attention over the
cache in place, then the o-projection. ``WanCrossAttention`` mirrors WanCrossAttention.forward
(model_fast.py:2753-2834): the context K/V are projected and normalised once per generation
into a cross cache (2784-2798), later calls only project q.

Numerics follow kernels/qk_post.py: q/k projections without bias in bf16, the bias added in
fp32 inside the norm kernel, one bf16 rounding after the norm and one after RoPE.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .attention import (PRESCALED_SOFTMAX_SCALE, attention_segments, cross_attention,
                        padding_start, prescaled_q_scale)
from .chunked_kv_cache import FlatKVCache, chunk_routing, ordered_chunks
from .fp8 import attention_fp8kv, quantize_kv_fp8
from .qk_post import qk_norm_rope_
from .rope import RopeTables, causal_rope_tables, wan_rope_freqs

__all__ = ["WanSelfAttention", "WanCrossAttention"]


def _no_rope(device, head_dim: int) -> RopeTables:
    """Tables for a zero-token grid: no row is rotated (the cross-attention q/k norm)."""
    c = head_dim // 2
    s1 = c // 3
    return RopeTables(torch.zeros(1, dtype=torch.float32, device=device), 0, 0, 0,
                      c - 2 * s1, s1, 0)


class WanSelfAttention:
    """Self-attention of one Wan block. Weights are bf16 ``[C, C]`` (q, k, v, o), biases and
    RMSNorm gammas bf16 ``[C]``."""

    def __init__(self, wq, bq, wk, bk, wv, bv, wo, bo, gq, gk, heads: int, eps: float = 1e-6,
                 freqs: torch.Tensor | None = None):
        self.C = wq.shape[0]
        self.heads = heads
        self.head_dim = self.C // heads
        self.eps = eps
        self.w_qkv = torch.cat([wq, wk, wv], 0).contiguous()         # [3C, C]
        # the GEMM epilogue adds V's bias (one rounding, as nn.Linear); q's and k's biases are
        # added in fp32 by the fused norm kernel (kernels/qk_post.py), so theirs are zero here
        self.b_qkv = None if bv is None else torch.cat([torch.zeros_like(bv), torch.zeros_like(bv), bv])
        self.bq, self.bk, self.bv = bq, bk, bv
        self.wo, self.bo = wo, bo
        self.gq, self.gk = gq, gk
        self.freqs = wan_rope_freqs(self.head_dim) if freqs is None else freqs

    def _project_norm_rope(self, x, grid, start_frame, k_out, v_out, q_scale=1.0):
        """x [1, L, C] -> q' [L, C] (bf16, times q_scale) and K/V written into k_out / v_out
        ([L, C] views)."""
        L = x.shape[1]
        qkv = F.linear(x[0], self.w_qkv, self.b_qkv)                    # [L, 3C] bf16
        C = self.C
        q_raw, k_raw, v = qkv[:, :C], qkv[:, C:2 * C], qkv[:, 2 * C:]   # row-strided views
        tabs = causal_rope_tables(self.freqs, grid, start_frame, device=x.device)
        q = torch.empty(L, C, dtype=torch.bfloat16, device=x.device)
        qk_norm_rope_(q_raw, k_raw, self.bq, self.bk, self.gq, self.gk, tabs, self.eps,
                      self.heads, q_out=q, k_out=k_out, v=v, v_out=v_out, q_scale=q_scale)
        return q

    def prefill(self, x, grid, start_frame, cache: FlatKVCache, current_start: int = 0):
        """Write the K/V of already generated frames (x [1, L, C]) into the flat cache."""
        L = x.shape[1]
        p = cache.plan(current_start, L)
        cache.apply_roll(p)
        ks, vs = cache.slot(p)
        self._project_norm_rope(x, grid, start_frame, ks[0].view(L, self.C),
                                vs[0].view(L, self.C))
        cache.commit(p)

    def forward(self, x, grid, start_frame, cache: FlatKVCache, current_start: int):
        """model_fast.py:1687-2583 (flat cache): x [1, L, C] bf16 -> [1, L, C] bf16."""
        L = x.shape[1]
        p = cache.plan(current_start, L)
        cache.apply_roll(p)
        ks, vs = cache.slot(p)
        # q pre-scaled by log2(e)/sqrt(d) in the norm kernel: the attention's folded softmax
        q = self._project_norm_rope(x, grid, start_frame, ks[0].view(L, self.C),
                                    vs[0].view(L, self.C), prescaled_q_scale(self.head_dim))
        cache.commit(p)
        o = attention_segments(q.view(1, L, self.heads, self.head_dim), [(cache.k, cache.v)],
                               kv_lo=p.attn_lo, kv_hi=p.attn_hi,
                               softmax_scale=PRESCALED_SOFTMAX_SCALE)
        return F.linear(o.view(1, L, self.C), self.wo, self.bo)

    def forward_chunked(self, x, grid, start_frame, chunks, chunk_index: int):
        """model_fast.py:2374-2420 (chunked cache): the chunk goes to its routed slot and the
        attention reads (leading..., destination) as segments, without concatenation."""
        L = x.shape[1]
        n = len(chunks["k"])
        dest, leading = chunk_routing(chunk_index, n)
        kd, vd = chunks["k"][dest], chunks["v"][dest]
        if kd.shape[1] != L:
            raise ValueError(f"chunk buffers hold {kd.shape[1]} tokens, the chunk has {L}")
        q = self._project_norm_rope(x, grid, start_frame, kd[0].view(L, self.C),
                                    vd[0].view(L, self.C), prescaled_q_scale(self.head_dim))
        kk, vv = ordered_chunks(chunks, dest, leading)
        o = attention_segments(q.view(1, L, self.heads, self.head_dim), list(zip(kk, vv)),
                               softmax_scale=PRESCALED_SOFTMAX_SCALE)
        return F.linear(o.view(1, L, self.C), self.wo, self.bo)


    def forward_chunked_fp8(self, x, grid, start_frame, chunks, chunk_index: int):
        """forward_chunked over an fp8-e4m3 chunked cache (allocate_self_kv_chunks_fp8): the
        fused kernel commits the chunk's roped K and V in bf16 to the staging pair, the
        quantiser writes codes + block scales into the routed slot (a second pass: the block
        scales need the amax of 64 tokens x 128 features per head, which the row-parallel q/k
        kernel does not see at once), and the attention reads the fp8 slots with bf16 q."""
        L = x.shape[1]
        n = len(chunks["k"])
        dest, leading = chunk_routing(chunk_index, n)
        kd, vd = chunks["k"][dest], chunks["v"][dest]
        if kd.codes.shape[1] != L:
            raise ValueError(f"chunk slots hold {kd.codes.shape[1]} tokens, the chunk has {L}")
        sk, sv = chunks["stage"]["k"], chunks["stage"]["v"]
        q = self._project_norm_rope(x, grid, start_frame, sk[0].view(L, self.C),
                                    sv[0].view(L, self.C))
        quantize_kv_fp8(sk, out=kd)
        quantize_kv_fp8(sv, out=vd)
        kk, vv = ordered_chunks(chunks, dest, leading)
        o = attention_fp8kv(q.view(1, L, self.heads, self.head_dim), list(zip(kk, vv)))
        return F.linear(o.view(1, L, self.C), self.wo, self.bo)


class WanCrossAttention:
    """Cross-attention of one Wan block to the text context, with the per-generation cache."""

    def __init__(self, wq, bq, wk, bk, wv, bv, wo, bo, gq, gk, heads: int, eps: float = 1e-6,
                 dedup: bool = False):
        self.C = wq.shape[0]
        self.heads = heads
        self.head_dim = self.C // heads
        self.eps = eps
        self.wq, self.bq, self.wk, self.bk, self.wv, self.bv = wq, bq, wk, bk, wv, bv
        self.wo, self.bo, self.gq, self.gk = wo, bo, gq, gk
        self.dedup = dedup      # attention.py:516-554: identical padding rows as one weighted key
        self.cache = None
        self.n_distinct = None

    def _norm(self, x_raw, bias, gamma):
        """RMSNorm of projected rows [L, C] (no rotation) through the fused kernel."""
        L = x_raw.shape[0]
        out = torch.empty(L, self.C, dtype=torch.bfloat16, device=x_raw.device)
        qk_norm_rope_(x_raw, None, bias, None, gamma, None, _no_rope(x_raw.device, self.head_dim),
                      self.eps, self.heads, q_out=out, k_out=None)
        return out

    def set_context(self, context):
        """model_fast.py:2784-2798: context [1, Lc, C] -> cached K (normalised) and V."""
        ctx = context[0]
        k = self._norm(F.linear(ctx, self.wk).contiguous(), self.bk, self.gk)
        v = F.linear(ctx, self.wv, self.bv)
        Lc = ctx.shape[0]
        self.cache = (k.view(1, Lc, self.heads, self.head_dim),
                      v.contiguous().view(1, Lc, self.heads, self.head_dim))
        self.n_distinct = padding_start(*self.cache) if self.dedup else None

    def forward(self, x, context=None, k_lens=None):
        """x [1, L, C] -> [1, L, C]; ``k_lens`` (int32 [1] on the device) masks the context's
        zero padding (the reference attends all rows: leave it None to match)."""
        if context is not None or self.cache is None:
            self.set_context(context)
        L = x.shape[1]
        q = self._norm(F.linear(x[0], self.wq).contiguous(), self.bq, self.gq)
        k, v = self.cache
        o = cross_attention(q.view(1, L, self.heads, self.head_dim), k, v, k_lens=k_lens,
                            n_distinct=self.n_distinct if k_lens is None else None)
        return F.linear(o.view(1, L, self.C), self.wo, self.bo)

