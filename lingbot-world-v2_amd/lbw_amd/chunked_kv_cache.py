"""KV-cache containers and write planning for the causal-chunk attention path (host side).

Mirrors wan/modules/chunked_kv_cache.py (chunked cache: N independent per-chunk buffers, chunk 0
the pinned sink, the rest rotating round-robin) and the flat windowed cache of
wan/modules/model_fast.py:2436-2545 (one [B, kv_size, N, D] buffer written at a moving offset,
rolled with a sink when full, attended through a [lo, hi) window). The attention kernels read
either layout in place: a chunk list is a list of KV segments, a flat cache is one segment
plus the window.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

__all__ = ["num_chunks", "chunk_routing", "allocate_self_kv_chunks",
           "allocate_self_kv_chunks_fp8", "ordered_chunks",
           "ordered_chunks_by_block", "chunk_bytes", "FlatWritePlan", "plan_flat_write",
           "FlatKVCache"]


def num_chunks(local_attn_size, chunk_size) -> int:
    """chunked_kv_cache.py:36-44: window // chunk in latent frames; 0 for a global cache."""
    if local_attn_size is None or local_attn_size < 0:
        return 0
    return max(1, int(local_attn_size) // max(1, int(chunk_size)))


def chunk_routing(chunk_index: int, n_chunks: int):
    """chunked_kv_cache.py:47-76: ``(destination, leading)`` for the chunk about to be
    written. Slot 0 is the sink (written once, by chunk 0); later chunks rotate over slots
    1..n-1; ``leading`` lists the other slots written so far, the destination goes last in the
    attention order."""
    i = int(chunk_index)
    if n_chunks <= 1:
        return 0, ()
    if i == 0:
        dest = 0
    else:
        dest = 1 + (i - 1) % (n_chunks - 1)
    written = i if i < n_chunks else n_chunks
    return dest, tuple(s for s in range(written) if s != dest)


def allocate_self_kv_chunks(num_layers, batch, chunk_tokens, heads, head_dim, n_chunks,
                            dtype=torch.bfloat16, device="cuda"):
    """chunked_kv_cache.py:79-169 (token-major layout): per layer ``n_chunks`` independent
    zero-filled K and V buffers ``[B, chunk_tokens, N, D]`` -> ``[{"k": [...], "v": [...]}]``.
    fp8 caches use the same shapes with uint8 codes plus scales (lbw_amd.fp8)."""
    cache = []
    for _ in range(num_layers):
        ks = [torch.zeros(batch, chunk_tokens, heads, head_dim, dtype=dtype, device=device)
              for _ in range(n_chunks)]
        vs = [torch.zeros(batch, chunk_tokens, heads, head_dim, dtype=dtype, device=device)
              for _ in range(n_chunks)]
        cache.append({"k": ks, "v": vs})
    return cache


def allocate_self_kv_chunks_fp8(num_layers, batch, chunk_tokens, heads, head_dim, n_chunks,
                                device="cuda"):
    """fp8-e4m3 variant of :func:`allocate_self_kv_chunks` (no reference counterpart): per
    layer ``n_chunks`` K and V slots of uint8 codes ``[B, chunk_tokens, N, D]`` with fp32
    scales ``[B, N, ceil(chunk_tokens / 64)]`` (``lbw_amd.fp8.Fp8KV``; an all-zero slot has
    codes 0 and scales 1), plus one bf16 staging pair ``[B, chunk_tokens, N, D]`` shared by
    the layers: the fused q/k kernel commits the chunk's roped K and V there and the quantiser
    turns them into the destination slot. Each slot is its own KV segment, so scale blocks
    start at the slot's first token and a 64-token block never straddles two chunks."""
    from .fp8 import BLOCK, Fp8KV
    nblk = (chunk_tokens + BLOCK - 1) // BLOCK

    def slot():
        return Fp8KV(torch.zeros(batch, chunk_tokens, heads, head_dim, dtype=torch.uint8,
                                 device=device),
                     torch.ones(batch, heads, nblk, dtype=torch.float32, device=device))

    stage = {"k": torch.zeros(batch, chunk_tokens, heads, head_dim, dtype=torch.bfloat16,
                              device=device),
             "v": torch.zeros(batch, chunk_tokens, heads, head_dim, dtype=torch.bfloat16,
                              device=device)}
    return [{"k": [slot() for _ in range(n_chunks)], "v": [slot() for _ in range(n_chunks)],
             "stage": stage} for _ in range(num_layers)]


def ordered_chunks(block_cache, destination, leading):
    """chunked_kv_cache.py:172-177: K and V buffers in ``(leading..., destination)`` order."""
    order = (*leading, destination)
    return (tuple(block_cache["k"][i] for i in order), tuple(block_cache["v"][i] for i in order))


def ordered_chunks_by_block(cache, destination, leading):
    """chunked_kv_cache.py:180-182: the same for every block."""
    pairs = [ordered_chunks(bc, destination, leading) for bc in cache]
    return tuple(p[0] for p in pairs), tuple(p[1] for p in pairs)


def chunk_bytes(cache) -> int:
    """chunked_kv_cache.py:193-200: bytes held by a chunked cache."""
    return sum(t.numel() * t.element_size() for bc in cache for key in ("k", "v")
               for t in bc.get(key, ()))


@dataclass(frozen=True)
class FlatWritePlan:
    """One chunk's write into a flat windowed cache (model_fast.py:2436-2545)."""
    roll: tuple | None      # (dst, src, length): cache[dst:dst+len] = cache[src:src+len]
    write: tuple            # (start, end) slot of the new chunk
    global_end: int
    local_end: int
    attn_lo: int            # attention window [attn_lo, attn_hi)
    attn_hi: int


def plan_flat_write(kv_cache_size: int, global_end: int, local_end: int, current_start: int,
                    num_new: int, sink_tokens: int, max_attention_size: int,
                    local_attn_size: int = 0) -> FlatWritePlan:
    """The eager write logic of model_fast.py:2463-2545 as plain integers: a global cache
    (``local_attn_size == -1``) writes at ``[current_start, current_end)``; a windowed cache
    that would overflow first rolls everything after the sink left by the evicted count."""
    current_end = current_start + num_new
    roll = None
    if local_attn_size == -1:
        start, end = current_start, current_end
    elif current_end > global_end and num_new + local_end > kv_cache_size:
        evicted = num_new + local_end - kv_cache_size
        kept = local_end - evicted - sink_tokens
        roll = (sink_tokens, sink_tokens + evicted, kept)
        end = local_end + current_end - global_end - evicted
        start = end - num_new
    else:
        end = local_end + current_end - global_end
        start = end - num_new
    lo = end - max_attention_size
    return FlatWritePlan(roll=roll, write=(start, end), global_end=current_end, local_end=end,
                         attn_lo=lo if lo > 0 else 0, attn_hi=end)


class FlatKVCache:
    """A flat windowed K/V cache ``[B, kv_size, N, D]`` with its indices on the host (the
    reference keeps ``global_end_index`` / ``local_end_index`` as device scalars and reads
    them with .item(); here they are plain ints, so planning never syncs the device)."""

    def __init__(self, batch, kv_size, heads, head_dim, dtype=torch.bfloat16, device="cuda",
                 sink_tokens=0, max_attention_size=None, local_attn_size=0):
        self.k = torch.zeros(batch, kv_size, heads, head_dim, dtype=dtype, device=device)
        self.v = torch.zeros_like(self.k)
        self.kv_size = kv_size
        self.sink_tokens = sink_tokens
        self.max_attention_size = kv_size if max_attention_size is None else max_attention_size
        self.local_attn_size = local_attn_size
        self.global_end = 0
        self.local_end = 0

    def plan(self, current_start: int, num_new: int) -> FlatWritePlan:
        return plan_flat_write(self.kv_size, self.global_end, self.local_end, current_start,
                               num_new, self.sink_tokens, self.max_attention_size,
                               self.local_attn_size)

    def apply_roll(self, p: FlatWritePlan):
        """Perform the plan's eviction roll (a device copy) before the new chunk is written."""
        if p.roll is not None:
            dst, src, n = p.roll
            if n > 0:
                self.k[:, dst:dst + n] = self.k[:, src:src + n].clone()
                self.v[:, dst:dst + n] = self.v[:, src:src + n].clone()

    def commit(self, p: FlatWritePlan):
        self.global_end, self.local_end = p.global_end, p.local_end

    def slot(self, p: FlatWritePlan):
        """The (K, V) views ``[B, L, N, D]`` the new chunk is written into."""
        s, e = p.write
        return self.k[:, s:e], self.v[:, s:e]
