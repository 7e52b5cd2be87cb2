"""lbw_amd -- MI355X (gfx950) causal-chunk attention path of LingBot-World.

Host-side mirror of the reference's attention interface (wan/modules/attention.py,
kernels/qk_post.py, wan/modules/chunked_kv_cache.py) over the C ABI of liblbw_attn.so
(include/lbw_attn.h). Importing is cheap; the HIP library loads on first use and raises
when it is missing.
"""
from .attention import (PRESCALED_SOFTMAX_SCALE, attention, attention_chain, attention_merge,
                        attention_merge_partials, attention_partial, attention_segments, prescaled_q_scale,
                        cross_attention, cross_attention_dedup, exact_attention, exact_attention_chunks,
                        flash_attention, padding_start)
from .chunked_kv_cache import (FlatKVCache, allocate_self_kv_chunks, allocate_self_kv_chunks_fp8,
                               chunk_routing, num_chunks)
from .fp8 import Fp8KV, attention_fp8kv, quantize_kv_fp8
from .layer import WanCrossAttention, WanSelfAttention
from .qk_post import (qk_norm_rope, qk_norm_rope3, qk_norm_rope_, qk_norm_rope_t, qk_norm_rope_t3,
                      x_norm_rope, x_norm_rope_t3)
from .rope import RopeTables, causal_rope_tables, rope_params, wan_rope_freqs

__all__ = [
    "attention", "flash_attention", "exact_attention", "exact_attention_chunks",
    "cross_attention", "cross_attention_dedup", "padding_start", "attention_partial", "attention_merge",
    "attention_merge_partials", "attention_chain", "attention_segments",
    "PRESCALED_SOFTMAX_SCALE", "prescaled_q_scale",
    "qk_norm_rope", "qk_norm_rope_", "qk_norm_rope3", "qk_norm_rope_t", "qk_norm_rope_t3",
    "x_norm_rope", "x_norm_rope_t3", "RopeTables", "causal_rope_tables", "rope_params",
    "wan_rope_freqs", "Fp8KV", "quantize_kv_fp8", "attention_fp8kv", "FlatKVCache",
    "allocate_self_kv_chunks", "allocate_self_kv_chunks_fp8", "chunk_routing", "num_chunks", "WanSelfAttention",
    "WanCrossAttention",
]
