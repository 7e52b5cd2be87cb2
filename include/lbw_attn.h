/*
 * lbw_attn.h -- C ABI of the MI355X (gfx950) causal-chunk attention path.
 *
 * Plain pointers and sizes only (no torch types). Every tensor pointer is a device pointer.
 * Element strides are in elements of the tensor's own type; the innermost (head_dim)
 * dimension is always contiguous. Every entry point returns 0 (LBW_OK) on success and a
 * nonzero LBW_ERR_* code otherwise, with a message in lbw_last_error() (per thread).
 * All work is enqueued on `stream` (a hipStream_t; NULL = the default stream) and is
 * asynchronous; nothing here synchronises the device or allocates memory.
 *
 * Reference interfaces replaced (paths inside the reference repository):
 *   lbw_attention_fwd      wan/modules/attention.py:1082-1143  attention(q, k, v, ...)
 *                          wan/modules/attention.py:1048-1058  exact_attention_chunks
 *                          wan/modules/attention.py:617-645    cte_partial (partials mode)
 *                          kernels/self_attention_nst.py:49    wan_flash_self_attn
 *                          kernels/attention_cte_lb.py:270     attention_cte
 *   lbw_cross_attention_fwd wan/modules/attention.py:280-311   _nki_cross_attention
 *                          kernels/cross_attention.py:17       wan_cross_attn
 *   lbw_cross_attention_dedup_fwd
 *                          wan/modules/attention.py:493-554    cross_dedup_bias +
 *                                                              cross_attention_dedup
 *                          kernels/cross_dedup.py              cross_dedup_kernel
 *   lbw_attn_merge         wan/modules/attention.py:963-990    cte_merge
 *   lbw_attn_merge_partials wan/modules/attention.py:654-694   cte_call's chain state
 *   lbw_qk_norm_rope       kernels/qk_post.py:404-413          qk_ss + qk_norm_rope
 *                          (caller wan/modules/model_fast.py:2596-2681 _qkv_post)
 *   lbw_kv_quant_fp8       no reference counterpart (new fp8-e4m3 KV cache)
 *   lbw_attention_fwd_fp8kv no reference counterpart; nearest is the delayed fp8 K
 *                          dequant of kernels/attention_cte_lb.py:645-647
 */
#ifndef LBW_ATTN_H
#define LBW_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 4: the fp8 entry point reads power-of-two block scales only (lbw_kv_quant_fp8 writes them). */
#define LBW_ABI_VERSION 4
#define LBW_MAX_KV_SEGMENTS 8
#define LBW_FP8_BLOCK 64

enum {
  LBW_OK = 0,
  LBW_ERR_INVALID = 1,     /* bad argument (shape, stride, pointer, size) */
  LBW_ERR_UNSUPPORTED = 2, /* valid but not implemented here (e.g. head_dim != 128) */
  LBW_ERR_HIP = 3,         /* a HIP runtime call failed */
  LBW_ERR_WORKSPACE = 4    /* workspace missing or too small */
};

/* One contiguous piece of the KV sequence, tokens-major [B, len, H, D]. The attention sees
 * the concatenation of the segments in order (e.g. the cached frames then the current
 * chunk, or the chunked cache's (leading..., destination) buffers), without a copy.
 * K may instead be d-major, the reference's N-major K cache [H, D, L] (and its pre-transposed
 * cross cache): k_stride_d > 0 puts element (b, t, h, d) of K at b * k_stride_b + h * k_stride_h
 * + d * k_stride_d + t, token stride 1 (k_stride_l must then be 1); bf16 entry points only,
 * every segment of the call d-major, len and the strides multiples of 8
 * (wan/modules/chunked_kv_cache.py:118-148, wan/modules/attention.py:494-499, 557-579). V is
 * token-major per head in both of those layouts ([H, L, D] is a strided [B, L, H, D]). */
typedef struct lbw_kv_segment {
  const void* k;        /* bf16, or e4m3fn codes (uint8) for the fp8 entry point */
  const void* v;
  int64_t len;          /* tokens in this segment */
  int64_t k_stride_b, k_stride_l, k_stride_h;
  int64_t v_stride_b, v_stride_l, v_stride_h;
  const float* k_scale; /* fp8 only: [B, H, ceil(len / 64)] fp32, contiguous */
  const float* v_scale;
  int64_t k_stride_d;   /* 0: K token-major (head dim contiguous); > 0: K d-major (above) */
} lbw_kv_segment;

typedef struct lbw_attn_params {
  int32_t batch, heads, head_dim, lq;
  const void* q;        /* bf16 [B, Lq, H, D] */
  int64_t q_stride_b, q_stride_l, q_stride_h;
  void* out;            /* bf16 (or fp32, see out_dtype) [B, Lq, H, D]; may be NULL when
                         * partials are requested */
  int64_t o_stride_b, o_stride_l, o_stride_h;
  int32_t n_segments;
  lbw_kv_segment seg[LBW_MAX_KV_SEGMENTS];
  int64_t kv_lo, kv_hi; /* window [kv_lo, kv_hi) over the concatenated keys; kv_hi < 0: all */
  const int32_t* k_lens;/* device int32 [B] valid key counts (masked cross-attention) or NULL */
  float softmax_scale;  /* <= 0: 1 / sqrt(head_dim). ln 2 (softmax_scale * log2(e) == 1 in
                         * fp32) marks a q pre-scaled by log2(e) / sqrt(head_dim): the bf16
                         * kernel then needs no per-score scaling (its fastest form) */
  int32_t num_splits;   /* KV splits merged by log-sum-exp; 0 = choose, 1 = single pass */
  /* Optional cte_partial outputs, fp32 and contiguous: O_unnorm [B, H, Lq, D],
   * m [B, H, Lq] (row max of the scaled scores), l [B, H, Lq] (row sum of exp(s - m)).
   * When set, the normalised `out` is not written and num_splits must be 1. */
  float* part_o;
  float* part_m;
  float* part_l;
  /* LBW_OUT_BF16 (0): `out` is bf16. LBW_OUT_FP32 (1): `out` is fp32 [B, Lq, H, D] (16-byte
   * aligned, strides multiples of 4), the normalised O / l before any bf16 rounding: a check
   * of the kernels' own arithmetic apart from the output rounding (same kernels, same plan). */
  int32_t out_dtype;
  /* Optional device int64 [1] window bounds, read by the kernel on the device, so that a caller
   * whose window lives in device tensors (the flat cache's attn_lo / attn_hi,
   * wan/modules/model_fast.py:2538-2550) needs no host synchronisation: the window is
   * [max(kv_lo, *kv_lo_dev), min(kv_hi, *kv_hi_dev)) clamped to the keys. NULL = the host
   * bounds alone. The split plan assumes the host window; cross-attention takes neither. */
  const int64_t* kv_lo_dev;
  const int64_t* kv_hi_dev;
  /* Optional per-key additive score bias, fp32 [total keys of the segments] on the device,
   * natural-log units added to the scaled scores and shared by every batch and head:
   * softmax(scale q k^T + bias) v, as cross_attention_dedup's bias (attention.py:532-554). NULL
   * = none. Not with partials outputs, the fp8 entry point or n_distinct (the dedup entry's own
   * bias). Calls with a bias run a kernel instance of their own. */
  const float* key_bias;
} lbw_attn_params;
#define LBW_OUT_BF16 0
#define LBW_OUT_FP32 1

/* Bytes of workspace lbw_attention_fwd needs for these params: the split-KV partials (when
 * the call is split) and 256 bytes of work-queue counters, which let the XCDs of the GPU share
 * out the workgroups by speed. A call given no (or too small a) workspace for an unsplit plan
 * still runs, with a static workgroup-to-XCD assignment. 0 when the params are invalid (the
 * attention call then reports why).
 * A workspace may back only one in-flight call: two calls that may overlap on the device
 * (e.g. on two streams) need two workspaces. */
size_t lbw_attention_workspace_size(const lbw_attn_params* p);

/* The same for lbw_attention_fwd_fp8kv (fp8 segments follow the fp8 stride and size rules). */
size_t lbw_attention_fp8kv_workspace_size(const lbw_attn_params* p);

/* Chunk self-attention: softmax(scale * Q K^T) V over the windowed concatenation of the KV
 * segments, bf16 MFMA, fp32 online softmax. */
int lbw_attention_fwd(const lbw_attn_params* p, void* workspace, size_t workspace_bytes,
                      void* stream);

/* lbw_attention_fwd for callers that cannot allocate (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc); no counterpart in the reference. Same
 * params and results, no workspace argument: the work-queue counters and split-KV partials
 * live in a static device array of LBW_NOALLOC_SCRATCH_BYTES that the library holds on each
 * GPU it runs on until the process ends. Nothing is allocated or freed. With num_splits = 0
 * the host's split choice is lowered, when needed, to the most splits whose partials fit;
 * an explicit num_splits whose partials do not fit fails with LBW_ERR_WORKSPACE. Every call
 * on one GPU shares that GPU's array, so calls that may overlap on one GPU (e.g. on two
 * streams) race: serialise them, or use lbw_attention_fwd with a workspace each. */
#define LBW_NOALLOC_SCRATCH_BYTES (64u << 20)
int lbw_attention_fwd_noalloc(const lbw_attn_params* p, void* stream);

/* Cross-attention to a short context (one segment of <= 4096 keys, typically 512), with the
 * optional per-batch valid length p->k_lens. Single pass, no workspace. Up to 320 attended keys
 * stay resident in LDS per (batch, head) (the masked 300-row context); a longer context with
 * every key attended (no k_lens: the reference's unmasked 512-row call) streams through an LDS
 * tile ring that runs across the persistent workgroups' rounds. */
int lbw_cross_attention_fwd(const lbw_attn_params* p, void* stream);

/* Exact deduplicated cross-attention (no mask): keys n_distinct .. len-1 of the one segment
 * must be identical rows (the context's zero padding after the projections); the result equals
 * attention over all len keys, computed over the distinct keys plus the r identical ones up to
 * the end of their 64-key tile, each of those with its score raised by ln((len - n_distinct) /
 * r). p->k_lens must be NULL and no window set. */
int lbw_cross_attention_dedup_fwd(const lbw_attn_params* p, int64_t n_distinct, void* stream);

/* fp8-e4m3 KV cache: K/V segments hold e4m3fn codes with per-(batch, head, 64-token block)
 * fp32 scales (lbw_kv_quant_fp8's layout); Q is given in bf16. Q K^T runs on the fp8 matrix
 * cores (each query split into two e4m3 operands that hold its bf16 values) with K's scale as
 * the product's exponent scale, P V in bf16 on V codes converted exactly at V's scale. The
 * scales must be powers of two (lbw_kv_quant_fp8 writes them so): a row that reads a tile whose
 * scale is not one comes out NaN. */
int lbw_attention_fwd_fp8kv(const lbw_attn_params* p, void* workspace, size_t workspace_bytes,
                            void* stream);

/* Log-sum-exp merge of n_parts partials (cte_merge): part_o[i] [B, H, Lq, D] fp32,
 * part_m[i], part_l[i] [B, H, Lq] fp32 -> out bf16 [B, Lq, H, D] (strided). */
int lbw_attn_merge(int32_t n_parts, const float* const* part_o, const float* const* part_m,
                   const float* const* part_l, int32_t batch, int32_t heads, int32_t lq,
                   int32_t head_dim, void* out, int64_t o_stride_b, int64_t o_stride_l,
                   int64_t o_stride_h, void* stream);

/* The same log-sum-exp merge into one partial triple instead of the normalised output: out_o
 * [B, H, Lq, D] = sum_i e^(m_i - M) O_i, out_m [B, H, Lq] = M = max_i m_i, out_l = sum_i
 * e^(m_i - M) l_i (all fp32, contiguous; M = -inf, O = 0, l = 0 for a row with no keys). The
 * running (O, max, sum) state of cte_call's chain: each call's partials merged into it keep it
 * one triple however many calls there are; lbw_attn_merge of the final triple normalises.
 * The outputs must not overlap the inputs. */
int lbw_attn_merge_partials(int32_t n_parts, const float* const* part_o,
                            const float* const* part_m, const float* const* part_l, int32_t batch,
                            int32_t heads, int32_t lq, int32_t head_dim, float* out_o,
                            float* out_m, float* out_l, void* stream);

/* Fused q/k post-processing of one chunk (kernels/qk_post.py semantics, full-row RMSNorm):
 *   y = x + b (fp32); r = rsqrt(sum(y^2)/C + eps); t = bf16(y*r) * gamma (fp32);
 *   Wan 3-D RoPE on interleaved pairs in fp32 with the output scale folded into cos and sin
 *   (kernels/qk_post.py:259-265): out = bf16(re*(cos*s) - im*(sin*s), re*(sin*s) + im*(cos*s)).
 * Tokens >= f*h*w pass the RoPE unrotated (out = bf16(t*s)). The RoPE tables are the per-axis
 * cos/sin rows, packed fp32: cos_t[f][s0], sin_t[f][s0], cos_h[h][s1], sin_h[h][s1],
 * cos_w[w][s1], sin_w[w][s1] with s0 + 2*s1 = head_dim/2. Optionally copies v into v_out (the
 * KV-cache commit of the new chunk's V; always rows). k_out/v_out may point into a KV cache slot.
 * out_layout LBW_QK_ROWS: q_out/k_out are bf16 rows [L, C], *_out_stride = row stride.
 * out_layout LBW_QK_DMAJOR (kernels/qk_post.py:216-306, qk_norm_rope_t): q_out/k_out are
 * [H, D, L] with token stride 1, *_out_stride = the d stride (>= L; e.g. the capacity of a
 * [H, D, capacity] cache, with the pointer at the slot's first token) and head stride
 * D * d stride.
 * k == NULL processes q alone (kernels/qk_post.py:144-215, 308-402: x_norm_rope,
 * x_norm_rope_t3); wk and k_out are then ignored. */
#define LBW_QK_ROWS 0
#define LBW_QK_DMAJOR 1
typedef struct lbw_qk_norm_rope_params {
  int32_t tokens, dim, heads;      /* L, C = heads * head_dim */
  const void* q; int64_t q_stride; /* bf16 rows [L, C], row stride in elements */
  const void* k; int64_t k_stride;
  const void* bq; const void* bk;  /* bf16 [C] or NULL */
  const void* wq; const void* wk;  /* bf16 [C] RMSNorm gamma */
  float eps;
  const float* rope;               /* packed per-axis tables (see above) */
  int32_t grid_f, grid_h, grid_w, s0, s1;
  void* q_out; int64_t q_out_stride;
  void* k_out; int64_t k_out_stride;
  float q_out_scale, k_out_scale;  /* 1.0 = none */
  const void* v; int64_t v_stride; /* optional V copy (bf16 [L, C]); NULL = none */
  void* v_out; int64_t v_out_stride;
  int32_t out_layout;              /* LBW_QK_ROWS or LBW_QK_DMAJOR */
} lbw_qk_norm_rope_params;

int lbw_qk_norm_rope(const lbw_qk_norm_rope_params* p, void* stream);

/* fp8-e4m3fn KV quantiser: x bf16 [B, L, H, D] (strided) -> codes uint8 [B, L, H, D]
 * (contiguous) and scales fp32 [B, H, ceil(L / block)] (contiguous). Per (b, h, block):
 * scale = the smallest power of two 2^k >= amax / 448, k >= -126 (1 if amax == 0);
 * code = rne_e4m3fn(x * 2^-k). */
int lbw_kv_quant_fp8(const void* x, int32_t batch, int64_t len, int32_t heads,
                     int32_t head_dim, int64_t s_b, int64_t s_l, int64_t s_h,
                     uint8_t* codes, float* scales, int32_t block, void* stream);

const char* lbw_last_error(void);
int lbw_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* LBW_ATTN_H */
