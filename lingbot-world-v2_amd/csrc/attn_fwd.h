// Kernel-argument structs and launchers of the attention kernels (internal to the library).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lbw {

constexpr int LBW_MAX_SEGS = 8;
enum { kModeNormalized = 0, kModePartials = 1 };

struct SegDesc {
  const uint16_t* k;  // bf16 elements (or fp8 codes reinterpreted by the fp8 kernel)
  const uint16_t* v;
  int64_t start;      // first logical key of this segment
  int64_t len;
  int64_t ksb, ksl, ksh;
  int64_t vsb, vsl, vsh;
  const float* ks;    // fp8 scales [B, H, nblk]
  const float* vs;
  int64_t nblk;       // scale blocks per (b, h)
  int64_t ksd;        // d-major K: the d stride (token stride 1); 0: K token-major
};

struct AttnKernelArgs {
  const uint16_t* q;
  int64_t qsb, qsl, qsh;
  uint16_t* out;
  int64_t osb, osl, osh;
  int o16;            // out and its strides allow 16-byte stores
  int o32;            // out is fp32 (16-byte aligned, strides multiples of 4) instead of bf16
  int nseg;
  SegDesc seg[LBW_MAX_SEGS];
  int64_t total;      // keys in the concatenation
  int64_t lo, hi;     // clamped window
  const int64_t* lo_dev;  // device window bounds (narrow [lo, hi) on the device), or null
  const int64_t* hi_dev;
  const int32_t* k_lens;
  float scale;        // softmax scale
  float scale_log2;   // scale * log2(e)
  int B, H, Lq;
  int n_qtiles, splits;
  uint32_t* queue;    // 8 work-queue counters (zeroed before the launch), or null: static order
  uint32_t* merge_cnt;  // split partials merged in-kernel: one arrival counter per unit (zeroed
                        // with the queue counters, right after them); null: a separate merge
  int mode;
  float* part_o;
  float* part_m;
  float* part_l;
  int64_t mult_key;   // first of the keys that each stand for several identical keys, or -1
  float mult_raw;     // ln(multiplicity) / scale: added to those keys' raw scores
  int track_max;      // partials must carry the true row max (cte_partial contract); otherwise
                      // any exponent reference consistent with O and l will do
  int k_dmajor;       // every segment's K is d-major (SegDesc::ksd)
  const float* key_bias;  // per-key score bias over the concatenated keys (natural log), or null
  float inv_scale;        // 1 / scale: the bias in raw-score units
};

struct MergeKernelArgs {
  int n;
  const float* o[16];
  const float* m[16];
  const float* l[16];
  int B, H, Lq, D;
  uint16_t* out;      // bf16, or fp32 when o32
  int64_t osb, osl, osh;
  int o32;
  // partial output (the merged (O, m, l) triple, [B, H, Lq, D] / [B, H, Lq], contiguous) instead
  // of the normalised `out`, when part_o is set
  float* part_o;
  float* part_m;
  float* part_l;
};

int attn_lds_bytes();
int attn_block_m();
int attn_block_n();
hipError_t launch_attn_fwd(const AttnKernelArgs& a, hipStream_t stream);
hipError_t launch_attn_fwd_fp8(const AttnKernelArgs& a, hipStream_t stream);
hipError_t launch_attn_merge(const MergeKernelArgs& a, hipStream_t stream);
// Cross-attention (cross_attn.hip): one segment, single pass, persistent workgroups on
// `num_cus` CUs; keys beyond cross_attn_max_keys_resident() run in chunks.
hipError_t launch_cross_attn(const AttnKernelArgs& a, int num_cus, hipStream_t stream);
int cross_attn_max_keys_resident();
// The ring form (cross_attn.hip): every key of [lo, hi) attended (no k_lens, no multiplicity
// bias), 320 < hi - lo <= 4096; the context streams through an LDS ring, persistent workgroups.
hipError_t launch_cross_ring(const AttnKernelArgs& a, int num_cus, hipStream_t stream);

struct QkNormRopeArgs {
  int L, C, H;
  const uint16_t* q; int64_t qs;
  const uint16_t* k; int64_t ks;
  const uint16_t* bq; const uint16_t* bk;
  const uint16_t* wq; const uint16_t* wk;
  float eps, inv_c;
  const float* rope;
  int gf, gh, gw, s0, s1;
  int ntab;            // floats of rope tables (0: no token is rotated)
  uint16_t* qo; int64_t qos;
  uint16_t* ko; int64_t kos;
  float q_scale, k_scale;
  const uint16_t* v; int64_t vs;
  uint16_t* vo; int64_t vos;
  int layout;          // QK_LAYOUT_ROWS: qos/kos are row strides; QK_LAYOUT_DMAJOR: d strides
  int qo_vec, ko_vec;  // d-major: outputs allow 16-byte stores of 8 tokens
};
constexpr int QK_LAYOUT_ROWS = 0;
constexpr int QK_LAYOUT_DMAJOR = 1;
hipError_t launch_qk_norm_rope(const QkNormRopeArgs& a, hipStream_t stream);
int qk_norm_rope_max_table_floats();
size_t qk_norm_rope_lds_bytes(int ntab, int C, int layout);
size_t qk_norm_rope_lds_limit();
int qk_norm_rope_dmajor_max_dim();

struct KvQuantArgs {
  const uint16_t* x;
  int B, H, D;
  int64_t L, sb, sl, sh;
  uint8_t* codes;
  float* scales;
  int block;
  int64_t nblk;
};
hipError_t launch_kv_quant_fp8(const KvQuantArgs& a, hipStream_t stream);

}  // namespace lbw
