// Fused q/k RMSNorm + Wan 3-D RoPE (+ optional V copy into the KV cache slot), gfx950.
//
// Restates kernels/qk_post.py:88-141 (qk_norm_rope) with the sum of squares of
// kernels/qk_post.py:49-73 folded in (one GPU holds the full row, so no all-reduce):
//   y = x + b (fp32); r = 1 / sqrt(sum(y^2) / C + eps); t = bf16(y * r) * gamma (fp32);
//   RoPE on interleaved pairs (fp32, separate multiplies and adds as torch does them);
//   out = bf16(rot * out_scale).
// RoPE angles follow wan/modules/model_fast.py:878-931: token (fi, hi, wi) of the
// frame-major grid takes pair j's cos/sin from the frame table (j < s0), the height table
// (j < s0 + s1) or the width table. The per-axis tables live in LDS; tokens past f*h*w are
// not rotated (model_fast.py:972-975).
//
// One wave per token row: 64 lanes x 16-byte chunks, the row held in registers between the
// reduction and the write-back (C <= 8192), the reduction done with cross-lane shuffles.

#include "common.h"
#include "attn_fwd.h"

namespace lbw {

constexpr int QK_WAVES = 4;
constexpr int QK_MAX_CHUNKS = 16;          // chunks of 8 per lane: C <= 16 * 64 * 8 = 8192
constexpr int QK_MAX_TABLE = 16384;        // floats of per-axis tables held in LDS (64 KB)

int qk_norm_rope_max_table_floats() { return QK_MAX_TABLE; }

struct RopePair {
  float c[4];
  float s[4];
};

__device__ __forceinline__ void rope_lookup(const float* tab, const QkNormRopeArgs& a, int fi,
                                            int hi, int wi, int j0, RopePair& rp) {
  const int base_h = 2 * a.gf * a.s0;
  const int base_w = base_h + 2 * a.gh * a.s1;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int j = j0 + i;
    int ci, si;
    if (j < a.s0) {
      ci = fi * a.s0 + j;
      si = ci + a.gf * a.s0;
    } else if (j < a.s0 + a.s1) {
      ci = base_h + hi * a.s1 + (j - a.s0);
      si = ci + a.gh * a.s1;
    } else {
      ci = base_w + wi * a.s1 + (j - a.s0 - a.s1);
      si = ci + a.gw * a.s1;
    }
    rp.c[i] = tab[ci];
    rp.s[i] = tab[si];
  }
}

// Process one [C] row: x (+bias) -> norm -> gamma -> rope -> out.
__device__ __forceinline__ void norm_rope_row(const QkNormRopeArgs& a, const float* tab,
                                              const uint16_t* x, const uint16_t* bias,
                                              const uint16_t* gamma, uint16_t* out,
                                              float out_scale, bool rotate, int fi, int hi,
                                              int wi, int lane) {
  const int nchunk = a.C / 8;
  float y[QK_MAX_CHUNKS][8];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < QK_MAX_CHUNKS; ++i) {
    const int ch = lane + 64 * i;
    if (ch < nchunk) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(x + 8 * ch);
      u32x4 bv = {0u, 0u, 0u, 0u};
      if (bias != nullptr) bv = *reinterpret_cast<const u32x4*>(bias + 8 * ch);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        y[i][2 * w] = __fadd_rn(bf16_lo(v[w]), bf16_lo(bv[w]));
        y[i][2 * w + 1] = __fadd_rn(bf16_hi(v[w]), bf16_hi(bv[w]));
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = __fmaf_rn(y[i][e], y[i][e], ss);
    }
  }
  ss = wave_reduce_sum(ss);
  const float r = 1.0f / sqrtf(__fadd_rn(__fmul_rn(ss, a.inv_c), a.eps));
  const int D = a.C / a.H;
#pragma unroll
  for (int i = 0; i < QK_MAX_CHUNKS; ++i) {
    const int ch = lane + 64 * i;
    if (ch < nchunk) {
      const u32x4 gv = *reinterpret_cast<const u32x4*>(gamma + 8 * ch);
      float t[8];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        t[2 * w] = __fmul_rn(round_bf16(__fmul_rn(y[i][2 * w], r)), bf16_lo(gv[w]));
        t[2 * w + 1] = __fmul_rn(round_bf16(__fmul_rn(y[i][2 * w + 1], r)), bf16_hi(gv[w]));
      }
      float o[8];
      if (rotate) {
        const int j0 = ((8 * ch) % D) / 2;
        RopePair rp;
        rope_lookup(tab, a, fi, hi, wi, j0, rp);
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const float re = t[2 * p], im = t[2 * p + 1];
          o[2 * p] = __fsub_rn(__fmul_rn(re, rp.c[p]), __fmul_rn(im, rp.s[p]));
          o[2 * p + 1] = __fadd_rn(__fmul_rn(re, rp.s[p]), __fmul_rn(im, rp.c[p]));
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = t[e];
      }
      if (out_scale != 1.0f) {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = __fmul_rn(o[e], out_scale);
      }
      u32x4 ov;
#pragma unroll
      for (int w = 0; w < 4; ++w) ov[w] = pack_bf16x2(o[2 * w], o[2 * w + 1]);
      *reinterpret_cast<u32x4*>(out + 8 * ch) = ov;
    }
  }
}

__global__ void __launch_bounds__(QK_WAVES * 64)
qk_norm_rope_kernel(const QkNormRopeArgs a) {
  __shared__ float tab[QK_MAX_TABLE];
  for (int i = threadIdx.x; i < a.ntab; i += blockDim.x) tab[i] = a.rope[i];
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int grid_tokens = a.gf * a.gh * a.gw;
  for (int row = blockIdx.x * QK_WAVES + wave; row < a.L; row += gridDim.x * QK_WAVES) {
    const bool rotate = row < grid_tokens;
    int fi = 0, hi = 0, wi = 0;
    if (rotate) {
      wi = row % a.gw;
      hi = (row / a.gw) % a.gh;
      fi = row / (a.gw * a.gh);
    }
    norm_rope_row(a, tab, a.q + a.qs * row, a.bq, a.wq, a.qo + a.qos * row, a.q_scale, rotate,
                  fi, hi, wi, lane);
    norm_rope_row(a, tab, a.k + a.ks * row, a.bk, a.wk, a.ko + a.kos * row, a.k_scale, rotate,
                  fi, hi, wi, lane);
    if (a.v != nullptr) {
      const uint16_t* vs = a.v + a.vs * row;
      uint16_t* vd = a.vo + a.vos * row;
      for (int ch = lane; ch < a.C / 8; ch += 64)
        *reinterpret_cast<u32x4*>(vd + 8 * ch) = *reinterpret_cast<const u32x4*>(vs + 8 * ch);
    }
  }
}

hipError_t launch_qk_norm_rope(const QkNormRopeArgs& a, hipStream_t stream) {
  int blocks = (a.L + QK_WAVES - 1) / QK_WAVES;
  if (blocks > 1024) blocks = 1024;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3(blocks), dim3(QK_WAVES * 64), 0, stream, a);
  return hipGetLastError();
}

}  // namespace lbw
