// Fused q/k RMSNorm + Wan 3-D RoPE (+ optional V copy into the KV cache slot), gfx950.
//
// Restates kernels/qk_post.py:88-141 (qk_norm_rope) with the sum of squares of
// kernels/qk_post.py:49-73 folded in (one GPU holds the full row, so no all-reduce):
//   y = x + b (fp32); r = 1 / sqrt(sum(y^2) / C + eps); t = bf16(y * r) * gamma (fp32);
//   RoPE on interleaved pairs (fp32, separate multiplies and adds as torch does them);
//   out = bf16(rot * out_scale).
// RoPE angles follow wan/modules/model_fast.py:878-931: token (fi, hi, wi) of the
// frame-major grid takes pair j's cos/sin from the frame table (j < s0), the height table
// (j < s0 + s1) or the width table. Tokens past f*h*w are not rotated (model_fast.py:972-975).
//
// HBM-bound: per token the kernel reads q, k (and v) rows and writes q', k' (and v). One wave
// per token row; lane l holds the 16-byte chunks l, l + 64, ... of the row (NCH of them), so
// with the head dim dividing 512 every chunk of a lane covers the same 4 rotation pairs and the
// lane fetches its 4 cos/sin pairs once per row (shared by q and k). The q and k rows are
// loaded together before any arithmetic, so each wave keeps two rows of loads in flight; the
// per-axis RoPE tables and the bias / gamma vectors sit in LDS.

#include "common.h"
#include "attn_fwd.h"

namespace lbw {

constexpr int QK_WAVES = 4;
constexpr int QK_MAX_TABLE = 16384;        // floats of per-axis tables held in LDS (64 KB)

int qk_norm_rope_max_table_floats() { return QK_MAX_TABLE; }

// LDS layout: [ntab floats of tables][bq | bk | gq | gk as bf16, C each]
__host__ __device__ inline int qk_table_floats(int ntab) { return (ntab + 3) & ~3; }
__host__ __device__ inline size_t qk_lds_bytes(int ntab, int C) {
  return (size_t)qk_table_floats(ntab) * 4 + (size_t)4 * C * 2;
}

template <int NCH>
__global__ void __launch_bounds__(QK_WAVES * 64)
qk_norm_rope_kernel(const QkNormRopeArgs a) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int C = a.C;
  const int nchunk = C / 8;
  float* tab = smem;
  uint16_t* vec = reinterpret_cast<uint16_t*>(smem + qk_table_floats(a.ntab));
  {
    // tables and vectors into LDS, several loads in flight per thread (unrolled by 4)
    const int nt2 = a.ntab / 2;  // cos/sin values come in pairs: 8-byte loads
#pragma unroll 4
    for (int i = threadIdx.x; i < nt2; i += blockDim.x)
      reinterpret_cast<u32x2*>(tab)[i] = reinterpret_cast<const u32x2*>(a.rope)[i];
    const uint16_t* src[4] = {a.bq, a.bk, a.wq, a.wk};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      if (src[v] != nullptr) {
#pragma unroll 4
        for (int ch = threadIdx.x; ch < nchunk; ch += blockDim.x)
          *reinterpret_cast<u32x4*>(vec + v * C + 8 * ch) =
              *reinterpret_cast<const u32x4*>(src[v] + 8 * ch);
      } else {
        for (int ch = threadIdx.x; ch < nchunk; ch += blockDim.x)
          *reinterpret_cast<u32x4*>(vec + v * C + 8 * ch) = u32x4{0u, 0u, 0u, 0u};
      }
    }
  }
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int D = C / a.H;
  const int j0 = ((8 * lane) % D) / 2;  // first rotation pair of every chunk of this lane
  const int grid_tokens = a.gf * a.gh * a.gw;
  const int base_h = 2 * a.gf * a.s0;
  const int base_w = base_h + 2 * a.gh * a.s1;

  for (int row = blockIdx.x * QK_WAVES + wave; row < a.L; row += gridDim.x * QK_WAVES) {
    // ---- loads: q and k rows together, then v if it is copied
    u32x4 xq[NCH], xk[NCH];
    const uint16_t* qr = a.q + a.qs * row;
    const uint16_t* kr = a.k + a.ks * row;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int ch = lane + 64 * i;
      if (i + 1 < NCH || ch < nchunk) {  // only the last chunk can run past the row
        xq[i] = *reinterpret_cast<const u32x4*>(qr + 8 * ch);
        xk[i] = *reinterpret_cast<const u32x4*>(kr + 8 * ch);
      }
    }

    // ---- this lane's 4 rotation pairs for the row's (frame, row, column)
    const bool rotate = row < grid_tokens;
    float cr[4], sr[4];
    if (rotate) {
      const int wi = row % a.gw;
      const int hi = (row / a.gw) % a.gh;
      const int fi = row / (a.gw * a.gh);
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const int j = j0 + p;
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
        cr[p] = tab[ci];
        sr[p] = tab[si];
      }
    }

    // ---- sums of squares of y = x + b (per lane in chunk order, then across the wave)
    float ssq = 0.0f, ssk = 0.0f;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int ch = lane + 64 * i;
      if (i + 1 < NCH || ch < nchunk) {
        const u32x4 bq = *reinterpret_cast<const u32x4*>(vec + 8 * ch);
        const u32x4 bk = *reinterpret_cast<const u32x4*>(vec + C + 8 * ch);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float q0 = __fadd_rn(bf16_lo(xq[i][w]), bf16_lo(bq[w]));
          const float q1 = __fadd_rn(bf16_hi(xq[i][w]), bf16_hi(bq[w]));
          const float k0 = __fadd_rn(bf16_lo(xk[i][w]), bf16_lo(bk[w]));
          const float k1 = __fadd_rn(bf16_hi(xk[i][w]), bf16_hi(bk[w]));
          ssq = __fmaf_rn(q0, q0, ssq);
          ssq = __fmaf_rn(q1, q1, ssq);
          ssk = __fmaf_rn(k0, k0, ssk);
          ssk = __fmaf_rn(k1, k1, ssk);
        }
      }
    }
    ssq = wave_reduce_sum(ssq);
    ssk = wave_reduce_sum(ssk);
    const float rq = 1.0f / sqrtf(__fadd_rn(__fmul_rn(ssq, a.inv_c), a.eps));
    const float rk = 1.0f / sqrtf(__fadd_rn(__fmul_rn(ssk, a.inv_c), a.eps));

    // ---- normalise, gamma, rotate, store
    auto finish = [&](const u32x4& x, const u32x4& bv, const u32x4& gv, float r, float scale,
                      uint16_t* dst) {
      float t[8];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float y0 = __fadd_rn(bf16_lo(x[w]), bf16_lo(bv[w]));
        const float y1 = __fadd_rn(bf16_hi(x[w]), bf16_hi(bv[w]));
        t[2 * w] = __fmul_rn(round_bf16(__fmul_rn(y0, r)), bf16_lo(gv[w]));
        t[2 * w + 1] = __fmul_rn(round_bf16(__fmul_rn(y1, r)), bf16_hi(gv[w]));
      }
      float o[8];
      if (rotate) {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const float re = t[2 * p], im = t[2 * p + 1];
          o[2 * p] = __fsub_rn(__fmul_rn(re, cr[p]), __fmul_rn(im, sr[p]));
          o[2 * p + 1] = __fadd_rn(__fmul_rn(re, sr[p]), __fmul_rn(im, cr[p]));
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = t[e];
      }
      if (scale != 1.0f) {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = __fmul_rn(o[e], scale);
      }
      u32x4 ov;
#pragma unroll
      for (int w = 0; w < 4; ++w) ov[w] = pack_bf16x2(o[2 * w], o[2 * w + 1]);
      *reinterpret_cast<u32x4*>(dst) = ov;
    };
    uint16_t* qo = a.qo + a.qos * row;
    uint16_t* ko = a.ko + a.kos * row;
    // recompute y = x + b below (bias re-read from LDS) rather than keeping the fp32 values
    // and bias chunks of the first pass alive
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      asm volatile("" : "+v"(xq[i]));
      asm volatile("" : "+v"(xk[i]));
    }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int ch = lane + 64 * i;
      if (i + 1 < NCH || ch < nchunk) {
        finish(xq[i], *reinterpret_cast<const u32x4*>(vec + 8 * ch),
               *reinterpret_cast<const u32x4*>(vec + 2 * C + 8 * ch), rq, a.q_scale, qo + 8 * ch);
        finish(xk[i], *reinterpret_cast<const u32x4*>(vec + C + 8 * ch),
               *reinterpret_cast<const u32x4*>(vec + 3 * C + 8 * ch), rk, a.k_scale, ko + 8 * ch);
      }
    }

    // ---- V copy into its cache slot
    if (a.v != nullptr) {
      const uint16_t* vs = a.v + a.vs * row;
      uint16_t* vd = a.vo + a.vos * row;
      u32x4 xv[NCH];
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const int ch = lane + 64 * i;
        if (i + 1 < NCH || ch < nchunk) xv[i] = *reinterpret_cast<const u32x4*>(vs + 8 * ch);
      }
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const int ch = lane + 64 * i;
        if (i + 1 < NCH || ch < nchunk) *reinterpret_cast<u32x4*>(vd + 8 * ch) = xv[i];
      }
    }
  }
}

template <int NCH>
static hipError_t launch_nch(const QkNormRopeArgs& a, hipStream_t stream) {
  static hipError_t attr = hipFuncSetAttribute((const void*)qk_norm_rope_kernel<NCH>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)qk_lds_bytes(QK_MAX_TABLE, 64 * 8 * NCH));
  if (attr != hipSuccess) return attr;
  // at most 1024 workgroups (two resident per CU by LDS, the rest queued), each wave looping
  // over rows so that the LDS fill is amortised
  int blocks = (a.L + QK_WAVES - 1) / QK_WAVES;
  if (blocks > 1024) blocks = 1024;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(qk_norm_rope_kernel<NCH>, dim3(blocks), dim3(QK_WAVES * 64),
                     qk_lds_bytes(a.ntab, a.C), stream, a);
  return hipGetLastError();
}

hipError_t launch_qk_norm_rope(const QkNormRopeArgs& a, hipStream_t stream) {
  const int nch = (a.C / 8 + 63) / 64;
  switch (nch) {
    case 1: return launch_nch<1>(a, stream);
    case 2: return launch_nch<2>(a, stream);
    case 3: return launch_nch<3>(a, stream);
    case 4: return launch_nch<4>(a, stream);
    case 5: return launch_nch<5>(a, stream);
    case 6: return launch_nch<6>(a, stream);
    case 7: return launch_nch<7>(a, stream);
    case 8: return launch_nch<8>(a, stream);
    case 9: return launch_nch<9>(a, stream);
    case 10: return launch_nch<10>(a, stream);
    case 11: return launch_nch<11>(a, stream);
    case 12: return launch_nch<12>(a, stream);
    case 13: return launch_nch<13>(a, stream);
    case 14: return launch_nch<14>(a, stream);
    case 15: return launch_nch<15>(a, stream);
    case 16: return launch_nch<16>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace lbw
