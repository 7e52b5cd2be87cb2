// Fused q/k RMSNorm + Wan 3-D RoPE (+ optional V copy into the KV cache slot), gfx950.
//
// Restates kernels/qk_post.py:88-141 (qk_norm_rope) with the sum of squares of
// kernels/qk_post.py:49-73 folded in (one GPU holds the full row, so no all-reduce):
//   y = x + b (fp32); r = 1 / sqrt(sum(y^2) / C + eps); t = bf16(y * r) * gamma (fp32);
//   RoPE on interleaved pairs (fp32, separate multiplies and adds as torch does them), the
//   output scale folded into cos and sin first as kernels/qk_post.py:259-265 does it
//   (cs = cos * s, sn = sin * s in fp32); out = bf16(rot). Rows that are not rotated are
//   out = bf16(t * s).
// RoPE angles follow wan/modules/model_fast.py:878-931: token (fi, hi, wi) of the
// frame-major grid takes pair j's cos/sin from the frame table (j < s0), the height table
// (j < s0 + s1) or the width table. Tokens past f*h*w are not rotated (model_fast.py:972-975).
//
// Two output layouts:
// - rows: q', k' as [L, C] rows (strided), the layout the attention kernel reads;
// - d-major: q', k' as [H, D, L] (token stride 1, a given d stride, head stride D * d stride),
//   the layout of kernels/qk_post.py:228-306 (qk_norm_rope_t). A workgroup of 16 waves takes 16
//   consecutive tokens, stages each 512-column slice of their outputs in LDS and writes it
//   transposed: 32 bytes of consecutive tokens per (head, d) line. Tiles are numbered so that
//   each XCD takes a contiguous run of them, and the two 32-byte halves of a 64-byte line are
//   usually written through the same L2.
// With k == NULL only q is processed (kernels/qk_post.py:144-215, 308-402: x_norm_rope and
// x_norm_rope_t3 on one tensor).
//
// HBM-bound, with enough VALU work per byte (unpacking, the bf16 rounding, the rotation) that
// the loads of some waves must overlap the arithmetic of others: one wave holds one tensor's
// token row (lane l holds the 16-byte chunks l, l + 64, ... of the row, NCH of them), which
// keeps it near 120 registers and four waves per SIMD. With the head dim dividing 512 every
// chunk of a lane covers the same 4 rotation pairs, fetched once per row. The per-axis RoPE
// tables and the bias / gamma vectors sit in LDS.

#include "common.h"
#include "attn_fwd.h"

namespace lbw {

constexpr int QK_WAVES = 8;                // waves per workgroup, rows layout
constexpr int QK_MAX_BLOCKS = 512;         // rows layout: two resident per CU, looping over rows
constexpr int QT_WAVES = 16;               // waves per workgroup, d-major layout
constexpr int QT_ROWS = 16;                // tokens per workgroup
constexpr int QT_MAX_NCH = 10;             // d-major: two rows of C <= 5120 fit 128 registers
constexpr int QT_PITCH = 520;              // bf16 per staged token row (512 + 8: no bank clash)
constexpr int QK_MAX_TABLE = 16384;        // floats of per-axis tables held in LDS (64 KB)
constexpr int LDS_LIMIT = 160 * 1024;

int qk_norm_rope_max_table_floats() { return QK_MAX_TABLE; }

// LDS layout: [ntab floats of tables][bq | bk | gq | gk as bf16, C each][d-major staging]
__host__ __device__ inline int qk_table_floats(int ntab) { return (ntab + 3) & ~3; }
__host__ __device__ inline size_t qk_lds_bytes(int ntab, int C) {
  return (size_t)qk_table_floats(ntab) * 4 + (size_t)4 * C * 2;
}
constexpr size_t QT_STAGE_BYTES = (size_t)2 * QT_ROWS * QT_PITCH * 2;

size_t qk_norm_rope_lds_bytes(int ntab, int C, int layout) {
  return qk_lds_bytes(ntab, C) + (layout == QK_LAYOUT_DMAJOR ? QT_STAGE_BYTES : 0);
}
size_t qk_norm_rope_lds_limit() { return LDS_LIMIT; }
int qk_norm_rope_dmajor_max_dim() { return QT_MAX_NCH * 64 * 8; }

// tables and vectors into LDS, several loads in flight per thread (unrolled by 4)
__device__ __forceinline__ void qk_fill_lds(const QkNormRopeArgs& a, float* tab, uint16_t* vec) {
  const int nchunk = a.C / 8;
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
        *reinterpret_cast<u32x4*>(vec + v * a.C + 8 * ch) =
            *reinterpret_cast<const u32x4*>(src[v] + 8 * ch);
    } else {
      for (int ch = threadIdx.x; ch < nchunk; ch += blockDim.x)
        *reinterpret_cast<u32x4*>(vec + v * a.C + 8 * ch) = u32x4{0u, 0u, 0u, 0u};
    }
  }
}

// One tensor's token row held by one wave: its raw chunks, the inverse norm and this lane's
// four rotation pairs with the tensor's output scale folded in.
template <int NCH>
struct QkOne {
  u32x4 x[NCH];
  float r;
  float c[4], sn[4];
  bool rotate;
};

// The operands of one tensor (t = 0: q, t = 1: k).
struct QkTensor {
  const uint16_t* x; int64_t xs;
  uint16_t* o; int64_t os;
  const uint16_t* bias;   // LDS, C bf16
  const uint16_t* gamma;  // LDS, C bf16
  float scale;
};

__device__ __forceinline__ QkTensor qk_tensor(const QkNormRopeArgs& a, const uint16_t* vec, int t) {
  QkTensor u;
  u.x = t ? a.k : a.q;
  u.xs = t ? a.ks : a.qs;
  u.o = t ? a.ko : a.qo;
  u.os = t ? a.kos : a.qos;
  u.bias = vec + t * a.C;
  u.gamma = vec + (2 + t) * a.C;
  u.scale = t ? a.k_scale : a.q_scale;
  return u;
}

// 16 bytes of a row read once: NT, the non-temporal hint (the d-major kernel: its rows stream
// past the caches, 17 % less time at the 14B 720p chunk; the rows kernel, whose outputs the
// attention reads next, measured 7 % slower with it in the layer sequence and keeps plain loads)
template <bool NT>
__device__ __forceinline__ u32x4 qk_load16(const uint16_t* p) {
  if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  else return *reinterpret_cast<const u32x4*>(p);
}

// issue the loads of one tensor's row (kept apart from qk_one_norm so that a wave can have the
// loads of several rows in flight)
template <int NCH, bool NT>
__device__ __forceinline__ void qk_one_load(const QkNormRopeArgs& a, const QkTensor& u, int row,
                                            int lane, QkOne<NCH>& s) {
  const int nchunk = a.C / 8;
  const uint16_t* xr = u.x + u.xs * row;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int ch = lane + 64 * i;
    if (i + 1 < NCH || ch < nchunk)  // only the last chunk can run past the row
      s.x[i] = qk_load16<NT>(xr + 8 * ch);
  }
}

// rotation pairs, sum of squares and inverse norm of a loaded row
template <int NCH>
__device__ __forceinline__ void qk_one_norm(const QkNormRopeArgs& a, const float* tab,
                                            const QkTensor& u, int row, int lane, QkOne<NCH>& s) {
  const int C = a.C;
  const int nchunk = C / 8;
  // ---- this lane's 4 rotation pairs for the row's (frame, row, column)
  const int D = C / a.H;
  const int j0 = ((8 * lane) % D) / 2;  // first rotation pair of every chunk of this lane
  s.rotate = row < a.gf * a.gh * a.gw;
  if (s.rotate) {
    const int base_h = 2 * a.gf * a.s0;
    const int base_w = base_h + 2 * a.gh * a.s1;
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
      s.c[p] = __fmul_rn(tab[ci], u.scale);
      s.sn[p] = __fmul_rn(tab[si], u.scale);
    }
  }

  // ---- sum of squares of y = x + b (per lane in chunk order, then across the wave)
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int ch = lane + 64 * i;
    if (i + 1 < NCH || ch < nchunk) {
      const u32x4 b = *reinterpret_cast<const u32x4*>(u.bias + 8 * ch);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float y0 = __fadd_rn(bf16_lo(s.x[i][w]), bf16_lo(b[w]));
        const float y1 = __fadd_rn(bf16_hi(s.x[i][w]), bf16_hi(b[w]));
        ss = __fmaf_rn(y0, y0, ss);
        ss = __fmaf_rn(y1, y1, ss);
      }
    }
  }
  ss = wave_reduce_sum(ss);
  s.r = 1.0f / sqrtf(__fadd_rn(__fmul_rn(ss, a.inv_c), a.eps));

  // recompute y = x + b when finishing (bias re-read from LDS) rather than keeping the fp32
  // values and bias chunks of the first pass alive
#pragma unroll
  for (int i = 0; i < NCH; ++i) asm volatile("" : "+v"(s.x[i]));
  asm volatile("" ::: "memory");
}

// normalise, gamma, rotate (scale folded into c/s) or scale, round: one 8-element chunk
__device__ __forceinline__ u32x4 qk_finish(const u32x4& x, const u32x4& bv, const u32x4& gv,
                                          float r, const float (&c)[4], const float (&sn)[4],
                                          bool rotate, float scale) {
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
      o[2 * p] = __fsub_rn(__fmul_rn(re, c[p]), __fmul_rn(im, sn[p]));
      o[2 * p + 1] = __fadd_rn(__fmul_rn(re, sn[p]), __fmul_rn(im, c[p]));
    }
  } else if (scale != 1.0f) {
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = __fmul_rn(t[e], scale);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = t[e];
  }
  u32x4 ov;
#pragma unroll
  for (int w = 0; w < 4; ++w) ov[w] = pack_bf16x2(o[2 * w], o[2 * w + 1]);
  return ov;
}

// copy the chunks i of a V row with i % nsplit == part (the row's waves share the copy); NT:
// as for qk_load16, the stores too
template <int NCH, bool NT>
__device__ __forceinline__ void qk_copy_v(const QkNormRopeArgs& a, int row, int lane, int part,
                                          int nsplit) {
  const int nchunk = a.C / 8;
  const uint16_t* vs = a.v + a.vs * row;
  uint16_t* vd = a.vo + a.vos * row;
  u32x4 xv[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int ch = lane + 64 * i;
    if (i % nsplit == part && (i + 1 < NCH || ch < nchunk))
      xv[i] = qk_load16<NT>(vs + 8 * ch);
  }
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int ch = lane + 64 * i;
    if (i % nsplit == part && (i + 1 < NCH || ch < nchunk))
      if constexpr (NT) __builtin_nontemporal_store(xv[i], reinterpret_cast<u32x4*>(vd + 8 * ch));
      else *reinterpret_cast<u32x4*>(vd + 8 * ch) = xv[i];
  }
}

// ---------------------------------------------------------------- rows layout
// One wave per (row, tensor): with q and k the workgroup's waves pair up, wave 2j taking row
// j's q and wave 2j + 1 its k (and half of its V copy each). A wave holds one tensor's row, so
// the kernel runs four waves per SIMD and one wave's loads overlap another's arithmetic.
template <int NCH>
__global__ void __launch_bounds__(QK_WAVES * 64)
qk_norm_rope_kernel(const QkNormRopeArgs a) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int C = a.C;
  const int nchunk = C / 8;
  float* tab = smem;
  uint16_t* vec = reinterpret_cast<uint16_t*>(smem + qk_table_floats(a.ntab));
  qk_fill_lds(a, tab, vec);
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int ntens = a.k != nullptr ? 2 : 1;
  const int t = wave % ntens;
  const int rows_per_block = QK_WAVES / ntens;
  const QkTensor u = qk_tensor(a, vec, t);

  for (int row = blockIdx.x * rows_per_block + wave / ntens; row < a.L;
       row += gridDim.x * rows_per_block) {
    QkOne<NCH> s;
    qk_one_load<NCH, false>(a, u, row, lane, s);
    qk_one_norm<NCH>(a, tab, u, row, lane, s);
    uint16_t* o = u.o + u.os * row;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int ch = lane + 64 * i;
      if (i + 1 < NCH || ch < nchunk)
        *reinterpret_cast<u32x4*>(o + 8 * ch) =
            qk_finish(s.x[i], *reinterpret_cast<const u32x4*>(u.bias + 8 * ch),
                      *reinterpret_cast<const u32x4*>(u.gamma + 8 * ch), s.r, s.c, s.sn,
                      s.rotate, u.scale);
    }
    if (a.v != nullptr) qk_copy_v<NCH, false>(a, row, lane, t, ntens);
  }
}

// ---------------------------------------------------------------- d-major layout
template <int NCH>
__global__ void __launch_bounds__(QT_WAVES * 64)
qk_norm_rope_dmajor_kernel(const QkNormRopeArgs a) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  // tile numbering: XCD x (= blockIdx % 8) takes tiles [x * per, (x + 1) * per)
  const int ntile = (a.L + QT_ROWS - 1) / QT_ROWS;
  const int per = (ntile + 7) / 8;
  const int tile = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if (tile >= ntile) return;  // whole workgroup, before any barrier

  const int C = a.C;
  const int nchunk = C / 8;
  float* tab = smem;
  uint16_t* vec = reinterpret_cast<uint16_t*>(smem + qk_table_floats(a.ntab));
  uint16_t* stage = vec + 4 * C;  // [2 tensors][QT_ROWS tokens][QT_PITCH]
  qk_fill_lds(a, tab, vec);
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int ntens = a.k != nullptr ? 2 : 1;
  const int t0 = tile * QT_ROWS;
  const int nvalid = min(QT_ROWS, a.L - t0);
  // (token, tensor) units: with q and k, wave w takes tensor w & 1 of tokens w / 2 and
  // w / 2 + QT_ROWS / 2; with q alone, token w. All loads are issued before any arithmetic.
  const int t = ntens == 2 ? (wave & 1) : 0;
  const int nunit = ntens;
  const int tok0 = ntens == 2 ? (wave >> 1) : wave;
  const QkTensor u = qk_tensor(a, vec, t);
  QkOne<NCH> s[2];
#pragma unroll
  for (int k = 0; k < 2; ++k)
    if (k < nunit && tok0 + (QT_ROWS / 2) * k < nvalid)
      qk_one_load<NCH, true>(a, u, t0 + tok0 + (QT_ROWS / 2) * k, lane, s[k]);
#pragma unroll
  for (int k = 0; k < 2; ++k)
    if (k < nunit && tok0 + (QT_ROWS / 2) * k < nvalid)
      qk_one_norm<NCH>(a, tab, u, t0 + tok0 + (QT_ROWS / 2) * k, lane, s[k]);

  // writer role of this thread: line e of the 512-column slice, tokens [8 * half, 8 * half + 8)
  const int e = threadIdx.x >> 1;
  const int half = threadIdx.x & 1;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int ch = lane + 64 * i;
    if (i + 1 < NCH || ch < nchunk) {
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int tok = tok0 + (QT_ROWS / 2) * k;
        if (k < nunit && tok < nvalid)
          *reinterpret_cast<u32x4*>(stage + (t * QT_ROWS + tok) * QT_PITCH + 8 * lane) =
              qk_finish(s[k].x[i], *reinterpret_cast<const u32x4*>(u.bias + 8 * ch),
                        *reinterpret_cast<const u32x4*>(u.gamma + 8 * ch), s[k].r, s[k].c,
                        s[k].sn, s[k].rotate, u.scale);
      }
    }
    __syncthreads();
    // line e = head * D + d of the slice starts at col * d_stride
    const int col = 512 * i + e;
    if (col < C) {
      for (int tw = 0; tw < ntens; ++tw) {
        const uint16_t* sp = stage + (tw * QT_ROWS + 8 * half) * QT_PITCH + e;
        uint16_t v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = sp[j * QT_PITCH];
        uint16_t* dst = (tw ? a.ko : a.qo) + (int64_t)col * (tw ? a.kos : a.qos) + t0 + 8 * half;
        const bool vec_ok = tw ? a.ko_vec : a.qo_vec;
        if (vec_ok && 8 * half + 8 <= nvalid) {
          u32x4 w;
#pragma unroll
          for (int j = 0; j < 4; ++j) w[j] = (uint32_t)v[2 * j] | ((uint32_t)v[2 * j + 1] << 16);
          *reinterpret_cast<u32x4*>(dst) = w;
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (8 * half + j < nvalid) dst[j] = v[j];
        }
      }
    }
    __syncthreads();  // the slice is read before the next one is staged
  }
  if (a.v != nullptr && wave < nvalid) qk_copy_v<NCH, true>(a, t0 + wave, lane, 0, 1);
}

template <int NCH>
static hipError_t launch_nch(const QkNormRopeArgs& a, hipStream_t stream) {
  if (a.layout == QK_LAYOUT_DMAJOR) {
    if constexpr (NCH > QT_MAX_NCH) return hipErrorInvalidValue;  // rejected by the host check
    static hipError_t attr = hipFuncSetAttribute(
        (const void*)qk_norm_rope_dmajor_kernel<NCH>, hipFuncAttributeMaxDynamicSharedMemorySize,
        (int)(qk_norm_rope_lds_bytes(QK_MAX_TABLE, 64 * 8 * NCH, QK_LAYOUT_DMAJOR) < LDS_LIMIT
                  ? qk_norm_rope_lds_bytes(QK_MAX_TABLE, 64 * 8 * NCH, QK_LAYOUT_DMAJOR)
                  : LDS_LIMIT));
    if (attr != hipSuccess) return attr;
    const int ntile = (a.L + QT_ROWS - 1) / QT_ROWS;
    const int blocks = 8 * ((ntile + 7) / 8);
    hipLaunchKernelGGL(qk_norm_rope_dmajor_kernel<NCH>, dim3(blocks), dim3(QT_WAVES * 64),
                       qk_norm_rope_lds_bytes(a.ntab, a.C, QK_LAYOUT_DMAJOR), stream, a);
    return hipGetLastError();
  }
  static hipError_t attr = hipFuncSetAttribute((const void*)qk_norm_rope_kernel<NCH>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)qk_lds_bytes(QK_MAX_TABLE, 64 * 8 * NCH));
  if (attr != hipSuccess) return attr;
  // at most QK_MAX_BLOCKS workgroups, each wave looping over rows so that the LDS fill is
  // amortised
  const int rows_per_block = a.k != nullptr ? QK_WAVES / 2 : QK_WAVES;
  int blocks = (a.L + rows_per_block - 1) / rows_per_block;
  if (blocks > QK_MAX_BLOCKS) blocks = QK_MAX_BLOCKS;
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
