// Flash-attention forward for a chunk of queries over a segmented KV sequence (gfx950).
//
// Semantics follow the reference's attention() SDPA path (wan/modules/attention.py:1127-1143)
// with the KV window of wan/modules/model_fast.py:2538-2545 and the chunk list of
// attention.py:1048-1058: out = softmax(scale * Q K^T) V over keys [lo, hi) of the
// concatenated segments; a query row with no keys yields 0 (as torch's SDPA does).
//
// Work decomposition: one workgroup = 4 waves = 256 queries of one (batch, head) and one KV
// split. Each wave owns 64 queries (two 32-query MFMA blocks). K/V stream through LDS in
// 64-key tiles, double buffered, one barrier per tile. Tiles are aligned to each segment's
// own token index (a tile never straddles two segments), so a tile has one base pointer and,
// for the fp8 cache, exactly one K and one V scale (the 64-token scale block).
//
// Transposed formulation: S^T = K Q^T (A = K tile from LDS, B = Q from registers) and
// O^T = V^T P^T (A = V^T from LDS, B = P^T straight from the S^T accumulators). With the
// 32x32 MFMA output layout every lane then holds one query column, so the row max, the
// row sum and the O rescale are lane-local (plus one exchange with lane ^ 32).
//
// P^T register order: accumulator register r of lane l holds key 8*(r/4) + 4*(l/32) + (r%4)
// of its 32-key block. The PV MFMA consumes registers 8m..8m+7 as its 8 k-values, so V^T is
// stored in LDS with the key order that matches: position 32kb + 16m + 8h + e holds key
// 32kb + 16m + 4h + 8(e/4) + (e%4). That is bits 2 and 3 of the in-tile key index swapped,
// which keeps runs of 4 consecutive keys contiguous, so the transposing LDS store is one
// 8-byte write per (d, key quad).
//
// Online softmax in base 2 with the scale folded into one FMA: p = exp2(s*cc - m*c) with
// c = scale*log2(e) and cc = c times the fp8 dequantisation factors. The running max used
// for the exponent is only raised when the true max exceeds it by more than 8 (log2 units),
// so P stays <= 256 and the O rescale (128 multiplies per lane) is skipped on almost every
// tile; the final normalisation divides O and l by the same exponent reference, so the
// result is exact.
//
// fp8 KV (e4m3fn codes, per-(b, h, 64-token block) fp32 scales): Q is quantised per query
// row in-kernel (scale = amax/448) and QK^T runs on the fp8 MFMA (32x32x64); the score
// dequantisation (q scale x k block scale) is folded into cc. V is dequantised (x its block
// scale) to bf16 on its way into LDS and PV runs on the bf16 MFMA.

#include "attn_tiles.h"

namespace lbw {

constexpr int BM = 256;
constexpr int NT = 256;
constexpr int VT_ROW = BN * 2 + 16;  // LDS bytes per V^T row (16 B pad: conflict-free reads)
constexpr int VT_BYTES = D * VT_ROW;
constexpr float TWO_POW_120 = 1.329227995784916e36f;

template <bool FP8>
struct Cfg {
  static constexpr int ESZ = FP8 ? 1 : 2;              // bytes per K/V element
  static constexpr int K_ROW = D * ESZ + 16;           // LDS bytes per K row
  static constexpr int K_BYTES = BN * K_ROW;
  static constexpr int BUF = K_BYTES + VT_BYTES;
  static constexpr int LDS = 2 * BUF;
};

// ------------------------------------------------------------------ global -> LDS staging
template <bool FP8>
struct TileRegs;
template <>
struct TileRegs<false> {
  u32x4 k[4];
  u32x4 v[4];
};
template <>
struct TileRegs<true> {
  u32x4 k[2];
  u32x2 v[4];
};

// bf16 K: thread t loads rows (t>>4) + 16i, 16-byte column t&15.
// fp8  K: thread t loads rows (t>>3) + 32i, 16-byte column t&7.
// V (both): thread t loads keys 4(t>>4) + i, d octet t&15.
// Rows outside the tile's valid range [vlo, vhi) load a valid row instead (clamped): their
// scores are masked to -inf and their probabilities are exactly 0, so the duplicate data
// never contributes, and no load waits on a branch or a select of its result.
template <bool FP8>
__device__ __forceinline__ void load_tile(const TileInfo& ti, TileRegs<FP8>& tr) {
  const int t = threadIdx.x;
  const int hi_row = ti.vhi - 1;
  auto row_addr = [&](const unsigned char* base, int64_t stride, int r) {
    r = r < ti.vlo ? ti.vlo : (r > hi_row ? hi_row : r);
    return base + (ti.row0 + r) * stride;
  };
  if constexpr (!FP8) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      tr.k[i] = *reinterpret_cast<const u32x4*>(row_addr(ti.kbase, ti.ks, (t >> 4) + 16 * i) + (t & 15) * 16);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      tr.v[i] = *reinterpret_cast<const u32x4*>(row_addr(ti.vbase, ti.vs, 4 * (t >> 4) + i) + (t & 15) * 16);
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      tr.k[i] = *reinterpret_cast<const u32x4*>(row_addr(ti.kbase, ti.ks, (t >> 3) + 32 * i) + (t & 7) * 16);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      tr.v[i] = *reinterpret_cast<const u32x2*>(row_addr(ti.vbase, ti.vs, 4 * (t >> 4) + i) + (t & 15) * 8);
  }
}

__device__ __forceinline__ uint32_t sel_lo(uint32_t a, uint32_t b) {  // (a.lo16, b.lo16)
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t sel_hi(uint32_t a, uint32_t b) {  // (a.hi16, b.hi16)
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// e4m3fn code (in byte `e` of w) -> fp32 times `f`, where f already carries 2^120: the code's
// 7 magnitude bits placed at float bits 20..26 read as 2^(e-127) * 1.mmm (or the denormal
// m * 2^-129), and 2^120 rebiases that to the e4m3 value.
__device__ __forceinline__ float e4m3_to_f32_scaled(uint32_t w, int e, float f) {
  const uint32_t c = (w >> (8 * e)) & 0xffu;
  const uint32_t bits = ((c & 0x80u) << 24) | ((c & 0x7fu) << 20);
  return __uint_as_float(bits) * f;
}

// V quad position in the P^T key order (see the file comment).
__device__ __forceinline__ int vt_pos0(int quad) {
  return 32 * (quad >> 3) + 16 * ((quad >> 2) & 1) + 8 * (quad & 1) + 4 * ((quad >> 1) & 1);
}

template <bool FP8>
__device__ __forceinline__ void store_tile(unsigned char* buf, const TileRegs<FP8>& tr, float sv) {
  const int t = threadIdx.x;
  const int quad = t >> 4;
  const int col = t & 15;
  unsigned char* vt = buf + Cfg<FP8>::K_BYTES;
  const int pos0 = vt_pos0(quad);
  if constexpr (!FP8) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<u32x4*>(buf + ((t >> 4) + 16 * i) * Cfg<FP8>::K_ROW + col * 16) = tr.k[i];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      u32x2 lo, hi;
      lo[0] = sel_lo(tr.v[0][w], tr.v[1][w]);
      lo[1] = sel_lo(tr.v[2][w], tr.v[3][w]);
      hi[0] = sel_hi(tr.v[0][w], tr.v[1][w]);
      hi[1] = sel_hi(tr.v[2][w], tr.v[3][w]);
      const int d = 8 * col + 2 * w;
      *reinterpret_cast<u32x2*>(vt + d * VT_ROW + pos0 * 2) = lo;
      *reinterpret_cast<u32x2*>(vt + (d + 1) * VT_ROW + pos0 * 2) = hi;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      *reinterpret_cast<u32x4*>(buf + ((t >> 3) + 32 * i) * Cfg<FP8>::K_ROW + (t & 7) * 16) = tr.k[i];
    const float f = sv * TWO_POW_120;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t w = e >> 2;
      const int be = e & 3;
      u32x2 o;
      o[0] = pack_bf16x2(e4m3_to_f32_scaled(tr.v[0][w], be, f), e4m3_to_f32_scaled(tr.v[1][w], be, f));
      o[1] = pack_bf16x2(e4m3_to_f32_scaled(tr.v[2][w], be, f), e4m3_to_f32_scaled(tr.v[3][w], be, f));
      *reinterpret_cast<u32x2*>(vt + (8 * col + e) * VT_ROW + pos0 * 2) = o;
    }
  }
}

// fp32 -> e4m3fn code (round to nearest even), for in-range values (|x| <= 448).
__device__ __forceinline__ uint32_t e4m3_encode(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t au = u & 0x7fffffffu;
  if (au < 0x3c800000u) return sign | (uint32_t)__float2int_rn(__uint_as_float(au) * 512.0f);
  const uint32_t r = au + 0x7ffffu + ((au >> 20) & 1u);
  const uint32_t code = (r >> 20) - (120u << 3);
  return sign | (code > 0x7eu ? 0x7eu : code);
}

// e4m3fn code -> its value as fp32 (exact), via the same bit placement as e4m3_to_f32_scaled.
__device__ __forceinline__ float e4m3_value(uint32_t c) {
  return __uint_as_float(((c & 0x80u) << 24) | ((c & 0x7fu) << 20)) * TWO_POW_120;
}

// ------------------------------------------------------------------ the kernel
template <bool FP8>
__global__ void __launch_bounds__(NT, 1)
attn_fwd_kernel(const AttnKernelArgs a) {
  using C = Cfg<FP8>;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hl = lane >> 5;  // k-group / row-half of this lane
  const int l32 = lane & 31;

  // ---- work item: (batch, head, split, q-tile), q-tile fastest, XCD-aware order
  const uint32_t id = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = id % a.n_qtiles;
  uint32_t rest = id / a.n_qtiles;
  const int split = rest % a.splits;
  rest /= a.splits;
  const int h = rest % a.H;
  const int b = rest / a.H;

  // ---- key range of this batch and split
  int64_t hi = a.hi;
  if (a.k_lens != nullptr) {
    const int64_t kl = a.k_lens[b];
    hi = kl < hi ? kl : hi;
  }
  const int64_t lo = a.lo;
  const int n_tiles = hi > lo ? count_tiles(a, lo, hi) : 0;
  const int per_split = (n_tiles + a.splits - 1) / a.splits;
  const int t0 = split * per_split;
  const int t1 = min(n_tiles, t0 + per_split);

  const int q0 = qt * BM + wave * 64;  // first query of this wave (wave-uniform)
  const bool wave_active = q0 < a.Lq;

  // ---- Q fragments (B operand of S^T = K Q^T)
  // bf16: qf[qb][s], d = 16s + 8hl .. +7.
  // fp8:  q = sq * (hi + lo/16) with hi, lo e4m3 codes; qf[qb][2s + j] holds hi codes of
  //       d = 64s + 32hl + 16j .. +15, qf[qb][4 + 2s + j] the lo codes of the same d.
  u32x4 qf[2][8];
  float qscale[2] = {1.0f, 1.0f};
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int q = q0 + 32 * qb + l32;
    const bool qv = q < a.Lq;
    if constexpr (!FP8) {
      const uint16_t* qp = a.q + a.qsb * b + a.qsl * (int64_t)q + a.qsh * h + 8 * hl;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        u32x4 v = {0u, 0u, 0u, 0u};
        if (qv) v = *reinterpret_cast<const u32x4*>(qp + 16 * s);
        qf[qb][s] = v;
      }
    } else {
      const uint16_t* qp = a.q + a.qsb * b + a.qsl * (int64_t)q + a.qsh * h + 32 * hl;
      u32x4 raw[8];  // raw[4s + c]: d = 64s + 32hl + 8c .. +7
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        u32x4 v = {0u, 0u, 0u, 0u};
        if (qv) v = *reinterpret_cast<const u32x4*>(qp + 64 * (i >> 2) + 8 * (i & 3));
        raw[i] = v;
      }
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int w = 0; w < 4; ++w)
          amax = fmaxf(amax, fmaxf(fabsf(bf16_lo(raw[i][w])), fabsf(bf16_hi(raw[i][w]))));
      amax = fmaxf(amax, __shfl_xor(amax, 32));
      const float sq = amax > 0.0f ? amax / 448.0f : 1.0f;
      const float inv = 1.0f / sq;
      qscale[qb] = sq;
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int dw = 0; dw < 8; ++dw) {  // dword dw of slice s: d offsets 4dw .. 4dw+3
          const u32x4& r = raw[4 * s + (dw >> 1)];
          const int w0 = (dw & 1) * 2;
          const float y[4] = {bf16_lo(r[w0]) * inv, bf16_hi(r[w0]) * inv,
                              bf16_lo(r[w0 + 1]) * inv, bf16_hi(r[w0 + 1]) * inv};
          uint32_t hw = 0, lw = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t hc = e4m3_encode(y[e]);
            const uint32_t lc = e4m3_encode((y[e] - e4m3_value(hc)) * 16.0f);
            hw |= hc << (8 * e);
            lw |= lc << (8 * e);
          }
          qf[qb][2 * s + (dw >> 2)][dw & 3] = hw;
          qf[qb][4 + 2 * s + (dw >> 2)][dw & 3] = lw;
        }
    }
  }

  floatx16 oacc[2][4];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[qb][db][r] = 0.0f;
  float m_used[2] = {-INFINITY, -INFINITY};  // exponent reference (true-score units)
  float m_true[2] = {-INFINITY, -INFINITY};  // running row max (true-score units)
  float lsum[2] = {0.0f, 0.0f};
  const float c = a.scale_log2;
  const float tau_raw = TAU / c;

  if (t0 < t1) {
    TileRegs<FP8> tr;
    TileInfo ti = tile_info<Cfg<FP8>::ESZ, FP8>(a, lo, hi, t0, b, h);
    load_tile<FP8>(ti, tr);
    store_tile<FP8>(lds, tr, ti.sv);
    __syncthreads();

    for (int t = t0; t < t1; ++t) {
      unsigned char* cur = lds + ((t - t0) & 1) * C::BUF;
      unsigned char* nxt = lds + ((t - t0 + 1) & 1) * C::BUF;
      const int vlo = ti.vlo, vhi = ti.vhi;
      const float sk = ti.sk;
      const bool has_next = (t + 1) < t1;
      if (has_next) {
        ti = tile_info<Cfg<FP8>::ESZ, FP8>(a, lo, hi, t + 1, b, h);
        load_tile<FP8>(ti, tr);
      }

      if (wave_active) {
        const unsigned char* vt = cur + C::K_BYTES;
        // Two 32-key sub-blocks per tile, one online-softmax step each.
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          // ---- S^T[qb] = K[kb] Q[qb]^T (32 keys x 32 queries per qb)
          floatx16 sacc[2];
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[qb][r] = 0.0f;
          if constexpr (!FP8) {
#pragma unroll
            for (int s = 0; s < 8; ++s) {
              const u32x4 kf = *reinterpret_cast<const u32x4*>(
                  cur + (32 * kb + l32) * C::K_ROW + (16 * s + 8 * hl) * 2);
#pragma unroll
              for (int qb = 0; qb < 2; ++qb) sacc[qb] = mfma32x32x16(kf, qf[qb][s], sacc[qb]);
            }
          } else {
#pragma unroll
            for (int s = 0; s < 2; ++s) {
              const unsigned char* kp = cur + (32 * kb + l32) * C::K_ROW + 64 * s + 32 * hl;
              const u32x4 k0 = *reinterpret_cast<const u32x4*>(kp);
              const u32x4 k1 = *reinterpret_cast<const u32x4*>(kp + 16);
              const i32x8 kf = {(int)k0[0], (int)k0[1], (int)k0[2], (int)k0[3],
                                (int)k1[0], (int)k1[1], (int)k1[2], (int)k1[3]};
#pragma unroll
              for (int qb = 0; qb < 2; ++qb) {
                const u32x4& h0 = qf[qb][2 * s];
                const u32x4& h1 = qf[qb][2 * s + 1];
                const u32x4& l0 = qf[qb][4 + 2 * s];
                const u32x4& l1 = qf[qb][4 + 2 * s + 1];
                const i32x8 qh = {(int)h0[0], (int)h0[1], (int)h0[2], (int)h0[3],
                                  (int)h1[0], (int)h1[1], (int)h1[2], (int)h1[3]};
                const i32x8 ql = {(int)l0[0], (int)l0[1], (int)l0[2], (int)l0[3],
                                  (int)l1[0], (int)l1[1], (int)l1[2], (int)l1[3]};
                // e8m0 operand scales: 127 = 1, 123 = 2^-4 (the lo part was scaled by 16)
                sacc[qb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                    kf, qh, sacc[qb], 0, 0, 0, 127, 0, 127);
                sacc[qb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                    kf, ql, sacc[qb], 0, 0, 0, 127, 0, 123);
              }
            }
          }
          if (vlo > 32 * kb || vhi < 32 * kb + 32) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int key = 32 * kb + 8 * (r >> 2) + 4 * hl + (r & 3);
              if (key < vlo || key >= vhi) {
                sacc[0][r] = -INFINITY;
                sacc[1][r] = -INFINITY;
              }
            }
          }
          // ---- online softmax (lazy rescale)
          float cc[2];
          bool need = false;
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) {
            const float dq = FP8 ? qscale[qb] * sk : 1.0f;  // raw score -> true score
            cc[qb] = c * dq;
            float mx = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[qb][r]);
            mx = wave_max_xor32(mx) * dq;
            m_true[qb] = fmaxf(m_true[qb], mx);
            need |= (m_true[qb] > m_used[qb] + tau_raw);
          }
          // P = exp2(S cc - m c) to bf16 (fp32 row sums), then O^T[db][qb] += V^T[db, kb] P^T[qb].
          auto pv = [&]() {
            u32x4 pf[2][2];  // [qb][m]
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) {
              // m_used is still -inf only while every key so far was masked: then p = 0.
              const float mc = (m_used[qb] == -INFINITY) ? 0.0f : m_used[qb] * c;
              float ls = lsum[qb];
#pragma unroll
              for (int m = 0; m < 2; ++m) {
                u32x4 w;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                  const float p0 = fast_exp2(__builtin_fmaf(sacc[qb][8 * m + 2 * e], cc[qb], -mc));
                  const float p1 = fast_exp2(__builtin_fmaf(sacc[qb][8 * m + 2 * e + 1], cc[qb], -mc));
                  w[e] = pack_bf16x2(p0, p1);
                  ls += p0 + p1;
                }
                pf[qb][m] = w;
              }
              lsum[qb] = ls;
            }
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
              for (int m = 0; m < 2; ++m) {
                const u32x4 vf = *reinterpret_cast<const u32x4*>(
                    vt + (32 * db + l32) * VT_ROW + (32 * kb + 16 * m + 8 * hl) * 2);
#pragma unroll
                for (int qb = 0; qb < 2; ++qb)
                  oacc[qb][db] = mfma32x32x16(vf, pf[qb][m], oacc[qb][db]);
              }
          };
          if (__any(need)) {
            // Rare: the row max outgrew the exponent reference. Rescale O and l first.
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) {
              const float alpha =
                  (m_used[qb] == -INFINITY) ? 0.0f : fast_exp2((m_used[qb] - m_true[qb]) * c);
              m_used[qb] = m_true[qb];
              lsum[qb] *= alpha;
#pragma unroll
              for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) oacc[qb][db][r] *= alpha;
            }
          }
          pv();
        }
      }

      if (has_next) store_tile<FP8>(nxt, tr, ti.sv);
      __syncthreads();
    }
  }

  if (!wave_active) return;

  // ---- epilogue
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int q = q0 + 32 * qb + l32;
    const float l_tot = wave_sum_xor32(lsum[qb]);
    if (a.mode == kModeNormalized) {
      const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
      if (q < a.Lq) {
        uint16_t* op = a.out + a.osb * b + a.osl * (int64_t)q + a.osh * h;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int d0 = 32 * db + 8 * g + 4 * hl;
            u32x2 w;
            w[0] = pack_bf16x2(oacc[qb][db][4 * g + 0] * inv, oacc[qb][db][4 * g + 1] * inv);
            w[1] = pack_bf16x2(oacc[qb][db][4 * g + 2] * inv, oacc[qb][db][4 * g + 3] * inv);
            *reinterpret_cast<u32x2*>(op + d0) = w;
          }
      }
    } else {
      // cte_partial contract: O and l relative to the true row max, m in scaled units.
      float f = 1.0f;
      float m_out = -INFINITY;
      if (l_tot > 0.0f) {
        f = fast_exp2((m_used[qb] - m_true[qb]) * c);
        m_out = m_true[qb] * a.scale;
      }
      if (q < a.Lq) {
        const int64_t row = ((int64_t)(split * a.B + b) * a.H + h) * a.Lq + q;
        float* po = a.part_o + row * D;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int d0 = 32 * db + 8 * g + 4 * hl;
            floatx4 w;
            w[0] = oacc[qb][db][4 * g + 0] * f;
            w[1] = oacc[qb][db][4 * g + 1] * f;
            w[2] = oacc[qb][db][4 * g + 2] * f;
            w[3] = oacc[qb][db][4 * g + 3] * f;
            *reinterpret_cast<floatx4*>(po + d0) = w;
          }
        if (hl == 0) {
          a.part_m[row] = m_out;
          a.part_l[row] = l_tot * f;
        }
      }
    }
  }
}

// Log-sum-exp merge of `n` partials: one thread per (b, h, q, 4 d's).
__global__ void __launch_bounds__(256)
attn_merge_kernel(const MergeKernelArgs a) {
  const int64_t total = (int64_t)a.B * a.H * a.Lq * (a.D / 4);
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int dq = (int)(i % (a.D / 4));
    const int64_t row = i / (a.D / 4);  // (b*H + h)*Lq + q
    const int q = (int)(row % a.Lq);
    const int64_t bh = row / a.Lq;
    const int h = (int)(bh % a.H);
    const int b = (int)(bh / a.H);
    float M = -INFINITY;
    for (int s = 0; s < a.n; ++s) M = fmaxf(M, a.m[s][row]);
    float den = 0.0f;
    floatx4 num = {0.f, 0.f, 0.f, 0.f};
    if (M != -INFINITY) {
      for (int s = 0; s < a.n; ++s) {
        const float ms = a.m[s][row];
        const float w = (ms == -INFINITY) ? 0.0f : expf(ms - M);
        den += w * a.l[s][row];
        const floatx4 o = *reinterpret_cast<const floatx4*>(a.o[s] + row * a.D + 4 * dq);
        num += w * o;
      }
    }
    const float inv = den > 0.0f ? 1.0f / den : 0.0f;
    uint16_t* op = a.out + a.osb * b + a.osl * (int64_t)q + a.osh * h + 4 * dq;
    u32x2 w;
    w[0] = pack_bf16x2(num[0] * inv, num[1] * inv);
    w[1] = pack_bf16x2(num[2] * inv, num[3] * inv);
    *reinterpret_cast<u32x2*>(op) = w;
  }
}

// ------------------------------------------------------------------------------ launchers
int attn_block_m() { return BM; }
int attn_block_n() { return BN; }

template <bool FP8>
static hipError_t launch_impl(const AttnKernelArgs& a, hipStream_t stream) {
  static hipError_t attr = hipFuncSetAttribute((const void*)attn_fwd_kernel<FP8>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               Cfg<FP8>::LDS);
  if (attr != hipSuccess) return attr;
  const uint32_t nwg = (uint32_t)a.n_qtiles * a.splits * a.H * a.B;
  hipLaunchKernelGGL(attn_fwd_kernel<FP8>, dim3(nwg), dim3(NT), Cfg<FP8>::LDS, stream, a);
  return hipGetLastError();
}

hipError_t launch_attn_fwd_fp8(const AttnKernelArgs& a, hipStream_t stream) {
  return launch_impl<true>(a, stream);
}

hipError_t launch_attn_merge(const MergeKernelArgs& a, hipStream_t stream) {
  const int64_t total = (int64_t)a.B * a.H * a.Lq * (a.D / 4);
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(attn_merge_kernel, dim3((uint32_t)blocks), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace lbw
