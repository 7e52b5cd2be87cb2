// Flash-attention forward over a segmented bf16 KV sequence (gfx950), the chunk
// self-attention hot path.
//
// Semantics follow the reference's attention() SDPA path (wan/modules/attention.py:1127-1143)
// with the KV window of wan/modules/model_fast.py:2538-2545 and the chunk list of
// attention.py:1048-1058: out = softmax(scale * Q K^T) V over keys [lo, hi) of the
// concatenated segments; a query row with no keys yields 0 (as torch's SDPA does).
//
// Work decomposition: one workgroup = 4 waves = 256 queries of one (batch, head) and one KV
// split; each wave owns 64 queries (two 32-query MFMA blocks). K and V stream through LDS in
// 64-key tiles with three stages in flight.
//
// Staging: tiles are copied HBM -> LDS by the direct global-to-LDS load (16 bytes per lane,
// no registers, no VALU), K and V both kept row-major ([key][d], 256 B per row). Each 16-byte
// chunk c of row r is stored at chunk c ^ swz(r), swz(r) = 4(r & 3) + ((r >> 2) & 3), which
// makes both LDS read patterns below conflict-free.
//
// Transposed formulation: S^T = K Q^T (A = K rows, ds_read_b128; B = Q from registers) and
// O^T = V^T P^T (A = V^T via the LDS transpose read ds_read_b64_tr_b16; B = P^T straight
// from the S^T accumulators). With the 32x32 MFMA output layout every lane holds one query
// column, so the row max, row sum and O rescale are lane-local plus one exchange with lane^32.
//
// P^T register order: accumulator register r of lane l holds key 8*(r/4) + 4*(l/32) + (r%4)
// of its 32-key block, so the PV MFMA's k-value e of k-group h (registers 8m + e) is key
// 16m + 4h + 8(e/4) + (e%4). The transpose read gives lane i of a 16-lane group the 4 keys
// K..K+3 of column d0 + i when source lane s points at row K + s/4, columns d0 + 4(s%4)..+3;
// two such reads (K = 16m + 4h and 16m + 4h + 8) fill the 8 k-values in exactly that order.
//
// Online softmax in base 2 with the scale folded into one FMA: p = exp2(s*c - m*c),
// c = scale*log2(e). The exponent reference m is only raised when the running max exceeds it
// by more than 8 (log2 units), so P <= 256 and the O rescale is skipped on almost every tile;
// O and l share the reference, so the final O / l is exact.

#include "attn_tiles.h"

namespace lbw {
namespace {

constexpr int BM = 256;                 // queries per workgroup
constexpr int ROWB = D * 2;             // bytes per K/V row in LDS
constexpr int TILE_B = BN * ROWB;       // 16 KB
constexpr int STAGE_B = 2 * TILE_B;     // K tile + V tile
constexpr int NSTAGE = 3;
constexpr int LDS_B = NSTAGE * STAGE_B; // 96 KB

__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

typedef short shortx4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) shortx4 lds_shortx4;
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ u32x2 lds_read_tr16(const unsigned char* p) {
  const shortx4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(p));
  return __builtin_bit_cast(u32x2, v);
}

__device__ __forceinline__ void dma16(const unsigned char* src, unsigned char* lds_dst) {
  __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)(lds_dst), 16, 0, 0);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt_le() {
  if constexpr (N == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else if constexpr (N == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  else static_assert(N == 8 || N == 4, "vmcnt");
}
__device__ __forceinline__ void wait_vmcnt_0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Scores of keys outside the tile's valid rows [tvlo, tvhi) -> -inf (S^T register layout).
// Called only for partial sub-blocks; the empty asm keeps the compiler from speculating the
// masking into the full sub-blocks' path.
__device__ __forceinline__ void mask_scores(floatx16& sc, int kb, int tvlo, int tvhi, int hl) {
  asm volatile("" ::: "memory");
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int key = 32 * kb + 8 * (r >> 2) + 4 * hl + (r & 3);
    if (key < tvlo || key >= tvhi) sc[r] = -INFINITY;
  }
}

// Online-softmax step of one 32-query block over 32 keys, branch-free. Updates the running
// max; when some row of the wave outgrew its exponent reference by more than TAU, every row
// moves its reference to its running max (alpha = the factor O must be scaled by, returned
// with `true`). P = exp2(s c - m c) is packed to bf16 in the PV B-operand order and the row
// sum is rescaled and accumulated.
__device__ __forceinline__ bool softmax_block(const floatx16& sc, float& m_true, float& m_used,
                                              float& lsum, float c, float tau_raw, u32x4 (&pf)[2],
                                              float& alpha) {
  float mx = sc[0];
#pragma unroll
  for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sc[r]);
  mx = wave_max_xor32(mx);
  m_true = fmaxf(m_true, mx);
  const bool move = __any(m_true > m_used + tau_raw);
  const float m_new = move ? m_true : m_used;
  alpha = (!move || m_used == -INFINITY) ? (move ? 0.0f : 1.0f) : fast_exp2((m_used - m_new) * c);
  m_used = m_new;
  // m_used is still -inf only while every key so far was masked: then p = 0.
  const float mc = (m_used == -INFINITY) ? 0.0f : m_used * c;
  float ls = 0.0f;
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float q0 = fast_exp2(__builtin_fmaf(sc[8 * m + 2 * e], c, -mc));
      const float q1 = fast_exp2(__builtin_fmaf(sc[8 * m + 2 * e + 1], c, -mc));
      w[e] = pack_bf16x2(q0, q1);
      ls += q0 + q1;
    }
    pf[m] = w;
  }
  lsum = __builtin_fmaf(lsum, alpha, ls);
  return move;
}

__device__ __forceinline__ void scale_acc(floatx16 (&o)[4], float alpha) {
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
}

// NW waves per workgroup: 4 (64 queries = two 32-query blocks per wave, one wave per SIMD,
// block-level interleaving in software) or 8 (32 queries per wave, two waves per SIMD that the
// hardware interleaves).
template <int NW>
__global__ void __launch_bounds__(NW * 64, 1)
attn_fwd_bf16_kernel(const AttnKernelArgs a) {
  constexpr int QB = 8 / NW;        // 32-query blocks per wave
  constexpr int NDMA = 16 / NW;     // 1 KB DMA blocks per wave per K (and per V) tile
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
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

  const int q0 = qt * BM + wave * 32 * QB;  // first query of this wave (wave-uniform)
  const bool wave_active = q0 < a.Lq;

  // ---- Q fragments (B operand of S^T = K Q^T): qf[qb][s] holds d = 16s + 8hl .. +7
  u32x4 qf[QB][8];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int q = q0 + 32 * qb + l32;
    const uint16_t* qp = a.q + a.qsb * b + a.qsl * (int64_t)q + a.qsh * h + 8 * hl;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (q < a.Lq) v = *reinterpret_cast<const u32x4*>(qp + 16 * s);
      qf[qb][s] = v;
    }
  }

  // ---- per-lane LDS offsets
  // DMA: this wave fills 1 KB blocks NDMA*wave + i of each tile; lane -> (row, physical chunk).
  int dma_row[NDMA], dma_col[NDMA];
#pragma unroll
  for (int i = 0; i < NDMA; ++i) {
    dma_row[i] = 4 * (NDMA * wave + i) + (lane >> 4);
    dma_col[i] = ((lane & 15) ^ swz(dma_row[i])) * 16;  // byte offset of the logical chunk
  }
  // K fragment (kb = 0) for d-slice s: row l32, logical chunk 2s + hl.
  int koff[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) koff[s] = l32 * ROWB + (((2 * s + hl) ^ swz(l32)) << 4);
  // V transpose reads (kb = m = 0) for d-block db and key half j: source row
  // 4hl + 8j + s/4, columns 32db + 16g + 4(s%4) .. +3 (s = lane % 16, g = (lane / 16) % 2).
  int voff[4][2];
  {
    const int s16 = lane & 15, g = (lane >> 4) & 1;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int r = 4 * hl + 8 * j + (s16 >> 2);
        const int lc = 4 * db + 2 * g + ((s16 & 3) >> 1);
        voff[db][j] = r * ROWB + ((lc ^ swz(r)) << 4) + 8 * (s16 & 1);
      }
  }

  floatx16 oacc[QB][4];
  float m_used[QB], m_true[QB], lsum[QB];  // exponent reference, running row max, row sum
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[qb][db][r] = 0.0f;
    m_used[qb] = -INFINITY;
    m_true[qb] = -INFINITY;
    lsum[qb] = 0.0f;
  }
  const float c = a.scale_log2;
  const float tau_raw = TAU / c;

  // DMA of the cursor's tile into a stage (2*NDMA x 16 B per lane). Full tiles use the
  // per-segment lane offsets; in a partial tile, rows outside the valid range [vlo, vhi)
  // fetch a valid row instead: their scores are masked to -inf and their probabilities are
  // exactly 0, so the duplicate never contributes.
  TileCursor cs;
  uint32_t lane_k[NDMA], lane_v[NDMA];
  auto seg_offsets = [&]() {
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      lane_k[i] = (uint32_t)(dma_row[i] * cs.ks + dma_col[i]);
      lane_v[i] = (uint32_t)(dma_row[i] * cs.vs + dma_col[i]);
    }
  };
  auto issue = [&](unsigned char* stage, int& tvlo, int& tvhi) {
    cursor_rows(cs, tvlo, tvhi);
    const int64_t row0 = cs.lt * BN;
    const unsigned char* kb = cs.kbase + row0 * cs.ks;
    const unsigned char* vb = cs.vbase + row0 * cs.vs;
    if (tvlo == 0 && tvhi == BN) {
#pragma unroll
      for (int i = 0; i < NDMA; ++i) {
        dma16(kb + lane_k[i], stage + 1024 * (NDMA * wave + i));
        dma16(vb + lane_v[i], stage + TILE_B + 1024 * (NDMA * wave + i));
      }
    } else {
      const int rhi = tvhi - 1;
#pragma unroll
      for (int i = 0; i < NDMA; ++i) {
        int r = dma_row[i];
        r = r < tvlo ? tvlo : (r > rhi ? rhi : r);
        dma16(kb + r * cs.ks + dma_col[i], stage + 1024 * (NDMA * wave + i));
        dma16(vb + r * cs.vs + dma_col[i], stage + TILE_B + 1024 * (NDMA * wave + i));
      }
    }
    if (cursor_next<2>(a, lo, hi, b, h, cs) && cs.seg < a.nseg) seg_offsets();
  };

  if (t0 < t1) {
    // valid-row ranges of the tiles in flight: [0] = current, [1] = next, [2] = after next
    int vlo[3] = {0, 0, 0}, vhi[3] = {BN, BN, BN};
    cursor_init<2>(a, lo, hi, t0, b, h, cs);
    seg_offsets();
    issue(lds, vlo[0], vhi[0]);
    if (t0 + 1 < t1) {
      issue(lds + STAGE_B, vlo[1], vhi[1]);
      wait_vmcnt_le<2 * NDMA>();
    } else {
      wait_vmcnt_0();
    }
    barrier_nofence();

    int st = 0;  // stage of tile t
    for (int t = t0; t < t1; ++t) {
      unsigned char* cur = lds + st * STAGE_B;
      const bool has2 = (t + 2) < t1;
      if (has2) {
        const int st2 = st >= 1 ? st - 1 : 2;  // (st + 2) % 3
        issue(lds + st2 * STAGE_B, vlo[2], vhi[2]);
      }

      if (wave_active) {
        const int tvlo = vlo[0], tvhi = vhi[0];
        const unsigned char* vt0 = cur + TILE_B;
        auto vfrag = [&](const unsigned char* vt, int db, int m) {
          const unsigned char* vb = vt + 16 * m * ROWB;
          const u32x2 v0 = lds_read_tr16(vb + voff[db][0]);
          const u32x2 v1 = lds_read_tr16(vb + voff[db][1]);
          return u32x4{v0[0], v0[1], v1[0], v1[1]};
        };
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const unsigned char* kt = cur + kb * 32 * ROWB;
          const unsigned char* vt = vt0 + kb * 32 * ROWB;
          const bool partial = tvlo > 32 * kb || tvhi < 32 * kb + 32;
          if constexpr (QB == 2) {
            // phase 1: S0 = K Q0^T
            u32x4 kf[8];
#pragma unroll
            for (int s = 0; s < 8; ++s) kf[s] = *reinterpret_cast<const u32x4*>(kt + koff[s]);
            floatx16 s0, s1;
#pragma unroll
            for (int r = 0; r < 16; ++r) { s0[r] = 0.0f; s1[r] = 0.0f; }
#pragma unroll
            for (int s = 0; s < 8; ++s) s0 = mfma32x32x16(kf[s], qf[0][s], s0);
            if (partial) mask_scores(s0, kb, tvlo, tvhi, hl);
            // phase 2: S1 = K Q1^T  |  softmax of query block 0
#pragma unroll
            for (int s = 0; s < 8; ++s) s1 = mfma32x32x16(kf[s], qf[QB - 1][s], s1);
            u32x4 p0[2];
            float alpha0;
            const bool r0 = softmax_block(s0, m_true[0], m_used[0], lsum[0], c, tau_raw, p0, alpha0);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
              __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);  // 8 VALU
            }
            if (partial) mask_scores(s1, kb, tvlo, tvhi, hl);
            if (r0) scale_acc(oacc[0], alpha0);
            // phase 3: O0 += V^T P0^T  |  softmax of query block 1
            u32x4 vf[4][2];
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
              for (int m = 0; m < 2; ++m) vf[db][m] = vfrag(vt, db, m);
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
              for (int m = 0; m < 2; ++m) oacc[0][db] = mfma32x32x16(vf[db][m], p0[m], oacc[0][db]);
            u32x4 p1[2];
            float alpha1;
            const bool r1 = softmax_block(s1, m_true[QB - 1], m_used[QB - 1], lsum[QB - 1], c,
                                          tau_raw, p1, alpha1);
            __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);   // the V transpose reads first
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
              __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
            }
            if (r1) scale_acc(oacc[QB - 1], alpha1);
            // phase 4: O1 += V^T P1^T
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
              for (int m = 0; m < 2; ++m)
                oacc[QB - 1][db] = mfma32x32x16(vf[db][m], p1[m], oacc[QB - 1][db]);
          } else {
            // one 32-query block: S = K Q^T, softmax, O += V^T P^T (the other wave on this
            // SIMD fills the gaps)
            floatx16 s0;
#pragma unroll
            for (int r = 0; r < 16; ++r) s0[r] = 0.0f;
#pragma unroll
            for (int s = 0; s < 8; ++s)
              s0 = mfma32x32x16(*reinterpret_cast<const u32x4*>(kt + koff[s]), qf[0][s], s0);
            if (partial) mask_scores(s0, kb, tvlo, tvhi, hl);
            u32x4 p0[2];
            float alpha0;
            const bool r0 = softmax_block(s0, m_true[0], m_used[0], lsum[0], c, tau_raw, p0, alpha0);
            if (r0) scale_acc(oacc[0], alpha0);
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
              for (int m = 0; m < 2; ++m)
                oacc[0][db] = mfma32x32x16(vfrag(vt, db, m), p0[m], oacc[0][db]);
          }
        }
      }

      // tile t+1 must be in LDS for every wave before the next iteration
      if (has2) wait_vmcnt_le<2 * NDMA>(); else wait_vmcnt_0();
      barrier_nofence();
      vlo[0] = vlo[1]; vhi[0] = vhi[1];
      vlo[1] = vlo[2]; vhi[1] = vhi[2];
      st = st == 2 ? 0 : st + 1;
    }
  }

  if (!wave_active) return;

  // ---- epilogue
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
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

}  // namespace

template <int NW>
static hipError_t launch_nw(const AttnKernelArgs& a, hipStream_t stream) {
  static hipError_t attr = hipFuncSetAttribute((const void*)attn_fwd_bf16_kernel<NW>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, LDS_B);
  if (attr != hipSuccess) return attr;
  const uint32_t nwg = (uint32_t)a.n_qtiles * a.splits * a.H * a.B;
  hipLaunchKernelGGL(attn_fwd_bf16_kernel<NW>, dim3(nwg), dim3(NW * 64), LDS_B, stream, a);
  return hipGetLastError();
}

#ifndef LBW_ATTN_WAVES
#define LBW_ATTN_WAVES 8
#endif

hipError_t launch_attn_fwd(const AttnKernelArgs& a, hipStream_t stream) {
  return launch_nw<LBW_ATTN_WAVES>(a, stream);
}

}  // namespace lbw
