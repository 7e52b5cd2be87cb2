// Flash-attention forward over a segmented bf16 KV sequence (gfx950), the chunk
// self-attention hot path.
//
// Semantics follow the reference's attention() SDPA path (wan/modules/attention.py:1127-1143)
// with the KV window of wan/modules/model_fast.py:2538-2545 and the chunk list of
// attention.py:1048-1058: out = softmax(scale * Q K^T) V over keys [lo, hi) of the
// concatenated segments; a query row with no keys yields 0 (as torch's SDPA does).
//
// Work decomposition: one workgroup = 8 waves = 256 queries of one (batch, head) and one KV
// split; each wave owns 32 queries, two waves share a SIMD. K and V stream through LDS in
// 64-key tiles, NSTAGE tiles resident or in flight.
//
// Staging: tiles are copied HBM -> LDS by the direct global-to-LDS load (16 bytes per lane,
// no registers, no VALU), K and V both kept row-major ([key][d], 256 B per row). Each 16-byte
// chunk c of row r is stored at chunk c ^ swz(r), swz(r) = 4(r & 3) + ((r >> 2) & 3), which
// makes both LDS read patterns below conflict-free. The K tiles of all stages sit in the
// first 64 KB and the V tiles from 64 KB on, so with the stage known at compile time every
// LDS read is a per-lane base register plus an immediate offset.
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
// Software pipeline (per wave, 32-key sub-blocks j): step j computes the softmax of S_j
// (VALU) while the MFMA pipe runs O += V_{j-1}^T P_{j-1}^T and S_{j+1} = K_{j+1} Q^T, so the
// VALU and MFMA work of one wave overlap; the second wave on the SIMD fills what is left.
//
// Online softmax in base 2 with the scale folded into one FMA: p = exp2(s*c - m*c),
// c = scale*log2(e), against an exponent reference m that moves lazily (the redo in the step);
// O and l share the reference, so the final O / l is exact. With a pre-scaled q (c == 1) the
// QK chain starts from -m and p = exp2(S) directly.

#include "attn_tiles.h"

namespace lbw {
namespace {


constexpr int NWAVE = 8;                // waves per workgroup (32 queries each)
constexpr int BM = 32 * NWAVE;          // queries per workgroup
constexpr int ROWB = D * 2;             // bytes per K/V row in LDS
constexpr int TILE_B = BN * ROWB;       // 16 KB
constexpr int HALF_B = TILE_B / 2;      // one 32-key sub-block
constexpr int NSTAGE = 3;               // tiles resident or in flight
constexpr int V_BASE = 65536;           // V tiles start here; K tiles at NSTAGE * 16 KB below
constexpr int LDS_B = V_BASE + NSTAGE * TILE_B;
constexpr int NDMA = TILE_B / (NWAVE * 64 * 16);  // 16-byte DMA blocks per lane per K/V tile
constexpr int BIAS_BASE = NSTAGE * TILE_B;        // key-bias stages (256 B each), below V_BASE
// MFMA pairs ahead that a step's K (QK chain) and V (PV) fragments are read from LDS
constexpr int K_AHEAD = 2, V_AHEAD = 2;
static_assert(NSTAGE * TILE_B <= V_BASE, "K tiles must fit below the V tiles");

// fp8 cache: K tiles of e4m3 codes (128-byte rows, 8 KB), then two staging slots per wave for
// the V codes (1 KB) and the tile's two block scales (256 B); the V tiles are bf16 as above.
constexpr int ROWB8 = D;                              // bytes per fp8 K row in LDS
constexpr int TILE8_B = BN * ROWB8;                   // 8 KB
constexpr int HALF8_B = TILE8_B / 2;
constexpr int RAW_BASE = NSTAGE * TILE8_B;            // + slot * TILE8_B + 1 KB * wave
constexpr int SC_BASE = RAW_BASE + 2 * TILE8_B;       // + slot * SC_SLOT_B + 256 B * wave
constexpr int SC_SLOT_B = NWAVE * 256;
static_assert(SC_BASE + 2 * SC_SLOT_B <= V_BASE, "fp8 staging must fit below the V tiles");
static_assert(TILE8_B == NWAVE * 64 * 16, "one 16-byte copy per lane per fp8 tile");

// LDS swizzle of the 128-byte fp8 K rows: 16-byte chunk c of row r at chunk c ^ swz8(r). The
// QK operand reads (lane (l32, h): row l32, chunk 4m + 2i + h) are then conflict-free: of any
// 16 consecutive lanes, the rows of one parity land on 8 distinct chunks.
__device__ __forceinline__ int swz8(int r) { return (r >> 1) & 7; }

// Waits until at most n of this wave's copies are in flight (n in 0..2).
__device__ __forceinline__ void wait_vm(int n) {
  if (n <= 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else if (n == 1) asm volatile("s_waitcnt vmcnt(1)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
}

// S^T += K Q^T on the fp8 matrix cores: v_mfma_scale_f32_32x32x64_f8f6f4 with both operands
// e4m3 (format 0). Operand byte j of lane (l32, h) is d = 64m + 16h + j (j < 16) or
// 64m + 32 + 16h + (j - 16) (j >= 16) of d-half m, for the K row and the query column alike;
// the operands carry the e8m0 scales `kscale` (K's block scale, a power of two) and `qscale`
// (2^(qscale - 127)), so the product is the true score q . k.
__device__ __forceinline__ floatx16 mfma_qk8(const i32x8& k, const i32x8& q, const floatx16& c,
                                             int kscale, int qscale) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(k, q, c, 0, 0, 0, kscale, 0, qscale);
}

// The query operand of the fp8 QK product: the lane's 64 bf16 values of its query (qf[4m + 2r +
// half] holds d = 64m + 32r + 16h + 8 half .. +7) as q = (hi + lo / 16) 2^e per query, hi and lo
// e4m3, e = floor(log2 max|q|) - 7 (so |q| 2^-e < 256 and |lo| <= 128, both inside e4m3's
// range). hi carries q's leading 4 significant bits and lo the next 4, so the pair holds a bf16
// value exactly unless it is below 2^-13 of the row's max (then the error is below 2^-21 of it).
// Returns 127 + e, the e8m0 scale of hi (lo's is 4 less).
__device__ __forceinline__ int q8_split(const u32x4 (&qf)[8], i32x8 (&qh)[2], i32x8 (&ql)[2]) {
  float amax = 0.0f;
#pragma unroll
  for (int s = 0; s < 8; ++s)
#pragma unroll
    for (int w = 0; w < 4; ++w)
      amax = fmaxf(amax, fmaxf(fabsf(bf16_lo(qf[s][w])), fabsf(bf16_hi(qf[s][w]))));
  amax = wave_max_xor32(amax);  // lanes l and l^32 hold the two halves of one query
  int e = (int)((__float_as_uint(amax) >> 23) & 0xffu) - 127 - 7;
  e = e < -120 ? -120 : (e > 120 ? 120 : e);
  const float sc = __uint_as_float((uint32_t)(127 - e) << 23);  // 2^-e, exact
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      // operand word w = bytes 4w .. 4w+3: run w / 4, elements 4 (w % 4) .. +3 of the run
      const int e0 = 4 * (w & 3);
      const u32x4& src = qf[4 * m + 2 * (w >> 2) + (e0 >> 3)];
      const uint32_t w0 = src[(e0 & 7) >> 1], w1 = src[((e0 & 7) >> 1) + 1];
      const float x0 = bf16_lo(w0) * sc, x1 = bf16_hi(w0) * sc;
      const float x2 = bf16_lo(w1) * sc, x3 = bf16_hi(w1) * sc;
      int hw = __builtin_amdgcn_cvt_pk_fp8_f32(x0, x1, 0, false);
      hw = __builtin_amdgcn_cvt_pk_fp8_f32(x2, x3, hw, true);
      // the residuals x - hi are exact in fp32 (x has 8 significant bits)
      const auto h01 = __builtin_amdgcn_cvt_pk_f32_fp8(hw, false);
      const auto h23 = __builtin_amdgcn_cvt_pk_f32_fp8(hw, true);
      int lw = __builtin_amdgcn_cvt_pk_fp8_f32((x0 - h01[0]) * 16.0f, (x1 - h01[1]) * 16.0f, 0, false);
      lw = __builtin_amdgcn_cvt_pk_fp8_f32((x2 - h23[0]) * 16.0f, (x3 - h23[1]) * 16.0f, lw, true);
      qh[m][w] = hw;
      ql[m][w] = lw;
    }
  return 127 + e;
}

// Waits until at most `n` tiles' DMA groups (2*NDMA loads each) of this wave are in flight.
__device__ __forceinline__ void wait_tiles_outstanding(int n) {
  static_assert(2 * NDMA == 4, "vmcnt immediates below assume 4 loads per tile");
  if (n <= 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else if (n == 1) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
}

// Work items. A unit is (batch, head, q-tile); each unit's keys are cut into `splits` equal
// pieces. XCD x owns the units [U x / 8, U (x + 1) / 8) and runs their pieces piece-major (the
// q-tiles of a head, which read the same keys, run side by side on one XCD and share its L2).
// Item j of XCD x is piece j / n_x of unit start_x + j % n_x; the id is piece * U + unit.
// The XCDs of one GPU do not run equally fast (measured: the odd-numbered ones take 3-5 %
// longer per item), so with a work queue a workgroup whose own XCD's share is gone takes the
// next item of another XCD's share.
__device__ __forceinline__ void xcd_units(uint32_t U, uint32_t x, uint32_t& start, uint32_t& n) {
  start = (U * x) / 8u;
  n = (U * (x + 1u)) / 8u - start;
}

// Next item for a workgroup on XCD x0 from the 8 per-XCD queues, its own XCD's first, then any
// other (so that faster XCDs take over the end of slower ones' shares); -1 when all are empty.
// A relaxed read skips exhausted queues without bumping their counters.
__device__ __forceinline__ int take_item(uint32_t* q, uint32_t U, uint32_t S, uint32_t x0) {
  for (uint32_t t = 0; t < 8u; ++t) {
    const uint32_t x = (x0 + t) & 7u;
    uint32_t st, n;
    xcd_units(U, x, st, n);
    const uint32_t size = S * n;
    if (__hip_atomic_load(&q[x], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= size) continue;
    const uint32_t k = __hip_atomic_fetch_add(&q[x], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (k < size) return (int)((k / n) * U + st + k % n);
  }
  return -1;
}

__global__ void __launch_bounds__(256) attn_queue_reset_kernel(uint32_t* q, int n) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) q[i] = 0u;
}

// Stores and loads of the split partials when the last piece of a unit merges them: at device
// scope (sc1), so that they reach, and are read from, the point where the XCDs' caches are
// coherent; the XCD's own L2 holds no line of them that another XCD could miss.
__device__ __forceinline__ void store_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_dev(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
constexpr int kDevScope = 16;  // buffer cache-policy bit sc1: device scope

// The log-sum-exp merge of the N split partials of one unit's `rows` rows (the
// attn_merge_kernel arithmetic, which it must match bit for bit), by the workgroup of the
// unit's last piece. `wl` is LDS scratch for N x 256 weights and 256 reciprocals.
template <int N>
__device__ void merge_unit(const AttnKernelArgs& a, int b, int h, int qt, int rows, float* wl) {
  const int64_t per = (int64_t)a.B * a.H * a.Lq;          // rows of one split
  const int64_t base = ((int64_t)b * a.H + h) * a.Lq + (int64_t)qt * BM;
  float* inv = wl + 16 * BM;
  for (int r = threadIdx.x; r < rows; r += NWAVE * 64) {
    float ms[N], ls[N];
#pragma unroll
    for (int s = 0; s < N; ++s) {
      ms[s] = load_dev(a.part_m + s * per + base + r);
      ls[s] = load_dev(a.part_l + s * per + base + r);
    }
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < N; ++s) M = fmaxf(M, ms[s]);
    float den = 0.0f;
#pragma unroll
    for (int s = 0; s < N; ++s) {
      const float w = (M == -INFINITY || ms[s] == -INFINITY) ? 0.0f : expf(ms[s] - M);
      den += w * ls[s];
      wl[s * BM + r] = w;
    }
    inv[r] = den > 0.0f ? 1.0f / den : 0.0f;
  }
  __syncthreads();
  const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.part_o + base * D), (short)0, 0x7fffffff, 0x00020000);
  const uint32_t sstride = (uint32_t)(per * D * 4);  // bytes between splits
  for (int c = threadIdx.x; c < rows * (D / 4); c += NWAVE * 64) {
    const int r = c / (D / 4), dq = c % (D / 4);
    floatx4 os[N];
#pragma unroll
    for (int s = 0; s < N; ++s)
      os[s] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(
          rp, (uint32_t)(r * D + 4 * dq) * 4u, s * sstride, kDevScope));
    floatx4 num = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < N; ++s) num += wl[s * BM + r] * os[s];
    const float iv = inv[r];
    const int q = qt * BM + r;
    const int64_t off = a.osb * b + a.osl * (int64_t)q + a.osh * h + 4 * dq;
    if (a.o32) {
      *reinterpret_cast<floatx4*>(reinterpret_cast<float*>(a.out) + off) = num * iv;
    } else {
      u32x2 w;
      w[0] = pack_bf16x2(num[0] * iv, num[1] * iv);
      w[1] = pack_bf16x2(num[2] * iv, num[3] * iv);
      *reinterpret_cast<u32x2*>(a.out + off) = w;
    }
  }
}

// FP8 = false: bf16 K/V, DMA'd straight into LDS. FP8 = true: e4m3 K/V codes with power-of-two
// fp32 scales per (batch, head, 64-token block). The K codes are copied into LDS as they are and S^T = K Q^T
// runs on the fp8 matrix cores, against Q split into two e4m3 operands (q8_split): four x64
// MFMAs per 32-key sub-block instead of eight bf16 ones, half the K bytes in LDS and no K
// conversion. The V codes and the tile's two scales go through a per-wave LDS staging slot
// (copied two steps ahead); the wave that copied them converts its rows exactly to bf16 (every
// e4m3 value times a power of two is a bf16 value) into the bf16 V tile, so P stays bf16 in the
// PV product. The block scales stay out of the softmax: K's is the exponent scale of the fp8
// product (whose result is then the true score), V's the scale of the exact conversion.
// FOLD: scale * log2(e) == 1, i.e. q already carries log2(e)/sqrt(d) (a pre-scaled q, as the
// fused q/k kernel writes it): the QK chain starts from -m instead of 0, so the MFMA result is
// already the exponent of p and the softmax needs no per-score FMA (see the step).
// SEGN = 1 or 2: that many KV segments (a flat cache's window; a cache and the current chunk),
// no multiplicity bias and, for two, the same row strides: the tile copies are addressed by the
// tile index (issue1, issue_raw1, issue_k81) instead of walked by the general cursor (SEGN 0).
// KDM: K is d-major (the reference's N-major K cache [H, D, L], token stride 1). A K tile is then
// held in LDS as its two 32-key halves, each [128 d-rows][32 keys] (64-byte rows), copied 16 bytes
// (8 keys of one d) per lane; the QK operand of a key is gathered from a d-row pair of reads by
// the LDS transpose read (as V^T is from V rows), which gives lane (key, hl) the d values
// 16s + 4hl + {0..3, 8..11} of d-slice s, and the query operand is loaded in that same d order.
// Every read pattern of a 32-lane pass covers the 64 banks once (four 64-byte rows), so the halves
// need no swizzle.
// BIAS: a per-key additive score bias (natural log, shared by batch and heads): each tile's 64
// bias values are copied with the tile into LDS by wave 0, and every step adds them to its scores
// (in raw-score units: bias / scale) before the softmax.
template <bool FP8, bool TRACK, bool FOLD, int SEGN, bool KDM = false, bool BIAS = false>
__global__ void __launch_bounds__(NWAVE * 64, 1)
attn_fwd_bf16_kernel(const AttnKernelArgs a) {
  static_assert(!FOLD || !TRACK, "the folded softmax is the plain form");
  static_assert(!KDM || (!FP8 && SEGN == 0), "d-major K: bf16, general tile cursor");
  static_assert(!BIAS || (!FP8 && !TRACK && !FOLD && SEGN == 0), "key bias: plain bf16 form");
  constexpr int ESZ = FP8 ? 1 : 2;  // bytes per K/V element in HBM
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hl = lane >> 5;  // k-group / row-half of this lane
  const int l32 = lane & 31;

  // ---- work item (piece, unit). With a work queue the items are handed out at run time;
  // without, workgroup i takes item i / 8 of XCD i % 8 (workgroups reach the XCDs round-robin).
  const uint32_t U = (uint32_t)a.n_qtiles * a.H * a.B;
  uint32_t id;
  {
    __shared__ int s_item;
    if (a.queue != nullptr) {
      if (threadIdx.x == 0) s_item = take_item(a.queue, U, a.splits, blockIdx.x & 7u);
      __syncthreads();
    } else if (threadIdx.x == 0) {
      uint32_t st, n;
      xcd_units(U, blockIdx.x & 7u, st, n);
      const uint32_t j = blockIdx.x >> 3;
      s_item = j < a.splits * n ? (int)((j / n) * U + st + j % n) : -1;
    }
    __syncthreads();
    const int item = s_item;
    if (item < 0) return;  // every wave of the workgroup
    id = (uint32_t)item;
  }
  const int split = id / U;
  const uint32_t unit = id % U;
  const int qt = unit % a.n_qtiles;
  const int h = (unit / a.n_qtiles) % a.H;
  const int b = unit / ((uint32_t)a.n_qtiles * a.H);

  const int q0 = qt * BM + wave * 32;  // first query of this wave (wave-uniform)
  const bool wave_active = q0 < a.Lq;

  // ---- Q fragments (B operand of S^T = K Q^T): qf[s] holds d = 16s + 8hl .. +7; for the fp8
  // operands (q8_split) d = 32 (s / 2) + 16hl + 8 (s % 2) .. +7
  u32x4 qf[8];
  {
    const int q = q0 + l32;
    const uint16_t* qp = a.q + a.qsb * b + a.qsl * (int64_t)q + a.qsh * h;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int d0 = FP8 ? 32 * (s >> 1) + 16 * hl + 8 * (s & 1) : 16 * s + 8 * hl;
      u32x4 v = {0u, 0u, 0u, 0u};
      if constexpr (KDM) {
        // d = 16s + 4hl + {0..3, 8..11}: the order of the d-major K operand (see the kernel note)
        if (q < a.Lq) {
          const u32x2 x0 = *reinterpret_cast<const u32x2*>(qp + 16 * s + 4 * hl);
          const u32x2 x1 = *reinterpret_cast<const u32x2*>(qp + 16 * s + 4 * hl + 8);
          v = u32x4{x0[0], x0[1], x1[0], x1[1]};
        }
      } else {
        if (q < a.Lq) v = *reinterpret_cast<const u32x4*>(qp + d0);
      }
      qf[s] = v;
    }
    // (waited for below, together with the first K/V tiles: one round trip, not two)
  }

  // ---- key range of this batch and split (the host window, narrowed by the device bounds and
  // k_lens when given)
  int64_t hi = a.hi, lo = a.lo;
  if (a.k_lens != nullptr) {
    const int64_t kl = a.k_lens[b];
    hi = kl < hi ? kl : hi;
  }
  if (a.hi_dev != nullptr) {
    const int64_t x = *a.hi_dev;
    hi = x < hi ? x : hi;
  }
  if (a.lo_dev != nullptr) {
    const int64_t x = *a.lo_dev;
    lo = x > lo ? x : lo;
  }
  if (hi < lo) hi = lo;
  const int n_tiles = hi > lo ? count_tiles(a, lo, hi) : 0;
  // this piece's tiles
  const int t0 = (int)((int64_t)n_tiles * split / a.splits);
  const int t1 = (int)((int64_t)n_tiles * (split + 1) / a.splits);

  // ---- per-lane LDS offsets
  // DMA: this wave fills 1 KB blocks NDMA*wave + i of each tile; lane -> (row, physical chunk).
  int dma_row[NDMA], dma_col[NDMA];
#pragma unroll
  for (int i = 0; i < NDMA; ++i) {
    dma_row[i] = 4 * (NDMA * wave + i) + (lane >> 4);
    dma_col[i] = ((lane & 15) ^ swz(dma_row[i])) * 16;  // byte offset of the logical chunk
  }
  // d-major K: block j = NDMA * wave + i is half j / 8, d-rows 16 (j % 8) + lane / 4 of it, and
  // the lane's 8 keys 32 (j / 8) + 8 (lane % 4) .. +7 of the tile (LDS byte 1024 j + 16 lane, as
  // for token-major rows)
  int kdm_row[NDMA], kdm_key[NDMA];
#pragma unroll
  for (int i = 0; i < NDMA; ++i) {
    const int j = NDMA * wave + i;
    kdm_row[i] = 16 * (j & 7) + (lane >> 2);
    kdm_key[i] = 32 * (j >> 3) + 8 * (lane & 3);
  }
  // LDS byte addresses of this lane's fragments in stage 0.
  // K fragment (sub-block rows 0..31) for d-slice s: row l32, logical chunk 2s + hl. fp8: the
  // x64 operand of d-half m is the two 16-byte reads koff[2m] (bytes 0-15, chunk 4m + hl) and
  // koff[2m + 1] (bytes 16-31, chunk 4m + 2 + hl), the same formula over 128-byte rows.
  const int lds0 = (int)lds_addr(lds);
  int koff[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    if constexpr (FP8)
      koff[s] = s < 4 ? opaque(lds0 + l32 * ROWB8 + (((2 * s + hl) ^ swz8(l32)) << 4)) : 0;
    else if constexpr (KDM)
      koff[s] = 0;
    else
      koff[s] = opaque(lds0 + l32 * ROWB + (((2 * s + hl) ^ swz(l32)) << 4));
  }
  // d-major K transpose reads (half 0, d-slice 0, first read): the 16-lane group (lane / 16)
  // takes keys 16 (group % 2) .. +15 of the half and d-rows 4hl .. +3; source lane s16 points at
  // d-row 4hl + s16 / 4, keys 16 (group % 2) + 4 (s16 % 4) .. +3 (byte 8 (s16 % 2) of its 16-byte
  // chunk). d-slice s adds 16 rows (1 KB), the second read 8 rows (512 B), half 1 adds 8 KB.
  int kdm_off = 0;
  if constexpr (KDM) {
    const int s16 = lane & 15, g = (lane >> 4) & 1;
    kdm_off = opaque(lds0 + (4 * hl + (s16 >> 2)) * 64 + (2 * g + ((s16 & 3) >> 1)) * 16 + 8 * (s16 & 1));
  }
  // V transpose reads (sub-block rows 0..31, k-step m = 0) for d-block db and key
  // half j: source row 4hl + 8j + s/4, columns 32db + 16g + 4(s%4) .. +3 (s = lane % 16,
  // g = (lane / 16) % 2).
  int voff[4][2];
  {
    const int s16 = lane & 15, g = (lane >> 4) & 1;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int r = 4 * hl + 8 * j + (s16 >> 2);
        const int lc = 4 * db + 2 * g + ((s16 & 3) >> 1);
        voff[db][j] = opaque(lds0 + V_BASE + r * ROWB + ((lc ^ swz(r)) << 4) + 8 * (s16 & 1));
      }
  }

  floatx16 oacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[db][r] = 0.0f;
  float m_used = M_INIT, m_true = -INFINITY, lsum = 0.0f;  // exponent ref, row max, row sum
  const float c = a.scale_log2;
  // FOLD: the exponent reference (log2 units, c = 1), and whether this row's has been set from a
  // valid score yet (before that, its O and l are 0)
  float mref = 0.0f;
  float mlim = -1.0f;  // the redo threshold of this row: -1 until its reference is set, then P_LIMIT
  const float mult_raw = sreg(a.mult_raw);
  // the call carries a multiplicity bias (mult_key >= 0: the sign of its high word)
  const int mult = sreg((int)(a.mult_key >> 32)) >= 0;
  const float tau_raw = TAU / c;

  // DMA of the cursor's tile into a stage (2*NDMA x 16 B per lane); returns the tile's row
  // info (pack_rows). Full tiles use the per-segment lane offsets; in a partial
  // tile, rows outside the valid range fetch a valid row instead: their scores are masked to
  // -inf and their probabilities are exactly 0, so the duplicate never contributes.
  TileCursor cs;
  uint32_t lane_k[NDMA], lane_v[NDMA];
  auto seg_offsets = [&]() {
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      lane_k[i] = KDM ? (uint32_t)kdm_row[i] * cs.ks + 2 * kdm_key[i]
                      : (uint32_t)dma_row[i] * cs.ks + dma_col[i];
      lane_v[i] = (uint32_t)dma_row[i] * cs.vs + dma_col[i];
    }
  };
  const uint32_t lds_wave = lds_addr(lds) + 1024 * NDMA * wave;  // this wave's 1 KB blocks
  auto issue = [&](int stage) -> int {
    const int rows = cs.rows;
    // (the base is re-materialised per call so that the per-stage addresses are not all kept live)
    const uint32_t kdst = (uint32_t)sreg((int)lds_wave) + stage * TILE_B;
    const uint32_t vdst = kdst + V_BASE;
    if ((rows & 0xffff) == (BN << 8)) {  // every row valid
#pragma unroll
      for (int i = 0; i < NDMA; ++i) {
        dma16(cs.kt, lane_k[i], kdst + 1024 * i);
        dma16(cs.vt, lane_v[i], vdst + 1024 * i);
      }
    } else {
      const int tvlo = rows & 0xff, rhi = ((rows >> 8) & 0xff) - 1;
#pragma unroll
      for (int i = 0; i < NDMA; ++i) {
        int r = dma_row[i];
        r = r < tvlo ? tvlo : (r > rhi ? rhi : r);
        if constexpr (KDM) {
          // a lane's 8 keys lie in the segment when its first does (len is a multiple of 8);
          // groups wholly outside the valid rows copy a valid group instead
          int kk = kdm_key[i];
          kk = kk < (tvlo & ~7) ? (tvlo & ~7) : (kk > (rhi & ~7) ? (rhi & ~7) : kk);
          dma16(cs.kt, (uint32_t)kdm_row[i] * cs.ks + 2 * kk, kdst + 1024 * i);
        } else {
          dma16(cs.kt, (uint32_t)r * cs.ks + dma_col[i], kdst + 1024 * i);
        }
        dma16(cs.vt, (uint32_t)r * cs.vs + dma_col[i], vdst + 1024 * i);
      }
    }
    if constexpr (BIAS) {
      // the tile's 64 key biases (clamped to the last key past the end: those keys are masked)
      if (wave == 0) {
        int64_t key = a.seg[cs.seg].start + (int64_t)cs.lt * BN + lane;
        key = key < a.total - 1 ? key : a.total - 1;
        dma4((uint64_t)(uintptr_t)(a.key_bias + key), (uint32_t)sreg(lds0) + BIAS_BASE + stage * 256);
      }
    }
    if (cursor_next<ESZ>(a, lo, hi, b, h, mult, cs) && cs.seg < a.nseg) seg_offsets();
    return rows;
  };
  // SEGN > 0: walk tile g lies in the walk's first segment while g < w_g1, else in its second;
  // it is local tile g + off of that segment, its K/V rows come from the index, and only a
  // segment's first and last tiles compute their valid rows. Nothing is carried from one copy to
  // the next, so the tile loop's only state is its counter.
  struct SegWalk {
    int off = 0, first = 0, last = 0, la = 0, lb = 0;  // local tile = g + off; ends; key range
    const unsigned char* kb = nullptr;                  // local tile 0, (b, h)
    const unsigned char* vb = nullptr;
    const float* ksc = nullptr;                         // fp8: block scales of local tile 0
    const float* vsc = nullptr;
  };
  SegWalk w0, w1;
  int w_g1 = 1 << 30;
  auto pick = [&](int g) -> SegWalk { return (SEGN == 2 && g >= w_g1) ? w1 : w0; };
  // packed valid rows of local tile lt at a segment's ends (no bias)
  auto rows_at = [&](const SegWalk& w, int lt) -> int {
    const int row0 = lt * BN;
    const int l = w.la - row0, u = w.lb - row0;
    return pack_rows(l > 0 ? l : 0, u < BN ? u : BN, 255);
  };
  auto issue1 = [&](int stage, int g) -> int {
    const SegWalk w = pick(g);
    const int lt = g + w.off;
    const unsigned char* kt = w.kb + (uint64_t)(uint32_t)lt * cs.kstep;
    const unsigned char* vt = w.vb + (uint64_t)(uint32_t)lt * cs.vstep;
    const uint32_t kdst = (uint32_t)sreg((int)lds_wave) + stage * TILE_B;
    const uint32_t vdst = kdst + V_BASE;
    if (lt > w.first && lt < w.last) {  // every row valid
#pragma unroll
      for (int i = 0; i < NDMA; ++i) {
        dma16(kt, lane_k[i], kdst + 1024 * i);
        dma16(vt, lane_v[i], vdst + 1024 * i);
      }
      return ROWS_FULL;
    }
    const int rows = rows_at(w, lt);
    const int tvlo = rows & 0xff, rhi = ((rows >> 8) & 0xff) - 1;
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      int r = dma_row[i];
      r = r < tvlo ? tvlo : (r > rhi ? rhi : r);
      dma16(kt, (uint32_t)r * cs.ks + dma_col[i], kdst + 1024 * i);
      dma16(vt, (uint32_t)r * cs.vs + dma_col[i], vdst + 1024 * i);
    }
    return rows;
  };

  // fp8: per tile, thread t (= 64 wave + lane) copies the K codes of row t / 8 into the K tile
  // (at physical chunk t % 8, so the logical chunk is (t % 8) ^ swz8) and the 16 V codes of
  // row vrow8, chunk vj8 into its wave's staging slot (at 16 lane); lanes 0 / 1 copy the K / V
  // block scale (dwords 0 and 1 of the wave's scale slot). Rows outside a partial tile's valid
  // range fetch a valid row instead, as above. The copying wave converts its own staged V.
  const int row8 = threadIdx.x >> 3, j8 = threadIdx.x & 7;
  const int kcol8 = (j8 ^ swz8(row8)) << 4;
  // The V codes are mapped for the conversion's bf16 writes: a 16-byte LDS write serves 8
  // lanes per clock over 32 banks (measured: SQ_LDS_BANK_CONFLICT is 0 only then), so each 8
  // lanes must write 8 distinct chunks mod 8. A lane's 16 codes become two adjacent bf16 chunks
  // (2 vj8, 2 vj8 + 1), which for 8 lanes of one row cover only 4 residues; so each group of 8
  // lanes takes half-rows of two rows 4 apart, whose swizzles differ in parity: row
  // (g & 3) + 4 (u / 4), chunk pair (u & 3) + 4 (g / 4) for lane 8 g + u.
  const int vrow8 = 8 * wave + ((lane >> 3) & 3) + 4 * ((lane >> 2) & 1);
  const int vj8 = (lane & 3) + 4 * (lane >> 5);
  const uint32_t raw_wave = lds_addr(lds) + RAW_BASE + 1024 * wave;  // + slot * TILE8_B
  const uint32_t sc_wave = lds_addr(lds) + SC_BASE + 256 * wave;     // + slot * SC_SLOT_B
  uint32_t lane_k8 = 0, lane_v8 = 0;
  auto seg_offsets8 = [&]() {
    lane_k8 = (uint32_t)row8 * cs.ks + kcol8;
    lane_v8 = (uint32_t)vrow8 * cs.vs + 16 * vj8;
  };
  auto clamped = [](int r, int rows) {
    const int tvlo = rows & 0xff, rhi = ((rows >> 8) & 0xff) - 1;
    return r < tvlo ? tvlo : (r > rhi ? rhi : r);
  };
  // V codes and scales of the cursor's tile into staging slot `slot` (2 copies per lane)
  auto issue_raw = [&](int slot) -> int {
    const int rows = cs.rows;
    uint32_t voff = lane_v8;
    if ((rows & 0xffff) != (BN << 8)) voff = (uint32_t)clamped(vrow8, rows) * cs.vs + 16 * vj8;
    dma16(cs.vt, voff, (uint32_t)sreg((int)raw_wave) + slot * TILE8_B);
    const uint64_t sp = (lane & 1) ? (uint64_t)(uintptr_t)cs.vsc : (uint64_t)(uintptr_t)cs.ksc;
    dma4(sp, (uint32_t)sreg((int)sc_wave) + slot * SC_SLOT_B);
    return rows;
  };
  // K codes of the cursor's tile into stage `stage` (1 copy per lane); then the cursor advances
  auto issue_k8 = [&](int stage) {
    const int rows = cs.rows;
    uint32_t koff8 = lane_k8;
    if ((rows & 0xffff) != (BN << 8)) koff8 = (uint32_t)clamped(row8, rows) * cs.ks + kcol8;
    dma16(cs.kt, koff8, (uint32_t)sreg(lds0) + stage * TILE8_B + 1024 * wave);
    if (cursor_next<1>(a, lo, hi, b, h, mult, cs) && cs.seg < a.nseg) seg_offsets8();
  };
  // SEGN > 0 forms of the two: tile g of the walk, addressed by its index
  auto issue_raw1 = [&](int slot, int g) -> int {
    const SegWalk w = pick(g);
    const int lt = g + w.off;
    const unsigned char* vt = w.vb + (uint64_t)(uint32_t)lt * cs.vstep;
    int rows = ROWS_FULL;
    uint32_t voff = lane_v8;
    if (!(lt > w.first && lt < w.last)) {
      rows = rows_at(w, lt);
      voff = (uint32_t)clamped(vrow8, rows) * cs.vs + 16 * vj8;
    }
    dma16(vt, voff, (uint32_t)sreg((int)raw_wave) + slot * TILE8_B);
    const uint64_t sp = (lane & 1) ? (uint64_t)(uintptr_t)(w.vsc + lt) : (uint64_t)(uintptr_t)(w.ksc + lt);
    dma4(sp, (uint32_t)sreg((int)sc_wave) + slot * SC_SLOT_B);
    return rows;
  };
  auto issue_k81 = [&](int stage, int g) {
    const SegWalk w = pick(g);
    const int lt = g + w.off;
    const unsigned char* kt = w.kb + (uint64_t)(uint32_t)lt * cs.kstep;
    uint32_t koff8 = lane_k8;
    if (!(lt > w.first && lt < w.last)) koff8 = (uint32_t)clamped(row8, rows_at(w, lt)) * cs.ks + kcol8;
    dma16(kt, koff8, (uint32_t)sreg(lds0) + stage * TILE8_B + 1024 * wave);
  };
  // (SEGN > 0) the walk's fixed addresses: segment values from a cursor on walk tile g, the
  // segment's first tile in the walk
  auto walk_enter = [&](SegWalk& w, const TileCursor& c, int g) {
    w.off = c.lt - g;
    w.first = c.la / BN;
    w.last = c.lt_end - 1;
    w.la = c.la;
    w.lb = c.lb;
    w.kb = c.kt - (int64_t)c.lt * c.kstep;
    w.vb = c.vt - (int64_t)c.lt * c.vstep;
    if constexpr (FP8) {
      w.ksc = c.ksc - c.lt;
      w.vsc = c.vsc - c.lt;
    }
  };
  auto seg_walk_enter = [&]() {
    walk_enter(w0, cs, 0);
    if constexpr (SEGN == 2) {
      // the next segment with keys, after the walk's tiles of the first
      TileCursor c2 = cs;
      const int n0 = cs.lt_end - cs.lt;
      c2.lt = c2.lt_end - 1;
      cursor_next<ESZ>(a, lo, hi, b, h, 0, c2);
      if (c2.seg < a.nseg) {
        w_g1 = n0;
        walk_enter(w1, c2, n0);
      }
    }
  };
  // this lane's 16 staged V codes of slot `slot` -> bf16 (times V's block scale, a power of two:
  // exact) into V stage `stage` (row vrow8, logical chunks 2 vj8 and 2 vj8 + 1); K's block scale
  // -> kse, as the e8m0 exponent of the fp8 product
  auto convert_v = [&](int slot, int stage, int& kse) {
    const u32x4 x = lds_read_b128((int)raw_wave + slot * TILE8_B + 16 * lane);
    const u32x2 sc = lds_read_b64((int)sc_wave + slot * SC_SLOT_B);
    // (a scale that is not a power of two, whose mantissa the exponent scale and the
    // conversion would drop, turns into NaN: e8m0 0xff for K, a NaN factor for V)
    const float sv = (sc[1] & 0x7fffffu) ? __uint_as_float(0x7fc00000u) : __uint_as_float(sc[1]);
    unsigned char* vd = lds + V_BASE + stage * TILE_B + vrow8 * ROWB;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const uint32_t w0 = x[2 * hf], w1 = x[2 * hf + 1];
      const u32x4 y = {
          __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, sv, false)),
          __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, sv, true)),
          __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, sv, false)),
          __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, sv, true))};
      *reinterpret_cast<u32x4*>(vd + (((2 * vj8 + hf) ^ swz(vrow8)) << 4)) = y;
    }
    kse = (sc[0] & 0x7fffffu) ? 0xff : (int)((sc[0] >> 23) & 0xffu);
  };

  const int T = t1 - t0;
  if (T > 0) {
    int vr[NSTAGE];  // valid rows of tiles u .. u+NSTAGE-1 (u = the tile being softmaxed)
    int kser[NSTAGE];  // fp8: K's block scales of the same tiles (e8m0)
#pragma unroll
    for (int k = 0; k < NSTAGE; ++k) { vr[k] = ROWS_FULL; kser[k] = 127; }
    i32x8 qh[2], ql[2];  // fp8: the query operands (hi, lo) of d-halves 0 and 1
    int sbh = 127, sbl = 127;  // and their e8m0 scales
    cursor_init<ESZ>(a, lo, hi, t0, b, h, cs);
    if constexpr (SEGN > 0) seg_walk_enter();
    if constexpr (FP8) {
      // tiles 0 and 1: staged V (slots 0, 1) and K (stages 0, 1)
      seg_offsets8();
#pragma unroll
      for (int k = 0; k < NSTAGE - 1; ++k)
        if (k < T) {
          if constexpr (SEGN > 0) {
            vr[k] = issue_raw1(k, k);
            issue_k81(k, k);
          } else {
            vr[k] = issue_raw(k);
            issue_k8(k);
          }
        }
    } else {
      seg_offsets();
#pragma unroll
      for (int k = 0; k < NSTAGE - 1; ++k)
        if (k < T) vr[k] = SEGN > 0 ? issue1(k, k) : issue(k);
    }
    // The first step's "previous sub-block" is the second half of stage NSTAGE-1's V tile
    // with P = 0: zero it so that 0 * V stays 0 (that stage is only filled after barrier 0).
    {
      const u32x4 z = {0u, 0u, 0u, 0u};
      unsigned char* zv = lds + V_BASE + (NSTAGE - 1) * TILE_B + HALF_B;
      *reinterpret_cast<u32x4*>(zv + 16 * threadIdx.x) = z;
    }
    // Q and the first tiles (issued after Q, so the in-order count covers both): wait for all
    // of them, explicitly and on every path, so that the compiler, which cannot see the asm
    // K/V copies, does not re-wait for all memory before the first MFMA of every iteration
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    if constexpr (FP8) {
      // tile 0's V into stage 0 (read from the end of step 0 on), and the fp8 query operands
      convert_v(0, 0, kser[0]);
      sbh = q8_split(qf, qh, ql);
      sbl = sbh - 4;
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the zero fill (and fp8 V tile) are done
    barrier_nofence();

    // Pipeline registers, double-buffered so that consecutive steps swap roles instead of
    // copying: S of the sub-block being softmaxed / being computed, P of the previous / current
    // sub-block. `pend` / `alpha_p` (TRACK): an O rescale decided at the start of the previous
    // step, applied at the start of the next one (after the PV MFMAs that still used the old
    // reference). The other forms decide a move after the step's MFMAs and rescale O right in
    // the redo branch, so the common path carries no rescale branch.
    floatx16 sA, sB, cinit;  // cinit (FOLD): -mref, the start of every QK chain
#pragma unroll
    for (int r = 0; r < 16; ++r) { sA[r] = 0.0f; sB[r] = 0.0f; cinit[r] = 0.0f; }
    u32x4 pA[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
    u32x4 pB[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
    bool pend = false;
    float alpha_p = 1.0f;

    // LDS fragments in flight: K of pair i in kf[i % KR], V in vf[i % VR]. The rings hold a
    // multiple of 8 slots' worth of indices (8 % KR == 0), so the last pairs of a step can read
    // the next step's first fragments into the slots that step expects.
    constexpr int KR = K_AHEAD + 2, VR = V_AHEAD + 2;
    static_assert(8 % KR == 0 && 8 % VR == 0, "fragment rings must divide 8");
    u32x4 kf[KR], vf[VR];
    i32x8 k8f[2];  // fp8: the K operands of d-halves 0 and 1
    auto load_k = [&](auto ko_c, int i) {
      constexpr int KO = decltype(ko_c)::value;
      if constexpr (FP8) {
        const u32x4 x0 = lds_read_b128(koff[2 * i] + KO), x1 = lds_read_b128(koff[2 * i + 1] + KO);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          k8f[i][j] = (int)x0[j];
          k8f[i][j + 4] = (int)x1[j];
        }
      } else if constexpr (KDM) {
        const u32x2 x0 = lds_read_tr16(kdm_off + KO + 1024 * i);
        const u32x2 x1 = lds_read_tr16(kdm_off + KO + 1024 * i + 512);
        kf[i % KR] = u32x4{x0[0], x0[1], x1[0], x1[1]};
      } else {
        kf[i % KR] = lds_read_b128(koff[i] + KO);
      }
    };
    auto load_v = [&](auto vo_c, int i) {
      constexpr int VO = decltype(vo_c)::value;
      const int db = i >> 1, m = i & 1;
      const u32x2 v0 = lds_read_tr16(voff[db][0] + VO + 16 * m * ROWB);
      const u32x2 v1 = lds_read_tr16(voff[db][1] + VO + 16 * m * ROWB);
      vf[i % VR] = u32x4{v0[0], v0[1], v1[0], v1[1]};
    };

    // S of sub-block 0 (tile 0, rows 0..31), and the first fragments of step 0: K of tile 0
    // rows 32..63, V of the zeroed "previous sub-block"
    if (wave_active) {
      if constexpr (FP8) {
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          load_k(std::integral_constant<int, 0>{}, m);
          sA = mfma_qk8(k8f[m], qh[m], sA, kser[0], sbh);
          sA = mfma_qk8(k8f[m], ql[m], sA, kser[0], sbl);
        }
        load_k(std::integral_constant<int, HALF8_B>{}, 0);
      } else {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          if constexpr (KDM) {
            const u32x2 x0 = lds_read_tr16(kdm_off + 1024 * s);
            const u32x2 x1 = lds_read_tr16(kdm_off + 1024 * s + 512);
            sA = mfma32x32x16(u32x4{x0[0], x0[1], x1[0], x1[1]}, qf[s], sA);
          } else {
            sA = mfma32x32x16(lds_read_b128(koff[s]), qf[s], sA);
          }
        }
#pragma unroll
        for (int i = 0; i < K_AHEAD; ++i) load_k(std::integral_constant<int, HALF_B>{}, i);
      }
#pragma unroll
      for (int i = 0; i < V_AHEAD; ++i)
        load_v(std::integral_constant<int, (NSTAGE - 1) * TILE_B + HALF_B>{}, i);
    }

    // One pipeline step: softmax of s_in (sub-block `kb` of a tile with valid rows vrow) into
    // p_out, O += V^T p_in^T from LDS offset VO, s_out = K Q^T from LDS offset KO (fp8: with K's
    // block scale kse, the e8m0 exponent of s_out's tile). KPRE / VPRE: the first K / V fragments were read by the
    // previous step; NKO / NVO (>= 0): read the next step's first fragments from there.
    auto step = [&](auto koff_c, auto voff_c, auto kpre_c, auto vpre_c, auto nko_c, auto nvo_c,
                    floatx16& s_in, floatx16& s_out, u32x4 (&p_in)[2], u32x4 (&p_out)[2], int kb,
                    int vrow, int kse) {
      constexpr bool KPRE = decltype(kpre_c)::value, VPRE = decltype(vpre_c)::value;
      constexpr int NKO = decltype(nko_c)::value, NVO = decltype(nvo_c)::value;
      if constexpr (!KPRE) {
        if constexpr (FP8) {
          load_k(koff_c, 0);
        } else {
#pragma unroll
          for (int i = 0; i < K_AHEAD; ++i) load_k(koff_c, i);
        }
      }
      if constexpr (!VPRE) {
#pragma unroll
        for (int i = 0; i < V_AHEAD; ++i) load_v(voff_c, i);
      }
      if constexpr (TRACK) {
        if (pend) scale_acc(oacc, alpha_p);
      }
      if constexpr (BIAS) {
        // this lane's keys 32 kb + 8 g + 4 hl .. +3 (registers 4g .. 4g+3) of the tile being
        // softmaxed (stage KS for the first half's step, the stage before SN for the second's)
        constexpr int KS = decltype(koff_c)::value / (FP8 ? TILE8_B : TILE_B);
        const int st = kb == 0 ? KS : (KS + NSTAGE - 1) % NSTAGE;
        const float inv_scale = a.inv_scale;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const u32x4 bv = lds_read_b128(lds0 + BIAS_BASE + 256 * st + 128 * kb + 32 * g + 16 * hl);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            s_in[4 * g + e] = __builtin_fmaf(__uint_as_float(bv[e]), inv_scale, s_in[4 * g + e]);
        }
      }
      const int vlo = vrow & 0xff, vhi = (vrow >> 8) & 0xff, mrow = vrow >> 16;
      if (vrow != ROWS_FULL && (vlo > 32 * kb || vhi < 32 * kb + 32 || mrow < 32 * kb + 32))
        mask_scores(s_in, kb, vlo, vhi, hl, mrow, mult_raw);
      // softmax, part 1 (TRACK): running max and exponent reference, decided before the
      // exponentials (wave-uniform). Without TRACK the exponentials use the current reference
      // and part 3 checks them afterwards.
      bool move = false;
      float alpha = 1.0f;
      if constexpr (TRACK) {
        // lanes l and l^32 hold the same query's running max: fold it in before the exchange
        float mx = m_true;
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s_in[r]);
        m_true = wave_max_xor32(mx);
        // Every lane sees the same valid keys, so m_true is -inf in all lanes or in none, and
        // a move never selects -inf.
        move = __any(m_true > m_used + tau_raw);
        const float m_new = move ? m_true : m_used;
        alpha = fast_exp2((m_used - m_new) * c);
        m_used = m_new;
      }
      // The reference starts at M_INIT, a finite stand-in for -inf, so no step needs an
      // infinity case: masked scores (-inf) give p = 0, and the first valid score moves it.
      // p = exp2(s c - m c)
      float ca = -m_used * c;
      // MFMAs of the neighbouring sub-blocks
      if constexpr (FOLD) {
        s_out = cinit;
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) s_out[r] = 0.0f;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (i + V_AHEAD < 8) load_v(voff_c, i + V_AHEAD);
        else if constexpr (NVO >= 0) load_v(nvo_c, i + V_AHEAD - 8);
        if constexpr (FP8) {
          // K of d-half 1 at once; the next step's d-half 0 once this step's last use of it
          // (the lo product at i = 2) is issued
          if (i == 0) load_k(koff_c, 1);
          if constexpr (NKO >= 0)
            if (i == 4) load_k(nko_c, 0);
        } else {
          if (i + K_AHEAD < 8) load_k(koff_c, i + K_AHEAD);
          else if constexpr (NKO >= 0) load_k(nko_c, i + K_AHEAD - 8);
        }
        if constexpr (FP8) {
          // QK on the fp8 cores at even i: (d-half i / 4) x (hi, lo)
          if ((i & 1) == 0) {
            const int m = i >> 2;
            s_out = (i & 2) ? mfma_qk8(k8f[m], ql[m], s_out, kse, sbl)
                            : mfma_qk8(k8f[m], qh[m], s_out, kse, sbh);
          }
        } else {
          s_out = mfma32x32x16(kf[i % KR], qf[i], s_out);
        }
        oacc[i >> 1] = mfma32x32x16(vf[i % VR], p_in[i & 1], oacc[i >> 1]);
      }
      // softmax, part 2: P packed to bf16 in the PV operand order, fp32 row sum
      auto exps = [&]() {
        float l;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float x0 = fast_exp2(FOLD ? s_in[8 * m + 2 * e] : __builtin_fmaf(s_in[8 * m + 2 * e], c, ca));
            const float x1 = fast_exp2(FOLD ? s_in[8 * m + 2 * e + 1]
                                            : __builtin_fmaf(s_in[8 * m + 2 * e + 1], c, ca));
            p_out[m][e] = pack_bf16x2(x0, x1);
            l = (m == 0 && e == 0) ? x0 + x1 : l + (x0 + x1);
          }
        }
        return l;
      };
      float ls = exps();
      // schedule of the step's block, which the groups must share with the MFMAs (ahead of the
      // redo branch below): the first pairs' fragments, then per MFMA pair: MFMA, 2 VALU, the LDS
      // reads of the pair K_AHEAD / V_AHEAD ahead, MFMA, 2 VALU; the rest of the VALU work is
      // left to the compiler. Measured against the compiler's own order and against 1, 3 or 4
      // VALU per MFMA and other places for the reads: 3.5 % faster than the next best.
      constexpr int NDS0 = (KPRE ? 0 : (FP8 ? 2 : K_AHEAD)) + (VPRE ? 0 : 2 * V_AHEAD);
      if constexpr (NDS0 > 0) __builtin_amdgcn_sched_group_barrier(0x100, NDS0, 0);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const bool rk = i + K_AHEAD < 8 || NKO >= 0, rv = i + V_AHEAD < 8 || NVO >= 0;
        if constexpr (FP8) {
          // the QK product (even i) and the PV product, 2 VALU after each, and between them
          // the LDS reads: K operands at i = 0 and 4, V fragments V_AHEAD pairs ahead
          // (folded: exponentials named as transcendentals, which the VALU class does not take:
          // per MFMA pair 1 + 1 with 1 + 2 VALU ops, after a lone PV MFMA 2 with 3; measured
          // 2.7 % faster than one of each after every MFMA)
          const int nds = ((i == 0 || (i == 4 && NKO >= 0)) ? 2 : 0) + (rv ? 2 : 0);
          if (i % 2 == 0) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if constexpr (FOLD) __builtin_amdgcn_sched_group_barrier(0x400, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, FOLD ? 1 : 2, 0);
          }
          if (nds == 4) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
          else if (nds == 2) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if constexpr (FOLD) {
            if (i % 2 == 0) {
              __builtin_amdgcn_sched_group_barrier(0x400, 1, 0);
              __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
            } else {
              __builtin_amdgcn_sched_group_barrier(0x400, 2, 0);
              __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
            }
          } else {
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
          }
          continue;
        }
        if constexpr (FOLD) {
          // (the VALU class does not take the exponentials, which without the FMAs would
          // otherwise bunch at the start of the step: one per MFMA, named as transcendentals)
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
          __builtin_amdgcn_sched_group_barrier(0x400, 1, 0);  // 1 exponential
          __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);  // 1 VALU
        } else {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // 2 VALU
        }
        if (rk && rv) __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);  // LDS reads
        else if (rv) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        else if (rk) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        if constexpr (FOLD) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x400, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
        } else {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
        }
      }
      // fp8: the next sub-block's S is finished in this block as well (the compiler would
      // otherwise sink its MFMA chain, used only by the next step, past the redo branch, where
      // the dependent MFMAs issue back to back)
      if constexpr (FP8) asm volatile("" ::"v"(s_out));
      if constexpr (FOLD) {
        asm volatile("" ::"v"(p_out[0]), "v"(p_out[1]), "v"(ls));
        // s_in is s - mref. Redo as below, and also while a row's reference is not yet set
        // (it starts at 0; the row's O and l are still 0 then, so it may move down, with no
        // rescale). mx is the row's (lanes l and l^32 agree), so both lanes move alike.
        if (__any(!(ls <= mlim))) {
          float mx = s_in[0];
#pragma unroll
          for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s_in[r]);
          mx = wave_max_xor32(mx);
          float d;  // the reference's move, log2 units
          if (mlim > 0.0f) {
            d = fmaxf(mx, 0.0f);
            alpha = fast_exp2(-d);
            // O (with this step's PV of the previous sub-block, at the old reference) and the
            // row sum move now
            scale_acc(oacc, alpha);
            lsum *= alpha;
          } else {
            const bool set = mx > -INFINITY;  // a fully masked sub-block leaves it unset
            d = set ? mx : 0.0f;
            mlim = set ? P_LIMIT : -1.0f;
          }
          move = true;
          mref += d;
          // s_out (the next sub-block, started from the old -mref in this step) moves too
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            s_in[r] -= d;
            s_out[r] -= d;
            cinit[r] = -mref;
          }
          ls = exps();
        }
      } else if constexpr (!TRACK) {
        // P is packed in this block, not in the redo branch's successors
        asm volatile("" ::"v"(p_out[0]), "v"(p_out[1]), "v"(ls));
        // softmax, part 3: a row sum beyond 2^16 (or not finite) means some p outgrew the
        // reference. Rare after a row's first tiles: move the reference to the row max of
        // this sub-block (and the old reference), redo the exponentials, and rescale O and l
        // by alpha like a tracked move. Exact either way: O and l share the reference.
        if (__any(!(ls <= P_LIMIT))) {
          float mx = s_in[0];
#pragma unroll
          for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s_in[r]);
          mx = wave_max_xor32(mx);
          const float m_new = fmaxf(mx, m_used);
          alpha = fast_exp2((m_used - m_new) * c);
          m_used = m_new;
          move = true;
          ca = -m_new * c;
          // O (with this step's PV of the previous sub-block, at the old reference) and the
          // row sum move now
          scale_acc(oacc, alpha);
          lsum *= alpha;
          ls = exps();
        }
      }
      // (TRACK decided its move before the exponentials; the other forms rescaled lsum in the
      // redo branch, so their common path is one add)
      if constexpr (TRACK) lsum = __builtin_fmaf(lsum, alpha, ls);
      else lsum += ls;
      // keep the exponentials in this step's block (not sunk into the next one)
      asm volatile("" ::"v"(p_out[0]), "v"(p_out[1]), "v"(lsum));
      pend = TRACK && move;  // (the other forms have rescaled O in the redo branch)
      alpha_p = alpha;
    };

    // Tile u lives in stage u % NSTAGE (K at stage*16 KB, V at V_BASE + stage*16 KB).
    // Step 2u: softmax of tile u half 0, PV of tile u-1 half 1, S of tile u half 1.
    // Step 2u+1: softmax of tile u half 1, PV of tile u half 0, S of tile u+1 half 0.
    // Between them: wait for tile u+1, barrier (every wave is past its reads of tile u-1),
    // refill tile u-1's stage with tile u+NSTAGE-1.
    // K tile bytes in LDS (bf16 16 KB, fp8 8 KB) and one sub-block's
    constexpr int KT_B = FP8 ? TILE8_B : TILE_B, KH_B = KT_B / 2;
    auto tile = [&](auto st_c, int u) {
      constexpr int ST = decltype(st_c)::value;
      constexpr int SP = (ST + NSTAGE - 1) % NSTAGE;  // stage of tile u-1
      constexpr int SN = (ST + 1) % NSTAGE;           // stage of tile u+1
      const int vrow = vr[0];

      if constexpr (FP8) {
        // Copies in flight per lane, in issue order: staged V of tile u+1 (2, issued at the
        // start of tile u-1), K of tile u+1 (1, after tile u-1's barrier). Tile u+1's V goes
        // into its stage, the one tile u-2 left: free since the last barrier and not read
        // before the next one. Then tile u+2's V and scales into the slot tile u's left.
        if (u + 1 < T) {
          wait_vm(1);
          convert_v((u + 1) & 1, SN, kser[1]);
        }
        if (u + 2 < T) vr[2] = SEGN > 0 ? issue_raw1(u & 1, u + 2) : issue_raw(u & 1);
      }
      // step 2u reads the V fragments of step 2u+1 (tile u, already resident); step 2u+1 reads
      // those of step 2u+2 (tile u+1 rows 32..63, resident since the barrier, and tile u)
      if (wave_active)
        step(std::integral_constant<int, ST * KT_B + KH_B>{},
             std::integral_constant<int, SP * TILE_B + HALF_B>{}, std::true_type{},
             std::true_type{}, std::integral_constant<int, -1>{},
             std::integral_constant<int, ST * TILE_B>{}, sA, sB, pA, pB, 0, vrow, kser[0]);
      if constexpr (FP8) {
        if (u + 1 < T) wait_vm(u + 2 < T ? 2 : 0);  // tile u+1's K (tile u+2's V may be in flight)
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the V conversion's writes are done
      } else {
        if (u + 1 < T) wait_tiles_outstanding(min(NSTAGE - 3, T - 2 - u));
      }
      barrier_nofence();
      if constexpr (FP8) {
        if (u + 2 < T) {
          if constexpr (SEGN > 0) issue_k81(SP, u + 2);
          else issue_k8(SP);
        }
      } else {
        if (u + NSTAGE - 1 < T) vr[NSTAGE - 1] = SEGN > 0 ? issue1(SP, u + NSTAGE - 1) : issue(SP);
      }
      if (wave_active)
        step(std::integral_constant<int, SN * KT_B>{},
             std::integral_constant<int, ST * TILE_B>{}, std::false_type{}, std::true_type{},
             std::integral_constant<int, SN * KT_B + KH_B>{},
             std::integral_constant<int, ST * TILE_B + HALF_B>{}, sB, sA, pB, pA, 1, vrow, kser[1]);
#pragma unroll
      for (int k = 0; k < NSTAGE - 1; ++k) {
        vr[k] = vr[k + 1];
        kser[k] = kser[k + 1];
      }
    };

#pragma unroll 1
    for (int u = 0; u < T; u += NSTAGE) {
      tile(std::integral_constant<int, 0>{}, u);
      if (u + 1 < T) tile(std::integral_constant<int, 1>{}, u + 1);
      if (u + 2 < T) tile(std::integral_constant<int, 2>{}, u + 2);
    }

    // drain: O += V^T P^T of the last sub-block (tile T-1 half 1, P in pA)
    if (wave_active) {
      if (pend) scale_acc(oacc, alpha_p);
      const int vo = ((T - 1) % NSTAGE) * TILE_B + HALF_B;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int db = i >> 1, m = i & 1;
        const u32x2 v0 = lds_read_tr16(voff[db][0] + vo + 16 * m * ROWB);
        const u32x2 v1 = lds_read_tr16(voff[db][1] + vo + 16 * m * ROWB);
        oacc[db] = mfma32x32x16(u32x4{v0[0], v0[1], v1[0], v1[1]}, pA[m], oacc[db]);
      }
    }
  }

  // Every wave is past its last LDS reads (the drain) before the LDS is reused for staging O.
  barrier_nofence();
  // (with the in-kernel merge every wave stays for the unit's arrival count)
  const bool fused = a.mode == kModePartials && a.merge_cnt != nullptr;
  if (!wave_active && !fused) return;

  // ---- epilogue
  // (a workgroup with no tiles still has its Q loads outstanding)
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  const float l_tot = wave_sum_xor32(lsum);
  // O leaves through this wave's 8 KB of LDS, 32 rows of 256 B with 16-byte chunk c of row r
  // at physical chunk c ^ (r & 15), and is written back as whole rows, 16 lanes per 256-byte
  // row segment: 4x fewer cache lines per store than storing the MFMA layout directly (lane
  // (l32, hl) holds d = 32db + 8g + 4hl .. +3 of row l32).
  unsigned char* stg = lds + 8192 * wave;
  const int rrow = lane >> 4, rch = lane & 15;  // read side: row in a 4-row group, chunk
  if (a.mode == kModeNormalized && !a.o32) {
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 w;
        w[0] = pack_bf16x2(oacc[db][4 * g + 0] * inv, oacc[db][4 * g + 1] * inv);
        w[1] = pack_bf16x2(oacc[db][4 * g + 2] * inv, oacc[db][4 * g + 3] * inv);
        *reinterpret_cast<u32x2*>(stg + l32 * 256 + (((4 * db + g) ^ (l32 & 15)) << 4) + 8 * hl) = w;
      }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int r = 4 * k + rrow;
      const u32x4 v = *reinterpret_cast<const u32x4*>(stg + r * 256 + ((rch ^ (r & 15)) << 4));
      const int qq = q0 + r;
      if (qq < a.Lq) {
        uint16_t* op = a.out + a.osb * b + a.osl * (int64_t)qq + a.osh * h + 8 * rch;
        if (a.o16) {
          *reinterpret_cast<u32x4*>(op) = v;
        } else {
          *reinterpret_cast<u32x2*>(op) = u32x2{v[0], v[1]};
          *reinterpret_cast<u32x2*>(op + 4) = u32x2{v[2], v[3]};
        }
      }
    }
  } else if (wave_active) {
    // fp32 rows: the normalised output of an fp32-output call, or the partials.
    // cte_partial contract (TRACK): O and l relative to the true row max, m in scaled units;
    // the split-KV partials for lbw's own merge keep the exponent reference instead.
    const bool norm32 = a.mode == kModeNormalized;
    float f = 1.0f;
    float m_out = -INFINITY;
    if (norm32) {
      f = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    } else if (l_tot > 0.0f) {
      if constexpr (TRACK) {
        f = fast_exp2((m_used - m_true) * c);
        m_out = m_true * a.scale;
      } else if constexpr (FOLD) {
        m_out = mref * a.scale;
      } else {
        m_out = m_used * a.scale;
      }
    }
    const int64_t row0 = ((int64_t)(split * a.B + b) * a.H + h) * a.Lq;
    const int q = q0 + l32;
    if (!norm32 && q < a.Lq && hl == 0) {
      if (fused) {
        store_dev(a.part_m + row0 + q, m_out);
        store_dev(a.part_l + row0 + q, l_tot * f);
      } else {
        a.part_m[row0 + q] = m_out;
        a.part_l[row0 + q] = l_tot * f;
      }
    }
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.part_o + row0 * D), (short)0, 0x7fffffff, 0x00020000);
    float* const out32 = reinterpret_cast<float*>(a.out) + a.osb * b + a.osh * h;
    // fp32 O in two halves of 64 d (256 B per row each)
#pragma unroll
    for (int half = 0; half < 2; ++half) {
#pragma unroll
      for (int dbh = 0; dbh < 2; ++dbh)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int db = 2 * half + dbh;
          floatx4 w;
          w[0] = oacc[db][4 * g + 0] * f;
          w[1] = oacc[db][4 * g + 1] * f;
          w[2] = oacc[db][4 * g + 2] * f;
          w[3] = oacc[db][4 * g + 3] * f;
          const int cc = 8 * dbh + 2 * g + hl;  // 16-byte chunk of the half-row
          *reinterpret_cast<floatx4*>(stg + l32 * 256 + ((cc ^ (l32 & 15)) << 4)) = w;
        }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int r = 4 * k + rrow;
        const floatx4 v = *reinterpret_cast<const floatx4*>(stg + r * 256 + ((rch ^ (r & 15)) << 4));
        const int qq = q0 + r;
        if (qq < a.Lq) {
          if (fused) {
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rp,
                                                   (uint32_t)(qq * D + 64 * half + 4 * rch) * 4u,
                                                   0, kDevScope);
          } else {
            float* dst = norm32 ? out32 + a.osl * (int64_t)qq : a.part_o + (row0 + qq) * D;
            *reinterpret_cast<floatx4*>(dst + 64 * half + 4 * rch) = v;
          }
        }
      }
    }
  }
  if (fused) {
    // The last piece of the unit to arrive merges the unit's partials: every store of this
    // workgroup is complete at device scope before its one arrival is counted, and the last
    // arrival reads the others' partials at device scope after its count returned.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __shared__ int s_last;
    __syncthreads();
    if (threadIdx.x == 0)
      s_last = __hip_atomic_fetch_add(a.merge_cnt + unit, 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)a.splits - 1u;
    __syncthreads();
    if (!s_last) return;
    const int rows = min(BM, a.Lq - qt * BM);
    float* wl = reinterpret_cast<float*>(lds + V_BASE);
    switch (a.splits) {
      case 2: merge_unit<2>(a, b, h, qt, rows, wl); break;
      case 3: merge_unit<3>(a, b, h, qt, rows, wl); break;
      case 4: merge_unit<4>(a, b, h, qt, rows, wl); break;
      case 5: merge_unit<5>(a, b, h, qt, rows, wl); break;
      case 6: merge_unit<6>(a, b, h, qt, rows, wl); break;
      case 7: merge_unit<7>(a, b, h, qt, rows, wl); break;
      default: merge_unit<8>(a, b, h, qt, rows, wl); break;
    }
  }
}

}  // namespace

template <bool FP8, bool TRACK, bool FOLD = false, int SEGN = 0, bool KDM = false, bool BIAS = false>
static hipError_t launch(const AttnKernelArgs& a, hipStream_t stream) {
  static hipError_t attr = hipFuncSetAttribute(
      (const void*)attn_fwd_bf16_kernel<FP8, TRACK, FOLD, SEGN, KDM, BIAS>,
      hipFuncAttributeMaxDynamicSharedMemorySize, LDS_B);
  if (attr != hipSuccess) return attr;
  const uint32_t U = (uint32_t)a.n_qtiles * a.H * a.B;
  const uint32_t per_xcd = a.splits * ((U + 7u) / 8u);  // items of the largest XCD share
  uint32_t nwg = 8u * per_xcd;
  if (a.queue != nullptr) {
    // spare workgroups, 1/16 of an XCD's share (at least one each): enough for the measured
    // spread of XCD speeds (a few percent)
    nwg += 8u * ((per_xcd + 15u) / 16u);
    // the 8 queue counters and, for the in-kernel merge, the U arrival counters after them
    const int n = 8 + (a.merge_cnt != nullptr ? (int)U : 0);
    hipLaunchKernelGGL(attn_queue_reset_kernel, dim3((n + 255) / 256 < 64 ? (n + 255) / 256 : 64),
                       dim3(256), 0, stream, a.queue, n);
  }
  hipLaunchKernelGGL((attn_fwd_bf16_kernel<FP8, TRACK, FOLD, SEGN, KDM, BIAS>), dim3(nwg),
                     dim3(NWAVE * 64), LDS_B, stream, a);
  return hipGetLastError();
}

// Segments the index-addressed copies take: 1, 2 (with equal row strides), or 0 for the cursor.
static int index_segments(const AttnKernelArgs& a) {
  if (a.mult_key >= 0) return 0;
  if (a.nseg == 1) return 1;
  if (a.nseg == 2 && a.seg[0].ksl == a.seg[1].ksl && a.seg[0].vsl == a.seg[1].vsl) return 2;
  return 0;
}

hipError_t launch_attn_fwd(const AttnKernelArgs& a, hipStream_t stream) {
  if (a.key_bias != nullptr) {  // a per-key bias: the plain form (any scale), general cursor
    return a.k_dmajor ? launch<false, false, false, 0, true, true>(a, stream)
                      : launch<false, false, false, 0, false, true>(a, stream);
  }
  if (a.k_dmajor) {  // d-major K: the general cursor
    if (a.track_max) return launch<false, true, false, 0, true>(a, stream);
    if (a.scale_log2 == 1.0f) return launch<false, false, true, 0, true>(a, stream);
    return launch<false, false, false, 0, true>(a, stream);
  }
  if (a.track_max) return launch<false, true>(a, stream);
  // a pre-scaled q (scale * log2(e) exactly 1 in fp32) takes the folded softmax
  const int segn = index_segments(a);
  if (a.scale_log2 == 1.0f) {
    if (segn == 1) return launch<false, false, true, 1>(a, stream);
    if (segn == 2) return launch<false, false, true, 2>(a, stream);
    return launch<false, false, true>(a, stream);
  }
  if (segn == 1) return launch<false, false, false, 1>(a, stream);
  if (segn == 2) return launch<false, false, false, 2>(a, stream);
  return launch<false, false>(a, stream);
}

hipError_t launch_attn_fwd_fp8(const AttnKernelArgs& a, hipStream_t stream) {
  if (a.track_max) return launch<true, true>(a, stream);
  const bool one = index_segments(a) == 1;
  if (a.scale_log2 == 1.0f)  // a pre-scaled q: the folded softmax
    return one ? launch<true, false, true, 1>(a, stream) : launch<true, false, true>(a, stream);
  return one ? launch<true, false, false, 1>(a, stream) : launch<true, false>(a, stream);
}

}  // namespace lbw
