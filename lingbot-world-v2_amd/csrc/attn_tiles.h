// Tile walk over the KV segments of an attention call (shared by the attention kernels).
//
// Segment i contributes the local key range [la, lb) = ([lo, hi) n [start, start+len)) - start
// and the 64-key tiles floor(la/64) .. ceil(lb/64) - 1 of its own token grid, so a tile never
// straddles two segments and (fp8 cache) covers exactly one 64-token scale block.
#pragma once

#include "common.h"
#include "attn_fwd.h"

namespace lbw {

constexpr int D = 128;
constexpr int BN = 64;
constexpr float TAU = 8.0f;  // lazy-rescale threshold, log2 units
constexpr float M_INIT = -1e30f;  // initial exponent reference (finite stand-in for -inf)
constexpr float P_LIMIT = 65536.0f;  // largest per-lane row sum before the reference moves

// ---- helpers shared by the attention kernels

// LDS row swizzle of the 256-byte K/V rows: 16-byte chunk c of row r is stored at chunk
// c ^ swz(r), which makes the K row reads and the V transpose reads conflict-free.
__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

typedef short shortx4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) shortx4 lds_shortx4;

typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) u32x2 lds_u32x2;

// LDS reads at an integer LDS byte address, so the constant part of an address folds into the
// instruction's offset field.
__device__ __forceinline__ u32x2 lds_read_tr16(int addr) {
  const shortx4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(uintptr_t)addr);
  return __builtin_bit_cast(u32x2, v);
}
__device__ __forceinline__ u32x4 lds_read_b128(int addr) {
  return *(const lds_u32x4*)(uintptr_t)addr;
}
__device__ __forceinline__ u32x2 lds_read_b64(int addr) {
  return *(const lds_u32x2*)(uintptr_t)addr;
}

// 16 bytes per lane HBM -> LDS (global_load_lds_dwordx4): lane l's bytes from sbase + voff land
// at LDS byte address lds_dst + 16 l. Inline asm rather than the builtin: the compiler's wait
// insertion treats an in-flight builtin copy as a hazard for every later LDS transpose read and
// waits for all copies before each one, which would serialise the prefetch. The kernel waits
// for the tiles it reads itself (wait_tiles_outstanding, then a barrier).
// The compiler does not insert the wait states an instruction inside inline asm needs: a vector
// memory instruction must not read an SGPR within 5 wait states of a VALU write of it (such as
// a v_readlane reload of a spilled SGPR, or a v_readfirstlane). The build checks the assembly of
// every kernel for that (check_dma_hazards.py); a copy it flags takes dma16_guarded.
__device__ __forceinline__ void dma16(const unsigned char* sbase, uint32_t voff, uint32_t lds_dst) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds_dst) : "memory");
}
// dma16 with the 5 wait states ahead of the copy (where the base may have been written by a
// VALU instruction just before)
__device__ __forceinline__ void dma16_guarded(const unsigned char* sbase, uint32_t voff,
                                              uint32_t lds_dst) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds_dst)
               : "memory");
}
// 4 bytes per lane from a per-lane 64-bit address (global_load_lds_dword): lane l's dword lands
// at LDS byte address lds_dst + 4 l.
__device__ __forceinline__ void dma4(uint64_t addr, uint32_t lds_dst) {
  asm volatile("global_load_lds_dword %0, off" ::"v"(addr), "{m0}"(lds_dst) : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const unsigned char* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) unsigned char*)p;
}

// Materialises a kernel argument in a scalar register at this point. Its scalar load is then
// waited for here, before the main loop: a scalar load still pending inside the loop (scalar
// loads complete out of order) turns every LDS wait there into a wait for all LDS reads.
__device__ __forceinline__ float sreg(float x) {
  asm volatile("" : "+s"(x));
  return x;
}
__device__ __forceinline__ int sreg(int x) {
  asm volatile("" : "+s"(x));
  return x;
}

// Hides a value from the optimiser (keeps a base register from being re-associated with
// constant offsets that would no longer fit the 16-bit LDS immediate).
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Scores of keys outside the tile's valid rows [tvlo, tvhi) -> -inf (S^T register layout);
// rows from mrow on get `add` (the log-multiplicity of deduplicated keys).
// Sign-bit arithmetic on per-lane integers instead of one comparison mask per element: the
// sixteen 64-bit lane masks would otherwise all be live in scalar registers at once.
__device__ __forceinline__ void mask_scores(floatx16& sc, int kb, int tvlo, int tvhi, int hl,
                                            int mrow, float add) {
  asm volatile("" ::: "memory");
  const int k0 = 32 * kb + 4 * hl;  // key of register 0 in this lane
  const int a = k0 - tvlo, bnd = tvhi - 1 - k0, cm = k0 - mrow;
  const uint32_t addb = __float_as_uint(add);
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int o = 8 * (r >> 2) + (r & 3);              // key - k0 of register r
    const uint32_t out = (uint32_t)(((a + o) | (bnd - o)) >> 31);  // ~0: key outside [tvlo, tvhi)
    const uint32_t biased = ~(uint32_t)((cm + o) >> 31);           // ~0: key >= mrow
    const float x = sc[r] + __uint_as_float(addb & biased);
    sc[r] = __uint_as_float((__float_as_uint(x) & ~out) | (0xff800000u & out));
  }
}

__device__ __forceinline__ void scale_acc(floatx16 (&o)[4], float alpha) {
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
}


// ---- tile walk

__device__ __forceinline__ int seg_tiles(const SegDesc& s, int64_t lo, int64_t hi, int64_t& la,
                                         int64_t& lb) {
  if (s.len <= 0) return 0;
  const int64_t st = s.start, en = s.start + s.len;
  const int64_t a = lo > st ? lo : st;
  const int64_t e = hi < en ? hi : en;
  if (e <= a) return 0;
  la = a - st;
  lb = e - st;
  return (int)((lb + BN - 1) / BN - la / BN);
}

__device__ __forceinline__ int count_tiles(const AttnKernelArgs& a, int64_t lo, int64_t hi) {
  if (a.nseg == 1) {  // the common call: a constant index lets the descriptor loads batch early
    int64_t la = 0, lb = 0;
    return seg_tiles(a.seg[0], lo, hi, la, lb);
  }
  int n = 0;
#pragma unroll 1
  for (int i = 0; i < a.nseg; ++i) {
    int64_t la = 0, lb = 0;
    n += seg_tiles(a.seg[i], lo, hi, la, lb);
  }
  return n;
}

// Packed valid rows of a tile: rows [vlo, vhi) hold keys of the window, rows from mrow on carry
// the multiplicity bias (255: none). ROWS_FULL: every row valid, no bias.
__host__ __device__ constexpr int pack_rows(int vlo, int vhi, int mrow) {
  return vlo | (vhi << 8) | (mrow << 16);
}
constexpr int ROWS_FULL = pack_rows(0, BN, 255);

// Sequential walk over the tiles of [lo, hi), in order. Stepping to the next tile of the same
// segment advances two tile pointers; only the first and last tile of a segment (and every tile
// of a call with a multiplicity bias) recompute their valid rows, and only entering a new segment
// reads its descriptor. Segment-local indices are 32-bit (the host limits segments to 2^30 keys).
struct TileCursor {
  const unsigned char* kt;  // row 0 of the current tile, K and V, for (b, h)
  const unsigned char* vt;
  const float* ksc;         // fp8 block scales of the current tile (fp8 cache only)
  const float* vsc;
  uint32_t kstep, vstep;    // bytes per tile (BN rows; the host keeps them below 4 GiB)
  uint32_t ks, vs;          // row strides in bytes
  int seg;                  // current segment; nseg when the walk is past the last tile
  int lt, lt_end;           // current and one-past-last local tile of the segment
  int la, lb;               // valid local key range of the segment
  int rows;                 // packed valid rows of the current tile (pack_rows)
};

// Valid rows of the cursor's tile and, when mult_key >= 0, the first row of the keys that stand
// for several identical keys.
__device__ __forceinline__ int cursor_rows(const AttnKernelArgs& a, const TileCursor& c) {
  const int row0 = c.lt * BN;
  const int l = c.la - row0, u = c.lb - row0;
  const int vlo = l > 0 ? l : 0;
  const int vhi = u < BN ? u : BN;
  int mrow = 255;
  if (a.mult_key >= 0) {
    const int64_t r = a.mult_key - (a.seg[c.seg].start + row0);
    if (r < vhi) mrow = r > vlo ? (int)r : vlo;
  }
  return pack_rows(vlo, vhi, mrow);
}

template <int ESZ>
__device__ __forceinline__ void cursor_enter(const AttnKernelArgs& a, int i, int64_t la,
                                             int64_t lb, int b, int h, int lt, TileCursor& c) {
  const SegDesc& s = a.seg[i];
  c.seg = i;
  c.la = (int)la;
  c.lb = (int)lb;
  c.lt = lt;
  c.lt_end = (int)((lb + BN - 1) / BN);
  // (d-major K: ks is the byte stride of its d-rows and a tile starts BN tokens further along
  // each row)
  c.ks = (uint32_t)((s.ksd != 0 ? s.ksd : s.ksl) * ESZ);
  c.vs = (uint32_t)(s.vsl * ESZ);
  c.kstep = (uint32_t)((s.ksd != 0 ? 1 : s.ksl) * ESZ * BN);
  c.vstep = (uint32_t)(s.vsl * ESZ * BN);
  c.kt = reinterpret_cast<const unsigned char*>(s.k) + (s.ksb * b + s.ksh * h) * ESZ +
         (int64_t)lt * c.kstep;
  c.vt = reinterpret_cast<const unsigned char*>(s.v) + (s.vsb * b + s.vsh * h) * ESZ +
         (int64_t)lt * c.vstep;
  const int64_t so = ((int64_t)b * a.H + h) * s.nblk + lt;
  c.ksc = s.ks != nullptr ? s.ks + so : nullptr;
  c.vsc = s.vs != nullptr ? s.vs + so : nullptr;
  c.rows = cursor_rows(a, c);
}

// Positions the cursor on tile g of the walk (the g-th tile holding keys of [lo, hi)).
template <int ESZ>
__device__ __forceinline__ void cursor_init(const AttnKernelArgs& a, int64_t lo, int64_t hi,
                                            int g, int b, int h, TileCursor& c) {
  int cum = 0;
  c.seg = a.nseg;
  if (a.nseg == 1) {
    int64_t la = 0, lb = 0;
    const int n = seg_tiles(a.seg[0], lo, hi, la, lb);
    if (g < n) cursor_enter<ESZ>(a, 0, la, lb, b, h, (int)(la / BN) + g, c);
    return;
  }
#pragma unroll 1
  for (int i = 0; i < a.nseg; ++i) {
    int64_t la = 0, lb = 0;
    const int n = seg_tiles(a.seg[i], lo, hi, la, lb);
    if (g < cum + n) {
      cursor_enter<ESZ>(a, i, la, lb, b, h, (int)(la / BN) + g - cum, c);
      return;
    }
    cum += n;
  }
}

// Advances to the next tile; returns true when the cursor entered a new segment (or ran past
// the last one). `mult` (kernel-uniform, nonzero): the call carries a multiplicity bias.
template <int ESZ>
__device__ __forceinline__ bool cursor_next(const AttnKernelArgs& a, int64_t lo, int64_t hi,
                                            int b, int h, int mult, TileCursor& c) {
  if (++c.lt < c.lt_end) {
    c.kt += c.kstep;
    c.vt += c.vstep;
    if constexpr (ESZ == 1) {
      ++c.ksc;
      ++c.vsc;
    }
    c.rows = (c.lt + 1 < c.lt_end && !mult) ? ROWS_FULL : cursor_rows(a, c);
    return false;
  }
#pragma unroll 1
  for (int i = c.seg + 1; i < a.nseg; ++i) {
    int64_t la = 0, lb = 0;
    if (seg_tiles(a.seg[i], lo, hi, la, lb) > 0) {
      cursor_enter<ESZ>(a, i, la, lb, b, h, (int)(la / BN), c);
      return true;
    }
  }
  c.seg = a.nseg;
  return true;
}

}  // namespace lbw
