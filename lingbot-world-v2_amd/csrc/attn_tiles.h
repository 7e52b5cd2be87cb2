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

struct TileInfo {
  const unsigned char* kbase;  // row 0 of the segment for (b, h)
  const unsigned char* vbase;
  int64_t ks, vs;              // row strides in bytes
  int64_t row0;                // first segment-local row of the tile
  int vlo, vhi;                // valid rows of the tile
  float sk, sv;                // fp8 block scales
};

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
  int n = 0;
#pragma unroll 1
  for (int i = 0; i < a.nseg; ++i) {
    int64_t la = 0, lb = 0;
    n += seg_tiles(a.seg[i], lo, hi, la, lb);
  }
  return n;
}

template <int ESZ, bool SCALES>
__device__ __forceinline__ TileInfo tile_info(const AttnKernelArgs& a, int64_t lo, int64_t hi,
                                              int g, int b, int h) {
  // Find the segment holding tile g (uniform loop: descriptors are read on demand).
  int cum = 0, i = 0;
  int64_t la = 0, lb = 0;
#pragma unroll 1
  for (; i < a.nseg - 1; ++i) {
    const int n = seg_tiles(a.seg[i], lo, hi, la, lb);
    if (g < cum + n) break;
    cum += n;
  }
  const SegDesc& s = a.seg[i];
  seg_tiles(s, lo, hi, la, lb);
  TileInfo ti;
  const int64_t lt = la / BN + (g - cum);
  constexpr int esz = ESZ;
  ti.kbase = reinterpret_cast<const unsigned char*>(s.k) + (s.ksb * b + s.ksh * h) * esz;
  ti.vbase = reinterpret_cast<const unsigned char*>(s.v) + (s.vsb * b + s.vsh * h) * esz;
  ti.ks = s.ksl * esz;
  ti.vs = s.vsl * esz;
  ti.row0 = lt * BN;
  const int64_t vlo = la - ti.row0, vhi = lb - ti.row0;
  ti.vlo = vlo > 0 ? (int)vlo : 0;
  ti.vhi = vhi < BN ? (int)vhi : BN;
  if constexpr (SCALES) {
    const int64_t bi = ((int64_t)b * a.H + h) * s.nblk + lt;
    ti.sk = s.ks[bi];
    ti.sv = s.vs[bi];
  } else {
    ti.sk = 1.0f;
    ti.sv = 1.0f;
  }
  return ti;
}

// Sequential walk over the tiles of [lo, hi), in order. The segment descriptors (kernel
// arguments) are read only when the walk enters a new segment, so stepping to the next tile
// is a handful of scalar instructions.
struct TileCursor {
  int seg;                    // current segment; nseg when the walk is past the last tile
  int64_t lt, lt_end;         // current and one-past-last local tile of the segment
  int64_t la, lb;             // valid local key range of the segment
  const unsigned char* kbase; // row 0 of the segment for (b, h)
  const unsigned char* vbase;
  int64_t ks, vs;             // row strides in bytes
  const float* ksc;           // fp8 block scales of (b, h) (fp8 cache only)
  const float* vsc;
};

template <int ESZ>
__device__ __forceinline__ void cursor_enter(const AttnKernelArgs& a, int i, int64_t la,
                                             int64_t lb, int b, int h, TileCursor& c) {
  const SegDesc& s = a.seg[i];
  c.seg = i;
  c.la = la;
  c.lb = lb;
  c.lt = la / BN;
  c.lt_end = (lb + BN - 1) / BN;
  c.kbase = reinterpret_cast<const unsigned char*>(s.k) + (s.ksb * b + s.ksh * h) * ESZ;
  c.vbase = reinterpret_cast<const unsigned char*>(s.v) + (s.vsb * b + s.vsh * h) * ESZ;
  c.ks = s.ksl * ESZ;
  c.vs = s.vsl * ESZ;
  const int64_t so = ((int64_t)b * a.H + h) * s.nblk;
  c.ksc = s.ks != nullptr ? s.ks + so : nullptr;
  c.vsc = s.vs != nullptr ? s.vs + so : nullptr;
}

// Positions the cursor on tile g of the walk (the g-th tile holding keys of [lo, hi)).
template <int ESZ>
__device__ __forceinline__ void cursor_init(const AttnKernelArgs& a, int64_t lo, int64_t hi,
                                            int g, int b, int h, TileCursor& c) {
  int cum = 0;
  c.seg = a.nseg;
#pragma unroll 1
  for (int i = 0; i < a.nseg; ++i) {
    int64_t la = 0, lb = 0;
    const int n = seg_tiles(a.seg[i], lo, hi, la, lb);
    if (g < cum + n) {
      cursor_enter<ESZ>(a, i, la, lb, b, h, c);
      c.lt += g - cum;
      return;
    }
    cum += n;
  }
}

// Advances to the next tile; returns true when the cursor entered a new segment.
template <int ESZ>
__device__ __forceinline__ bool cursor_next(const AttnKernelArgs& a, int64_t lo, int64_t hi,
                                            int b, int h, TileCursor& c) {
  if (++c.lt < c.lt_end) return false;
#pragma unroll 1
  for (int i = c.seg + 1; i < a.nseg; ++i) {
    int64_t la = 0, lb = 0;
    if (seg_tiles(a.seg[i], lo, hi, la, lb) > 0) {
      cursor_enter<ESZ>(a, i, la, lb, b, h, c);
      return true;
    }
  }
  c.seg = a.nseg;
  return true;
}

// Valid rows [vlo, vhi) of the cursor's tile.
__device__ __forceinline__ void cursor_rows(const TileCursor& c, int& vlo, int& vhi) {
  const int64_t row0 = c.lt * BN;
  const int64_t l = c.la - row0, u = c.lb - row0;
  vlo = l > 0 ? (int)l : 0;
  vhi = u < BN ? (int)u : BN;
}

}  // namespace lbw
