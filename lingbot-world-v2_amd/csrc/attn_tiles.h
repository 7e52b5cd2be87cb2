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

}  // namespace lbw
