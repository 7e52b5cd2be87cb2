// Cross-attention of the chunk's queries to a short context (gfx950), kernel 3 of the path: the
// reference's wan_cross_attn (kernels/cross_attention.py:17-123) behind _nki_cross_attention
// (wan/modules/attention.py:280-311), a single softmax over the (<= 512) context keys.
//
// out = softmax(scale Q K^T) V over the keys [lo, hi) of one context segment; hi is limited per
// batch by k_lens (the masked mode), and for the exact dedup of attention.py:493-554 the keys from
// mult_key on carry the log of their multiplicity (mult_raw, added to their raw scores).
//
// Schedule: persistent workgroups (one per CU, 8 waves). The work is cut into rounds, a round
// being 256 queries (8 waves x 32) of one (batch, head); workgroup g runs a contiguous range of
// the rounds, in (batch, head)-major order, and XCD x holds an eighth of the range, so the heads
// of an XCD share its L2. The K and V rows of the round's (batch, head) -- up to 320 keys -- sit
// in LDS whole (160 KB: the CU's entire LDS) and stay there across the consecutive rounds of that
// head: loaded once per head and workgroup, and within a head the waves run their queries with
// no barrier at all, so one wave's Q loads and output stores overlap the MFMA work of the
// others. A context longer than 320 keys is processed in 320-key chunks, every round reloading
// every chunk (a barrier around each load), the per-wave softmax state carrying across chunks.
//
// Per wave the arithmetic is the chunk kernel's (attn_fwd_bf16.hip): S^T = K Q^T and
// O^T = V^T P^T with v_mfma_f32_32x32x16_bf16 (one query per lane column, Q in registers, K rows
// and V^T fragments from the swizzled LDS rows), an online softmax in base 2 against an exponent
// reference that moves lazily (a sub-block whose row sum passes 2^16 moves it to the row max and
// redoes its exponentials; O and l share the reference, so O / l is exact), and the softmax of
// sub-block j on the VALU overlapping the MFMAs of S_{j+1} and PV_{j-1}.

#include "attn_tiles.h"

namespace lbw {
namespace {

constexpr int XW = 8;                     // waves per workgroup
constexpr int XCH = 320;                  // keys resident in LDS per chunk
constexpr int XSB = XCH / 32;             // 32-key sub-blocks per chunk
constexpr int XROWB = D * 2;              // bytes per K/V row
constexpr int XSUBB = 32 * XROWB;         // bytes per sub-block (8 KB)
constexpr int XV0 = XCH * XROWB;          // V rows follow the K rows (80 KB)
constexpr int XLDS = 2 * XCH * XROWB;     // 160 KB
constexpr int XKA = 2, XVA = 2;           // MFMA pairs ahead that K / V fragments are read
constexpr int XKR = XKA + 2, XVR = XVA + 2;
static_assert(8 % XKR == 0 && 8 % XVR == 0, "fragment rings must divide 8");
static_assert(XLDS <= 160 * 1024, "K and V chunks must fit the LDS");

// K sub-block j lies at j * 8 KB, V sub-block j at XV0 + j * 8 KB. An LDS read's immediate offset reaches 64 KB, less than a chunk's 80 KB of K (or V) rows: the
// K bases move up by 5 sub-blocks at the start of step XKSW and the V bases at step XVSW (and
// back after the chunk), so that every read of step J, of sub-block SB, is a base register plus
// the immediate (SB - shift(J)) * 8 KB < 64 KB.
constexpr int XKSW = 6, XVSW = 8;
constexpr int XSHIFT = 5 * XSUBB;
template <int J, int SB> constexpr int k_off() { return (SB - (J >= XKSW ? 5 : 0)) * XSUBB; }
template <int J, int SB> constexpr int v_off() { return (SB - (J >= XVSW ? 5 : 0)) * XSUBB; }
template <int V> using I = std::integral_constant<int, V>;

// A wave-uniform int32 read through the scalar cache. As a vector load, the compiler waits for
// it with vmcnt(0), which would also wait for the Q prefetch and the output stores in flight.
__device__ __forceinline__ int load_scalar_i32(const int32_t* p) {
  int v;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
  return v;
}

// OUT: the output form, a template parameter so that the epilogue has one store sequence and
// the compiler counts its stores exactly. 0: bf16 with 16-byte stores (aligned out, strides
// multiples of 8); 1: bf16 with 8-byte stores; 2: fp32.
enum { kOutBf16x16 = 0, kOutBf16x8 = 1, kOutF32 = 2 };

// O / l of one wave's 32 query rows q0 .. q0 + 31 of (b, h), straight from the registers: lane
// (l32, hl) holds d = 32 db + 8 g + 4 hl .. +3 of query q0 + l32 (registers 4g .. 4g + 3 of
// oacc[db]); one exchange with lane ^ 32 (v_permlane32_swap, no LDS) gives each lane 8
// consecutive d (16 bytes) for the bf16 store. Rows past Lq store nothing: the buffer range check
// drops them.
template <int OUT>
__device__ __forceinline__ void store_rows(const AttnKernelArgs& a, int b, int h, int q0,
                                           const floatx16 (&oacc)[4], float lsum, int l32, int hl) {
  const float l_tot = wave_sum_xor32(lsum);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  const int q = q0 + l32;
  constexpr int esz = OUT == kOutF32 ? 4 : 2;
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(reinterpret_cast<unsigned char*>(a.out) + (a.osb * b + a.osh * h) * esz), (short)0,
      (int)((uint32_t)a.Lq * (uint32_t)(a.osl * esz)), 0x00020000);
  const uint32_t orow = (uint32_t)(q * a.osl) * (uint32_t)esz;
  if constexpr (OUT == kOutF32) {
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        floatx4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = oacc[db][4 * g + e] * inv;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, w), ro,
                                               orow + 4 * (32 * db + 8 * g + 4 * hl), 0, 0);
      }
  } else {
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int gx = 2 * k, gy = 2 * k + 1;
        const uint32_t x0 = pack_bf16x2(oacc[db][4 * gx] * inv, oacc[db][4 * gx + 1] * inv);
        const uint32_t x1 = pack_bf16x2(oacc[db][4 * gx + 2] * inv, oacc[db][4 * gx + 3] * inv);
        const uint32_t y0 = pack_bf16x2(oacc[db][4 * gy] * inv, oacc[db][4 * gy + 1] * inv);
        const uint32_t y1 = pack_bf16x2(oacc[db][4 * gy + 2] * inv, oacc[db][4 * gy + 3] * inv);
        // the swap of (x, y) leaves in lane l < 32 its own x and lane l + 32's x, in lane l + 32
        // lane l's y and its own y: d 32 db + 16 k + 8 hl .. +7 of the row in both halves
        const u32x2 s0 = __builtin_bit_cast(u32x2, __builtin_amdgcn_permlane32_swap(x0, y0, false, false));
        const u32x2 s1 = __builtin_bit_cast(u32x2, __builtin_amdgcn_permlane32_swap(x1, y1, false, false));
        const u32x4 w = {s0[0], s1[0], s0[1], s1[1]};
        const uint32_t off = orow + 2 * (32 * db + 16 * k + 8 * hl);
        if constexpr (OUT == kOutBf16x16) {
          __builtin_amdgcn_raw_buffer_store_b128(w, ro, off, 0, 0);
        } else {
          __builtin_amdgcn_raw_buffer_store_b64(u32x2{w[0], w[1]}, ro, off, 0, 0);
          __builtin_amdgcn_raw_buffer_store_b64(u32x2{w[2], w[3]}, ro, off + 8, 0, 0);
        }
      }
  }
}

template <int OUT>
__global__ void __launch_bounds__(XW * 64, 1) cross_attn_kernel(const AttnKernelArgs a) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hl = lane >> 5;
  const int l32 = lane & 31;

  // ---- this workgroup's rounds: XCD x (= blockIdx % 8) owns ranks [x G/8, (x+1) G/8)
  const int G = gridDim.x;
  const int rank = (G % 8 == 0) ? (int)(blockIdx.x & 7u) * (G / 8) + (int)(blockIdx.x >> 3)
                                : (int)blockIdx.x;
  const int nqb = (a.Lq + 31) / 32;       // 32-query blocks per (batch, head)
  const int rpb = (nqb + XW - 1) / XW;    // rounds per (batch, head)
  const int64_t R = (int64_t)a.B * a.H * rpb;
  const int r0 = (int)(R * rank / G), r1 = (int)(R * (rank + 1) / G);

  const SegDesc& sg = a.seg[0];
  const uint32_t ks = (uint32_t)(sg.ksl * 2), vs = (uint32_t)(sg.vsl * 2);  // row strides, bytes
  const float c = sreg(a.scale_log2);
  const float mult_raw = sreg(a.mult_raw);
  const int64_t lo = a.lo;

  // ---- per-lane LDS addresses
  const int lds0 = (int)lds_addr(lds);
  // K fragment s (d = 16s + 8hl .. +7) of sub-block row l32
  int kb[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) kb[s] = opaque(lds0 + l32 * XROWB + (((2 * s + hl) ^ swz(l32)) << 4));
  // V transpose reads for d-block db and key half jj (see attn_fwd_bf16.hip)
  int vb[4][2];
  {
    const int s16 = lane & 15, g = (lane >> 4) & 1;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int r = 4 * hl + 8 * jj + (s16 >> 2);
        const int lc = 4 * db + 2 * g + ((s16 & 3) >> 1);
        vb[db][jj] = opaque(lds0 + XV0 + r * XROWB + ((lc ^ swz(r)) << 4) + 8 * (s16 & 1));
      }
  }
  // fragment s of K sub-block SB / fragment i of V sub-block SB, as read in step J
  auto read_k = [&](auto j_c, auto sb_c, int s) -> u32x4 {
    return lds_read_b128(kb[s] + k_off<decltype(j_c)::value, decltype(sb_c)::value>());
  };
  auto read_v = [&](auto j_c, auto sb_c, int i) -> u32x4 {
    constexpr int OFF = v_off<decltype(j_c)::value, decltype(sb_c)::value>();
    const int db = i >> 1, m = i & 1;
    const u32x2 v0 = lds_read_tr16(vb[db][0] + OFF + m * 16 * XROWB);
    const u32x2 v1 = lds_read_tr16(vb[db][1] + OFF + m * 16 * XROWB);
    return u32x4{v0[0], v0[1], v1[0], v1[1]};
  };

  int res_bh = -1, res_ch = -1;  // (batch*head, chunk) resident in LDS

  // Q fragments (B operand of S^T = K Q^T) of round r's item: qf[s] holds d = 16s + 8hl .. +7
  // of query q0 + l32. The next round's are loaded into qn while this round computes. Q and O
  // go through buffer loads and stores whose range check covers the (b, h) rows [0, Lq): rows
  // past Lq (a partial last block, waves with no item) load 0 and store nothing with no branch,
  // so the compiler counts the loads and stores in flight exactly and waits for the prefetch
  // only, not for every store before it.
  auto load_q = [&](int r, u32x4 (&dst)[8]) {
    const int bh = r < r1 ? r / rpb : 0, rr = r % rpb;
    const int b = bh / a.H, h = bh % a.H;
    const int q = (rr * XW + wave) * 32 + l32;
    const uint32_t bytes = r < r1 ? (uint32_t)a.Lq * (uint32_t)(a.qsl * 2) : 0u;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.q + a.qsb * b + a.qsh * h), (short)0, (int)bytes, 0x00020000);
    const uint32_t off = (uint32_t)(q * a.qsl + 8 * hl) * 2u;
#pragma unroll
    for (int s = 0; s < 8; ++s)
      dst[s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 32 * s, 0, 0));
  };
  u32x4 qf[8], qn[8];
  load_q(r0, qf);
  int kl_b = -1;            // the batch whose valid key count kl_v holds
  int64_t kl_v = 0;

#pragma unroll 1
  for (int r = r0; r < r1; ++r) {
    const int bh = r / rpb, rr = r % rpb;
    const int b = bh / a.H, h = bh % a.H;
    load_q(r + 1, qn);
    int64_t hi = a.hi;
    if (a.k_lens != nullptr) {
      if (b != kl_b) {  // (a scalar round trip, so only when the batch changes)
        kl_v = load_scalar_i32(a.k_lens + b);
        kl_b = b;
      }
      hi = kl_v < hi ? kl_v : hi;
    }
    const int n_all = hi > lo ? (int)(hi - lo) : 0;  // attended keys (<= 4096, host-checked)
    const int nch = (n_all + XCH - 1) / XCH;
    const int qb = rr * XW + wave;
    const bool active = qb < nqb;
    const int q0 = qb * 32;

    floatx16 oacc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) oacc[db][e] = 0.0f;
    float m_used = M_INIT, lsum = 0.0f;

#pragma unroll 1
    for (int ch = 0; ch < nch; ++ch) {
      const int kbase = ch * XCH;                                 // first key of the chunk
      const int n = n_all - kbase < XCH ? n_all - kbase : XCH;    // keys in the chunk
      const int nsub = (n + 31) / 32;
      // dedup: first key of the chunk with the multiplicity bias (1 << 20: none)
      int mrow = 1 << 20;
      if (a.mult_key >= 0) {
        const int64_t mr = a.mult_key - lo - kbase;
        mrow = mr < 0 ? 0 : (mr > (1 << 20) ? (1 << 20) : (int)mr);
      }

      if (bh != res_bh || ch != res_ch) {
        // every wave is past its reads of the old contents
        barrier_nofence();
        // rows [kbase, kbase + 32 nsub) of this (b, h) into LDS rows [0, 32 nsub); rows past the
        // valid keys fetch the last valid key (finite, masked to p = 0 in the softmax)
        const int64_t row0 = lo + kbase;
        const unsigned char* kg = reinterpret_cast<const unsigned char*>(sg.k) +
                                  (sg.ksb * b + sg.ksh * h + sg.ksl * row0) * 2;
        const unsigned char* vg = reinterpret_cast<const unsigned char*>(sg.v) +
                                  (sg.vsb * b + sg.vsh * h + sg.vsl * row0) * 2;
        const int nblk = 8 * nsub;  // 1 KB (4-row) blocks per tensor
#pragma unroll 1
        for (int blk = wave; blk < nblk; blk += XW) {
          const int row = 4 * blk + (lane >> 4);
          const int src = row < n ? row : n - 1;
          const uint32_t col = (uint32_t)(((lane & 15) ^ swz(row)) << 4);
          const uint32_t dst = (uint32_t)lds0 + 1024u * blk;
          dma16(kg, (uint32_t)src * ks + col, dst);
          dma16(vg, (uint32_t)src * vs + col, dst + XV0);
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's rows (and its Q) are in
        barrier_nofence();
        res_bh = bh;
        res_ch = ch;
      }
      if (!active || nsub == 0) continue;

      // ---- the pipelined sub-block loop of this chunk
      floatx16 sA, sB;
      u32x4 pA[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
      u32x4 pB[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
      u32x4 kf[XKR], vf[XVR];
#pragma unroll
      for (int e = 0; e < 16; ++e) { sA[e] = 0.0f; sB[e] = 0.0f; }
      // S_0, and the first K fragments of S_1 and V fragments of PV_0 (read by step 1)
#pragma unroll
      for (int s = 0; s < 8; ++s) sA = mfma32x32x16(read_k(I<0>{}, I<0>{}, s), qf[s], sA);
#pragma unroll
      for (int i = 0; i < XKA; ++i) kf[i % XKR] = read_k(I<0>{}, I<1>{}, i);

      // One step: softmax of S_J (s_in) into p_out; O += V_{J-1}^T p_in^T (J >= 1); with NEXT,
      // s_out = S_{J+1} = K_{J+1} Q^T. The first XKA / XVA fragments of a step are read by the
      // step before it.
      auto step = [&](auto j_c, auto next_c, floatx16& s_in, floatx16& s_out, u32x4 (&p_in)[2],
                      u32x4 (&p_out)[2]) {
        constexpr int J = decltype(j_c)::value;
        constexpr bool NEXT = decltype(next_c)::value;
        constexpr bool PV = J >= 1;
        if constexpr (J == XKSW) {
#pragma unroll
          for (int s = 0; s < 8; ++s) kb[s] = opaque(kb[s] + XSHIFT);
        }
        if constexpr (J == XVSW) {
#pragma unroll
          for (int db = 0; db < 4; ++db) {
            vb[db][0] = opaque(vb[db][0] + XSHIFT);
            vb[db][1] = opaque(vb[db][1] + XSHIFT);
          }
        }
        if (32 * J + 32 > n || mrow < 32 * J + 32) mask_scores(s_in, J, 0, n, hl, mrow, mult_raw);
        if constexpr (J == 0) {
          // a round's first sub-block: O and l are still 0, so the reference is set to the
          // sub-block's row max directly (key 0 is valid, so it is finite) instead of starting
          // at M_INIT, overflowing and redoing the exponentials
          if (ch == 0) {
            float mx = s_in[0];
#pragma unroll
            for (int e = 1; e < 16; ++e) mx = fmaxf(mx, s_in[e]);
            m_used = wave_max_xor32(mx);
          }
        }
        float ca = -m_used * c;
        if constexpr (NEXT) {
#pragma unroll
          for (int e = 0; e < 16; ++e) s_out[e] = 0.0f;
        }
        if constexpr (PV && J == 1) {
          // PV_0's first fragments (the step before had none to read)
#pragma unroll
          for (int i = 0; i < XVA; ++i) vf[i % XVR] = read_v(I<J>{}, I<0>{}, i);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if constexpr (NEXT) {
            if (i + XKA < 8) kf[(i + XKA) % XKR] = read_k(I<J>{}, I<J + 1>{}, i + XKA);
            else if (J + 2 < XSB) kf[(i + XKA) % XKR] = read_k(I<J>{}, I<(J + 2 < XSB ? J + 2 : J + 1)>{}, i + XKA - 8);
          }
          if constexpr (PV) {
            if (i + XVA < 8) vf[(i + XVA) % XVR] = read_v(I<J>{}, I<J - 1>{}, i + XVA);
            else vf[(i + XVA) % XVR] = read_v(I<J>{}, I<J>{}, i + XVA - 8);
          }
          if constexpr (NEXT) s_out = mfma32x32x16(kf[i % XKR], qf[i], s_out);
          if constexpr (PV) oacc[i >> 1] = mfma32x32x16(vf[i % XVR], p_in[i & 1], oacc[i >> 1]);
        }
        auto exps = [&]() {
          float l;
#pragma unroll
          for (int m = 0; m < 2; ++m) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float x0 = fast_exp2(__builtin_fmaf(s_in[8 * m + 2 * e], c, ca));
              const float x1 = fast_exp2(__builtin_fmaf(s_in[8 * m + 2 * e + 1], c, ca));
              p_out[m][e] = pack_bf16x2(x0, x1);
              l = (m == 0 && e == 0) ? x0 + x1 : l + (x0 + x1);
            }
          }
          return l;
        };
        float ls = exps();
        if constexpr (NEXT && PV) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // 2 VALU
            __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);  // LDS reads
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
          }
        } else if constexpr (PV) {
          // the tenth step: the 8 PV MFMAs, the V reads, the softmax spread between them
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
          }
        }
        asm volatile("" ::"v"(p_out[0]), "v"(p_out[1]), "v"(ls));
        // The next sub-block's S and the next step's first fragments stay in this step's block:
        // they are used only if there is a next step, and the compiler would otherwise sink them
        // into that step's branch, where the QK chain and its LDS reads then issue back to back
        // ahead of the softmax instead of interleaved with it.
        if constexpr (NEXT) asm volatile("" ::"v"(s_out));
        asm volatile("" ::"v"(kf[0]), "v"(kf[1]), "v"(kf[2]), "v"(kf[3]));
        asm volatile("" ::"v"(vf[0]), "v"(vf[1]), "v"(vf[2]), "v"(vf[3]));
        // a row sum beyond 2^16 (or not finite) means some p outgrew the reference: move it to
        // the row max of this sub-block (and the old reference), redo, and rescale O and l
        float alpha = 1.0f;
        if (__any(!(ls <= P_LIMIT))) {
          float mx = s_in[0];
#pragma unroll
          for (int e = 1; e < 16; ++e) mx = fmaxf(mx, s_in[e]);
          mx = wave_max_xor32(mx);
          const float m_new = fmaxf(mx, m_used);
          alpha = fast_exp2((m_used - m_new) * c);
          m_used = m_new;
          ca = -m_new * c;
          // O (with this step's PV of the previous sub-block, at the old reference) moves now
          scale_acc(oacc, alpha);
          ls = exps();
        }
        lsum = __builtin_fmaf(lsum, alpha, ls);
        asm volatile("" ::"v"(p_out[0]), "v"(p_out[1]), "v"(lsum));
      };
      auto run = [&](auto j_c, floatx16& s_in, floatx16& s_out, u32x4 (&p_in)[2],
                     u32x4 (&p_out)[2]) -> bool {
        constexpr int J = decltype(j_c)::value;
        // (every step but the chunk's tenth computes S_{J+1}, used if J + 1 < nsub: a last step
        // without it as a branch of its own doubles the live ranges the register allocator sees
        // and spills; a chunk of fewer than 10 sub-blocks wastes 8 of its 8 + 16 nsub MFMAs)
        step(j_c, std::bool_constant<(J + 1 < XSB)>{}, s_in, s_out, p_in, p_out);
        return J + 1 < nsub;
      };
      static_assert(XSB == 10, "the unrolled sub-block sequence below covers 10 sub-blocks");
      run(I<0>{}, sA, sB, pB, pA) && run(I<1>{}, sB, sA, pA, pB) && run(I<2>{}, sA, sB, pB, pA) &&
          run(I<3>{}, sB, sA, pA, pB) && run(I<4>{}, sA, sB, pB, pA) &&
          run(I<5>{}, sB, sA, pA, pB) && run(I<6>{}, sA, sB, pB, pA) &&
          run(I<7>{}, sB, sA, pA, pB) && run(I<8>{}, sA, sB, pB, pA) && run(I<9>{}, sB, sA, pA, pB);
      // drain: O += V_J^T P_J^T of the chunk's last sub-block J = nsub - 1 (P_J is in pA for
      // even J, pB for odd), with the V bases as step J left them
      {
        const int jl = nsub - 1;
        const int voff = (jl - (jl >= XVSW ? 5 : 0)) * XSUBB;
        u32x4 pl[2];
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
          for (int e = 0; e < 4; ++e) pl[m][e] = (jl & 1) ? pB[m][e] : pA[m][e];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int db = i >> 1, m = i & 1;
          const u32x2 v0 = lds_read_tr16(vb[db][0] + voff + m * 16 * XROWB);
          const u32x2 v1 = lds_read_tr16(vb[db][1] + voff + m * 16 * XROWB);
          oacc[db] = mfma32x32x16(u32x4{v0[0], v0[1], v1[0], v1[1]}, pl[m], oacc[db]);
        }
      }
      // the bases back where the next chunk's step 0 expects them
      if (nsub > XKSW) {
#pragma unroll
        for (int s = 0; s < 8; ++s) kb[s] = opaque(kb[s] - XSHIFT);
      }
      if (nsub > XVSW) {
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          vb[db][0] = opaque(vb[db][0] - XSHIFT);
          vb[db][1] = opaque(vb[db][1] - XSHIFT);
        }
      }
    }
    // ---- epilogue
    store_rows<OUT>(a, b, h, q0, oacc, lsum, l32, hl);
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[s] = qn[s];
  }
}


// ---- The ring form: a context longer than the resident chunk, all of it attended (the
// reference's unmasked 512-row call, model.py:554-561 with context_lens None).
//
// The workgroup runs its contiguous range of rounds as one stream of 64-key tiles (round-major),
// copied through a 3-stage LDS ring exactly as the chunk kernel's tiles are (one barrier per tile:
// wait for tile g + 1, barrier, refill tile g - 1's stage with tile g + 2), except that the ring
// runs on across rounds: the next round's first tiles are in flight while a round ends. Each
// wave's Q rows of the next round are copied into LDS (its own 8 KB) during the round and read at
// its last tile, and the round boundary is pipelined like any other step: the last tile's second
// step computes S of the next round's first sub-block with the new Q, and the next round's first
// step, which starts a fresh softmax, still adds the old round's last P V into the old O, which
// is then stored and cleared.
//
// LDS: K tiles [0, 48 KB), the waves' Q rows [48, 112 KB), V tiles [112, 160 KB).
constexpr int GST = 3;                        // ring stages
constexpr int GTILE = BN * XROWB;             // 16 KB: a K (or V) tile
constexpr int GHALF = GTILE / 2;              // one 32-key sub-block
constexpr int GQ0 = GST * GTILE;              // Q rows, 8 KB per wave
constexpr int GV0 = GQ0 + XW * 32 * XROWB;    // V tiles
constexpr int GLDS = GV0 + GST * GTILE;
constexpr int GNDMA = GTILE / (XW * 64 * 16); // 16-byte copies per lane per K (or V) tile
static_assert(GLDS <= 160 * 1024, "ring, Q rows and V ring must fit the LDS");
static_assert(GNDMA == 2, "two 1 KB blocks of each tile per wave");

// A 64-bit pointer that is the same in every lane, held in scalar registers (the Q copies' base;
// written by v_readfirstlane, so the copies that read it take dma16_guarded; the tile copies'
// bases are stepped by scalar adds and go through dma16, which the build's assembly check covers).
__device__ __forceinline__ const unsigned char* uniform_ptr(const unsigned char* p) {
  const uint64_t x = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(x >> 32));
  return reinterpret_cast<const unsigned char*>((uintptr_t)(((uint64_t)hi << 32) | lo));
}

template <int OUT, bool FOLD>
__global__ void __launch_bounds__(XW * 64, 1) cross_ring_kernel(const AttnKernelArgs a) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hl = lane >> 5;
  const int l32 = lane & 31;

  // ---- this workgroup's rounds, as in cross_attn_kernel
  const int G = gridDim.x;
  const int rank = (G % 8 == 0) ? (int)(blockIdx.x & 7u) * (G / 8) + (int)(blockIdx.x >> 3)
                                : (int)blockIdx.x;
  const int nqb = (a.Lq + 31) / 32;
  const int rpb = (nqb + XW - 1) / XW;
  const int64_t R = (int64_t)a.B * a.H * rpb;
  const int r0 = (int)(R * rank / G), r1 = (int)(R * (rank + 1) / G);
  if (r0 >= r1) return;  // every wave of the workgroup

  const SegDesc& sg = a.seg[0];
  const uint32_t ks = (uint32_t)(sg.ksl * 2), vs = (uint32_t)(sg.vsl * 2);  // row strides, bytes
  const float c = sreg(a.scale_log2);
  const int64_t lo = a.lo;
  const int n = (int)(a.hi - a.lo);        // keys of every round (host: 320 < n <= 4096)
  const int T = (n + BN - 1) / BN;         // tiles per round (>= 6)
  const int vlast = n - BN * (T - 1);      // valid rows of a round's last tile
  const int vrow_last = vlast == BN ? ROWS_FULL : pack_rows(0, vlast, 255);
  const int NT = (r1 - r0) * T;            // tiles of the workgroup

  // ---- per-lane LDS addresses (the chunk kernel's layout: 256-byte rows, chunk c of row r at
  // c ^ swz(r))
  const int lds0 = (int)lds_addr(lds);
  int koff[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) koff[s] = opaque(lds0 + l32 * XROWB + (((2 * s + hl) ^ swz(l32)) << 4));
  int voff[4][2];
  {
    const int s16 = lane & 15, g = (lane >> 4) & 1;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int r = 4 * hl + 8 * jj + (s16 >> 2);
        const int lc = 4 * db + 2 * g + ((s16 & 3) >> 1);
        voff[db][jj] = opaque(lds0 + GV0 + r * XROWB + ((lc ^ swz(r)) << 4) + 8 * (s16 & 1));
      }
  }
  // copies: this wave fills 1 KB blocks GNDMA * wave + i of each tile (and blocks 0..7 of its Q
  // rows); lane -> row 4 block + lane / 16, logical chunk (lane % 16) ^ swz(row)
  // (the row offsets are formed at each copy: registers are scarcer than the two VALU ops)
  int dma_row[GNDMA];
  uint32_t dma_col[GNDMA];
#pragma unroll
  for (int i = 0; i < GNDMA; ++i) {
    dma_row[i] = 4 * (GNDMA * wave + i) + (lane >> 4);
    dma_col[i] = (uint32_t)(((lane & 15) ^ swz(dma_row[i])) << 4);
  }
  const uint32_t lds_wave = (uint32_t)lds0 + 1024u * GNDMA * wave;
  const int qlds = lds0 + GQ0 + 8192 * wave;  // this wave's Q rows

  // ---- round positions (batch, head, round of the head), stepped without divisions
  struct RPos {
    int b, h, rr;
  };
  auto rpos_next = [&](RPos x) {
    if (++x.rr == rpb) {
      x.rr = 0;
      if (++x.h == a.H) {
        x.h = 0;
        ++x.b;
      }
    }
    return x;
  };
  RPos pos0;
  pos0.rr = r0 % rpb;
  pos0.h = (r0 / rpb) % a.H;
  pos0.b = (r0 / rpb) / a.H;

  // ---- the copy side: tile `it` of round `ir` (at ipos) is the next to be copied, its K and V
  // rows from kt / vt (stepped by a tile's bytes; set from the round's position at a round change)
  int ir = r0, it = 0;
  RPos ipos = pos0;
  const unsigned char* kt = nullptr;
  const unsigned char* vt = nullptr;
  auto copy_base = [&]() {
    kt = reinterpret_cast<const unsigned char*>(sg.k) +
         (sg.ksb * ipos.b + sg.ksh * ipos.h + sg.ksl * lo) * 2;
    vt = reinterpret_cast<const unsigned char*>(sg.v) +
         (sg.vsb * ipos.b + sg.vsh * ipos.h + sg.vsl * lo) * 2;
  };
  copy_base();
  const int t_full = vlast == BN ? T : T - 1;  // tiles of a round with every row valid
  auto issue_tile = [&](int stage) {
    const uint32_t kdst = (uint32_t)sreg((int)lds_wave) + stage * GTILE;
    const uint32_t vdst = kdst + GV0;
    if (it < t_full) {
#pragma unroll
      for (int i = 0; i < GNDMA; ++i) {
        const uint32_t row = (uint32_t)opaque(dma_row[i]);
        dma16(kt, row * ks + dma_col[i], kdst + 1024 * i);
        dma16(vt, row * vs + dma_col[i], vdst + 1024 * i);
      }
    } else {
      // rows past the context fetch its last key instead (masked to p = 0 in the softmax)
#pragma unroll
      for (int i = 0; i < GNDMA; ++i) {
        const int r = dma_row[i] < vlast ? dma_row[i] : vlast - 1;
        dma16(kt, (uint32_t)r * ks + dma_col[i], kdst + 1024 * i);
        dma16(vt, (uint32_t)r * vs + dma_col[i], vdst + 1024 * i);
      }
    }
    if (++it == T) {
      it = 0;
      ipos = rpos_next(ipos);
      if (++ir < r1) copy_base();
    } else {
      kt += BN * ks;
      vt += BN * vs;
    }
  };
  // this wave's 32 Q rows of the round at x into its LDS rows, 1 KB blocks i0 .. i0 + n - 1 of 8
  // (rows past Lq fetch row Lq - 1; their outputs are dropped by the store's range check)
  auto issue_q = [&](const RPos& x, int i0, int n) {
    const int qb = x.rr * XW + wave;
    const unsigned char* qg = uniform_ptr(reinterpret_cast<const unsigned char*>(a.q + a.qsb * x.b + a.qsh * x.h));
#pragma unroll
    for (int i = i0; i < i0 + n; ++i) {
      const int row = 4 * i + (lane >> 4);
      int q = qb * 32 + row;
      q = q < a.Lq ? q : a.Lq - 1;
      const uint32_t col = (uint32_t)(((lane & 15) ^ swz(row)) << 4);
      dma16_guarded(qg, (uint32_t)q * (uint32_t)(a.qsl * 2) + col, (uint32_t)qlds + 1024u * i);
    }
  };

  // Q fragments (B operand of S^T = K Q^T): qf[s] holds d = 16s + 8hl .. +7 of query q0 + l32
  u32x4 qf[8];
  auto read_q = [&]() {
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[s] = lds_read_b128(koff[s] + (GQ0 + 8192 * wave));
  };

  // ---- start: round r0's Q, tiles 0 and 1; the V sub-block the first step's PV reads (P = 0)
  // is zeroed (tile 2 is copied into that stage only after the first barrier)
  issue_q(pos0, 0, 8);
  issue_tile(0);
  if (NT > 1) issue_tile(1);
  {
    const u32x4 z = {0u, 0u, 0u, 0u};
    *reinterpret_cast<u32x4*>(lds + GV0 + (GST - 1) * GTILE + GHALF + 16 * threadIdx.x) = z;
  }
  // Q and tile 0 (tile 1's 4 copies, issued last, may still be in flight: tile 0's wait covers
  // them), and the zeroed sub-block
  asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  barrier_nofence();
  read_q();

  floatx16 oacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[db][e] = 0.0f;
  float m_used = M_INIT, lsum = 0.0f;
  // FOLD (q pre-scaled: scale * log2(e) == 1): the exponent reference mref (log2 units) starts
  // every QK chain (cinit = -mref), so the MFMA result is the exponent of p; mlim, the redo
  // threshold, is -1 while a round's reference is unset (its first step sets it from the row max
  // without rescaling O, which then still holds the previous round)
  float mref = 0.0f, mlim = -1.0f;
  floatx16 cinit;
#pragma unroll
  for (int e = 0; e < 16; ++e) cinit[e] = 0.0f;

  floatx16 sA, sB;
#pragma unroll
  for (int e = 0; e < 16; ++e) { sA[e] = 0.0f; sB[e] = 0.0f; }
  u32x4 pA[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
  u32x4 pB[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
  u32x4 kf[XKR], vf[XVR];
  auto load_k = [&](auto ko_c, int i) {
    constexpr int KO = decltype(ko_c)::value;
    kf[i % XKR] = lds_read_b128(koff[i] + KO);
  };
  auto load_v = [&](auto vo_c, int i) {
    constexpr int VO = decltype(vo_c)::value;
    const int db = i >> 1, m = i & 1;
    const u32x2 v0 = lds_read_tr16(voff[db][0] + VO + 16 * m * XROWB);
    const u32x2 v1 = lds_read_tr16(voff[db][1] + VO + 16 * m * XROWB);
    vf[i % XVR] = u32x4{v0[0], v0[1], v1[0], v1[1]};
  };
  // S of tile 0's first sub-block, and the first fragments of step 0: K of tile 0 rows 32..63,
  // V of the zeroed sub-block
#pragma unroll
  for (int s = 0; s < 8; ++s) sA = mfma32x32x16(lds_read_b128(koff[s]), qf[s], sA);
#pragma unroll
  for (int i = 0; i < XKA; ++i) load_k(I<GHALF>{}, i);
#pragma unroll
  for (int i = 0; i < XVA; ++i) load_v(I<(GST - 1) * GTILE + GHALF>{}, i);

  // One step: softmax of s_in (sub-block kb of a tile with valid rows vrow) into p_out,
  // O += V^T p_in^T from V offset VO, s_out = K Q^T from K offset KO. KPRE: the first K fragments
  // were read by the step before; NKO / NVO (>= 0): read the next step's first fragments. A
  // round's first step (`first`) starts a fresh softmax: its reference is the sub-block's row
  // max, and its PV still belongs to the previous round's O, which a move must not rescale.
  auto step = [&](auto ko_c, auto vo_c, auto kpre_c, auto nko_c, auto nvo_c, floatx16& s_in,
                  floatx16& s_out, u32x4 (&p_in)[2], u32x4 (&p_out)[2], int kb, int vrow,
                  bool first) {
    constexpr bool KPRE = decltype(kpre_c)::value;
    constexpr int NKO = decltype(nko_c)::value, NVO = decltype(nvo_c)::value;
    if constexpr (!KPRE) {
#pragma unroll
      for (int i = 0; i < XKA; ++i) load_k(ko_c, i);
    }
    const int vhi = (vrow >> 8) & 0xff;
    if (vrow != ROWS_FULL && vhi < 32 * kb + 32) mask_scores(s_in, kb, 0, vhi, hl, 1 << 20, 0.0f);
    if constexpr (!FOLD) {
      if (first) {
        float mx = s_in[0];
#pragma unroll
        for (int e = 1; e < 16; ++e) mx = fmaxf(mx, s_in[e]);
        m_used = wave_max_xor32(mx);
      }
    }
    float ca = -m_used * c;
    if constexpr (FOLD) {
      s_out = cinit;
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) s_out[e] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i + XVA < 8) load_v(vo_c, i + XVA);
      else if constexpr (NVO >= 0) load_v(nvo_c, i + XVA - 8);
      if (i + XKA < 8) load_k(ko_c, i + XKA);
      else if constexpr (NKO >= 0) load_k(nko_c, i + XKA - 8);
      s_out = mfma32x32x16(kf[i % XKR], qf[i], s_out);
      oacc[i >> 1] = mfma32x32x16(vf[i % XVR], p_in[i & 1], oacc[i >> 1]);
    }
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
    // the chunk kernel's schedules: per MFMA pair, MFMA, 2 VALU, the LDS reads, MFMA, 2 VALU;
    // folded, MFMA, 1 exponential, 1 VALU, the reads, MFMA, 1 exponential, 2 VALU
    constexpr int NDS0 = KPRE ? 0 : XKA;
    if constexpr (NDS0 > 0) __builtin_amdgcn_sched_group_barrier(0x100, NDS0, 0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bool rk = i + XKA < 8 || NKO >= 0, rv = i + XVA < 8 || NVO >= 0;
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if constexpr (FOLD) {
        __builtin_amdgcn_sched_group_barrier(0x400, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);
      } else {
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
      }
      if (rk && rv) __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
      else if (rv) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      else if (rk) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if constexpr (FOLD) __builtin_amdgcn_sched_group_barrier(0x400, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
    }
    asm volatile("" ::"v"(p_out[0]), "v"(p_out[1]), "v"(ls));
    asm volatile("" ::"v"(s_out));
    if constexpr (FOLD) {
      // s_in is s - mref. A row sum beyond 2^16 (or not finite) moves the reference up to the
      // row max, with O and l rescaled; an unset reference (a round's first step) is set to the
      // row max with no rescale. The next sub-block's S, started from the old -mref, moves too.
      if (__any(!(ls <= mlim))) {
        float mx = s_in[0];
#pragma unroll
        for (int e = 1; e < 16; ++e) mx = fmaxf(mx, s_in[e]);
        mx = wave_max_xor32(mx);
        float d;
        if (mlim > 0.0f) {
          d = fmaxf(mx, 0.0f);
          const float alpha = fast_exp2(-d);
          scale_acc(oacc, alpha);
          lsum *= alpha;
        } else {
          const bool set = mx > -INFINITY;
          d = set ? mx : 0.0f;
          mlim = set ? P_LIMIT : -1.0f;
        }
        mref += d;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          s_in[e] -= d;
          s_out[e] -= d;
          cinit[e] = -mref;
        }
        ls = exps();
      }
    } else if (__any(!(ls <= P_LIMIT))) {
      // a row sum beyond 2^16 (or not finite): move the reference to the row max, redo, and
      // rescale O and l (not in a round's first step, whose O is the previous round's)
      float mx = s_in[0];
#pragma unroll
      for (int e = 1; e < 16; ++e) mx = fmaxf(mx, s_in[e]);
      mx = wave_max_xor32(mx);
      const float m_new = fmaxf(mx, m_used);
      const float alpha = fast_exp2((m_used - m_new) * c);
      m_used = m_new;
      ca = -m_new * c;
      if (!first) {
        scale_acc(oacc, alpha);
        lsum *= alpha;
      }
      ls = exps();
    }
    lsum += ls;
    asm volatile("" ::"v"(p_out[0]), "v"(p_out[1]), "v"(lsum));
  };

  // output rows of the round at x (this wave's 32 queries)
  auto store_round = [&](const RPos& x, float l) {
    store_rows<OUT>(a, x.b, x.h, (x.rr * XW + wave) * 32, oacc, l, l32, hl);
  };

  // Tile g (round r, tile t of it) lives in stage g % GST.
  // Step A: softmax of tile g half 0, PV of tile g-1 half 1, S of tile g half 1.
  // Step B: softmax of tile g half 1, PV of tile g half 0, S of tile g+1 half 0 (with the next
  // round's Q when tile g is its round's last).
  // Between them: wait for tile g+1, barrier, refill tile g-1's stage with tile g+2.
  // The next round's Q rows are copied in pairs of 1 KB blocks after the tile copies of tiles
  // 1 .. 4 (a round has at least 6 tiles), so that the whole chip's Q reads do not come in one
  // burst at the round's end, and the tile waits after them leave those 2 loads in flight (the
  // loads complete in order; a wait with the round's stores outstanding waits for everything).
  int r = r0, t = 0;
  RPos cpos = pos0, ppos = pos0;  // rounds r and r - 1
  auto tile = [&](auto st_c, int g) {
    constexpr int ST = decltype(st_c)::value;
    constexpr int SP = (ST + GST - 1) % GST, SN = (ST + 1) % GST;
    const bool first = t == 0, last = t == T - 1;
    const int vrow = last ? vrow_last : ROWS_FULL;
    float l_prev = 0.0f;
    if (first) {
      l_prev = lsum;
      lsum = 0.0f;
      if constexpr (FOLD) mlim = -1.0f;
    }
    step(I<ST * GTILE + GHALF>{}, I<SP * GTILE + GHALF>{}, std::true_type{}, I<-1>{},
         I<ST * GTILE>{}, sA, sB, pA, pB, 0, vrow, first);
    if (g + 1 < NT) {
      if (t >= 2 && t <= 5 && !last && r + 1 < r1)
        asm volatile("s_waitcnt vmcnt(2)" ::: "memory");  // tile g+1, not the 2 Q loads after it
      else
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): tile g+1 and everything before it
    }
    barrier_nofence();
    // (copies and stores are issued right after a barrier, ahead of the tile copy, so that the
    // next wait for a tile covers them too)
    if (first) {
      // the previous round's O is complete (its last PV was this step's)
      if (r > r0) store_round(ppos, l_prev);
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[db][e] = 0.0f;
    }
    // the next round's Q (copied during this round) for step B's S
    if (last && r + 1 < r1) read_q();
    if (g + 2 < NT) issue_tile(SP);
    if (t >= 1 && t <= 4 && r + 1 < r1) issue_q(rpos_next(cpos), 2 * (t - 1), 2);
    step(I<SN * GTILE>{}, I<ST * GTILE>{}, std::false_type{}, I<SN * GTILE + GHALF>{},
         I<ST * GTILE + GHALF>{}, sB, sA, pB, pA, 1, vrow, false);
    if (last) {
      ppos = cpos;
      cpos = rpos_next(cpos);
    }
    // (selects, not a branch on the counters: they stay scalar registers)
    r += last ? 1 : 0;
    t = last ? 0 : t + 1;
  };

#pragma unroll 1
  for (int g = 0; g < NT; g += GST) {
    tile(I<0>{}, g);
    if (g + 1 < NT) tile(I<1>{}, g + 1);
    if (g + 2 < NT) tile(I<2>{}, g + 2);
  }

  // drain: O += V^T P^T of the last sub-block (tile NT-1 half 1, P in pA), then the last round
  {
    const int vo = ((NT - 1) % GST) * GTILE + GHALF;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int db = i >> 1, m = i & 1;
      const u32x2 v0 = lds_read_tr16(voff[db][0] + vo + 16 * m * XROWB);
      const u32x2 v1 = lds_read_tr16(voff[db][1] + vo + 16 * m * XROWB);
      oacc[db] = mfma32x32x16(u32x4{v0[0], v0[1], v1[0], v1[1]}, pA[m], oacc[db]);
    }
  }
  store_round(ppos, lsum);
}
}  // namespace

int cross_attn_max_keys_resident() { return XCH; }

template <int OUT>
static hipError_t set_lds_attr() {
  static hipError_t attr = hipFuncSetAttribute((const void*)cross_attn_kernel<OUT>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, XLDS);
  return attr;
}

hipError_t launch_cross_attn(const AttnKernelArgs& a, int num_cus, hipStream_t stream) {
  const int out = a.o32 ? kOutF32 : (a.o16 ? kOutBf16x16 : kOutBf16x8);
  hipError_t attr = out == kOutF32 ? set_lds_attr<kOutF32>()
                    : out == kOutBf16x16 ? set_lds_attr<kOutBf16x16>() : set_lds_attr<kOutBf16x8>();
  if (attr != hipSuccess) return attr;
  const int nqb = (a.Lq + 31) / 32;
  const int64_t rounds = (int64_t)a.B * a.H * ((nqb + XW - 1) / XW);
  int64_t g = rounds < num_cus ? rounds : num_cus;
  if (g >= 8) g -= g % 8;  // a multiple of 8: each XCD gets an equal share of the ranks
  if (g < 1) g = 1;
  const dim3 grid((uint32_t)g), block(XW * 64);
  if (out == kOutF32) hipLaunchKernelGGL(cross_attn_kernel<kOutF32>, grid, block, XLDS, stream, a);
  else if (out == kOutBf16x16) hipLaunchKernelGGL(cross_attn_kernel<kOutBf16x16>, grid, block, XLDS, stream, a);
  else hipLaunchKernelGGL(cross_attn_kernel<kOutBf16x8>, grid, block, XLDS, stream, a);
  return hipGetLastError();
}


template <int OUT, bool FOLD>
static hipError_t launch_ring(const AttnKernelArgs& a, dim3 grid, hipStream_t stream) {
  static hipError_t attr = hipFuncSetAttribute((const void*)cross_ring_kernel<OUT, FOLD>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, GLDS);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL((cross_ring_kernel<OUT, FOLD>), grid, dim3(XW * 64), GLDS, stream, a);
  return hipGetLastError();
}

hipError_t launch_cross_ring(const AttnKernelArgs& a, int num_cus, hipStream_t stream) {
  // (a round copies the next round's Q during its tiles 1 .. 4 and reads it in its last)
  if (a.hi - a.lo <= 5 * BN || a.hi - a.lo > 4096) return hipErrorInvalidValue;
  const int nqb = (a.Lq + 31) / 32;
  const int64_t rounds = (int64_t)a.B * a.H * ((nqb + XW - 1) / XW);
  int64_t g = rounds < num_cus ? rounds : num_cus;
  if (g >= 8) g -= g % 8;
  if (g < 1) g = 1;
  const dim3 grid((uint32_t)g);
  // a pre-scaled q (scale * log2(e) exactly 1 in fp32) takes the folded softmax
  const bool fold = a.scale_log2 == 1.0f;
  if (a.o32) return fold ? launch_ring<kOutF32, true>(a, grid, stream) : launch_ring<kOutF32, false>(a, grid, stream);
  if (a.o16)
    return fold ? launch_ring<kOutBf16x16, true>(a, grid, stream) : launch_ring<kOutBf16x16, false>(a, grid, stream);
  return fold ? launch_ring<kOutBf16x8, true>(a, grid, stream) : launch_ring<kOutBf16x8, false>(a, grid, stream);
}

}  // namespace lbw
