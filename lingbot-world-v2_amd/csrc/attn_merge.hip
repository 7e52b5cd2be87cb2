// Log-sum-exp merge of split-KV attention partials (gfx950), the cte_merge contract of
// wan/modules/attention.py:963-990: given per split s the unnormalised O_s (relative to the
// split's row max), the row max m_s (scaled scores) and the row sum l_s,
//   out = sum_s e^(m_s - M) O_s / sum_s e^(m_s - M) l_s,  M = max_s m_s,
// written as bf16 (fp32 for an fp32-output call); a row whose every split is empty (all m_s =
// -inf) yields 0. The partial form (PART) writes the merged triple instead -- O = sum_s
// e^(m_s - M) O_s, m = M, l = sum_s e^(m_s - M) l_s -- the running (O, max, sum) state of
// cte_call's chain (attention.py:654-694), which later calls extend and the last normalises.
//
// HBM-bound: per (b, h, q) row it reads n * (D + 2) fp32 values and writes D output values.
// One thread per (row, 4 consecutive d), so every load and store is a 16 / 8-byte vector. The
// split count is a template parameter, so that a thread issues all of its 3 n loads before it
// waits for any of them (with a runtime count the loops kept one round trip per load in flight).

#include "attn_tiles.h"

namespace lbw {

template <int N, bool O32, bool PART = false>
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
    float ms[N], ls[N];
    floatx4 os[N];
#pragma unroll
    for (int s = 0; s < N; ++s) {
      ms[s] = a.m[s][row];
      ls[s] = a.l[s][row];
      os[s] = *reinterpret_cast<const floatx4*>(a.o[s] + row * a.D + 4 * dq);
    }
    float M = -INFINITY;
#pragma unroll
    for (int s = 0; s < N; ++s) M = fmaxf(M, ms[s]);
    float den = 0.0f;
    floatx4 num = {0.f, 0.f, 0.f, 0.f};
    if (M != -INFINITY) {
#pragma unroll
      for (int s = 0; s < N; ++s) {
        const float w = (ms[s] == -INFINITY) ? 0.0f : expf(ms[s] - M);
        den += w * ls[s];
        num += w * os[s];
      }
    }
    if constexpr (PART) {
      *reinterpret_cast<floatx4*>(a.part_o + row * a.D + 4 * dq) = num;
      if (dq == 0) {
        a.part_m[row] = M;
        a.part_l[row] = den;
      }
      continue;
    }
    const float inv = den > 0.0f ? 1.0f / den : 0.0f;
    const int64_t off = a.osb * b + a.osl * (int64_t)q + a.osh * h + 4 * dq;
    if constexpr (O32) {
      *reinterpret_cast<floatx4*>(reinterpret_cast<float*>(a.out) + off) = num * inv;
    } else {
      u32x2 w;
      w[0] = pack_bf16x2(num[0] * inv, num[1] * inv);
      w[1] = pack_bf16x2(num[2] * inv, num[3] * inv);
      *reinterpret_cast<u32x2*>(a.out + off) = w;
    }
  }
}

// Work-decomposition constants of the attention kernels, for the host-side planning.
int attn_block_m() { return 256; }
int attn_block_n() { return BN; }

template <bool O32, bool PART>
static hipError_t launch_merge_n(const MergeKernelArgs& a, dim3 grid, dim3 block,
                                 hipStream_t stream) {
  switch (a.n) {
#define LBW_MERGE_CASE(n) \
    case n: hipLaunchKernelGGL((attn_merge_kernel<n, O32, PART>), grid, block, 0, stream, a); break;
    LBW_MERGE_CASE(1) LBW_MERGE_CASE(2) LBW_MERGE_CASE(3) LBW_MERGE_CASE(4)
    LBW_MERGE_CASE(5) LBW_MERGE_CASE(6) LBW_MERGE_CASE(7) LBW_MERGE_CASE(8)
    LBW_MERGE_CASE(9) LBW_MERGE_CASE(10) LBW_MERGE_CASE(11) LBW_MERGE_CASE(12)
    LBW_MERGE_CASE(13) LBW_MERGE_CASE(14) LBW_MERGE_CASE(15) LBW_MERGE_CASE(16)
#undef LBW_MERGE_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_attn_merge(const MergeKernelArgs& a, hipStream_t stream) {
  const int64_t total = (int64_t)a.B * a.H * a.Lq * (a.D / 4);
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  const dim3 grid((uint32_t)blocks), block(256);
  if (a.part_o != nullptr) return launch_merge_n<false, true>(a, grid, block, stream);
  return a.o32 ? launch_merge_n<true, false>(a, grid, block, stream)
               : launch_merge_n<false, false>(a, grid, block, stream);
}

}  // namespace lbw
