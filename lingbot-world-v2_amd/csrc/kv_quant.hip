// fp8-e4m3fn KV-cache quantiser (gfx950). No reference counterpart: the format is defined
// here. Per (batch, head, block of `block` tokens by absolute index in the buffer):
//   amax  = max |x| over the block's tokens and all head_dim features (fp32)
//   scale = the smallest power of two 2^k >= amax / 448 (k >= -126), or 1 when amax == 0
//   inv   = 1 / scale = 2^-k (exact)
//   code  = round_to_nearest_even_e4m3fn(x * inv)
// Power-of-two scales make a code times its scale exact in bf16: the attention kernel applies
// K's scale as the exponent scale of its fp8 matrix-core product and V's in the exact
// conversion of the codes to bf16, so neither enters the softmax arithmetic.
// One workgroup per (b, h, block): the block's 64 x 128 bf16 values are read once into
// registers (16-byte loads, 16 lanes per token row), reduced to amax, encoded and written.
// Workgroups are numbered with (b, h) fastest.

#include "common.h"
#include "attn_fwd.h"

namespace lbw {

// fp32 -> OCP e4m3fn code, round to nearest even; |x| >= 480 -> NaN (0x7f), matching
// torch's float8_e4m3fn cast. Written with integer ops so the result does not depend on a
// hardware conversion mode.
__device__ __forceinline__ uint32_t e4m3fn_encode(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t au = u & 0x7fffffffu;
  if (au >= 0x43f00000u) return sign | 0x7fu;            // >= 480 or NaN
  if (au < 0x3c800000u) {                                // < 2^-6: subnormal, step 2^-9
    const float ax = __uint_as_float(au);
    const uint32_t m = (uint32_t)__float2int_rn(ax * 512.0f);  // exact scale, RNE
    return sign | m;                                     // m == 8 is the min normal
  }
  const uint32_t r = au + 0x7ffffu + ((au >> 20) & 1u);  // RNE on the 20 dropped bits
  const uint32_t code = (r >> 20) - (120u << 3);         // rebias 127 -> 7
  return sign | (code > 0x7fu ? 0x7fu : code);
}

__global__ void __launch_bounds__(256)
kv_quant_fp8_kernel(const KvQuantArgs a) {
  __shared__ float red[4];
  // heads fastest: neighbouring workgroups read and write the same token rows (each row holds
  // every head), which keeps the HBM accesses of concurrent workgroups together
  const int64_t nbh = (int64_t)a.B * a.H;
  const int64_t bh = blockIdx.x % nbh;
  const int64_t blk = blockIdx.x / nbh;
  const int h = (int)(bh % a.H);
  const int b = (int)(bh / a.H);
  const int t = threadIdx.x;
  const int cpr = a.D / 8;               // 16-byte chunks per token row
  const int rows_per_pass = 256 / cpr;
  const int col = t % cpr;
  const int r0 = t / cpr;
  const int64_t tok0 = blk * a.block;

  float v[8][8];
  float amax = 0.0f;
  const int passes = (a.block + rows_per_pass - 1) / rows_per_pass;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = r0 + i * rows_per_pass;
    const int64_t tok = tok0 + row;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[i][e] = 0.0f;
    if (i < passes && row < a.block && tok < a.L) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(a.x + a.sb * b + a.sl * tok + a.sh * h +
                                                      8 * col);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[i][2 * k] = bf16_lo(w[k]);
        v[i][2 * k + 1] = bf16_hi(w[k]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[i][e]));
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  if ((t & 63) == 0) red[t >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  // amax = m 2^E, m in [1, 2): amax / 2^k <= 1.75 * 2^8 from k = E - 8 on when m <= 1.75
  // (mantissa field <= 0x600000), else from k = E - 7; a subnormal amax gets k = -126
  int k = 0;
  if (amax > 0.0f) {
    const uint32_t u = __float_as_uint(amax);
    const int eb = (int)(u >> 23);
    k = eb == 0 ? -126 : eb - 127 - ((u & 0x7fffffu) <= 0x600000u ? 8 : 7);
    k = k < -126 ? -126 : k;
  }
  const float scale = __uint_as_float((uint32_t)(127 + k) << 23);
  const float inv = __uint_as_float((uint32_t)(127 - k) << 23);
  if (t == 0) a.scales[bh * a.nblk + blk] = scale;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = r0 + i * rows_per_pass;
    const int64_t tok = tok0 + row;
    if (i < passes && row < a.block && tok < a.L) {
      u32x2 o;
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        uint32_t wd = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) wd |= e4m3fn_encode(__fmul_rn(v[i][4 * k + e], inv)) << (8 * e);
        o[k] = wd;
      }
      *reinterpret_cast<u32x2*>(a.codes + (((int64_t)b * a.L + tok) * a.H + h) * a.D + 8 * col) = o;
    }
  }
}

hipError_t launch_kv_quant_fp8(const KvQuantArgs& a, hipStream_t stream) {
  const int64_t nwg = (int64_t)a.B * a.H * a.nblk;
  hipLaunchKernelGGL(kv_quant_fp8_kernel, dim3((uint32_t)nwg), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace lbw
