// extern "C" entry points of liblbw_attn.so: argument validation, work decomposition and
// kernel launches. No allocation and no device synchronisation happens here.

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <functional>
#include <mutex>
#include <queue>
#include <string>
#include <vector>

#include "lbw_attn.h"
#include "attn_fwd.h"

using namespace lbw;

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(LBW_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool mult8(int64_t s) { return (s & 7) == 0; }

int num_cus() {
  static std::mutex mu;
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lk(mu);
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

// Estimated run time, in tile steps, of a launch with s KV splits: greedy list scheduling of
// the workgroups in dispatch order (q-tile fastest, then split, then batch x head) over the
// CUs, one workgroup per CU. A workgroup costs its tile count times (0.3 + 0.7 * its share of
// active query waves); each split beyond the first adds 3 % (partials written and merged).
// The constants are fitted to measured gfx950 times of the 1.3B/14B chunk shapes.
double split_cost(int64_t bh, int lq, int bm, int64_t ntiles, int s, int cus) {
  const int nq = (lq + bm - 1) / bm;
  const int tail_q = lq - (nq - 1) * bm;                  // queries in the last q-tile
  const double tail_w = (double)((tail_q + 31) / 32) / (bm / 32);
  const int64_t per = (ntiles + s - 1) / s;
  std::priority_queue<double, std::vector<double>, std::greater<double>> cu;
  for (int i = 0; i < cus; ++i) cu.push(0.0);
  for (int64_t g = 0; g < bh; ++g)
    for (int sp = 0; sp < s; ++sp) {
      const int64_t t0 = sp * per, t1 = std::min<int64_t>(ntiles, t0 + per);
      const double tiles = t1 > t0 ? (double)(t1 - t0) : 0.0;
      for (int qt = 0; qt < nq; ++qt) {
        const double w = qt + 1 < nq ? 1.0 : tail_w;
        const double t = cu.top();
        cu.pop();
        cu.push(t + tiles * (0.3 + 0.7 * w));
      }
    }
  double span = 0.0;
  while (!cu.empty()) { span = cu.top(); cu.pop(); }
  return span * (1.0 + 0.03 * (s - 1));
}

// Number of KV splits (1..8) with the lowest estimated time; decisions are cached per shape.
int choose_splits(int64_t bh, int lq, int bm, int64_t ntiles, int cus) {
  struct Entry { int64_t bh, ntiles; int lq, cus, splits; };
  static std::mutex mu;
  static Entry cache[64];
  static int n_cached = 0, next = 0;
  {
    std::lock_guard<std::mutex> lk(mu);
    for (int i = 0; i < n_cached; ++i) {
      const Entry& e = cache[i];
      if (e.bh == bh && e.ntiles == ntiles && e.lq == lq && e.cus == cus) return e.splits;
    }
  }
  int best_s = 1;
  const int64_t nq = (lq + bm - 1) / bm;
  if (bh * nq * 8 <= 200000) {  // keep the simulation cheap; huge launches need no split
    double best = split_cost(bh, lq, bm, ntiles, 1, cus);
    for (int s = 2; s <= 8 && ntiles / s >= 8; ++s) {
      const double c = split_cost(bh, lq, bm, ntiles, s, cus);
      if (c < best) { best = c; best_s = s; }
    }
  }
  std::lock_guard<std::mutex> lk(mu);
  cache[next] = Entry{bh, ntiles, lq, cus, best_s};
  next = (next + 1) % 64;
  if (n_cached < 64) ++n_cached;
  return best_s;
}

constexpr size_t kQueueBytes = 256;  // 8 work-queue counters, padded

// Split calls of up to this many pieces merge their partials in the attention kernel (the last
// piece of each unit); more pieces run the separate merge kernel.
constexpr int kMaxFusedSplits = 8;

struct Plan {
  AttnKernelArgs a;
  int splits;
  bool fused_merge;   // the pieces merge in-kernel (no merge launch)
  size_t part_bytes;  // split partials
  size_t queue_off;   // work-queue counters
  size_t ws_bytes;
};

// Validates the params and fills the kernel arguments (everything but the output mode).
int make_plan(const lbw_attn_params* p, bool fp8, Plan* plan) {
  if (p == nullptr) return fail(LBW_ERR_INVALID, "params is NULL");
  if (p->head_dim != 128)
    return fail(LBW_ERR_UNSUPPORTED, "head_dim %d: only 128 is supported", p->head_dim);
  if (p->batch < 1 || p->heads < 1 || p->lq < 0)
    return fail(LBW_ERR_INVALID, "bad sizes batch=%d heads=%d lq=%d", p->batch, p->heads, p->lq);
  if (p->n_segments < 1 || p->n_segments > LBW_MAX_KV_SEGMENTS)
    return fail(LBW_ERR_INVALID, "n_segments %d not in [1, %d]", p->n_segments,
                LBW_MAX_KV_SEGMENTS);
  if (p->lq > 0 && (p->q == nullptr || !aligned16(p->q)))
    return fail(LBW_ERR_INVALID, "q must be a 16-byte aligned device pointer");
  if (!mult8(p->q_stride_b) || !mult8(p->q_stride_l) || !mult8(p->q_stride_h))
    return fail(LBW_ERR_INVALID, "q strides must be multiples of 8 elements");
  const bool partials = p->part_o != nullptr || p->part_m != nullptr || p->part_l != nullptr;
  if (partials && (p->part_o == nullptr || p->part_m == nullptr || p->part_l == nullptr))
    return fail(LBW_ERR_INVALID, "part_o, part_m and part_l must be given together");
  if (partials && !aligned16(p->part_o)) return fail(LBW_ERR_INVALID, "part_o must be 16-byte aligned");
  if (p->out_dtype != LBW_OUT_BF16 && p->out_dtype != LBW_OUT_FP32)
    return fail(LBW_ERR_INVALID, "out_dtype %d: LBW_OUT_BF16 or LBW_OUT_FP32", p->out_dtype);
  const bool o32 = p->out_dtype == LBW_OUT_FP32;
  if (!partials) {
    const uintptr_t amask = o32 ? 15u : 7u;
    if (p->lq > 0 && (p->out == nullptr || (reinterpret_cast<uintptr_t>(p->out) & amask) != 0))
      return fail(LBW_ERR_INVALID, "out must be a %d-byte aligned device pointer", (int)amask + 1);
    if ((p->o_stride_b & 3) || (p->o_stride_l & 3) || (p->o_stride_h & 3))
      return fail(LBW_ERR_INVALID, "out strides must be multiples of 4 elements");
  }
  if (partials && p->num_splits > 1)
    return fail(LBW_ERR_INVALID, "partial outputs need num_splits <= 1");

  AttnKernelArgs& a = plan->a;
  memset(&a, 0, sizeof(a));
  a.mult_key = -1;
  a.q = static_cast<const uint16_t*>(p->q);
  a.qsb = p->q_stride_b; a.qsl = p->q_stride_l; a.qsh = p->q_stride_h;
  a.out = static_cast<uint16_t*>(p->out);
  a.osb = p->o_stride_b; a.osl = p->o_stride_l; a.osh = p->o_stride_h;
  a.o16 = aligned16(p->out) && mult8(p->o_stride_b) && mult8(p->o_stride_l) && mult8(p->o_stride_h);
  a.o32 = o32 ? 1 : 0;
  a.nseg = p->n_segments;
  // d-major K: every segment or none, bf16 only
  a.k_dmajor = p->seg[0].k_stride_d != 0;
  for (int i = 0; i < p->n_segments; ++i) {
    const lbw_kv_segment& s = p->seg[i];
    if ((s.k_stride_d != 0) != (a.k_dmajor != 0))
      return fail(LBW_ERR_INVALID, "segment %d: every segment's K must be d-major, or none", i);
    if (s.k_stride_d == 0) continue;
    if (fp8) return fail(LBW_ERR_UNSUPPORTED, "d-major K: bf16 segments only");
    if (s.k_stride_d < 0 || s.k_stride_l != 1)
      return fail(LBW_ERR_INVALID, "segment %d: d-major K needs k_stride_l = 1 and k_stride_d > 0", i);
    if ((s.len & 7) || (s.k_stride_d & 7) || (s.k_stride_b & 7) || (s.k_stride_h & 7))
      return fail(LBW_ERR_INVALID,
                  "segment %d: d-major K needs len and its strides multiples of 8 elements", i);
    if (s.len > 0 && s.k_stride_d < s.len)
      return fail(LBW_ERR_INVALID, "segment %d: d-major K d stride %lld below len %lld", i,
                  (long long)s.k_stride_d, (long long)s.len);
    // a tile's 128 d-rows are addressed with 32-bit offsets from its first
    if (s.k_stride_d * 2 * 128 >= (int64_t(1) << 32))
      return fail(LBW_ERR_UNSUPPORTED, "segment %d: d-major K d stride too large", i);
  }
  int64_t start = 0;
  for (int i = 0; i < p->n_segments; ++i) {
    const lbw_kv_segment& s = p->seg[i];
    if (s.len < 0) return fail(LBW_ERR_INVALID, "segment %d: negative length", i);
    // the kernels index keys within a segment with 32-bit integers
    if (s.len > (int64_t(1) << 30))
      return fail(LBW_ERR_UNSUPPORTED, "segment %d: more than 2^30 keys", i);
    if (s.len > 0) {
      if (s.k == nullptr || s.v == nullptr || !aligned16(s.k) || !aligned16(s.v))
        return fail(LBW_ERR_INVALID, "segment %d: k/v must be 16-byte aligned device pointers", i);
      const int64_t el = fp8 ? 16 : 8;  // 16-byte granules in elements
      if ((s.k_stride_b % el) || (s.k_stride_l % el && s.k_stride_d == 0) || (s.k_stride_h % el) ||
          (s.v_stride_b % el) || (s.v_stride_l % el) || (s.v_stride_h % el))
        return fail(LBW_ERR_INVALID, "segment %d: strides must be multiples of %lld elements", i,
                    (long long)el);
      // a tile's 64 rows must be addressable with 32-bit offsets from its first row
      const int64_t esz = fp8 ? 1 : 2;
      if (s.k_stride_l * esz * 64 >= (int64_t(1) << 32) || s.v_stride_l * esz * 64 >= (int64_t(1) << 32))
        return fail(LBW_ERR_UNSUPPORTED, "segment %d: row stride too large", i);
      if (fp8 && (s.k_scale == nullptr || s.v_scale == nullptr))
        return fail(LBW_ERR_INVALID, "segment %d: fp8 scales missing", i);
    }
    SegDesc& d = a.seg[i];
    d.k = static_cast<const uint16_t*>(s.k);
    d.v = static_cast<const uint16_t*>(s.v);
    d.start = start;
    d.len = s.len;
    d.ksb = s.k_stride_b; d.ksl = s.k_stride_l; d.ksh = s.k_stride_h;
    d.vsb = s.v_stride_b; d.vsl = s.v_stride_l; d.vsh = s.v_stride_h;
    d.ks = s.k_scale; d.vs = s.v_scale;
    d.nblk = (s.len + LBW_FP8_BLOCK - 1) / LBW_FP8_BLOCK;
    d.ksd = s.k_stride_d;
    start += s.len;
  }
  a.total = start;
  a.lo = p->kv_lo > 0 ? p->kv_lo : 0;
  a.hi = (p->kv_hi < 0 || p->kv_hi > start) ? start : p->kv_hi;
  if (a.hi < a.lo) a.hi = a.lo;
  a.lo_dev = p->kv_lo_dev;
  a.hi_dev = p->kv_hi_dev;
  a.key_bias = p->key_bias;
  if (a.key_bias != nullptr && (fp8 || partials))
    return fail(LBW_ERR_UNSUPPORTED, "key_bias: bf16 normalised outputs only (no fp8, no partials)");
  a.k_lens = p->k_lens;
  const float scale = p->softmax_scale > 0.0f ? p->softmax_scale : 1.0f / sqrtf((float)p->head_dim);
  a.scale = scale;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.inv_scale = 1.0f / scale;
  a.B = p->batch; a.H = p->heads; a.Lq = p->lq;
  const int bm = attn_block_m(), bn = attn_block_n();
  a.n_qtiles = (p->lq + bm - 1) / bm;
  a.part_o = p->part_o; a.part_m = p->part_m; a.part_l = p->part_l;
  a.mode = partials ? kModePartials : kModeNormalized;
  a.track_max = partials ? 1 : 0;  // split partials only feed lbw's own merge

  // KV splits: more workgroups when (q-tiles x heads x batch) leaves the last dispatch round
  // of the CUs mostly empty. Each extra split costs one fp32 partial per query row.
  int splits = 1;
  if (!partials) {
    if (p->num_splits > 0) {
      splits = p->num_splits > 16 ? 16 : p->num_splits;
    } else {
      const int64_t ntiles = (a.hi - a.lo + bn - 1) / bn;
      splits = choose_splits((int64_t)a.H * a.B, p->lq, bm, ntiles, num_cus());
    }
  }
  plan->splits = splits;
  // [split partials][8 work-queue counters at a 256-byte boundary, then (split calls whose
  // pieces merge in-kernel) one arrival counter per unit]
  plan->part_bytes = splits > 1 ? (size_t)splits * a.B * a.H * a.Lq * (p->head_dim + 2) * sizeof(float) : 0;
  plan->queue_off = (plan->part_bytes + 255) & ~(size_t)255;
  plan->fused_merge = splits > 1 && splits <= kMaxFusedSplits;
  const size_t units = (size_t)a.n_qtiles * a.H * a.B;
  const size_t cnt_bytes = (8 + (plan->fused_merge ? units : 0)) * sizeof(uint32_t);
  plan->ws_bytes = plan->queue_off + std::max(kQueueBytes, (cnt_bytes + 255) & ~(size_t)255);
  a.splits = splits;
  return LBW_OK;
}

int run_attention(const lbw_attn_params* p, bool fp8, void* ws, size_t ws_bytes, void* stream,
                  int64_t mult_key = -1, double mult = 1.0, bool cross = false) {
  Plan plan;
  int rc = make_plan(p, fp8, &plan);
  if (rc != LBW_OK) return rc;
  if (p->lq == 0) return LBW_OK;
  AttnKernelArgs& a = plan.a;
  if (mult_key >= 0) {
    a.mult_key = mult_key;
    a.mult_raw = (float)(log(mult) / (double)a.scale);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  // Cross-attention: the persistent kernel whenever the keys may fit its LDS-resident chunk
  // (per-batch k_lens are only known on the device; longer batches run there in chunks). A
  // context the host knows to be longer, every key attended (the reference's unmasked 512-row
  // call), streams through the ring form; a longer one with the dedup's multiplicity bias goes
  // to the chunk kernel as a single pass.
  // (the cross kernels read K token-major and take no general bias: such a context runs the
  // chunk kernel, one pass)
  if (cross && (a.k_dmajor || a.key_bias != nullptr)) cross = false;
  bool ring = false;
  if (cross && a.k_lens == nullptr && a.hi - a.lo > cross_attn_max_keys_resident()) {
    cross = false;
    ring = a.mult_key < 0;
  }
  if (ring) {
    // Q and O rows of one (batch, head) are addressed with 31-bit byte offsets
    const int64_t rows = (int64_t)p->lq + 512;
    if (rows * p->q_stride_l * 2 >= (int64_t(1) << 31) || rows * p->o_stride_l * 4 >= (int64_t(1) << 31))
      return fail(LBW_ERR_UNSUPPORTED, "cross-attention: q/out rows span more than 2 GiB");
    hipError_t e = launch_cross_ring(a, num_cus(), st);
    if (e != hipSuccess) return hip_fail(e, "cross-attention ring kernel launch");
    return LBW_OK;
  }
  if (cross) {
    // one segment, single pass: the persistent cross-attention kernel; its chunk loads address
    // up to 320 rows with 32-bit offsets from the chunk's first row
    const lbw_kv_segment& s0 = p->seg[0];
    if (s0.k_stride_l * 2 * cross_attn_max_keys_resident() >= (int64_t(1) << 32) ||
        s0.v_stride_l * 2 * cross_attn_max_keys_resident() >= (int64_t(1) << 32))
      return fail(LBW_ERR_UNSUPPORTED, "cross-attention: K/V row stride too large");
    // Q and O rows of one (batch, head) are addressed with 31-bit byte offsets (buffer ranges)
    const int64_t rows = (int64_t)p->lq + 512;
    if (rows * p->q_stride_l * 2 >= (int64_t(1) << 31) || rows * p->o_stride_l * 4 >= (int64_t(1) << 31))
      return fail(LBW_ERR_UNSUPPORTED, "cross-attention: q/out rows span more than 2 GiB");
    hipError_t e = launch_cross_attn(a, num_cus(), st);
    if (e != hipSuccess) return hip_fail(e, "cross-attention kernel launch");
    return LBW_OK;
  }
  const bool ws_ok = ws != nullptr && ws_bytes >= plan.ws_bytes && aligned16(ws);
  if (ws_ok) {
    a.queue = reinterpret_cast<uint32_t*>(static_cast<unsigned char*>(ws) + plan.queue_off);
  }
  if (plan.splits > 1) {
    if (!ws_ok)
      return fail(LBW_ERR_WORKSPACE, "workspace of %zu bytes needed (got %zu)", plan.ws_bytes, ws_bytes);
    const size_t rows = (size_t)plan.splits * a.B * a.H * a.Lq;
    float* base = static_cast<float*>(ws);
    a.part_o = base;
    a.part_m = base + rows * p->head_dim;
    a.part_l = a.part_m + rows;
    a.mode = kModePartials;
    if (plan.fused_merge) a.merge_cnt = a.queue + 8;
  }
  hipError_t e = fp8 ? launch_attn_fwd_fp8(a, st) : launch_attn_fwd(a, st);
  if (e != hipSuccess) return hip_fail(e, "attention kernel launch");
  if (plan.splits > 1 && !plan.fused_merge) {
    MergeKernelArgs m;
    memset(&m, 0, sizeof(m));
    m.n = plan.splits;
    const size_t per = (size_t)a.B * a.H * a.Lq;
    for (int s = 0; s < plan.splits; ++s) {
      m.o[s] = a.part_o + s * per * p->head_dim;
      m.m[s] = a.part_m + s * per;
      m.l[s] = a.part_l + s * per;
    }
    m.B = a.B; m.H = a.H; m.Lq = a.Lq; m.D = p->head_dim;
    m.out = static_cast<uint16_t*>(p->out);
    m.osb = p->o_stride_b; m.osl = p->o_stride_l; m.osh = p->o_stride_h;
    m.o32 = a.o32;
    e = launch_attn_merge(m, st);
    if (e != hipSuccess) return hip_fail(e, "merge kernel launch");
  }
  return LBW_OK;
}

// ---- scratch of lbw_attention_fwd_noalloc
// The work-queue counters and split partials of that entry point live in this file-scope device
// array instead of a caller's workspace: each GPU the library runs on holds its own copy, at its
// own address, until the process ends. In host code `scratch` names a host-side stand-in, not
// the device memory: host code only ever uses the address hipGetSymbolAddress returns for the
// current device (noalloc_scratch), never the array's name. Calls that overlap on one GPU share
// the array and race.
static __device__ __align__(256) unsigned char scratch[LBW_NOALLOC_SCRATCH_BYTES];

// Device address of the current device's `scratch`, looked up once per device (with that
// device current); nullptr with the error set when the lookup fails.
void* noalloc_scratch() {
  static std::mutex mu;
  static void* ptrs[64] = {nullptr};
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    hip_fail(e, "hipGetDevice");
    return nullptr;
  }
  if (dev < 0 || dev >= 64) {
    fail(LBW_ERR_UNSUPPORTED, "device %d: the no-alloc entry point serves devices 0..63", dev);
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(mu);
  if (ptrs[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
      return nullptr;
    }
    ptrs[dev] = ptr;
  }
  return ptrs[dev];
}

}  // namespace

extern "C" {

const char* lbw_last_error(void) { return g_err.c_str(); }
int lbw_abi_version(void) { return LBW_ABI_VERSION; }

size_t lbw_attention_workspace_size(const lbw_attn_params* p) {
  Plan plan;
  if (make_plan(p, false, &plan) != LBW_OK) return 0;
  return plan.ws_bytes;
}

size_t lbw_attention_fp8kv_workspace_size(const lbw_attn_params* p) {
  Plan plan;
  if (make_plan(p, true, &plan) != LBW_OK) return 0;
  return plan.ws_bytes;
}

int lbw_attention_fwd(const lbw_attn_params* p, void* workspace, size_t workspace_bytes,
                      void* stream) {
  return run_attention(p, false, workspace, workspace_bytes, stream);
}

int lbw_cross_attention_fwd(const lbw_attn_params* p, void* stream) {
  if (p == nullptr) return fail(LBW_ERR_INVALID, "params is NULL");
  if (p->n_segments != 1) return fail(LBW_ERR_INVALID, "cross-attention takes one KV segment");
  if (p->seg[0].len > 4096)
    return fail(LBW_ERR_INVALID, "cross-attention context of %lld keys exceeds 4096",
                (long long)p->seg[0].len);
  if (p->num_splits > 1) return fail(LBW_ERR_INVALID, "cross-attention is single pass");
  if (p->part_o != nullptr || p->part_m != nullptr || p->part_l != nullptr)
    return fail(LBW_ERR_INVALID, "cross-attention has no partials mode");
  if (p->kv_lo_dev != nullptr || p->kv_hi_dev != nullptr)
    return fail(LBW_ERR_INVALID, "cross-attention takes no device window bounds");
  lbw_attn_params q = *p;
  q.num_splits = 1;
  return run_attention(&q, false, nullptr, 0, stream, -1, 1.0, true);
}

int lbw_cross_attention_dedup_fwd(const lbw_attn_params* p, int64_t n_distinct, void* stream) {
  if (p == nullptr) return fail(LBW_ERR_INVALID, "params is NULL");
  if (p->n_segments != 1) return fail(LBW_ERR_INVALID, "cross-attention takes one KV segment");
  const int64_t L = p->seg[0].len;
  if (L > 4096)
    return fail(LBW_ERR_INVALID, "cross-attention context of %lld keys exceeds 4096", (long long)L);
  if (n_distinct < 0 || n_distinct > L)
    return fail(LBW_ERR_INVALID, "n_distinct %lld not in [0, %lld]", (long long)n_distinct,
                (long long)L);
  if (p->k_lens != nullptr || p->kv_lo != 0 || p->kv_hi >= 0 || p->kv_lo_dev != nullptr ||
      p->kv_hi_dev != nullptr)
    return fail(LBW_ERR_INVALID, "dedup attends the whole context: no k_lens or window");
  if (p->key_bias != nullptr)
    return fail(LBW_ERR_INVALID, "dedup carries its own bias: no key_bias");
  if (p->num_splits > 1) return fail(LBW_ERR_INVALID, "cross-attention is single pass");
  if (p->part_o != nullptr || p->part_m != nullptr || p->part_l != nullptr)
    return fail(LBW_ERR_INVALID, "cross-attention has no partials mode");
  lbw_attn_params q = *p;
  q.num_splits = 1;
  if (n_distinct == L) return run_attention(&q, false, nullptr, 0, stream, -1, 1.0, true);
  // The distinct keys plus the r identical ones up to the end of their 64-key tile (free: the
  // tile is read anyway), each of those weighted m / r (m = L - n_distinct identical rows in
  // all): cross_dedup_bias's log(m / r) form. Spreading the weight over r bf16 probabilities
  // keeps the rounding error of that dominant term close to the undeduplicated call's.
  const int64_t bn = attn_block_n();
  const int64_t end = std::min<int64_t>(L, (n_distinct / bn + 1) * bn);
  q.kv_lo = 0;
  q.kv_hi = end;
  return run_attention(&q, false, nullptr, 0, stream, n_distinct,
                       (double)(L - n_distinct) / (double)(end - n_distinct), true);
}

int lbw_attention_fwd_noalloc(const lbw_attn_params* p, void* stream) {
  Plan plan;
  int rc = make_plan(p, false, &plan);
  if (rc != LBW_OK) return rc;
  lbw_attn_params q = *p;
  if (plan.ws_bytes > LBW_NOALLOC_SCRATCH_BYTES) {
    if (p->num_splits > 0)
      return fail(LBW_ERR_WORKSPACE,
                  "num_splits %d needs %zu bytes of scratch; lbw_attention_fwd_noalloc holds %zu "
                  "(ask for fewer splits, 0 = the most that fit, or use lbw_attention_fwd)",
                  p->num_splits, plan.ws_bytes, (size_t)LBW_NOALLOC_SCRATCH_BYTES);
    // the host's choice does not fit: the largest split count whose partials do (1 always does)
    // next to the counters (8 + one per unit) and the alignment gap
    const size_t per = (size_t)p->batch * p->heads * p->lq * (p->head_dim + 2) * sizeof(float);
    const size_t units = (size_t)plan.a.n_qtiles * p->heads * p->batch;
    const size_t fixed = 512 + (8 + units) * sizeof(uint32_t);
    const size_t room = LBW_NOALLOC_SCRATCH_BYTES > fixed ? LBW_NOALLOC_SCRATCH_BYTES - fixed : 0;
    q.num_splits = (int)std::max<size_t>(1, std::min<size_t>(plan.splits - 1, room / per));
  }
  void* ws = noalloc_scratch();
  if (ws == nullptr) return LBW_ERR_HIP;
  return run_attention(&q, false, ws, LBW_NOALLOC_SCRATCH_BYTES, stream);
}

int lbw_attention_fwd_fp8kv(const lbw_attn_params* p, void* workspace, size_t workspace_bytes,
                            void* stream) {
  return run_attention(p, true, workspace, workspace_bytes, stream);
}

int lbw_attn_merge(int32_t n_parts, const float* const* part_o, const float* const* part_m,
                   const float* const* part_l, int32_t batch, int32_t heads, int32_t lq,
                   int32_t head_dim, void* out, int64_t o_stride_b, int64_t o_stride_l,
                   int64_t o_stride_h, void* stream) {
  if (n_parts < 1 || n_parts > 16) return fail(LBW_ERR_INVALID, "n_parts %d not in [1, 16]", n_parts);
  if (head_dim != 128) return fail(LBW_ERR_UNSUPPORTED, "head_dim %d: only 128", head_dim);
  if (batch < 1 || heads < 1 || lq < 0) return fail(LBW_ERR_INVALID, "bad sizes");
  if (part_o == nullptr || part_m == nullptr || part_l == nullptr || out == nullptr)
    return fail(LBW_ERR_INVALID, "NULL pointer");
  if ((reinterpret_cast<uintptr_t>(out) & 7u) || (o_stride_b & 3) || (o_stride_l & 3) ||
      (o_stride_h & 3))
    return fail(LBW_ERR_INVALID, "out must be 8-byte aligned with strides multiple of 4");
  if (lq == 0) return LBW_OK;
  MergeKernelArgs m;
  memset(&m, 0, sizeof(m));
  m.n = n_parts;
  for (int i = 0; i < n_parts; ++i) {
    if (part_o[i] == nullptr || part_m[i] == nullptr || part_l[i] == nullptr || !aligned16(part_o[i]))
      return fail(LBW_ERR_INVALID, "partial %d: NULL or misaligned pointer", i);
    m.o[i] = part_o[i];
    m.m[i] = part_m[i];
    m.l[i] = part_l[i];
  }
  m.B = batch; m.H = heads; m.Lq = lq; m.D = head_dim;
  m.out = static_cast<uint16_t*>(out);
  m.osb = o_stride_b; m.osl = o_stride_l; m.osh = o_stride_h;
  hipError_t e = launch_attn_merge(m, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "merge kernel launch");
  return LBW_OK;
}

int lbw_attn_merge_partials(int32_t n_parts, const float* const* part_o,
                            const float* const* part_m, const float* const* part_l, int32_t batch,
                            int32_t heads, int32_t lq, int32_t head_dim, float* out_o,
                            float* out_m, float* out_l, void* stream) {
  if (n_parts < 1 || n_parts > 16) return fail(LBW_ERR_INVALID, "n_parts %d not in [1, 16]", n_parts);
  if (head_dim != 128) return fail(LBW_ERR_UNSUPPORTED, "head_dim %d: only 128", head_dim);
  if (batch < 1 || heads < 1 || lq < 0) return fail(LBW_ERR_INVALID, "bad sizes");
  if (part_o == nullptr || part_m == nullptr || part_l == nullptr || out_o == nullptr ||
      out_m == nullptr || out_l == nullptr || !aligned16(out_o))
    return fail(LBW_ERR_INVALID, "NULL or misaligned pointer");
  if (lq == 0) return LBW_OK;
  MergeKernelArgs m;
  memset(&m, 0, sizeof(m));
  m.n = n_parts;
  for (int i = 0; i < n_parts; ++i) {
    if (part_o[i] == nullptr || part_m[i] == nullptr || part_l[i] == nullptr || !aligned16(part_o[i]))
      return fail(LBW_ERR_INVALID, "partial %d: NULL or misaligned pointer", i);
    m.o[i] = part_o[i];
    m.m[i] = part_m[i];
    m.l[i] = part_l[i];
  }
  m.B = batch; m.H = heads; m.Lq = lq; m.D = head_dim;
  m.part_o = out_o; m.part_m = out_m; m.part_l = out_l;
  hipError_t e = launch_attn_merge(m, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "merge kernel launch");
  return LBW_OK;
}

int lbw_qk_norm_rope(const lbw_qk_norm_rope_params* p, void* stream) {
  if (p == nullptr) return fail(LBW_ERR_INVALID, "params is NULL");
  if (p->tokens < 0 || p->heads < 1 || p->dim < 8 || p->dim % p->heads != 0)
    return fail(LBW_ERR_INVALID, "bad sizes tokens=%d dim=%d heads=%d", p->tokens, p->dim, p->heads);
  const int D = p->dim / p->heads;
  if (D % 8 != 0 || 512 % D != 0 || p->dim % 8 != 0 || p->dim > 8192)
    return fail(LBW_ERR_UNSUPPORTED,
                "dim %d / head_dim %d: need head_dim a power of two in [8, 512], dim a multiple "
                "of 8 and <= 8192", p->dim, D);
  if (p->s0 < 0 || p->s1 < 0 || p->s0 + 2 * p->s1 != D / 2)
    return fail(LBW_ERR_INVALID, "rope split s0=%d s1=%d does not cover head_dim/2=%d", p->s0,
                p->s1, D / 2);
  if (p->grid_f < 0 || p->grid_h < 0 || p->grid_w < 0)
    return fail(LBW_ERR_INVALID, "negative grid");
  const int64_t gt = (int64_t)p->grid_f * p->grid_h * p->grid_w;
  if (gt > 0 && (p->grid_h == 0 || p->grid_w == 0)) return fail(LBW_ERR_INVALID, "bad grid");
  const int64_t ntab = 2 * ((int64_t)p->grid_f * p->s0 + (int64_t)p->grid_h * p->s1 +
                            (int64_t)p->grid_w * p->s1);
  if (ntab > qk_norm_rope_max_table_floats())
    return fail(LBW_ERR_UNSUPPORTED, "rope tables of %lld floats exceed %d", (long long)ntab,
                qk_norm_rope_max_table_floats());
  if (gt > 0 && p->rope == nullptr) return fail(LBW_ERR_INVALID, "rope tables missing");
  if (p->out_layout != LBW_QK_ROWS && p->out_layout != LBW_QK_DMAJOR)
    return fail(LBW_ERR_INVALID, "out_layout %d: LBW_QK_ROWS or LBW_QK_DMAJOR", p->out_layout);
  const bool dmajor = p->out_layout == LBW_QK_DMAJOR;
  if (dmajor && p->dim > qk_norm_rope_dmajor_max_dim())
    return fail(LBW_ERR_UNSUPPORTED, "d-major output: dim %d above %d", p->dim,
                qk_norm_rope_dmajor_max_dim());
  if (dmajor && qk_norm_rope_lds_bytes((int)ntab, p->dim, QK_LAYOUT_DMAJOR) > qk_norm_rope_lds_limit())
    return fail(LBW_ERR_UNSUPPORTED, "d-major output: rope tables (%lld floats) and dim %d exceed LDS",
                (long long)ntab, p->dim);
  if (p->tokens == 0) return LBW_OK;
  const bool has_k = p->k != nullptr;
  const void* ptrs[] = {p->q, p->wq, has_k ? p->k : p->q, has_k ? p->wk : p->wq};
  for (const void* q : ptrs)
    if (q == nullptr || !aligned16(q)) return fail(LBW_ERR_INVALID, "q/k/gamma must be 16-byte aligned");
  if ((p->bq && !aligned16(p->bq)) || (has_k && p->bk && !aligned16(p->bk)))
    return fail(LBW_ERR_INVALID, "bias must be 16-byte aligned");
  if (!mult8(p->q_stride) || (has_k && !mult8(p->k_stride)))
    return fail(LBW_ERR_INVALID, "input row strides must be multiples of 8 elements");
  if (p->q_out == nullptr || (has_k && p->k_out == nullptr))
    return fail(LBW_ERR_INVALID, "q_out/k_out missing");
  if (!dmajor) {
    if (!aligned16(p->q_out) || (has_k && !aligned16(p->k_out)))
      return fail(LBW_ERR_INVALID, "row outputs must be 16-byte aligned");
    if (!mult8(p->q_out_stride) || (has_k && !mult8(p->k_out_stride)))
      return fail(LBW_ERR_INVALID, "output row strides must be multiples of 8 elements");
  } else {
    if ((reinterpret_cast<uintptr_t>(p->q_out) & 1) ||
        (has_k && (reinterpret_cast<uintptr_t>(p->k_out) & 1)))
      return fail(LBW_ERR_INVALID, "d-major outputs must be 2-byte aligned");
    if (p->q_out_stride < p->tokens || (has_k && p->k_out_stride < p->tokens))
      return fail(LBW_ERR_INVALID, "d-major outputs: d stride %lld/%lld below tokens %d",
                  (long long)p->q_out_stride, (long long)p->k_out_stride, p->tokens);
  }
  if (p->v != nullptr && (p->v_out == nullptr || !aligned16(p->v) || !aligned16(p->v_out) ||
                          !mult8(p->v_stride) || !mult8(p->v_out_stride)))
    return fail(LBW_ERR_INVALID, "v copy: aligned v and v_out with 8-element strides needed");
  QkNormRopeArgs a;
  memset(&a, 0, sizeof(a));
  a.L = p->tokens; a.C = p->dim; a.H = p->heads;
  a.q = static_cast<const uint16_t*>(p->q); a.qs = p->q_stride;
  if (has_k) {
    a.k = static_cast<const uint16_t*>(p->k); a.ks = p->k_stride;
    a.bk = static_cast<const uint16_t*>(p->bk); a.wk = static_cast<const uint16_t*>(p->wk);
  }
  a.bq = static_cast<const uint16_t*>(p->bq); a.wq = static_cast<const uint16_t*>(p->wq);
  a.eps = p->eps;
  a.inv_c = 1.0f / (float)p->dim;
  a.rope = p->rope;
  a.gf = p->grid_f; a.gh = p->grid_h; a.gw = p->grid_w; a.s0 = p->s0; a.s1 = p->s1;
  a.ntab = (int)ntab;
  if (gt == 0) { a.gf = 0; a.gh = 1; a.gw = 1; a.ntab = 0; }
  a.qo = static_cast<uint16_t*>(p->q_out); a.qos = p->q_out_stride;
  if (has_k) { a.ko = static_cast<uint16_t*>(p->k_out); a.kos = p->k_out_stride; }
  a.layout = dmajor ? QK_LAYOUT_DMAJOR : QK_LAYOUT_ROWS;
  a.qo_vec = aligned16(p->q_out) && mult8(p->q_out_stride);
  a.ko_vec = has_k && aligned16(p->k_out) && mult8(p->k_out_stride);
  a.q_scale = p->q_out_scale; a.k_scale = p->k_out_scale;
  a.v = static_cast<const uint16_t*>(p->v); a.vs = p->v_stride;
  a.vo = static_cast<uint16_t*>(p->v_out); a.vos = p->v_out_stride;
  hipError_t e = launch_qk_norm_rope(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "qk_norm_rope launch");
  return LBW_OK;
}

int lbw_kv_quant_fp8(const void* x, int32_t batch, int64_t len, int32_t heads, int32_t head_dim,
                     int64_t s_b, int64_t s_l, int64_t s_h, uint8_t* codes, float* scales,
                     int32_t block, void* stream) {
  if (head_dim != 128) return fail(LBW_ERR_UNSUPPORTED, "head_dim %d: only 128", head_dim);
  if (block != LBW_FP8_BLOCK) return fail(LBW_ERR_UNSUPPORTED, "block %d: only %d", block, LBW_FP8_BLOCK);
  if (batch < 1 || heads < 1 || len < 0) return fail(LBW_ERR_INVALID, "bad sizes");
  if (len == 0) return LBW_OK;
  if (x == nullptr || codes == nullptr || scales == nullptr || !aligned16(x) || !aligned16(codes))
    return fail(LBW_ERR_INVALID, "x/codes must be 16-byte aligned device pointers, scales non-NULL");
  if (!mult8(s_b) || !mult8(s_l) || !mult8(s_h))
    return fail(LBW_ERR_INVALID, "x strides must be multiples of 8 elements");
  KvQuantArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.B = batch; a.H = heads; a.D = head_dim; a.L = len;
  a.sb = s_b; a.sl = s_l; a.sh = s_h;
  a.codes = codes; a.scales = scales; a.block = block;
  a.nblk = (len + block - 1) / block;
  hipError_t e = launch_kv_quant_fp8(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "kv_quant_fp8 launch");
  return LBW_OK;
}

}  // extern "C"
