// torch.ops.lbw: the C ABI of liblbw_attn.so (include/lbw_attn.h) registered as PyTorch
// operators, so that calls from Python go through the dispatcher (no ctypes structs per call)
// and the functional ops trace under torch.compile (fake/Meta kernels give their shapes).
//
// The reference wraps its NKI kernels the same way, as torch ops via wrap_nki
// (wan/modules/attention.py:143-160, kernels/qk_post.py:404-413); these ops take the tensors
// its call sites pass. Every op runs on the tensors' device, on torch's current stream there;
// a nonzero status of the library raises RuntimeError with the library's message. Shape rules
// are those of the C ABI (head_dim 128, contiguous head dim, 16-byte aligned rows); the Python
// wrappers in lbw_amd check them first and raise ValueError with the argument's name.
//
// Host-only C++ (no device code): built with g++ against torch's headers and libraries and
// linked to liblbw_attn.so.

#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <cstring>
#include <vector>

#include "lbw_attn.h"

namespace {

void check(int rc, const char* what) {
  TORCH_CHECK(rc == LBW_OK, what, " failed (status ", rc, "): ", lbw_last_error());
}

void* stream_of(const at::Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.get_device()).stream();
}

void check_bf16_4d(const char* name, const at::Tensor& t, bool dmajor_ok = false) {
  TORCH_CHECK(t.is_cuda(), name, " must be a GPU tensor");
  TORCH_CHECK(t.dim() == 4, name, " must be [B, L, N, D]");
  TORCH_CHECK(t.stride(3) == 1 || (dmajor_ok && t.stride(1) == 1), name,
              dmajor_ok ? " needs a contiguous head dim, or token stride 1 (d-major)"
                        : " needs a contiguous head dim");
}

// A device window bound: a one-element integer tensor on q's device (the flat cache's attn_lo /
// attn_hi, model_fast.py:2538-2550). The kernel reads it on the device; a bound of another
// integer type is converted to int64 there (queued on the current stream, no host sync), and
// `keep` holds the converted tensor until the call has been queued.
const int64_t* dev_bound(const std::optional<at::Tensor>& t, const at::Tensor& q, at::Tensor& keep,
                         const char* name) {
  if (!t.has_value()) return nullptr;
  TORCH_CHECK(t->device() == q.device() && t->numel() == 1 &&
                  at::isIntegralType(t->scalar_type(), /*includeBool=*/false),
              name, " must be a one-element integer tensor on q's device");
  keep = t->scalar_type() == at::kLong ? *t : t->to(at::kLong);
  return keep.data_ptr<int64_t>();
}

// The device bounds of a call, converted where needed (see dev_bound).
struct DevBounds {
  at::Tensor lo, hi;
  void set(lbw_attn_params& p, const std::optional<at::Tensor>& kv_lo_dev,
           const std::optional<at::Tensor>& kv_hi_dev, const at::Tensor& q) {
    p.kv_lo_dev = dev_bound(kv_lo_dev, q, lo, "kv_lo_dev");
    p.kv_hi_dev = dev_bound(kv_hi_dev, q, hi, "kv_hi_dev");
  }
};

// Fills the params common to the attention ops (everything but the output); the K/V segments
// hold kv_type elements (bf16, or the uint8 codes of the fp8 cache).
lbw_attn_params base_params(const at::Tensor& q, at::TensorList k, at::TensorList v,
                            int64_t kv_lo, int64_t kv_hi, double softmax_scale,
                            int64_t num_splits, at::ScalarType kv_type = at::kBFloat16) {
  check_bf16_4d("q", q);
  TORCH_CHECK(q.scalar_type() == at::kBFloat16, "q must be bf16");
  TORCH_CHECK(k.size() == v.size(), "k and v segment lists differ in length");
  TORCH_CHECK(k.size() >= 1 && k.size() <= LBW_MAX_KV_SEGMENTS, k.size(),
              " KV segments: 1..", LBW_MAX_KV_SEGMENTS, " supported");
  lbw_attn_params p;
  std::memset(&p, 0, sizeof(p));
  p.batch = (int32_t)q.size(0);
  p.lq = (int32_t)q.size(1);
  p.heads = (int32_t)q.size(2);
  p.head_dim = (int32_t)q.size(3);
  p.q = q.data_ptr();
  p.q_stride_b = q.stride(0);
  p.q_stride_l = q.stride(1);
  p.q_stride_h = q.stride(2);
  p.n_segments = (int32_t)k.size();
  for (size_t i = 0; i < k.size(); ++i) {
    const at::Tensor& kt = k[i];
    const at::Tensor& vt = v[i];
    check_bf16_4d("k", kt, kv_type == at::kBFloat16);  // (a d-major K view: token stride 1)
    check_bf16_4d("v", vt);
    TORCH_CHECK(kt.device() == q.device() && vt.device() == q.device(),
                "k/v must be on q's device");
    TORCH_CHECK(kt.scalar_type() == kv_type && vt.scalar_type() == kv_type, "k/v of segment ", i,
                " must be ", kv_type == at::kByte ? "uint8 fp8 codes" : "bf16");
    TORCH_CHECK(kt.size(1) == vt.size(1), "k and v of segment ", i, " differ in length");
    lbw_kv_segment& s = p.seg[i];
    s.k = kt.data_ptr();
    s.v = vt.data_ptr();
    s.len = kt.size(1);
    s.k_stride_b = kt.stride(0); s.k_stride_l = kt.stride(1); s.k_stride_h = kt.stride(2);
    s.k_stride_d = kt.stride(3) == 1 ? 0 : kt.stride(3);
    s.v_stride_b = vt.stride(0); s.v_stride_l = vt.stride(1); s.v_stride_h = vt.stride(2);
  }
  p.kv_lo = kv_lo;
  p.kv_hi = kv_hi;
  p.softmax_scale = (float)softmax_scale;
  p.num_splits = (int32_t)num_splits;
  return p;
}

void set_out(lbw_attn_params& p, const at::Tensor& out, const at::Tensor& q) {
  TORCH_CHECK(out.sizes() == q.sizes(), "out must have q's shape");
  TORCH_CHECK(out.scalar_type() == at::kBFloat16 || out.scalar_type() == at::kFloat,
              "out must be bf16 or fp32");
  TORCH_CHECK(out.device() == q.device() && out.stride(3) == 1,
              "out must be on q's device with a contiguous head dim");
  p.out = out.data_ptr();
  p.o_stride_b = out.stride(0);
  p.o_stride_l = out.stride(1);
  p.o_stride_h = out.stride(2);
  p.out_dtype = out.scalar_type() == at::kFloat ? LBW_OUT_FP32 : LBW_OUT_BF16;
}

void set_k_lens(lbw_attn_params& p, const std::optional<at::Tensor>& k_lens,
                const at::Tensor& q) {
  if (!k_lens.has_value()) return;
  const at::Tensor& kl = *k_lens;
  TORCH_CHECK(kl.scalar_type() == at::kInt && kl.is_contiguous() && kl.device() == q.device() &&
                  kl.numel() == q.size(0),
              "k_lens must be a contiguous int32 [B] tensor on q's device");
  p.k_lens = kl.data_ptr<int32_t>();
}

at::Tensor new_out(const at::Tensor& q, bool out_fp32) {
  return at::empty(q.sizes(), q.options().dtype(out_fp32 ? at::kFloat : at::kBFloat16));
}

// Runs an attention entry point that takes a workspace: the split partials and queue counters
// come from torch's caching allocator on the current stream, so calls on different streams
// never share them.
template <typename Fn, typename SizeFn>
void run_with_workspace(const lbw_attn_params& p, const at::Tensor& q, Fn fn, SizeFn size_fn,
                        const char* what) {
  const size_t ws_bytes = size_fn(&p);
  at::Tensor ws;
  if (ws_bytes > 0) ws = at::empty({(int64_t)ws_bytes}, q.options().dtype(at::kByte));
  check(fn(&p, ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes, stream_of(q)), what);
}

// The per-key score bias: fp32, contiguous, one value per key of the segments, on q's device.
void set_key_bias(lbw_attn_params& p, const std::optional<at::Tensor>& key_bias,
                  const at::Tensor& q) {
  if (!key_bias.has_value()) return;
  const at::Tensor& kb = *key_bias;
  int64_t total = 0;
  for (int i = 0; i < p.n_segments; ++i) total += p.seg[i].len;
  TORCH_CHECK(kb.scalar_type() == at::kFloat && kb.is_contiguous() && kb.device() == q.device() &&
                  kb.numel() == total,
              "key_bias must be a contiguous fp32 tensor of ", total, " values (one per key) on "
              "q's device");
  p.key_bias = kb.data_ptr<float>();
}

void attention_out(const at::Tensor& q, at::TensorList k, at::TensorList v, int64_t kv_lo,
                   int64_t kv_hi, const std::optional<at::Tensor>& k_lens, double softmax_scale,
                   int64_t num_splits, const at::Tensor& out,
                   const std::optional<at::Tensor>& kv_lo_dev,
                   const std::optional<at::Tensor>& kv_hi_dev,
                   const std::optional<at::Tensor>& key_bias) {
  c10::DeviceGuard guard(q.device());
  lbw_attn_params p = base_params(q, k, v, kv_lo, kv_hi, softmax_scale, num_splits);
  set_out(p, out, q);
  set_k_lens(p, k_lens, q);
  set_key_bias(p, key_bias, q);
  DevBounds db;
  db.set(p, kv_lo_dev, kv_hi_dev, q);
  run_with_workspace(p, q, lbw_attention_fwd, lbw_attention_workspace_size, "lbw_attention_fwd");
}

at::Tensor attention(const at::Tensor& q, at::TensorList k, at::TensorList v, int64_t kv_lo,
                     int64_t kv_hi, const std::optional<at::Tensor>& k_lens, double softmax_scale,
                     int64_t num_splits, bool out_fp32, const std::optional<at::Tensor>& kv_lo_dev,
                     const std::optional<at::Tensor>& kv_hi_dev,
                     const std::optional<at::Tensor>& key_bias) {
  at::Tensor out = new_out(q, out_fp32);
  attention_out(q, k, v, kv_lo, kv_hi, k_lens, softmax_scale, num_splits, out, kv_lo_dev,
                kv_hi_dev, key_bias);
  return out;
}

void cross_attention_out(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                         const std::optional<at::Tensor>& k_lens, int64_t n_distinct,
                         int64_t kv_lo, int64_t kv_hi, double softmax_scale,
                         const at::Tensor& out) {
  c10::DeviceGuard guard(q.device());
  const at::Tensor ks[1] = {k};
  const at::Tensor vs[1] = {v};
  lbw_attn_params p = base_params(q, at::TensorList(ks, 1), at::TensorList(vs, 1), kv_lo, kv_hi,
                                  softmax_scale, 1);
  set_out(p, out, q);
  set_k_lens(p, k_lens, q);
  if (n_distinct >= 0) {
    TORCH_CHECK(!k_lens.has_value(), "dedup reproduces the unmasked attention: no k_lens");
    check(lbw_cross_attention_dedup_fwd(&p, n_distinct, stream_of(q)),
          "lbw_cross_attention_dedup_fwd");
  } else {
    check(lbw_cross_attention_fwd(&p, stream_of(q)), "lbw_cross_attention_fwd");
  }
}

at::Tensor cross_attention(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                           const std::optional<at::Tensor>& k_lens, int64_t n_distinct,
                           int64_t kv_lo, int64_t kv_hi, double softmax_scale, bool out_fp32) {
  at::Tensor out = new_out(q, out_fp32);
  cross_attention_out(q, k, v, k_lens, n_distinct, kv_lo, kv_hi, softmax_scale, out);
  return out;
}

void attention_fp8kv_out(const at::Tensor& q, at::TensorList k, at::TensorList v,
                         at::TensorList k_scale, at::TensorList v_scale, int64_t kv_lo,
                         int64_t kv_hi, double softmax_scale, int64_t num_splits,
                         const at::Tensor& out, const std::optional<at::Tensor>& kv_lo_dev,
                         const std::optional<at::Tensor>& kv_hi_dev) {
  c10::DeviceGuard guard(q.device());
  TORCH_CHECK(k_scale.size() == k.size() && v_scale.size() == k.size(),
              "one scale tensor per fp8 segment");
  // the codes are uint8 [B, L, N, D]
  lbw_attn_params p = base_params(q, k, v, kv_lo, kv_hi, softmax_scale, num_splits, at::kByte);
  for (size_t i = 0; i < k.size(); ++i) {
    TORCH_CHECK(k_scale[i].scalar_type() == at::kFloat && k_scale[i].is_contiguous() &&
                    v_scale[i].scalar_type() == at::kFloat && v_scale[i].is_contiguous() &&
                    k_scale[i].device() == q.device() && v_scale[i].device() == q.device(),
                "fp8 scales must be contiguous fp32 [B, N, nblk] on q's device");
    const int64_t nblk = (k[i].size(1) + LBW_FP8_BLOCK - 1) / LBW_FP8_BLOCK;
    TORCH_CHECK(k_scale[i].numel() == k[i].size(0) * k[i].size(2) * nblk &&
                    v_scale[i].numel() == k_scale[i].numel(),
                "fp8 scales of segment ", i, " must be [B, N, ", nblk, "]");
    p.seg[i].k_scale = k_scale[i].data_ptr<float>();
    p.seg[i].v_scale = v_scale[i].data_ptr<float>();
  }
  set_out(p, out, q);
  DevBounds db;
  db.set(p, kv_lo_dev, kv_hi_dev, q);
  run_with_workspace(p, q, lbw_attention_fwd_fp8kv, lbw_attention_fp8kv_workspace_size,
                     "lbw_attention_fwd_fp8kv");
}

at::Tensor attention_fp8kv(const at::Tensor& q, at::TensorList k, at::TensorList v,
                           at::TensorList k_scale, at::TensorList v_scale, int64_t kv_lo,
                           int64_t kv_hi, double softmax_scale, int64_t num_splits,
                           bool out_fp32, const std::optional<at::Tensor>& kv_lo_dev,
                           const std::optional<at::Tensor>& kv_hi_dev) {
  at::Tensor out = new_out(q, out_fp32);
  attention_fp8kv_out(q, k, v, k_scale, v_scale, kv_lo, kv_hi, softmax_scale, num_splits, out,
                      kv_lo_dev, kv_hi_dev);
  return out;
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> attention_partial(
    const at::Tensor& q, at::TensorList k, at::TensorList v, int64_t kv_lo, int64_t kv_hi,
    double softmax_scale, const std::optional<at::Tensor>& kv_lo_dev,
    const std::optional<at::Tensor>& kv_hi_dev) {
  c10::DeviceGuard guard(q.device());
  lbw_attn_params p = base_params(q, k, v, kv_lo, kv_hi, softmax_scale, 1);
  DevBounds db;
  db.set(p, kv_lo_dev, kv_hi_dev, q);
  const int64_t B = q.size(0), Lq = q.size(1), H = q.size(2), D = q.size(3);
  at::Tensor po = at::empty({B, H, Lq, D}, q.options().dtype(at::kFloat));
  at::Tensor pm = at::empty({B, H, Lq}, q.options().dtype(at::kFloat));
  at::Tensor pl = at::empty({B, H, Lq}, q.options().dtype(at::kFloat));
  p.part_o = po.data_ptr<float>();
  p.part_m = pm.data_ptr<float>();
  p.part_l = pl.data_ptr<float>();
  check(lbw_attention_fwd(&p, nullptr, 0, stream_of(q)), "lbw_attention_fwd(partials)");
  return {po, pm, pl};
}

void attention_merge_out(at::TensorList o, at::TensorList m, at::TensorList l,
                         const at::Tensor& out) {
  TORCH_CHECK(o.size() >= 1 && o.size() <= 16 && m.size() == o.size() && l.size() == o.size(),
              "1..16 partials of (O, m, l)");
  TORCH_CHECK(out.is_cuda() && o[0].dim() == 4, "out must be a GPU tensor, O [B, N, Lq, D]");
  c10::DeviceGuard guard(out.device());
  const int64_t B = o[0].size(0), H = o[0].size(1), Lq = o[0].size(2), D = o[0].size(3);
  std::vector<const float*> po, pm, pl;
  for (size_t i = 0; i < o.size(); ++i) {
    TORCH_CHECK(o[i].sizes() == o[0].sizes() && m[i].dim() == 3 && m[i].size(0) == B &&
                    m[i].size(1) == H && m[i].size(2) == Lq && l[i].sizes() == m[i].sizes(),
                "partials differ in shape: O [B, N, Lq, D], m and l [B, N, Lq]");
    TORCH_CHECK(o[i].device() == out.device() && m[i].device() == out.device() &&
                    l[i].device() == out.device(),
                "partials must be on out's device");
    TORCH_CHECK(o[i].is_contiguous() && m[i].is_contiguous() && l[i].is_contiguous() &&
                    o[i].scalar_type() == at::kFloat && m[i].scalar_type() == at::kFloat &&
                    l[i].scalar_type() == at::kFloat,
                "partials must be contiguous fp32");
    po.push_back(o[i].data_ptr<float>());
    pm.push_back(m[i].data_ptr<float>());
    pl.push_back(l[i].data_ptr<float>());
  }
  TORCH_CHECK(out.scalar_type() == at::kBFloat16 && out.dim() == 4 && out.size(0) == B &&
                  out.size(1) == Lq && out.size(2) == H && out.size(3) == D && out.stride(3) == 1,
              "out must be bf16 [B, Lq, N, D] with a contiguous head dim");
  check(lbw_attn_merge((int32_t)o.size(), po.data(), pm.data(), pl.data(), (int32_t)B,
                       (int32_t)H, (int32_t)Lq, (int32_t)D, out.data_ptr(), out.stride(0),
                       out.stride(1), out.stride(2), stream_of(out)),
        "lbw_attn_merge");
}

// The partials of (O, m, l) merged into one triple (cte_call's running chain state).
std::tuple<at::Tensor, at::Tensor, at::Tensor> attention_merge_partials(at::TensorList o,
                                                                       at::TensorList m,
                                                                       at::TensorList l) {
  TORCH_CHECK(o.size() >= 1 && o.size() <= 16 && m.size() == o.size() && l.size() == o.size(),
              "1..16 partials of (O, m, l)");
  TORCH_CHECK(o[0].is_cuda() && o[0].dim() == 4, "O must be a GPU tensor [B, N, Lq, D]");
  c10::DeviceGuard guard(o[0].device());
  const int64_t B = o[0].size(0), H = o[0].size(1), Lq = o[0].size(2), D = o[0].size(3);
  std::vector<const float*> po, pm, pl;
  for (size_t i = 0; i < o.size(); ++i) {
    TORCH_CHECK(o[i].sizes() == o[0].sizes() && m[i].dim() == 3 && m[i].size(0) == B &&
                    m[i].size(1) == H && m[i].size(2) == Lq && l[i].sizes() == m[i].sizes(),
                "partials differ in shape: O [B, N, Lq, D], m and l [B, N, Lq]");
    TORCH_CHECK(o[i].device() == o[0].device() && m[i].device() == o[0].device() &&
                    l[i].device() == o[0].device(),
                "partials must be on one device");
    TORCH_CHECK(o[i].is_contiguous() && m[i].is_contiguous() && l[i].is_contiguous() &&
                    o[i].scalar_type() == at::kFloat && m[i].scalar_type() == at::kFloat &&
                    l[i].scalar_type() == at::kFloat,
                "partials must be contiguous fp32");
    po.push_back(o[i].data_ptr<float>());
    pm.push_back(m[i].data_ptr<float>());
    pl.push_back(l[i].data_ptr<float>());
  }
  at::Tensor ro = at::empty_like(o[0]), rm = at::empty_like(m[0]), rl = at::empty_like(l[0]);
  check(lbw_attn_merge_partials((int32_t)o.size(), po.data(), pm.data(), pl.data(), (int32_t)B,
                                (int32_t)H, (int32_t)Lq, (int32_t)D, ro.data_ptr<float>(),
                                rm.data_ptr<float>(), rl.data_ptr<float>(), stream_of(o[0])),
        "lbw_attn_merge_partials");
  return {ro, rm, rl};
}

at::Tensor attention_merge(at::TensorList o, at::TensorList m, at::TensorList l) {
  TORCH_CHECK(!o.empty(), "no partials");
  at::Tensor out = at::empty({o[0].size(0), o[0].size(2), o[0].size(1), o[0].size(3)},
                             o[0].options().dtype(at::kBFloat16));
  attention_merge_out(o, m, l, out);
  return out;
}

// Row stride of a rows-layout tensor, or the d stride of a d-major [H, D, L] one.
int64_t out_stride(const at::Tensor& t, int64_t layout) {
  return layout == LBW_QK_DMAJOR ? t.stride(1) : t.stride(0);
}

void qk_norm_rope_(const at::Tensor& q, const std::optional<at::Tensor>& k,
                   const std::optional<at::Tensor>& bq, const std::optional<at::Tensor>& bk,
                   const at::Tensor& wq, const std::optional<at::Tensor>& wk,
                   const at::Tensor& rope, at::IntArrayRef rope_dims, double eps, int64_t heads,
                   const at::Tensor& q_out, const std::optional<at::Tensor>& k_out,
                   const std::optional<at::Tensor>& v, const std::optional<at::Tensor>& v_out,
                   double q_scale, double k_scale, int64_t layout) {
  c10::DeviceGuard guard(q.device());
  TORCH_CHECK(rope_dims.size() == 5, "rope_dims = (f, h, w, s0, s1)");
  TORCH_CHECK(q.is_cuda() && q.dim() == 2 && q.scalar_type() == at::kBFloat16 && q.stride(1) == 1,
              "q must be bf16 [L, C] rows on the GPU");
  const int64_t C = q.size(1);
  // every other tensor: bf16 on q's device (the RoPE tables fp32), the vectors of C elements
  auto on_dev = [&](const at::Tensor& t, at::ScalarType st, const char* name) {
    TORCH_CHECK(t.device() == q.device() && t.scalar_type() == st, name, " must be ",
                st == at::kFloat ? "fp32" : "bf16", " on q's device");
  };
  auto vec = [&](const std::optional<at::Tensor>& t, const char* name) {
    if (!t.has_value()) return;
    on_dev(*t, at::kBFloat16, name);
    TORCH_CHECK(t->is_contiguous() && t->numel() == C, name, " must be a contiguous [C] vector");
  };
  vec(bq, "bq");
  vec(bk, "bk");
  vec(wq, "wq");
  vec(wk, "wk");
  on_dev(rope, at::kFloat, "rope");
  TORCH_CHECK(rope.is_contiguous(), "rope must be contiguous");
  // the packed per-axis tables: cos and sin of f x s0, h x s1 and w x s1 angles
  const int64_t ntab = 2 * (rope_dims[0] * rope_dims[3] + (rope_dims[1] + rope_dims[2]) * rope_dims[4]);
  TORCH_CHECK(rope_dims[0] >= 0 && rope_dims[1] >= 0 && rope_dims[2] >= 0 && rope_dims[3] >= 0 &&
                  rope_dims[4] >= 0 && rope.numel() >= ntab,
              "rope holds ", rope.numel(), " floats; rope_dims ", rope_dims, " need ", ntab);
  // [L, C] rows with a contiguous row; the outputs of the d-major layout are [H, D, L] with
  // token stride 1 and head stride D * (d stride)
  auto rows = [&](const at::Tensor& t, const char* name) {
    on_dev(t, at::kBFloat16, name);
    TORCH_CHECK(t.dim() == 2 && t.sizes() == q.sizes() && t.stride(1) == 1, name,
                " must be [L, C] rows of q's shape");
  };
  auto out = [&](const at::Tensor& t, const char* name) {
    if (layout != LBW_QK_DMAJOR) return rows(t, name);
    on_dev(t, at::kBFloat16, name);
    TORCH_CHECK(heads > 0 && C % heads == 0, "heads must divide C");
    const int64_t D = C / heads;
    TORCH_CHECK(t.dim() == 3 && t.size(0) == heads && t.size(1) == D && t.size(2) == q.size(0) &&
                    t.stride(2) == 1 && t.stride(0) == D * t.stride(1),
                name, " must be [H, D, L] with strides (D * s, s, 1)");
  };
  out(q_out, "q_out");
  if (k.has_value()) {
    rows(*k, "k");
    TORCH_CHECK(k_out.has_value(), "k needs k_out");
    out(*k_out, "k_out");
  }
  if (v.has_value()) {
    rows(*v, "v");
    TORCH_CHECK(v_out.has_value(), "v needs v_out");
    rows(*v_out, "v_out");
  }
  lbw_qk_norm_rope_params p;
  std::memset(&p, 0, sizeof(p));
  p.tokens = (int32_t)q.size(0);
  p.dim = (int32_t)q.size(1);
  p.heads = (int32_t)heads;
  p.q = q.data_ptr();
  p.q_stride = q.stride(0);
  p.bq = bq.has_value() ? bq->data_ptr() : nullptr;
  p.wq = wq.data_ptr();
  p.eps = (float)eps;
  p.rope = rope.data_ptr<float>();
  p.grid_f = (int32_t)rope_dims[0];
  p.grid_h = (int32_t)rope_dims[1];
  p.grid_w = (int32_t)rope_dims[2];
  p.s0 = (int32_t)rope_dims[3];
  p.s1 = (int32_t)rope_dims[4];
  p.q_out = q_out.data_ptr();
  p.q_out_stride = out_stride(q_out, layout);
  p.q_out_scale = (float)q_scale;
  p.k_out_scale = (float)k_scale;
  p.out_layout = (int32_t)layout;
  if (k.has_value()) {
    TORCH_CHECK(wk.has_value() && k_out.has_value(), "k needs wk and k_out");
    p.k = k->data_ptr();
    p.k_stride = k->stride(0);
    p.bk = bk.has_value() ? bk->data_ptr() : nullptr;
    p.wk = wk->data_ptr();
    p.k_out = k_out->data_ptr();
    p.k_out_stride = out_stride(*k_out, layout);
  }
  if (v.has_value()) {
    TORCH_CHECK(v_out.has_value(), "v needs v_out");
    p.v = v->data_ptr();
    p.v_stride = v->stride(0);
    p.v_out = v_out->data_ptr();
    p.v_out_stride = v_out->stride(0);
  }
  check(lbw_qk_norm_rope(&p, stream_of(q)), "lbw_qk_norm_rope");
}

void kv_quant_fp8_(const at::Tensor& x, const at::Tensor& codes, const at::Tensor& scales) {
  c10::DeviceGuard guard(x.device());
  check_bf16_4d("x", x);
  TORCH_CHECK(x.scalar_type() == at::kBFloat16, "x must be bf16");
  TORCH_CHECK(codes.scalar_type() == at::kByte && codes.is_contiguous() &&
                  codes.sizes() == x.sizes(),
              "codes must be contiguous uint8 of x's shape");
  TORCH_CHECK(scales.scalar_type() == at::kFloat && scales.is_contiguous(),
              "scales must be contiguous fp32");
  TORCH_CHECK(codes.device() == x.device() && scales.device() == x.device(),
              "codes and scales must be on x's device");
  const int64_t nblk = (x.size(1) + LBW_FP8_BLOCK - 1) / LBW_FP8_BLOCK;
  TORCH_CHECK(scales.numel() == x.size(0) * x.size(2) * nblk, "scales must be [B, N, ", nblk,
              "] (", x.size(0) * x.size(2) * nblk, " floats), got ", scales.numel());
  check(lbw_kv_quant_fp8(x.data_ptr(), (int32_t)x.size(0), x.size(1), (int32_t)x.size(2),
                         (int32_t)x.size(3), x.stride(0), x.stride(1), x.stride(2),
                         codes.data_ptr<uint8_t>(), scales.data_ptr<float>(), LBW_FP8_BLOCK,
                         stream_of(x)),
        "lbw_kv_quant_fp8");
}

// ---- shapes for tracing (Meta / fake tensors): outputs only, no work
using OptT = std::optional<at::Tensor>;
at::Tensor attention_meta(const at::Tensor& q, at::TensorList, at::TensorList, int64_t, int64_t,
                          const OptT&, double, int64_t, bool out_fp32, const OptT&, const OptT&,
                          const OptT&) {
  return new_out(q, out_fp32);
}
at::Tensor cross_attention_meta(const at::Tensor& q, const at::Tensor&, const at::Tensor&,
                                const std::optional<at::Tensor>&, int64_t, int64_t, int64_t,
                                double, bool out_fp32) {
  return new_out(q, out_fp32);
}
at::Tensor attention_fp8kv_meta(const at::Tensor& q, at::TensorList, at::TensorList,
                                at::TensorList, at::TensorList, int64_t, int64_t, double,
                                int64_t, bool out_fp32, const OptT&, const OptT&) {
  return new_out(q, out_fp32);
}
void attention_fp8kv_out_meta(const at::Tensor&, at::TensorList, at::TensorList, at::TensorList,
                              at::TensorList, int64_t, int64_t, double, int64_t,
                              const at::Tensor&, const OptT&, const OptT&) {}
void cross_attention_out_meta(const at::Tensor&, const at::Tensor&, const at::Tensor&,
                              const OptT&, int64_t, int64_t, int64_t, double, const at::Tensor&) {}
std::tuple<at::Tensor, at::Tensor, at::Tensor> attention_partial_meta(
    const at::Tensor& q, at::TensorList, at::TensorList, int64_t, int64_t, double, const OptT&,
    const OptT&) {
  const int64_t B = q.size(0), Lq = q.size(1), H = q.size(2), D = q.size(3);
  auto f = q.options().dtype(at::kFloat);
  return {at::empty({B, H, Lq, D}, f), at::empty({B, H, Lq}, f), at::empty({B, H, Lq}, f)};
}
std::tuple<at::Tensor, at::Tensor, at::Tensor> attention_merge_partials_meta(
    at::TensorList o, at::TensorList m, at::TensorList l) {
  return {at::empty_like(o[0]), at::empty_like(m[0]), at::empty_like(l[0])};
}
at::Tensor attention_merge_meta(at::TensorList o, at::TensorList, at::TensorList) {
  return at::empty({o[0].size(0), o[0].size(2), o[0].size(1), o[0].size(3)},
                   o[0].options().dtype(at::kBFloat16));
}
void attention_out_meta(const at::Tensor&, at::TensorList, at::TensorList, int64_t, int64_t,
                        const OptT&, double, int64_t, const at::Tensor&, const OptT&,
                        const OptT&, const OptT&) {}
void attention_merge_out_meta(at::TensorList, at::TensorList, at::TensorList,
                              const at::Tensor&) {}
void qk_norm_rope_meta(const at::Tensor&, const std::optional<at::Tensor>&,
                       const std::optional<at::Tensor>&, const std::optional<at::Tensor>&,
                       const at::Tensor&, const std::optional<at::Tensor>&, const at::Tensor&,
                       at::IntArrayRef, double, int64_t, const at::Tensor&,
                       const std::optional<at::Tensor>&, const std::optional<at::Tensor>&,
                       const std::optional<at::Tensor>&, double, double, int64_t) {}
void kv_quant_fp8_meta(const at::Tensor&, const at::Tensor&, const at::Tensor&) {}

}  // namespace

TORCH_LIBRARY(lbw, m) {
  // kv_lo_dev / kv_hi_dev: one-element integer tensors on q's device (the window read on the
  // device, no host sync); they narrow the host window kv_lo / kv_hi
  // key_bias: fp32 [keys] score bias (natural log) shared by batch and heads
  m.def("attention(Tensor q, Tensor[] k, Tensor[] v, int kv_lo=0, int kv_hi=-1, "
        "Tensor? k_lens=None, float softmax_scale=0., int num_splits=0, bool out_fp32=False, "
        "Tensor? kv_lo_dev=None, Tensor? kv_hi_dev=None, Tensor? key_bias=None) -> Tensor");
  m.def("attention_out(Tensor q, Tensor[] k, Tensor[] v, int kv_lo, int kv_hi, Tensor? k_lens, "
        "float softmax_scale, int num_splits, Tensor(a!) out, Tensor? kv_lo_dev=None, "
        "Tensor? kv_hi_dev=None, Tensor? key_bias=None) -> ()");
  m.def("cross_attention(Tensor q, Tensor k, Tensor v, Tensor? k_lens=None, int n_distinct=-1, "
        "int kv_lo=0, int kv_hi=-1, float softmax_scale=0., bool out_fp32=False) -> Tensor");
  m.def("cross_attention_out(Tensor q, Tensor k, Tensor v, Tensor? k_lens, int n_distinct, "
        "int kv_lo, int kv_hi, float softmax_scale, Tensor(a!) out) -> ()");
  m.def("attention_fp8kv(Tensor q, Tensor[] k, Tensor[] v, Tensor[] k_scale, Tensor[] v_scale, "
        "int kv_lo=0, int kv_hi=-1, float softmax_scale=0., int num_splits=0, "
        "bool out_fp32=False, Tensor? kv_lo_dev=None, Tensor? kv_hi_dev=None) -> Tensor");
  m.def("attention_fp8kv_out(Tensor q, Tensor[] k, Tensor[] v, Tensor[] k_scale, "
        "Tensor[] v_scale, int kv_lo, int kv_hi, float softmax_scale, int num_splits, "
        "Tensor(a!) out, Tensor? kv_lo_dev=None, Tensor? kv_hi_dev=None) -> ()");
  m.def("attention_partial(Tensor q, Tensor[] k, Tensor[] v, int kv_lo=0, int kv_hi=-1, "
        "float softmax_scale=0., Tensor? kv_lo_dev=None, Tensor? kv_hi_dev=None) "
        "-> (Tensor, Tensor, Tensor)");
  m.def("attention_merge(Tensor[] o, Tensor[] m, Tensor[] l) -> Tensor");
  m.def("attention_merge_partials(Tensor[] o, Tensor[] m, Tensor[] l) -> (Tensor, Tensor, Tensor)");
  m.def("attention_merge_out(Tensor[] o, Tensor[] m, Tensor[] l, Tensor(a!) out) -> ()");
  m.def("qk_norm_rope_(Tensor q, Tensor? k, Tensor? bq, Tensor? bk, Tensor wq, Tensor? wk, "
        "Tensor rope, int[] rope_dims, float eps, int heads, Tensor(a!) q_out, "
        "Tensor(b!)? k_out, Tensor? v, Tensor(c!)? v_out, float q_scale, float k_scale, "
        "int layout) -> ()");
  m.def("kv_quant_fp8_(Tensor x, Tensor(a!) codes, Tensor(b!) scales) -> ()");
}

TORCH_LIBRARY_IMPL(lbw, CUDA, m) {
  m.impl("attention", &attention);
  m.impl("attention_out", &attention_out);
  m.impl("cross_attention", &cross_attention);
  m.impl("cross_attention_out", &cross_attention_out);
  m.impl("attention_fp8kv", &attention_fp8kv);
  m.impl("attention_fp8kv_out", &attention_fp8kv_out);
  m.impl("attention_partial", &attention_partial);
  m.impl("attention_merge", &attention_merge);
  m.impl("attention_merge_partials", &attention_merge_partials);
  m.impl("attention_merge_out", &attention_merge_out);
  m.impl("qk_norm_rope_", &qk_norm_rope_);
  m.impl("kv_quant_fp8_", &kv_quant_fp8_);
}

TORCH_LIBRARY_IMPL(lbw, Meta, m) {
  m.impl("attention", &attention_meta);
  m.impl("attention_out", &attention_out_meta);
  m.impl("cross_attention", &cross_attention_meta);
  m.impl("cross_attention_out", &cross_attention_out_meta);
  m.impl("attention_fp8kv", &attention_fp8kv_meta);
  m.impl("attention_fp8kv_out", &attention_fp8kv_out_meta);
  m.impl("attention_partial", &attention_partial_meta);
  m.impl("attention_merge", &attention_merge_meta);
  m.impl("attention_merge_partials", &attention_merge_partials_meta);
  m.impl("attention_merge_out", &attention_merge_out_meta);
  m.impl("qk_norm_rope_", &qk_norm_rope_meta);
  m.impl("kv_quant_fp8_", &kv_quant_fp8_meta);
}
