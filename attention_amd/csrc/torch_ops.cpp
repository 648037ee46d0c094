// Thin PyTorch-ROCm binding: registers the reference's `qd_attention` op
// schemas and forwards to the C ABI of libqd_attention.so.
//
// Schemas   csrc/binding/torch_ops.cpp:47-56 (reference tree)
// Impl key  CUDA (PyTorch-ROCm's key for HIP devices), as torch_ops.cpp:59-77
// Host path csrc/cuda/dense/gqa_decode.cu:96-183: validation in the
//           reference's order and words, device guard, empty_like output,
//           early return for B == 0, workspace checks, launch on the
//           current stream, launch-error check.  No host synchronization.

#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <hip/hip_runtime_api.h>
#include <torch/library.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

#include "qd_attention.h"

namespace {

int dtype_code(const at::Tensor& t) {
  switch (t.scalar_type()) {
    case at::kFloat: return QD_DTYPE_F32;
    case at::kHalf: return QD_DTYPE_F16;
    case at::kBFloat16: return QD_DTYPE_BF16;
    case at::kInt: return QD_DTYPE_I32;
    case at::kLong: return QD_DTYPE_I64;
    default: return QD_DTYPE_OTHER;
  }
}

qd_tensor_desc describe(const at::Tensor& t) {
  qd_tensor_desc d{};
  if (!t.defined()) return d;
  d.defined = 1;
  d.is_device = t.is_cuda() ? 1 : 0;
  d.device_index = t.is_cuda() ? t.get_device() : -1;
  d.contiguous = t.is_contiguous() ? 1 : 0;
  d.dtype = dtype_code(t);
  d.ndim = static_cast<int32_t>(t.dim());
  for (int64_t i = 0; i < t.dim() && i < 8; ++i) d.sizes[i] = t.size(i);
  return d;
}

// Explicit-split path (gqa_decode.cu:96-183 with splits >= 1).
at::Tensor decode_impl(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                       const at::Tensor& table, const at::Tensor& lens, double scale,
                       int64_t splits, const c10::optional<at::Tensor>& workspace) {
  const qd_tensor_desc dq = describe(q), dk = describe(k), dv = describe(v), dt = describe(table),
                       dl = describe(lens);
  char msg[256];
  int st = qd_gqa_decode_validate(&dq, &dk, &dv, &dt, &dl, scale, splits, msg, sizeof(msg));
  TORCH_CHECK(st == QD_OK, msg);

  // PyTorch-ROCm reports HIP devices as device type "cuda".
  c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  auto out = at::empty_like(q);
  if (q.size(0) == 0) return out;

  const int B = static_cast<int>(q.size(0));
  const int Hq = static_cast<int>(q.size(1));
  const int D = static_cast<int>(q.size(2));
  const int P = static_cast<int>(k.size(1));
  const int Hkv = static_cast<int>(k.size(2));
  const int maxP = static_cast<int>(table.size(1));

  at::Tensor ws;
  const int nsplit = static_cast<int>(splits);
  const int chunk = 0;
  if (workspace.has_value()) {
    const qd_tensor_desc dw = describe(*workspace);
    st = qd_gqa_decode_validate_workspace(&dq, &dw, splits, msg, sizeof(msg));
    TORCH_CHECK(st == QD_OK, msg);
    ws = *workspace;
  } else {
    if (nsplit > 1) ws = at::empty({B, Hq, nsplit, D + 2}, q.options().dtype(at::kFloat));
  }
  const size_t ws_bytes = ws.defined() ? static_cast<size_t>(ws.numel()) * sizeof(float) : 0;
  hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(q.get_device()).stream();
  st = qd_gqa_decode_launch(q.data_ptr(), k.data_ptr(), v.data_ptr(), table.data_ptr<int32_t>(),
                            lens.data_ptr<int32_t>(), out.data_ptr(),
                            ws.defined() ? ws.data_ptr<float>() : nullptr, ws_bytes, B, Hq, Hkv, D,
                            P, maxP, k.size(0), dq.dtype, static_cast<float>(scale), nsplit, chunk,
                            0, stream);
  TORCH_CHECK(st == QD_OK, qd_error_string(st));
  return out;
}

// Workspace of the automatic path for a call on `stream`.  Its first
// qd_gqa_decode_auto_counter_bytes() bytes are arrival counters that must
// be zero before first use and that every call leaves zero, so one
// workspace per (device, stream) is allocated zeroed and then reused by
// every call on that stream (calls on one stream never overlap; calls on
// different streams get different workspaces).  It grows (a new zeroed
// tensor) when a call needs more.  Under stream capture the call instead
// gets a fresh workspace from the graph's private pool, zeroed by a fill
// kernel captured with it, so every replay starts from zero counters on
// whatever stream it runs.  The map is never destroyed: its tensors must not
// be freed after the HIP runtime at process exit.
at::Tensor auto_workspace(const at::Tensor& q, size_t bytes, hipStream_t stream) {
  const int64_t n = static_cast<int64_t>(std::max<size_t>(bytes, 16));
  const auto opts = q.options().dtype(at::kByte);
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &capture) != hipSuccess) {
    (void)hipGetLastError();
    capture = hipStreamCaptureStatusNone;
  }
  if (capture != hipStreamCaptureStatusNone) return at::zeros({n}, opts);
  static std::mutex mu;
  static auto* cache = new std::map<std::pair<int, hipStream_t>, at::Tensor>();
  std::lock_guard<std::mutex> lock(mu);
  at::Tensor& ws = (*cache)[{static_cast<int>(q.get_device()), stream}];
  if (!ws.defined() || ws.numel() < n) ws = at::zeros({n}, opts);
  return ws;
}

// The reference's gqa_decode (gqa_decode.cu:186-188): same validation and
// output, body replaced by the library's automatic path (balanced MFMA
// partition or planned splits).  The workspace (auto_workspace) is kept per
// stream rather than allocated per call as the reference allocates its
// split partials (gqa_decode.cu:154), because the fused merge's counters
// must start at zero.
at::Tensor gqa_decode_hip(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                          const at::Tensor& table, const at::Tensor& lens, double scale) {
  const qd_tensor_desc dq = describe(q), dk = describe(k), dv = describe(v), dt = describe(table),
                       dl = describe(lens);
  char msg[256];
  int st = qd_gqa_decode_validate(&dq, &dk, &dv, &dt, &dl, scale, 1, msg, sizeof(msg));
  TORCH_CHECK(st == QD_OK, msg);
  c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  auto out = at::empty_like(q);
  if (q.size(0) == 0) return out;
  const int B = static_cast<int>(q.size(0));
  const int Hq = static_cast<int>(q.size(1));
  const int D = static_cast<int>(q.size(2));
  const int P = static_cast<int>(k.size(1));
  const int Hkv = static_cast<int>(k.size(2));
  const int maxP = static_cast<int>(table.size(1));
  const size_t ws_bytes = qd_gqa_decode_auto_workspace_bytes(B, Hq, Hkv, D, P, maxP, dq.dtype);
  hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(q.get_device()).stream();
  const at::Tensor ws = auto_workspace(q, ws_bytes, stream);
  st = qd_gqa_decode_auto(q.data_ptr(), k.data_ptr(), v.data_ptr(), table.data_ptr<int32_t>(),
                          lens.data_ptr<int32_t>(), out.data_ptr(), ws.data_ptr(), ws_bytes, B, Hq, Hkv, D,
                          P, maxP, k.size(0), dq.dtype, static_cast<float>(scale), stream);
  TORCH_CHECK(st == QD_OK, qd_error_string(st));
  return out;
}

at::Tensor gqa_decode_split_hip(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                const at::Tensor& table, const at::Tensor& lens, double scale,
                                int64_t splits) {
  TORCH_CHECK(splits >= 1 && splits <= 65535, "splits must be in [1, 65535]");
  return decode_impl(q, k, v, table, lens, scale, splits, c10::nullopt);
}

at::Tensor gqa_decode_split_workspace_hip(const at::Tensor& q, const at::Tensor& k,
                                          const at::Tensor& v, const at::Tensor& table,
                                          const at::Tensor& lens, double scale, int64_t splits,
                                          const at::Tensor& workspace) {
  TORCH_CHECK(splits >= 1 && splits <= 65535, "splits must be in [1, 65535]");
  return decode_impl(q, k, v, table, lens, scale, splits, workspace);
}

// kv_append (reference kv_append.cu:29-56): validation in the reference's
// order and words, device guard, B == 0 no-op, launch on the current stream.
void kv_append_hip(const at::Tensor& key, const at::Tensor& value, at::Tensor k_cache, at::Tensor v_cache,
                   const at::Tensor& table, const at::Tensor& positions) {
  const qd_tensor_desc dk = describe(key), dv = describe(value), dkc = describe(k_cache),
                       dvc = describe(v_cache), dt = describe(table), dp = describe(positions);
  char msg[256];
  int st = qd_kv_append_validate(&dk, &dv, &dkc, &dvc, &dt, &dp, msg, sizeof(msg));
  TORCH_CHECK(st == QD_OK, msg);
  c10::hip::HIPGuardMasqueradingAsCUDA guard(key.device());
  if (key.size(0) == 0) return;
  hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(key.get_device()).stream();
  st = qd_kv_append_launch(key.data_ptr(), value.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                           table.data_ptr<int32_t>(), positions.data_ptr<int32_t>(),
                           static_cast<int>(key.size(0)), static_cast<int>(key.size(1)),
                           static_cast<int>(key.size(2)), static_cast<int>(k_cache.size(1)),
                           static_cast<int>(table.size(1)), k_cache.size(0), dk.dtype, stream);
  TORCH_CHECK(st == QD_OK, qd_error_string(st));
}

// ---- Paged MLA decode (reference csrc/cuda/mla/mla.cu:138-198) ----------

at::Tensor byte_workspace(const at::Tensor& like, size_t bytes) {
  return at::empty({static_cast<int64_t>(std::max<size_t>(bytes, 16))}, like.options().dtype(at::kByte));
}

const int32_t* optional_indices(const c10::optional<at::Tensor>& indices) {
  return indices.has_value() ? indices->data_ptr<int32_t>() : nullptr;
}

// mla_project (mla.cu:138-150).
at::Tensor mla_project_hip(const at::Tensor& x, const at::Tensor& w, bool absorb) {
  const qd_tensor_desc dx = describe(x), dw = describe(w);
  char msg[256];
  int st = qd_mla_project_validate(&dx, &dw, absorb ? 1 : 0, msg, sizeof(msg));
  TORCH_CHECK(st == QD_OK, msg);
  const int64_t dout = absorb ? w.size(2) : w.size(1);
  auto out = at::empty({x.size(0), x.size(1), x.size(2), dout}, x.options());
  if (out.numel() == 0) return out;
  c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
  hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(x.get_device()).stream();
  st = qd_mla_project(x.data_ptr(), w.data_ptr(), out.data_ptr(), x.size(0) * x.size(1),
                      static_cast<int>(x.size(2)), static_cast<int>(x.size(3)), static_cast<int>(dout),
                      absorb ? 1 : 0, dx.dtype, 0, stream);
  TORCH_CHECK(st == QD_OK, qd_error_string(st));
  return out;
}

// latent_kv_write (mla.cu:151-160).
void latent_kv_write_hip(const at::Tensor& latent, const at::Tensor& rope, at::Tensor cache,
                         const at::Tensor& slots) {
  const qd_tensor_desc dl = describe(latent), dr = describe(rope), dc = describe(cache), ds = describe(slots);
  char msg[256];
  int st = qd_latent_kv_write_validate(&dl, &dr, &dc, &ds, msg, sizeof(msg));
  TORCH_CHECK(st == QD_OK, msg);
  if (!latent.size(0)) return;
  c10::hip::HIPGuardMasqueradingAsCUDA guard(latent.device());
  hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(latent.get_device()).stream();
  st = qd_latent_kv_write(latent.data_ptr(), rope.data_ptr(), cache.data_ptr(), slots.data_ptr<int64_t>(),
                          latent.size(0), static_cast<int>(latent.size(1)), static_cast<int>(rope.size(1)),
                          cache.size(0) * cache.size(1), dl.dtype, stream);
  TORCH_CHECK(st == QD_OK, qd_error_string(st));
}

// mla_attend (mla.cu:161-181).
at::Tensor mla_attend_hip(const at::Tensor& q, const at::Tensor& qr, const at::Tensor& cache,
                          const at::Tensor& table, const at::Tensor& lens, const at::Tensor& positions,
                          const c10::optional<at::Tensor>& indices, double scale, bool causal) {
  const qd_tensor_desc dq = describe(q), dr = describe(qr), dc = describe(cache), dt = describe(table),
                       dl = describe(lens), dp = describe(positions);
  const qd_tensor_desc di = indices.has_value() ? describe(*indices) : qd_tensor_desc{};
  char msg[256];
  int st = qd_mla_attend_validate(&dq, &dr, &dc, &dt, &dl, &dp, &di, scale, msg, sizeof(msg));
  TORCH_CHECK(st == QD_OK, msg);
  auto out = at::empty_like(q);
  if (q.numel() == 0) return out;
  c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  const int B = static_cast<int>(q.size(0)), T = static_cast<int>(q.size(1)), H = static_cast<int>(q.size(2));
  const int Dc = static_cast<int>(q.size(3)), Dr = static_cast<int>(qr.size(3));
  const int P = static_cast<int>(cache.size(1)), maxP = static_cast<int>(table.size(1));
  const int nk = indices.has_value() ? static_cast<int>(indices->size(2)) : -1;
  const size_t bytes = qd_mla_attend_workspace_bytes(B, T, H, Dc, Dr, P, maxP, nk, dq.dtype, 0, 0);
  at::Tensor ws;
  if (bytes > 0) ws = byte_workspace(q, bytes);
  hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(q.get_device()).stream();
  st = qd_mla_attend(q.data_ptr(), qr.data_ptr(), cache.data_ptr(), table.data_ptr<int32_t>(),
                     lens.data_ptr<int32_t>(), positions.data_ptr<int32_t>(), optional_indices(indices),
                     out.data_ptr(), ws.defined() ? ws.data_ptr() : nullptr, bytes, B, T, H, Dc, Dr, P, maxP,
                     cache.size(0), nk, causal ? 1 : 0, dq.dtype, static_cast<float>(scale), 0, 0, stream);
  TORCH_CHECK(st == QD_OK, qd_error_string(st));
  return out;
}

// mla_decode_fused (mla.cu:184-198): absorption, paged latent attention
// and value projection.
at::Tensor mla_decode_fused_hip(const at::Tensor& q, const at::Tensor& qr, const at::Tensor& cache,
                                const at::Tensor& table, const at::Tensor& lens, const at::Tensor& positions,
                                const at::Tensor& wk, const at::Tensor& wv,
                                const c10::optional<at::Tensor>& indices, double scale, bool causal) {
  const qd_tensor_desc dq = describe(q), dr = describe(qr), dc = describe(cache), dt = describe(table),
                       dl = describe(lens), dp = describe(positions), dk = describe(wk), dv = describe(wv);
  const qd_tensor_desc di = indices.has_value() ? describe(*indices) : qd_tensor_desc{};
  char msg[256];
  int st = qd_mla_decode_validate(&dq, &dr, &dc, &dt, &dl, &dp, &dk, &dv, &di, scale, msg, sizeof(msg));
  TORCH_CHECK(st == QD_OK, msg);
  auto out = at::empty({q.size(0), q.size(1), q.size(2), wv.size(1)}, q.options());
  if (!out.numel()) return out;
  c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  const int B = static_cast<int>(q.size(0)), T = static_cast<int>(q.size(1)), H = static_cast<int>(q.size(2));
  const int Dn = static_cast<int>(q.size(3)), Dc = static_cast<int>(wk.size(2)), Dr = static_cast<int>(qr.size(3));
  const int Dv = static_cast<int>(wv.size(1));
  const int P = static_cast<int>(cache.size(1)), maxP = static_cast<int>(table.size(1));
  const int nk = indices.has_value() ? static_cast<int>(indices->size(2)) : -1;
  const size_t bytes = qd_mla_decode_workspace_bytes(B, T, H, Dc, Dr, P, maxP, nk, dq.dtype, 0, 0);
  const at::Tensor ws = byte_workspace(q, bytes);
  hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(q.get_device()).stream();
  st = qd_mla_decode(q.data_ptr(), qr.data_ptr(), cache.data_ptr(), table.data_ptr<int32_t>(),
                     lens.data_ptr<int32_t>(), positions.data_ptr<int32_t>(), wk.data_ptr(), wv.data_ptr(),
                     optional_indices(indices), out.data_ptr(), ws.data_ptr(), bytes, B, T, H, Dn, Dc, Dr, Dv,
                     P, maxP, cache.size(0), nk, causal ? 1 : 0, dq.dtype, static_cast<float>(scale), 0, 0,
                     stream);
  TORCH_CHECK(st == QD_OK, qd_error_string(st));
  return out;
}

}  // namespace

TORCH_LIBRARY(qd_attention, m) {
  m.def(
      "mla_decode_fused(Tensor q, Tensor qr, Tensor cache, Tensor table, Tensor lens, Tensor positions, "
      "Tensor wk, Tensor wv, Tensor? indices, float scale, bool causal) -> Tensor");
  m.def("mla_project(Tensor x, Tensor weight, bool absorb) -> Tensor");
  m.def("latent_kv_write(Tensor latent, Tensor rope, Tensor(a!) cache, Tensor slots) -> ()");
  m.def(
      "mla_attend(Tensor q, Tensor q_rope, Tensor cache, Tensor table, Tensor lens, Tensor positions, "
      "Tensor? indices, float scale, bool causal) -> Tensor");
  m.def(
      "kv_append(Tensor key, Tensor value, Tensor(a!) k_cache, Tensor(b!) v_cache, Tensor block_table, "
      "Tensor positions) -> ()");
  m.def(
      "gqa_decode_split_workspace(Tensor q, Tensor k, Tensor v, Tensor table, Tensor lengths, "
      "float scale, int splits, Tensor(a!) workspace) -> Tensor");
  m.def(
      "gqa_decode_split(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_table, "
      "Tensor context_lens, float scale, int splits) -> Tensor");
  m.def(
      "gqa_decode(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_table, "
      "Tensor context_lens, float scale) -> Tensor");
}

TORCH_LIBRARY_IMPL(qd_attention, CUDA, m) {
  m.impl("mla_decode_fused", TORCH_FN(mla_decode_fused_hip));
  m.impl("mla_project", TORCH_FN(mla_project_hip));
  m.impl("latent_kv_write", TORCH_FN(latent_kv_write_hip));
  m.impl("mla_attend", TORCH_FN(mla_attend_hip));
  m.impl("kv_append", TORCH_FN(kv_append_hip));
  m.impl("gqa_decode_split_workspace", TORCH_FN(gqa_decode_split_workspace_hip));
  m.impl("gqa_decode_split", TORCH_FN(gqa_decode_split_hip));
  m.impl("gqa_decode", TORCH_FN(gqa_decode_hip));
}
