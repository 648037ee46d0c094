// Thin PyTorch-ROCm binding: registers the reference's `qd_attention` op
// schemas and forwards to the C ABI of libqd_attention.so.
//
// Schemas   csrc/binding/torch_ops.cpp:52-56 (reference tree)
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

// The automatic path's workspace, one per (device, stream), kept for the
// life of the process like a BLAS handle's workspace.  It is zero-filled on
// the stream when created or grown (the library needs its control region
// zero on entry and leaves it zero), so only the first call on a stream, or
// one that needs a larger workspace, pays for an allocation and a fill.
// Calls on one stream run in order and share it; calls on different
// streams never share one.
at::Tensor stream_workspace(const at::Tensor& like, hipStream_t stream, size_t bytes) {
  static std::mutex mu;
  // Never destroyed: tensors must not be freed after the allocator is gone
  // at process exit.
  static auto* cache = new std::map<std::pair<int, hipStream_t>, at::Tensor>();
  const std::pair<int, hipStream_t> key{like.get_device(), stream};
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache->find(key);
  if (it != cache->end() && static_cast<size_t>(it->second.numel()) >= bytes) return it->second;
  at::Tensor ws = at::zeros({static_cast<int64_t>(std::max<size_t>(bytes, 256))},
                            like.options().dtype(at::kByte));
  (*cache)[key] = ws;
  return ws;
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

// The reference's gqa_decode (gqa_decode.cu:186-188): same validation and
// output, body replaced by the library's automatic path (balanced MFMA
// partition or planned splits), with a per-call workspace from the caching
// allocator.
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
  const at::Tensor ws = stream_workspace(q, stream, ws_bytes);
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

}  // namespace

TORCH_LIBRARY(qd_attention, m) {
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
  m.impl("kv_append", TORCH_FN(kv_append_hip));
  m.impl("gqa_decode_split_workspace", TORCH_FN(gqa_decode_split_workspace_hip));
  m.impl("gqa_decode_split", TORCH_FN(gqa_decode_split_hip));
  m.impl("gqa_decode", TORCH_FN(gqa_decode_hip));
}
