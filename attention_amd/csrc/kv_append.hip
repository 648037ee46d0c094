// Paged KV-cache append for MI355X (gfx950): writes one token per sequence
// into the [num_blocks, block_size, kv_heads, head_dim] caches that the
// decode kernels read.  C ABI in include/qd_attention.h.
//
// Reference semantics (paths relative to the reference tree):
//   destination (table[b, pos/P], pos % P), row of Hkv*D elements
//                                           csrc/cuda/cache/kv_append.cu:11-19
//   16-byte vector path when the row is a multiple of 16 bytes and every
//   pointer is 16-byte aligned                kv_append.cu:46-51
//   validation order and messages             kv_append.cu:32-45
//
// One wave64 per sequence: a row of K and a row of V (2*Hkv*D*s bytes) are
// copied with 16-byte loads and stores (nontemporal: neither side is reread
// by this kernel), or element by element when a row is not a multiple of 16
// bytes.  Positions and page ids are caller-owned, as in the reference; an
// entry that would address outside the table or the cache is skipped
// instead of written, so invalid metadata cannot corrupt memory.

#include <hip/hip_runtime.h>

#include <stdint.h>
#include <string.h>

#include <string>

#include "qd_attention.h"

// Records the calling thread's last failure for qd_error_string (defined
// with the decode entry points).
void qd_set_last_error(int status, const std::string& msg);

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct AppendParams {
  const char* key;
  const char* value;
  char* kc;
  char* vc;
  const int32_t* table;
  const int32_t* pos;
  int64_t row_bytes;  // Hkv * D * element size
  int elem_bytes;
  int P, maxP;
  int64_t num_blocks;
};

// Byte offset of sequence b's destination row, or -1 to skip it.
__device__ __forceinline__ int64_t dest_offset(const AppendParams& p, int b) {
  const int t = p.pos[b];
  if (t < 0 || static_cast<int64_t>(t) >= static_cast<int64_t>(p.maxP) * p.P) return -1;
  const int32_t phys = p.table[static_cast<int64_t>(b) * p.maxP + t / p.P];
  if (phys < 0 || phys >= p.num_blocks) return -1;
  return (static_cast<int64_t>(phys) * p.P + t % p.P) * p.row_bytes;
}

// grid B, block 64.
__global__ __launch_bounds__(64) void kv_append_vec16_kernel(AppendParams p) {
  const int b = blockIdx.x;
  const int64_t dst = dest_offset(p, b);
  if (dst < 0) return;
  const int64_t src = static_cast<int64_t>(b) * p.row_bytes;
  const int64_t nvec = p.row_bytes >> 4;
  for (int64_t i = threadIdx.x; i < nvec; i += 64) {
    const u32x4 kv = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.key + src) + i);
    const u32x4 vv = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.value + src) + i);
    __builtin_nontemporal_store(kv, reinterpret_cast<u32x4*>(p.kc + dst) + i);
    __builtin_nontemporal_store(vv, reinterpret_cast<u32x4*>(p.vc + dst) + i);
  }
}

// grid B, block 64; element copies (2 or 4 bytes).
template <typename T>
__global__ __launch_bounds__(64) void kv_append_elem_kernel(AppendParams p) {
  const int b = blockIdx.x;
  const int64_t dst = dest_offset(p, b);
  if (dst < 0) return;
  const int64_t src = static_cast<int64_t>(b) * p.row_bytes;
  const int64_t n = p.row_bytes / static_cast<int64_t>(sizeof(T));
  const T* ks = reinterpret_cast<const T*>(p.key + src);
  const T* vs = reinterpret_cast<const T*>(p.value + src);
  T* kd = reinterpret_cast<T*>(p.kc + dst);
  T* vd = reinterpret_cast<T*>(p.vc + dst);
  for (int64_t i = threadIdx.x; i < n; i += 64) {
    kd[i] = ks[i];
    vd[i] = vs[i];
  }
}

int append_fail(char* msg, size_t cap, const char* text) {
  qd_set_last_error(QD_ERR_INVALID_VALUE, text);
  if (msg && cap) {
    size_t n = strlen(text);
    if (n >= cap) n = cap - 1;
    memcpy(msg, text, n);
    msg[n] = '\0';
  }
  return QD_ERR_INVALID_VALUE;
}

bool same_shape(const qd_tensor_desc* a, const qd_tensor_desc* b) {
  if (a->ndim != b->ndim) return false;
  for (int i = 0; i < a->ndim && i < 8; ++i)
    if (a->sizes[i] != b->sizes[i]) return false;
  return true;
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace

extern "C" {

int qd_kv_append_validate(const qd_tensor_desc* key, const qd_tensor_desc* value,
                          const qd_tensor_desc* k_cache, const qd_tensor_desc* v_cache,
                          const qd_tensor_desc* block_table, const qd_tensor_desc* positions, char* msg,
                          size_t msg_cap) {
  const qd_tensor_desc* all[6] = {key, value, k_cache, v_cache, block_table, positions};
  for (int i = 0; i < 6; ++i)
    if (!all[i]) return append_fail(msg, msg_cap, "null tensor descriptor");
  for (int i = 0; i < 6; ++i) {
    if (!all[i]->defined || !all[i]->is_device || !all[i]->contiguous)
      return append_fail(msg, msg_cap, "all tensors must be contiguous CUDA tensors");
    if (all[i]->device_index != key->device_index)
      return append_fail(msg, msg_cap, "all tensors must share a device");
  }
  if (!(key->ndim == 3 && same_shape(value, key))) return append_fail(msg, msg_cap, "key/value must be [B, Hkv, D]");
  if (!(k_cache->ndim == 4 && same_shape(v_cache, k_cache)))
    return append_fail(msg, msg_cap, "cache must be [Nblocks, P, Hkv, D]");
  if (!(key->sizes[1] == k_cache->sizes[2] && key->sizes[2] == k_cache->sizes[3]))
    return append_fail(msg, msg_cap, "cache head shape mismatch");
  if (!(k_cache->sizes[0] > 0 && k_cache->sizes[1] > 0 && key->sizes[1] > 0 && key->sizes[2] > 0))
    return append_fail(msg, msg_cap, "invalid dimensions");
  if (!(block_table->ndim == 2 && block_table->sizes[0] == key->sizes[0] && block_table->sizes[1] > 0 &&
        positions->ndim == 1 && positions->sizes[0] == key->sizes[0]))
    return append_fail(msg, msg_cap, "invalid metadata shape");
  if (!(block_table->dtype == QD_DTYPE_I32 && positions->dtype == QD_DTYPE_I32))
    return append_fail(msg, msg_cap, "metadata must be int32");
  if (!(key->dtype == value->dtype && key->dtype == k_cache->dtype && key->dtype == v_cache->dtype))
    return append_fail(msg, msg_cap, "dtype mismatch");
  if (!(key->dtype == QD_DTYPE_F32 || key->dtype == QD_DTYPE_F16 || key->dtype == QD_DTYPE_BF16))
    return append_fail(msg, msg_cap, "unsupported dtype");
  if (msg && msg_cap) msg[0] = '\0';
  return QD_OK;
}

int qd_kv_append_launch(const void* key, const void* value, void* k_cache, void* v_cache,
                        const int32_t* block_table, const int32_t* positions, int batch, int kv_heads,
                        int head_dim, int block_size, int max_pages, int64_t num_blocks, int dtype,
                        void* stream) {
  if (batch < 0 || batch > 2147483647) return append_fail(nullptr, 0, "batch must be >= 0");
  if (kv_heads <= 0 || head_dim <= 0 || block_size <= 0 || max_pages <= 0 || num_blocks <= 0)
    return append_fail(nullptr, 0, "invalid dimensions");
  int elem = 0;
  switch (dtype) {
    case QD_DTYPE_F32: elem = 4; break;
    case QD_DTYPE_F16:
    case QD_DTYPE_BF16: elem = 2; break;
    default: return append_fail(nullptr, 0, "unsupported dtype");
  }
  if (batch == 0) return QD_OK;
  if (!key || !value || !k_cache || !v_cache || !block_table || !positions)
    return append_fail(nullptr, 0, "null tensor pointer");
  AppendParams prm;
  prm.key = static_cast<const char*>(key);
  prm.value = static_cast<const char*>(value);
  prm.kc = static_cast<char*>(k_cache);
  prm.vc = static_cast<char*>(v_cache);
  prm.table = block_table;
  prm.pos = positions;
  prm.row_bytes = static_cast<int64_t>(kv_heads) * head_dim * elem;
  prm.elem_bytes = elem;
  prm.P = block_size;
  prm.maxP = max_pages;
  prm.num_blocks = num_blocks;
  hipStream_t st = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  if (prm.row_bytes % 16 == 0 && aligned16(key) && aligned16(value) && aligned16(k_cache) && aligned16(v_cache)) {
    hipLaunchKernelGGL(kv_append_vec16_kernel, dim3(batch), dim3(64), 0, st, prm);
  } else if (elem == 4) {
    hipLaunchKernelGGL(kv_append_elem_kernel<uint32_t>, dim3(batch), dim3(64), 0, st, prm);
  } else {
    hipLaunchKernelGGL(kv_append_elem_kernel<uint16_t>, dim3(batch), dim3(64), 0, st, prm);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    qd_set_last_error(static_cast<int>(e), std::string("kv_append kernel launch failed: ") + hipGetErrorString(e));
    return static_cast<int>(e);
  }
  return QD_OK;
}

}  // extern "C"
