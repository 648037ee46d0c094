// Paged-metadata validator for MI355X (gfx950), the device-side body of
// attention.validation.validate_paged_metadata (reference
// attention/validation.py:5-39).  C ABI in include/qd_attention.h.
//
// The reference walks the batch on the host and raises the first failure in
// this order: for b = 0, 1, ...: the length (validation.py:24-25), each
// used page id (:26-28), then, when appending, the position (:30-32), its
// page id (:33-35) and a destination already taken by an earlier sequence
// (:36-38).  Here one wave per sequence evaluates the same checks in the
// same order and records (b, check, page) as a 64-bit key; the smallest
// key over the batch is exactly the failure the reference reports first.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include <string>

#include "qd_attention.h"

void qd_set_last_error(int status, const std::string& msg);

namespace {

struct ValidateParams {
  const int32_t* table;
  const int32_t* lens;
  const int32_t* pos;  // nullable
  int B, maxP, P;
  int64_t num_blocks;
  unsigned long long* result;
};

constexpr unsigned long long kNoError = ~0ull;

__device__ __forceinline__ unsigned long long make_key(int b, int check, int page) {
  return (static_cast<unsigned long long>(b) << 35) | (static_cast<unsigned long long>(check) << 32) |
         static_cast<unsigned int>(page);
}

// Destination slot of sequence j, or -1 when its position or page is invalid.
__device__ __forceinline__ int64_t destination(const ValidateParams& p, int j) {
  const int t = p.pos[j];
  if (t < 0 || static_cast<int64_t>(t) >= static_cast<int64_t>(p.maxP) * p.P) return -1;
  const int32_t page = p.table[static_cast<int64_t>(j) * p.maxP + t / p.P];
  if (page < 0 || page >= p.num_blocks) return -1;
  return static_cast<int64_t>(page) * p.P + t % p.P;
}

__global__ void init_kernel(unsigned long long* result) { *result = kNoError; }

// grid B, block 64.
__global__ __launch_bounds__(64) void validate_kernel(ValidateParams p) {
  const int b = blockIdx.x;
  const int lane = threadIdx.x;
  const int len = p.lens[b];
  int check = 0, page_idx = 0;
  if (len < 0 || static_cast<int64_t>(len) > static_cast<int64_t>(p.maxP) * p.P) {
    check = QD_META_BAD_LENGTH;
  } else {
    const int npages = (len + p.P - 1) / p.P;
    const int32_t* row = p.table + static_cast<int64_t>(b) * p.maxP;
    for (int c = 0; c < npages && check == 0; c += 64) {
      const int pg = c + lane;
      const bool bad = pg < npages && (row[pg] < 0 || row[pg] >= p.num_blocks);
      const unsigned long long m = __ballot(bad);
      if (m) {
        check = QD_META_BAD_PAGE;
        page_idx = c + __builtin_ctzll(m);
      }
    }
  }
  if (check == 0 && p.pos) {
    const int t = p.pos[b];
    if (t < 0 || static_cast<int64_t>(t) >= static_cast<int64_t>(p.maxP) * p.P) {
      check = QD_META_BAD_POSITION;
    } else {
      const int64_t mine = destination(p, b);
      if (mine < 0) {
        check = QD_META_BAD_APPEND_PAGE;
      } else {
        for (int c = 0; c < b && check == 0; c += 64) {
          const int j = c + lane;
          if (__ballot(j < b && destination(p, j) == mine)) check = QD_META_CONFLICT;
        }
      }
    }
  }
  if (check != 0 && lane == 0) atomicMin(p.result, make_key(b, check, page_idx));
}

}  // namespace

extern "C" {

int qd_validate_paged_metadata(const int32_t* block_table, const int32_t* context_lens,
                               const int32_t* positions, int batch, int max_pages, int block_size,
                               int64_t num_blocks, unsigned long long* result, void* stream) {
  if (batch < 0 || batch >= (1 << 28) || max_pages <= 0 || block_size <= 0 || num_blocks <= 0) {
    qd_set_last_error(QD_ERR_INVALID_VALUE, "block_size and num_blocks must be positive");
    return QD_ERR_INVALID_VALUE;
  }
  if (!result || (batch > 0 && (!block_table || !context_lens))) {
    qd_set_last_error(QD_ERR_INVALID_VALUE, "null pointer");
    return QD_ERR_INVALID_VALUE;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  hipLaunchKernelGGL(init_kernel, dim3(1), dim3(1), 0, st, result);
  if (batch > 0) {
    ValidateParams prm{block_table, context_lens, positions, batch, max_pages, block_size, num_blocks, result};
    hipLaunchKernelGGL(validate_kernel, dim3(batch), dim3(64), 0, st, prm);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    qd_set_last_error(static_cast<int>(e), std::string("validation kernel launch failed: ") + hipGetErrorString(e));
    return static_cast<int>(e);
  }
  return QD_OK;
}

}  // extern "C"
