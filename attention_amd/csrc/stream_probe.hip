// Streaming-read probes for the diagnostic library (libqd_attention_diag.so,
// loaded only by bench.py --mode read): the HBM read rate the decode kernel
// could reach with its access pattern and none of its work.
//
//   probe_paged_kernel   the balanced decode kernel's loads without the
//                        math, partition or merge: W workgroups of `waves`
//                        waves; workgroup w streams pages [w*N/W,
//                        (w+1)*N/W) of a page list (a shuffled permutation of
//                        the pool), 16-token groups in order; wave j reads
//                        kv-heads j, j+waves, ... of each group (K: four 1 KiB
//                        coalesced loads, V: four 16-byte row loads per lane,
//                        head_dim 128), PF groups in flight (2 as the decode
//                        kernel, or 1-4), nontemporal 16-byte loads, a
//                        workgroup barrier every PF groups (the decode
//                        kernel's lockstep), optionally a chain of dependent
//                        multiply-adds per group in place of the decode math.
//                        With `split` 2 the waves come in two sets that take
//                        alternate groups of the range (waves = 2 * kv-head
//                        waves): twice the waves per CU for caches with few
//                        kv-heads; a set with one group fewer re-reads its
//                        last group so that both meet the same barriers.
//   probe_linear_kernel  a plain contiguous read of the same bytes (K pool
//                        then V pool), W workgroups of `waves` waves, each
//                        a contiguous 1/W share, nontemporal 16-byte loads,
//                        8 loads in flight per lane.
// Each wave folds what it read into one word (XOR) and writes it, so that
// nothing is optimized away.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qd_attention.h"
#include "qd_device.h"

namespace {

constexpr int kProbeD = 128;       // head_dim of the paged probe (16-bit elements)
constexpr int kProbeMaxWaves = 8;

struct ProbeGroup {
  u32x4 k[4];
  u32x4 v[4];
};

__device__ __forceinline__ void probe_issue(ProbeGroup& g, const char* kb, const char* vb, int64_t row_bytes,
                                            int lane) {
  // K: rows 4c + lane/16 (c = 0..3), bytes 16*(lane%16) of the kv-head slice.
#pragma unroll
  for (int c = 0; c < 4; ++c) g.k[c] = stream_load16(kb + (4 * c + lane / 16) * row_bytes + 16 * (lane % 16));
  // V: rows 4*(lane/16) + i, bytes 16*(lane%16).
#pragma unroll
  for (int i = 0; i < 4; ++i) g.v[i] = stream_load16(vb + (4 * (lane / 16) + i) * row_bytes + 16 * (lane % 16));
  __builtin_amdgcn_sched_barrier(0);
}

__device__ __forceinline__ uint32_t probe_fold(const ProbeGroup& g) {
  uint32_t x = 0;
#pragma unroll
  for (int c = 0; c < 4; ++c) x ^= g.k[c][0] ^ g.k[c][1] ^ g.k[c][2] ^ g.k[c][3];
#pragma unroll
  for (int i = 0; i < 4; ++i) x ^= g.v[i][0] ^ g.v[i][1] ^ g.v[i][2] ^ g.v[i][3];
  return x;
}

// Optional per-wave stamps (stamps != nullptr): {entry, end, XCD id} as
// s_memrealtime ticks (100 MHz) at stamps[(workgroup * waves + wave) * 4].
__device__ __forceinline__ uint64_t probe_xcc() {
  uint32_t x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  return x;
}

// A dependent chain of `n` VALU multiply-adds on the group's data, standing
// in for the decode kernel's math per group (the wave is busy, its next
// loads wait); n = 0 leaves only the XOR fold.
__device__ __forceinline__ uint32_t probe_work(uint32_t x, int n) {
  float f = __uint_as_float((x & 0x007FFFFFu) | 0x3F800000u);  // in [1, 2)
  for (int i = 0; i < n; ++i) f = fmaf(f, 0.999f, 0.001f);
  return x ^ __float_as_uint(f);
}

template <int PF>
__global__ __launch_bounds__(64 * kProbeMaxWaves) void probe_paged_kernel(const char* k, const char* v,
                                                                          const int32_t* pages, int64_t npages,
                                                                          int P, int Hkv, int waves, int work,
                                                                          int split, uint32_t* sink,
                                                                          uint64_t* stamps) {
  constexpr int kProbePf = PF;
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const uint64_t t_entry = __builtin_amdgcn_s_memrealtime();
  const int64_t W = gridDim.x;
  const int64_t p0 = blockIdx.x * npages / W;
  const int64_t p1 = (blockIdx.x + 1) * npages / W;
  const int gpp = P / 16;
  const int64_t ngroups_all = (p1 - p0) * gpp;
  const int hw = waves / split;   // waves per set
  const int par = wid / hw;       // this wave's set: groups par, par + split, ...
  const int64_t ngroups = (ngroups_all + split - 1) / split;
  const int64_t row_bytes = static_cast<int64_t>(Hkv) * kProbeD * 2;
  const bool lockstep = Hkv == hw;
  uint32_t acc = 0;
  for (int kvh = wid % hw; kvh < Hkv; kvh += hw) {
    auto base = [&](int64_t gk, const char* pool) {
      int64_t gi = gk * split + par;
      gi = gi < ngroups_all ? gi : ngroups_all - 1;
      const int64_t page = pages[p0 + gi / gpp];
      return pool + (page * P + 16 * (gi % gpp)) * row_bytes + static_cast<int64_t>(kvh) * kProbeD * 2;
    };
    ProbeGroup buf[kProbePf];
    int64_t i = 0;
#pragma unroll
    for (int u = 0; u < kProbePf - 1; ++u)
      if (u < ngroups) probe_issue(buf[u], base(u, k), base(u, v), row_bytes, lane);
    for (; i + 2 * kProbePf - 2 < ngroups; i += kProbePf) {
      if (lockstep) __builtin_amdgcn_s_barrier();
#pragma unroll
      for (int u = 0; u < kProbePf; ++u) {
        const int64_t nx = i + u + kProbePf - 1;
        probe_issue(buf[(u + kProbePf - 1) % kProbePf], base(nx, k), base(nx, v), row_bytes, lane);
        acc ^= probe_work(probe_fold(buf[u]), work);
      }
    }
    for (; i < ngroups; i += kProbePf) {
#pragma unroll
      for (int u = 0; u < kProbePf; ++u) {
        const int64_t nx = i + u + kProbePf - 1;
        if (nx < ngroups) probe_issue(buf[(u + kProbePf - 1) % kProbePf], base(nx, k), base(nx, v), row_bytes, lane);
        if (i + u < ngroups) acc ^= probe_work(probe_fold(buf[u]), work);
      }
    }
  }
  sink[static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x] = acc;
  if (stamps && lane == 0) {
    uint64_t* s = stamps + (static_cast<int64_t>(blockIdx.x) * waves + wid) * 4;
    s[0] = t_entry;
    s[1] = __builtin_amdgcn_s_memrealtime();
    s[2] = probe_xcc();
  }
}

__global__ __launch_bounds__(64 * kProbeMaxWaves) void probe_linear_kernel(const char* a, const char* b,
                                                                           int64_t bytes_each, uint32_t* sink) {
  // 16-byte words of the two buffers, one contiguous share per workgroup.
  const int64_t words = 2 * (bytes_each / 16);
  const int64_t W = gridDim.x;
  const int64_t w0 = blockIdx.x * words / W;
  const int64_t w1 = (blockIdx.x + 1) * words / W;
  const int64_t per_a = bytes_each / 16;
  constexpr int kUnroll = 8;
  uint32_t acc = 0;
  const int64_t stride = blockDim.x;
  for (int64_t x = w0 + threadIdx.x; x < w1; x += stride * kUnroll) {
    u32x4 r[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t y = x + u * stride;
      const int64_t z = y < w1 ? y : w0;
      const char* src = z < per_a ? a + 16 * z : b + 16 * (z - per_a);
      r[u] = stream_load16(src);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= r[u][0] ^ r[u][1] ^ r[u][2] ^ r[u][3];
  }
  sink[static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x] = acc;
}

}  // namespace

extern "C" {

// mode 0: probe_paged_kernel over pages[0, npages) of k and v ([N, P, Hkv,
// 128] 16-bit pools, P a multiple of 16) with `pf` (1-4) groups in flight
// per wave, `work` dependent multiply-adds per group, `split` (1 or 2,
// dividing `waves`) sets of waves on alternate groups, and per-wave
// stamps when `stamps` (wgs*waves*4 words) is not NULL; mode 1:
// probe_linear_kernel over npages*P*Hkv*128*2 bytes of each pool.  `sink`
// holds wgs*waves*64 words.  Returns 0, or a HIP error (invalid shapes:
// QD_ERR_INVALID_VALUE).
int qd_diag_stream_read(const void* k, const void* v, const int32_t* pages, int64_t npages, int P, int Hkv,
                        int wgs, int waves, int mode, int pf, int work, int split, void* sink, void* stamps,
                        void* stream) {
  if (!k || !v || !sink || npages <= 0 || P <= 0 || P % 16 != 0 || Hkv <= 0 || wgs <= 0 || waves <= 0 ||
      waves > kProbeMaxWaves || (mode == 0 && !pages) || (mode != 0 && mode != 1) || pf < 1 || pf > 4 ||
      work < 0 || work > 100000 || (split != 1 && split != 2) || waves % split != 0)
    return QD_ERR_INVALID_VALUE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  if (mode == 0) {
    auto fn = pf == 1 ? probe_paged_kernel<1> : pf == 2 ? probe_paged_kernel<2> : pf == 3 ? probe_paged_kernel<3>
                                                                                        : probe_paged_kernel<4>;
    hipLaunchKernelGGL(fn, dim3(wgs), dim3(64 * waves), 0, st, static_cast<const char*>(k),
                       static_cast<const char*>(v), pages, npages, P, Hkv, waves, work, split,
                       static_cast<uint32_t*>(sink), static_cast<uint64_t*>(stamps));
  } else {
    const int64_t bytes = npages * P * static_cast<int64_t>(Hkv) * kProbeD * 2;
    hipLaunchKernelGGL(probe_linear_kernel, dim3(wgs), dim3(64 * waves), 0, st, static_cast<const char*>(k),
                       static_cast<const char*>(v), bytes, static_cast<uint32_t*>(sink));
  }
  return static_cast<int>(hipGetLastError());
}

}  // extern "C"
