// Device helpers shared by the gfx950 kernels of libqd_attention.so:
// element types, vector types, the MFMA wrappers, cross-lane reductions and
// streaming loads.  Included by the .hip sources only; everything lives in
// an anonymous namespace so each translation unit keeps its own copy.
#ifndef QD_DEVICE_H
#define QD_DEVICE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qd_attention.h"

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ----------------------------------------------------------------------------
// Element types
// ----------------------------------------------------------------------------

template <int DT>
struct Elem;
template <>
struct Elem<QD_DTYPE_F32> {
  using S = float;
  __device__ static float to_f(S x) { return x; }
  __device__ static S from_f(float x) { return x; }
};
template <>
struct Elem<QD_DTYPE_F16> {
  using S = _Float16;
  __device__ static float to_f(S x) { return static_cast<float>(x); }
  __device__ static S from_f(float x) { return static_cast<_Float16>(x); }  // RNE
};
template <>
struct Elem<QD_DTYPE_BF16> {
  using S = __bf16;
  __device__ static float to_f(S x) { return static_cast<float>(x); }
  __device__ static S from_f(float x) { return static_cast<__bf16>(x); }  // RNE
};

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ----------------------------------------------------------------------------
// Cross-lane reductions (wave64)
// ----------------------------------------------------------------------------

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum over each row of 16 lanes; every lane of the row gets the same bits.
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_f<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp_f<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp_f<0x141>(x);  // row_half_mirror
  x += dpp_f<0x140>(x);  // row_mirror
  return x;
}

__device__ __forceinline__ float wave_max(float x) {
  for (int off = 32; off >= 1; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

__device__ __forceinline__ int64_t wave_sum_i64(int64_t x) {
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

// Inclusive prefix sum over the wave's 64 lanes.
__device__ __forceinline__ int64_t wave_incl_scan_i64(int64_t x, int lane) {
  for (int off = 1; off < 64; off <<= 1) {
    const int64_t t = __shfl_up(x, off);
    if (lane >= off) x += t;
  }
  return x;
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_add_i32(int x) {
  // Lanes whose DPP source is outside the row (or whose row is masked off)
  // add the `old` operand, 0.
  return x + __builtin_amdgcn_update_dpp(0, x, CTRL, ROW_MASK, 0xF, false);
}

// Inclusive prefix sum over the wave's 64 lanes of non-negative values.
// When every lane's value is below 2^25 (the 64-lane total then fits in 31
// bits) it is a 32-bit DPP scan: row_shr 1, 2, 4, 8 within each 16-lane
// row, then row_bcast:15 (rows 1 and 3 add lane 15 of the row before) and
// row_bcast:31 (rows 2 and 3 add lane 31); otherwise the shuffle scan.
__device__ __forceinline__ int64_t wave_incl_scan_small(int64_t x, int lane) {
  if (__ballot(x >= (int64_t{1} << 25)) != 0) return wave_incl_scan_i64(x, lane);
  int y = static_cast<int>(x);
  y = dpp_add_i32<0x111, 0xF>(y);  // row_shr:1
  y = dpp_add_i32<0x112, 0xF>(y);  // row_shr:2
  y = dpp_add_i32<0x114, 0xF>(y);  // row_shr:4
  y = dpp_add_i32<0x118, 0xF>(y);  // row_shr:8
  y = dpp_add_i32<0x142, 0xA>(y);  // row_bcast:15
  y = dpp_add_i32<0x143, 0xC>(y);  // row_bcast:31
  return y;
}

// n / d for n >= 0, d > 0: a 32-bit division when both fit (the 64-bit one
// expands to several times the instructions).
__device__ __forceinline__ int64_t div_nonneg(int64_t n, int64_t d) {
  if (static_cast<uint64_t>(n) <= 0xFFFFFFFFull && static_cast<uint64_t>(d) <= 0xFFFFFFFFull)
    return static_cast<uint32_t>(n) / static_cast<uint32_t>(d);
  return n / d;
}

// Lane `src` (wave-uniform) of a 64-bit value, through v_readlane.
__device__ __forceinline__ int64_t readlane_i64(int64_t x, int src) {
  const uint64_t u = static_cast<uint64_t>(x);
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(u), src);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(u >> 32), src);
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// ----------------------------------------------------------------------------
// MFMA wrappers
// ----------------------------------------------------------------------------
//
// mma32: v_mfma_f32_16x16x32 (A 16x32, B 32x16, C 16x16).  Lane l holds
//   A row l%16, k = 8*(l/16) .. +7;  B column l%16, same k;  C column l%16,
//   rows 4*(l/16) .. +3.
// pv:    v_mfma_f32_16x16x16 (k = 4*(l/16) .. +3 per lane).

template <int DT>
struct MfmaOps;

template <>
struct MfmaOps<QD_DTYPE_BF16> {
  __device__ static f32x4 qk(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ static f32x4 mma32(u32x4 a, u32x4 b, f32x4 c) { return qk(a, b, c); }
  __device__ static f32x4 pv(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                     __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
  }
  __device__ static uint32_t pack2(float x, float y) {
    const f32x2 v = {x, y};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  }
  // Sum of the two 16-bit values packed in w, in fp32.
  __device__ static float sum2(uint32_t w) { return __uint_as_float(w << 16) + __uint_as_float(w & 0xFFFF0000u); }
  // Weights for the PV product as hi + lo: bf16 keeps 8 significant bits,
  // and a single rounding of the softmax weights (relative 2^-9 each) put
  // the output past the 16-bit bar on random inputs (the reference keeps
  // them in fp32).  lo = pack2 of what hi left out, so hi + lo holds each
  // weight to about 2^-17 and the PV product takes two MFMAs.
  static constexpr bool kSplitWeights = true;
  __device__ static uint32_t rest2(float x, float y, uint32_t hi) {
    return pack2(x - __uint_as_float(hi << 16), y - __uint_as_float(hi & 0xFFFF0000u));
  }
};

template <>
struct MfmaOps<QD_DTYPE_F16> {
  __device__ static f32x4 qk(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static f32x4 mma32(u32x4 a, u32x4 b, f32x4 c) { return qk(a, b, c); }
  __device__ static f32x4 pv(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                                 __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
  }
  __device__ static uint32_t pack2(float x, float y) {
    const f32x2 v = {x, y};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
  }
  __device__ static float sum2(uint32_t w) {
    const f32x2 v = __builtin_convertvector(__builtin_bit_cast(f16x2, w), f32x2);
    return v[0] + v[1];
  }
  // fp16 keeps 11 significant bits: one rounding of the weights stays far
  // inside the 16-bit bar (measured 0.2 of it at worst), so no split.
  static constexpr bool kSplitWeights = false;
  __device__ static uint32_t rest2(float, float, uint32_t) { return 0u; }
};

// 8x8 transpose of 16-bit elements held in one lane: in[t] holds elements
// (t, 0..7), two per 32-bit word with element 0 in the low half.  Column e
// is returned in the same packing: elements (0..7, e).  4 v_perm_b32.
__device__ __forceinline__ u32x4 transpose8x8_col_b16(const u32x4 (&in)[8], int e) {
  const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
  u32x4 out;
#pragma unroll
  for (int j = 0; j < 4; ++j) out[j] = __builtin_amdgcn_perm(in[2 * j + 1][e >> 1], in[2 * j][e >> 1], sel);
  return out;
}

// All 8 columns: out[e] = transpose8x8_col_b16(in, e).
__device__ __forceinline__ void transpose8x8_b16(const u32x4 (&in)[8], u32x4 (&out)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = transpose8x8_col_b16(in, e);
}

// ----------------------------------------------------------------------------
// Data exchanged between workgroups of one launch
// ----------------------------------------------------------------------------
//
// Each XCD of gfx950 has its own L2, and plain stores may stay dirty in the
// writer's L2 until the kernel ends.  Relaxed agent-scope atomics avoid the
// whole-L2 writeback/invalidate of an agent-scope fence: the stores carry
// sc1 (written through to the device coherence point) and the loads carry
// sc1 (never answered from a stale line in the reader's L2).  Once a wave's
// `s_waitcnt vmcnt(0)` has retired its sc1 stores, they are visible to sc1
// loads from any XCD.  8 bytes per access (two floats).

__device__ __forceinline__ void coherent_store2(float* p, float a, float b) {
  const uint64_t v = static_cast<uint64_t>(__float_as_uint(a)) | (static_cast<uint64_t>(__float_as_uint(b)) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ f32x2 coherent_load2(const float* p) {
  const uint64_t v = __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<float*>(p)), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  return f32x2{__uint_as_float(static_cast<uint32_t>(v)), __uint_as_float(static_cast<uint32_t>(v >> 32))};
}

// Buffer resource over [base, base + bytes) for raw buffer loads (word 3:
// the gfx9 raw-buffer format, 32-bit elements).  A load's address is base +
// voffset (VGPR) + soffset (SGPR) + an immediate; bytes past `bytes` read 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                           0x00020000);
}

// Cache-policy operand of the raw buffer builtins on gfx950: bit 4 = sc1.
constexpr int kBufferSc1 = 16;

// 8 bytes at base + voffset + soffset with an sc1 load (see above).
__device__ __forceinline__ f32x2 coherent_buffer_load2(__amdgpu_buffer_rsrc_t rs, uint32_t voffset, uint32_t soffset) {
  const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, voffset, soffset, kBufferSc1));
  return f32x2{__uint_as_float(v[0]), __uint_as_float(v[1])};
}

// Waits until every memory access this wave issued has completed (for sc1
// stores: reached the coherence point).
__device__ __forceinline__ void wait_memory_retired() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ----------------------------------------------------------------------------
// Streaming loads
// ----------------------------------------------------------------------------

// Caches are streamed once per call: nontemporal loads (the NT cache policy)
// keep them from displacing reusable lines and measure ~15% more read
// bandwidth than plain loads on MI355X.
__device__ __forceinline__ u32x4 stream_load16(const char* ptr) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ptr));
}

__device__ __forceinline__ u32x2 stream_load8(const char* ptr) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(ptr));
}
__device__ __forceinline__ uint32_t stream_load4(const char* ptr) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(ptr));
}

// Streaming (nontemporal) load when NT, else a plain cached load: data that
// other workgroups of the same XCD read soon after should stay in L2.
template <bool NT>
__device__ __forceinline__ u32x4 load16(const char* ptr) {
  if constexpr (NT) return stream_load16(ptr);
  else return *reinterpret_cast<const u32x4*>(ptr);
}

template <bool NT>
__device__ __forceinline__ u32x2 load8(const char* ptr) {
  if constexpr (NT) return stream_load8(ptr);
  else return *reinterpret_cast<const u32x2*>(ptr);
}

}  // namespace

#endif  // QD_DEVICE_H
