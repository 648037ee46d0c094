// Paged MLA (multi-head latent attention) decode for MI355X (gfx950).
// C ABI in include/qd_attention.h.
//
// Reference operators replaced (paths relative to the reference tree):
//   latent_kv_write   csrc/cuda/mla/mla.cu:28-32 (write_cache), :151-160
//   mla_project       csrc/cuda/mla/mla.cu:16-27 (projection), :138-150
//   mla_attend        csrc/cuda/mla/mla.cu:34-82 (attend, attend_split,
//                     attend_merge), :161-181
//   mla_decode_fused  csrc/cuda/mla/mla.cu:86-134 (fused_decode, fused_split,
//                     fused_split_merge), :184-198
//
// Layouts: cache [N, P, W] with W = Dc + Dr (latent | rope), q / out
// [B, T, H, Dc], q_rope [B, T, H, Dr], table [B, maxP], lengths [B],
// positions [B, T], indices [B, T, K] (logical token ids, -1 = none).
//
// Design.  All H heads of a query row read the same latent row, so the
// attention is one shared K/V stream per row: a workgroup stages 32-token
// tiles of whole cache rows in LDS (each row read from HBM once per
// workgroup) and each of its waves runs 16 heads on the matrix cores:
//   S^T[32 tok x 16 heads] = C[32 x W] . [q | q_rope]^T   v_mfma 16x16x32
//   O^T[Dc x 16 heads]    += C[:, :Dc]^T . P^T            v_mfma 16x16x32
// with the fp32 online softmax per lane (one head per lane column).  A
// context can be split over workgroups; partials {m, l, acc[Dc]} are merged
// with the reference's log-sum-exp rule.  The query absorption and value
// projection are per-head GEMMs over all rows of the batch, so the weights
// are read once per call rather than once per row as in the reference's
// fused kernels; the rounding points (absorbed query, latent output, final
// output, each rounded to the input dtype) are the reference's.

#include <hip/hip_runtime.h>


#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <type_traits>
#include <string>

#include "qd_attention.h"
#include "qd_device.h"

// Records the calling thread's last failure for qd_error_string (defined
// with the decode entry points).
void qd_set_last_error(int status, const std::string& msg);

namespace {

constexpr int kTileTokens = 32;
constexpr int kAttendThreads = 256;  // 4 waves: up to 64 heads, all load
constexpr int kMaxSplits = 64;

// ----------------------------------------------------------------------------
// latent_kv_write
// ----------------------------------------------------------------------------

struct LatentWriteParams {
  const char* latent;
  const char* rope;
  char* cache;
  const int64_t* slots;
  int64_t lat_bytes, rope_bytes, row_bytes;
  int64_t rows;  // Nblocks * P
};

// grid n, block 64: row t -> cache row slots[t] (skipped when out of range).
__global__ __launch_bounds__(64) void latent_write_vec16_kernel(LatentWriteParams p) {
  const int64_t t = blockIdx.x;
  const int64_t s = p.slots[t];
  if (s < 0 || s >= p.rows) return;
  char* dst = p.cache + s * p.row_bytes;
  const char* la = p.latent + t * p.lat_bytes;
  const char* ro = p.rope + t * p.rope_bytes;
  const int64_t nl = p.lat_bytes >> 4, nr = p.rope_bytes >> 4;
  for (int64_t i = threadIdx.x; i < nl + nr; i += 64) {
    const u32x4 v = i < nl ? *reinterpret_cast<const u32x4*>(la + 16 * i)
                           : *reinterpret_cast<const u32x4*>(ro + 16 * (i - nl));
    *reinterpret_cast<u32x4*>(dst + 16 * i) = v;
  }
}

template <typename E>
__global__ __launch_bounds__(64) void latent_write_elem_kernel(LatentWriteParams p) {
  const int64_t t = blockIdx.x;
  const int64_t s = p.slots[t];
  if (s < 0 || s >= p.rows) return;
  const int64_t nl = p.lat_bytes / static_cast<int64_t>(sizeof(E));
  const int64_t nr = p.rope_bytes / static_cast<int64_t>(sizeof(E));
  E* dst = reinterpret_cast<E*>(p.cache + s * p.row_bytes);
  const E* la = reinterpret_cast<const E*>(p.latent + t * p.lat_bytes);
  const E* ro = reinterpret_cast<const E*>(p.rope + t * p.rope_bytes);
  for (int64_t i = threadIdx.x; i < nl + nr; i += 64) dst[i] = i < nl ? la[i] : ro[i - nl];
}

// ----------------------------------------------------------------------------
// Per-head projection (query absorption / value up-projection)
// ----------------------------------------------------------------------------
//
// out[r, h, o] = sum_k x[r, h, k] * W_h(k, o) over rows r = (b, t), with
//   absorb: W_h(k, o) = w[h, k, o]   (w [H, Dn, Dc], k = Dn, o = Dc)
//   value:  W_h(k, o) = w[h, o, k]   (w [H, Dv, Dc], k = Dc, o = Dv)
// fp32 accumulation, one rounding to the dtype (mla.cu:21-26).

// Half-precision partial rows (shared-tile and wave kernels): {m, l, s0, s1,
// s2, s3, 0, 0} in fp32, then Dc = 512 fp16 values acc / s_k for latent
// columns [128 k, 128 k + 128), s_k the block's largest |acc| for the head.
constexpr int kHalfHeader = 8;                         // floats before the fp16 values
constexpr int kHalfPst = kHalfHeader + 512 / 2;        // floats per partial row

// One step of the log-sum-exp fold of partial rows (online_softmax.cuh:17-24)
// as every merge here runs it: state (M, L, acc[N]) absorbs the partial
// (ms, ls, v[N]).  Shared so that a merge inside another kernel rounds
// exactly as the merge kernel does.
template <int N>
__device__ __forceinline__ void lse_fold(float& M, float& L, float (&acc)[N], float ms, float ls, const float (&v)[N]) {
  const float mn = fmaxf(M, ms);
  const float a = L == 0.f ? 0.f : fast_exp2((M - mn) * kLog2e);
  const float bw = fast_exp2((ms - mn) * kLog2e);
  // Explicit fused multiply-adds: the same rounding whichever kernel inlines it.
  L = __builtin_fmaf(a, L, bw * ls);
#pragma unroll
  for (int j = 0; j < N; ++j) acc[j] = __builtin_fmaf(a, acc[j], bw * v[j]);
  M = mn;
}

struct ProjParams {
  const void* x;
  const void* w;
  void* out;
  int64_t rows;
  int H, di, dout;
  // Value projection with the merge of split attention rows folded in
  // (MERGE): the half-precision partials, their row spans and tile count.
  const float* part = nullptr;
  const int* meta = nullptr;
  const int64_t* gtotal = nullptr;
  int wgs = 0;
};

// grid (ceil(dout/128), H, ceil(rows/(16 RT))), block 256.  The workgroup
// owns 128 output columns of one head for 16*RT rows; its 4 waves split the
// k range (groups of PAIR 32-wide chunks: wave v takes chunks PAIR*v ..
// PAIR*v + PAIR-1, then the same plus 4*PAIR, ..., all loads of a group in
// flight together) and their partial tiles are summed in LDS.  A wave covers
// 16*RT rows x 128 columns: RT row tiles x 8 column tiles of
// v_mfma_f32_16x16x32, column tile e holding columns base + 8*(l%16) + e, so
// the absorb layout (columns contiguous in memory) is turned into the B
// operand by an 8x8 in-register transpose and the value layout (k
// contiguous) is loaded as is.  Small batches take RT = 1 (four times the
// workgroups; the per-head weights are then re-read from L2) and, for a long
// k range, PAIR = 4 (one round trip for a wave's loads).
//
// MERGE (value projection of mla_decode, RT = 1, di = 512): the x rows of
// attention rows split across workgroups are merged here from their
// half-precision partials (lse_fold in the merge kernel's order, rounded to
// the input dtype as the merge kernel rounds them) into an LDS tile, the
// other rows copied there from x.  (Issuing the first weight loads before
// the merge measured no faster and held 128 more registers.)
//
// HC (value layout): half-width column tiles, so that small grids cover
// every CU: workgroup x serves column blocks e = 4 (x % 2) .. + 3 of tile
// x / 2 (columns 128 (x / 2) + 8 n + e).
template <int DT, bool ABSORB, int RT, int PAIR, bool MERGE = false, bool HC = false>
__global__ __launch_bounds__(256) void mla_project_mfma_kernel(ProjParams p) {
  using E = Elem<DT>;
  using Ops = MfmaOps<DT>;
  using S = typename E::S;
  constexpr int kPair = PAIR;
  constexpr int NE = HC ? 4 : 8;  // MFMA column blocks per workgroup
  static_assert(!MERGE || (!ABSORB && RT == 1), "the merged input serves the value projection's 16-row tiles");
  static_assert(!HC || !ABSORB, "half-width tiles serve the value layout");
  constexpr int kXtStride = 512 + 8;  // merged tile row (elements): 16 bytes of padding, no bank conflicts
  __shared__ f32x4 red[4][8][64];
  __shared__ __align__(16) S stage[16][128];
  __shared__ __align__(16) S xt[MERGE ? 16 : 1][MERGE ? kXtStride : 8];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int r16 = lane & 15, q4 = lane >> 4;
  const int h = blockIdx.y;
  const int cbase = 128 * static_cast<int>(HC ? blockIdx.x >> 1 : blockIdx.x);
  const int e0 = HC ? 4 * static_cast<int>(blockIdx.x & 1) : 0;
  const int64_t r0 = 16 * RT * static_cast<int64_t>(blockIdx.z);
  const int col = min(cbase + 8 * r16, p.dout - 8);  // clamped load column
  const int nch = p.di / 32;
  const char* xb = static_cast<const char*>(p.x);
  const char* wb = static_cast<const char*>(p.w);
  S* out = static_cast<S*>(p.out);
  f32x4 acc[RT][NE];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int e = 0; e < NE; ++e) acc[rt][e] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto load_w = [&](int c, u32x4 (&bop)[NE]) {
    const int k0 = 32 * c + 8 * q4;
    if constexpr (ABSORB) {
      u32x4 raw[8];
#pragma unroll
      for (int t = 0; t < 8; ++t)
        raw[t] = *reinterpret_cast<const u32x4*>(wb + ((static_cast<int64_t>(h) * p.di + k0 + t) * p.dout + col) * 2);
      transpose8x8_b16(raw, bop);
    } else {
#pragma unroll
      for (int e = 0; e < NE; ++e)
        bop[e] = *reinterpret_cast<const u32x4*>(wb + ((static_cast<int64_t>(h) * p.dout + col + e0 + e) * p.di + k0) * 2);
    }
  };
  if constexpr (MERGE) {
    // Thread (row, seg) builds columns 32 seg .. 32 seg + 31 of tile row `row`.
    const int row = static_cast<int>(threadIdx.x) >> 4, seg = static_cast<int>(threadIdx.x) & 15;
    int64_t rr = r0 + row;
    if (rr >= p.rows) rr = p.rows - 1;
    const int first = p.meta[2 * rr], nwg = p.meta[2 * rr + 1];
    u32x4 v16[4];
    if (nwg < 2 || first < 0 || first + nwg > p.wgs) {
      // Written whole by the attention kernel (or zero-filled): as stored.
#pragma unroll
      for (int i = 0; i < 4; ++i)
        v16[i] = *reinterpret_cast<const u32x4*>(xb + ((rr * p.H + h) * p.di + 32 * seg + 8 * i) * 2);
    } else {
      const int64_t G = *p.gtotal;
      // Workgroup k's range [k G / wgs, (k + 1) G / wgs) holds a partial row
      // when it is not empty, which it never is for G >= wgs (skips two
      // 64-bit divisions per slot and lane).
      const bool dense = G >= p.wgs;
      auto present = [&](int k) {
        return dense || static_cast<int64_t>(k) * G / p.wgs != static_cast<int64_t>(k + 1) * G / p.wgs;
      };
      const int64_t stride = static_cast<int64_t>(p.H) * kHalfPst;
      const float* base = p.part + (rr * p.H + h) * static_cast<int64_t>(kHalfPst);
      constexpr int kBatch = 8;
      float M = -INFINITY, L = 0.f, am[32];
#pragma unroll
      for (int j = 0; j < 32; ++j) am[j] = 0.f;
      for (int c = 0; c < nwg; c += kBatch) {
        float ms[kBatch], ls[kBatch], sc[kBatch];
        f16x8 hv[kBatch][4];
#pragma unroll
        for (int t = 0; t < kBatch; ++t) {
          ms[t] = -INFINITY;
          ls[t] = 0.f;
          sc[t] = 0.f;
          const int k = first + c + t;
          if (c + t < nwg && present(k)) {
            const float* pr = base + k * stride;
            const f32x4 hd = *reinterpret_cast<const f32x4*>(pr);
            const f32x4 hs = *reinterpret_cast<const f32x4*>(pr + 4);
            ms[t] = hd[0];
            ls[t] = hd[1];
            const int kb = seg >> 2;  // 128-column block
            sc[t] = kb == 0 ? hd[2] : kb == 1 ? hd[3] : kb == 2 ? hs[0] : hs[1];
#pragma unroll
            for (int i = 0; i < 4; ++i)
              hv[t][i] = *reinterpret_cast<const f16x8*>(reinterpret_cast<const char*>(pr + kHalfHeader) + 64 * seg + 16 * i);
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) hv[t][i] = f16x8{};
          }
        }
#pragma unroll
        for (int t = 0; t < kBatch; ++t) {
          if (ls[t] == 0.f) continue;  // absent or empty partial
          float v[32];
#pragma unroll
          for (int j = 0; j < 32; ++j) v[j] = static_cast<float>(hv[t][j / 8][j % 8]) * sc[t];
          lse_fold(M, L, am, ms[t], ls[t], v);
        }
      }
      const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        S o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = E::from_f(am[8 * i + j] * inv);
        v16[i] = __builtin_bit_cast(u32x4, o);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(&xt[row][32 * seg + 8 * i]) = v16[i];
    __syncthreads();
  }
  for (int c0 = kPair * wv; c0 < nch; c0 += 4 * kPair) {
    u32x4 bop[kPair][NE], a[kPair][RT];
#pragma unroll
    for (int u = 0; u < kPair; ++u) {
      const int c = min(c0 + u, nch - 1);  // a missing second chunk repeats the first, weight 0 below
      const int k0 = 32 * c + 8 * q4;
      load_w(c, bop[u]);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        if constexpr (MERGE) {
          a[u][rt] = *reinterpret_cast<const u32x4*>(&xt[r16][k0]);
        } else {
          int64_t row = r0 + 16 * rt + r16;
          if (row >= p.rows) row = p.rows - 1;
          a[u][rt] = *reinterpret_cast<const u32x4*>(xb + ((row * p.H + h) * p.di + k0) * 2);
        }
      }
      if (c0 + u >= nch) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) a[u][rt] = u32x4{0u, 0u, 0u, 0u};
      }
    }
    // Every load of the group is issued before the first MFMA: left free,
    // the scheduler sank each load next to its MFMA with a full wait between
    // them, one memory round trip per MFMA.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kPair; ++u)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int e = 0; e < NE; ++e) acc[rt][e] = Ops::mma32(a[u][rt], bop[u][e], acc[rt][e]);
  }
  // The 4 waves' partial tiles are summed through LDS and the 16 x 128 output
  // tile is staged there as well, so that each lane writes 16 contiguous
  // bytes (8 columns of one row) instead of 8 scattered 2-byte stores.
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
    for (int e = 0; e < NE; ++e) red[wv][e][lane] = acc[rt][e];
    __syncthreads();
#pragma unroll
    for (int ee = 0; ee < NE / 4; ++ee) {
      const int e = (NE / 4) * wv + ee;
      const f32x4 s = red[0][e][lane] + red[1][e][lane] + red[2][e][lane] + red[3][e][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) stage[4 * q4 + i][8 * r16 + e0 + e] = E::from_f(s[i]);
    }
    __syncthreads();
    {
      const int orow = static_cast<int>(threadIdx.x) >> 4;  // 0..15
      const int oc = 8 * (static_cast<int>(threadIdx.x) & 15);
      const int64_t row = r0 + 16 * rt + orow;
      if (row < p.rows && cbase + oc < p.dout) {  // dout % 8 == 0: whole 8-column groups
        if constexpr (HC)
          *reinterpret_cast<u32x2*>(out + (row * p.H + h) * p.dout + cbase + oc + e0) =
              *reinterpret_cast<const u32x2*>(&stage[orow][oc + e0]);
        else
          *reinterpret_cast<u32x4*>(out + (row * p.H + h) * p.dout + cbase + oc) =
              *reinterpret_cast<const u32x4*>(&stage[orow][oc]);
      }
    }
    __syncthreads();
  }
}

// Any dtype/shape: one thread per output element, k summed in order (the
// reference's loop, mla.cu:18-26).
template <int DT, bool ABSORB>
__global__ __launch_bounds__(256) void mla_project_generic_kernel(ProjParams p) {
  using E = Elem<DT>;
  using S = typename E::S;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= p.rows * p.H * p.dout) return;
  const int o = static_cast<int>(i % p.dout);
  const int h = static_cast<int>((i / p.dout) % p.H);
  const int64_t r = i / (static_cast<int64_t>(p.H) * p.dout);
  const S* x = static_cast<const S*>(p.x) + (r * p.H + h) * p.di;
  const S* w = static_cast<const S*>(p.w);
  float sum = 0.f;
  for (int k = 0; k < p.di; ++k) {
    const int64_t wi = ABSORB ? (static_cast<int64_t>(h) * p.di + k) * p.dout + o
                              : (static_cast<int64_t>(h) * p.dout + o) * p.di + k;
    sum = fmaf(E::to_f(x[k]), E::to_f(w[wi]), sum);
  }
  static_cast<S*>(p.out)[i] = E::from_f(sum);
}

// ----------------------------------------------------------------------------
// Paged latent attention
// ----------------------------------------------------------------------------

struct MlaParams {
  const void* q;    // [R, H, Dc]
  const void* qr;   // [R, H, Dr]
  const void* cache;
  const int32_t* table;
  const int32_t* lens;
  const int32_t* pos;  // [R]
  const int32_t* idx;  // [R, nk] when nk >= 0
  void* out;           // [R, H, Dc]
  float* part;         // VALU kernel: [R, H, splits, Dc + 2] (splits > 1);
                       // MFMA kernel: [wgs + R, H, pst] stream-K partials
  int B, T, H, Dc, Dr, W, P, maxP;
  int nk;  // indices per row, -1 = all tokens (dense)
  int causal, splits;
  int head_groups;  // MFMA kernel: head groups (workgroups per tile range)
  int kch;          // MFMA kernel: ceil(W / 32)
  int nht, ds;      // MFMA kernel: head tiles per workgroup, latent slices per head tile
  int wgs;          // MFMA kernel: workgroups per head group (stream-K ranges)
  int* meta;        // MFMA kernel: [rows][2] {first workgroup, workgroups} per row
  int pst;          // MFMA kernel: floats per partial row: {m, l, acc[Dc]} fp32, or (shared-tile
                    // and wave kernels) kHalfHeader floats + Dc fp16 (kHalfPst)
  int64_t* gtotal;  // MFMA kernel: tiles G of the batch (merge: skips empty ranges)
  int64_t num_blocks;
  float sl2;        // scale * log2(e)
#ifdef QD_STAMPS
  uint64_t* stamps;  // diagnostic build: per-wave timestamps of the shared-tile kernel (mla_stamp)
#endif
};

#ifdef QD_STAMPS
// Diagnostic build only (-DQD_STAMPS): 16 words per wave of
// mla_attend_shared_kernel at stamps[(block * 4 + wave) * 16]: s_memrealtime
// (100 MHz) at entry [0], after the prologue [1], when the loop starts (first
// tile and query landed) [2], after the last tile [3], at the end [4]; the XCD
// id [5]; tiles of the range [6]; shader clocks (s_memtime) spent in row ends
// [7]; s_memtime at entry [8] and after the last tile [9]; the workgroup's
// range [10] and head group [11]; row ends [12].  Only workgroups with tiles
// write.
__device__ __forceinline__ void mla_stamp(const MlaParams& p, int slot, uint64_t value) {
  if (p.stamps && (threadIdx.x & 63) == 0)
    p.stamps[(static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * 16 + slot] = value;
}
__device__ __forceinline__ uint64_t mla_xcc() {
  uint32_t x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  return x;
}
#define QD_MLA_STAMP(slot, value) mla_stamp(p, (slot), (value))
#define QD_MLA_STAMPS_ON 1
#else
#define QD_MLA_STAMP(slot, value) ((void)0)
#define QD_MLA_STAMPS_ON 0
#endif

// Scale s of a half-precision partial block: the values are stored as o / s
// in fp16.  s is the block's largest |o|, clamped up to the smallest normal
// float when it is below it (1 / s must stay finite: a subnormal s would
// overflow 1 / s to inf, and a zero column then stores 0 * inf = NaN), and 1
// for an all-zero block.
__device__ __forceinline__ float half_partial_scale(float amax) {
  return amax >= __FLT_MIN__ ? amax : (amax > 0.f ? __FLT_MIN__ : 1.f);
}

// Two floats as fp16, round to nearest even, lo in the low half.
__device__ __forceinline__ uint32_t pack_f16_rne(float lo, float hi) {
  const f16x2 v = __builtin_convertvector(f32x2{lo, hi}, f16x2);
  return __builtin_bit_cast(uint32_t, v);
}

// Visible prefix of query row r (mla.cu:37), clamped to the table capacity
// so that a length beyond the table never reads past the table row.
__device__ __forceinline__ int row_end(const MlaParams& p, int b, int64_t r) {
  const int64_t cap = static_cast<int64_t>(p.maxP) * p.P;
  int64_t end = p.lens[b];
  if (p.causal) {
    const int64_t lim = static_cast<int64_t>(p.pos[r]) + 1;
    end = min(end, max(static_cast<int64_t>(0), lim));
  }
  end = min(end, cap);
  return end > 0 ? static_cast<int>(end) : 0;
}

// Token list positions [i0, i1) of split s over `count` entries (mla.cu:60).
__device__ __forceinline__ void split_range(int count, int s, int splits, int& i0, int& i1) {
  i0 = static_cast<int>(static_cast<int64_t>(count) * s / splits);
  i1 = static_cast<int>(static_cast<int64_t>(count) * (s + 1) / splits);
}

// Element offset of logical token `tok` of sequence b (mla.cu:45-46);
// out-of-range page ids are clamped so every access stays in the cache.
__device__ __forceinline__ int64_t token_offset(const MlaParams& p, int b, int tok) {
  int32_t phys = p.table[static_cast<int64_t>(b) * p.maxP + tok / p.P];
  if (phys < 0) phys = 0;
  if (phys >= p.num_blocks) phys = static_cast<int32_t>(p.num_blocks - 1);
  return (static_cast<int64_t>(phys) * p.P + tok % p.P) * p.W;
}

// Stores a row's result: the normalized output (splits == 1) or the
// partial {m (natural-log units), l, acc[Dc]} (mla.cu:71-73).
__device__ __forceinline__ float* partial_row(const MlaParams& p, int64_t r, int h, int s) {
  return p.part + ((r * p.H + h) * p.splits + s) * static_cast<int64_t>(p.Dc + 2);
}

// Max over the 4 lanes l % 16 == const (lanes l, l^16, l^32, l^48) with
// gfx950's v_permlane32_swap / v_permlane16_swap: swapping a register with
// itself leaves the lane's value and its partner's (l^32, resp. l^16) in the
// returned pair.  No LDS round trip, unlike ds_bpermute.
__device__ __forceinline__ float max_over_lane_groups(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Sum over the same 4 lanes; every lane gets the same bits (each step adds
// a pair, and the pair's order does not change a sum).
__device__ __forceinline__ float sum_over_lane_groups(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Workgroup barrier for LDS traffic only: waits for this wave's LDS
// operations, not for its outstanding loads (the staged tiles keep
// flowing; __syncthreads() would wait for every load, vmcnt(0)).  The empty
// asm statements keep the compiler from moving memory accesses across.
__device__ __forceinline__ void lds_barrier() {
  constexpr int imm = 0x3F | (0x3 << 14) | (0x7 << 4) | (0x0 << 8);  // vmcnt max, lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(imm);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Tiles in flight ahead of the one being computed, staged in registers
// (CPT u32x4 per thread per tile): as deep as the register file allows for
// the wave layout (4 slices of one head tile, or 2 x 2).
__host__ __device__ constexpr int stage_depth(int cpt, int ds) {
  return ds == 4 ? (cpt <= 5 ? 6 : 4) : (cpt <= 5 ? 4 : 3);
}
constexpr int kRingTiles = 2;   // LDS tile buffers: the tile being computed and the next
constexpr int kMetaSlots = 8;   // per-tile metadata slots (>= stage depth + 2)
constexpr int kWinPages = 256;  // page-table window (dense rows)
constexpr int kFlagFirst = 1;   // first tile of a row segment in this workgroup
constexpr int kFlagLast = 2;    // last tile of a row segment in this workgroup
constexpr int kFlagWhole = 4;   // (with kFlagLast) the segment is the whole row

__host__ __device__ constexpr size_t mla_mfma_lds_bytes(int cpt) {
  return static_cast<size_t>(kRingTiles) * cpt * 4096  // tile ring
         + kMetaSlots * kTileTokens * 8                 // row offsets
         + kMetaSlots * 8 * 2                           // tile rows, tile bases
         + kMetaSlots * 4 * 2                           // masks, flags
         + kWinPages * 4                                // page window
         + 32                                           // prologue results
         + kAttendThreads * 32                          // score exchange
         + 1024;                                        // slack
}

// Tiles of 32 listed tokens of query row r (dense: the visible prefix).
__device__ __forceinline__ int row_tiles(const MlaParams& p, int64_t r) {
  const int count = p.nk >= 0 ? p.nk : row_end(p, static_cast<int>(r / p.T), r);
  return (count + kTileTokens - 1) / kTileTokens;
}

// MFMA kernel, stream-K.  The (query row, 32-token tile) space of the batch
// (G tiles) is cut into p.wgs equal ranges; workgroup w of head group g
// processes tiles [w*G/wgs, (w+1)*G/wgs) for heads 16*nht*g .. +16*nht.  A
// row whose tiles all fall in one workgroup is written directly; a row split
// across workgroups leaves {m, l, acc} partials in slot (w + row) and the
// merge kernel folds them, guided by meta[row] = {first workgroup, count}
// written by the workgroup holding the row's first tile.  Grid:
// ceil(wgs/8)*8*head_groups; workgroup L serves w = ((L/8)/hg)*8 + L%8 and
// head group (L/8)%hg, so the head groups of one tile range (same cache rows)
// run on one XCD and share its L2.
//
// Waves: wave v works on head tile v % nht (16 heads) and latent slice
// v / nht (NBLKW blocks of 128 columns).  Every wave of a head tile computes
// the same scores (the QK product is cheap next to the stream) and the PV
// product for its own slice only.  Per 32-token tile:
//   load     all 256 threads load the tile's cache rows into registers
//            (CPT 16-byte nontemporal loads per thread, 1 KB per wave
//            instruction) PF = stage_depth tiles ahead, and write a tile
//            into one of two LDS buffers just before it is computed, so the
//            bytes in flight are bounded by the register file rather than by
//            LDS.  Rows are unpadded (2W bytes); when W/8 is a multiple of 8,
//            16-byte column c of row r sits at c ^ (r & 7) so the operand
//            reads spread over the banks.  Wave 0 walks the rows PF + 1
//            tiles ahead: per tile it writes the row offsets (from a
//            page-table window in LDS for dense rows, from the index list
//            for sparse rows), the visibility mask, the row and the segment
//            flags.  A token that is not visible is loaded as a duplicate of
//            a visible row of its tile and gets weight 0.  Loads complete in
//            issue order, so the query of a row segment is loaded PF tiles
//            before the segment starts (a load at the start would wait for
//            every tile in flight).
//   QK       lane (r16, q4): A = row r16 (+16), 16-byte column 4c + q4,
//            B = [q | q_rope | 0] of head r16, elements 32c + 8 q4 .. +7
//            -> S0/S1: tokens 4 q4 + i and 16 + 4 q4 + i.
//   softmax  per lane (one head per lane column), max over the 4 lane
//            groups with permlane swaps; the accumulator is rescaled only
//            when a head's running max rises (wave-uniform branch).
//   PV       k index 8 q4 + e <-> token 4 q4 + e (e < 4) / 16 + 4 q4 + e - 4,
//            so B = P^T is the lane's own 8 probabilities (as hi + lo for
//            bf16: two MFMAs with the same A); A = C^T for
//            latent columns 128 blk + 8 r16 + e of those tokens (8 LDS
//            reads + 8x8 transpose); C tile (blk, e) row r <-> column
//            128 blk + 8 r + e: lane rows 4 q4 + i hold the 32 contiguous
//            columns 128 blk + 32 q4 .. +31.
template <int DT, int DS, int CPT>
__global__ __launch_bounds__(kAttendThreads) void mla_attend_mfma_kernel(MlaParams p) {
  using E = Elem<DT>;
  using Ops = MfmaOps<DT>;
  using S = typename E::S;
  constexpr int KMAX = 2 * CPT;            // W <= 64 CPT  ->  ceil(W/32) <= 2 CPT
  constexpr int NBLKW = 4 / DS;            // latent blocks of 128 columns per wave
  constexpr int QCH = (KMAX + DS - 1) / DS;  // query chunks per wave (c = slice + DS i)
  constexpr int PF = stage_depth(CPT, DS);
  static_assert(kMetaSlots >= PF + 2, "metadata slots");
  constexpr int kTileBytes = CPT * 4096;
  extern __shared__ __align__(16) char smem[];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int r16 = lane & 15, q4 = lane >> 4;

  const int L = blockIdx.x;
  const int hg = (L >> 3) % p.head_groups;
  const int w = ((L >> 3) / p.head_groups) * 8 + (L & 7);
  if (w >= p.wgs) return;  // whole workgroup: uniform

  char* ring = smem;
  int64_t* offs = reinterpret_cast<int64_t*>(smem + kRingTiles * kTileBytes);  // [slots][32]
  int64_t* tile_row = offs + kMetaSlots * kTileTokens;                         // [slots]
  int64_t* tile_base = tile_row + kMetaSlots;                                  // [slots]
  uint32_t* masks = reinterpret_cast<uint32_t*>(tile_base + kMetaSlots);       // [slots]
  int* flags = reinterpret_cast<int*>(masks + kMetaSlots);                     // [slots]
  int32_t* win = flags + kMetaSlots;                                           // [kWinPages]
  f32x4* sx = reinterpret_cast<f32x4*>(win + kWinPages + 8);               // [waves][2][64] partial scores

  const int64_t rows = static_cast<int64_t>(p.B) * p.T;
  const bool sparse = p.nk >= 0;
  const int nblk = (p.Dc + 127) / 128;

  // Wave roles.
  const int ht = wv % p.nht, slice = wv / p.nht;
  const int h0 = 16 * (p.nht * hg + ht);
  const bool active = wv < p.nht * DS && h0 < p.H;
  const int h = h0 + r16;
  const bool head_ok = h < p.H;
  const int blk0 = slice * NBLKW;

  // Prologue, in every wave: the visible end and the tile count of rows
  // 64 c + lane (c < kRegChunks) stay in registers (one round trip for up
  // to 256 rows; later rows are re-read), then the total G, this
  // workgroup's first (row, tile) and the empty rows it zero-fills.
  constexpr int kRegChunks = 4;
  constexpr int64_t kRegRows = 64 * kRegChunks;
  int end_r[kRegChunks], nt_r[kRegChunks];
  int64_t incl_r[kRegChunks];
  auto tiles_for = [&](int end) {
    const int count = sparse ? p.nk : end;
    return (count + kTileTokens - 1) / kTileTokens;
  };
#pragma unroll
  for (int c = 0; c < kRegChunks; ++c) {
    const int64_t r = 64 * c + lane;
    end_r[c] = r < rows ? row_end(p, static_cast<int>(r / p.T), r) : 0;
    nt_r[c] = r < rows ? tiles_for(end_r[c]) : 0;
  }
  int64_t carry = 0;
#pragma unroll
  for (int c = 0; c < kRegChunks; ++c) {
    incl_r[c] = carry + wave_incl_scan_i64(nt_r[c], lane);
    carry = __shfl(incl_r[c], 63);
  }
  for (int64_t base = kRegRows; base < rows; base += 64) {
    const int64_t r = base + lane;
    carry += wave_sum_i64(r < rows ? row_tiles(p, r) : 0);
  }
  const int64_t G = carry;
  const int64_t g0 = static_cast<int64_t>(w) * G / p.wgs;
  const int ntiles = static_cast<int>(static_cast<int64_t>(w + 1) * G / p.wgs - g0);
  if (w == 0 && hg == 0 && threadIdx.x == 0) *p.gtotal = G;

  // Row and tile of flattened tile g0.
  int64_t row0 = 0;
  int tir0 = 0;
  if (ntiles > 0) {
    bool found = false;
#pragma unroll
    for (int c = 0; c < kRegChunks; ++c) {
      const uint64_t hit = __ballot(64 * c + lane < rows && incl_r[c] > g0);
      if (!found && hit) {
        const int f = __builtin_ctzll(hit);
        row0 = 64 * c + f;
        tir0 = static_cast<int>(g0 - (__shfl(incl_r[c], f) - __shfl(nt_r[c], f)));
        found = true;
      }
    }
    int64_t cr = __shfl(incl_r[kRegChunks - 1], 63);
    for (int64_t base = kRegRows; !found && base < rows; base += 64) {
      const int64_t r = base + lane;
      const int64_t n = r < rows ? row_tiles(p, r) : 0;
      const int64_t incl = cr + wave_incl_scan_i64(n, lane);
      const uint64_t hit = __ballot(r < rows && incl > g0);
      if (hit) {
        const int f = __builtin_ctzll(hit);
        row0 = base + f;
        tir0 = static_cast<int>(g0 - (__shfl(incl, f) - __shfl(n, f)));
        found = true;
      }
      cr = __shfl(incl, 63);
    }
  }

  // Rows with no tile: zeros from workgroup (row % wgs), meta {0, 0}.
  auto zero_row = [&](int64_t r) {
    if (active && head_ok) {
      S* orow = static_cast<S*>(p.out) + (r * p.H + h) * p.Dc;
#pragma unroll
      for (int bb = 0; bb < NBLKW; ++bb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int dc0 = 128 * (blk0 + bb) + 32 * q4 + 8 * i;
          if (blk0 + bb < nblk && dc0 < p.Dc) *reinterpret_cast<u32x4*>(orow + dc0) = u32x4{0u, 0u, 0u, 0u};
        }
    }
    if (hg == 0 && threadIdx.x == 0) {
      p.meta[2 * r] = 0;
      p.meta[2 * r + 1] = 0;
    }
  };
#pragma unroll
  for (int c = 0; c < kRegChunks; ++c) {
    const int64_t r = 64 * c + lane;
    uint64_t zm = __ballot(r < rows && nt_r[c] == 0 && r % p.wgs == w);
    while (zm) {
      zero_row(64 * c + __builtin_ctzll(zm));
      zm &= zm - 1;
    }
  }
  for (int64_t r = kRegRows + (w - kRegRows % p.wgs + p.wgs) % p.wgs; r < rows; r += p.wgs)
    if (row_tiles(p, r) == 0) zero_row(r);

  // Per-row values of the cursor: from the registers, or re-read past them.
  auto pick = [&](const int (&arr)[kRegChunks], int64_t r) {
    const int c = static_cast<int>(r >> 6);
    const int v = c == 0 ? arr[0] : c == 1 ? arr[1] : c == 2 ? arr[2] : arr[3];
    return __builtin_amdgcn_readlane(v, static_cast<int>(r & 63));
  };
  auto end_of = [&](int64_t r) {
    return r < kRegRows ? pick(end_r, r)
                        : __builtin_amdgcn_readfirstlane(row_end(p, static_cast<int>(r / p.T), r));
  };
  auto tiles_of = [&](int64_t r) {
    return r < kRegRows ? pick(nt_r, r) : __builtin_amdgcn_readfirstlane(row_tiles(p, r));
  };

  const int kch = p.kch;
  (void)kch;
  const int w8 = p.W / 8;
  const int swz = (w8 & 7) == 0 ? 7 : 0;
  const char* cache = static_cast<const char*>(p.cache);

  // This thread's share of a tile: LDS chunk k*256 + tid is row-major
  // (row, c) = divmod(., W/8) and holds global column c ^ (row & swz);
  // chunks past the 32 rows are fillers that reread row 0.
  const int total_chunks = kTileTokens * w8;
  const int dtid = static_cast<int>(threadIdx.x) & 255;
  const int row0d = dtid / w8, col0d = dtid % w8;
  const int step_rows = 256 / w8, step_cols = 256 % w8;

  // Dense rows with P a multiple of 32: every tile is one page's rows.
  const bool contig = !sparse && p.P % kTileTokens == 0;

  // Wave 0's cursor over the workgroup's tiles.
  int64_t cur_row = row0;
  int cur_tir = tir0;
  int cur_n = 0, cur_end = 0, cur_b = 0, seg_tir = cur_tir;
  int64_t g_cur = g0;
  int win_base = -kWinPages;
  // Wave 0 reads metadata (lengths, positions, page table, index lists)
  // while tiles are in flight.  Loads complete in issue order, so a value
  // loaded here waits for every tile issued before it; each such value is
  // consumed inside the branch that loads it (wave-uniform values through
  // readfirstlane), so the steady path, which loads nothing, keeps exact
  // wait counts for the tiles.
  auto enter_row = [&]() {
    cur_b = static_cast<int>(cur_row / p.T);
    cur_end = end_of(cur_row);
    cur_n = tiles_of(cur_row);
    win_base = -kWinPages;  // window belongs to one sequence
  };
  auto load_window = [&](int first) {
    for (int i = lane; i < kWinPages; i += 64) {
      const int pg = first + i;
      win[i] = pg < p.maxP ? p.table[static_cast<int64_t>(cur_b) * p.maxP + pg] : 0;
    }
    __builtin_amdgcn_s_waitcnt(0);
    win_base = first;
  };
  auto clamp_phys = [&](int32_t phys) {
    if (phys < 0) phys = 0;
    if (phys >= p.num_blocks) phys = static_cast<int32_t>(p.num_blocks - 1);
    return phys;
  };
  // wave 0: metadata of the workgroup's tile t (called for t = 0, 1, ...).
  auto compute_offsets = [&](int t) {
    int fl = 0;
    if (t == 0 || cur_tir == 0) {
      fl |= kFlagFirst;
      seg_tir = cur_tir;
    }
    if (t == ntiles - 1 || cur_tir == cur_n - 1) {
      fl |= kFlagLast;
      if (seg_tir == 0 && cur_tir == cur_n - 1) fl |= kFlagWhole;
    }
    const int sl = t % kMetaSlots;
    if (contig) {
      // Dense row, P a multiple of 32: the tile is rows tok0 .. tok0 + 31
      // of one page; rows past the visible end read row 0 (finite data,
      // weight 0).
      const int tok0 = kTileTokens * cur_tir;
      const int pg = tok0 / p.P;
      if (pg < win_base || pg >= win_base + kWinPages) load_window(pg);
      const int32_t phys = clamp_phys(win[pg - win_base]);
      const int nv = min(kTileTokens, cur_end - tok0);
      if (lane == 0) {
        tile_base[sl] = (static_cast<int64_t>(phys) * p.P + (tok0 - pg * p.P)) * p.W;
        masks[sl] = nv >= kTileTokens ? 0xFFFFFFFFu : ((1u << nv) - 1u);
        flags[sl] = fl;
        tile_row[sl] = cur_row;
      }
    } else {
    const int count = sparse ? p.nk : cur_end;
    const int i = kTileTokens * cur_tir + lane;
    bool valid = lane < kTileTokens && i < count;
    int64_t off = 0;
    if (sparse) {
      const int tok = valid ? p.idx[cur_row * p.nk + i] : -1;
      valid = valid && tok >= 0 && tok < cur_end;
      const int32_t phys = clamp_phys(valid ? p.table[static_cast<int64_t>(cur_b) * p.maxP + tok / p.P] : 0);
      off = valid ? (static_cast<int64_t>(phys) * p.P + tok % p.P) * p.W : 0;
      __builtin_amdgcn_s_waitcnt(0);  // consumed here: see above
    } else {
      const int first = (kTileTokens * cur_tir) / p.P;
      const int last = (min(kTileTokens * cur_tir + kTileTokens, count) - 1) / p.P;
      if (first < win_base || last >= win_base + kWinPages) load_window(first);
      const int32_t phys = clamp_phys(valid ? win[i / p.P - win_base] : 0);
      off = valid ? (static_cast<int64_t>(phys) * p.P + i % p.P) * p.W : 0;
    }
    const uint32_t mask = static_cast<uint32_t>(__ballot(valid));
    const int fv = mask ? __builtin_ctz(mask) : 0;
    const int64_t dummy = __shfl(off, fv);
    if (lane < kTileTokens) offs[sl * kTileTokens + lane] = valid ? off : dummy;
    if (lane == 0) {
      tile_base[sl] = -1;
      masks[sl] = mask;
      flags[sl] = fl;
      tile_row[sl] = cur_row;
    }
    }
    if (cur_tir == 0 && hg == 0) {
      // This workgroup holds the row's first tile: record its span.  The
      // wait keeps the stores from leaving loads and stores both pending on
      // the steady path (the compiler would then wait for everything).
      const int64_t last_g = g_cur + cur_n - 1;
      const int64_t last_w = ((last_g + 1) * p.wgs - 1) / G;
      if (lane == 0) {
        p.meta[2 * cur_row] = w;
        p.meta[2 * cur_row + 1] = static_cast<int>(last_w - w + 1);
      }
      __builtin_amdgcn_s_waitcnt(0);
    }
    ++g_cur;
    ++cur_tir;
    if (cur_tir == cur_n && t + 1 < ntiles) {
      do {
        ++cur_row;
      } while (tiles_of(cur_row) == 0);
      cur_tir = 0;
      enter_row();
    }
  };
  // Loads tile t's chunks of this thread into registers; past the last
  // tile (live false) every lane loads the first 16 bytes of the cache
  // instead (one line per instruction), so every path issues the same loads
  // and the compiler's wait counts stay exact.
  auto issue = [&](int t, bool live, u32x4 (&dst)[CPT]) {
    const int sl = t % kMetaSlots;
    const int64_t tb = tile_base[sl];
    int row = row0d, col = col0d;
    if (tb >= 0) {  // contiguous tile: row r at tb + r W
      const int nv = __popc(masks[sl]);
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        const bool real = dtid + k * 256 < total_chunks;
        const int rr = real && row < nv ? row : 0;
        const char* src = cache + 2 * (tb + static_cast<int64_t>(rr) * p.W) + (real ? 16 * (col ^ (row & swz)) : 0);
        dst[k] = stream_load16(live ? src : cache);
        row += step_rows;
        col += step_cols;
        if (col >= w8) {
          col -= w8;
          ++row;
        }
      }
    } else {  // gathered rows
      const int64_t* o = offs + sl * kTileTokens;
#pragma unroll
      for (int k = 0; k < CPT; ++k) {
        const bool real = dtid + k * 256 < total_chunks;
        const char* src = cache + 2 * o[real ? row : 0] + (real ? 16 * (col ^ (row & swz)) : 0);
        dst[k] = stream_load16(live ? src : cache);
        row += step_rows;
        col += step_cols;
        if (col >= w8) {
          col -= w8;
          ++row;
        }
      }
    }
    // Keep each tile's loads in program order relative to the other tiles'
    // (the waits assume the oldest tile completes first).
    __builtin_amdgcn_sched_barrier(0);
  };
  // Writes tile t's registers into its LDS buffer.
  auto stage = [&](int t, const u32x4 (&src)[CPT]) {
    char* buf = ring + (t & 1) * kTileBytes;
#pragma unroll
    for (int k = 0; k < CPT; ++k) *reinterpret_cast<u32x4*>(buf + 16 * (dtid + 256 * k)) = src[k];
  };

  // Query operand [q | q_rope | 0] of head h, chunks of 32 elements: Dc and
  // Dr are multiples of 8, so each lane's 8-element group lies in q, in
  // q_rope or past W (zero) and is one 16-byte load.
  auto load_query = [&](int64_t r, u32x4 (&qv)[QCH]) {
    const char* qrow = static_cast<const char*>(p.q) + (r * p.H + (head_ok ? h : 0)) * p.Dc * 2;
    const char* rrow = static_cast<const char*>(p.qr) + (r * p.H + (head_ok ? h : 0)) * p.Dr * 2;
#pragma unroll
    for (int i = 0; i < QCH; ++i) {
      const int c = slice + DS * i;
      const int k = 32 * c + 8 * q4;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (head_ok && k < p.Dc) v = *reinterpret_cast<const u32x4*>(qrow + 2 * k);
      else if (head_ok && k < p.W) v = *reinterpret_cast<const u32x4*>(rrow + 2 * (k - p.Dc));
      qv[i] = v;
    }
  };

  u32x4 st[PF][CPT];            // tiles in flight: tile t in st[t % PF]
  u32x4 qv[QCH], qn[QCH];       // query of the current segment / of the next one
  int qn_tile = -1;             // tile whose segment query sits in qn
  float m_run = -INFINITY, l_run = 0.f;
  f32x4 acc[NBLKW][8];

  // One tile: stage it into LDS, refill its registers with tile j + PF,
  // compute, and close the row segment on its last tile.  Segment bounds
  // come from the per-tile flags wave 0 wrote (identical in every wave, so
  // every wave runs the same barriers).
  // Steps past the last tile (the rest of the last group of PF) only stage,
  // synchronize and issue their placeholder loads.
  auto step = [&](int j, u32x4 (&stu)[CPT]) {
    stage(j, stu);
    // Tile j is in LDS for every wave, and every wave is past tile j-1 (so
    // the buffer written next, tile j-2's, is free).  This barrier also
    // publishes wave 0's per-tile metadata: tile_row, flags and masks for
    // slot j % kMetaSlots (and the row offsets the staging reads) are
    // written by wave 0 ahead of the pipeline, and no other wave may read
    // them before it.  Every wave reaches it once per step, live or not.
    lds_barrier();
    const bool live = j < ntiles;
    const int sl = j % kMetaSlots;
    const int fl = live ? flags[sl] : 0;
    const uint32_t mask = live ? masks[sl] : 0u;
    const int64_t row = tile_row[sl];
    if (j + PF < ntiles) {
      const int sn = (j + PF) % kMetaSlots;
      if (active && qn_tile < 0 && (flags[sn] & kFlagFirst)) {
        load_query(tile_row[sn], qn);
        qn_tile = j + PF;
      }
    }
    issue(j + PF, j + PF < ntiles, stu);
    if ((fl & kFlagFirst) && active) {
      if (qn_tile == j) {
#pragma unroll
        for (int i = 0; i < QCH; ++i) qv[i] = qn[i];
        qn_tile = -1;
      } else if (j > 0) {
        // Two segments began within PF tiles: load now and wait (this path
        // only), so that qv is never pending on the steady path.
        load_query(row, qv);
        __builtin_amdgcn_s_waitcnt(0);
      }
      m_run = -INFINITY;
      l_run = 0.f;
#pragma unroll
      for (int bb = 0; bb < NBLKW; ++bb)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[bb][e] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const char* buf = ring + (j & 1) * kTileBytes;
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
    if (mask != 0u) {
      // S^T = C . Qcat^T for tokens 0-15 (s0) and 16-31 (s1).  The DS
      // waves of a head tile take the 32-element chunks c = slice + DS i
      // and add their partial scores through LDS (in slice order, so every
      // wave of the head tile gets the same bits).  All 2*CPT chunks are
      // covered: the query is zero past W, and a chunk past W reads the
      // next row or the tile's filler chunks (finite cache data, inside
      // the tile buffer since W/8 <= 8*CPT).
      if (active) {
        const int ra = r16, rb = 16 + r16;
#pragma unroll
        for (int i = 0; i < QCH; ++i) {
          const int c = slice + DS * i;
          if (KMAX % DS == 0 || c < KMAX) {
            const int c4 = 4 * c + q4;
            const u32x4 a0 = *reinterpret_cast<const u32x4*>(buf + 16 * (ra * w8 + (c4 ^ (ra & swz))));
            const u32x4 a1 = *reinterpret_cast<const u32x4*>(buf + 16 * (rb * w8 + (c4 ^ (rb & swz))));
            s0 = Ops::mma32(a0, qv[i], s0);
            s1 = Ops::mma32(a1, qv[i], s1);
          }
        }
      }
      if constexpr (DS > 1) {
        // [wave][half][lane]: lane-contiguous, free of bank conflicts.
        sx[(wv * 2) * 64 + lane] = s0;
        sx[(wv * 2 + 1) * 64 + lane] = s1;
        lds_barrier();
        s0 = f32x4{0.f, 0.f, 0.f, 0.f};
        s1 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int sl2 = 0; sl2 < DS; ++sl2) {
          const int src = ht + p.nht * sl2;
          s0 += sx[(src * 2) * 64 + lane];
          s1 += sx[(src * 2 + 1) * 64 + lane];
        }
      }
    }
    if (active && mask != 0u) {
      // Online softmax in log2 units.  The accumulator is rescaled only on
      // tiles that raise some head's running max (a wave-uniform branch;
      // rare once the max has been seen), so every probability is <= 1 and
      // the largest score's is exactly 1.
      float x[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[i] = (mask >> (4 * q4 + i)) & 1u ? s0[i] * p.sl2 : -INFINITY;
        x[4 + i] = (mask >> (16 + 4 * q4 + i)) & 1u ? s1[i] * p.sl2 : -INFINITY;
      }
      float mx = x[0];
#pragma unroll
      for (int e = 1; e < 8; ++e) mx = fmaxf(mx, x[e]);
      mx = max_over_lane_groups(mx);
      const bool move = mx > m_run;
      if (__ballot(move)) {
        const float alpha = move ? fast_exp2(m_run - mx) : 1.f;
        m_run = move ? mx : m_run;
        l_run *= alpha;
#pragma unroll
        for (int bb = 0; bb < NBLKW; ++bb)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[bb][e] *= alpha;
      }
      // The denominator sums the weights the PV product uses: for bf16 both
      // carry them as hi + lo (MfmaOps::kSplitWeights, ~2^-17), for fp16 the
      // 16-bit values, so the output is a normalized average of values.
      const float m_use = m_run == -INFINITY ? 0.f : m_run;
      float pr[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) pr[e] = fast_exp2(x[e] - m_use);
      const u32x4 pb = {Ops::pack2(pr[0], pr[1]), Ops::pack2(pr[2], pr[3]), Ops::pack2(pr[4], pr[5]),
                        Ops::pack2(pr[6], pr[7])};
      u32x4 pl = {0u, 0u, 0u, 0u};
      if constexpr (Ops::kSplitWeights) {
        pl = u32x4{Ops::rest2(pr[0], pr[1], pb[0]), Ops::rest2(pr[2], pr[3], pb[1]), Ops::rest2(pr[4], pr[5], pb[2]),
                   Ops::rest2(pr[6], pr[7], pb[3])};
        l_run += ((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7]));
      } else {
        l_run += (Ops::sum2(pb[0]) + Ops::sum2(pb[1])) + (Ops::sum2(pb[2]) + Ops::sum2(pb[3]));
      }

      // O^T += C[:, slice]^T . P^T
#pragma unroll
      for (int bb = 0; bb < NBLKW; ++bb) {
        if (blk0 + bb < nblk) {
          const int cc = min(16 * (blk0 + bb) + r16, p.Dc / 8 - 1);
          u32x4 raw[8];
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            const int tok = t < 4 ? 4 * q4 + t : 16 + 4 * q4 + (t - 4);
            raw[t] = *reinterpret_cast<const u32x4*>(buf + 16 * (tok * w8 + (cc ^ (tok & swz))));
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const u32x4 va = transpose8x8_col_b16(raw, e);
            acc[bb][e] = Ops::mma32(va, pb, acc[bb][e]);
            if constexpr (Ops::kSplitWeights) acc[bb][e] = Ops::mma32(va, pl, acc[bb][e]);
          }
        }
      }
    }

    if ((fl & kFlagLast) && active) {
      const float l = sum_over_lane_groups(l_run);
      if (head_ok) {
      if (fl & kFlagWhole) {
        const float inv = l > 0.f ? 1.f / l : 0.f;
        S* orow = static_cast<S*>(p.out) + (row * p.H + h) * p.Dc;
#pragma unroll
        for (int bb = 0; bb < NBLKW; ++bb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int dc0 = 128 * (blk0 + bb) + 32 * q4 + 8 * i;
            if (blk0 + bb < nblk && dc0 < p.Dc) {
              uint32_t wd[4];
#pragma unroll
              for (int e = 0; e < 8; e += 2) wd[e / 2] = Ops::pack2(acc[bb][e][i] * inv, acc[bb][e + 1][i] * inv);
              *reinterpret_cast<u32x4*>(orow + dc0) = u32x4{wd[0], wd[1], wd[2], wd[3]};
            }
          }
      } else {
        float* pr = p.part + ((w + row) * p.H + h) * static_cast<int64_t>(p.Dc + 2);
        if (slice == 0 && q4 == 0) {
          pr[0] = m_run == -INFINITY ? -INFINITY : m_run * kLn2;
          pr[1] = l;
        }
#pragma unroll
        for (int bb = 0; bb < NBLKW; ++bb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int dc0 = 128 * (blk0 + bb) + 32 * q4 + 8 * i;
            if (blk0 + bb < nblk && dc0 < p.Dc) {
#pragma unroll
              for (int e = 0; e < 8; ++e) pr[2 + dc0 + e] = acc[bb][e][i];
            }
          }
      }
      }
      // Stores pending next to the tile loads would make every later wait
      // a full drain; drain once here (segment ends only) instead.
      __builtin_amdgcn_s_waitcnt(0);
    }
    if (wv == 0 && j + PF + 1 < ntiles) compute_offsets(j + PF + 1);
  };

  // A tile's registers are waited for by the compiler, and its wait counts
  // stay exact (not vmcnt(0)) only where every path into a wait issued the
  // same loads: the loop runs whole groups of PF steps with unconditional
  // issues.
  if (ntiles > 0) {
    if (wv == 0) {
      enter_row();
      for (int t = 0; t < PF + 1 && t < ntiles; ++t) compute_offsets(t);
    }
    __syncthreads();
    // Queries first (the oldest loads): the first segment's, and the next
    // segment's when it starts within the first PF tiles.
    if (active) {
      load_query(tile_row[0], qv);
      for (int t = 1; t < PF && t < ntiles; ++t)
        if (flags[t % kMetaSlots] & kFlagFirst) {
          load_query(tile_row[t % kMetaSlots], qn);
          qn_tile = t;
          break;
        }
    }
#pragma unroll
    for (int u = 0; u < PF; ++u) issue(u, u < ntiles, st[u]);
    for (int j0 = 0; j0 < ntiles; j0 += PF) {
#pragma unroll
      for (int u = 0; u < PF; ++u) step(j0 + u, st[u]);
    }
  }
}

// ----------------------------------------------------------------------------
// Paged latent attention, wave-streamed kernel: dense rows, latent width
// 128*NB, rope width 32*RC, up to 16 heads per head group
// ----------------------------------------------------------------------------

constexpr int kSubTokens = 16;        // tokens per wave tile
constexpr int kWaveRows = 1024;       // query rows the prologue scans in LDS
constexpr int kWaveListTiles = 1024;  // tiles of one workgroup's range
constexpr int kWavePF = 2;            // tiles staged per wave
#ifndef QD_MLA_ROW_COST
#define QD_MLA_ROW_COST 24
#endif
// Partition cost of a row's start, in tile units: the row merge, the query
// pseudo-tile and the pipeline refill a workgroup pays entering a row cost
// about this many tiles of streaming.
constexpr int kWaveRowCost = QD_MLA_ROW_COST;
#ifndef QD_MLA_LAZY_LOG2
#define QD_MLA_LAZY_LOG2 8
#endif
constexpr float kWaveLazyLog2 = QD_MLA_LAZY_LOG2;

template <int NB, int RC>
struct WaveLayout {
  static constexpr int kDc = 128 * NB;
  static constexpr int kW = kDc + 32 * RC;
  static constexpr int kChunks = 4 * NB + RC;        // 32-element QK chunks
  // Rows padded by 32 bytes: the operand reads then meet fewer LDS bank
  // conflicts than with 16 (measured: 14% of LDS cycles against 34%).
  static constexpr int kStride = 2 * kW + 32;
  static constexpr int kBuf = kSubTokens * kStride;  // one wave's tile buffer
  static constexpr int kRopeBytes = 4 * RC;          // rope bytes per lane per row
};

__host__ __device__ constexpr size_t mla_wave_lds_bytes(int nb, int rc) {
  return 5 * static_cast<size_t>(kSubTokens) * (2 * (128 * nb + 32 * rc) + 32)  // wave tiles, query; merge exchange
         + 4 * 16 * 2 * 4                                                       // merge m, l
         + static_cast<size_t>(kWaveRows) * (4 + 4 + 8)                         // row tiles, ends, prefix
         + static_cast<size_t>(kWaveListTiles) * 16                             // tiles {base, rows, row}
         + 256;
}

// Registers of one tile in flight: lane (r16, q4) holds rows 4 q4 + i of
// latent columns 128 blk + 8 r16 .. +7 and rope columns Dc + 2 RC r16 ..
template <int NB, int RC>
struct WaveTile {
  u32x4 c[NB][4];
  uint32_t r[4][RC];
};

// Stream-K like mla_attend_mfma_kernel (same grid, meta, slots and merge),
// over 16-token tiles.  Each workgroup's range of tiles is dealt round-robin
// to its 4 waves (tile g to wave (g - g0) % 4); each wave streams its tiles
// on its own, with no per-tile barrier:
//   load     the 16 cache rows of a tile (one page: P % 16 == 0) into
//            registers, kWavePF tiles ahead, in the layout of the PV operand
//            (4 rows x 16 bytes per lane per latent block); the row's query
//            enters the same stream as a 16-row pseudo-tile (heads for
//            tokens) when a wave reaches a new row, so a row change never
//            waits for the tiles in flight (loads complete in issue order).
//   QK       the tile is written to the wave's LDS buffer (rows padded by 32
//            bytes) and read back as A = rows (tokens) x 32 columns; B = the
//            same chunks of the row's query, which the waves stage into one
//            shared LDS slot -> S^T[token 4 q4 + i][head r16]; operands are
//            read 3 chunks ahead into two accumulators.
//   softmax  fp32, with a lazy reference max (it may trail a head's
//            running max by up to 2^kWaveLazyLog2; the accumulators are
//            rescaled only past that).
//   PV       16x16x16 with A = C^T from 4 LDS rows (8x8 transposes by byte
//            permutes) and B = P^T, the lane's own 4 weights (for bf16 as
//            hi + lo: one 16x16x32 with the 4 tokens twice in A); C tile
//            (blk, e) row r <-> latent column 128 blk + 8 r + e.
// At the end of a row segment the 4 waves' states are merged through LDS
// (the only barriers of the main loop; every wave merges every row of the
// range in order): common max, rescale, then per 128-column block one wave
// sums the 4 accumulators and writes the output (whole row) or the partial.
// The prologue scans the rows' lengths into LDS, lists this range's tiles
// (row, page base, visible count: one page-table round trip for all of
// them), writes meta, gtotal and the empty rows.
// NT: nontemporal cache loads (one head group); with several head groups the
// tiles are loaded into L2 for the other groups' workgroups on the XCD.
template <int DT, int NB, int RC, bool NT>
__global__ __launch_bounds__(kAttendThreads) void mla_attend_wave_kernel(MlaParams p) {
  using E = Elem<DT>;
  using Ops = MfmaOps<DT>;
  using S = typename E::S;
  using Lay = WaveLayout<NB, RC>;
  using Tile = WaveTile<NB, RC>;
  constexpr int PF = kWavePF;
  constexpr int KC = Lay::kChunks;
  extern __shared__ __align__(16) char smem[];
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, q4 = lane >> 4;

  const int L = blockIdx.x;
  const int hg = (L >> 3) % p.head_groups;
  const int w = ((L >> 3) / p.head_groups) * 8 + (L & 7);
  if (w >= p.wgs) return;  // whole workgroup: uniform

  char* tbuf = smem + wv * Lay::kBuf;                                     // this wave's tile
  char* qbuf = smem + 4 * Lay::kBuf;                                      // the current row's query
  // [wave][e][lane] f32x4: consecutive lanes at consecutive 16 bytes, so
  // the exchange's LDS accesses are free of bank conflicts.
  float* ml = reinterpret_cast<float*>(smem + 5 * Lay::kBuf);           // [4][16][2]
  int* rt = reinterpret_cast<int*>(ml + 4 * 16 * 2);                      // [rows] tiles
  int* re = rt + kWaveRows;                                               // [rows] visible end
  int64_t* incl = reinterpret_cast<int64_t*>(re + kWaveRows);            // [rows] prefix of tiles
  // [tiles] {element offset of the tile's row 0 (2 words), visible rows, query row}
  int* tl = reinterpret_cast<int*>(incl + kWaveRows);

  const int rows = p.B * p.T;  // <= kWaveRows (host check)
  const int h0 = 16 * hg;
  const int nh = min(16, p.H - h0);
  const int h = h0 + r16;
  const bool head_ok = r16 < nh;
  const char* cache = static_cast<const char*>(p.cache);

  // --- Prologue -----------------------------------------------------------
  for (int r = tid; r < rows; r += kAttendThreads) {
    const int end = row_end(p, r / p.T, r);
    re[r] = end;
    rt[r] = (end + kSubTokens - 1) / kSubTokens;
  }
  __syncthreads();
  auto row_cost = [&](int tiles) { return tiles > 0 ? tiles + kWaveRowCost : 0; };
  if (wv == 0) {
    int64_t carry = 0;
    for (int base = 0; base < rows; base += 64) {
      const int r = base + lane;
      const int64_t n = r < rows ? row_cost(rt[r]) : 0;
      const int64_t v = carry + wave_incl_scan_i64(n, lane);
      if (r < rows) incl[r] = v;
      carry = __shfl(v, 63);
    }
  }
  __syncthreads();
  const int64_t G = incl[rows - 1];
  const int64_t g0 = static_cast<int64_t>(w) * G / p.wgs;
  const int64_t g1 = static_cast<int64_t>(w + 1) * G / p.wgs;
  const int nt = static_cast<int>(g1 - g0);  // positions, <= kWaveListTiles (host check)
  if (w == 0 && hg == 0 && tid == 0) *p.gtotal = G;
  auto wg_of = [&](int64_t x) { return static_cast<int>(((x + 1) * p.wgs - 1) / G); };
  // This range's cost positions: row (binary search of the prefix); the
  // first kWaveRowCost positions of a row hold no tile (row -1), the others
  // tile i: page base and visible rows.
  for (int t = tid; t < nt; t += kAttendThreads) {
    const int64_t g = g0 + t;
    int lo = 0, hi = rows - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (incl[mid] > g) hi = mid; else lo = mid + 1;
    }
    const int r = lo;
    const int tir = static_cast<int>(g - (incl[r] - rt[r]));
    if (tir < 0) {
      *reinterpret_cast<i32x4*>(tl + 4 * t) = i32x4{0, 0, 0, -1};
      continue;
    }
    const int tok0 = kSubTokens * tir;
    const int pg = tok0 / p.P;
    int32_t phys = p.table[static_cast<int64_t>(r / p.T) * p.maxP + pg];
    if (phys < 0) phys = 0;
    if (phys >= p.num_blocks) phys = static_cast<int32_t>(p.num_blocks - 1);
    const int64_t base = (static_cast<int64_t>(phys) * p.P + (tok0 - pg * p.P)) * Lay::kW;
    *reinterpret_cast<i32x4*>(tl + 4 * t) =
        i32x4{static_cast<int>(base & 0xFFFFFFFF), static_cast<int>(base >> 32), min(kSubTokens, re[r] - tok0), r};
    if (tir == 0 && hg == 0) {
      // This workgroup holds the row's first tile: record its span.
      p.meta[2 * r] = w;
      p.meta[2 * r + 1] = wg_of(incl[r] - 1) - w + 1;
    }
  }
  // Rows with no tile: zeros from workgroup (row % wgs), meta {0, 0}.
  for (int r = w; r < rows; r += p.wgs) {
    if (rt[r] != 0) continue;
    S* orow = static_cast<S*>(p.out) + (static_cast<int64_t>(r) * p.H + h0) * Lay::kDc;
    for (int i = tid; i < nh * Lay::kDc / 8; i += kAttendThreads)
      *reinterpret_cast<u32x4*>(orow + 8 * i) = u32x4{0u, 0u, 0u, 0u};
    if (hg == 0 && tid == 0) {
      p.meta[2 * r] = 0;
      p.meta[2 * r + 1] = 0;
    }
  }
  __syncthreads();

  // --- Per-wave item stream -------------------------------------------------
  // Items in order: for each row of this wave's tiles, the query pseudo-tile,
  // then the row's tiles.  Past the end, placeholder loads of the first
  // cache bytes keep every path's load count equal (exact wait counts).
  constexpr int kNone = 0, kQuery = 1, kTile = 2;
  int is_k = 0;        // next tile ordinal of this wave: g = g0 + wv + 4 k
  int is_row = -1;     // row of the last issued item
  auto issue = [&](Tile& dst, int& kind, int& row, int& nv) {
    int t = wv + 4 * is_k;
    kind = kNone;
    row = -1;
    nv = 0;
    int64_t tbase = 0;
    i32x4 m = {0, 0, 0, -1};
    while (t < nt) {  // skip the rows' start positions (no tile)
      m = *reinterpret_cast<const i32x4*>(tl + 4 * t);
      if (m[3] >= 0) break;
      ++is_k;
      t += 4;
    }
    if (t < nt) {
      row = m[3];
      if (row != is_row) {
        kind = kQuery;
        is_row = row;
      } else {
        kind = kTile;
        nv = m[2];
        tbase = static_cast<int64_t>(static_cast<uint32_t>(m[0])) | (static_cast<int64_t>(m[1]) << 32);
        ++is_k;
      }
    }
    // Row offsets (elements) of rows 4 q4 + i and the base of each column.
    const char* lat;
    const char* rop;
    int64_t rs_l, rs_r;  // row strides in bytes
    int nrow;            // valid rows (others reread row 0)
    if (kind == kTile) {
      const int64_t b = tbase;
      lat = cache + 2 * b;
      rop = cache + 2 * (b + Lay::kDc);
      rs_l = rs_r = 2 * static_cast<int64_t>(Lay::kW);
      nrow = nv;
    } else if (kind == kQuery) {
      lat = static_cast<const char*>(p.q) + (static_cast<int64_t>(row) * p.H + h0) * Lay::kDc * 2;
      rop = static_cast<const char*>(p.qr) + (static_cast<int64_t>(row) * p.H + h0) * (32 * RC) * 2;
      rs_l = 2 * Lay::kDc;
      rs_r = 2 * 32 * RC;
      nrow = nh;
    } else {
      lat = rop = cache;
      rs_l = rs_r = 0;
      nrow = 1;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rr = 4 * q4 + i < nrow ? 4 * q4 + i : 0;
      const char* lrow_p = lat + rr * rs_l + 16 * r16;
#pragma unroll
      for (int blk = 0; blk < NB; ++blk) dst.c[blk][i] = load16<NT>(lrow_p + 256 * blk);
      const char* rp = rop + rr * rs_r + Lay::kRopeBytes * r16;
      if constexpr (RC == 1) {
        dst.r[i][0] = NT ? __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(rp))
                         : *reinterpret_cast<const uint32_t*>(rp);
      } else if constexpr (RC == 2) {
        const u32x2 x = load8<NT>(rp);
        dst.r[i][0] = x[0];
        dst.r[i][1] = x[1];
      } else {
        const u32x4 x = load16<NT>(rp);
#pragma unroll
        for (int k = 0; k < RC; ++k) dst.r[i][k] = x[k];
      }
    }
    // Keep each item's loads in program order relative to the others'.
    __builtin_amdgcn_sched_barrier(0);
  };
  // Writes an item's rows (4 q4 + i) into an LDS buffer.
  auto stage = [&](const Tile& src, int valid, char* buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool ok = 4 * q4 + i < valid;
      char* rowp = buf + (4 * q4 + i) * Lay::kStride;
#pragma unroll
      for (int blk = 0; blk < NB; ++blk)
        *reinterpret_cast<u32x4*>(rowp + 256 * blk + 16 * r16) = ok ? src.c[blk][i] : u32x4{0u, 0u, 0u, 0u};
      char* rp = rowp + 2 * Lay::kDc + Lay::kRopeBytes * r16;
      if constexpr (RC == 1) {
        *reinterpret_cast<uint32_t*>(rp) = ok ? src.r[i][0] : 0u;
      } else if constexpr (RC == 2) {
        *reinterpret_cast<u32x2*>(rp) = ok ? u32x2{src.r[i][0], src.r[i][1]} : u32x2{0u, 0u};
      } else {
        *reinterpret_cast<u32x4*>(rp) = ok ? u32x4{src.r[i][0], src.r[i][1], src.r[i][2], src.r[i][3]}
                                           : u32x4{0u, 0u, 0u, 0u};
      }
    }
  };

  // --- State and the row merge ----------------------------------------------
  float m_run = -INFINITY, l_run = 0.f;
  f32x4 acc[NB][8];
  auto reset = [&]() {
    m_run = -INFINITY;
    l_run = 0.f;
#pragma unroll
    for (int bb = 0; bb < NB; ++bb)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[bb][e] = f32x4{0.f, 0.f, 0.f, 0.f};
  };
  reset();
  // Rows of the range in order; merged_row: the next one to merge.
  auto row_at = [&](int64_t from) {  // row of the first tile at or after position from
    for (int64_t x = from; x < g1; ++x) {
      const int r = tl[4 * (x - g0) + 3];
      if (r >= 0) return r;
    }
    return rows;
  };
  int merge_row = row_at(g0);
  auto merge = [&](int r) {
    const float lw = sum_over_lane_groups(l_run);
    if (q4 == 0) {
      ml[(wv * 16 + r16) * 2] = m_run;
      ml[(wv * 16 + r16) * 2 + 1] = lw;
    }
    lds_barrier();
    float M = -INFINITY;
#pragma unroll
    for (int v = 0; v < 4; ++v) M = fmaxf(M, ml[(v * 16 + r16) * 2]);
    float Lt = 0.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float mv = ml[(v * 16 + r16) * 2];
      if (mv != -INFINITY) Lt += ml[(v * 16 + r16) * 2 + 1] * fast_exp2(mv - M);
    }
    const float sc = m_run == -INFINITY ? 0.f : fast_exp2(m_run - M);
    const int64_t first_tile = incl[r] - rt[r];
    const bool whole = first_tile >= g0 && incl[r] <= g1;
    // Two rounds of two 128-column blocks.  Every wave deposits its scaled
    // blocks 2k and 2k + 1 (16 KB) in the tile buffers, idle during the
    // merge (xr: [wave][8 jb + e][lane] f32x4, lane-contiguous); then wave v
    // sums half e = 4 (v % 2) .. + 3 of block 2k + v / 2, so all four sum at
    // once.  The block's fp16 scale is the larger of the two halves' |max|,
    // exchanged through ml (free once every wave has read M and L).
    static_assert(NB == 4, "two rounds of two blocks");
    static_assert(4 * 16 * 64 * 16 <= 4 * Lay::kBuf, "the exchange fits in the four tile buffers");
    float* xr = reinterpret_cast<float*>(smem);
    const int eh = 4 * (wv & 1);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          *reinterpret_cast<f32x4*>(xr + 4 * ((wv * 16 + 8 * jb + e) * 64 + lane)) = acc[2 * k + jb][e] * sc;
      lds_barrier();
      const int bb = 2 * k + (wv >> 1);
      f32x4 o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int j = 8 * (wv >> 1) + eh + e;
        o[e] = *reinterpret_cast<const f32x4*>(xr + 4 * ((0 * 16 + j) * 64 + lane));
#pragma unroll
        for (int v = 1; v < 4; ++v) o[e] += *reinterpret_cast<const f32x4*>(xr + 4 * ((v * 16 + j) * 64 + lane));
      }
      float amax = 0.f;
      if (!whole) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          amax = fmaxf(amax, fmaxf(fmaxf(fabsf(o[e][0]), fabsf(o[e][1])), fmaxf(fabsf(o[e][2]), fabsf(o[e][3]))));
        amax = fmaxf(amax, __shfl_xor(amax, 16));
        amax = fmaxf(amax, __shfl_xor(amax, 32));
        if (q4 == 0) ml[wv * 16 + r16] = amax;
      }
      lds_barrier();  // every wave has read xr (the next round rewrites it) and written its half's max
      if (head_ok) {
        if (whole) {
          const float inv = Lt > 0.f ? 1.f / Lt : 0.f;
          S* orow = static_cast<S*>(p.out) + (static_cast<int64_t>(r) * p.H + h) * Lay::kDc;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            *reinterpret_cast<u32x2*>(orow + 128 * bb + 32 * q4 + 8 * i + eh) =
                u32x2{Ops::pack2(o[0][i] * inv, o[1][i] * inv), Ops::pack2(o[2][i] * inv, o[3][i] * inv)};
        } else {
          // Half-precision partial row (kHalfHeader): block bb as fp16
          // values o / s_bb, s_bb the block's largest |o| for the head.
          const float sbb = half_partial_scale(fmaxf(amax, ml[(wv ^ 1) * 16 + r16]));
          const float isc = 1.f / sbb;
          float* pr = p.part + ((static_cast<int64_t>(w) + r) * p.H + h) * static_cast<int64_t>(kHalfPst);
          if (q4 == 0 && eh == 0) {
            if (bb == 0) {
              pr[0] = M == -INFINITY ? -INFINITY : M * kLn2;
              pr[1] = Lt;
              pr[6] = 0.f;
              pr[7] = 0.f;
            }
            pr[2 + bb] = sbb;
          }
          // Lane (r16, q4), row i: columns 128 bb + 32 q4 + 8 i + eh + e, e = 0..3.
          char* pa = reinterpret_cast<char*>(pr + kHalfHeader) + 2 * (128 * bb + 32 * q4 + eh);
#pragma unroll
          for (int i = 0; i < 4; ++i)
            *reinterpret_cast<u32x2*>(pa + 16 * i) =
                u32x2{pack_f16_rne(o[0][i] * isc, o[1][i] * isc), pack_f16_rne(o[2][i] * isc, o[3][i] * isc)};
        }
      }
    }
    lds_barrier();  // the tile buffers and ml are read; the next row may stage and merge
    // Stores pending next to the loads in flight would make every later
    // wait a full drain; drain here (row ends only) instead.
    __builtin_amdgcn_s_waitcnt(0);
    reset();
  };
  // Merges the rows before row r (r = rows: all of them).
  auto merge_before = [&](int r) {
    while (merge_row < r) {
      merge(merge_row);
      merge_row = row_at(incl[merge_row]);  // first tile of the following rows
    }
  };

  // --- Main loop --------------------------------------------------------------
  Tile st[PF];
  int s_kind[PF], s_row[PF], s_nv[PF];
#pragma unroll
  for (int u = 0; u < PF; ++u) issue(st[u], s_kind[u], s_row[u], s_nv[u]);
  int pending = 0;
#pragma unroll
  for (int u = 0; u < PF; ++u) pending += s_kind[u] != kNone;

  auto step = [&](Tile& stu, int& skind, int& srow, int& snv) {
    const int kind = skind, row = srow, nv = snv;
    if (kind == kQuery) {
      // The row's query goes to the shared slot: every wave with tiles in
      // the row writes the same rows, after the previous row's merge (no
      // wave still reads the old query).
      merge_before(row);
      stage(stu, nh, qbuf);
    } else if (kind == kTile) {
      stage(stu, kSubTokens, tbuf);
    }
    issue(stu, skind, srow, snv);
    pending += (skind != kNone) - (kind != kNone);
    if (kind == kTile) {
      // A = cache rows (tokens), B = query rows (heads), both row r16.
      f32x4 s = {0.f, 0.f, 0.f, 0.f};
      // Operands read kAhead chunks before their MFMA (LDS latency), two
      // accumulators to halve the dependent MFMA chain.
      constexpr int kAhead = 3;
      const char* ta = tbuf + r16 * Lay::kStride + 16 * q4;
      const char* qa = qbuf + r16 * Lay::kStride + 16 * q4;
      u32x4 ar[kAhead], br[kAhead];
#pragma unroll
      for (int c = 0; c < kAhead; ++c) {
        ar[c] = *reinterpret_cast<const u32x4*>(ta + 64 * c);
        br[c] = *reinterpret_cast<const u32x4*>(qa + 64 * c);
      }
      // The scheduling barriers keep each chunk's reads kAhead MFMAs ahead:
      // left free, the scheduler sinks them next to their MFMA and every
      // MFMA waits out a whole LDS round trip.
      __builtin_amdgcn_sched_barrier(0);
      f32x4 s2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        const u32x4 a = ar[c % kAhead], b = br[c % kAhead];
        if (c & 1)
          s2 = Ops::mma32(a, b, s2);
        else
          s = Ops::mma32(a, b, s);
        if (c + kAhead < KC) {
          ar[c % kAhead] = *reinterpret_cast<const u32x4*>(ta + 64 * (c + kAhead));
          br[c % kAhead] = *reinterpret_cast<const u32x4*>(qa + 64 * (c + kAhead));
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      s += s2;
      float x[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = 4 * q4 + i < nv ? s[i] * p.sl2 : -INFINITY;
      float mx = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
      mx = max_over_lane_groups(mx);
      // Lazy reference max: a head's m_run may trail its running max by up
      // to kWaveLazyLog2, so its weights stay <= 2^kWaveLazyLog2 (exact
      // scaling in fp32, far inside the 16-bit range).  The accumulators,
      // 128 AGPRs a lane, are rescaled only when some head's max moves past
      // that, and then every head catches up.  With the exact max, 16 heads
      // rescaled on about 80% of the tiles.
      const bool move = mx > m_run + kWaveLazyLog2;
      if (__ballot(move)) {
        const float mn = fmaxf(m_run, mx);
        const float alpha = mn == m_run ? 1.f : fast_exp2(m_run - mn);  // m_run = -inf: 0
        m_run = mn;
        l_run *= alpha;
#pragma unroll
        for (int bb = 0; bb < NB; ++bb)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[bb][e] *= alpha;
      }
      const float m_use = m_run == -INFINITY ? 0.f : m_run;
      float pr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) pr[i] = fast_exp2(x[i] - m_use);
      // Weights as hi + lo for bf16 (MfmaOps::kSplitWeights); the
      // denominator sums what the PV product uses.
      const u32x2 pb = {Ops::pack2(pr[0], pr[1]), Ops::pack2(pr[2], pr[3])};
      u32x4 pbl = {pb[0], pb[1], 0u, 0u};
      if constexpr (Ops::kSplitWeights) {
        pbl[2] = Ops::rest2(pr[0], pr[1], pb[0]);
        pbl[3] = Ops::rest2(pr[2], pr[3], pb[1]);
        l_run += (pr[0] + pr[1]) + (pr[2] + pr[3]);
      } else {
        l_run += Ops::sum2(pb[0]) + Ops::sum2(pb[1]);
      }
      // The next block's 4 rows are read while this block multiplies.
      const char* pv0 = tbuf + 4 * q4 * Lay::kStride + 16 * r16;
      u32x4 nraw[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) nraw[i] = *reinterpret_cast<const u32x4*>(pv0 + i * Lay::kStride);
#pragma unroll
      for (int bb = 0; bb < NB; ++bb) {
        u32x4 raw[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) raw[i] = nraw[i];
        if (bb + 1 < NB) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            nraw[i] = *reinterpret_cast<const u32x4*>(pv0 + i * Lay::kStride + 256 * (bb + 1));
        }
        // As in QK: the next block's reads stay ahead of this block's MFMAs.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int wd = e >> 1;
          const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
          const u32x2 a = {__builtin_amdgcn_perm(raw[1][wd], raw[0][wd], sel),
                           __builtin_amdgcn_perm(raw[3][wd], raw[2][wd], sel)};
          // bf16: one 16x16x32 MFMA over the lane's 4 tokens twice, [hi, lo]
          // weights in B (any consistent k order sums the same).
          if constexpr (Ops::kSplitWeights)
            acc[bb][e] = Ops::mma32(u32x4{a[0], a[1], a[0], a[1]}, pbl, acc[bb][e]);
          else
            acc[bb][e] = Ops::pv(a, pb, acc[bb][e]);
        }
      }
    }
  };
  while (pending > 0) {
#pragma unroll
    for (int u = 0; u < PF; ++u) step(st[u], s_kind[u], s_row[u], s_nv[u]);
  }
  merge_before(rows);
}

// ----------------------------------------------------------------------------
// Paged latent attention, shared-tile kernel: dense rows, Dc 512, Dr 64,
// 64 heads per workgroup of four waves, 32-token cache tiles fed to LDS by
// DMA and shared by all four waves
// ----------------------------------------------------------------------------

constexpr int kShThreads = 256;                         // four waves, 16 heads each
constexpr int kShTokens = 32;                           // tokens per tile
constexpr int kShBufs = 4;                              // LDS tile ring
constexpr int kShRowBytes = 2 * 576;                    // cache row: 512 latent + 64 rope, 16-bit
#ifndef QD_MLA_SHARED_ROW_PAD
#define QD_MLA_SHARED_ROW_PAD 32
#endif
constexpr int kShLatStride = 1024 + QD_MLA_SHARED_ROW_PAD;  // LDS bytes per latent row (padded)
constexpr int kShLatBytes = kShTokens * kShLatStride;   // latent part of a tile
constexpr int kShTileBytes = kShLatBytes + kShTokens * 128;  // + rope rows
constexpr int kShRows = 1024;                           // query rows (prologue arrays in the ring)
constexpr int kShListTiles = 512;                       // tiles of one workgroup's range
constexpr int kShCtlPad = 8;                            // placeholder entries after the tile list
constexpr int kShDma = 9;                               // DMA instructions per wave per tile
constexpr int kShColBlocks = 512 / 16;                  // PV output blocks of 16 latent columns
#ifndef QD_MLA_SHARED_PV_AHEAD
#define QD_MLA_SHARED_PV_AHEAD 4
#endif
constexpr int kShPvAhead = QD_MLA_SHARED_PV_AHEAD;      // PV operand blocks read ahead of their MFMAs
static_assert(kShDma <= 18, "one DMA instruction per QK chunk");
#ifndef QD_MLA_SHARED_ROW_COST
#define QD_MLA_SHARED_ROW_COST 4
#endif
// Partition cost of a row's start, in tile units: the row's query load and
// output stores drain the tile pipeline once.
constexpr int kShRowCost = QD_MLA_SHARED_ROW_COST;
#ifndef QD_MLA_SHARED_QK_AHEAD
#define QD_MLA_SHARED_QK_AHEAD 6
#endif

__host__ __device__ constexpr size_t mla_shared_lds_bytes() {
  return static_cast<size_t>(kShBufs) * kShTileBytes    // tile ring (prologue arrays before the first tile)
         + static_cast<size_t>(kShListTiles + kShCtlPad) * 16;  // tile list
}

static_assert(kShRows * (4 + 4 + 8) + kShListTiles * 16 <= kShBufs * kShTileBytes,
              "shared-tile kernel prologue arrays exceed the tile ring");

// Wait for all but the last kVm vector-memory operations of this wave (loads
// into LDS included) and for its LDS operations, then the workgroup
// barrier.  The empty asm statements keep the compiler from moving memory
// accesses across.
template <int kVm>
__device__ __forceinline__ void dma_ring_barrier() {
  static_assert(kVm >= 0 && kVm < 64, "vmcnt is 6 bits");
  constexpr int imm = (kVm & 0xF) | ((kVm >> 4) << 14) | (0x7 << 4) | (0x0 << 8);  // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(imm);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// vmcnt(0) alone (expcnt and lgkmcnt left free).
__device__ __forceinline__ void wait_vm_all() { __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xF << 8)); }

// f(std::integral_constant<int, I>) for I = B .. E-1, in order.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// LDS byte address of a pointer into this workgroup's LDS.
__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p));
}

// ds_read_b64_tr_b16 at LDS address base + OFF, as inline asm.  The
// compiler's wait insertion treats the builtin form as a read of any LDS
// buffer a DMA (global_load_lds) may be filling and waits for every DMA in
// flight before it; the asm form is not tracked, so its result may be used
// only after lds_wait_tied.
template <int OFF>
struct TrRead {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset is 16 bits");
  __device__ __forceinline__ static void issue(uint32_t base, u32x2& out) {
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(out) : "v"(base), "i"(OFF));
  }
};

// Waits until at most N LDS (and scalar-memory) operations are outstanding.
// LDS operations complete in order, so with N = the number of LDS reads
// issued after the ones that produced a and b, those are complete (other
// operations outstanding only make the wait longer).  a and b are tied to
// the wait so that no use of them is scheduled before it.
template <int N>
__device__ __forceinline__ void lds_wait_tied(u32x2& a, u32x2& b) {
  static_assert(N >= 0 && N < 16, "lgkmcnt is 4 bits");
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "i"(N));
}


// Stream-K over (query row, 32-token tile) like mla_attend_wave_kernel (same
// grid mapping, meta and merge kernel; fp16 partial rows), one workgroup per
// CU with 64 heads, every wave on every tile of the workgroup's range.  Wave
// v serves heads 16 v .. 16 v + 15 of the workgroup's:
//   load     each wave DMAs a quarter of the tile's 32 cache rows (latent
//            rows 8v .. 8v + 7, 1 KB per instruction, and their rope bytes)
//            into one of kShBufs LDS buffers (global_load_lds), kShBufs - 1
//            tiles ahead, one instruction per QK chunk of the current tile
//            (issued back to back after the barrier, the four waves' loads
//            queued on the CU's load path for as long as the QK products
//            take); no registers hold tiles in flight.  Latent rows are 1 KB
//            apart plus kShLatStride - 1024 bytes (each instruction has its
//            own LDS base), so the operand reads take immediate offsets from
//            one lane address; rope chunk c of row R sits at c ^ (R/2 % 8).
//            Rows past the tile's visible count re-read its last visible row
//            and get weight 0.
//   QK       per 16-row block of the tile: S^T = K chunk x [q | q_rope]
//            chunk over the 18 32-element chunks (query in registers, loaded
//            when a row segment starts).
//   softmax  fp32 over the tile's 32 tokens, with the lazy reference max of
//            the wave kernel.
//   PV       one 16x16x32 per 16 output columns over all 32 tokens, A = V^T
//            from transposing LDS reads; bf16 weights as hi + lo (two MFMAs
//            on the same A).
// No per-tile exchange between waves: one barrier per tile, for the ring.
// At the end of a row segment each wave stores its heads: the output (whole
// row) or the partial {m, l, scales, acc} in slot (w + row); the next row's
// query is loaded there too, and one wait for every load in flight covers
// both (the stores would otherwise hold the tile waits behind them).
// NT: nontemporal cache loads (one head group); with several head groups
// the tiles stay in L2 for the other groups' workgroups on the XCD.
template <int DT, bool NT>
__global__ __launch_bounds__(kShThreads) void mla_attend_shared_kernel(MlaParams p) {
  using E = Elem<DT>;
  using Ops = MfmaOps<DT>;
  using S = typename E::S;
  constexpr int kDc = 512;
  constexpr int kW = 576;
  extern __shared__ __align__(16) char smem[];
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, q4 = lane >> 4;
  [[maybe_unused]] const uint64_t st_entry = QD_MLA_STAMPS_ON ? __builtin_amdgcn_s_memrealtime() : 0;
  [[maybe_unused]] const uint64_t st_clk0 = QD_MLA_STAMPS_ON ? __builtin_amdgcn_s_memtime() : 0;
  [[maybe_unused]] uint64_t st_rowend = 0;
  [[maybe_unused]] int st_rowends = 0;

  const int L = blockIdx.x;
  const int hg = (L >> 3) % p.head_groups;
  const int w = ((L >> 3) / p.head_groups) * 8 + (L & 7);
  if (w >= p.wgs) return;  // whole workgroup: uniform

  char* ring = smem;
  i32x4* ctl = reinterpret_cast<i32x4*>(smem + kShBufs * kShTileBytes);
  // Prologue arrays, inside the ring.
  int* rt = reinterpret_cast<int*>(ring);                      // [rows] tiles
  int* re = rt + kShRows;                                      // [rows] visible end
  int64_t* incl = reinterpret_cast<int64_t*>(re + kShRows);   // [rows] prefix of costs
  i32x4* tl = reinterpret_cast<i32x4*>(incl + kShRows);       // [positions]
  int* nreal = reinterpret_cast<int*>(tl + kShListTiles);     // real tiles of the range

  const int rows = p.B * p.T;  // <= kShRows (host check)
  constexpr int kHeads = 64;   // per workgroup
  const int h0 = kHeads * hg;
  const int h = h0 + 16 * wv + r16;  // this lane's head
  const char* cache = static_cast<const char*>(p.cache);

  // --- Prologue -----------------------------------------------------------
  for (int r = tid; r < rows; r += kShThreads) {
    const int end = row_end(p, r / p.T, r);
    re[r] = end;
    rt[r] = (end + kShTokens - 1) / kShTokens;
  }
  __syncthreads();
  auto row_cost = [&](int tiles) { return tiles > 0 ? tiles + kShRowCost : 0; };
  if (wv == 0) {
    int64_t carry = 0;
    for (int base = 0; base < rows; base += 64) {
      const int r = base + lane;
      const int64_t n = r < rows ? row_cost(rt[r]) : 0;
      const int64_t v = carry + wave_incl_scan_i64(n, lane);
      if (r < rows) incl[r] = v;
      carry = __shfl(v, 63);
    }
  }
  __syncthreads();
  const int64_t G = incl[rows - 1];
  const int64_t g0 = static_cast<int64_t>(w) * G / p.wgs;
  const int64_t g1 = static_cast<int64_t>(w + 1) * G / p.wgs;
  const int npos = static_cast<int>(g1 - g0);  // <= kShListTiles (host check)
  if (w == 0 && hg == 0 && tid == 0) *p.gtotal = G;
  auto wg_of = [&](int64_t x) { return static_cast<int>(((x + 1) * p.wgs - 1) / G); };
  // Positions of this range: the first kShRowCost positions of a row hold no
  // tile (row -1); the others tile i of the row: element offset of its first
  // cache row, visible rows | whole-row flag << 16, row.
  for (int t = tid; t < npos; t += kShThreads) {
    const int64_t g = g0 + t;
    int lo = 0, hi = rows - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (incl[mid] > g) hi = mid; else lo = mid + 1;
    }
    const int r = lo;
    const int64_t first = incl[r] - rt[r];
    const int tir = static_cast<int>(g - first);
    if (tir < 0) {
      tl[t] = i32x4{0, 0, 0, -1};
      continue;
    }
    const int tok0 = kShTokens * tir;
    const int pg = tok0 / p.P;  // the tile lies in one page (P % 32 == 0)
    int32_t phys = p.table[static_cast<int64_t>(r / p.T) * p.maxP + pg];
    if (phys < 0) phys = 0;
    if (phys >= p.num_blocks) phys = static_cast<int32_t>(p.num_blocks - 1);
    const int64_t base = (static_cast<int64_t>(phys) * p.P + (tok0 - pg * p.P)) * kW;
    const int whole = (first >= g0 && incl[r] <= g1) ? 1 : 0;
    tl[t] = i32x4{static_cast<int>(base & 0xFFFFFFFF), static_cast<int>(base >> 32),
                  min(kShTokens, re[r] - tok0) | (whole << 16), r};
    if (tir == 0 && hg == 0) {
      // This workgroup holds the row's first tile: record its span.
      p.meta[2 * r] = w;
      p.meta[2 * r + 1] = wg_of(incl[r] - 1) - w + 1;
    }
  }
  // Rows with no tile: zeros from workgroup (row % wgs), meta {0, 0}.
  for (int r = w; r < rows; r += p.wgs) {
    if (rt[r] != 0) continue;
    for (int i = tid; i < kHeads * kDc / 8; i += kShThreads) {
      const int hh = h0 + i / (kDc / 8);
      if (hh < p.H)
        *reinterpret_cast<u32x4*>(static_cast<S*>(p.out) + (static_cast<int64_t>(r) * p.H + hh) * kDc +
                                  8 * (i % (kDc / 8))) = u32x4{0u, 0u, 0u, 0u};
    }
    if (hg == 0 && tid == 0) {
      p.meta[2 * r] = 0;
      p.meta[2 * r + 1] = 0;
    }
  }
  __syncthreads();
  // Compact the tiles (wave 0).
  if (wv == 0) {
    int count = 0;
    for (int base = 0; base < npos; base += 64) {
      const int t = base + lane;
      const i32x4 e = t < npos ? tl[t] : i32x4{0, 0, 0, -1};
      const bool real = e[3] >= 0;
      const uint64_t bal = __ballot(real);
      const int before = __popcll(bal & ((uint64_t{1} << lane) - 1));
      if (real) ctl[count + before] = e;
      count += __popcll(bal);
    }
    if (lane == 0) *nreal = count;
    // Placeholders past the last tile: the cache's first row, no query row.
    if (lane < kShCtlPad) ctl[count + lane] = i32x4{0, 0, 1, -1};
  }
  __syncthreads();
  const int n = *nreal;
  __syncthreads();  // every wave has read the count before the ring is written
  if (n == 0) return;  // whole workgroup: uniform
  QD_MLA_STAMP(0, st_entry);
  QD_MLA_STAMP(1, __builtin_amdgcn_s_memrealtime());

  // --- Main loop ------------------------------------------------------------
  // DMA of tile t from its list entry e (past the end a placeholder: a
  // re-read of the cache's first row into the unused slot, so every step
  // issues the same loads).
  // Instruction k < 8 loads latent row 8 wv + k, instruction 8 the rope
  // bytes of rows 8 wv .. 8 wv + 7.
  auto dma_one = [&](int t, const i32x4 e, int k) {
    char* slot = ring + (t % kShBufs) * kShTileBytes;
    const int64_t base = static_cast<int64_t>(static_cast<uint32_t>(e[0])) | (static_cast<int64_t>(e[1]) << 32);
    const int nv = e[2] & 0xFFFF;
    const char* tb = cache + 2 * base;
    if (k < 8) {
      const int R = 8 * wv + k;
      const int Rc = R < nv ? R : nv - 1;
      const char* src = tb + Rc * kShRowBytes + 16 * lane;
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src),
                                       (__attribute__((address_space(3))) void*)(slot + R * kShLatStride), 16, 0,
                                       NT ? 2 : 0);
    } else {
      const int R = 8 * wv + (lane >> 3);
      const int Rc = R < nv ? R : nv - 1;
      const int c = (lane & 7) ^ ((R >> 1) & 7);
      const char* src = tb + Rc * kShRowBytes + 2 * kDc + 16 * c;
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src),
                                       (__attribute__((address_space(3))) void*)(slot + kShLatBytes + wv * 1024), 16,
                                       0, NT ? 2 : 0);
    }
  };
  auto dma = [&](int t, const i32x4 e) {
#pragma unroll
    for (int k = 0; k < kShDma; ++k) dma_one(t, e, k);
  };
  // This lane's head's query, 18 chunks of 32 elements ([q | q_rope]).
  // Heads past H read head 0's query (never stored; no select on the loaded
  // values, which would wait for every load in flight).
  u32x4 qv[18];
  auto load_q = [&](int r) {
    const int64_t hr = static_cast<int64_t>(r) * p.H + (h < p.H ? h : 0);
    const char* qrow = static_cast<const char*>(p.q) + hr * kDc * 2;
    const char* rrow = static_cast<const char*>(p.qr) + hr * (kW - kDc) * 2;
#pragma unroll
    for (int c = 0; c < 18; ++c)
      qv[c] = c < 16 ? *reinterpret_cast<const u32x4*>(qrow + (32 * c + 8 * q4) * 2)
                     : *reinterpret_cast<const u32x4*>(rrow + (32 * (c - 16) + 8 * q4) * 2);
  };

  float m_run = -INFINITY, l_run = 0.f;
  f32x4 acc[kShColBlocks];  // acc[cb][i]: this lane's head, latent column 16 cb + 4 q4 + i
  auto reset = [&]() {
    m_run = -INFINITY;
    l_run = 0.f;
#pragma unroll
    for (int cb = 0; cb < kShColBlocks; ++cb) acc[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  };

  // The first tiles in flight and the first query, waited for here so that
  // no register load is pending when the loop starts (the compiler would
  // otherwise wait for every load in flight, the whole ring, in every step).
#pragma unroll
  for (int t = 0; t < kShBufs - 1; ++t) dma(t, ctl[t]);
  load_q(ctl[0][3]);
  // List entries are read one step ahead of their use (an LDS round trip
  // at the top of each step would sit on the critical path): e_cur = tile
  // t, r_nxt = row of tile t + 1, e_dma = tile t + kShBufs - 1.
  i32x4 e_cur = ctl[0], e_dma = ctl[kShBufs - 1];
  int r_nxt = ctl[1][3];
  wait_vm_all();
  QD_MLA_STAMP(2, __builtin_amdgcn_s_memrealtime());
  int row = -1;
  for (int t = 0; t < n; ++t) {
    dma_ring_barrier<(kShBufs - 2) * kShDma>();  // tile t in LDS; tile t-1 done by every wave
    const i32x4 ed = e_dma;                       // tile t + kShBufs - 1, into tile t-1's slot
    const i32x4 e = e_cur;
    const int r1 = r_nxt;
    e_cur = ctl[t + 1];
    r_nxt = ctl[t + 2][3];
    e_dma = ctl[t + kShBufs];
    const int nv = e[2] & 0xFFFF;
    const bool whole = (e[2] >> 16) != 0;
    const int r = e[3];
    const bool last = r1 != r;
    if (r != row) {
      row = r;
      reset();
    }
    const char* slot = ring + (t % kShBufs) * kShTileBytes;

    // QK for both 16-row blocks together (two MFMAs per chunk, one per
    // block), operands read kAhead chunks ahead: one chunk's MFMAs take 32
    // cycles, an LDS read under this load well over 100.  The scheduling
    // barriers keep that distance (left free, the scheduler sinks each read
    // next to its MFMA).
    f32x4 s[2];
    {
      const char* lat = slot + r16 * kShLatStride + 16 * q4;
      const char* rop = slot + kShLatBytes + r16 * 128;
      auto a_chunk = [&](int c, int tb) {
        if (c < 16) return *reinterpret_cast<const u32x4*>(lat + 16 * kShLatStride * tb + 64 * c);
        return *reinterpret_cast<const u32x4*>(rop + 16 * 128 * tb + 16 * ((4 * (c - 16) + q4) ^ ((r16 >> 1) & 7)));
      };
      constexpr int kAhead = QD_MLA_SHARED_QK_AHEAD;
      u32x4 a[kAhead][2];
#pragma unroll
      for (int c = 0; c < kAhead; ++c) {
        a[c][0] = a_chunk(c, 0);
        a[c][1] = a_chunk(c, 1);
      }
      __builtin_amdgcn_sched_barrier(0);
      s[0] = s[1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 18; ++c) {
        const u32x4 a0 = a[c % kAhead][0], a1 = a[c % kAhead][1];
        if (c + kAhead < 18) {
          a[c % kAhead][0] = a_chunk(c + kAhead, 0);
          a[c % kAhead][1] = a_chunk(c + kAhead, 1);
        }
        s[0] = Ops::mma32(a0, qv[c], s[0]);
        s[1] = Ops::mma32(a1, qv[c], s[1]);
        // The next tile's DMA, one instruction per chunk: issued together
        // after the barrier, the four waves' loads queue on the CU's load
        // path for about as long as the QK products take.
        if (c < kShDma) dma_one(t + kShBufs - 1, ed, c);
        __builtin_amdgcn_sched_barrier(0);
      }
    }

    // The first PV operand reads, in flight during the softmax (inline asm,
    // TrRead: the builtin form would wait for the next tiles' DMA, issued
    // during QK).
    const uint32_t trb = lds_addr(slot) + (4 * q4 + (r16 >> 2)) * kShLatStride + 8 * (r16 & 3);
    u32x2 av[kShPvAhead][2];
    static_for<0, kShPvAhead>([&](auto c) {
      constexpr int cb = decltype(c)::value;
      TrRead<32 * cb>::issue(trb, av[cb][0]);
      TrRead<16 * kShLatStride + 32 * cb>::issue(trb, av[cb][1]);
    });

    // Softmax over the tile's 32 tokens: lane holds tokens 16 tb + 4 q4 + i.
    // Rows past the visible count hold a copy of the last visible row (the
    // DMA clamps them), so their scores cannot raise the max: only their
    // weights are zeroed, and only in a tile with such rows.
    float x[2][4];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      const f32x4 st = s[tb];
#pragma unroll
      for (int i = 0; i < 4; ++i) x[tb][i] = st[i] * p.sl2;
    }
    float mx = fmaxf(fmaxf(fmaxf(x[0][0], x[0][1]), fmaxf(x[0][2], x[0][3])),
                     fmaxf(fmaxf(x[1][0], x[1][1]), fmaxf(x[1][2], x[1][3])));
    mx = max_over_lane_groups(mx);
    if (__ballot(mx > m_run + kWaveLazyLog2)) {
      const float mn = fmaxf(m_run, mx);
      const float alpha = mn == m_run ? 1.f : fast_exp2(m_run - mn);  // m_run = -inf: 0
      m_run = mn;
      l_run *= alpha;
#pragma unroll
      for (int cb = 0; cb < kShColBlocks; ++cb) acc[cb] *= alpha;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    u32x4 pbl[2];
    u32x2 pb[2];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      float pr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) pr[i] = fast_exp2(x[tb][i] - m_use);
      if (nv < kShTokens) {  // uniform
#pragma unroll
        for (int i = 0; i < 4; ++i) pr[i] = 16 * tb + 4 * q4 + i < nv ? pr[i] : 0.f;
      }
      pb[tb] = u32x2{Ops::pack2(pr[0], pr[1]), Ops::pack2(pr[2], pr[3])};
      pbl[tb] = u32x4{pb[tb][0], pb[tb][1], 0u, 0u};
      if constexpr (Ops::kSplitWeights) {
        pbl[tb][2] = Ops::rest2(pr[0], pr[1], pb[tb][0]);
        pbl[tb][3] = Ops::rest2(pr[2], pr[3], pb[tb][1]);
        l_run += (pr[0] + pr[1]) + (pr[2] + pr[3]);
      } else {
        l_run += Ops::sum2(pb[tb][0]) + Ops::sum2(pb[tb][1]);
      }
    }

    // PV: one 16x16x32 per 16-column block cb over the tile's 32 tokens: k =
    // 8 q4 + e is token 4 q4 + e of row block 0 for e < 4 and of row block 1
    // for e >= 4, in A and in B (the lane's own weights); bf16 adds the lo
    // weights with a second MFMA on the same A.  A = V^T for columns 16 cb ..
    // 16 cb + 15 comes from two transposing LDS reads (ds_read_b64_tr_b16):
    // within each 16-lane group, result lane j element t is element j % 4 of
    // what source lane 4 t + j / 4 addressed, so source lane (t, u) = (l16 /
    // 4, l16 % 4) of group q4 addresses row 16 h + 4 q4 + t, columns 16 cb + 4
    // u .. + 3, and lane j receives column 16 cb + j at tokens 16 h + 4 q4 +
    // 0..3.  C tile cb: lane (head r16, q4) holds columns 16 cb + 4 q4 + i.
    // Reads run kShPvAhead blocks ahead of their MFMAs.
    const u32x4 bhi = {pb[0][0], pb[0][1], pb[1][0], pb[1][1]};
    const u32x4 blo = {pbl[0][2], pbl[0][3], pbl[1][2], pbl[1][3]};
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, kShColBlocks>([&](auto c) {
      constexpr int cb = decltype(c)::value;
      constexpr int j = cb % kShPvAhead;
      // LDS reads issued after this block's two: the later blocks in flight.
      constexpr int later = 2 * (kShColBlocks - 1 - cb < kShPvAhead - 1 ? kShColBlocks - 1 - cb : kShPvAhead - 1);
      lds_wait_tied<later>(av[j][0], av[j][1]);
      const u32x4 a = {av[j][0][0], av[j][0][1], av[j][1][0], av[j][1][1]};
      if constexpr (cb + kShPvAhead < kShColBlocks) {
        TrRead<32 * (cb + kShPvAhead)>::issue(trb, av[j][0]);
        TrRead<16 * kShLatStride + 32 * (cb + kShPvAhead)>::issue(trb, av[j][1]);
      }
      acc[cb] = Ops::mma32(a, bhi, acc[cb]);
      if constexpr (Ops::kSplitWeights) acc[cb] = Ops::mma32(a, blo, acc[cb]);
      __builtin_amdgcn_sched_barrier(0);
    });

    if (last) {
      [[maybe_unused]] const uint64_t st_re0 = QD_MLA_STAMPS_ON ? __builtin_amdgcn_s_memtime() : 0;
      // This wave's heads for the row segment, then the next row's query;
      // one wait covers the stores, the query and the tiles in flight.
      const float Lt = sum_over_lane_groups(l_run);
      if (h < p.H) {
        if (whole) {
          const float inv = Lt > 0.f ? 1.f / Lt : 0.f;
          S* orow = static_cast<S*>(p.out) + (static_cast<int64_t>(r) * p.H + h) * kDc;
#pragma unroll
          for (int cb = 0; cb < kShColBlocks; ++cb)
            *reinterpret_cast<u32x2*>(orow + 16 * cb + 4 * q4) =
                u32x2{Ops::pack2(acc[cb][0] * inv, acc[cb][1] * inv), Ops::pack2(acc[cb][2] * inv, acc[cb][3] * inv)};
        } else {
          // Half-precision partial (kHalfHeader): acc / s_k in fp16, s_k the
          // largest |acc| of the head's 128-column block k (the 4 lanes q4 of
          // r16 hold it): every value lies in [-1, 1] and keeps 11 bits
          // relative to s_k, half the bytes of fp32.
          float sk[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            float amax = 0.f;
#pragma unroll
            for (int cb = 8 * k; cb < 8 * k + 8; ++cb)
              amax = fmaxf(amax, fmaxf(fmaxf(fabsf(acc[cb][0]), fabsf(acc[cb][1])),
                                       fmaxf(fabsf(acc[cb][2]), fabsf(acc[cb][3]))));
            amax = fmaxf(amax, __shfl_xor(amax, 16));
            amax = fmaxf(amax, __shfl_xor(amax, 32));
            sk[k] = half_partial_scale(amax);
          }
          float* pr = p.part + ((static_cast<int64_t>(w) + r) * p.H + h) * static_cast<int64_t>(kHalfPst);
          if (q4 == 0) {
            *reinterpret_cast<f32x4*>(pr) = f32x4{m_run == -INFINITY ? -INFINITY : m_run * kLn2, Lt, sk[0], sk[1]};
            *reinterpret_cast<f32x4*>(pr + 4) = f32x4{sk[2], sk[3], 0.f, 0.f};
          }
          char* pa = reinterpret_cast<char*>(pr + kHalfHeader) + 8 * q4;
#pragma unroll
          for (int cb = 0; cb < kShColBlocks; ++cb) {
            const float isc = 1.f / sk[cb / 8];
            *reinterpret_cast<u32x2*>(pa + 32 * cb) =
                u32x2{pack_f16_rne(acc[cb][0] * isc, acc[cb][1] * isc), pack_f16_rne(acc[cb][2] * isc, acc[cb][3] * isc)};
          }
        }
      }
      if (t + 1 < n) load_q(r1);
      wait_vm_all();
      if constexpr (QD_MLA_STAMPS_ON) {
        st_rowend += __builtin_amdgcn_s_memtime() - st_re0;
        ++st_rowends;
      }
    }
  }
  QD_MLA_STAMP(3, __builtin_amdgcn_s_memrealtime());
  QD_MLA_STAMP(9, __builtin_amdgcn_s_memtime());
  // Drain the placeholder loads before the workgroup's LDS is released.
  __builtin_amdgcn_s_waitcnt(0);
#ifdef QD_STAMPS
  QD_MLA_STAMP(4, __builtin_amdgcn_s_memrealtime());
  QD_MLA_STAMP(5, mla_xcc());
  QD_MLA_STAMP(6, static_cast<uint64_t>(n));
  QD_MLA_STAMP(7, st_rowend);
  QD_MLA_STAMP(8, st_clk0);
  QD_MLA_STAMP(10, static_cast<uint64_t>(w));
  QD_MLA_STAMP(11, static_cast<uint64_t>(hg));
  QD_MLA_STAMP(12, static_cast<uint64_t>(st_rowends));
#endif
}

// ----------------------------------------------------------------------------
// Merge of the stream-K partials: one wave per (row, head) of a row split
// across workgroups (meta[row] = {first, count >= 2}); the partial of
// workgroup k is in slot k + row, for the k in [first, first + count) whose
// tile range is not empty (with fewer tiles than workgroups some are).  The
// partials are folded in workgroup order with the log-sum-exp merge of
// online_softmax.cuh:17-24 (empty partials skipped, an all-empty row gives
// zeros), kBatch of them loaded per memory round trip: one trip after the
// meta entry covers a typical row.
//
// HALF: half-precision rows of the shared-tile and wave kernels
// (kHalfHeader, Dc = 512); lane j folds columns 8 j .. 8 j + 7 (one 16-byte
// load per row and one store).
template <int DT, bool HALF>
__global__ __launch_bounds__(256) void mla_merge_sk_kernel(MlaParams p) {
  using E = Elem<DT>;
  using S = typename E::S;
  constexpr int kAcc = 8;
  constexpr int kBatch = 8;
  const int lane = threadIdx.x & 63;
  const int64_t wid = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (wid >= static_cast<int64_t>(p.B) * p.T * p.H) return;
  const int64_t r = wid / p.H;
  const int h = static_cast<int>(wid % p.H);
  const int first = p.meta[2 * r], nwg = p.meta[2 * r + 1];
  if (nwg < 2 || first < 0 || first + nwg > p.wgs) return;  // spans are always inside [0, wgs)
  const int64_t G = *p.gtotal;
  const int64_t stride = static_cast<int64_t>(p.H) * p.pst;
  const float* base = p.part + (r * p.H + h) * static_cast<int64_t>(p.pst);  // slot k: + (k) * stride
  const int aoff = p.pst - p.Dc;                                             // accumulator offset
  // Workgroup k's range [k G / wgs, (k + 1) G / wgs) holds a partial row
  // when it is not empty, which it never is for G >= wgs.
  const bool dense = G >= p.wgs;
  auto present = [&](int k) {
    return dense || static_cast<int64_t>(k) * G / p.wgs != static_cast<int64_t>(k + 1) * G / p.wgs;
  };
  float M = -INFINITY, L = 0.f;
  float acc[kAcc];
#pragma unroll
  for (int j = 0; j < kAcc; ++j) acc[j] = 0.f;
  for (int c = 0; c < nwg; c += kBatch) {
    float ms[kBatch], ls[kBatch], v[kBatch][kAcc];
#pragma unroll
    for (int t = 0; t < kBatch; ++t) {
      ms[t] = -INFINITY;
      ls[t] = 0.f;
#pragma unroll
      for (int j = 0; j < kAcc; ++j) v[t][j] = 0.f;
      const int k = first + c + t;
      if (c + t < nwg && present(k)) {  // wave-uniform
        const float* pr = base + k * stride;
        if constexpr (HALF) {
          const f32x4 hd = *reinterpret_cast<const f32x4*>(pr);
          const f32x4 hs = *reinterpret_cast<const f32x4*>(pr + 4);
          const f16x8 hv = *reinterpret_cast<const f16x8*>(reinterpret_cast<const char*>(pr + kHalfHeader) + 16 * lane);
          ms[t] = hd[0];
          ls[t] = hd[1];
          // Lane j holds columns 8 j .. 8 j + 7, of block j / 16.
          const int kb = lane >> 4;
          const float sc = kb == 0 ? hd[2] : kb == 1 ? hd[3] : kb == 2 ? hs[0] : hs[1];
#pragma unroll
          for (int j = 0; j < kAcc; ++j) v[t][j] = static_cast<float>(hv[j]) * sc;
        } else {
          ms[t] = pr[0];
          ls[t] = pr[1];
#pragma unroll
          for (int j = 0; j < kAcc; ++j) {
            const int d = lane + 64 * j;
            if (d < p.Dc) v[t][j] = pr[aoff + d];
          }
        }
      }
    }
#pragma unroll
    for (int t = 0; t < kBatch; ++t) {
      if (ls[t] == 0.f) continue;  // absent or empty partial
      lse_fold(M, L, acc, ms[t], ls[t], v[t]);
    }
  }
  S* orow = static_cast<S*>(p.out) + wid * p.Dc;
  const float inv = L > 0.f ? 1.f / L : 0.f;
  if constexpr (HALF) {
    S o[kAcc];
#pragma unroll
    for (int j = 0; j < kAcc; ++j) o[j] = E::from_f(acc[j] * inv);
    *reinterpret_cast<u32x4*>(orow + 8 * lane) = __builtin_bit_cast(u32x4, o);
  } else {
#pragma unroll
    for (int j = 0; j < kAcc; ++j) {
      const int d = lane + 64 * j;
      if (d < p.Dc) orow[d] = E::from_f(acc[j] * inv);
    }
  }
}

// Any dtype/shape (mla.cu:34-82 on the VALU): one wave per (row, head,
// split), one token per step, lanes over the W columns of the cache row.
template <int DT>
__global__ __launch_bounds__(256) void mla_attend_generic_kernel(MlaParams p) {
  using E = Elem<DT>;
  using S = typename E::S;
  constexpr int kAcc = 8;  // Dc <= 512 = 8 * 64
  const int lane = threadIdx.x & 63;
  const int64_t wid = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t per_row = static_cast<int64_t>(p.H) * p.splits;
  if (wid >= static_cast<int64_t>(p.B) * p.T * per_row) return;
  const int64_t r = wid / per_row;
  const int h = static_cast<int>((wid / p.splits) % p.H);
  const int s = static_cast<int>(wid % p.splits);
  const int b = static_cast<int>(r / p.T);
  const int end = row_end(p, b, r);
  const int count = p.nk >= 0 ? p.nk : end;
  int i0, i1;
  split_range(count, s, p.splits, i0, i1);

  const S* qrow = static_cast<const S*>(p.q) + (r * p.H + h) * p.Dc;
  const S* rrow = static_cast<const S*>(p.qr) + (r * p.H + h) * p.Dr;
  const S* cache = static_cast<const S*>(p.cache);
  float m_run = -INFINITY, l_run = 0.f;
  float acc[kAcc];
#pragma unroll
  for (int j = 0; j < kAcc; ++j) acc[j] = 0.f;
  for (int i = i0; i < i1; ++i) {
    const int tok = p.nk >= 0 ? p.idx[r * p.nk + i] : i;
    if (tok < 0 || tok >= end) continue;
    const S* row = cache + token_offset(p, b, tok);
    float cv[kAcc];
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < kAcc; ++j) {
      const int d = lane + 64 * j;
      cv[j] = d < p.Dc ? E::to_f(row[d]) : 0.f;
      if (d < p.Dc) dot = fmaf(E::to_f(qrow[d]), cv[j], dot);
    }
    for (int d = lane; d < p.Dr; d += 64) dot = fmaf(E::to_f(rrow[d]), E::to_f(row[p.Dc + d]), dot);
    const float x = wave_sum(dot) * p.sl2;
    const float m_new = fmaxf(m_run, x);
    const float alpha = l_run == 0.f ? 0.f : fast_exp2(m_run - m_new);
    const float pw = fast_exp2(x - m_new);
    l_run = alpha * l_run + pw;
    m_run = m_new;
#pragma unroll
    for (int j = 0; j < kAcc; ++j) acc[j] = alpha * acc[j] + pw * cv[j];
  }
  if (p.splits == 1) {
    S* orow = static_cast<S*>(p.out) + (r * p.H + h) * p.Dc;
    const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
#pragma unroll
    for (int j = 0; j < kAcc; ++j) {
      const int d = lane + 64 * j;
      if (d < p.Dc) orow[d] = E::from_f(acc[j] * inv);
    }
  } else {
    float* pr = partial_row(p, r, h, s);
    if (lane == 0) {
      pr[0] = m_run == -INFINITY ? -INFINITY : m_run * kLn2;
      pr[1] = l_run;
    }
#pragma unroll
    for (int j = 0; j < kAcc; ++j) {
      const int d = lane + 64 * j;
      if (d < p.Dc) pr[2 + d] = acc[j];
    }
  }
}

// Log-sum-exp merge of [R, H, splits, Dc+2] partials (mla.cu:75-82, rule
// of online_softmax.cuh:17-24): one wave per (row, head), splits folded in
// order, empty partials skipped, an all-empty row gives zeros.
template <int DT>
__global__ __launch_bounds__(256) void mla_merge_kernel(MlaParams p) {
  using E = Elem<DT>;
  using S = typename E::S;
  constexpr int kAcc = 8;
  const int lane = threadIdx.x & 63;
  const int64_t wid = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t nrows = static_cast<int64_t>(p.B) * p.T * p.H;
  if (wid >= nrows) return;
  const float* base = p.part + wid * p.splits * static_cast<int64_t>(p.Dc + 2);
  float M = -INFINITY, Lsum = 0.f;
  float acc[kAcc];
#pragma unroll
  for (int j = 0; j < kAcc; ++j) acc[j] = 0.f;
  for (int s = 0; s < p.splits; ++s) {
    const float* pr = base + s * static_cast<int64_t>(p.Dc + 2);
    const float ms = pr[0], ls = pr[1];
    if (ls == 0.f) continue;
    const float mn = fmaxf(M, ms);
    const float a = Lsum == 0.f ? 0.f : fast_exp2((M - mn) * kLog2e);
    const float bb = fast_exp2((ms - mn) * kLog2e);
    Lsum = a * Lsum + bb * ls;
    M = mn;
#pragma unroll
    for (int j = 0; j < kAcc; ++j) {
      const int d = lane + 64 * j;
      if (d < p.Dc) acc[j] = a * acc[j] + bb * pr[2 + d];
    }
  }
  S* orow = static_cast<S*>(p.out) + wid * p.Dc;
  const float inv = Lsum > 0.f ? 1.f / Lsum : 0.f;
#pragma unroll
  for (int j = 0; j < kAcc; ++j) {
    const int d = lane + 64 * j;
    if (d < p.Dc) orow[d] = E::from_f(acc[j] * inv);
  }
}

// ----------------------------------------------------------------------------
// Host side
// ----------------------------------------------------------------------------

int mla_fail(char* msg, size_t cap, const char* text) {
  qd_set_last_error(QD_ERR_INVALID_VALUE, text);
  if (msg && cap) {
    size_t n = strlen(text);
    if (n >= cap) n = cap - 1;
    memcpy(msg, text, n);
    msg[n] = '\0';
  }
  return QD_ERR_INVALID_VALUE;
}

int mla_ok(char* msg, size_t cap) {
  if (msg && cap) msg[0] = '\0';
  return QD_OK;
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    qd_set_last_error(static_cast<int>(e), std::string(what) + " kernel launch failed: " + hipGetErrorString(e));
    return static_cast<int>(e);
  }
  return QD_OK;
}

// The reference's check(): contiguous CUDA tensor on `base`'s device.
bool placed(const qd_tensor_desc* x, const qd_tensor_desc* base) {
  return x->defined && x->is_device && x->contiguous && x->device_index == base->device_index;
}

bool float_dtype(int dt) { return dt == QD_DTYPE_F32 || dt == QD_DTYPE_F16 || dt == QD_DTYPE_BF16; }

int elem_size(int dt) {
  switch (dt) {
    case QD_DTYPE_F32: return 4;
    case QD_DTYPE_F16:
    case QD_DTYPE_BF16: return 2;
    default: return 0;
  }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

int device_max_lds() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 65536;
  if (cached[dev] == 0) {
    int bytes = 0;
    if (hipDeviceGetAttribute(&bytes, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
        bytes <= 0)
      bytes = 65536;
    cached[dev] = bytes;
  }
  return cached[dev];
}

// Shape of one attention call.
struct AttendShape {
  int B, T, H, Dc, Dr, P, maxP, nk, dtype;
};

// Launch plan of the attention.  VALU kernel: context splits per row.
// MFMA kernel: stream-K ranges (workgroups per head group), head tiles per
// workgroup and latent slices per head tile, DMA chunks per thread.  Depends
// on static shapes and the device only.
struct AttendPlan {
  bool mfma;
  int nblk, cpt, kch, head_groups, nht, ds, wgs;
  size_t lds;
  int splits;  // VALU kernel
  bool wave;   // MFMA path through mla_attend_wave_kernel
  bool shared;  // MFMA path through mla_attend_shared_kernel
};

// Smallest instantiated DMA-chunk count covering ceil(W/64), 0 if none.
int cpt_for(int W) {
  const int need = (W + 63) / 64;
  for (int c : {2, 5, 9, 10})
    if (need <= c) return c;
  return 0;
}

AttendPlan plan_attend(const AttendShape& a, int forced, int flags) {
  AttendPlan pl{};
  const int W = a.Dc + a.Dr;
  pl.nblk = (a.Dc + 127) / 128;
  pl.kch = (W + 31) / 32;
  pl.cpt = cpt_for(W);
  pl.lds = pl.cpt ? mla_mfma_lds_bytes(pl.cpt) : 0;
  const int ht = (a.H + 15) / 16;
  // 4 waves = head tiles x latent slices: one head tile split 4 ways for up
  // to 16 heads, else 2 head tiles split 2 ways.
  if (ht == 1) {
    pl.nht = 1;
    pl.ds = 4;
  } else {
    pl.nht = 2;
    pl.ds = 2;
  }
  pl.head_groups = (ht + pl.nht - 1) / pl.nht;
  pl.mfma = (flags & QD_FLAG_FORCE_GENERIC) == 0 && (a.dtype == QD_DTYPE_F16 || a.dtype == QD_DTYPE_BF16) &&
            a.Dc % 8 == 0 && a.Dr % 8 == 0 && a.Dc <= 512 && pl.cpt > 0 &&
            pl.lds <= static_cast<size_t>(device_max_lds());
  const int64_t rows = static_cast<int64_t>(a.B) * a.T;
  if (pl.mfma) {
    // One resident workgroup per CU (the LDS ring), shared by the head groups.
    pl.wgs = forced > 0 ? forced : std::max(1, device_cus() / pl.head_groups);
    pl.splits = 1;
    // The wave-streamed kernel: dense rows, Dc 512 / Dr 64 (instantiated),
    // pages of whole 16-token tiles, rows and tiles per workgroup within its
    // LDS lists.  Each group of 16 heads is a workgroup of its own over the
    // same tile range, on the same XCD (shared L2), one per CU in all.
    const int64_t gmax =
        rows * ((static_cast<int64_t>(a.maxP) * a.P + kSubTokens - 1) / kSubTokens + kWaveRowCost);
    const size_t wlds = mla_wave_lds_bytes(4, 2);
    // The shared-tile kernel: the same dense shapes with 64 heads or more
    // and pages of whole 32-token tiles, 64 heads per workgroup of four
    // waves, one workgroup per CU.
    const size_t slds = mla_shared_lds_bytes();
    const bool dense512 = a.Dc == 512 && a.Dr == 64 && a.nk < 0 && a.P % kSubTokens == 0;
    if ((flags & (QD_FLAG_MLA_STAGED | QD_FLAG_MLA_WAVE)) == 0 && dense512 && a.P % kShTokens == 0 && a.H >= 64 &&
        rows <= kShRows && slds <= static_cast<size_t>(device_max_lds())) {
      const int groups = (a.H + 63) / 64;
      const int wgs = forced > 0 ? forced : std::max(1, device_cus() / groups);
      const int64_t smax =
          rows * ((static_cast<int64_t>(a.maxP) * a.P + kShTokens - 1) / kShTokens + kShRowCost);
      if ((smax + wgs - 1) / wgs + 1 <= kShListTiles) {
        pl.shared = true;
        pl.nht = 1;
        pl.head_groups = groups;
        pl.wgs = wgs;
        pl.lds = slds;
      }
    }
    if (!pl.shared && (flags & QD_FLAG_MLA_STAGED) == 0 && dense512 && rows <= kWaveRows &&
        wlds <= static_cast<size_t>(device_max_lds())) {
      const int groups = ht;
      const int wgs = forced > 0 ? forced : std::max(1, device_cus() / groups);
      if ((gmax + wgs - 1) / wgs + 1 <= kWaveListTiles) {
        pl.wave = true;
        pl.nht = 1;
        pl.head_groups = groups;
        pl.wgs = wgs;
        pl.lds = wlds;
      }
    }
  } else if (forced > 0) {
    pl.splits = forced;
  } else {
    // Two resident workgroups per CU, at least 256 listed tokens per split,
    // at most kMaxSplits.
    const int64_t cap = a.nk >= 0 ? a.nk : static_cast<int64_t>(a.maxP) * a.P;
    const int64_t per_row = (static_cast<int64_t>(a.H) + 3) / 4;
    const int64_t target = 2 * static_cast<int64_t>(device_cus());
    const int64_t want = (target + rows * per_row - 1) / (rows * per_row);
    int64_t sp = std::min<int64_t>(want, std::max<int64_t>(1, cap / 256));
    pl.splits = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(sp, kMaxSplits)));
  }
  return pl;
}

size_t round_up256(size_t x) { return (x + 255) / 256 * 256; }

// Workspace of the attention: VALU kernel [R, H, splits, Dc+2] fp32 when
// splits > 1; MFMA kernel [wgs + R, H, Dc+2] fp32 partials, then the tile
// count G (int64) and [R][2] int32 row spans.
// Floats per stream-K partial row: {m, l, acc[Dc]}, or {m, l, pad, pad,
// acc[Dc]} for the shared-tile kernel (16-byte accumulator stores).
// Floats per partial row: the half-precision rows of the shared-tile and
// wave kernels (kHalfPst), the staged kernel's {m, l} + Dc fp32.
bool half_partials(const AttendPlan& pl) { return pl.shared || pl.wave; }
int partial_stride(const AttendShape& a, const AttendPlan& pl) {
  return half_partials(pl) ? kHalfPst : a.Dc + 2;
}

size_t attend_partial_bytes(const AttendShape& a, const AttendPlan& pl) {
  const int64_t rows = static_cast<int64_t>(a.B) * a.T;
  if (pl.mfma)
    return round_up256(static_cast<size_t>(pl.wgs + rows) * a.H * partial_stride(a, pl) * sizeof(float)) +
           round_up256(sizeof(int64_t) + static_cast<size_t>(rows) * 2 * sizeof(int));
  if (pl.splits <= 1) return 0;
  return static_cast<size_t>(rows) * a.H * pl.splits * (a.Dc + 2) * sizeof(float);
}

template <int DT, int DS, int CPT>
hipError_t launch_attend_mfma(const MlaParams& prm, const AttendPlan& pl, int64_t grid, hipStream_t st) {
  auto fn = mla_attend_mfma_kernel<DT, DS, CPT>;
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [&] {
    attr = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                               static_cast<int>(mla_mfma_lds_bytes(CPT)));
  });
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(grid)), dim3(64 * pl.nht * pl.ds), pl.lds, st, prm);
  return hipSuccess;
}

template <int DT, bool NT>
hipError_t launch_attend_wave(const MlaParams& prm, const AttendPlan& pl, int64_t grid, hipStream_t st) {
  auto fn = mla_attend_wave_kernel<DT, 4, 2, NT>;
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [&] {
    attr = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                               static_cast<int>(mla_wave_lds_bytes(4, 2)));
  });
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(grid)), dim3(kAttendThreads), pl.lds, st, prm);
  return hipSuccess;
}

template <int DT, bool NT>
hipError_t launch_attend_shared(const MlaParams& prm, const AttendPlan& pl, int64_t grid, hipStream_t st) {
  auto fn = mla_attend_shared_kernel<DT, NT>;
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [&] {
    attr = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                               static_cast<int>(mla_shared_lds_bytes()));
  });
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(grid)), dim3(kShThreads), pl.lds, st, prm);
  return hipSuccess;
}

template <int DT>
hipError_t dispatch_attend_mfma(const MlaParams& prm, const AttendPlan& pl, int64_t grid, hipStream_t st) {
  switch (pl.cpt * 8 + pl.ds) {
    case 2 * 8 + 4: return launch_attend_mfma<DT, 4, 2>(prm, pl, grid, st);
    case 2 * 8 + 2: return launch_attend_mfma<DT, 2, 2>(prm, pl, grid, st);
    case 5 * 8 + 4: return launch_attend_mfma<DT, 4, 5>(prm, pl, grid, st);
    case 5 * 8 + 2: return launch_attend_mfma<DT, 2, 5>(prm, pl, grid, st);
    case 9 * 8 + 4: return launch_attend_mfma<DT, 4, 9>(prm, pl, grid, st);
    case 9 * 8 + 2: return launch_attend_mfma<DT, 2, 9>(prm, pl, grid, st);
    case 10 * 8 + 4: return launch_attend_mfma<DT, 4, 10>(prm, pl, grid, st);
    case 10 * 8 + 2: return launch_attend_mfma<DT, 2, 10>(prm, pl, grid, st);
    default: return hipErrorInvalidValue;
  }
}

// Enqueues attention (+ merge) writing [R, H, Dc] of the dtype to `out`.
// Where the stream-K MFMA kernels keep their partial rows, the tile count G
// and the row spans `meta`, inside the partial workspace.
struct PartialRefs {
  float* part;
  int64_t* gtotal;
  int* meta;
};
PartialRefs partial_refs(const AttendShape& a, const AttendPlan& pl, void* part_ws) {
  const int64_t rows = static_cast<int64_t>(a.B) * a.T;
  char* meta =
      static_cast<char*>(part_ws) + round_up256(static_cast<size_t>(pl.wgs + rows) * a.H * partial_stride(a, pl) * 4);
  return {static_cast<float*>(part_ws), reinterpret_cast<int64_t*>(meta), reinterpret_cast<int*>(meta + sizeof(int64_t))};
}

#ifdef QD_STAMPS
uint64_t* g_mla_stamps = nullptr;  // diagnostic build: qd_diag_set_mla_stamps
#endif

// skip_merge: the caller merges the split rows itself (mla_decode's value
// projection, MFMA kernels with half-precision partials only).
int run_attend(const AttendShape& a, const void* q, const void* qr, const void* cache, const int32_t* table,
               const int32_t* lens, const int32_t* pos, const int32_t* idx, int causal, int64_t num_blocks,
               float scale, void* out, void* part_ws, size_t part_bytes, const AttendPlan& pl, hipStream_t st,
               bool skip_merge = false) {
  MlaParams prm{};
#ifdef QD_STAMPS
  prm.stamps = g_mla_stamps;
#endif
  prm.q = q;
  prm.qr = qr;
  prm.cache = cache;
  prm.table = table;
  prm.lens = lens;
  prm.pos = pos;
  prm.idx = idx;
  prm.out = out;
  prm.part = static_cast<float*>(part_ws);
  prm.B = a.B;
  prm.T = a.T;
  prm.H = a.H;
  prm.Dc = a.Dc;
  prm.Dr = a.Dr;
  prm.W = a.Dc + a.Dr;
  prm.P = a.P;
  prm.maxP = a.maxP;
  prm.nk = a.nk;
  prm.causal = causal ? 1 : 0;
  prm.splits = pl.splits;
  prm.head_groups = pl.head_groups;
  prm.kch = pl.kch;
  prm.nht = pl.nht;
  prm.ds = pl.ds;
  prm.wgs = pl.wgs;
  prm.pst = partial_stride(a, pl);
  prm.num_blocks = num_blocks;
  const int64_t rows = static_cast<int64_t>(a.B) * a.T;
  prm.sl2 = scale * kLog2e;
  const size_t need = attend_partial_bytes(a, pl);
  if (need > 0 && (part_bytes < need || !part_ws || !aligned16(part_ws)))
    return mla_fail(nullptr, 0, "workspace too small for the attention partials");
  if (pl.mfma) {
    const PartialRefs pr = partial_refs(a, pl, part_ws);
    prm.gtotal = pr.gtotal;
    prm.meta = pr.meta;
  }
  (void)hipGetLastError();
  hipError_t err = hipSuccess;
  if (pl.mfma) {
    const int64_t grid = (static_cast<int64_t>(pl.wgs) + 7) / 8 * 8 * pl.head_groups;
    if (grid > 2147483647LL) return mla_fail(nullptr, 0, "mla_attend grid exceeds launch limits");
    if (pl.shared && pl.head_groups == 1)
      err = a.dtype == QD_DTYPE_BF16 ? launch_attend_shared<QD_DTYPE_BF16, true>(prm, pl, grid, st)
                                     : launch_attend_shared<QD_DTYPE_F16, true>(prm, pl, grid, st);
    else if (pl.shared)
      err = a.dtype == QD_DTYPE_BF16 ? launch_attend_shared<QD_DTYPE_BF16, false>(prm, pl, grid, st)
                                     : launch_attend_shared<QD_DTYPE_F16, false>(prm, pl, grid, st);
    else if (pl.wave && pl.head_groups == 1)
      err = a.dtype == QD_DTYPE_BF16 ? launch_attend_wave<QD_DTYPE_BF16, true>(prm, pl, grid, st)
                                     : launch_attend_wave<QD_DTYPE_F16, true>(prm, pl, grid, st);
    else if (pl.wave)
      err = a.dtype == QD_DTYPE_BF16 ? launch_attend_wave<QD_DTYPE_BF16, false>(prm, pl, grid, st)
                                     : launch_attend_wave<QD_DTYPE_F16, false>(prm, pl, grid, st);
    else
      err = a.dtype == QD_DTYPE_BF16 ? dispatch_attend_mfma<QD_DTYPE_BF16>(prm, pl, grid, st)
                                     : dispatch_attend_mfma<QD_DTYPE_F16>(prm, pl, grid, st);
  } else {
    const int64_t waves = rows * a.H * pl.splits;
    const int64_t grid = (waves + 3) / 4;
    if (grid > 2147483647LL) return mla_fail(nullptr, 0, "mla_attend grid exceeds launch limits");
    switch (a.dtype) {
      case QD_DTYPE_F32:
        hipLaunchKernelGGL(mla_attend_generic_kernel<QD_DTYPE_F32>, dim3(grid), dim3(256), 0, st, prm);
        break;
      case QD_DTYPE_F16:
        hipLaunchKernelGGL(mla_attend_generic_kernel<QD_DTYPE_F16>, dim3(grid), dim3(256), 0, st, prm);
        break;
      default:
        hipLaunchKernelGGL(mla_attend_generic_kernel<QD_DTYPE_BF16>, dim3(grid), dim3(256), 0, st, prm);
        break;
    }
  }
  if (err != hipSuccess) {
    qd_set_last_error(static_cast<int>(err), std::string("mla_attend launch setup failed: ") + hipGetErrorString(err));
    return static_cast<int>(err);
  }
  int rc = launch_status("mla_attend");
  if (rc != QD_OK || (!pl.mfma && pl.splits == 1) || (skip_merge && pl.mfma && half_partials(pl))) return rc;
  const int64_t mgrid = (rows * a.H + 3) / 4;
  if (pl.mfma) {
    using MergeFn = void (*)(MlaParams);
    MergeFn fn = nullptr;
    if (a.dtype == QD_DTYPE_BF16)
      fn = half_partials(pl) ? mla_merge_sk_kernel<QD_DTYPE_BF16, true> : mla_merge_sk_kernel<QD_DTYPE_BF16, false>;
    else
      fn = half_partials(pl) ? mla_merge_sk_kernel<QD_DTYPE_F16, true> : mla_merge_sk_kernel<QD_DTYPE_F16, false>;
    hipLaunchKernelGGL(fn, dim3(mgrid), dim3(256), 0, st, prm);
    return launch_status("mla_attend merge");
  }
  switch (a.dtype) {
    case QD_DTYPE_F32: hipLaunchKernelGGL(mla_merge_kernel<QD_DTYPE_F32>, dim3(mgrid), dim3(256), 0, st, prm); break;
    case QD_DTYPE_F16: hipLaunchKernelGGL(mla_merge_kernel<QD_DTYPE_F16>, dim3(mgrid), dim3(256), 0, st, prm); break;
    default: hipLaunchKernelGGL(mla_merge_kernel<QD_DTYPE_BF16>, dim3(mgrid), dim3(256), 0, st, prm); break;
  }
  return launch_status("mla_attend merge");
}

// The value projection of mla_decode with the merge of split rows folded in
// (mla_project_mfma_kernel MERGE): the 16-row, 4-chunk-group tiling that
// launch_project picks for small batches with di = 512.
// Half-width column tiles when full ones would leave CUs idle (mla-h16:
// 128 workgroups; each tile's rows are then merged twice, once per half).
template <int DT>
void launch_project_merge(const ProjParams& prm, hipStream_t st) {
  const int64_t col_tiles = (prm.dout + 127) / 128;
  const int64_t row_tiles = (prm.rows + 15) / 16;
  const bool half = col_tiles * prm.H * row_tiles < device_cus();
  const dim3 grid(static_cast<unsigned>(col_tiles * (half ? 2 : 1)), prm.H, static_cast<unsigned>(row_tiles));
  if (half)
    hipLaunchKernelGGL((mla_project_mfma_kernel<DT, false, 1, 4, true, true>), grid, dim3(256), 0, st, prm);
  else
    hipLaunchKernelGGL((mla_project_mfma_kernel<DT, false, 1, 4, true>), grid, dim3(256), 0, st, prm);
}

bool project_mfma_applies(int64_t rows, int di, int dout, int dtype, const void* x, const void* w,
                          const void* out) {
  return (dtype == QD_DTYPE_F16 || dtype == QD_DTYPE_BF16) && di % 32 == 0 && dout % 8 == 0 && dout >= 8 &&
         (rows + 63) / 64 <= 65535 && aligned16(x) && aligned16(w) && aligned16(out);  // grid.z limit
}

template <int DT>
void launch_project(const ProjParams& prm, bool absorb, bool mfma, hipStream_t st) {
  if constexpr (DT != QD_DTYPE_F32) {
    if (mfma) {
      // 64-row workgroups when they already fill the GPU twice over and
      // their row tiles are full, else 16-row ones (grid.z stays within
      // 65535: rows are few then).
      const int64_t col_tiles = (prm.dout + 127) / 128;
      const bool small = (prm.rows < 64 ||
                          col_tiles * prm.H * ((prm.rows + 63) / 64) < 2 * static_cast<int64_t>(device_cus())) &&
                         (prm.rows + 15) / 16 <= 65535;
      const bool long_k = prm.di / 32 >= 16;
      const dim3 grid(static_cast<unsigned>(col_tiles), prm.H,
                      static_cast<unsigned>(small ? (prm.rows + 15) / 16 : (prm.rows + 63) / 64));
      auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, dim3(256), 0, st, prm); };
      if (absorb) {
        if (!small) go(mla_project_mfma_kernel<DT, true, 4, 2>);
        else if (long_k) go(mla_project_mfma_kernel<DT, true, 1, 4>);
        else go(mla_project_mfma_kernel<DT, true, 1, 1>);
      } else {
        if (!small) {
          go(mla_project_mfma_kernel<DT, false, 4, 2>);
        } else if (long_k && col_tiles * prm.H * ((prm.rows + 15) / 16) < device_cus()) {
          // Half-width column tiles: twice the workgroups (same arithmetic).
          const dim3 hgrid(static_cast<unsigned>(2 * col_tiles), prm.H, static_cast<unsigned>((prm.rows + 15) / 16));
          hipLaunchKernelGGL((mla_project_mfma_kernel<DT, false, 1, 4, false, true>), hgrid, dim3(256), 0, st, prm);
        } else if (long_k) {
          go(mla_project_mfma_kernel<DT, false, 1, 4>);
        } else {
          go(mla_project_mfma_kernel<DT, false, 1, 1>);
        }
      }
      return;
    }
  }
  {
    const int64_t n = prm.rows * prm.H * prm.dout;
    const dim3 grid(static_cast<unsigned>((n + 255) / 256));
    if (absorb)
      hipLaunchKernelGGL((mla_project_generic_kernel<DT, true>), grid, dim3(256), 0, st, prm);
    else
      hipLaunchKernelGGL((mla_project_generic_kernel<DT, false>), grid, dim3(256), 0, st, prm);
  }
}

int run_project(const void* x, const void* w, void* out, int64_t rows, int H, int di, int dout, bool absorb,
                int dtype, int flags, hipStream_t st) {
  if (rows < 0 || H <= 0 || di <= 0 || dout <= 0) return mla_fail(nullptr, 0, "invalid projection shape");
  if (!float_dtype(dtype)) return mla_fail(nullptr, 0, "dtype must be float32/float16/bfloat16");
  if (rows == 0) return QD_OK;
  if (!x || !w || !out) return mla_fail(nullptr, 0, "null tensor pointer");
  ProjParams prm{x, w, out, rows, H, di, dout};
  const bool mfma = (flags & QD_FLAG_FORCE_GENERIC) == 0 && project_mfma_applies(rows, di, dout, dtype, x, w, out);
  if (!mfma && (rows * H * static_cast<int64_t>(dout) + 255) / 256 > 2147483647LL)
    return mla_fail(nullptr, 0, "mla_project grid exceeds launch limits");
  (void)hipGetLastError();
  switch (dtype) {
    case QD_DTYPE_F32: launch_project<QD_DTYPE_F32>(prm, absorb, false, st); break;
    case QD_DTYPE_F16: launch_project<QD_DTYPE_F16>(prm, absorb, mfma, st); break;
    default: launch_project<QD_DTYPE_BF16>(prm, absorb, mfma, st); break;
  }
  return launch_status("mla_project");
}

// Workspace of the fused decode: absorbed query and latent output
// ([R, H, Dc] of the dtype each), then the split partials.
struct DecodeLayout {
  size_t qa, latent, part, total;
};

DecodeLayout decode_layout(const AttendShape& a, const AttendPlan& pl) {
  DecodeLayout d{};
  const size_t n = static_cast<size_t>(a.B) * a.T * a.H * a.Dc * elem_size(a.dtype);
  d.qa = 0;
  d.latent = round_up256(n);
  d.part = d.latent + round_up256(n);
  d.total = d.part + attend_partial_bytes(a, pl);
  return d;
}

bool attend_shape_ok(const AttendShape& a) {
  return a.B >= 0 && a.T >= 0 && a.H > 0 && a.Dc > 0 && a.Dc <= 512 && a.Dr > 0 && a.P > 0 && a.maxP > 0 &&
         a.nk >= -1 && float_dtype(a.dtype) && a.B <= 65535 && a.T <= 65535;
}

}  // namespace

extern "C" {

int qd_latent_kv_write_validate(const qd_tensor_desc* latent, const qd_tensor_desc* rope,
                                const qd_tensor_desc* cache, const qd_tensor_desc* slots, char* msg,
                                size_t msg_cap) {
  if (!latent || !rope || !cache || !slots) return mla_fail(msg, msg_cap, "null tensor descriptor");
  if (!placed(latent, latent)) return mla_fail(msg, msg_cap, "latent must be contiguous and on the same CUDA device");
  if (!placed(rope, latent)) return mla_fail(msg, msg_cap, "rope must be contiguous and on the same CUDA device");
  if (!placed(cache, latent)) return mla_fail(msg, msg_cap, "cache must be contiguous and on the same CUDA device");
  if (!placed(slots, latent)) return mla_fail(msg, msg_cap, "slots must be contiguous and on the same CUDA device");
  if (!float_dtype(latent->dtype)) return mla_fail(msg, msg_cap, "dtype must be float32/float16/bfloat16");
  if (!(latent->ndim == 2 && rope->ndim == 2 && cache->ndim == 3 && slots->ndim == 1 &&
        latent->sizes[0] == rope->sizes[0] && slots->sizes[0] == latent->sizes[0]))
    return mla_fail(msg, msg_cap, "invalid latent/rope/cache/slots shape");
  if (!(latent->sizes[1] > 0 && rope->sizes[1] > 0 && cache->sizes[1] > 0 &&
        cache->sizes[2] == latent->sizes[1] + rope->sizes[1]))
    return mla_fail(msg, msg_cap, "invalid cache width");
  if (!(slots->dtype == QD_DTYPE_I64 && latent->dtype == rope->dtype && latent->dtype == cache->dtype))
    return mla_fail(msg, msg_cap, "slots must be int64 and tensors must share dtype");
  return mla_ok(msg, msg_cap);
}

int qd_latent_kv_write(const void* latent, const void* rope, void* cache, const int64_t* slots, int64_t tokens,
                       int latent_dim, int rope_dim, int64_t cache_rows, int dtype, void* stream) {
  const int es = elem_size(dtype);
  if (es == 0) return mla_fail(nullptr, 0, "dtype must be float32/float16/bfloat16");
  if (tokens < 0 || latent_dim <= 0 || rope_dim <= 0 || cache_rows < 0)
    return mla_fail(nullptr, 0, "invalid latent/rope/cache/slots shape");
  if (tokens > 2147483647LL) return mla_fail(nullptr, 0, "too many tokens for one launch");
  if (tokens == 0) return QD_OK;
  if (!latent || !rope || !cache || !slots) return mla_fail(nullptr, 0, "null tensor pointer");
  LatentWriteParams prm;
  prm.latent = static_cast<const char*>(latent);
  prm.rope = static_cast<const char*>(rope);
  prm.cache = static_cast<char*>(cache);
  prm.slots = slots;
  prm.lat_bytes = static_cast<int64_t>(latent_dim) * es;
  prm.rope_bytes = static_cast<int64_t>(rope_dim) * es;
  prm.row_bytes = prm.lat_bytes + prm.rope_bytes;
  prm.rows = cache_rows;
  hipStream_t st = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  const dim3 grid(static_cast<unsigned>(tokens));
  if (prm.lat_bytes % 16 == 0 && prm.rope_bytes % 16 == 0 && aligned16(latent) && aligned16(rope) &&
      aligned16(cache))
    hipLaunchKernelGGL(latent_write_vec16_kernel, grid, dim3(64), 0, st, prm);
  else if (es == 4)
    hipLaunchKernelGGL(latent_write_elem_kernel<uint32_t>, grid, dim3(64), 0, st, prm);
  else
    hipLaunchKernelGGL(latent_write_elem_kernel<uint16_t>, grid, dim3(64), 0, st, prm);
  return launch_status("latent_kv_write");
}

int qd_mla_project_validate(const qd_tensor_desc* x, const qd_tensor_desc* w, int absorb, char* msg,
                            size_t msg_cap) {
  if (!x || !w) return mla_fail(msg, msg_cap, "null tensor descriptor");
  if (!placed(x, x)) return mla_fail(msg, msg_cap, "x must be contiguous and on the same CUDA device");
  if (!placed(w, x)) return mla_fail(msg, msg_cap, "w must be contiguous and on the same CUDA device");
  if (!float_dtype(x->dtype)) return mla_fail(msg, msg_cap, "dtype must be float32/float16/bfloat16");
  if (x->dtype != w->dtype) return mla_fail(msg, msg_cap, "dtype mismatch");
  if (!(x->ndim == 4 && w->ndim == 3 && x->sizes[2] == w->sizes[0]))
    return mla_fail(msg, msg_cap, "x [B,T,H,D], weight [H,Dn,Dc] or [H,Dv,Dc]");
  const int64_t di = x->sizes[3], dout = absorb ? w->sizes[2] : w->sizes[1];
  if (!(di > 0 && dout > 0 && (absorb ? w->sizes[1] == di : w->sizes[2] == di)))
    return mla_fail(msg, msg_cap, "projection dimension mismatch");
  return mla_ok(msg, msg_cap);
}

int qd_mla_project(const void* x, const void* w, void* out, int64_t rows, int heads, int in_dim, int out_dim,
                   int absorb, int dtype, int flags, void* stream) {
  return run_project(x, w, out, rows, heads, in_dim, out_dim, absorb != 0, dtype, flags,
                     static_cast<hipStream_t>(stream));
}

int qd_mla_attend_validate(const qd_tensor_desc* q, const qd_tensor_desc* q_rope, const qd_tensor_desc* cache,
                           const qd_tensor_desc* table, const qd_tensor_desc* lengths,
                           const qd_tensor_desc* positions, const qd_tensor_desc* indices, double scale,
                           char* msg, size_t msg_cap) {
  if (!q || !q_rope || !cache || !table || !lengths || !positions)
    return mla_fail(msg, msg_cap, "null tensor descriptor");
  if (!placed(q, q)) return mla_fail(msg, msg_cap, "q must be contiguous and on the same CUDA device");
  if (!placed(q_rope, q)) return mla_fail(msg, msg_cap, "q_rope must be contiguous and on the same CUDA device");
  if (!placed(cache, q)) return mla_fail(msg, msg_cap, "cache must be contiguous and on the same CUDA device");
  if (!placed(table, q)) return mla_fail(msg, msg_cap, "table must be contiguous and on the same CUDA device");
  if (!placed(lengths, q)) return mla_fail(msg, msg_cap, "lengths must be contiguous and on the same CUDA device");
  if (!placed(positions, q))
    return mla_fail(msg, msg_cap, "positions must be contiguous and on the same CUDA device");
  if (!float_dtype(q->dtype)) return mla_fail(msg, msg_cap, "dtype must be float32/float16/bfloat16");
  if (!(q->ndim == 4 && q_rope->ndim == 4 && cache->ndim == 3 && table->ndim == 2 && lengths->ndim == 1 &&
        positions->ndim == 2))
    return mla_fail(msg, msg_cap, "invalid tensor ranks");
  const int64_t* qs = q->sizes;
  if (!(qs[0] == q_rope->sizes[0] && qs[1] == q_rope->sizes[1] && qs[2] == q_rope->sizes[2] &&
        qs[0] == table->sizes[0] && qs[0] == lengths->sizes[0] && positions->sizes[0] == qs[0] &&
        positions->sizes[1] == qs[1]))
    return mla_fail(msg, msg_cap, "shape mismatch");
  if (!(qs[3] > 0 && qs[3] <= 512 && q_rope->sizes[3] > 0 && cache->sizes[2] == qs[3] + q_rope->sizes[3] &&
        cache->sizes[0] > 0 && cache->sizes[1] > 0 && table->sizes[1] > 0 && qs[2] > 0))
    return mla_fail(msg, msg_cap, "invalid dimensions");
  if (!(qs[0] <= 65535 && qs[1] <= 65535)) return mla_fail(msg, msg_cap, "CUDA grid limit");
  if (!(q->dtype == q_rope->dtype && q->dtype == cache->dtype)) return mla_fail(msg, msg_cap, "dtype mismatch");
  if (!(table->dtype == QD_DTYPE_I32 && lengths->dtype == QD_DTYPE_I32 && positions->dtype == QD_DTYPE_I32))
    return mla_fail(msg, msg_cap, "metadata must be int32");
  if (!(std::isfinite(scale) && scale > 0)) return mla_fail(msg, msg_cap, "scale must be positive and finite");
  if (indices && indices->defined) {
    if (!placed(indices, q))
      return mla_fail(msg, msg_cap, "indices must be contiguous and on the same CUDA device");
    if (!(indices->ndim == 3 && indices->sizes[0] == qs[0] && indices->sizes[1] == qs[1] &&
          indices->dtype == QD_DTYPE_I32))
      return mla_fail(msg, msg_cap, "indices must be int32 [B,T,K]");
  }
  return mla_ok(msg, msg_cap);
}

size_t qd_mla_attend_workspace_bytes(int batch, int q_len, int heads, int latent_dim, int rope_dim,
                                     int block_size, int max_pages, int num_indices, int dtype, int splits,
                                     int flags) {
  const AttendShape a{batch, q_len, heads, latent_dim, rope_dim, block_size, max_pages, num_indices, dtype};
  if (!attend_shape_ok(a)) return 0;
  return attend_partial_bytes(a, plan_attend(a, splits, flags));
}

int qd_mla_attend_info(int batch, int q_len, int heads, int latent_dim, int rope_dim, int block_size,
                       int max_pages, int num_indices, int dtype, int splits, int flags, int* out_splits,
                       int* head_groups) {
  const AttendShape a{batch, q_len, heads, latent_dim, rope_dim, block_size, max_pages, num_indices, dtype};
  if (!attend_shape_ok(a)) return -1;
  const AttendPlan pl = plan_attend(a, splits, flags);
  if (out_splits) *out_splits = pl.mfma ? pl.wgs : pl.splits;
  if (head_groups) *head_groups = pl.mfma ? pl.head_groups : 0;
  return pl.mfma ? (pl.shared ? 3 : pl.wave ? 2 : 1) : 0;
}

int qd_mla_attend(const void* q, const void* q_rope, const void* cache, const int32_t* block_table,
                  const int32_t* lengths, const int32_t* positions, const int32_t* indices, void* out,
                  void* workspace, size_t workspace_bytes, int batch, int q_len, int heads, int latent_dim,
                  int rope_dim, int block_size, int max_pages, int64_t num_blocks, int num_indices, int causal,
                  int dtype, float scale, int splits, int flags, void* stream) {
  const AttendShape a{batch, q_len, heads, latent_dim, rope_dim, block_size, max_pages, num_indices, dtype};
  if (!attend_shape_ok(a) || num_blocks <= 0) return mla_fail(nullptr, 0, "invalid dimensions");
  if (num_indices > 0 && !indices) return mla_fail(nullptr, 0, "null indices with num_indices > 0");
  if (splits < 0 || splits > 65535) return mla_fail(nullptr, 0, "splits must be in [0, 65535]");
  if (!(std::isfinite(scale) && scale > 0.f)) return mla_fail(nullptr, 0, "scale must be positive and finite");
  if (static_cast<int64_t>(batch) * q_len == 0) return QD_OK;
  if (!q || !q_rope || !cache || !block_table || !lengths || !positions || !out)
    return mla_fail(nullptr, 0, "null tensor pointer");
  AttendPlan pl = plan_attend(a, splits, flags);
  if (pl.mfma && !(aligned16(cache) && aligned16(out))) pl.mfma = false;
  return run_attend(a, q, q_rope, cache, block_table, lengths, positions, indices, causal, num_blocks, scale, out,
                    workspace, workspace_bytes, pl, static_cast<hipStream_t>(stream));
}

int qd_mla_decode_validate(const qd_tensor_desc* q_nope, const qd_tensor_desc* q_rope, const qd_tensor_desc* cache,
                           const qd_tensor_desc* table, const qd_tensor_desc* lengths,
                           const qd_tensor_desc* positions, const qd_tensor_desc* w_uk, const qd_tensor_desc* w_uv,
                           const qd_tensor_desc* indices, double scale, char* msg, size_t msg_cap) {
  const qd_tensor_desc* all[8] = {q_nope, q_rope, cache, table, lengths, positions, w_uk, w_uv};
  for (int i = 0; i < 8; ++i)
    if (!all[i]) return mla_fail(msg, msg_cap, "null tensor descriptor");
  for (int i = 0; i < 8; ++i)
    if (!placed(all[i], q_nope)) return mla_fail(msg, msg_cap, "input must be contiguous and on the same CUDA device");
  if (!float_dtype(q_nope->dtype)) return mla_fail(msg, msg_cap, "dtype must be float32/float16/bfloat16");
  if (!(q_nope->ndim == 4 && q_rope->ndim == 4 && cache->ndim == 3 && table->ndim == 2 && lengths->ndim == 1 &&
        positions->ndim == 2 && w_uk->ndim == 3 && w_uv->ndim == 3))
    return mla_fail(msg, msg_cap, "invalid tensor ranks");
  const int64_t* qs = q_nope->sizes;
  if (!(qs[0] == q_rope->sizes[0] && qs[1] == q_rope->sizes[1] && qs[2] == q_rope->sizes[2] &&
        qs[0] == table->sizes[0] && qs[0] == lengths->sizes[0] && positions->sizes[0] == qs[0] &&
        positions->sizes[1] == qs[1]))
    return mla_fail(msg, msg_cap, "shape mismatch");
  const int64_t dc = w_uk->sizes[2];
  if (!(qs[2] > 0 && qs[3] > 0 && q_rope->sizes[3] > 0 && dc > 0 && dc <= 512 && w_uv->sizes[1] > 0 &&
        w_uk->sizes[0] == qs[2] && w_uk->sizes[1] == qs[3] && w_uv->sizes[0] == qs[2] && w_uv->sizes[2] == dc &&
        cache->sizes[2] == dc + q_rope->sizes[3] && cache->sizes[0] > 0 && cache->sizes[1] > 0 &&
        table->sizes[1] > 0 && qs[0] <= 65535 && qs[1] <= 65535))
    return mla_fail(msg, msg_cap, "invalid dimensions");
  if (!(q_nope->dtype == q_rope->dtype && q_nope->dtype == cache->dtype && q_nope->dtype == w_uk->dtype &&
        q_nope->dtype == w_uv->dtype))
    return mla_fail(msg, msg_cap, "dtype mismatch");
  if (!(table->dtype == QD_DTYPE_I32 && lengths->dtype == QD_DTYPE_I32 && positions->dtype == QD_DTYPE_I32 &&
        std::isfinite(scale) && scale > 0))
    return mla_fail(msg, msg_cap, "invalid metadata or scale");
  if (indices && indices->defined) {
    if (!placed(indices, q_nope))
      return mla_fail(msg, msg_cap, "indices must be contiguous and on the same CUDA device");
    if (!(indices->ndim == 3 && indices->sizes[0] == qs[0] && indices->sizes[1] == qs[1] &&
          indices->dtype == QD_DTYPE_I32))
      return mla_fail(msg, msg_cap, "invalid indices");
  }
  return mla_ok(msg, msg_cap);
}

size_t qd_mla_decode_workspace_bytes(int batch, int q_len, int heads, int latent_dim, int rope_dim,
                                     int block_size, int max_pages, int num_indices, int dtype, int splits,
                                     int flags) {
  const AttendShape a{batch, q_len, heads, latent_dim, rope_dim, block_size, max_pages, num_indices, dtype};
  if (!attend_shape_ok(a)) return 0;
  return decode_layout(a, plan_attend(a, splits, flags)).total;
}

int qd_mla_decode(const void* q_nope, const void* q_rope, const void* cache, const int32_t* block_table,
                  const int32_t* lengths, const int32_t* positions, const void* w_uk, const void* w_uv,
                  const int32_t* indices, void* out, void* workspace, size_t workspace_bytes, int batch, int q_len,
                  int heads, int nope_dim, int latent_dim, int rope_dim, int value_dim, int block_size,
                  int max_pages, int64_t num_blocks, int num_indices, int causal, int dtype, float scale,
                  int splits, int flags, void* stream) {
  const AttendShape a{batch, q_len, heads, latent_dim, rope_dim, block_size, max_pages, num_indices, dtype};
  if (!attend_shape_ok(a) || nope_dim <= 0 || value_dim <= 0 || num_blocks <= 0)
    return mla_fail(nullptr, 0, "invalid dimensions");
  if (num_indices > 0 && !indices) return mla_fail(nullptr, 0, "null indices with num_indices > 0");
  if (splits < 0 || splits > 65535) return mla_fail(nullptr, 0, "splits must be in [0, 65535]");
  if (!(std::isfinite(scale) && scale > 0.f)) return mla_fail(nullptr, 0, "scale must be positive and finite");
  const int64_t rows = static_cast<int64_t>(batch) * q_len;
  if (rows == 0) return QD_OK;
  if (!q_nope || !q_rope || !cache || !block_table || !lengths || !positions || !w_uk || !w_uv || !out)
    return mla_fail(nullptr, 0, "null tensor pointer");
  AttendPlan pl = plan_attend(a, splits, flags);
  const DecodeLayout lay = decode_layout(a, pl);
  if (!workspace || workspace_bytes < lay.total || !aligned16(workspace))
    return mla_fail(nullptr, 0, "workspace must hold qd_mla_decode_workspace_bytes() bytes, 16-byte aligned");
  char* ws = static_cast<char*>(workspace);
  void* qa = ws + lay.qa;
  void* latent = ws + lay.latent;
  hipStream_t st = static_cast<hipStream_t>(stream);
  int rc = run_project(q_nope, w_uk, qa, rows, heads, nope_dim, latent_dim, true, dtype, flags, st);
  if (rc != QD_OK) return rc;
  if (pl.mfma && !aligned16(cache)) pl.mfma = false;
  // The merge of split rows folded into the value projection when it runs
  // the 16-row MFMA tiling (launch_project's choice for small batches).
  const int64_t fill = 2 * static_cast<int64_t>(device_cus());
  const bool fuse = pl.mfma && half_partials(pl) && latent_dim == 512 && (flags & QD_FLAG_FORCE_GENERIC) == 0 &&
                    project_mfma_applies(rows, latent_dim, value_dim, dtype, latent, w_uv, out) &&
                    (rows < 64 || (value_dim + 127) / 128 * heads * ((rows + 63) / 64) < fill) &&
                    (rows + 15) / 16 <= 65535;
  rc = run_attend(a, qa, q_rope, cache, block_table, lengths, positions, indices, causal, num_blocks, scale, latent,
                  ws + lay.part, workspace_bytes - lay.part, pl, st, fuse);
  if (rc != QD_OK) return rc;
  if (!fuse) return run_project(latent, w_uv, out, rows, heads, latent_dim, value_dim, false, dtype, flags, st);
  ProjParams prm{latent, w_uv, out, rows, heads, latent_dim, value_dim};
  const PartialRefs refs = partial_refs(a, pl, ws + lay.part);
  prm.part = refs.part;
  prm.meta = refs.meta;
  prm.gtotal = refs.gtotal;
  prm.wgs = pl.wgs;
  (void)hipGetLastError();
  if (dtype == QD_DTYPE_BF16)
    launch_project_merge<QD_DTYPE_BF16>(prm, st);
  else
    launch_project_merge<QD_DTYPE_F16>(prm, st);
  return launch_status("mla_decode value projection");
}

#ifdef QD_STAMPS
// Diagnostic build only: per-wave timestamps of mla_attend_shared_kernel go
// to `buffer` (16 words per wave, 4 waves per workgroup, the grid's
// workgroups in order) for the launches that follow, until called again
// (NULL stops them).
void qd_diag_set_mla_stamps(void* buffer) { g_mla_stamps = static_cast<uint64_t*>(buffer); }
#endif

}  // extern "C"
