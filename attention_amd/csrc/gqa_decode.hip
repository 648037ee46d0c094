// Paged grouped-query decode attention for MI355X (gfx950 / CDNA4).
//
// Kernels and the C ABI declared in include/qd_attention.h:
//
//   decode_mfma_sk_kernel  the automatic path for 16-bit caches, head_dim
//                          64/128/256, block_size a multiple of 16, group
//                          size <= 16.  The (sequence, 16-token group)
//                          space of the whole batch is cut into W equal
//                          ranges, one per resident workgroup, so every
//                          workgroup (and every XCD) streams the same number
//                          of K/V bytes whatever the length mix; the waves of
//                          a workgroup cover all kv-heads of the same tokens.
//                          A sequence split across workgroups leaves
//                          {m, l, acc} partials that merge_sk_kernel
//                          combines.
//   decode_mfma_kernel     the same per-wave pipeline over the reference's
//                          explicit split layout: one wave per (sequence,
//                          kv-head, split), partials [B,Hq,S,D+2].
//   decode_generic_kernel  every other shape/dtype the reference accepts
//                          (fp32, any head_dim in [1,256], any block_size,
//                          any group size) on the VALU: 16 lanes per token
//                          row, DPP row reductions.
//   combine_rows_kernel    log-sum-exp merge of [B,Hq,S,D+2] partials (head_dim
//                          64/128/256, four lane groups per head);
//   combine_kernel         the same for any head_dim or alignment.
//
// MFMA pipeline (one wave): each 16-token group is S^T = K.Q^T with
// v_mfma_f32_16x16x32 (K rows feed the A operand straight from 16-byte
// global loads), then O^T += V^T.P^T with v_mfma_f32_16x16x16 (the QK
// accumulator layout is already the B operand; V is repacked in registers
// with v_perm_b32).  Softmax state stays per lane in fp32; kPrefetch groups
// of K/V are in flight.
//
// Reference semantics followed (paths relative to the reference tree):
//   kv-head map h / (Hq/Hkv)                    csrc/cuda/dense/gqa_decode.cu:31
//   page/slot addressing, 64-bit offsets        csrc/cuda/dense/gqa_decode.cu:43-47
//   zero output for empty rows                  csrc/cuda/dense/gqa_decode.cu:64-65
//   partial layout [B,Hq,S,D+2] = {m, l, acc}   csrc/cuda/dense/gqa_decode.cu:66-69
//   streaming softmax update / merge            csrc/cuda/common/online_softmax.cuh:10-24
//   merge kernel output                         csrc/cuda/dense/gqa_decode.cu:74-87
//
// Splits cover whole pages (the reference splits the token range
// [len*z/S, len*(z+1)/S), gqa_decode.cu:40-41); the merged result is the same
// softmax, and page-aligned splits keep every 16-token group inside one page.

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <type_traits>

#include "qd_attention.h"
#include "qd_device.h"

namespace {

struct DecodeParams {
  const void* q;
  const void* k;
  const void* v;
  const int32_t* table;
  const int32_t* lens;
  void* out;
  float* ws;
  int B, Hq, Hkv, D, P, maxP, g;
  int splits;       // launched splits per (sequence, kv-head); waves W on the stream-K path
  int chunk_pages;  // 0: ceil(npages / splits) per sequence, else fixed
  int head_chunks;  // generic kernel: ceil(g / generic_heads(g))
  int64_t num_blocks;
  float sl2;  // scale * log2(e)
  int* meta;      // stream-K path: per sequence {first workgroup, workgroups}
  int wg_waves;   // stream-K path: waves per workgroup
  uint32_t* ctr;  // fused stream-K path: arrival counter per (sequence, kv-head), zero between calls
  int stage_bytes;  // stream-K path: LDS bytes per wave for result rows held until the range ends
  // Stream-K path, groups of more than kMfmaHeads q-heads: each kv-head is
  // served as kv_split virtual kv-heads (Hkv = kv_rows * kv_split) of up to
  // g q-heads each, the last one of a kv-head possibly fewer (the real
  // group is kv_g); virtual kv-head v reads K/V column v / kv_split of token
  // rows of kv_rows kv-heads (vhead_base, vhead_count).  Otherwise 1, Hkv
  // and g.
  int kv_split;
  int kv_rows;
  int kv_g;
#ifdef QD_STAMPS
  uint64_t* stamps;  // diagnostic build: per-wave timestamps (stamp_wave)
#endif
};

#ifdef QD_STAMPS
// Diagnostic build only (-DQD_STAMPS): 16 words per wave of the stream-K
// kernel, at stamps[(workgroup * waves + wave) * 16]: s_memrealtime (100 MHz)
// at entry [0], after the partition search [1], at the end of streaming [2],
// after the partial stores retired [3], after the arrival atomics returned
// [4], after the last merge [5]; the XCD id [6]; merges done [7]; the shader
// clock counter (s_memtime) at entry [8] and at the end of streaming [9].
__device__ __forceinline__ void stamp_wave(const DecodeParams& p, int slot, uint64_t value) {
  if (p.stamps && (threadIdx.x & 63) == 0)
    p.stamps[(static_cast<int64_t>(blockIdx.x) * p.wg_waves + (threadIdx.x >> 6)) * 16 + slot] = value;
}
__device__ __forceinline__ uint64_t stamp_now() { return __builtin_amdgcn_s_memrealtime(); }
__device__ __forceinline__ uint64_t stamp_clock() { return __builtin_amdgcn_s_memtime(); }
__device__ __forceinline__ uint64_t stamp_xcc() {
  uint32_t x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  return x;
}
#define QD_STAMP(p, slot, value) stamp_wave((p), (slot), (value))
#else
#define QD_STAMP(p, slot, value) ((void)0)
#endif

// Bytes of item records at the start of a wave's result staging area
// (MfmaWave::stage_*): 8 records of 16 bytes.
constexpr int kStageRecordBytes = 128;

// Valid tokens of a sequence: lengths are clamped to the table capacity
// max_pages*block_size so that a length beyond the table never reads past
// the table row; a length <= 0 has none.
__device__ __forceinline__ int clamp_len(const DecodeParams& p, int len_raw) {
  const int64_t cap = static_cast<int64_t>(p.maxP) * p.P;
  if (len_raw <= 0) return 0;
  return static_cast<int>(len_raw < cap ? static_cast<int64_t>(len_raw) : cap);
}

// Token range [tb, te) of split z and the number of non-empty splits of a
// sequence.
struct ChunkInfo {
  int tb, te, nch;
};

__device__ __forceinline__ ChunkInfo chunk_info(const DecodeParams& p, int len_raw, int z) {
  ChunkInfo c{0, 0, 0};
  const int64_t len = clamp_len(p, len_raw);
  if (len <= 0) return c;
  const int64_t npages = (len + p.P - 1) / p.P;
  const int64_t cp = p.chunk_pages > 0 ? p.chunk_pages : (npages + p.splits - 1) / p.splits;
  int64_t nch = (npages + cp - 1) / cp;
  if (nch > p.splits) nch = p.splits;
  c.nch = static_cast<int>(nch);
  const int64_t tb = static_cast<int64_t>(z) * cp * p.P;
  int64_t te = tb + cp * p.P;
  if (te > len) te = len;
  c.tb = static_cast<int>(tb < len ? tb : len);
  c.te = static_cast<int>(te);
  return c;
}

__device__ __forceinline__ int clamp_page(int32_t phys, int64_t num_blocks) {
  // Out-of-range page ids are caller errors (unchecked by the reference);
  // clamping keeps every access inside the cache.
  if (phys < 0) return 0;
  if (phys >= num_blocks) return static_cast<int>(num_blocks - 1);
  return phys;
}


// Inclusive prefix sum over the 64 lanes.
// ----------------------------------------------------------------------------
// Portable VALU kernel
// ----------------------------------------------------------------------------

constexpr int kGenericHeads = 8;

// Heads per wave of the generic kernel: 4 for groups of at most 4 q-heads
// (half the query and accumulator registers, so twice the resident waves),
// else kGenericHeads.
__host__ __device__ constexpr int generic_heads(int g) { return g <= 4 ? 4 : kGenericHeads; }

// Fewest tokens in a split of the explicit split plan (qd_gqa_decode_plan).
#ifndef QD_PLAN_MIN_TOKENS
#define QD_PLAN_MIN_TOKENS 32
#endif
constexpr int kPlanMinTokens = QD_PLAN_MIN_TOKENS;
// Waves per CU the explicit split plan aims for (splits x (sequence, kv-head)).
constexpr int64_t kPlanWavesPerCu = 4;

// grid: (splits * head_chunks, Hkv, B), block 64.
// Lane layout: row = lane/16 is one of 4 token slots, col = lane%16 owns
// elements [col*EPL, col*EPL + EPL) of head_dim.  Each row keeps its own
// streaming softmax state over the tokens it visits; rows are merged at the
// end with the log-sum-exp rule.
template <int DT, int EPL, bool FULL, int GH = kGenericHeads>
__global__ __launch_bounds__(64) void decode_generic_kernel(DecodeParams p) {
  using E = Elem<DT>;
  using S = typename E::S;
  const int lane = threadIdx.x;
  const int row = lane >> 4;
  const int col = lane & 15;
  const int e0 = col * EPL;
  const int z = blockIdx.x % p.splits;
  const int hc = blockIdx.x / p.splits;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int D = p.D;

  const ChunkInfo ci = chunk_info(p, p.lens[b], z);
  const bool direct = ci.nch <= 1;
  if (z >= (ci.nch > 1 ? ci.nch : 1)) return;

  const int h0 = kvh * p.g + hc * GH;
  const int nh = min(GH, p.g - hc * GH);
  const S* __restrict__ q = static_cast<const S*>(p.q);
  const S* __restrict__ kc = static_cast<const S*>(p.k);
  const S* __restrict__ vc = static_cast<const S*>(p.v);

  float qf[GH][EPL];
#pragma unroll
  for (int h = 0; h < GH; ++h) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const int d = e0 + e;
      qf[h][e] = (h < nh && (FULL || d < D))
                     ? E::to_f(q[(static_cast<int64_t>(b) * p.Hq + h0 + h) * D + d])
                     : 0.f;
    }
  }

  float m[GH], l[GH], acc[GH][EPL];
#pragma unroll
  for (int h = 0; h < GH; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[h][e] = 0.f;
  }

  const int64_t rs = static_cast<int64_t>(p.Hkv) * D;
  const int32_t* __restrict__ trow = p.table + static_cast<int64_t>(b) * p.maxP;
  // One 4-token step: row `row` of the wave adds its token (when valid).
  auto token_step = [&](bool valid, const float* kf, const float* vf) {
    float s[GH];
#pragma unroll
    for (int h = 0; h < GH; ++h) {
      float dot = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) dot = fmaf(qf[h][e], kf[e], dot);
      s[h] = row16_sum(dot);
    }
#pragma unroll
    for (int h = 0; h < GH; ++h) {
      const float x = valid ? s[h] * p.sl2 : -INFINITY;
      const float mn = fmaxf(m[h], x);
      const float mref = mn == -INFINITY ? 0.f : mn;
      const float alpha = fast_exp2(m[h] - mref);
      const float pr = fast_exp2(x - mref);
      l[h] = fmaf(l[h], alpha, pr);
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[h][e] = fmaf(acc[h][e], alpha, pr * vf[e]);
      m[h] = mn;
    }
  };
  if constexpr (EPL <= 8) {
    // Head_dim <= 128.  The tokens go in windows of 64 pages: lane l holds
    // the table entry of page wb + l, so a token's page id is a lane read,
    // not a dependent load.  Within a window two 4-token steps are in
    // flight: the next step's K and V rows are loaded before this step's
    // math.  A row past the window re-reads the window's last token and is
    // masked, so every load is unconditional (the compiler's wait then
    // covers only the step in use).
    auto load = [&](int w_hi, int wb, int tblv, int t0, float* kf, float* vf) {
      const int t = t0 + row;
      const int tt = t < w_hi ? t : w_hi - 1;
      const int page = tt / p.P;
      const int slot = tt - page * p.P;
      const int phys = clamp_page(__shfl(tblv, page - wb), p.num_blocks);
      const int64_t base = (static_cast<int64_t>(phys) * p.P + slot) * rs + static_cast<int64_t>(kvh) * D + e0;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const bool ok = FULL || (e0 + e < D);
        kf[e] = ok ? E::to_f(kc[base + e]) : 0.f;
        vf[e] = ok ? E::to_f(vc[base + e]) : 0.f;
      }
    };
    float kA[EPL], vA[EPL], kB[EPL], vB[EPL];
    for (int w_lo = ci.tb; w_lo < ci.te;) {
      const int wb = w_lo / p.P;
      const int tblv = lane < p.maxP - wb ? trow[wb + lane] : 0;
      const int64_t w_end = static_cast<int64_t>(wb + 64) * p.P;
      const int w_hi = w_end < ci.te ? static_cast<int>(w_end) : ci.te;
      load(w_hi, wb, tblv, w_lo, kA, vA);
      for (int t0 = w_lo; t0 < w_hi; t0 += 8) {
        load(w_hi, wb, tblv, t0 + 4, kB, vB);
        token_step(t0 + row < w_hi, kA, vA);
        load(w_hi, wb, tblv, t0 + 8, kA, vA);
        token_step(t0 + 4 + row < w_hi, kB, vB);
      }
      w_lo = w_hi;
    }
  } else {
    // Head_dim 256: one step at a time (a second buffer does not fit the
    // register file).
    for (int t0 = ci.tb; t0 < ci.te; t0 += 4) {
      const int t = t0 + row;
      const bool valid = t < ci.te;
      const int tt = valid ? t : ci.te - 1;
      const int page = tt / p.P;
      const int slot = tt - page * p.P;
      const int phys = clamp_page(trow[page], p.num_blocks);
      const int64_t base = (static_cast<int64_t>(phys) * p.P + slot) * rs +
                           static_cast<int64_t>(kvh) * D + e0;
      float kf[EPL], vf[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const bool ok = FULL || (e0 + e < D);
        kf[e] = ok ? E::to_f(kc[base + e]) : 0.f;
        vf[e] = ok ? E::to_f(vc[base + e]) : 0.f;
      }
      token_step(valid, kf, vf);
    }
  }

  // Merge the four token rows (xor 16, xor 32).
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
#pragma unroll
    for (int h = 0; h < GH; ++h) {
      const float mo = __shfl_xor(m[h], off);
      const float lo = __shfl_xor(l[h], off);
      const float mn = fmaxf(m[h], mo);
      const float mref = mn == -INFINITY ? 0.f : mn;
      const float a = fast_exp2(m[h] - mref);
      const float bb = fast_exp2(mo - mref);
      l[h] = l[h] * a + lo * bb;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float ao = __shfl_xor(acc[h][e], off);
        acc[h][e] = acc[h][e] * a + ao * bb;
      }
      m[h] = mn;
    }
  }

  if (row != 0) return;
  if (direct) {
    S* __restrict__ out = static_cast<S*>(p.out);
#pragma unroll
    for (int h = 0; h < GH; ++h) {
      if (h >= nh) break;
      const float inv = l[h] > 0.f ? 1.f / l[h] : 0.f;
      const int64_t ob = (static_cast<int64_t>(b) * p.Hq + h0 + h) * D;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const int d = e0 + e;
        if (FULL || d < D) out[ob + d] = E::from_f(l[h] > 0.f ? acc[h][e] * inv : 0.f);
      }
    }
  } else {
#pragma unroll
    for (int h = 0; h < GH; ++h) {
      if (h >= nh) break;
      float* w = p.ws + ((static_cast<int64_t>(b) * p.Hq + h0 + h) * p.splits + z) * (D + 2);
      if (col == 0) {
        w[0] = m[h] * kLn2;
        w[1] = l[h];
      }
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const int d = e0 + e;
        if (FULL || d < D) w[2 + d] = acc[h][e];
      }
    }
  }
}

// ----------------------------------------------------------------------------
// ----------------------------------------------------------------------------
// MFMA pipeline
// ----------------------------------------------------------------------------

// V bytes one lane loads from one cache row: head_dim/16 elements.
template <int D>
struct VRow {
  static constexpr int kElems = D / 16;
  static constexpr int kWords = kElems / 2;  // 32-bit words
  uint32_t w[kWords];
};


template <int D>
__device__ __forceinline__ VRow<D> load_vrow(const char* ptr) {
  VRow<D> r;
  if constexpr (VRow<D>::kWords == 2) {
    const u32x2 x = stream_load8(ptr);
    r.w[0] = x[0];
    r.w[1] = x[1];
  } else if constexpr (VRow<D>::kWords == 3) {  // head_dim 96: 12 bytes, 4-byte aligned
    r.w[0] = stream_load4(ptr);
    r.w[1] = stream_load4(ptr + 4);
    r.w[2] = stream_load4(ptr + 8);
  } else {
#pragma unroll
    for (int i = 0; i < VRow<D>::kWords / 4; ++i) {
      const u32x4 x = stream_load16(ptr + 16 * i);
      r.w[4 * i + 0] = x[0];
      r.w[4 * i + 1] = x[1];
      r.w[4 * i + 2] = x[2];
      r.w[4 * i + 3] = x[3];
    }
  }
  return r;
}

// Registers for one 16-token group in flight, for NKV kv-heads.
// Stores NW 32-bit words at dst: one 8-byte store for 2, 16-byte stores for
// a multiple of 4 (dst aligned to match), else one word at a time.
template <int NW>
__device__ __forceinline__ void store_words(char* dst, const uint32_t* wv) {
  if constexpr (NW == 2) {
    *reinterpret_cast<u32x2*>(dst) = u32x2{wv[0], wv[1]};
  } else if constexpr (NW % 4 == 0) {
#pragma unroll
    for (int t = 0; t < NW / 4; ++t)
      *reinterpret_cast<u32x4*>(dst + 16 * t) = u32x4{wv[4 * t], wv[4 * t + 1], wv[4 * t + 2], wv[4 * t + 3]};
  } else {
#pragma unroll
    for (int t = 0; t < NW; ++t) reinterpret_cast<uint32_t*>(dst)[t] = wv[t];
  }
}

template <int D, int NKV>
struct GroupBuf {
  static constexpr int KC = D / 32;
  u32x4 k[NKV][KC];   // K, coalesced: piece KTile<D>::col_bytes(c, lane) of row KTile<D>::row(c, lane)
  VRow<D> v[NKV][4];  // V rows 4*(lane/16)+i, elements (D/16)*(lane%16) ..
  int tg;             // first token of the group
};

// K of one 16-token group moves HBM -> VGPR -> LDS -> VGPR.  The global
// loads are coalesced (each instruction reads whole 2*D-byte row segments,
// 1 KB per instruction), which streams measurably faster than loading the
// MFMA operand layout directly (16 rows x 64 bytes per instruction; 5-8%
// slower at head_dim 96, about 10% at 128).  The LDS tile re-reads it in the
// MFMA A layout.  Rows are padded by 32 bytes: measured free of LDS bank
// conflicts for D = 128 (16 bytes left 20% of the LDS cycles in conflicts,
// none left 64%).
//
// Load c, lane l reads the 16-byte piece 64c + l of the group's 16 rows in
// row order: row (64c + l) / kLanesPerRow, piece (64c + l) % kLanesPerRow.
// At head_dim 96 (12 pieces per row) a load ends inside a row.
template <int D, int ES = 2>
struct KTile {
  static constexpr int kRowBytes = ES * D;  // ES: bytes per element (4 for fp32 caches)
  static constexpr int kStride = kRowBytes + 32;
  static constexpr int kLanesPerRow = kRowBytes / 16;  // 8, 12, 16, 32 (16-bit), 16, 32 (fp32)
  static constexpr bool kWholeRows = 64 % kLanesPerRow == 0;
  static constexpr int kBytes = 16 * kStride;
  __device__ static int row(int c, int lane) {
    if constexpr (kWholeRows) return c * (64 / kLanesPerRow) + lane / kLanesPerRow;
    return (64 * c + lane) / kLanesPerRow;
  }
  __device__ static int col_bytes(int c, int lane) {
    if constexpr (kWholeRows) return 16 * (lane % kLanesPerRow);
    return 16 * ((64 * c + lane) % kLanesPerRow);
  }
};

// First q-head and q-head count of (virtual) kv-head v.
__device__ __forceinline__ int vhead_base(const DecodeParams& p, int v) {
  return p.kv_split > 1 ? (v / p.kv_split) * p.kv_g + (v % p.kv_split) * p.g : v * p.g;
}
__device__ __forceinline__ int vhead_count(const DecodeParams& p, int v) {
  return p.kv_split > 1 ? min(p.g, p.kv_g - (v % p.kv_split) * p.g) : p.g;
}

// One wave's decode state for NKV adjacent kv-heads (kvh0 .. kvh0+NKV-1) of
// one sequence.  Serving two kv-heads from one wave (one wave per SIMD)
// keeps the K/V streams of a SIMD in one instruction stream: two waves on a
// SIMD were served unevenly (the older one finished ~30% earlier, leaving
// half the loads in flight for the rest of the kernel).
//
// Lane l, r16 = l % 16, q4 = l / 16, for each kv-head:
//   QK  A = K      lane holds K[token r16][8 elems]     (16x16x32 A layout,
//                  read from the LDS tile)
//       B = Q^T    lane holds Q[head  r16][same elems]
//       C = S^T    lane holds S[token 4*q4+i][head r16], i = 0..3
//   PV  A = V^T    lane holds V[token 4*q4+i][d = DV*r16 + j], i = 0..3
//       B = P^T    lane holds P[head r16][token 4*q4+i]  == C layout of QK
//       C = O^T    lane holds O[head r16][d = DV*(4*q4+i) + j]
// so every lane owns one head's softmax state and a contiguous slice of
// DV*4 output elements of that head.  Heads r16 >= group size carry zero
// queries and are never stored.
template <int D, int DT, int PF, int NKV>
struct MfmaWave {
  using Ops = MfmaOps<DT>;
  using Buf = GroupBuf<D, NKV>;
  static constexpr int KC = D / 32;
  static constexpr int DV = D / 16;
  static constexpr int VB = DV * 2;  // bytes per lane per V row

  int lane, r16, q4;
  u32x4 qv[NKV][KC];
  float m_run[NKV], l_run[NKV];
  f32x4 acc[NKV][DV];
  // Item being processed.
  const char* kbase;  // kv-head kvh0; kv-head kvh0+j is 2*D*j bytes further
  const char* vbase;
  const int32_t* trow;
  int hcount;  // q-heads of each kv-head of the item (vhead_count; p.g unless split)
  int len;    // valid tokens of the item (or of the split)
  int wbase;  // first page of the table window held in tblv
  int tblv;   // table entry (wbase + lane)

  __device__ void init_lane() {
    lane = threadIdx.x & 63;  // lane within the wave (workgroups may hold several)
    r16 = lane & 15;
    q4 = lane >> 4;
    res_lds = nullptr;
    res_cap = 0;
    res_used = 0;
    res_items = 0;
  }

  // Starts item (b, kvh0..) whose run() begins at group g_first.  The page
  // table window of g_first is loaded before the query, so the first K/V
  // loads wait for the table alone; the query is needed only at compute.
  __device__ void begin_item(const DecodeParams& p, int b, int kvh0, int valid_tokens, int g_first) {
    hcount = vhead_count(p, kvh0);  // NKV is 1 whenever kv-heads are split
    const bool head_ok = r16 < hcount;
    trow = p.table + static_cast<int64_t>(b) * p.maxP;
    wbase = g_first / (p.P >> 4);
    tblv = (lane < p.maxP - wbase) ? trow[wbase + lane] : 0;
#pragma unroll
    for (int j = 0; j < NKV; ++j) {
      const char* qp = static_cast<const char*>(p.q) +
                       (static_cast<int64_t>(b) * p.Hq + vhead_base(p, kvh0 + j) + (head_ok ? r16 : 0)) * D * 2;
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        const u32x4 x = *reinterpret_cast<const u32x4*>(qp + (32 * c + 8 * q4) * 2);
        const u32x4 zero = {0u, 0u, 0u, 0u};
        qv[j][c] = head_ok ? x : zero;
      }
      m_run[j] = -INFINITY;
      l_run[j] = 0.f;
#pragma unroll
      for (int d = 0; d < DV; ++d) acc[j][d] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // Virtual kv-heads (kv_split > 1) come with one kv-head per wave (NKV 1).
    const int64_t col = p.kv_split > 1 ? kvh0 / p.kv_split : kvh0;
    kbase = static_cast<const char*>(p.k) + col * D * 2;
    vbase = static_cast<const char*>(p.v) + col * D * 2;
    len = valid_tokens;
  }

  // Issues the K/V loads of group gi (tokens 16*gi .. 16*gi+15 of the item).
  // The group lies inside one page (block_size is a multiple of 16); rows at
  // or past `len` re-read the last valid row and are masked in compute().
  __device__ void issue(const DecodeParams& p, Buf& buf, int gi) {
    const int gpp = p.P >> 4;
    const int tg = 16 * gi;
    buf.tg = tg;
    const int pl = gi / gpp;               // page index within the item
    const int row0 = 16 * (gi - pl * gpp);  // first row inside the page
    const int phys = clamp_page(__builtin_amdgcn_readlane(tblv, pl - wbase), p.num_blocks);
    const int64_t row_bytes = static_cast<int64_t>(p.kv_rows) * D * 2;
    const int64_t off = (static_cast<int64_t>(phys) * p.P + row0) * row_bytes;
    const char* kp = kbase + off;
    const char* vp = vbase + off;
    const uint32_t rb32 = static_cast<uint32_t>(row_bytes);
    const int last = len - 1 - tg;  // rows > last are past the end: reuse row `last`
#pragma unroll
    for (int j = 0; j < NKV; ++j) {
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        const uint32_t rk = static_cast<uint32_t>(min(KTile<D>::row(c, lane), last));
        buf.k[j][c] = stream_load16(kp + j * 2 * D + rk * rb32 + KTile<D>::col_bytes(c, lane));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t rv = static_cast<uint32_t>(min(4 * q4 + i, last));
        buf.v[j][i] = load_vrow<D>(vp + j * 2 * D + rv * rb32 + VB * r16);
      }
    }
    // Keep each group's loads in program order relative to the other
    // groups': the wait before a compute then covers only that group.
    __builtin_amdgcn_sched_barrier(0);
  }

  __device__ void compute(const DecodeParams& p, const Buf& buf, char* ktile) {
    const int last = len - 1 - buf.tg;
#pragma unroll
    for (int j = 0; j < NKV; ++j) {
      // Transpose K through LDS into the A layout: lane (r16, q4), chunk c
      // holds row r16, bytes [64c + 16q4, +16).
      u32x4 ka[KC];
#pragma unroll
      for (int c = 0; c < KC; ++c)
        *reinterpret_cast<u32x4*>(ktile + KTile<D>::row(c, lane) * KTile<D>::kStride +
                                  KTile<D>::col_bytes(c, lane)) = buf.k[j][c];
#pragma unroll
      for (int c = 0; c < KC; ++c)
        ka[c] = *reinterpret_cast<const u32x4*>(ktile + r16 * KTile<D>::kStride + 64 * c + 16 * q4);
      f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < KC; ++c) s = Ops::qk(ka[c], qv[j][c], s);
      float x[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = (4 * q4 + i <= last) ? s[i] : -INFINITY;
      float mx = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mn = fmaxf(m_run[j], mx * p.sl2);
      const float mref = mn == -INFINITY ? 0.f : mn;
      const float alpha = fast_exp2(m_run[j] - mref);
      float pr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) pr[i] = fast_exp2(fmaf(x[i], p.sl2, -mref));
      l_run[j] = fmaf(l_run[j], alpha, (pr[0] + pr[1]) + (pr[2] + pr[3]));
      m_run[j] = mn;
      if (__builtin_amdgcn_read_exec() & __ballot(alpha != 1.f)) {
#pragma unroll
        for (int d = 0; d < DV; ++d) acc[j][d] *= alpha;
      }
      // The weights as hi + lo for bf16 (MfmaOps::kSplitWeights): the PV
      // product then sees them to ~2^-17, as the fp32 denominator does.
      // One 16x16x32 MFMA takes both: a lane's k-block of 8 is its 4 tokens
      // twice, V in A and [hi, lo] in B (the MFMA sums over any consistent
      // k order), so the split costs no extra instruction.
      const u32x2 pb = {Ops::pack2(pr[0], pr[1]), Ops::pack2(pr[2], pr[3])};
      const u32x4 pbl = {pb[0], pb[1], Ops::rest2(pr[0], pr[1], pb[0]), Ops::rest2(pr[2], pr[3], pb[1])};
#pragma unroll
      for (int d = 0; d < DV; ++d) {
        const int w = d >> 1;
        const uint32_t sel = (d & 1) ? 0x07060302u : 0x05040100u;
        const u32x2 a = {__builtin_amdgcn_perm(buf.v[j][1].w[w], buf.v[j][0].w[w], sel),
                         __builtin_amdgcn_perm(buf.v[j][3].w[w], buf.v[j][2].w[w], sel)};
        if constexpr (Ops::kSplitWeights)
          acc[j][d] = Ops::mma32(u32x4{a[0], a[1], a[0], a[1]}, pbl, acc[j][d]);
        else
          acc[j][d] = Ops::pv(a, pb, acc[j][d]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  // Streams groups [ga, gb) of the current item.  Groups are processed in
  // runs that stay inside one 64-page table window; the window is loaded
  // only between runs, never while K/V loads are in flight, so waiting for
  // it never drains the K/V prefetch.  Within a run PF groups are in
  // flight: the steady-state loop issues unconditionally (static buffer
  // slots, no branches around loads) so the compiler's wait counts cover
  // only the group being consumed.
  //
  // lockstep: a workgroup barrier every PF groups, for workgroups whose
  // waves all stream the same groups (one item each, same [ga, gb)).  Two
  // waves sharing a SIMD are not issued evenly: without it the older wave
  // of each pair ran ahead and the other finished its range alone with half
  // the loads in flight (per-wave timestamps: waves of one workgroup ended
  // 4-8 us apart).  gfx950's barrier does not wait for outstanding loads,
  // so the prefetched groups stay in flight across it.
  __device__ void run(const DecodeParams& p, int ga, int gb, char* ktile, bool lockstep = false) {
    const int gpp = p.P >> 4;
    for (int g_lo = ga; g_lo < gb;) {
      if (g_lo != ga) {  // the first window came with begin_item
        wbase = g_lo / gpp;
        tblv = (lane < p.maxP - wbase) ? trow[wbase + lane] : 0;
      }
      const int g_hi = min(gb, (wbase + 64) * gpp);
      const int n = g_hi - g_lo;
      Buf buf[PF];
      int i = 0;
      if (n >= 2 * PF - 1) {
#pragma unroll
        for (int u = 0; u < PF - 1; ++u) issue(p, buf[u], g_lo + u);
        for (; i + 2 * PF - 2 < n; i += PF) {
          if (lockstep) __builtin_amdgcn_s_barrier();
#pragma unroll
          for (int u = 0; u < PF; ++u) {
            issue(p, buf[(u + PF - 1) % PF], g_lo + i + u + PF - 1);
            compute(p, buf[u], ktile);
          }
        }
      } else {
#pragma unroll
        for (int u = 0; u < PF - 1; ++u)
          if (u < n) issue(p, buf[u], g_lo + u);
      }
      // Tail: the remaining (< 2*PF-1) groups, with guarded issues.
      for (; i < n; i += PF) {
#pragma unroll
        for (int u = 0; u < PF; ++u) {
          if (i + u + PF - 1 < n) issue(p, buf[(u + PF - 1) % PF], g_lo + i + u + PF - 1);
          if (i + u < n) compute(p, buf[u], ktile);
        }
      }
      g_lo = g_hi;
    }
  }

  // Softmax denominator of this lane's head (lanes of one head hold partial
  // sums over their 4 tokens of every group).
  __device__ float total_l(int j) const {
    float l = l_run[j] + __shfl_xor(l_run[j], 16);
    return l + __shfl_xor(l, 32);
  }

  // Result rows held back until the range ends.  On gfx950 a store counts
  // in vmcnt with the loads and vmcnt retires in issue order, so every
  // load issued after a store waits for the store's acknowledgement, and
  // while the K/V stream saturates HBM the memory system acknowledges
  // writes late.  Stores between items therefore stalled the following
  // item's loads (and, through the lockstep barrier, the workgroup) by
  // microseconds: on cfg5 (256 short sequences, an output or partial per
  // item) the decode kernel took 91 us with its stores removed against 103
  // us with them, and stores moved behind the next item's first loads or
  // merged into contiguous chunks changed nothing.  So an item's rows go to
  // this wave's LDS area in their memory layout (stage_direct /
  // stage_partial), and flush_results copies them out with contiguous 16-
  // or 8-byte stores when the range ends (or when the area is full).  The
  // area starts with kStageMaxItems 16-byte records {destination, bytes,
  // chunk} (in LDS, so that nothing more stays live in registers across
  // the streaming loop); the rows follow.
  static constexpr int kStageMaxItems = kStageRecordBytes / 16;
  static constexpr int kStageHeader = kStageRecordBytes;
  char* res_lds;     // this wave's area (header, then rows)
  int res_cap;       // bytes for rows after the header
  int res_used;      // row bytes staged so far (16-byte multiples)
  int res_items;     // items staged

  __device__ static int round16(int x) { return (x + 15) & ~15; }

  // Makes room for `bytes` more, flushing what is staged if needed; returns
  // the LDS address the item's rows go to.
  __device__ char* stage_slot(int bytes) {
    if (res_used + round16(bytes) > res_cap || res_items == kStageMaxItems) flush_results();
    return res_lds + kStageHeader + res_used;
  }

  __device__ void stage_direct(const DecodeParams& p, char* area, int jk, float l_tot) {
    using S = typename Elem<DT>::S;
    if (r16 >= hcount) return;
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    S* o = reinterpret_cast<S*>(area) + (jk * p.g + r16) * D;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t wv[DV / 2];
#pragma unroll
      for (int j = 0; j < DV; j += 2)
        wv[j / 2] = Ops::pack2(l_tot > 0.f ? acc[jk][j][i] * inv : 0.f,
                               l_tot > 0.f ? acc[jk][j + 1][i] * inv : 0.f);
      uint32_t* dst = reinterpret_cast<uint32_t*>(o + DV * (4 * q4 + i));
#pragma unroll
      for (int t = 0; t < DV / 2; ++t) dst[t] = wv[t];
    }
  }

  __device__ void stage_partial(const DecodeParams& p, char* area, int jk, float l_tot) {
    if (r16 >= hcount) return;
    float* w = reinterpret_cast<float*>(area) + (jk * p.g + r16) * (D + 2);
    if (q4 == 0) {
      w[0] = m_run[jk] * kLn2;
      w[1] = l_tot;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float* dst = w + 2 + DV * (4 * q4 + i);
#pragma unroll
      for (int j = 0; j < DV; ++j) dst[j] = acc[jk][j][i];
    }
  }

  // Records the item just staged at stage_slot(bytes): `bytes` to `dst`
  // in `chunk`-byte stores (16 for output rows, 8 for partial rows).
  __device__ void stage_commit(char* dst, int bytes, int chunk) {
    if (lane == 0) {
      const uint64_t d = reinterpret_cast<uint64_t>(dst);
      *reinterpret_cast<u32x4*>(res_lds + 16 * res_items) =
          u32x4{static_cast<uint32_t>(d), static_cast<uint32_t>(d >> 32), static_cast<uint32_t>(bytes),
                static_cast<uint32_t>(chunk)};
    }
    res_used += round16(bytes);
    ++res_items;
  }

  __device__ void flush_results() {
    if (res_items == 0) return;
    // The staged rows and records were written by other lanes of this
    // wave: the LDS writes complete first, and nothing is reordered across
    // this point.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    int off = 0;
    for (int t = 0; t < res_items; ++t) {
      const u32x4 rec = *reinterpret_cast<const u32x4*>(res_lds + 16 * t);  // same address in every lane
      const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(rec[0])));
      const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(rec[1])));
      const int bytes = __builtin_amdgcn_readfirstlane(static_cast<int>(rec[2]));
      const int chunk = __builtin_amdgcn_readfirstlane(static_cast<int>(rec[3]));
      char* dst = reinterpret_cast<char*>((static_cast<uint64_t>(hi) << 32) | lo);
      const char* src = res_lds + kStageHeader + off;
      if (chunk == 16) {
        for (int c = lane; c < bytes / 16; c += 64)
          *reinterpret_cast<u32x4*>(dst + 16 * c) = *reinterpret_cast<const u32x4*>(src + 16 * c);
      } else {
        for (int c = lane; c < bytes / 8; c += 64)
          *reinterpret_cast<u32x2*>(dst + 8 * c) = *reinterpret_cast<const u32x2*>(src + 8 * c);
      }
      off += round16(bytes);
    }
    asm volatile("" ::: "memory");
    res_items = 0;
    res_used = 0;
  }

  // out[b, vhead_base(kvh0+jk) + r16, :] = acc / l (zeros when l == 0), one
  // rounding.
  __device__ void store_direct(const DecodeParams& p, int b, int kvh0, int jk, float l_tot) {
    using S = typename Elem<DT>::S;
    if (r16 >= hcount) return;
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    S* o = static_cast<S*>(p.out) + (static_cast<int64_t>(b) * p.Hq + vhead_base(p, kvh0 + jk) + r16) * D;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t wv[DV / 2];
#pragma unroll
      for (int j = 0; j < DV; j += 2)
        wv[j / 2] = Ops::pack2(l_tot > 0.f ? acc[jk][j][i] * inv : 0.f,
                               l_tot > 0.f ? acc[jk][j + 1][i] * inv : 0.f);
      store_words<DV / 2>(reinterpret_cast<char*>(o + DV * (4 * q4 + i)), wv);
    }
  }

  // Fused merge: a partial that would be stored in the middle of the
  // workgroup's range waits in LDS until the range ends instead.  An sc1
  // store completes only at the device coherence point, and the wave's
  // next loads (the following item's K/V) count behind it in vmcnt, so a
  // mid-range store stalled the next item's pipeline (and, through the
  // lockstep barrier, the workgroup's).  Area per kv-head: kStashFields rows
  // of 64 floats, field-major (lane l at column l: conflict-free).
  static constexpr int kStashFields = 2 + 4 * DV;

  __device__ void stash_partial(int jk, float* stash, float l_tot) const {
    float* s = stash + jk * kStashFields * 64 + lane;
    s[0] = m_run[jk] * kLn2;
    s[64] = l_tot;
#pragma unroll
    for (int d = 0; d < DV; ++d)
#pragma unroll
      for (int i = 0; i < 4; ++i) s[(2 + 4 * d + i) * 64] = acc[jk][d][i];
  }

  // Stores a stashed partial as store_partial<true> stores a live one.
  __device__ void store_stashed(const DecodeParams& p, int jk, const float* stash, float* w,
                                int64_t head_stride) const {
    if (r16 >= hcount) return;
    const float* s = stash + jk * kStashFields * 64 + lane;
    w += r16 * head_stride;
    if (q4 == 0) coherent_store2(w, s[0], s[64]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float* dst = w + 2 + DV * (4 * q4 + i);
#pragma unroll
      for (int j = 0; j < DV; j += 2)
        coherent_store2(dst + j, s[(2 + 4 * j + i) * 64], s[(2 + 4 * (j + 1) + i) * 64]);
    }
  }

  // Partial {m (natural-log units), l, acc[D]} of kv-head kvh0+jk, this
  // lane's head, at w + head*head_stride (head_stride even).  COH: sc1
  // stores, for a merge by another workgroup of the same launch.
  template <bool COH = false>
  __device__ void store_partial(const DecodeParams& p, int jk, float* w, int64_t head_stride, float l_tot) {
    if (r16 >= hcount) return;
    w += r16 * head_stride;
    if (q4 == 0) {
      if constexpr (COH) {
        coherent_store2(w, m_run[jk] * kLn2, l_tot);
      } else {
        w[0] = m_run[jk] * kLn2;
        w[1] = l_tot;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float* dst = w + 2 + DV * (4 * q4 + i);
#pragma unroll
      for (int j = 0; j < DV; j += 2) {
        if constexpr (COH)
          coherent_store2(dst + j, acc[jk][j][i], acc[jk][j + 1][i]);
        else
          *reinterpret_cast<f32x2*>(dst + j) = f32x2{acc[jk][j][i], acc[jk][j + 1][i]};
      }
    }
  }
};

// One wave's decode state for one kv-head of an fp32 cache, on the matrix
// cores in fp32 (v_mfma_f32_16x16x4_f32: fp32 products and sums, the
// reference's arithmetic).  Lane l, r16 = l % 16, q4 = l / 16:
//   QK  MFMA (c, e), c < D/16, e < 4, over dims 16c + 4*q4 + e:
//       A = K      lane holds K[token r16][16c + 4*q4 + e] (16 bytes of row
//                  r16 of the LDS tile per c: coalesced loads, transposed
//                  through LDS as in MfmaWave)
//       B = Q^T    lane holds Q[head r16][16c + 4*q4 + e]
//       C = S^T    lane holds S[token 4*q4+i][head r16], i = 0..3 (the C
//                  layout of every 16x16 MFMA, as in MfmaWave)
//   PV  MFMA (d, c), d < D/16, c < 4: lane group q4's k index is token
//       4*q4 + c, so
//       B = P^T    is the lane's own weight of token 4*q4 + c (QK's C)
//       A = V^T    lane holds V[token 4*q4+c][DV*r16 + d]: DV contiguous
//                  floats of that row, 16 lanes reading the row whole
//       C = O^T    lane holds O[head r16][DV*(4*q4+i) + d], MfmaWave's
//                  accumulator layout, so its partial-row and staging
//                  stores serve this wave unchanged.
// The softmax is MfmaWave's (exact running max, base 2, scale folded in);
// the weights enter the PV product unrounded.
template <int D, int PF>
struct MfmaWaveF32 : MfmaWave<D, QD_DTYPE_F32, PF, 1> {
  static_assert(D == 64 || D == 128, "fp32 MFMA decode serves head_dim 64 and 128");
  using Base = MfmaWave<D, QD_DTYPE_F32, PF, 1>;
  using Tile = KTile<D, 4>;
  static constexpr int KQ = D / 16;  // 16-byte pieces of K (per group) and of the query, per lane
  static constexpr int DV = D / 16;
  struct Buf {
    u32x4 k[KQ];
    VRow<2 * D> v[4];  // DV floats of rows 4*q4 + c
    int tg;
  };
  u32x4 qf[KQ];

  __device__ void begin_item(const DecodeParams& p, int b, int kvh0, int valid_tokens, int g_first) {
    this->hcount = vhead_count(p, kvh0);
    const bool head_ok = this->r16 < this->hcount;
    this->trow = p.table + static_cast<int64_t>(b) * p.maxP;
    this->wbase = g_first / (p.P >> 4);
    this->tblv = (this->lane < p.maxP - this->wbase) ? this->trow[this->wbase + this->lane] : 0;
    const char* qp = static_cast<const char*>(p.q) +
                     (static_cast<int64_t>(b) * p.Hq + vhead_base(p, kvh0) + (head_ok ? this->r16 : 0)) * D * 4;
#pragma unroll
    for (int c = 0; c < KQ; ++c) {
      const u32x4 x = *reinterpret_cast<const u32x4*>(qp + 64 * c + 16 * this->q4);
      const u32x4 zero = {0u, 0u, 0u, 0u};
      qf[c] = head_ok ? x : zero;
    }
    this->m_run[0] = -INFINITY;
    this->l_run[0] = 0.f;
#pragma unroll
    for (int d = 0; d < DV; ++d) this->acc[0][d] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int64_t col = p.kv_split > 1 ? kvh0 / p.kv_split : kvh0;
    this->kbase = static_cast<const char*>(p.k) + col * D * 4;
    this->vbase = static_cast<const char*>(p.v) + col * D * 4;
    this->len = valid_tokens;
  }

  // Issues the K/V loads of group gi, as MfmaWave::issue.
  __device__ void issue(const DecodeParams& p, Buf& buf, int gi) {
    const int gpp = p.P >> 4;
    const int tg = 16 * gi;
    buf.tg = tg;
    const int pl = gi / gpp;
    const int row0 = 16 * (gi - pl * gpp);
    const int phys = clamp_page(__builtin_amdgcn_readlane(this->tblv, pl - this->wbase), p.num_blocks);
    const int64_t row_bytes = static_cast<int64_t>(p.kv_rows) * D * 4;
    const int64_t off = (static_cast<int64_t>(phys) * p.P + row0) * row_bytes;
    const char* kp = this->kbase + off;
    const char* vp = this->vbase + off;
    const uint32_t rb32 = static_cast<uint32_t>(row_bytes);
    const int last = this->len - 1 - tg;
#pragma unroll
    for (int c = 0; c < KQ; ++c) {
      const uint32_t rk = static_cast<uint32_t>(min(Tile::row(c, this->lane), last));
      buf.k[c] = stream_load16(kp + rk * rb32 + Tile::col_bytes(c, this->lane));
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t rv = static_cast<uint32_t>(min(4 * this->q4 + c, last));
      buf.v[c] = load_vrow<2 * D>(vp + rv * rb32 + 4 * DV * this->r16);
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  __device__ void compute(const DecodeParams& p, const Buf& buf, char* ktile) {
    const int last = this->len - 1 - buf.tg;
#pragma unroll
    for (int c = 0; c < KQ; ++c)
      *reinterpret_cast<u32x4*>(ktile + Tile::row(c, this->lane) * Tile::kStride + Tile::col_bytes(c, this->lane)) =
          buf.k[c];
    u32x4 ka[KQ];
#pragma unroll
    for (int c = 0; c < KQ; ++c)
      ka[c] = *reinterpret_cast<const u32x4*>(ktile + this->r16 * Tile::kStride + 64 * c + 16 * this->q4);
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < KQ; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        s = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(ka[c][e]), __uint_as_float(qf[c][e]), s, 0, 0, 0);
    float x[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = (4 * this->q4 + i <= last) ? s[i] : -INFINITY;
    float mx = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mn = fmaxf(this->m_run[0], mx * p.sl2);
    const float mref = mn == -INFINITY ? 0.f : mn;
    const float alpha = fast_exp2(this->m_run[0] - mref);
    float pr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) pr[i] = fast_exp2(fmaf(x[i], p.sl2, -mref));
    this->l_run[0] = fmaf(this->l_run[0], alpha, (pr[0] + pr[1]) + (pr[2] + pr[3]));
    this->m_run[0] = mn;
    if (__builtin_amdgcn_read_exec() & __ballot(alpha != 1.f)) {
#pragma unroll
      for (int d = 0; d < DV; ++d) this->acc[0][d] *= alpha;
    }
#pragma unroll
    for (int d = 0; d < DV; ++d)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        this->acc[0][d] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(buf.v[c].w[d]), pr[c],
                                                               this->acc[0][d], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  }

  // MfmaWave::run with this wave's issue and compute.
  __device__ void run(const DecodeParams& p, int ga, int gb, char* ktile, bool lockstep = false) {
    const int gpp = p.P >> 4;
    for (int g_lo = ga; g_lo < gb;) {
      if (g_lo != ga) {
        this->wbase = g_lo / gpp;
        this->tblv = (this->lane < p.maxP - this->wbase) ? this->trow[this->wbase + this->lane] : 0;
      }
      const int g_hi = min(gb, (this->wbase + 64) * gpp);
      const int n = g_hi - g_lo;
      Buf buf[PF];
      int i = 0;
      if (n >= 2 * PF - 1) {
#pragma unroll
        for (int u = 0; u < PF - 1; ++u) issue(p, buf[u], g_lo + u);
        for (; i + 2 * PF - 2 < n; i += PF) {
          if (lockstep) __builtin_amdgcn_s_barrier();
#pragma unroll
          for (int u = 0; u < PF; ++u) {
            issue(p, buf[(u + PF - 1) % PF], g_lo + i + u + PF - 1);
            compute(p, buf[u], ktile);
          }
        }
      } else {
#pragma unroll
        for (int u = 0; u < PF - 1; ++u)
          if (u < n) issue(p, buf[u], g_lo + u);
      }
      for (; i < n; i += PF) {
#pragma unroll
        for (int u = 0; u < PF; ++u) {
          if (i + u + PF - 1 < n) issue(p, buf[(u + PF - 1) % PF], g_lo + i + u + PF - 1);
          if (i + u < n) compute(p, buf[u], ktile);
        }
      }
      g_lo = g_hi;
    }
  }

  // Output rows in fp32: DV contiguous floats per (lane, i).
  __device__ void store_direct(const DecodeParams& p, int b, int kvh0, int, float l_tot) {
    if (this->r16 >= this->hcount) return;
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    float* o = static_cast<float*>(p.out) + (static_cast<int64_t>(b) * p.Hq + vhead_base(p, kvh0) + this->r16) * D;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float* dst = o + DV * (4 * this->q4 + i);
#pragma unroll
      for (int d = 0; d < DV; d += 4) {
        f32x4 v;
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = l_tot > 0.f ? this->acc[0][d + t][i] * inv : 0.f;
        *reinterpret_cast<f32x4*>(dst + d) = v;
      }
    }
  }

  __device__ void stage_direct(const DecodeParams& p, char* area, int, float l_tot) {
    if (this->r16 >= this->hcount) return;
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    float* o = reinterpret_cast<float*>(area) + this->r16 * D;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float* dst = o + DV * (4 * this->q4 + i);
#pragma unroll
      for (int d = 0; d < DV; ++d) dst[d] = l_tot > 0.f ? this->acc[0][d][i] * inv : 0.f;
    }
  }
};

// VALU compute of the same per-wave pipeline, for comparison with the MFMA
// one (head_dim 128, one kv-head per wave, at most GV heads per group).
// Same loads, table windows and partition as MfmaWave; only the math
// differs.  Lane l, a = l % 16, r = l / 16:
//   K  from the coalesced load: rows 4c + r (c = 0..3), elements 8a .. 8a+7
//   Q  the same 8 elements of every head, packed 16-bit pairs
//   S  4 dot2 per (row, head), then a sum over the 16 lanes of the row (DPP):
//      every lane of row r holds S[4c + r][h] for c = 0..3
//   P  written to LDS as P[token][head], read back as P[4*q4 + i][h]
//   V  rows 4*q4 + i (i = 0..3), elements 8a .. 8a+7: fp32 FMAs into
//      acc[h][e], a partial over the lane's 4 tokens, summed over q4 at the
//      end of the item.
// The softmax state is the same (exact running max, base 2, scale folded in).
template <int D, int DT, int PF, int GV>
struct ValuWave : MfmaWave<D, DT, PF, 1> {
  using Base = MfmaWave<D, DT, PF, 1>;
  using Buf = typename Base::Buf;
  using Ops = MfmaOps<DT>;
  static_assert(D == 128, "the VALU comparison kernel serves head_dim 128");
  uint32_t qk[GV][4];
  float vm[GV], vl[GV];
  float vacc[GV][8];

  __device__ __forceinline__ static float dot2(uint32_t x, uint32_t y, float c) {
    if constexpr (DT == QD_DTYPE_BF16)
      return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x), __builtin_bit_cast(bf16x2, y), c, false);
    else
      return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, x), __builtin_bit_cast(f16x2, y), c, false);
  }
  __device__ __forceinline__ static void unpack2(uint32_t w, float& lo, float& hi) {
    if constexpr (DT == QD_DTYPE_BF16) {
      lo = __uint_as_float(w << 16);
      hi = __uint_as_float(w & 0xFFFF0000u);
    } else {
      const f32x2 v = __builtin_convertvector(__builtin_bit_cast(f16x2, w), f32x2);
      lo = v[0];
      hi = v[1];
    }
  }

  __device__ __forceinline__ void begin_item(const DecodeParams& p, int b, int kvh, int valid_tokens, int g_first) {
    const int a = this->r16;
    this->trow = p.table + static_cast<int64_t>(b) * p.maxP;
    this->wbase = g_first / (p.P >> 4);
    this->tblv = (this->lane < p.maxP - this->wbase) ? this->trow[this->wbase + this->lane] : 0;
#pragma unroll
    for (int h = 0; h < GV; ++h) {
      const bool ok = h < p.g;
      const char* qp = static_cast<const char*>(p.q) +
                       (static_cast<int64_t>(b) * p.Hq + kvh * p.g + (ok ? h : 0)) * D * 2 + 16 * a;
      const u32x4 x = *reinterpret_cast<const u32x4*>(qp);
#pragma unroll
      for (int w = 0; w < 4; ++w) qk[h][w] = ok ? x[w] : 0u;
      vm[h] = -INFINITY;
      vl[h] = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) vacc[h][e] = 0.f;
    }
    const int64_t col = p.kv_split > 1 ? kvh / p.kv_split : kvh;
    this->kbase = static_cast<const char*>(p.k) + col * D * 2;
    this->vbase = static_cast<const char*>(p.v) + col * D * 2;
    this->len = valid_tokens;
  }

  // ptile: this wave's LDS area (KTile<D>::kBytes >= 16 x 16 floats).
  __device__ __forceinline__ void compute(const DecodeParams& p, const Buf& buf, char* ptile) {
    const int a = this->r16, r = this->q4;
    const int last = this->len - 1 - buf.tg;
    float s[4][GV];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const u32x4 kv = buf.k[0][c];
#pragma unroll
      for (int h = 0; h < GV; ++h) {
        float d = dot2(kv[0], qk[h][0], 0.f);
        d = dot2(kv[1], qk[h][1], d);
        d = dot2(kv[2], qk[h][2], d);
        s[c][h] = row16_sum(dot2(kv[3], qk[h][3], d));
      }
    }
    float* P = reinterpret_cast<float*>(ptile);
    bool rescale = false;
    float alpha[GV];
#pragma unroll
    for (int h = 0; h < GV; ++h) {
      float mx = -INFINITY;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        s[c][h] = (4 * c + r <= last) ? s[c][h] * p.sl2 : -INFINITY;
        mx = fmaxf(mx, s[c][h]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mn = fmaxf(vm[h], mx);
      const float mref = mn == -INFINITY ? 0.f : mn;
      alpha[h] = fast_exp2(vm[h] - mref);
      rescale |= alpha[h] != 1.f;
      float lsum = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        s[c][h] = fast_exp2(s[c][h] - mref);
        lsum += s[c][h];
      }
      vl[h] = fmaf(vl[h], alpha[h], lsum);
      vm[h] = mn;
    }
    // P[token][head]: lane a < GV of row r writes its head's 4 weights.
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float w = 0.f;
#pragma unroll
      for (int h = 0; h < GV; ++h) w = (a == h) ? s[c][h] : w;
      if (a < GV) P[(4 * c + r) * 16 + a] = w;
    }
    if (__builtin_amdgcn_read_exec() & __ballot(rescale)) {
#pragma unroll
      for (int h = 0; h < GV; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) vacc[h][e] *= alpha[h];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v[8];
#pragma unroll
      for (int w = 0; w < 4; ++w) unpack2(buf.v[0][i].w[w], v[2 * w], v[2 * w + 1]);
      const float* prow = P + (4 * r + i) * 16;
#pragma unroll
      for (int h = 0; h < GV; ++h) {
        const float ph = prow[h];
#pragma unroll
        for (int e = 0; e < 8; ++e) vacc[h][e] = fmaf(ph, v[e], vacc[h][e]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  // Same structure as MfmaWave::run, with this compute.
  __device__ __forceinline__ void run(const DecodeParams& p, int ga, int gb, char* ptile, bool = false) {
    const int gpp = p.P >> 4;
    for (int g_lo = ga; g_lo < gb;) {
      if (g_lo != ga) {
        this->wbase = g_lo / gpp;
        this->tblv = (this->lane < p.maxP - this->wbase) ? this->trow[this->wbase + this->lane] : 0;
      }
      const int g_hi = min(gb, (this->wbase + 64) * gpp);
      const int n = g_hi - g_lo;
      Buf buf[PF];
      int i = 0;
      if (n >= 2 * PF - 1) {
#pragma unroll
        for (int u = 0; u < PF - 1; ++u) this->issue(p, buf[u], g_lo + u);
        for (; i + 2 * PF - 2 < n; i += PF) {
#pragma unroll
          for (int u = 0; u < PF; ++u) {
            this->issue(p, buf[(u + PF - 1) % PF], g_lo + i + u + PF - 1);
            compute(p, buf[u], ptile);
          }
        }
      } else {
#pragma unroll
        for (int u = 0; u < PF - 1; ++u)
          if (u < n) this->issue(p, buf[u], g_lo + u);
      }
      for (; i < n; i += PF) {
#pragma unroll
        for (int u = 0; u < PF; ++u) {
          if (i + u + PF - 1 < n) this->issue(p, buf[(u + PF - 1) % PF], g_lo + i + u + PF - 1);
          if (i + u < n) compute(p, buf[u], ptile);
        }
      }
      g_lo = g_hi;
    }
  }

  // Sums the lane partials over the four token rows (q4) and, for head h,
  // returns the softmax denominator; acc becomes the full output slice.
  __device__ __forceinline__ void finish_item() {
#pragma unroll
    for (int h = 0; h < GV; ++h) {
      vl[h] += __shfl_xor(vl[h], 16);
      vl[h] += __shfl_xor(vl[h], 32);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        vacc[h][e] += __shfl_xor(vacc[h][e], 16);
        vacc[h][e] += __shfl_xor(vacc[h][e], 32);
      }
    }
  }

  __device__ __forceinline__ void store_direct(const DecodeParams& p, int b, int kvh) {
    using S = typename Elem<DT>::S;
    if (this->q4 != 0) return;
#pragma unroll
    for (int h = 0; h < GV; ++h) {
      if (h >= p.g) break;
      const float inv = vl[h] > 0.f ? 1.f / vl[h] : 0.f;
      uint32_t wv[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2)
        wv[e / 2] = Ops::pack2(vl[h] > 0.f ? vacc[h][e] * inv : 0.f, vl[h] > 0.f ? vacc[h][e + 1] * inv : 0.f);
      S* o = static_cast<S*>(p.out) + (static_cast<int64_t>(b) * p.Hq + kvh * p.g + h) * D + 8 * this->r16;
      *reinterpret_cast<u32x4*>(o) = u32x4{wv[0], wv[1], wv[2], wv[3]};
    }
  }

  // Partial rows {m (natural log), l, acc[D]} of the kv-head's heads, head h at w + h*(D+2).
  __device__ __forceinline__ void store_partial(const DecodeParams& p, float* w) {
    if (this->q4 != 0) return;
#pragma unroll
    for (int h = 0; h < GV; ++h) {
      if (h >= p.g) break;
      float* row = w + static_cast<int64_t>(h) * (D + 2);
      if (this->r16 == 0) *reinterpret_cast<f32x2*>(row) = f32x2{vm[h] * kLn2, vl[h]};
#pragma unroll
      for (int e = 0; e < 8; e += 2)
        *reinterpret_cast<f32x2*>(row + 2 + 8 * this->r16 + e) = f32x2{vacc[h][e], vacc[h][e + 1]};
    }
  }
};

// Explicit split layout.  grid: (splits, Hkv, B), block 64 (one wave per
// (sequence, kv-head, split)).  Split z of a sequence covers whole pages
// (chunk_info); a sequence with a single non-empty split is written
// directly, otherwise every non-empty split writes its partial to
// ws[b, h, z, :] for the split merge (combine_rows_kernel / combine_kernel).
template <int D, int DT, int PF>
__global__ __launch_bounds__(64) void decode_mfma_kernel(DecodeParams p) {
  const int z = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const ChunkInfo ci = chunk_info(p, p.lens[b], z);
  if (z >= (ci.nch > 1 ? ci.nch : 1)) return;

  __shared__ __align__(16) char ktile[KTile<D>::kBytes];
  MfmaWave<D, DT, PF, 1> wv;
  wv.init_lane();
  wv.begin_item(p, b, kvh, ci.te, ci.tb >> 4);
  wv.run(p, ci.tb >> 4, (ci.te + 15) >> 4, ktile);  // tb is page aligned
  const float l_tot = wv.total_l(0);
  if (ci.nch <= 1) {
    wv.store_direct(p, b, kvh, 0, l_tot);
  } else {
    float* w = p.ws + ((static_cast<int64_t>(b) * p.Hq + kvh * p.g) * p.splits + z) * (D + 2);
    wv.store_partial(p, 0, w, static_cast<int64_t>(p.splits) * (D + 2), l_tot);
  }
}

// 16-token groups of a sequence with `len` valid tokens.
__device__ __forceinline__ int seq_groups(const DecodeParams& p, int len_raw) {
  return (clamp_len(p, len_raw) + 15) >> 4;
}

// Merge of partial rows, in place of the reference's merge kernel
// (gqa_decode.cu:74-87).  Each partial row is {m (natural log), l, acc[D]};
// a lane group folds its rows in order with SoftmaxState::merge
// (online_softmax.cuh:17-24): a row with l == 0 is skipped, the running
// state is rescaled by exp(m - max).  Output acc/l rounded once, zeros when
// l == 0 (gqa_decode.cu:84-86).  Each 16-lane group (j4 = lane / 16) holds
// one head's state, D/16 consecutive elements per lane (one vector store):
// four heads per wave, or one head whose rows the four groups share
// (combine_groups).  Partials from an earlier kernel on the same stream are
// read with plain loads; COH: sc1 loads, for partials that other workgroups
// of the same launch wrote with sc1 stores.
template <int D, int KB, bool COH = false>
struct MergeRows {
  static constexpr int EPL = D / 16;
  static constexpr int kBatch = KB;  // rows loaded per memory round trip
  int c16;
  float M = -INFINITY, L = 0.f;
  float acc[EPL];
  float ms[kBatch], ls[kBatch], av[kBatch][EPL];

  __device__ MergeRows() : c16(threadIdx.x & 15) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
  }

  // Loads row t < kBatch of the batch from `row` (the lane's head) when
  // `present` (uniform over the lane's 16-lane group).
  __device__ void load(int t, bool present, const float* row) {
    ms[t] = -INFINITY;
    ls[t] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) av[t][e] = 0.f;
    if (present) {
      // Rows are D+2 floats (D even): every pair is 8-byte aligned.
      const f32x2 ml = COH ? coherent_load2(row) : *reinterpret_cast<const f32x2*>(row);
      ms[t] = ml[0];
      ls[t] = ml[1];
#pragma unroll
      for (int e = 0; e < EPL; e += 2) {
        const float* src = row + 2 + c16 * EPL + e;
        const f32x2 x = COH ? coherent_load2(src) : *reinterpret_cast<const f32x2*>(src);
        av[t][e] = x[0];
        av[t][e + 1] = x[1];
      }
    }
  }

  // Folds rows t < n of the loaded batch, in order.
  __device__ void fold(int n) {
#pragma unroll
    for (int t = 0; t < kBatch; ++t) {
      if (t >= n || ls[t] == 0.f) continue;
      const float mn = fmaxf(M, ms[t]);
      const float a = L == 0.f ? 0.f : fast_exp2((M - mn) * kLog2e);
      const float bb = fast_exp2((ms[t] - mn) * kLog2e);
      L = a * L + bb * ls[t];
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[e] = a * acc[e] + bb * av[t][e];
      M = mn;
    }
  }

  // Folds `nrows` rows at base + r*row_stride (the lane's head), kBatch
  // rows per round trip; only rows that exist are loaded.
  __device__ void fold_rows(const float* base, int64_t row_stride, int nrows) {
    for (int s0 = 0; s0 < nrows; s0 += kBatch) {
#pragma unroll
      for (int t = 0; t < kBatch; ++t) load(t, s0 + t < nrows, base + static_cast<int64_t>(s0 + t) * row_stride);
      fold(nrows - s0);
    }
  }

  // Folds the states of the four 16-lane groups (which hold the same head
  // and columns, over different rows) into each lane: two butterfly
  // exchanges, each a SoftmaxState::merge (online_softmax.cuh:17-24).
  __device__ void combine_groups() {
#pragma unroll
    for (int off = 16; off <= 32; off *= 2) {
      const float mo = __shfl_xor(M, off);
      const float lo = __shfl_xor(L, off);
      float ao[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) ao[e] = __shfl_xor(acc[e], off);
      if (lo == 0.f) continue;
      const float mn = fmaxf(M, mo);
      const float a = L == 0.f ? 0.f : fast_exp2((M - mn) * kLog2e);
      const float bb = fast_exp2((mo - mn) * kLog2e);
      L = a * L + bb * lo;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[e] = a * acc[e] + bb * ao[e];
      M = mn;
    }
  }

  // Writes head j4's output row at out (when the head exists); out is
  // 16-byte aligned (8-byte for 16-bit rows of D = 64).
  template <int DT>
  __device__ void store(bool active, typename Elem<DT>::S* out) const {
    if (!active) return;
    const float inv = L > 0.f ? 1.f / L : 0.f;
    if constexpr (DT == QD_DTYPE_F32) {
      static_assert(EPL % 4 == 0, "fp32 rows: head_dim a multiple of 64");
      float* dst = out + c16 * EPL;
#pragma unroll
      for (int e = 0; e < EPL; e += 4)
        *reinterpret_cast<f32x4*>(dst + e) = f32x4{L > 0.f ? acc[e] * inv : 0.f, L > 0.f ? acc[e + 1] * inv : 0.f,
                                                   L > 0.f ? acc[e + 2] * inv : 0.f, L > 0.f ? acc[e + 3] * inv : 0.f};
    } else {
      uint32_t wv[EPL / 2];
#pragma unroll
      for (int e = 0; e < EPL; e += 2)
        wv[e / 2] = MfmaOps<DT>::pack2(L > 0.f ? acc[e] * inv : 0.f, L > 0.f ? acc[e + 1] * inv : 0.f);
      store_words<EPL / 2>(reinterpret_cast<char*>(out + c16 * EPL), wv);
    }
  }
};

constexpr int kMaxWgWaves = 8;

// Waves per stream-K workgroup at most: 8 serving one kv-head each, or 4
// (one per SIMD, so each may use 512 registers) serving two each, with
// head_dim 256, or with 3 groups in flight above head_dim 64.
#ifndef QD_VALU_WAVES
#define QD_VALU_WAVES 8
#endif
#ifndef QD_VALU_PF
#define QD_VALU_PF 1
#endif
// The VALU comparison variant holds more state per wave (scores for every
// head, fp32 output slices): QD_VALU_WAVES waves per workgroup at most and
// QD_VALU_PF groups in flight.  Measured on cfg2/cfg5/cfg3 and a group-8
// shape, 8 waves with one group in flight was its fastest form (4 waves with
// 2 or 3 groups, one wave per SIMD and 512 registers, were 9-32% slower; 8
// waves with 2 groups spill).
constexpr int kValuMaxWaves = QD_VALU_WAVES;
constexpr int kValuPrefetch = QD_VALU_PF;

template <int D, int NKV, int GV = 0, int PF = 2, int DT = QD_DTYPE_BF16>
constexpr int sk_max_waves() {
  if (GV > 0) return kValuMaxWaves;
  if (DT == QD_DTYPE_F32) return D <= 64 ? kMaxWgWaves : kMaxWgWaves / 2;  // fp32 head_dim 128: 512 registers
  return (NKV == 1 && D <= 128 && (PF <= 2 || D <= 64)) ? kMaxWgWaves : kMaxWgWaves / 2;
}

#ifndef QD_SK_SEQ_COST
#define QD_SK_SEQ_COST 6
#endif
// Partition cost units: a 16-token group costs kSkGroupCost, and every
// non-empty sequence adds kSkSeqCost at its start for the pipeline refill
// (page-table window and first K/V round trips) that the workgroup entering
// it pays; measured at about one group's streaming time.
constexpr int64_t kSkGroupCost = 4;
constexpr int64_t kSkSeqCost = QD_SK_SEQ_COST;

__device__ __forceinline__ int64_t seq_cost(int groups) {
  return groups > 0 ? kSkGroupCost * groups + kSkSeqCost : 0;
}

// Fused merge of one (sequence, kv-head item) by the wave that arrived last
// (see decode_mfma_sk_kernel): heads [h_begin, h_begin + nheads) of sequence
// b, from the partial slots first+b .. first+b+nwg-1 written with sc1 stores
// by the workgroups that hold the sequence.  Same fold as merge_sk_kernel
// (SoftmaxState::merge, online_softmax.cuh:17-24; output as
// gqa_decode.cu:84-86): four heads per pass (16 lanes each, D/16 columns
// per lane), sc1 buffer loads addressed by one VGPR offset per lane and a
// scalar row offset, fused_merge_rows() rows per memory round trip.
template <int D>
constexpr int fused_merge_rows() {
  return D <= 128 ? 16 : 8;
}

template <int D, int DT>
__device__ void merge_item_fused(const DecodeParams& p, int b, int h_begin, int nheads, int first, int nwg) {
  using S = typename Elem<DT>::S;
  constexpr int EPL = D / 16;
  constexpr int KB = fused_merge_rows<D>();
  const int lane = threadIdx.x & 63;
  const int j4 = lane >> 4;
  const int c16 = lane & 15;
  const uint32_t slot_bytes = static_cast<uint32_t>(p.Hq) * (D + 2) * 4;
  const float* slots = p.ws + static_cast<int64_t>(first + b) * p.Hq * (D + 2);
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(slots, static_cast<uint32_t>(nwg) * slot_bytes);
  for (int h4 = 0; h4 < nheads; h4 += 4) {
    const bool active = h4 + j4 < nheads;
    const int h = h_begin + (active ? h4 + j4 : 0);
    const uint32_t v_ml = static_cast<uint32_t>(h) * (D + 2) * 4;  // {m, l} of the lane's head
    const uint32_t v_acc = v_ml + 8 + c16 * EPL * 4;               // its columns of acc
    float M = -INFINITY, L = 0.f;
    float acc[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
    for (int s0 = 0; s0 < nwg; s0 += KB) {
      // Every row slot of the batch is loaded (rows past the last repeat
      // it, unused), so the loads form one branch-free clause.
      float ms[KB], ls[KB], av[KB][EPL];
#pragma unroll
      for (int t = 0; t < KB; ++t) {
        const uint32_t so = static_cast<uint32_t>(min(s0 + t, nwg - 1)) * slot_bytes;
        const f32x2 ml = coherent_buffer_load2(rs, v_ml, so);
        ms[t] = ml[0];
        ls[t] = ml[1];
#pragma unroll
        for (int e = 0; e < EPL; e += 2) {
          const f32x2 x = coherent_buffer_load2(rs, v_acc + 4 * e, so);
          av[t][e] = x[0];
          av[t][e + 1] = x[1];
        }
      }
#pragma unroll
      for (int t = 0; t < KB; ++t) {
        if (s0 + t >= nwg || ls[t] == 0.f) continue;
        const float mn = fmaxf(M, ms[t]);
        const float a = L == 0.f ? 0.f : fast_exp2((M - mn) * kLog2e);
        const float bb = fast_exp2((ms[t] - mn) * kLog2e);
        L = a * L + bb * ls[t];
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[e] = a * acc[e] + bb * av[t][e];
        M = mn;
      }
    }
    if (active) {
      const float inv = L > 0.f ? 1.f / L : 0.f;
      uint32_t wv[EPL / 2];
#pragma unroll
      for (int e = 0; e < EPL; e += 2)
        wv[e / 2] = MfmaOps<DT>::pack2(L > 0.f ? acc[e] * inv : 0.f, L > 0.f ? acc[e + 1] * inv : 0.f);
      store_words<EPL / 2>(
          reinterpret_cast<char*>(static_cast<S*>(p.out) + (static_cast<int64_t>(b) * p.Hq + h) * D + c16 * EPL), wv);
    }
  }
}

// Arrival of this wave's item (sequence b, kv-heads kvh0..) at its counter:
// lane 0 increments it with wrap-around at nwg - 1 (the last of the nwg
// arrivals reads nwg - 1 and leaves 0 behind).  Returns the value read.
__device__ __forceinline__ uint32_t arrive(const DecodeParams& p, int b, int kvh0, int nwg) {
  uint32_t old = 0;
  if ((threadIdx.x & 63) == 0)
    old = __builtin_amdgcn_atomic_inc32(p.ctr + static_cast<int64_t>(b) * p.Hkv + kvh0, static_cast<uint32_t>(nwg - 1),
                                        __ATOMIC_RELAXED, "agent");
  return old;
}

// Balanced ("stream-K") layout.  grid: W = p.splits workgroups of
// p.wg_waves waves; wave j of a workgroup serves kv-heads j*NKV .. j*NKV +
// NKV-1, then the same plus wg_waves*NKV, ... so that a workgroup reads
// whole cache rows (all kv-heads of a token) at once, which streams faster
// from HBM than kv-head slices read at unrelated times.
//
// Sequence b has n_b = ceil(len_b/16) groups and costs c_b = U*n_b + V
// cost units (U = kSkGroupCost, V = kSkSeqCost; 0 when n_b = 0).  The
// sequences are laid end to end into C = sum_b c_b units: sequence b spans
// [C_b, C_b + c_b), its first V units are the start cost and group i owns
// unit x_{b,i} = C_b + V + U*i.  The first Wu = min(W, C/U) workgroups take
// the unit ranges [w*C/Wu, (w+1)*C/Wu) (each at least U long, so every
// workgroup between the holders of a sequence's first and last group holds
// at least one of its groups) and process the groups whose unit they hold.
// For every sequence it touches, a workgroup either writes the output rows
// directly (it holds the whole sequence) or writes a partial for all Hq
// heads into slot (w + b) of the workspace (Hq*(D+2) floats per slot; the
// slot is unique per (sequence, workgroup) because the workgroups of
// sequence b+1 start at or after the last one of b, so W + B slots
// suffice).  Rows of empty sequences are zero-filled by workgroup b % W.
//
// Only the first and the last sequence of a workgroup's range can be split
// (every sequence in between lies wholly inside the range).  The split
// sequences are merged either by merge_sk_kernel (FUSED = false; the
// workgroup holding a sequence's first group records its span in p.meta)
// or here (FUSED = true): every wave stores its partials with sc1 stores,
// and after its whole range it waits for them to retire and arrives at the
// counter of each of its split items (sequence, kv-heads); the arrival
// that completes a counter (the nwg-th) merges that item's heads from all
// nwg slots and resets the counter to zero.  No wave ever waits for
// another, and the counters are left as they were found (zero).
template <int D, int DT, int PF, int NKV, int GV = 0, bool FUSED = false, bool HOLD = false>
__global__ __launch_bounds__((64 * sk_max_waves<D, NKV, GV, PF, DT>())) void decode_mfma_sk_kernel(DecodeParams p) {
  static_assert(!(HOLD && (FUSED || GV > 0)), "results are held only by the MFMA kernel with the merge kernel");
  using S = typename Elem<DT>::S;
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int nw = p.wg_waves;
  const int w = blockIdx.x;
  const int W = p.splits;
  const int B = p.B;
  static_assert(DT != QD_DTYPE_F32 || (NKV == 1 && GV == 0 && !FUSED), "fp32 caches: one kv-head per wave, merge kernel");
  __shared__ __align__(16) char ktile[sk_max_waves<D, NKV, GV, PF, DT>()][KTile<D, DT == QD_DTYPE_F32 ? 4 : 2>::kBytes];
  QD_STAMP(p, 0, stamp_now());
  QD_STAMP(p, 8, stamp_clock());
  QD_STAMP(p, 6, stamp_xcc());

  // Prologue, one memory round trip for B <= 64*kRegChunks: every lane loads
  // the lengths of sequences c*64 + lane, and the group counts and the
  // running sums of the costs stay in registers.
  constexpr int kRegChunks = 4;
  int len_r[kRegChunks];
  int n_r[kRegChunks];
  int64_t incl_r[kRegChunks];
#pragma unroll
  for (int c = 0; c < kRegChunks; ++c) {
    const int bb = c * 64 + lane;
    len_r[c] = bb < B ? clamp_len(p, p.lens[bb]) : 0;
    n_r[c] = (len_r[c] + 15) >> 4;
  }
  // Chunks past the batch hold zeros and are not scanned.
  int64_t carry = 0;
#pragma unroll
  for (int c = 0; c < kRegChunks; ++c) {
    incl_r[c] = carry;
    if (c == 0 || c * 64 < B) {
      incl_r[c] += wave_incl_scan_small(seq_cost(n_r[c]), lane);
      carry = readlane_i64(incl_r[c], 63);
    }
  }
  for (int c = 64 * kRegChunks; c < B; c += 64) {  // larger batches: re-read
    const int bb = c + lane;
    carry += wave_sum_i64(seq_cost(bb < B ? seq_groups(p, p.lens[bb]) : 0));
  }
  const int64_t C = carry;

  // Empty sequences (no workgroup holds them): workgroup b % W writes their
  // zero rows (and, for merge_sk_kernel, a meta entry that says to skip them).
  auto zero_fill = [&](uint64_t mask, int c0) {
    while (mask) {
      const int bb = c0 + __builtin_ctzll(mask);
      mask &= mask - 1;
      S* o = static_cast<S*>(p.out) + static_cast<int64_t>(bb) * p.Hq * p.D;
      for (int i = threadIdx.x; i < p.Hq * p.D; i += 64 * nw) o[i] = Elem<DT>::from_f(0.f);
      if (!FUSED && threadIdx.x == 0) {
        p.meta[2 * bb] = 0;
        p.meta[2 * bb + 1] = 0;
      }
    }
  };
#pragma unroll
  for (int c = 0; c < kRegChunks; ++c) {
    const int bb = c * 64 + lane;
    zero_fill(__ballot(bb < B && n_r[c] == 0 && bb % W == w), c * 64);
  }
  for (int c = 64 * kRegChunks; c < B; c += 64) {
    const int bb = c + lane;
    zero_fill(__ballot(bb < B && bb % W == w && seq_groups(p, p.lens[bb]) == 0), c);
  }

  // Workgroups in use (uniform across the grid).
  const int64_t wu_cap = C / kSkGroupCost;
  const int Wu = static_cast<int>(wu_cap < W ? (wu_cap > 0 ? wu_cap : 1) : W);
  if (w >= Wu || C == 0) return;
  const int64_t c0 = div_nonneg(static_cast<int64_t>(w) * C, Wu);
  const int64_t c1 = div_nonneg(static_cast<int64_t>(w + 1) * C, Wu);

  // The sequence whose unit range holds c0 (the first whose running cost
  // end exceeds c0) and its first unit cs; its clamped length comes from the
  // registers when the prologue holds it.
  int b = B;
  int64_t cs = 0;
  int len_first = -1;
#pragma unroll
  for (int c = 0; c < kRegChunks; ++c) {
    if (b == B && c * 64 < B) {
      const int bb = c * 64 + lane;
      const int cnt = __popcll(__ballot(bb < B && incl_r[c] <= c0));
      if (cnt < min(64, B - c * 64)) {
        b = c * 64 + cnt;
        cs = readlane_i64(incl_r[c] - seq_cost(n_r[c]), cnt);
        len_first = __builtin_amdgcn_readlane(len_r[c], cnt);
      }
    }
  }
  if (b == B) {
    carry = readlane_i64(incl_r[kRegChunks - 1], 63);
    for (int c = 64 * kRegChunks; c < B; c += 64) {
      const int bb = c + lane;
      const int64_t n = bb < B ? seq_cost(seq_groups(p, p.lens[bb])) : 0;
      const int64_t incl = carry + wave_incl_scan_small(n, lane);
      const int cnt = __popcll(__ballot(bb < B && incl <= c0));
      if (cnt < min(64, B - c)) {
        b = c + cnt;
        cs = readlane_i64(incl - n, cnt);
        break;
      }
      carry = readlane_i64(incl, 63);
    }
  }
  if (b >= B) return;  // unreachable when C is consistent
  QD_STAMP(p, 1, stamp_now());

  // Workgroup whose unit range holds unit x.
  auto wg_of = [&](int64_t x) { return static_cast<int>(div_nonneg((x + 1) * Wu - 1, C)); };
  // Groups of the current sequence whose unit lies below x.
  auto groups_below = [&](int64_t x, int64_t x0, int nb) {
    if (x <= x0) return 0;
    const int64_t i = (x - x0 + kSkGroupCost - 1) / kSkGroupCost;
    return static_cast<int>(i < nb ? i : nb);
  };

  // GV > 0: the VALU comparison variant (ValuWave, GV heads per group).
  using Wave = std::conditional_t<
      GV == 0,
      std::conditional_t<DT == QD_DTYPE_F32, MfmaWaveF32<D, PF>, MfmaWave<D, DT, PF, NKV>>,
      ValuWave<D, DT, PF, (GV > 0 ? GV : 4)>>;
  Wave wv;
  wv.init_lane();
  const int64_t slot_floats = static_cast<int64_t>(p.Hq) * (D + 2);
  // FUSED: the split sequences of this range, {sequence, first workgroup,
  // workgroups}; the second is used when the range ends inside a sequence.
  int sp_b0 = -1, sp_f0 = 0, sp_n0 = 0, sp_b1 = -1, sp_f1 = 0, sp_n1 = 0;
  bool sp_stashed = false;  // the first split sequence's partials wait in LDS
  // Dynamic LDS, per wave: FUSED, the stash (one item per kv-head group the
  // wave serves); otherwise the staged result rows (NKV*g rows of D+2
  // floats).
  extern __shared__ __align__(16) float qd_dyn_lds[];
  float* stash = nullptr;
  if constexpr (FUSED && GV == 0) {
    const int items = (p.Hkv + nw * NKV - 1) / (nw * NKV);
    stash = qd_dyn_lds + static_cast<int64_t>(wid) * items * NKV * Wave::kStashFields * 64;
  } else if constexpr (HOLD) {
    wv.res_cap = p.stage_bytes - Wave::kStageHeader;
    wv.res_lds = reinterpret_cast<char*>(qd_dyn_lds) + static_cast<int64_t>(wid) * p.stage_bytes;
  }
  while (true) {
    const int len = len_first >= 0 ? len_first : clamp_len(p, p.lens[b]);
    len_first = -1;
    const int nb = (len + 15) >> 4;
    const int64_t x0 = cs + kSkSeqCost;  // unit of group 0
    const int i0 = groups_below(c0, x0, nb);
    const int i1 = groups_below(c1, x0, nb);
    if (i1 > i0) {
      const bool whole = i0 == 0 && i1 == nb;
      // The range goes on past this sequence (only its first sequence can
      // then be split).
      const bool mid_range = cs + seq_cost(nb) < c1;
      if (FUSED && !whole && mid_range) sp_stashed = true;
      float* slot = p.ws + static_cast<int64_t>(w + b) * slot_floats;
      for (int kvh0 = wid * NKV; kvh0 < p.Hkv; kvh0 += nw * NKV) {
        wv.begin_item(p, b, kvh0, len, i0);
        // Every wave runs exactly one item here when the workgroup's waves
        // cover the kv-heads once, so all reach the same barriers.
        wv.run(p, i0, i1, ktile[wid], p.Hkv == nw * NKV);
        if constexpr (GV == 0 && FUSED) {
#pragma unroll
          for (int j = 0; j < NKV; ++j) {
            const float l_tot = wv.total_l(j);
            if (whole)
              wv.store_direct(p, b, kvh0, j, l_tot);
            else if (mid_range)
              wv.stash_partial(j, stash + ((kvh0 - wid * NKV) / (nw * NKV)) * NKV * Wave::kStashFields * 64, l_tot);
            else
              wv.template store_partial<true>(p, j, slot + static_cast<int64_t>(vhead_base(p, kvh0 + j)) * (D + 2),
                                               D + 2, l_tot);
          }
        } else if constexpr (GV == 0 && !HOLD) {
#pragma unroll
          for (int j = 0; j < NKV; ++j) {
            const float l_tot = wv.total_l(j);
            if (whole)
              wv.store_direct(p, b, kvh0, j, l_tot);
            else
              wv.store_partial(p, j, slot + static_cast<int64_t>(vhead_base(p, kvh0 + j)) * (D + 2), D + 2, l_tot);
          }
        } else if constexpr (HOLD) {
          // The item's heads (fewer than NKV * g for a short last chunk of
          // a split kv-head): the flush writes exactly these rows.
          const int nheads = p.kv_split > 1 ? wv.hcount : NKV * p.g;
          const int bytes = whole ? nheads * D * static_cast<int>(sizeof(S)) : nheads * (D + 2) * 4;
          char* area = wv.stage_slot(bytes);
#pragma unroll
          for (int j = 0; j < NKV; ++j) {
            const float l_tot = wv.total_l(j);
            if (whole)
              wv.stage_direct(p, area, j, l_tot);
            else
              wv.stage_partial(p, area, j, l_tot);
          }
          if (whole)
            wv.stage_commit(reinterpret_cast<char*>(static_cast<S*>(p.out) +
                                                    (static_cast<int64_t>(b) * p.Hq + vhead_base(p, kvh0)) * D),
                            bytes, 16);
          else
            wv.stage_commit(reinterpret_cast<char*>(slot + static_cast<int64_t>(vhead_base(p, kvh0)) * (D + 2)),
                            bytes, 8);
        } else {
          wv.finish_item();
          if (whole)
            wv.store_direct(p, b, kvh0);
          else
            wv.store_partial(p, slot + static_cast<int64_t>(vhead_base(p, kvh0)) * (D + 2));
        }
      }
      if constexpr (FUSED) {
        if (!whole) {
          const int first = wg_of(x0);
          const int nwg = wg_of(x0 + kSkGroupCost * (nb - 1)) - first + 1;
          if (sp_b0 < 0) {
            sp_b0 = b;
            sp_f0 = first;
            sp_n0 = nwg;
          } else {
            sp_b1 = b;
            sp_f1 = first;
            sp_n1 = nwg;
          }
        }
      } else {
        // The workgroup holding a sequence's first group records which
        // workgroups span it, for merge_sk_kernel (also for a whole sequence,
        // so that nothing from an earlier call survives); wave 0 holds the
        // entry back with its result rows.
        if (i0 == 0 && wid == 0) {
          const int first = wg_of(x0);
          const int count = wg_of(x0 + kSkGroupCost * (nb - 1)) - first + 1;
          if constexpr (HOLD) {
            char* area = wv.stage_slot(8);
            if (lane == 0) *reinterpret_cast<int2*>(area) = make_int2(first, count);
            wv.stage_commit(reinterpret_cast<char*>(p.meta + 2 * b), 8, 8);
          } else if (lane == 0) {
            p.meta[2 * b] = first;
            p.meta[2 * b + 1] = count;
          }
        }
      }
    }
    cs += seq_cost(nb);
    if (cs >= c1) break;
    do {
      ++b;
    } while (b < B && p.lens[b] <= 0);
    if (b >= B) break;  // unreachable when C is consistent
  }
  if constexpr (HOLD) wv.flush_results();  // the range's held items
  QD_STAMP(p, 2, stamp_now());
  QD_STAMP(p, 9, stamp_clock());

  if constexpr (FUSED && GV == 0) {
    if (sp_b0 >= 0) {
      if (sp_stashed) {
        float* slot0 = p.ws + static_cast<int64_t>(w + sp_b0) * slot_floats;
        for (int kvh0 = wid * NKV; kvh0 < p.Hkv; kvh0 += nw * NKV) {
          const float* st = stash + ((kvh0 - wid * NKV) / (nw * NKV)) * NKV * Wave::kStashFields * 64;
#pragma unroll
          for (int j = 0; j < NKV; ++j)
            wv.store_stashed(p, j, st, slot0 + static_cast<int64_t>(vhead_base(p, kvh0 + j)) * (D + 2), D + 2);
        }
      }
      wait_memory_retired();  // this wave's sc1 partial stores are visible device-wide
      QD_STAMP(p, 3, stamp_now());
      int merged = 0;
      for (int kvh0 = wid * NKV; kvh0 < p.Hkv; kvh0 += nw * NKV) {
        // Both arrivals are issued before either result is used.
        const uint32_t o0 = arrive(p, sp_b0, kvh0, sp_n0);
        const uint32_t o1 = sp_b1 >= 0 ? arrive(p, sp_b1, kvh0, sp_n1) : 0u;
        const bool last0 = __builtin_amdgcn_readfirstlane(o0) == static_cast<uint32_t>(sp_n0 - 1);
        const bool last1 = sp_b1 >= 0 && __builtin_amdgcn_readfirstlane(o1) == static_cast<uint32_t>(sp_n1 - 1);
        QD_STAMP(p, 4, stamp_now());
        if (last0) merge_item_fused<D, DT>(p, sp_b0, kvh0 * p.g, NKV * p.g, sp_f0, sp_n0);
        if (last1) merge_item_fused<D, DT>(p, sp_b1, kvh0 * p.g, NKV * p.g, sp_f1, sp_n1);
        merged += static_cast<int>(last0) + static_cast<int>(last1);
      }
      QD_STAMP(p, 5, stamp_now());
      QD_STAMP(p, 7, static_cast<uint64_t>(merged));
    }
  }
}

// Stream-K merge of sequence b = blockIdx.y from slots first+b ..
// first+b+nwg-1 (its meta entry), block 64.  Two dependent memory round
// trips: the meta entry, then the partial rows.
//   RG = 1: grid (ceil(Hq/4), B); one wave merges heads 4*blockIdx.x + j4
//           (16 lanes per head), KB rows per round trip.  For batches whose
//           sequences are split over few workgroups.
//   RG = 4: grid (Hq, B); one wave merges head blockIdx.x, lane group j4
//           folds rows j4, j4+4, ... (4*KB rows per round trip), then the
//           four group states are combined.  For sequences split over many
//           workgroups.
template <int D, int DT, int KB, int RG>
__global__ __launch_bounds__(64) void merge_sk_kernel(DecodeParams p) {
  using S = typename Elem<DT>::S;
  const int b = blockIdx.y;
  const int first = p.meta[2 * b];
  const int nwg = p.meta[2 * b + 1];
  if (nwg <= 1) return;  // written directly, or an empty sequence (zero-filled)
  if (first < 0 || first + nwg > p.splits) return;  // spans are always inside [0, W)
  const int j4 = (threadIdx.x & 63) >> 4;
  const int64_t slot_floats = static_cast<int64_t>(p.Hq) * (D + 2);
  const float* slots = p.ws + static_cast<int64_t>(first + b) * slot_floats;
  MergeRows<D, KB> mr;
  if constexpr (RG == 1) {
    const int hh = 4 * blockIdx.x + j4;
    const bool active = hh < p.Hq;
    const int64_t h = active ? hh : 0;
    mr.fold_rows(slots + h * (D + 2), slot_floats, nwg);
    mr.template store<DT>(active, static_cast<S*>(p.out) + (static_cast<int64_t>(b) * p.Hq + h) * D);
  } else {
    const int64_t h = blockIdx.x;
    const int nrows = nwg > j4 ? (nwg - j4 + RG - 1) / RG : 0;
    mr.fold_rows(slots + (h + static_cast<int64_t>(j4) * p.Hq) * (D + 2), RG * slot_floats, nrows);
    mr.combine_groups();
    mr.template store<DT>(j4 == 0, static_cast<S*>(p.out) + (static_cast<int64_t>(b) * p.Hq + h) * D);
  }
}

// ----------------------------------------------------------------------------
// Log-sum-exp merge of partials {m, l, acc[D]}
// ----------------------------------------------------------------------------

// Merges `nrows` partial rows (row r at base + r*row_stride) of one head
// into out[0..D): skip rows with l == 0 (online_softmax.cuh:18), weights
// exp(m_r - max m), output sum_r w_r*acc_r / sum_r w_r*l_r, or zeros when
// the total is 0 (gqa_decode.cu:84-86).  One wave; the m/l of all rows
// (lane r) and the first kCombineBatch rows of acc are loaded together, so
// one memory round trip covers a typical merge.
template <int DT>
__device__ __forceinline__ void merge_rows(const float* base, int64_t row_stride, int nrows, int D,
                                           typename Elem<DT>::S* o) {
  using E = Elem<DT>;
  constexpr int kCombineBatch = 8;
  const int lane = threadIdx.x;
  float accv[kCombineBatch][4];
  auto load_rows = [&](int s0) {
#pragma unroll
    for (int t = 0; t < kCombineBatch; ++t) {
      const int s = min(s0 + t, nrows - 1);
      const float* row = base + static_cast<int64_t>(s) * row_stride + 2;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = lane + 64 * r;
        accv[t][r] = d < D ? row[d] : 0.f;
      }
    }
  };
  float lown = 0.f, mown = -INFINITY;
  if (lane < nrows) {
    lown = base[static_cast<int64_t>(lane) * row_stride + 1];
    mown = base[static_cast<int64_t>(lane) * row_stride];
  }
  load_rows(0);
  float mloc = -INFINITY;
  for (int s = lane; s < nrows; s += 64) {
    const float ls = s == lane ? lown : base[static_cast<int64_t>(s) * row_stride + 1];
    const float ms = s == lane ? mown : base[static_cast<int64_t>(s) * row_stride];
    if (ls != 0.f) mloc = fmaxf(mloc, ms);
  }
  const float M = wave_max(mloc);
  const float Mref = M == -INFINITY ? 0.f : M;

  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  float lsum = 0.f;
  for (int s0 = 0; s0 < nrows; s0 += 64) {
    const int s = s0 + lane;
    float wgt = 0.f;
    if (s < nrows) {
      const float ls = s0 == 0 ? lown : base[static_cast<int64_t>(s) * row_stride + 1];
      const float ms = s0 == 0 ? mown : base[static_cast<int64_t>(s) * row_stride];
      if (ls != 0.f) {
        wgt = fast_exp2((ms - Mref) * kLog2e);
        lsum = fmaf(wgt, ls, lsum);
      }
    }
    const int n = min(64, nrows - s0);
    for (int t0 = 0; t0 < n; t0 += kCombineBatch) {
      if (s0 + t0 > 0) load_rows(s0 + t0);
#pragma unroll
      for (int t = 0; t < kCombineBatch; ++t) {
        const float wt = t0 + t < n ? __shfl(wgt, t0 + t) : 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] = fmaf(wt, accv[t][r], acc[r]);
      }
    }
  }
  const float L = wave_sum(lsum);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int d = lane + 64 * r;
    if (d < D) o[d] = E::from_f(L > 0.f ? acc[r] / L : 0.f);
  }
}

// Explicit split layout: grid (Hq, B), block 64; ws [B, Hq, splits, D+2].
template <int DT>
__global__ __launch_bounds__(64) void combine_kernel(DecodeParams p) {
  using S = typename Elem<DT>::S;
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const ChunkInfo ci = chunk_info(p, p.lens[b], 0);
  if (ci.nch <= 1) return;  // written directly by the decode kernel
  const int D = p.D;
  const float* base = p.ws + (static_cast<int64_t>(b) * p.Hq + h) * p.splits * (D + 2);
  merge_rows<DT>(base, D + 2, ci.nch, D, static_cast<S*>(p.out) + (static_cast<int64_t>(b) * p.Hq + h) * D);
}

// Same merge for head_dim D in {64, 128, 256}, a 16-byte aligned output and
// an 8-byte aligned workspace: grid (Hq, B), one wave per head.  Lane group
// j4 folds the partials z = j4, j4 + 4, ... in order (combine_rows<D>()
// of them per memory round trip each, so 4x that many per wave, against
// merge_rows' kCombineBatch), then the four group states are combined
// (SoftmaxState::merge) and group 0 stores the row.
template <int D>
constexpr int combine_rows() {
  return D <= 128 ? 16 : 8;
}

template <int D, int DT>
__global__ __launch_bounds__(64) void combine_rows_kernel(DecodeParams p) {
  using S = typename Elem<DT>::S;
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const ChunkInfo ci = chunk_info(p, p.lens[b], 0);
  if (ci.nch <= 1) return;  // written directly by the decode kernel
  const int j4 = (threadIdx.x & 63) >> 4;
  const float* base = p.ws + (static_cast<int64_t>(b) * p.Hq + h) * p.splits * (D + 2);
  const int nrows = ci.nch > j4 ? (ci.nch - j4 + 3) / 4 : 0;
  MergeRows<D, combine_rows<D>()> mr;
  mr.fold_rows(base + static_cast<int64_t>(j4) * (D + 2), 4 * (D + 2), nrows);
  mr.combine_groups();
  mr.template store<DT>(j4 == 0, static_cast<S*>(p.out) + (static_cast<int64_t>(b) * p.Hq + h) * D);
}

// ----------------------------------------------------------------------------
// Host side
// ----------------------------------------------------------------------------

thread_local std::string g_last_error;
thread_local int g_last_status = 0;

}  // namespace

// Shared with the other entry points of the library (kv_append.hip).
void qd_set_last_error(int status, const std::string& msg) {
  g_last_status = status;
  g_last_error = msg;
}

namespace {

int fail(int status, const std::string& msg) {
  qd_set_last_error(status, msg);
  return status;
}

void copy_msg(char* msg, size_t cap, const char* text) {
  if (!msg || cap == 0) return;
  size_t n = strlen(text);
  if (n >= cap) n = cap - 1;
  memcpy(msg, text, n);
  msg[n] = '\0';
}

int invalid(char* msg, size_t cap, const char* text) {
  copy_msg(msg, cap, text);
  return fail(QD_ERR_INVALID_VALUE, text);
}

bool same_sizes(const qd_tensor_desc* a, const qd_tensor_desc* b) {
  if (a->ndim != b->ndim) return false;
  const int n = a->ndim < 8 ? a->ndim : 8;
  for (int i = 0; i < n; ++i)
    if (a->sizes[i] != b->sizes[i]) return false;
  return true;
}

constexpr int kMfmaHeads = 16;

// fp32 caches on the balanced path (MfmaWaveF32): head_dim 64 or 128, whole
// 16-token groups per page, at most 16 q-heads per kv-head, and a batch whose
// static capacity (batch * max_pages * block_size) is at least
// kF32SkTokens.  Graph replays on the reference's fp32 sweep shape (Hq32/Hkv8)
// against the split layout: head_dim 64 B16/L4096 78.1 -> 49.7 us, head_dim
// 128 B16/L4096 98.6 -> 93.5 and B32/L4096 184.4 -> 167.7 us; below that
// capacity the split layout's single launch was faster (head_dim 128 B1/L128
// 10.9 against 15.6 us, B4/L4096 34.2 against 38.7, B16/L1024 34.1 against
// 39.3; head_dim 64 B4/L1024 12.5 against 14.1).  At head_dim 128 a wave
// holds 32 KB of K/V per group in flight and runs one per SIMD; one group in
// flight at two waves per SIMD, or K loaded straight in the MFMA layout,
// measured slower.
constexpr int64_t kF32SkTokens = 65536;

bool f32_sk_applies(int batch, int q_heads, int kv_heads, int head_dim, int block_size, int max_pages, int dtype) {
  if (dtype != QD_DTYPE_F32 || (head_dim != 64 && head_dim != 128) || block_size % 16 != 0) return false;
  if (static_cast<int64_t>(batch) * max_pages * block_size < kF32SkTokens) return false;
  return kv_heads > 0 && q_heads % kv_heads == 0 && q_heads / kv_heads <= kMfmaHeads;
}

bool mfma_applies(int q_heads, int kv_heads, int head_dim, int block_size, int dtype) {
  if (dtype != QD_DTYPE_F16 && dtype != QD_DTYPE_BF16) return false;
  if (head_dim != 64 && head_dim != 96 && head_dim != 128 && head_dim != 256) return false;
  if (block_size % 16 != 0) return false;
  if (kv_heads <= 0 || q_heads % kv_heads != 0) return false;
  return q_heads / kv_heads <= kMfmaHeads;
}

#ifndef QD_PREFETCH
#define QD_PREFETCH 2
#endif
// 16-token groups in flight per wave (D <= 128).  2 measured best for one
// kv-head per wave on the stream-K path (cfg3's kernel 79.4 -> 78.7 us
// against 3; 4 spills).
constexpr int kPrefetch = QD_PREFETCH;
// At head_dim 64 a group is half the bytes: 3 in flight (178-199 VGPRs,
// still two waves per SIMD) took the stream-K kernel 7-9% faster on group
// sizes 4-8 (graph replays, B8-B128, 1-8K tokens); 4 was slower than 3.  At
// head_dim 96 a third group measured no faster.
constexpr int kPrefetch64 = 3;

// Stream-K path limits: each wave scans all lengths, so the batch is capped.
constexpr int kSkMaxBatch = 4096;
// Grid of a batch below the resident workgroups, from static shapes (Gmax
// groups of the largest possible batch, S = their K/V bytes):
//   W = min(resident, Gmax / kSkMinGroups,
//           max(kSkRowsShort * B, min(ceil(S / kSkWgBytes), kSkRowsLong * B))).
// A sequence split over W/B workgroups leaves that many partial rows per head
// for the merge (kSkRowsShort of them fold in one round trip per merge wave),
// and a workgroup's range streams at about 45-60 GB/s until HBM saturates:
// short batches take as many workgroups as one merge round trip allows, long
// ones one per kSkWgBytes up to two round trips.  Measured against the
// earlier floor of 4 groups per workgroup (graph replays, bf16, Hq32 Hkv8
// D128 P16): B1/L128 12.7 -> 9.8 us, B16/L128 14.8 -> 11.4, B1/L1024 13.6 ->
// 10.9, B4/L1024 14.3 -> 13.1, B1/L16384 26.2 -> 24.2, head_dim 256 B1/L2048
// 18.6 -> 16.3; of 34 shapes one slower (B100/L128, 16.9 -> 17.8 us: its old
// grid of 200 took the held-results kernel, 256 does not); batches that fill
// the resident grid (cfg2-cfg5) are unchanged.  A hard cap of 64 per sequence took
// B1/L32768 from 35.6 to 51.9 us (too few workgroups to saturate HBM).
#ifndef QD_SK_MIN_GROUPS
#define QD_SK_MIN_GROUPS 1
#endif
constexpr int64_t kSkMinGroups = QD_SK_MIN_GROUPS;
constexpr int64_t kSkRowsShort = 64;
constexpr int64_t kSkRowsLong = 128;
constexpr int64_t kSkWgBytes = int64_t{256} << 10;
// Waves launched per resident wave slot.  Above 1 the hardware dispatcher
// hands the later waves to whichever CUs finish first.
#ifndef QD_SK_OVERSUB
#define QD_SK_OVERSUB 1
#endif
constexpr int kSkOversubscribe = QD_SK_OVERSUB;

using KernelFn = void (*)(DecodeParams);

template <int DT>
KernelFn pick_mfma(int D) {
  switch (D) {
    case 64: return decode_mfma_kernel<64, DT, kPrefetch>;
    case 96: return decode_mfma_kernel<96, DT, kPrefetch>;
    case 128: return decode_mfma_kernel<128, DT, kPrefetch>;
    default: return decode_mfma_kernel<256, DT, 2>;
  }
}

#ifndef QD_PREFETCH_DUAL
#define QD_PREFETCH_DUAL 2
#endif
// Groups in flight per wave when a wave serves two kv-heads (twice the
// bytes per group).
constexpr int kPrefetchDual = QD_PREFETCH_DUAL;

// Groups in flight per wave for 4 kv-heads at head_dim 128 (sk_wide_applies):
// one workgroup of 4 waves per CU, one wave per SIMD with up to 512
// registers.  4-wave workgroups of the 2-in-flight kernel sit two per CU,
// and the older workgroup of each pair ran ahead of the other as the older
// wave of a SIMD does (cfg3's decode kernel: 78.8 us, against 76.7-77.1 us
// with 3 or 4 in flight and one workgroup per CU).
constexpr int kSkWidePrefetch = 3;

template <int DT, bool FUSED, bool HOLD>
KernelFn pick_mfma_sk(int D, int nkv, bool wide) {
  if (wide) return decode_mfma_sk_kernel<128, DT, kSkWidePrefetch, 1, 0, FUSED, HOLD>;
  if (nkv == 2) {
    switch (D) {
      case 64: return decode_mfma_sk_kernel<64, DT, kPrefetchDual, 2, 0, FUSED, HOLD>;
      default: return decode_mfma_sk_kernel<128, DT, kPrefetchDual, 2, 0, FUSED, HOLD>;
    }
  }
  switch (D) {
    case 64: return decode_mfma_sk_kernel<64, DT, kPrefetch64, 1, 0, FUSED, HOLD>;
    case 96: return decode_mfma_sk_kernel<96, DT, kPrefetch, 1, 0, FUSED, HOLD>;
    case 128: return decode_mfma_sk_kernel<128, DT, kPrefetch, 1, 0, FUSED, HOLD>;
    default: return decode_mfma_sk_kernel<256, DT, 2, 1, 0, FUSED, HOLD>;
  }
}

// fused: the fused-merge kernel; hold: the kernel that holds its result rows
// in LDS until its range ends (never both).
KernelFn pick_mfma_sk_dt(int dtype, int D, int nkv, bool wide = false, bool fused = false, bool hold = false) {
  const bool f16 = dtype == QD_DTYPE_F16;
  if (dtype == QD_DTYPE_F32) {  // f32_sk_applies: head_dim 64 or 128, one kv-head per wave, never fused
    if (D == 64)
      return hold ? decode_mfma_sk_kernel<64, QD_DTYPE_F32, kPrefetch, 1, 0, false, true>
                  : decode_mfma_sk_kernel<64, QD_DTYPE_F32, kPrefetch, 1, 0, false, false>;
    return hold ? decode_mfma_sk_kernel<128, QD_DTYPE_F32, kPrefetch, 1, 0, false, true>
                : decode_mfma_sk_kernel<128, QD_DTYPE_F32, kPrefetch, 1, 0, false, false>;
  }
  if (fused)
    return f16 ? pick_mfma_sk<QD_DTYPE_F16, true, false>(D, nkv, wide)
               : pick_mfma_sk<QD_DTYPE_BF16, true, false>(D, nkv, wide);
  if (hold)
    return f16 ? pick_mfma_sk<QD_DTYPE_F16, false, true>(D, nkv, wide)
               : pick_mfma_sk<QD_DTYPE_BF16, false, true>(D, nkv, wide);
  return f16 ? pick_mfma_sk<QD_DTYPE_F16, false, false>(D, nkv, wide)
             : pick_mfma_sk<QD_DTYPE_BF16, false, false>(D, nkv, wide);
}

// One wave per SIMD needs exactly 4 single-kv-head waves per workgroup;
// fewer kv-heads would leave SIMDs idle.
bool sk_wide_applies(int kv_heads, int head_dim) { return kv_heads == 4 && head_dim == 128; }

// The VALU comparison variant of the balanced kernel: head_dim 128, one
// kv-head per wave, group size <= 8.
bool valu_sk_applies(int q_heads, int kv_heads, int head_dim, int dtype) {
  return head_dim == 128 && (dtype == QD_DTYPE_F16 || dtype == QD_DTYPE_BF16) && kv_heads > 0 &&
         q_heads % kv_heads == 0 && q_heads / kv_heads <= 8;
}

KernelFn pick_valu_sk_dt(int dtype, int g) {
  if (dtype == QD_DTYPE_F16)
    return g <= 4 ? decode_mfma_sk_kernel<128, QD_DTYPE_F16, kValuPrefetch, 1, 4>
                  : decode_mfma_sk_kernel<128, QD_DTYPE_F16, kValuPrefetch, 1, 8>;
  return g <= 4 ? decode_mfma_sk_kernel<128, QD_DTYPE_BF16, kValuPrefetch, 1, 4>
                : decode_mfma_sk_kernel<128, QD_DTYPE_BF16, kValuPrefetch, 1, 8>;
}

template <int DT, int KB, int RG>
KernelFn pick_merge_sk(int D) {
  switch (D) {
    case 64: return merge_sk_kernel<64, DT, KB, RG>;
    case 96: return merge_sk_kernel<96, DT, KB, RG>;
    case 128: return merge_sk_kernel<128, DT, KB, RG>;
    default: return merge_sk_kernel<256, DT, KB, RG>;
  }
}

// Merge layout for a batch: one wave per head (four row groups, up to 64
// rows per round trip) while the Hq*B waves fit the GPU at once at the
// kernel's occupancy (2 waves per SIMD), else four heads per wave with 8
// rows per round trip (fewer registers, 4 waves per SIMD).
constexpr int64_t kMergeOneHeadWaves = 2048;

bool merge_one_head_per_wave(int batch, int q_heads) {
  return static_cast<int64_t>(batch) * q_heads <= kMergeOneHeadWaves;
}

KernelFn pick_merge_sk_dt(int dtype, int D, bool one_head) {
  if (dtype == QD_DTYPE_F32) {
    if (one_head)
      return D == 64 ? merge_sk_kernel<64, QD_DTYPE_F32, 16, 4> : merge_sk_kernel<128, QD_DTYPE_F32, 16, 4>;
    return D == 64 ? merge_sk_kernel<64, QD_DTYPE_F32, 8, 1> : merge_sk_kernel<128, QD_DTYPE_F32, 8, 1>;
  }
  if (one_head)
    return dtype == QD_DTYPE_F16 ? pick_merge_sk<QD_DTYPE_F16, 16, 4>(D)
                                 : pick_merge_sk<QD_DTYPE_BF16, 16, 4>(D);
  return dtype == QD_DTYPE_F16 ? pick_merge_sk<QD_DTYPE_F16, 8, 1>(D) : pick_merge_sk<QD_DTYPE_BF16, 8, 1>(D);
}

template <int DT, int GH>
KernelFn pick_generic_gh(int D) {
  if (D <= 16) return D == 16 ? decode_generic_kernel<DT, 1, true, GH> : decode_generic_kernel<DT, 1, false, GH>;
  if (D <= 32) return D == 32 ? decode_generic_kernel<DT, 2, true, GH> : decode_generic_kernel<DT, 2, false, GH>;
  if (D <= 64) return D == 64 ? decode_generic_kernel<DT, 4, true, GH> : decode_generic_kernel<DT, 4, false, GH>;
  if (D <= 128) return D == 128 ? decode_generic_kernel<DT, 8, true, GH> : decode_generic_kernel<DT, 8, false, GH>;
  return D == 256 ? decode_generic_kernel<DT, 16, true, GH> : decode_generic_kernel<DT, 16, false, GH>;
}

template <int DT>
KernelFn pick_generic(int D, int g) {
  return generic_heads(g) == 4 ? pick_generic_gh<DT, 4>(D) : pick_generic_gh<DT, kGenericHeads>(D);
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

template <int DT>
KernelFn pick_combine_rows(int D) {
  switch (D) {
    case 64: return combine_rows_kernel<64, DT>;
    case 128: return combine_rows_kernel<128, DT>;
    default: return combine_rows_kernel<256, DT>;
  }
}

// The split layout's merge: combine_rows_kernel where its vector loads and
// stores apply (head_dim 64/128/256, 16-byte aligned output, 8-byte aligned
// workspace), else combine_kernel (any head_dim, element stores).
KernelFn pick_combine(int dtype, int head_dim, const void* out, const float* ws) {
  const bool rows = (head_dim == 64 || head_dim == 128 || head_dim == 256) && aligned16(out) &&
                    (reinterpret_cast<uintptr_t>(ws) & 7u) == 0;
  switch (dtype) {
    case QD_DTYPE_F32: return rows ? pick_combine_rows<QD_DTYPE_F32>(head_dim) : combine_kernel<QD_DTYPE_F32>;
    case QD_DTYPE_F16: return rows ? pick_combine_rows<QD_DTYPE_F16>(head_dim) : combine_kernel<QD_DTYPE_F16>;
    default: return rows ? pick_combine_rows<QD_DTYPE_BF16>(head_dim) : combine_kernel<QD_DTYPE_BF16>;
  }
}

// Resident workgroups of `fn` (block of `threads`) on the current device:
// CUs x blocks per CU from the HIP occupancy calculator; cached per
// (device, fn, threads).
int resident_blocks(KernelFn fn, int threads, size_t dyn_lds = 0) {
  struct Entry {
    int device;
    KernelFn fn;
    int threads;
    size_t dyn_lds;
    int blocks;
  };
  static std::mutex mu;
  static Entry cache[64];
  static int used = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < used; ++i)
    if (cache[i].device == dev && cache[i].fn == fn && cache[i].threads == threads && cache[i].dyn_lds == dyn_lds)
      return cache[i].blocks;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(fn), threads, dyn_lds) !=
          hipSuccess ||
      per_cu <= 0)
    per_cu = 1;
  (void)hipGetLastError();
  const int blocks = cus * per_cu;
  if (used < 64) cache[used++] = Entry{dev, fn, threads, dyn_lds, blocks};
  return blocks;
}

// Dynamic LDS of the stream-K kernels at most: the staged result rows
// (stage_lds_bytes) or the fused kernel's partials kept until the range
// ends; with the K tiles well inside gfx950's 160 KiB.
constexpr size_t kFusedMaxStash = 96 << 10;

// Result rows are held in LDS until a workgroup's range ends (instead of
// stored after each item) when the batch has at least one sequence per
// kHoldWgsPerSeq workgroups: then ranges cross sequence boundaries often
// and every store between items stalls the loads behind it.  Measured on
// the decode kernel: cfg5 (256 sequences, 256 workgroups) 101-102 -> 92-96
// us; cfg3 (64 sequences) 78-80 -> 82-87 us, cfg2 (32) unchanged, so the
// shorter batches keep the stores after each item.
constexpr int64_t kHoldWgsPerSeq = 2;

bool hold_results(int batch, int64_t wgs) { return static_cast<int64_t>(batch) * kHoldWgsPerSeq >= wgs; }

// LDS per wave for the result rows a wave holds until its range ends
// (MfmaWave::stage_*): room for kStageItems items of NKV*g partial rows of
// D+2 floats (an output row needs less), as many as fit in kFusedMaxStash
// per workgroup, at least one.  A range with more items flushes early.
constexpr int kStageItems = 4;

int stage_wave_bytes(int g, int head_dim, int nkv, int wg_waves) {
  const int item = (nkv * g * (head_dim + 2) * 4 + 15) & ~15;
  int items = static_cast<int>(kFusedMaxStash / static_cast<size_t>(wg_waves) - kStageRecordBytes) / item;
  if (items > kStageItems) items = kStageItems;
  if (items < 1) items = 1;
  return kStageRecordBytes + items * item;
}

size_t stage_lds_bytes(int g, int head_dim, int nkv, int wg_waves) {
  return static_cast<size_t>(wg_waves) * stage_wave_bytes(g, head_dim, nkv, wg_waves);
}

// Raises `fn`'s dynamic LDS limit to kFusedMaxStash (above the default
// 64 KiB), once per (device, kernel); false when HIP refuses.  Without a
// device (plans made for sizing only, as resident_blocks' fallback) it
// reports true.
bool allow_dyn_lds(KernelFn fn) {
  struct Entry {
    int device;
    KernelFn fn;
    bool ok;
  };
  static std::mutex mu;
  static Entry cache[64];
  static int used = 0;
  int dev = 0, count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
    (void)hipGetLastError();
    return true;
  }
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < used; ++i)
    if (cache[i].device == dev && cache[i].fn == fn) return cache[i].ok;
  const bool ok = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(kFusedMaxStash)) == hipSuccess;
  (void)hipGetLastError();
  if (used < 64) cache[used++] = Entry{dev, fn, ok};
  return ok;
}

// Kv-heads per wave on the stream-K path.  One (a workgroup of up to 8
// waves holds two per SIMD) hides the start of each item behind the other
// wave of its SIMD: it wins on short and ragged batches (cfg2 decode 54.9
// against 56.9 us, cfg5 101.6 against 103.8 us).  Two (one wave per SIMD,
// 512 registers, 8 or more kv-heads with head_dim <= 128) stream faster once
// every workgroup has long runs (cfg4 333 against 342 us): chosen when the
// batch's static token capacity, B * max_pages * block_size, is at least
// kSkDualTokensPerWg per resident workgroup (cfg4: 4096, cfg5: 1024, cfg2:
// 512 on 256 CUs).  Static shapes only, as gqa_decode_auto's heuristic
// (core.py:80-96).
constexpr int64_t kSkDualTokensPerWg = 2048;

bool sk_dual_applies(int batch, int kv_heads, int head_dim, int block_size, int max_pages,
                     int resident_wgs) {
  if ((head_dim != 64 && head_dim != 128) || kv_heads % 2 != 0 || kv_heads < 8) return false;
  const int64_t cap = static_cast<int64_t>(batch) * max_pages * block_size;
  return cap >= kSkDualTokensPerWg * resident_wgs;
}

// Waves per stream-K workgroup: the largest divisor of kv_heads / nkv that
// fits the kernel's bound, so every wave serves the same number of
// kv-heads.
int sk_wg_waves(int kv_heads, int nkv, int head_dim, bool valu = false, bool wide = false) {
  const int units = kv_heads / nkv;
  const int cap = valu ? kValuMaxWaves : (nkv == 1 && head_dim <= 128 && !wide) ? kMaxWgWaves : kMaxWgWaves / 2;
  for (int n = cap; n > 1; --n)
    if (units % n == 0) return n;
  return 1;
}

// Arrival counters of the fused stream-K path: one 32-bit word per
// (sequence, kv-head), at the start of every automatic-path workspace.  The
// place and size are fixed, so calls of any shape sharing a workspace never
// write partials over them; they must be zero before the workspace's first
// use, and every call leaves them zero.
constexpr int64_t kFusedMaxCounters = 65536;
constexpr size_t kCounterBytes = static_cast<size_t>(kFusedMaxCounters) * sizeof(uint32_t);  // 256 KiB

// The automatic plan merges split sequences with merge_sk_kernel; the fused
// merge (decode_mfma_sk_kernel<..., FUSED = true>) is kept as the
// QD_STAGE_FUSED measurement option.  Per-wave timestamps on cfg2's shape
// (bench.py --mode stamps) put the fused chain after a wave's last group
// at 1.4 us (sc1 partial stores retiring) + 1.0 us (arrival atomic) +
// 6-8 us (sc1 row reads, all merging waves at once), against about 4.7 us
// for the separate kernel including its launch: 78 against 59 us per call.
constexpr bool kFusedByDefault = false;

// Fused merge cost bound: the merging wave folds NKV*g heads, four per pass,
// over about ceil(W/B) rows, fused_merge_rows() per memory round trip.  The
// fused path is taken when that is at most kFusedMaxTrips dependent round
// trips, since the last merge of the launch is not hidden behind streaming;
// beyond it merge_sk_kernel's one-head-per-wave layout finishes sooner.
constexpr int64_t kFusedMaxTrips = 2;

struct AutoPlan {
  bool stream_k;
  int wgs;          // stream-K grid (workgroups)
  int wg_waves;     // stream-K waves per workgroup
  int kv_per_wave;  // stream-K kv-heads per wave
  bool wide;        // stream-K: one wave per SIMD, kSkWidePrefetch groups in flight
  bool fused;       // stream-K: split sequences merged inside the decode kernel
  size_t stash_bytes;  // fused: dynamic LDS per workgroup for mid-range partials
  size_t stage_bytes;  // otherwise: dynamic LDS per workgroup for staged result rows
  int splits;       // explicit-split path
  int chunk_pages;
  size_t ws_bytes;  // scratch bytes (kCounterBytes of counters first)
  size_t meta_offset;  // stream-K: byte offset of the meta table in the scratch
  int kv_split;     // stream-K: virtual kv-heads per kv-head (DecodeParams::kv_split)
};

// Virtual kv-heads per kv-head for the stream-K path: 1 for groups of at
// most kMfmaHeads q-heads, else the fewest chunks of at most kMfmaHeads
// q-heads, c = ceil(g / kMfmaHeads), of ceil(g / c) q-heads each but the
// last (48 is 3 x 16, 40 is 3 x 14 with 12 in the last, 71 is 5 x 15 with
// 11), at most kMaxWgWaves of them so that one kv-head's chunks are waves
// of one workgroup, reading the same K/V rows in the same steps; 0 for
// groups above kMaxWgWaves * kMfmaHeads (128).
int kv_split_for(int q_heads, int kv_heads) {
  if (kv_heads <= 0 || q_heads % kv_heads != 0) return 0;
  const int g = q_heads / kv_heads;
  const int c = (g + kMfmaHeads - 1) / kMfmaHeads;
  return c <= kMaxWgWaves ? c : 0;
}

// q-heads per virtual kv-head (the chunk size; the real group when c = 1).
int kv_chunk_heads(int q_heads, int kv_heads, int c) {
  const int g = q_heads / kv_heads;
  return c > 1 ? (g + c - 1) / c : g;
}

// Shapes the fused merge can address: one counter per (sequence, kv-head)
// in the counter area, and 32-bit buffer offsets over a sequence's slots.
bool fused_fits(int batch, int q_heads, int kv_heads, int head_dim, int64_t wgs) {
  return static_cast<int64_t>(batch) * kv_heads <= kFusedMaxCounters &&
         (wgs + batch) * q_heads * (head_dim + 2) * 4 < (int64_t{1} << 31);
}

// Dynamic LDS of the fused kernel: each wave keeps one partial per kv-head
// group it serves, (2 + head_dim/4) fields x 64 lanes x 4 bytes per kv-head.

size_t fused_stash_bytes(int kv_heads, int head_dim, int nkv, int wg_waves) {
  const int items = (kv_heads + wg_waves * nkv - 1) / (wg_waves * nkv);
  return static_cast<size_t>(wg_waves) * items * nkv * (2 + head_dim / 4) * 64 * sizeof(float);
}

bool fused_applies(int batch, int q_heads, int kv_heads, int head_dim, int nkv, int64_t wgs) {
  if (!fused_fits(batch, q_heads, kv_heads, head_dim, wgs)) return false;
  const int64_t heads = static_cast<int64_t>(nkv) * (q_heads / kv_heads);
  const int64_t passes = (heads + 3) / 4;
  const int64_t rows = (wgs + batch - 1) / batch + 1;  // a sequence may touch one more workgroup
  const int64_t kb = head_dim <= 128 ? 16 : 8;
  return passes * ((rows + kb - 1) / kb) <= kFusedMaxTrips;
}

// Chooses the automatic path from static shapes only.  `aligned` says
// whether q/k/v/out are 16-byte aligned (the MFMA kernels' vector loads).
int auto_plan(int batch, int q_heads, int kv_heads, int head_dim, int block_size, int max_pages,
              int dtype, bool aligned, AutoPlan* ap, bool valu = false) {
  *ap = AutoPlan{false, 0, 1, 1, false, false, 0, 0, 1, 0, kCounterBytes, 0, 1};
  if (batch <= 0) return QD_OK;
  const int split = kv_split_for(q_heads, kv_heads);
  const int vkv = kv_heads * (split > 0 ? split : 1);  // kv-heads as the stream-K kernel serves them
  const int gv = split > 0 ? kv_chunk_heads(q_heads, kv_heads, split) : 0;  // q-heads per one of them, at most
  const bool f32 = dtype == QD_DTYPE_F32;
  if (aligned && split > 0 && (split == 1 || !valu) &&
      (f32 ? !valu && f32_sk_applies(batch, q_heads, kv_heads, head_dim, block_size, max_pages, dtype)
           : mfma_applies(vkv * gv, vkv, head_dim, block_size, dtype)) &&
      batch <= kSkMaxBatch) {
    int nkv = 1;
    const bool wide = !valu && !f32 && sk_wide_applies(vkv, head_dim);
    // fp32 at head_dim 128 holds 64 KB of K/V per group in flight: one wave
    // per SIMD (the 4-wave cap of the wide layout).
    int nw = sk_wg_waves(vkv, nkv, head_dim, valu, wide || (f32 && head_dim > 64));
    // The chunks of one kv-head in one pass of the workgroup's waves.
    for (int n = nw; split > 1 && n >= split; --n) {
      if (vkv % n == 0 && n % split == 0) {
        nw = n;
        break;
      }
    }
    const int g = gv;
    KernelFn fn = valu ? pick_valu_sk_dt(dtype, g) : pick_mfma_sk_dt(dtype, head_dim, nkv, wide);
    int resident = resident_blocks(fn, 64 * nw);
    if (!valu && !f32 && split == 1 && sk_dual_applies(batch, kv_heads, head_dim, block_size, max_pages, resident)) {
      nkv = 2;
      nw = sk_wg_waves(kv_heads, nkv, head_dim);
      fn = pick_mfma_sk_dt(dtype, head_dim, nkv);
      resident = resident_blocks(fn, 64 * nw);
    }
    const int64_t gmax = static_cast<int64_t>(batch) *
                         ((static_cast<int64_t>(max_pages) * block_size + 15) / 16);
    const int64_t by_work = (gmax + kSkMinGroups - 1) / kSkMinGroups;
    const int64_t group_bytes = int64_t{16} * kv_heads * head_dim * 2 * (dtype == QD_DTYPE_F32 ? 4 : 2);
    const int64_t by_bytes = (gmax * group_bytes + kSkWgBytes - 1) / kSkWgBytes;
    const int64_t by_rows = std::max(kSkRowsShort * batch, std::min(by_bytes, kSkRowsLong * batch));
    auto grid = [&](int res) {
      int64_t w = static_cast<int64_t>(res) * kSkOversubscribe;
      if (w > by_work) w = by_work;
      if (w > by_rows) w = by_rows;
      return w < 1 ? int64_t{1} : w;
    };
    int64_t w = grid(resident);
    // Result rows held in LDS until the range ends: the kernel's occupancy
    // with that LDS sets the grid.  Not where each wave runs alone on its
    // SIMD and serves a single kv-head per sequence (4 kv-heads at head_dim
    // 128, head_dim 256 or fp32 head_dim 128 with at most 4 kv-heads): there
    // the stores after each item measured faster (graph replays, B128/L1024:
    // Qwen2.5-7B's shape 51.5 -> 47.2 us, Gemma-2-2B's 96.2 -> 87.4 us),
    // while with two kv-heads per wave (Gemma-2-9B's shape) holding was level.
    const bool one_per_simd = nkv == 1 && (wide || head_dim > 128 || (f32 && head_dim > 64));
    if (!valu && !(one_per_simd && nw == vkv) && hold_results(batch, w)) {
      const KernelFn hfn = pick_mfma_sk_dt(dtype, head_dim, nkv, wide && nkv == 1, false, true);
      ap->stage_bytes = stage_lds_bytes(g, head_dim, nkv, nw);
      if (!allow_dyn_lds(hfn)) return fail(QD_ERR_INVALID_VALUE, "dynamic LDS limit not raised");
      w = grid(resident_blocks(hfn, 64 * nw, ap->stage_bytes));
    }
    if (valu) {
      // The comparison variant runs on the product plan's grid (and fits its
      // workspace).
      AutoPlan prod;
      auto_plan(batch, q_heads, kv_heads, head_dim, block_size, max_pages, dtype, aligned, &prod, false);
      if (prod.stream_k && w > prod.wgs) w = prod.wgs;
    }
    ap->stream_k = true;
    ap->kv_split = split;
    ap->wgs = static_cast<int>(w);
    ap->wg_waves = nw;
    ap->kv_per_wave = nkv;
    ap->wide = wide && nkv == 1;
    ap->stash_bytes = fused_stash_bytes(vkv, head_dim, nkv, nw);  // used by the fused kernel only (split == 1)
    const KernelFn ffn = pick_mfma_sk_dt(dtype, head_dim, nkv, ap->wide, true);
    if (kFusedByDefault && !valu && split == 1 && fused_applies(batch, q_heads, kv_heads, head_dim, nkv, w) &&
        ap->stash_bytes <= kFusedMaxStash && allow_dyn_lds(ffn)) {
      // The fused kernel's own occupancy (registers and the stash) bounds
      // the grid; without waits between workgroups a larger grid would
      // still be correct, only slower.
      const int64_t rf = resident_blocks(ffn, 64 * nw, ap->stash_bytes) * kSkOversubscribe;
      if (w > rf) w = rf;
      ap->wgs = static_cast<int>(w);
      ap->fused = fused_fits(batch, q_heads, kv_heads, head_dim, w);
    }
    ap->meta_offset = kCounterBytes + static_cast<size_t>(w + batch) * q_heads * (head_dim + 2) * sizeof(float);
    ap->ws_bytes = ap->meta_offset + static_cast<size_t>(batch) * 2 * sizeof(int);
    return QD_OK;
  }
  int s = 1, c = 0;
  const int st = qd_gqa_decode_plan(batch, q_heads, kv_heads, head_dim, block_size, max_pages, dtype,
                                    0, &s, &c);
  if (st != QD_OK) return st;
  ap->splits = s;
  ap->chunk_pages = c;
  ap->ws_bytes = kCounterBytes + qd_gqa_decode_workspace_bytes(batch, q_heads, head_dim, s);
  return QD_OK;
}

int check_launch_shapes(int batch, int q_heads, int kv_heads, int head_dim, int block_size,
                        int max_pages, int64_t num_blocks, int dtype, float scale) {
  if (batch < 0) return fail(QD_ERR_INVALID_VALUE, "batch must be >= 0");
  if (q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads != 0)
    return fail(QD_ERR_INVALID_VALUE, "Hq must be divisible by Hkv");
  if (head_dim < 1 || head_dim > 256) return fail(QD_ERR_INVALID_VALUE, "supported head_dim is [1, 256]");
  if (block_size <= 0 || num_blocks <= 0)
    return fail(QD_ERR_INVALID_VALUE, "cache must have positive blocks and block_size");
  if (max_pages <= 0) return fail(QD_ERR_INVALID_VALUE, "block_table must have at least one page");
  if (dtype != QD_DTYPE_F32 && dtype != QD_DTYPE_F16 && dtype != QD_DTYPE_BF16)
    return fail(QD_ERR_INVALID_VALUE, "q/k/v must be float32/float16/bfloat16");
  if (!(isfinite(scale) && scale > 0.f)) return fail(QD_ERR_INVALID_VALUE, "scale must be positive and finite");
  // The split and merge grids put the batch (and the explicit split layout
  // the kv-heads) in a grid dimension limited to 65535.  The reference
  // validates these sizes only up to INT_MAX (gqa_decode.cu:133-138) and a
  // launch beyond the grid fails with "gqa_decode kernel launch failed:
  // <error>" (:179-181); the same error and text are reported here before
  // any launch.
  if (batch > 65535 || kv_heads > 65535)
    return fail(static_cast<int>(hipErrorInvalidConfiguration),
                std::string("gqa_decode kernel launch failed: ") + hipGetErrorString(hipErrorInvalidConfiguration));
  return QD_OK;
}

#ifdef QD_STAMPS
uint64_t* g_stamps = nullptr;  // diagnostic build: qd_diag_set_stamps
#endif

DecodeParams make_params(const void* q, const void* k_cache, const void* v_cache,
                         const int32_t* block_table, const int32_t* context_lens, void* out,
                         void* workspace, int batch, int q_heads, int kv_heads, int head_dim,
                         int block_size, int max_pages, int64_t num_blocks, float scale, int splits,
                         int chunk_pages) {
  DecodeParams prm;
  prm.q = q;
  prm.k = k_cache;
  prm.v = v_cache;
  prm.table = block_table;
  prm.lens = context_lens;
  prm.out = out;
  prm.ws = static_cast<float*>(workspace);
  prm.B = batch;
  prm.Hq = q_heads;
  prm.Hkv = kv_heads;
  prm.D = head_dim;
  prm.P = block_size;
  prm.maxP = max_pages;
  prm.g = q_heads / kv_heads;
  prm.splits = splits;
  prm.chunk_pages = chunk_pages;
  prm.head_chunks = (prm.g + generic_heads(prm.g) - 1) / generic_heads(prm.g);
  prm.num_blocks = num_blocks;
  prm.sl2 = scale * kLog2e;
  prm.meta = nullptr;
  prm.wg_waves = 1;
  prm.ctr = nullptr;
  prm.stage_bytes = 0;
  prm.kv_split = 1;
  prm.kv_rows = kv_heads;
  prm.kv_g = prm.g;
#ifdef QD_STAMPS
  prm.stamps = g_stamps;
#endif
  return prm;
}

// Scratch bytes the automatic path needs for these shapes: the larger of
// the aligned and unaligned plans, so that the size does not depend on
// pointer alignment (QD_STAGE_VALU's plan runs on the same grid and fits).
// 0 for invalid shapes.
size_t auto_scratch_bytes(int batch, int q_heads, int kv_heads, int head_dim, int block_size, int max_pages,
                          int dtype) {
  if (check_launch_shapes(batch, q_heads, kv_heads, head_dim, block_size, max_pages, 1, dtype, 1.f) != QD_OK)
    return 0;
  AutoPlan a, b;
  if (auto_plan(batch, q_heads, kv_heads, head_dim, block_size, max_pages, dtype, true, &a) != QD_OK ||
      auto_plan(batch, q_heads, kv_heads, head_dim, block_size, max_pages, dtype, false, &b) != QD_OK)
    return 0;
  return a.ws_bytes > b.ws_bytes ? a.ws_bytes : b.ws_bytes;
}

int launch_error() {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(static_cast<int>(e), std::string("gqa_decode kernel launch failed: ") + hipGetErrorString(e));
  return QD_OK;
}

// Scratch of the no-allocation entry point: one array per GPU the library
// runs on, held until the process ends.  In host code `scratch` names a
// host-side stand-in, not device memory: the device address comes from
// hipGetSymbolAddress, once per device (no_alloc_scratch below).
constexpr size_t kNoAllocScratchBytes = size_t{16} << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

// Device address of `scratch` on the current device (looked up on the first
// call on that device, with it current), or null with *status set.
void* no_alloc_scratch(int* status) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    *status = fail(e != hipSuccess ? static_cast<int>(e) : QD_ERR_INVALID_VALUE,
                   "no current device for the no-allocation scratch");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      *status = fail(e != hipSuccess ? static_cast<int>(e) : QD_ERR_INVALID_VALUE,
                     std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
      return nullptr;
    }
    addr[dev] = ptr;
  }
  *status = QD_OK;
  return addr[dev];
}

}  // namespace

extern "C" {

int qd_abi_version(void) { return QD_ATTENTION_ABI_VERSION; }

const char* qd_error_string(int status) {
  if (status == QD_OK) return "success";
  if (status == g_last_status && !g_last_error.empty()) return g_last_error.c_str();
  return hipGetErrorString(static_cast<hipError_t>(status));
}

int qd_gqa_decode_validate(const qd_tensor_desc* q, const qd_tensor_desc* k,
                           const qd_tensor_desc* v, const qd_tensor_desc* table,
                           const qd_tensor_desc* lens, double scale, int64_t splits, char* msg,
                           size_t cap) {
  if (!q || !k || !v || !table || !lens) return invalid(msg, cap, "null tensor descriptor");
  if (!(splits >= 1 && splits <= 65535)) return invalid(msg, cap, "splits must be in [1, 65535]");
  const qd_tensor_desc* all[5] = {q, k, v, table, lens};
  const char* names[5] = {"q", "k_cache", "v_cache", "block_table", "context_lens"};
  for (int i = 0; i < 5; ++i) {
    if (!all[i]->defined || !all[i]->is_device) {
      std::string m = std::string(names[i]) + " must be a CUDA tensor";
      return invalid(msg, cap, m.c_str());
    }
    if (!all[i]->contiguous) {
      std::string m = std::string(names[i]) + " must be contiguous";
      return invalid(msg, cap, m.c_str());
    }
  }
  if (q->ndim != 3) return invalid(msg, cap, "q must be [B, Hq, D]");
  if (k->ndim != 4) return invalid(msg, cap, "k_cache must be [Nblocks, BlockSize, Hkv, D]");
  if (!same_sizes(v, k)) return invalid(msg, cap, "v_cache shape mismatch");
  if (table->ndim != 2) return invalid(msg, cap, "block_table must be [B, MaxPages]");
  if (lens->ndim != 1) return invalid(msg, cap, "context_lens must be [B]");
  for (int i = 1; i < 5; ++i)
    if (all[i]->device_index != q->device_index)
      return invalid(msg, cap, "all tensors must use one CUDA device");
  if (q->dtype != k->dtype || q->dtype != v->dtype) return invalid(msg, cap, "q/k/v dtype must match");
  if (q->dtype != QD_DTYPE_F32 && q->dtype != QD_DTYPE_F16 && q->dtype != QD_DTYPE_BF16)
    return invalid(msg, cap, "q/k/v must be float32/float16/bfloat16");
  if (table->dtype != QD_DTYPE_I32 || lens->dtype != QD_DTYPE_I32)
    return invalid(msg, cap, "block_table and context_lens must be int32");
  if (q->sizes[0] != table->sizes[0] || q->sizes[0] != lens->sizes[0])
    return invalid(msg, cap, "batch sizes must match");
  if (q->sizes[2] != k->sizes[3]) return invalid(msg, cap, "q head_dim and cache head_dim must match");
  if (!(q->sizes[1] > 0 && k->sizes[2] > 0 && q->sizes[1] % k->sizes[2] == 0))
    return invalid(msg, cap, "Hq must be divisible by Hkv");
  if (!(q->sizes[2] > 0 && q->sizes[2] <= 256)) return invalid(msg, cap, "supported head_dim is [1, 256]");
  if (!(k->sizes[0] > 0 && k->sizes[1] > 0))
    return invalid(msg, cap, "cache must have positive blocks and block_size");
  if (!(table->sizes[1] > 0)) return invalid(msg, cap, "block_table must have at least one page");
  if (!(isfinite(scale) && scale > 0.0)) return invalid(msg, cap, "scale must be positive and finite");
  const int64_t imax = 2147483647;
  if (!(q->sizes[0] <= imax && q->sizes[1] <= imax && k->sizes[2] <= imax && k->sizes[1] <= imax &&
        table->sizes[1] <= imax))
    return invalid(msg, cap, "tensor sizes exceed int32 CUDA launch limits");
  copy_msg(msg, cap, "");
  return QD_OK;
}

int qd_gqa_decode_validate_workspace(const qd_tensor_desc* q, const qd_tensor_desc* ws,
                                     int64_t splits, char* msg, size_t cap) {
  if (!q || !ws) return invalid(msg, cap, "null tensor descriptor");
  if (!(splits > 1)) return invalid(msg, cap, "workspace requires splits > 1");
  if (!(ws->defined && ws->is_device && ws->device_index == q->device_index && ws->contiguous &&
        ws->dtype == QD_DTYPE_F32))
    return invalid(msg, cap, "workspace must be contiguous float32 on q device");
  if (!(ws->ndim == 4 && ws->sizes[0] == q->sizes[0] && ws->sizes[1] == q->sizes[1] &&
        ws->sizes[2] == splits && ws->sizes[3] == q->sizes[2] + 2))
    return invalid(msg, cap, "workspace shape must be [B,Hq,splits,D+2]");
  copy_msg(msg, cap, "");
  return QD_OK;
}

int qd_gqa_decode_plan(int batch, int q_heads, int kv_heads, int head_dim, int block_size,
                       int max_pages, int dtype, int cu_count, int* splits, int* chunk_pages) {
  (void)q_heads;
  (void)head_dim;
  (void)dtype;
  if (!splits || !chunk_pages) return fail(QD_ERR_INVALID_VALUE, "null plan output");
  if (batch < 0 || kv_heads <= 0 || block_size <= 0 || max_pages <= 0)
    return fail(QD_ERR_INVALID_VALUE, "invalid shapes for plan");
  const int64_t cus = cu_count > 0 ? cu_count : 256;
  // Work items are (sequence, kv-head) pairs; each split of one item is a
  // wave.  Aim for ~kPlanWavesPerCu waves per CU, and keep every split at
  // least kPlanMinTokens tokens and at most 64 pages, so that split partials
  // stay a small fraction of the K/V bytes (for 32 tokens and 4 heads per
  // kv-head: 2 KB of fp32 partials against 16-32 KB of K/V).  Short
  // sequences get many short splits: a wave streams its split's tokens in
  // order.  Measured on the fp32 sweep shapes (Hq32 Hkv8 D128, every split
  // count from 8 to 512): the fastest split count gave about 4 waves per CU
  // at B1/L16384 (S128), B4/L4096 (S32), B16/L1024 and B16/L4096 (S8), where
  // 8 per CU took 10-27% longer (more split starts, and rows for the merge).
  const int64_t items = static_cast<int64_t>(batch) * kv_heads;
  const int64_t target_waves = cus * kPlanWavesPerCu;
  int64_t want = items > 0 ? (target_waves + items - 1) / items : 1;
  if (want < 1) want = 1;
  const int64_t min_pages = (kPlanMinTokens + block_size - 1) / block_size;
  int64_t cp = (max_pages + want - 1) / want;
  if (cp < min_pages) cp = min_pages;
  if (cp > 64) cp = 64;
  if (cp > max_pages) cp = max_pages;
  int64_t s = (max_pages + cp - 1) / cp;
  if (s > 65535) {
    s = 65535;
    cp = (max_pages + s - 1) / s;
  }
  *splits = static_cast<int>(s);
  *chunk_pages = static_cast<int>(cp);
  return QD_OK;
}

size_t qd_gqa_decode_workspace_bytes(int batch, int q_heads, int head_dim, int splits) {
  if (splits <= 1 || batch <= 0 || q_heads <= 0 || head_dim <= 0) return 0;
  return static_cast<size_t>(batch) * q_heads * splits * (head_dim + 2) * sizeof(float);
}

int qd_gqa_decode_kernel_kind(int q_heads, int kv_heads, int head_dim, int block_size, int dtype,
                              int flags) {
  if (flags & QD_FLAG_FORCE_GENERIC) return 0;
  return mfma_applies(q_heads, kv_heads, head_dim, block_size, dtype) ? 1 : 0;
}

int qd_gqa_decode_launch(const void* q, const void* k_cache, const void* v_cache,
                         const int32_t* block_table, const int32_t* context_lens, void* out,
                         float* workspace, size_t workspace_bytes, int batch, int q_heads,
                         int kv_heads, int head_dim, int block_size, int max_pages,
                         int64_t num_blocks, int dtype, float scale, int splits, int chunk_pages,
                         int flags, void* stream) {
  int st = check_launch_shapes(batch, q_heads, kv_heads, head_dim, block_size, max_pages, num_blocks,
                               dtype, scale);
  if (st != QD_OK) return st;
  if (splits < 1 || splits > 65535) return fail(QD_ERR_INVALID_VALUE, "splits must be in [1, 65535]");
  if (chunk_pages < 0) return fail(QD_ERR_INVALID_VALUE, "chunk_pages must be >= 0");
  if (chunk_pages > 0 && static_cast<int64_t>(chunk_pages) * splits < max_pages)
    return fail(QD_ERR_INVALID_VALUE, "splits * chunk_pages must cover max_pages");
  if (batch == 0) return QD_OK;
  if (!q || !k_cache || !v_cache || !block_table || !context_lens || !out)
    return fail(QD_ERR_INVALID_VALUE, "null tensor pointer");
  if (splits > 1) {
    const size_t need = qd_gqa_decode_workspace_bytes(batch, q_heads, head_dim, splits);
    if (!workspace || workspace_bytes < need)
      return fail(QD_ERR_INVALID_VALUE, "workspace too small for [B,Hq,splits,D+2] float32");
  }

  DecodeParams prm = make_params(q, k_cache, v_cache, block_table, context_lens, out, workspace, batch,
                                 q_heads, kv_heads, head_dim, block_size, max_pages, num_blocks, scale,
                                 splits, chunk_pages);
  hipStream_t stm = static_cast<hipStream_t>(stream);
  // The MFMA kernel's vector loads and stores need 16-byte aligned tensors
  // and an 8-byte aligned workspace (its partials are stored in float pairs);
  // the generic kernel stores single elements.
  const bool use_mfma = qd_gqa_decode_kernel_kind(q_heads, kv_heads, head_dim, block_size, dtype, flags) &&
                        aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && aligned16(out) &&
                        (splits <= 1 || (reinterpret_cast<uintptr_t>(workspace) & 7u) == 0);
  (void)hipGetLastError();  // start from a clean error state
  if (use_mfma) {
    const KernelFn fn = dtype == QD_DTYPE_F16 ? pick_mfma<QD_DTYPE_F16>(head_dim)
                                              : pick_mfma<QD_DTYPE_BF16>(head_dim);
    hipLaunchKernelGGL(fn, dim3(splits, kv_heads, batch), dim3(64), 0, stm, prm);
  } else {
    KernelFn fn;
    switch (dtype) {
      case QD_DTYPE_F32: fn = pick_generic<QD_DTYPE_F32>(head_dim, prm.g); break;
      case QD_DTYPE_F16: fn = pick_generic<QD_DTYPE_F16>(head_dim, prm.g); break;
      default: fn = pick_generic<QD_DTYPE_BF16>(head_dim, prm.g); break;
    }
    const int64_t gx = static_cast<int64_t>(splits) * prm.head_chunks;
    if (gx > 2147483647) return fail(QD_ERR_INVALID_VALUE, "splits * head chunks exceed the grid limit");
    hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(gx), kv_heads, batch), dim3(64), 0, stm, prm);
  }
  if (splits > 1) {
    hipLaunchKernelGGL(pick_combine(dtype, head_dim, out, workspace), dim3(q_heads, batch), dim3(64), 0, stm, prm);
  }
  return launch_error();
}

size_t qd_gqa_decode_auto_workspace_bytes(int batch, int q_heads, int kv_heads, int head_dim,
                                          int block_size, int max_pages, int dtype) {
  return auto_scratch_bytes(batch, q_heads, kv_heads, head_dim, block_size, max_pages, dtype);
}

size_t qd_gqa_decode_auto_counter_bytes(void) { return kCounterBytes; }

int qd_gqa_decode_auto_stages(const void* q, const void* k_cache, const void* v_cache,
                              const int32_t* block_table, const int32_t* context_lens, void* out,
                              void* workspace, size_t workspace_bytes, int batch, int q_heads,
                              int kv_heads, int head_dim, int block_size, int max_pages,
                              int64_t num_blocks, int dtype, float scale, int stages, void* stream) {
  const bool valu = (stages & QD_STAGE_VALU) != 0;
  const bool unfused = (stages & QD_STAGE_UNFUSED) != 0;
  const bool force_fused = (stages & QD_STAGE_FUSED) != 0;
  stages &= ~(QD_STAGE_VALU | QD_STAGE_UNFUSED | QD_STAGE_FUSED);
  if ((stages & ~QD_STAGE_ALL) != 0 || stages == 0)
    return fail(QD_ERR_INVALID_VALUE, "stages must be a non-empty mask of QD_STAGE_*");
  if (unfused && force_fused) return fail(QD_ERR_INVALID_VALUE, "QD_STAGE_UNFUSED and QD_STAGE_FUSED exclude each other");
  int st = check_launch_shapes(batch, q_heads, kv_heads, head_dim, block_size, max_pages, num_blocks,
                               dtype, scale);
  if (st != QD_OK) return st;
  if (batch == 0) return QD_OK;
  if (!q || !k_cache || !v_cache || !block_table || !context_lens || !out)
    return fail(QD_ERR_INVALID_VALUE, "null tensor pointer");
  const bool aligned = aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && aligned16(out);
  if (valu && !(aligned && valu_sk_applies(q_heads, kv_heads, head_dim, dtype) &&
                mfma_applies(q_heads, kv_heads, head_dim, block_size, dtype) && batch <= kSkMaxBatch))
    return fail(QD_ERR_INVALID_VALUE, "QD_STAGE_VALU needs the balanced path with head_dim 128 and group size <= 8");
  AutoPlan ap;
  st = auto_plan(batch, q_heads, kv_heads, head_dim, block_size, max_pages, dtype, aligned, &ap, valu);
  if (st != QD_OK) return st;
  if (!workspace || workspace_bytes < ap.ws_bytes || !aligned16(workspace))
    return fail(QD_ERR_INVALID_VALUE, "workspace smaller than qd_gqa_decode_auto_workspace_bytes()");
  char* scratch = static_cast<char*>(workspace);
  if (!ap.stream_k) {
    if (stages != QD_STAGE_ALL)
      return fail(QD_ERR_INVALID_VALUE, "stages apply to the balanced MFMA path only");
    return qd_gqa_decode_launch(q, k_cache, v_cache, block_table, context_lens, out,
                                reinterpret_cast<float*>(scratch + kCounterBytes), ap.ws_bytes - kCounterBytes,
                                batch, q_heads, kv_heads, head_dim, block_size, max_pages, num_blocks,
                                dtype, scale, ap.splits, ap.chunk_pages, 0, stream);
  }
  bool fused = ap.fused;
  if (unfused) fused = false;
  if (force_fused) {
    if (valu || dtype == QD_DTYPE_F32 || ap.kv_split > 1 || !fused_fits(batch, q_heads, kv_heads, head_dim, ap.wgs) ||
        ap.stash_bytes > kFusedMaxStash ||
        !allow_dyn_lds(pick_mfma_sk_dt(dtype, head_dim, ap.kv_per_wave, ap.wide, true)))
      return fail(QD_ERR_INVALID_VALUE, "QD_STAGE_FUSED needs 16-bit MFMA math, at most 16 q-heads per kv-head, "
                                        "batch * kv_heads <= 65536 and partial slots below 2 GiB");
    fused = true;
  }
  DecodeParams prm = make_params(q, k_cache, v_cache, block_table, context_lens, out, scratch + kCounterBytes,
                                 batch, q_heads, kv_heads, head_dim, block_size, max_pages, num_blocks, scale,
                                 ap.wgs, 0);
  prm.meta = reinterpret_cast<int*>(scratch + ap.meta_offset);
  prm.ctr = reinterpret_cast<uint32_t*>(scratch);
  prm.wg_waves = ap.wg_waves;
  prm.stage_bytes = ap.stage_bytes ? static_cast<int>(ap.stage_bytes / ap.wg_waves) : 0;
  if (ap.kv_split > 1) {
    prm.Hkv = kv_heads * ap.kv_split;
    prm.g = kv_chunk_heads(q_heads, kv_heads, ap.kv_split);
    prm.kv_split = ap.kv_split;
    prm.kv_rows = kv_heads;
    prm.kv_g = q_heads / kv_heads;
  }
  hipStream_t stm = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  if (fused) {
    // One kernel: decode and merge.  QD_STAGE_MERGE alone has nothing to do.
    if (stages & QD_STAGE_DECODE)
      hipLaunchKernelGGL(pick_mfma_sk_dt(dtype, head_dim, ap.kv_per_wave, ap.wide, true), dim3(ap.wgs),
                         dim3(64 * ap.wg_waves), ap.stash_bytes, stm, prm);
    return launch_error();
  }
  if (stages & QD_STAGE_DECODE)
    hipLaunchKernelGGL(valu ? pick_valu_sk_dt(dtype, q_heads / kv_heads)
                            : pick_mfma_sk_dt(dtype, head_dim, ap.kv_per_wave, ap.wide, false, ap.stage_bytes > 0),
                       dim3(ap.wgs), dim3(64 * ap.wg_waves), ap.stage_bytes, stm, prm);
  if (stages & QD_STAGE_MERGE) {
    const bool one_head = merge_one_head_per_wave(batch, q_heads);
    hipLaunchKernelGGL(pick_merge_sk_dt(dtype, head_dim, one_head),
                       dim3(one_head ? q_heads : (q_heads + 3) / 4, batch), dim3(64), 0, stm, prm);
  }
  return launch_error();
}

int qd_gqa_decode_auto(const void* q, const void* k_cache, const void* v_cache,
                       const int32_t* block_table, const int32_t* context_lens, void* out,
                       void* workspace, size_t workspace_bytes, int batch, int q_heads, int kv_heads,
                       int head_dim, int block_size, int max_pages, int64_t num_blocks, int dtype,
                       float scale, void* stream) {
  return qd_gqa_decode_auto_stages(q, k_cache, v_cache, block_table, context_lens, out, workspace,
                                   workspace_bytes, batch, q_heads, kv_heads, head_dim, block_size,
                                   max_pages, num_blocks, dtype, scale, QD_STAGE_ALL, stream);
}

size_t qd_gqa_decode_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

int qd_gqa_decode_auto_noalloc(const void* q, const void* k_cache, const void* v_cache,
                               const int32_t* block_table, const int32_t* context_lens, void* out, int batch,
                               int q_heads, int kv_heads, int head_dim, int block_size, int max_pages,
                               int64_t num_blocks, int dtype, float scale, void* stream) {
  int st = check_launch_shapes(batch, q_heads, kv_heads, head_dim, block_size, max_pages, num_blocks, dtype,
                               scale);
  if (st != QD_OK) return st;
  if (batch == 0) return QD_OK;
  const size_t need = auto_scratch_bytes(batch, q_heads, kv_heads, head_dim, block_size, max_pages, dtype);
  if (need > kNoAllocScratchBytes)
    return fail(QD_ERR_INVALID_VALUE, "shapes need " + std::to_string(need) +
                                          " bytes of scratch, more than the no-allocation scratch holds (" +
                                          std::to_string(kNoAllocScratchBytes) + ")");
  void* ws = no_alloc_scratch(&st);
  if (!ws) return st;
  return qd_gqa_decode_auto_stages(q, k_cache, v_cache, block_table, context_lens, out, ws, kNoAllocScratchBytes,
                                   batch, q_heads, kv_heads, head_dim, block_size, max_pages, num_blocks, dtype,
                                   scale, QD_STAGE_ALL, stream);
}

int qd_gqa_decode_auto_info(int batch, int q_heads, int kv_heads, int head_dim, int block_size,
                            int max_pages, int dtype, int* waves, int* splits, int* chunk_pages) {
  if (check_launch_shapes(batch, q_heads, kv_heads, head_dim, block_size, max_pages, 1, dtype, 1.f) !=
      QD_OK)
    return -1;
  AutoPlan ap;
  if (auto_plan(batch, q_heads, kv_heads, head_dim, block_size, max_pages, dtype, true, &ap) != QD_OK)
    return -1;
  if (waves) *waves = ap.stream_k ? ap.wgs * ap.wg_waves : 0;
  if (splits) *splits = ap.splits;
  if (chunk_pages) *chunk_pages = ap.chunk_pages;
  return ap.stream_k ? (ap.fused ? 2 : 1) : 0;
}

#ifdef QD_STAMPS
// Diagnostic build only: per-wave timestamps of the stream-K kernel go to
// `buffer` (16 words per wave, the grid's waves in order) for the launches
// that follow, until called again (NULL stops them).
int qd_diag_set_stamps(void* buffer) {
  g_stamps = static_cast<uint64_t*>(buffer);
  return QD_OK;
}
#endif

}  // extern "C"
