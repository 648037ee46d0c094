/*
 * qd_attention.h — C ABI of the MI355X (gfx950) paged grouped-query decode
 * attention library `libqd_attention.so`.
 *
 * Everything here is plain C: pointers, sizes and integer codes.  No torch,
 * no C++ and no HIP types cross this boundary (a HIP stream is passed as an
 * opaque `void*`, NULL meaning the null stream).  The torch binding
 * (`attention_amd/csrc/torch_ops.cpp`) is one caller; a ctypes/cffi/cgo
 * binding is another.
 *
 * Reference interfaces replaced (paths relative to the reference tree):
 *   qd_gqa_decode_validate            csrc/cuda/dense/gqa_decode.cu:103-138
 *   qd_gqa_decode_validate_workspace  csrc/cuda/dense/gqa_decode.cu:148-152
 *   qd_gqa_decode_plan                attention/core.py:80-96 (gqa_decode_auto)
 *   qd_gqa_decode_workspace_bytes     csrc/cuda/dense/gqa_decode.cu:152-154
 *   qd_gqa_decode_launch              csrc/cuda/dense/gqa_decode.cu:140-183,
 *                                     kernels :18-87 (explicit splits)
 *   qd_gqa_decode_auto(+_stages, _workspace_bytes, _info)
 *                                     csrc/cuda/dense/gqa_decode.cu:186-188
 *                                     and attention/core.py:80-96
 *
 * Tensor layouts (all row-major, contiguous, on one device):
 *   q            [batch, q_heads, head_dim]                   dtype
 *   k/v cache    [num_blocks, block_size, kv_heads, head_dim] dtype
 *   block_table  [batch, max_pages]                           int32
 *   context_lens [batch]                                      int32
 *   out          [batch, q_heads, head_dim]                   dtype
 *   workspace    [batch, q_heads, splits, head_dim + 2]       float32
 *                per (b, h, s): {max scaled score, sum exp, acc[head_dim]}
 *
 * Metadata contents (page ids, lengths) are caller-owned and never checked
 * here: only table entries [0, ceil(len/block_size)) of each row are read,
 * and a length <= 0 yields an all-zero output row.
 */
#ifndef QD_ATTENTION_H
#define QD_ATTENTION_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QD_ATTENTION_ABI_VERSION 2

/* Element type codes shared by every entry point. */
enum {
  QD_DTYPE_F32 = 0,
  QD_DTYPE_F16 = 1,
  QD_DTYPE_BF16 = 2,
  QD_DTYPE_I32 = 3,
  QD_DTYPE_I64 = 4,
  QD_DTYPE_OTHER = -1
};

/* Status codes.  0 is success; any other value is a hipError_t code
 * (hipErrorInvalidValue = 1 for argument errors).  qd_error_string() gives
 * the message of the last failure on the calling thread. */
enum { QD_OK = 0, QD_ERR_INVALID_VALUE = 1 };

/* Kernel-selection flags (qd_gqa_decode_launch, qd_mla_*). */
enum {
  /* Use the portable VALU kernel even where the MFMA kernel applies. */
  QD_FLAG_FORCE_GENERIC = 1,
  /* MLA attention: use the workgroup-staged MFMA kernel even where the
   * wave-streamed or the shared-tile kernel applies (testing and
   * comparison). */
  QD_FLAG_MLA_STAGED = 2,
  /* MLA attention: use the wave-streamed MFMA kernel even where the
   * shared-tile kernel applies (testing and comparison). */
  QD_FLAG_MLA_WAVE = 4
};

/* Shape/placement descriptor of one tensor, for validation only. */
typedef struct qd_tensor_desc {
  int32_t defined;      /* 0: argument absent (optional workspace)        */
  int32_t is_device;    /* 1: GPU tensor                                   */
  int32_t device_index; /* device ordinal (ignored when !is_device)        */
  int32_t contiguous;   /* 1: row-major contiguous                         */
  int32_t dtype;        /* QD_DTYPE_*                                      */
  int32_t ndim;         /* number of dimensions, <= 8                      */
  int64_t sizes[8];
} qd_tensor_desc;

/* ABI version of the loaded library (QD_ATTENTION_ABI_VERSION). */
int qd_abi_version(void);

/* Message for `status`: the detailed text of the calling thread's last
 * failure when it matches, else the HIP error name. Never NULL. */
const char* qd_error_string(int status);

/* Checks shapes, dtypes and placement in the reference's order
 * (gqa_decode.cu:103-138).  Returns 0, or QD_ERR_INVALID_VALUE with the
 * reference's message copied into msg (NUL-terminated, truncated to
 * msg_cap).  Reads no tensor contents. */
int qd_gqa_decode_validate(const qd_tensor_desc* q, const qd_tensor_desc* k_cache,
                           const qd_tensor_desc* v_cache, const qd_tensor_desc* block_table,
                           const qd_tensor_desc* context_lens, double scale, int64_t splits,
                           char* msg, size_t msg_cap);

/* Workspace checks of the split path (gqa_decode.cu:148-152); call after
 * qd_gqa_decode_validate succeeded and only when batch > 0. */
int qd_gqa_decode_validate_workspace(const qd_tensor_desc* q, const qd_tensor_desc* workspace,
                                     int64_t splits, char* msg, size_t msg_cap);

/* Launch plan for the automatic path: number of context splits and pages
 * per split, chosen from static shapes only (no device reads, no sync).
 * cu_count <= 0 means 256 (MI355X).  Writes *splits >= 1 and
 * *chunk_pages >= 1 (pages of block_size tokens per split). */
int qd_gqa_decode_plan(int batch, int q_heads, int kv_heads, int head_dim, int block_size,
                       int max_pages, int dtype, int cu_count, int* splits, int* chunk_pages);

/* Bytes of float32 workspace [batch, q_heads, splits, head_dim + 2]; 0 when
 * splits <= 1 (the single-split path needs none). */
size_t qd_gqa_decode_workspace_bytes(int batch, int q_heads, int head_dim, int splits);

/* Enqueues paged GQA decode on `stream` (a hipStream_t, NULL = null stream).
 *   splits      >= 1.  1: each (sequence, kv-head) in one pass, no
 *               workspace.  > 1: split-context partials into `workspace`
 *               and a log-sum-exp combine.
 *   chunk_pages 0: split s of a sequence with n pages covers pages
 *               [s*c, (s+1)*c), c = ceil(n/splits) (reference split API);
 *               > 0: fixed c = chunk_pages for every sequence (plan path;
 *               requires splits * chunk_pages >= max_pages).
 *   workspace   device float32 buffer of workspace_bytes >= the value of
 *               qd_gqa_decode_workspace_bytes(); may be NULL if splits == 1.
 * Does not allocate, does not synchronize and does not read metadata on
 * the host.  Returns 0 or a status code (argument errors are reported
 * before anything is enqueued). */
int qd_gqa_decode_launch(const void* q, const void* k_cache, const void* v_cache,
                         const int32_t* block_table, const int32_t* context_lens, void* out,
                         float* workspace, size_t workspace_bytes, int batch, int q_heads,
                         int kv_heads, int head_dim, int block_size, int max_pages,
                         int64_t num_blocks, int dtype, float scale, int splits,
                         int chunk_pages, int flags, void* stream);

/* Which kernel qd_gqa_decode_launch would run for these shapes:
 * 1 = MFMA kernel, 0 = portable VALU kernel. */
int qd_gqa_decode_kernel_kind(int q_heads, int kv_heads, int head_dim, int block_size,
                              int dtype, int flags);

/* ---- Automatic path: the body of attention.gqa_decode ----------------
 * Replaces csrc/cuda/dense/gqa_decode.cu:186-188 (gqa_decode_cuda, always
 * one split) and the split heuristic of attention/core.py:80-96.  The
 * partition is chosen from static shapes and the device (CU count and
 * kernel occupancy), never from context_lens on the host:
 *   - 16-bit caches with head_dim 64/96/128/256, block_size a multiple of 16,
 *     group size <= 128 (a group above 16 is served as ceil(g/16) chunks of
 *     at most 16 q-heads, each like a kv-head of its own) and batch <= 4096,
 *     and fp32 caches with head_dim 64/128, block_size a multiple of 16,
 *     group size <= 16 and batch * max_pages * block_size >= 65536 (fp32
 *     matrix-core products):
 *     the (sequence, 16-token group)
 *     space is cut into cost-balanced ranges, one per resident workgroup;
 *     a sequence split across workgroups leaves one partial per workgroup,
 *     folded (log-sum-exp) either inside the same kernel by the last
 *     workgroup to finish a piece of it (the fused merge, when the merge is
 *     short: see qd_gqa_decode_auto_info) or by a second kernel on the same
 *     stream;
 *   - otherwise: the split layout of qd_gqa_decode_launch with the plan of
 *     qd_gqa_decode_plan.
 * The workspace is device memory, 16-byte aligned, of at least
 * qd_gqa_decode_auto_workspace_bytes() bytes.  Its first
 * qd_gqa_decode_auto_counter_bytes() bytes are the fused merge's arrival
 * counters: they must be zero before the workspace's first use (zero the
 * whole workspace once when allocating it), and every call leaves them
 * zero, so a workspace is reused as it is.  The rest needs no
 * initialization: every call writes what it reads.  Calls that may run
 * concurrently (different streams, or replays of captured graphs on
 * different streams) need different workspaces.  Workspace size and
 * partition depend on the current device (hipGetDevice), so query and
 * launch with the same device current.  Does not allocate or synchronize. */
size_t qd_gqa_decode_auto_workspace_bytes(int batch, int q_heads, int kv_heads, int head_dim,
                                          int block_size, int max_pages, int dtype);

/* Bytes of arrival counters at the start of every automatic-path workspace
 * (fixed: 256 KiB). */
size_t qd_gqa_decode_auto_counter_bytes(void);

int qd_gqa_decode_auto(const void* q, const void* k_cache, const void* v_cache,
                       const int32_t* block_table, const int32_t* context_lens, void* out,
                       void* workspace, size_t workspace_bytes, int batch, int q_heads,
                       int kv_heads, int head_dim, int block_size, int max_pages,
                       int64_t num_blocks, int dtype, float scale, void* stream);

/* The automatic path's kernels, for callers that time or schedule them
 * separately (the balanced MFMA path only; the split path needs
 * QD_STAGE_ALL).  With the fused merge, QD_STAGE_DECODE is the whole call
 * and QD_STAGE_MERGE alone does nothing.  Otherwise QD_STAGE_DECODE alone
 * leaves split sequences unmerged, and a following QD_STAGE_MERGE call with
 * the same arguments and workspace on the same stream completes the
 * output. */
enum { QD_STAGE_DECODE = 1, QD_STAGE_MERGE = 2, QD_STAGE_ALL = 3 };
/* OR'ed into `stages` for measurement only: run the balanced path's decode
 * kernel with VALU math (packed dot products and fp32 FMAs) in place of the
 * MFMA instructions, same loads and partition (never fused).  Head_dim 128,
 * group size <= 8, one kv-head per wave; other shapes are rejected. */
enum { QD_STAGE_VALU = 4 };
/* OR'ed into `stages` for measurement only: merge split sequences with the
 * separate merge kernel (QD_STAGE_UNFUSED) or inside the decode kernel
 * (QD_STAGE_FUSED; batch * kv_heads <= 65536 and the partial slots below
 * 2 GiB) whatever the plan chose. */
enum { QD_STAGE_UNFUSED = 8, QD_STAGE_FUSED = 16 };

int qd_gqa_decode_auto_stages(const void* q, const void* k_cache, const void* v_cache,
                              const int32_t* block_table, const int32_t* context_lens, void* out,
                              void* workspace, size_t workspace_bytes, int batch, int q_heads,
                              int kv_heads, int head_dim, int block_size, int max_pages,
                              int64_t num_blocks, int dtype, float scale, int stages, void* stream);

/* ---- Automatic path without allocation ------------------------------
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same as qd_gqa_decode_auto, but its scratch is a
 * file-scope device array of qd_gqa_decode_noalloc_scratch_bytes() bytes
 * (16 MiB) per GPU, held until the process ends; shapes whose
 * qd_gqa_decode_auto_workspace_bytes() exceed it are rejected with
 * QD_ERR_INVALID_VALUE before anything is enqueued.  Nothing is allocated
 * (the array's address is looked up once per device).  Every call on a GPU
 * uses that GPU's one array: calls that may overlap on one GPU (different
 * streams, host threads) race and must be serialized by the caller. */
size_t qd_gqa_decode_noalloc_scratch_bytes(void);

int qd_gqa_decode_auto_noalloc(const void* q, const void* k_cache, const void* v_cache,
                               const int32_t* block_table, const int32_t* context_lens, void* out, int batch,
                               int q_heads, int kv_heads, int head_dim, int block_size, int max_pages,
                               int64_t num_blocks, int dtype, float scale, void* stream);

/* Describes the automatic path's choice (assuming aligned pointers):
 * returns 2 for the balanced MFMA path with the fused merge, 1 for it with
 * the separate merge kernel (*waves = its total wave count), 0 for the split
 * path (*splits, *chunk_pages), -1 for invalid shapes.  Any output pointer
 * may be NULL. */
int qd_gqa_decode_auto_info(int batch, int q_heads, int kv_heads, int head_dim, int block_size,
                            int max_pages, int dtype, int* waves, int* splits, int* chunk_pages);

/* ---- Paged KV-cache append ------------------------------------------
 * Replaces csrc/cuda/cache/kv_append.cu:29-56 (kv_append_cuda) behind the
 * op kv_append (csrc/binding/torch_ops.cpp:52; attention/core.py:59-63).
 *   key, value   [batch, kv_heads, head_dim]                   dtype
 *   k/v cache    [num_blocks, block_size, kv_heads, head_dim]  dtype (written)
 *   block_table  [batch, max_pages] int32, positions [batch] int32
 * Sequence b's token goes to row (block_table[b][pos/block_size],
 * pos % block_size) of both caches.  Destinations are caller-owned and
 * must be distinct; a position outside [0, max_pages*block_size) or a page
 * id outside [0, num_blocks) is skipped (never written). */

/* The reference's checks in order (kv_append.cu:32-43), messages included. */
int qd_kv_append_validate(const qd_tensor_desc* key, const qd_tensor_desc* value,
                          const qd_tensor_desc* k_cache, const qd_tensor_desc* v_cache,
                          const qd_tensor_desc* block_table, const qd_tensor_desc* positions, char* msg,
                          size_t msg_cap);

/* Enqueues the append on `stream`; no allocation, no synchronization. */
int qd_kv_append_launch(const void* key, const void* value, void* k_cache, void* v_cache,
                        const int32_t* block_table, const int32_t* positions, int batch, int kv_heads,
                        int head_dim, int block_size, int max_pages, int64_t num_blocks, int dtype,
                        void* stream);

/* ---- Paged metadata validation --------------------------------------
 * Device-side body of attention.validation.validate_paged_metadata
 * (attention/validation.py:5-39).  Checks, per sequence b in order: the
 * length is in [0, max_pages*block_size]; every used page id
 * (ceil(len/block_size) of them) is in [0, num_blocks); and, when
 * `positions` is not NULL, the append position is in
 * [0, max_pages*block_size), its page id is in [0, num_blocks) and its
 * (page, slot) destination is not taken by an earlier sequence.
 * Writes to device memory `*result` the first failure in the reference's
 * order as (b << 35) | (check << 32) | page, or all ones when the metadata
 * is valid; `page` is the failing page index for QD_META_BAD_PAGE.
 * Enqueues two kernels on `stream`; the caller reads *result after them.
 * Requires batch < 2^28, max_pages > 0, block_size > 0, num_blocks > 0. */
enum {
  QD_META_BAD_LENGTH = 1,      /* "invalid length at batch {b}"          */
  QD_META_BAD_PAGE = 2,        /* "invalid block at batch {b}, page {p}" */
  QD_META_BAD_POSITION = 3,    /* "invalid append position at batch {b}" */
  QD_META_BAD_APPEND_PAGE = 4, /* "invalid append page at batch {b}"     */
  QD_META_CONFLICT = 5         /* "conflicting append destinations"      */
};

int qd_validate_paged_metadata(const int32_t* block_table, const int32_t* context_lens,
                               const int32_t* positions, int batch, int max_pages, int block_size,
                               int64_t num_blocks, unsigned long long* result, void* stream);

/* ---- Paged MLA (multi-head latent attention) decode -----------------
 * Replaces the reference's MLA decode operators (csrc/cuda/mla/mla.cu,
 * ops mla_project / latent_kv_write / mla_attend / mla_decode_fused,
 * csrc/binding/torch_ops.cpp:47-50; Python attention/mla.py:16-53).
 * Layouts (row-major, contiguous, one device, one dtype unless noted):
 *   cache        [num_blocks, block_size, latent_dim + rope_dim]
 *                (latent | rope key per token)
 *   block_table  [batch, max_pages] int32; lengths [batch] int32
 *   positions    [batch, q_len] int32 (absolute position of each query)
 *   indices      [batch, q_len, num_indices] int32 logical token ids;
 *                num_indices = -1 (indices unused, may be NULL) attends to
 *                all visible tokens; ids outside [0, end) are skipped
 *   q / q_nope   [batch, q_len, heads, latent_dim / nope_dim]
 *   q_rope       [batch, q_len, heads, rope_dim]
 *   w_uk [heads, nope_dim, latent_dim]; w_uv [heads, value_dim, latent_dim]
 * Query row (b, t) sees tokens [0, end) with end = min(len, max(0, pos+1))
 * when `causal`, else len (clamped to max_pages*block_size); a row with no
 * visible token is zero.  `splits` 0 picks the partition from static shapes
 * and the device; > 0 forces it: for the MFMA kernel (16-bit, latent and
 * rope widths multiples of 8, latent <= 512) the number of workgroups that
 * share the batch's (row, 32-token tile) space in equal ranges (stream-K),
 * (16-token tiles for the wave-streamed kernel, in cost units), for the
 * VALU kernel the number of context splits per row.
 * qd_mla_attend_info() reports the kernel and the partition.  flags:
 * QD_FLAG_FORCE_GENERIC selects the VALU kernels, QD_FLAG_MLA_STAGED the
 * workgroup-staged MFMA kernel where the wave-streamed or shared-tile kernel
 * would run, QD_FLAG_MLA_WAVE the wave-streamed kernel where the shared-tile
 * kernel would run.
 * Nothing here allocates or synchronizes. */

/* Reference checks in order, messages included (mla.cu:152-155). */
int qd_latent_kv_write_validate(const qd_tensor_desc* latent, const qd_tensor_desc* rope,
                                const qd_tensor_desc* cache, const qd_tensor_desc* slots, char* msg,
                                size_t msg_cap);

/* Writes [latent | rope] of token t to flat cache row slots[t] (int64) of
 * the [num_blocks*block_size, latent_dim+rope_dim] view (mla.cu:28-32,
 * :151-160).  Rows outside [0, cache_rows) are skipped. */
int qd_latent_kv_write(const void* latent, const void* rope, void* cache, const int64_t* slots, int64_t tokens,
                       int latent_dim, int rope_dim, int64_t cache_rows, int dtype, void* stream);

/* Reference checks in order, messages included (mla.cu:139-142). */
int qd_mla_project_validate(const qd_tensor_desc* x, const qd_tensor_desc* w, int absorb, char* msg,
                            size_t msg_cap);

/* Per-head projection over rows = batch*q_len (mla.cu:16-27, :138-150):
 *   absorb != 0: out[r,h,o] = sum_k x[r,h,k] * w[h,k,o]  (w [H, in, out])
 *   absorb == 0: out[r,h,o] = sum_k x[r,h,k] * w[h,o,k]  (w [H, out, in])
 * fp32 accumulation, output rounded to the dtype. */
int qd_mla_project(const void* x, const void* w, void* out, int64_t rows, int heads, int in_dim, int out_dim,
                   int absorb, int dtype, int flags, void* stream);

/* Reference checks of mla_attend in order, messages included
 * (mla.cu:162-171); `indices` may be NULL or undefined. */
int qd_mla_attend_validate(const qd_tensor_desc* q, const qd_tensor_desc* q_rope, const qd_tensor_desc* cache,
                           const qd_tensor_desc* table, const qd_tensor_desc* lengths,
                           const qd_tensor_desc* positions, const qd_tensor_desc* indices, double scale,
                           char* msg, size_t msg_cap);

/* Workspace bytes qd_mla_attend needs (partials of rows split across
 * workgroups or splits, and per-row spans); 0 when none is needed. */
size_t qd_mla_attend_workspace_bytes(int batch, int q_len, int heads, int latent_dim, int rope_dim,
                                     int block_size, int max_pages, int num_indices, int dtype, int splits,
                                     int flags);

/* The plan qd_mla_attend would use: returns 3 for the shared-tile MFMA
 * kernel (dense rows, latent 512, rope 64, 32-token pages, 64 heads or more),
 * 2 for the wave-streamed MFMA kernel (dense rows, latent 512, rope 64,
 * 16-token pages, other head counts), 1 for the
 * workgroup-staged MFMA kernel (*out_splits = stream-K workgroups per head
 * group, *head_groups = head groups for both), 0 for the VALU kernel
 * (*out_splits = context splits per row, *head_groups = 0), -1 for invalid
 * shapes. */
int qd_mla_attend_info(int batch, int q_len, int heads, int latent_dim, int rope_dim, int block_size,
                       int max_pages, int num_indices, int dtype, int splits, int flags, int* out_splits,
                       int* head_groups);

/* Paged latent attention (mla.cu:34-82, :161-181): out [batch, q_len,
 * heads, latent_dim] = softmax((q . c + q_rope . k_rope) * scale) . c. */
int qd_mla_attend(const void* q, const void* q_rope, const void* cache, const int32_t* block_table,
                  const int32_t* lengths, const int32_t* positions, const int32_t* indices, void* out,
                  void* workspace, size_t workspace_bytes, int batch, int q_len, int heads, int latent_dim,
                  int rope_dim, int block_size, int max_pages, int64_t num_blocks, int num_indices, int causal,
                  int dtype, float scale, int splits, int flags, void* stream);

/* Reference checks of mla_decode_fused in order, messages included
 * (mla.cu:185-191). */
int qd_mla_decode_validate(const qd_tensor_desc* q_nope, const qd_tensor_desc* q_rope, const qd_tensor_desc* cache,
                           const qd_tensor_desc* table, const qd_tensor_desc* lengths,
                           const qd_tensor_desc* positions, const qd_tensor_desc* w_uk, const qd_tensor_desc* w_uv,
                           const qd_tensor_desc* indices, double scale, char* msg, size_t msg_cap);

/* Workspace bytes of qd_mla_decode (absorbed query, latent output and
 * split partials); 16-byte aligned device memory, no zeroing needed. */
size_t qd_mla_decode_workspace_bytes(int batch, int q_len, int heads, int latent_dim, int rope_dim,
                                     int block_size, int max_pages, int num_indices, int dtype, int splits,
                                     int flags);

/* Absorbed paged MLA decode (mla.cu:86-134, :184-198): query absorption,
 * latent attention and value projection, with the reference's rounding
 * points (absorbed query and latent output rounded to the dtype).
 * out [batch, q_len, heads, value_dim]. */
int qd_mla_decode(const void* q_nope, const void* q_rope, const void* cache, const int32_t* block_table,
                  const int32_t* lengths, const int32_t* positions, const void* w_uk, const void* w_uv,
                  const int32_t* indices, void* out, void* workspace, size_t workspace_bytes, int batch, int q_len,
                  int heads, int nope_dim, int latent_dim, int rope_dim, int value_dim, int block_size,
                  int max_pages, int64_t num_blocks, int num_indices, int causal, int dtype, float scale,
                  int splits, int flags, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QD_ATTENTION_H */
