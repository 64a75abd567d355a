/*
 * tsfa.h -- C ABI of libtsfa.so, the MI355X (gfx950) tree-sparse attention
 * library for EAGLE-style speculative-decoding verification.
 *
 * Every entry point is extern "C", stateless apart from a per-device cache of
 * the compute-unit count, takes plain pointers and sizes, enqueues its work on
 * the caller's stream and returns an int status (TSFA_OK == 0).  Device
 * pointers must be device memory of the current HIP device.  No entry point
 * allocates device memory: scratch comes in through `workspace`.
 *
 * Reference interfaces replaced (LUOseu/eagle3-tree-sparse-flashattn):
 *   tsfa_meta_build   prepare_tree_sparse_metadata     tree_sparse_flashattn.py:67-160
 *   tsfa_pack_bits    _pack_block_mask_to_int32         tree_sparse_flashattn.py:44-64
 *   tsfa_*_host       the same on a CPU mask (no device)
 *   tsfa_fwd          block_sparse_tree_fwd_kernel[grid] tree_sparse_flashattn.py:163-339
 *                     (argument list: tree_sparse_flashattn.py:164-203,
 *                      call sites eagle_tree_sparse_bridge.py:119-158,
 *                      benchmark.py:183-194)
 *   tsfa_tree_attention  run_tree_sparse_kernel            eagle_tree_sparse_bridge.py:76-159
 *                     (metadata build + forward in one call)
 */
#ifndef TSFA_H_
#define TSFA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* tsfa_stream_t; /* a hipStream_t; NULL = default stream */

enum tsfa_status {
  TSFA_OK = 0,
  TSFA_ERR_INVALID_ARGUMENT = 1, /* shapes/values the reference rejects (ValueError / assert) */
  TSFA_ERR_UNSUPPORTED = 2,      /* valid for the reference, outside this library's kernels */
  TSFA_ERR_WORKSPACE = 3,        /* workspace missing or smaller than *_workspace_bytes() */
  TSFA_ERR_LAUNCH = 4,           /* the HIP runtime refused a launch */
  TSFA_ERR_DEVICE = 5            /* no usable HIP device / attribute query failed */
};

enum tsfa_dtype { TSFA_DTYPE_FP16 = 0, TSFA_DTYPE_BF16 = 1, TSFA_DTYPE_FP32 = 2 };

/* Block codes of blk_type (tree_sparse_flashattn.py:11-12). ZERO blocks are absent. */
enum { TSFA_FULL_BLOCK = 0, TSFA_MIXED_BLOCK = 1 };

int tsfa_version(void);
const char* tsfa_status_string(int status);

/* ---------------------------------------------------------------- metadata
 * Builds the CSR + tri-state metadata of `n_seq` tree masks, bit-exact with
 * prepare_tree_sparse_metadata (tree_sparse_flashattn.py:67-160) applied to
 * each mask: mask[s][i][j] != 0 means visible (tree_sparse_flashattn.py:90).
 *
 * mask      uint8 [n_seq][q_len][q_len], element (s,i,j) at
 *           s*mask_seq_stride + i*mask_row_stride + j
 * Outputs use capacity strides so one launch serves every sequence
 * (nqb = ceil(q_len/block_m), ntb = ceil(q_len/block_n),
 *  W = ceil(block_m*block_n/32), cap = nqb*ntb):
 *   row_ptr  int32 [n_seq][nqb+1]
 *   col_idx  int32 [n_seq][cap]     first nnz[s] valid
 *   blk_type int8  [n_seq][cap]     first nnz[s] valid
 *   payload  int32 [n_seq][cap*W]   first n_mixed[s]*W valid
 *   offset   int32 [n_seq][cap]     first nnz[s] valid; the reference returns
 *                                   an EMPTY tensor when n_mixed[s] == 0
 *                                   (tree_sparse_flashattn.py:145-147)
 *   counts   int32 [n_seq][2]       {nnz, n_mixed}
 * Errors (tree_sparse_flashattn.py:85-88): block sizes <= 0 or q_len < 0 ->
 * TSFA_ERR_INVALID_ARGUMENT.
 */
int tsfa_meta_check_args(int n_seq, int q_len, int block_m, int block_n);
size_t tsfa_meta_workspace_bytes(int n_seq, int q_len, int block_m, int block_n);
int tsfa_meta_build(const uint8_t* mask, int64_t mask_seq_stride, int64_t mask_row_stride,
                    int n_seq, int q_len, int block_m, int block_n,
                    int32_t* row_ptr, int32_t* col_idx, int8_t* blk_type,
                    int32_t* payload, int32_t* offset, int32_t* counts,
                    void* workspace, size_t workspace_bytes, tsfa_stream_t stream);

/* Packs n_bits bools (uint8, nonzero = 1) row-major into ceil(n_bits/32)
 * int32 words, bit i of word w = bits[32w+i] (tree_sparse_flashattn.py:44-64). */
int tsfa_pack_bits(const uint8_t* bits, int64_t n_bits, int32_t* words, tsfa_stream_t stream);

/* The same two on the host (every pointer host memory, no device needed):
 * prepare_tree_sparse_metadata and _pack_block_mask_to_int32 of a CPU mask,
 * as the reference runs them (tree_sparse_flashattn.py:44-160, README.md
 * quick start).  Output layout and errors as tsfa_meta_build / tsfa_pack_bits. */
int tsfa_meta_build_host(const uint8_t* mask, int64_t mask_seq_stride, int64_t mask_row_stride,
                         int n_seq, int q_len, int block_m, int block_n,
                         int32_t* row_ptr, int32_t* col_idx, int8_t* blk_type,
                         int32_t* payload, int32_t* offset, int32_t* counts);
int tsfa_pack_bits_host(const uint8_t* bits, int64_t n_bits, int32_t* words);

/* ----------------------------------------------------------------- forward
 * Tree-sparse attention forward: for every (b, h, t) row,
 *   O = softmax(Q K^T * sm_scale + mask) V
 * over keys [0, prefix_len) (dense prefix) and the tree keys
 * prefix_len + tb*block_n + c (< kv_len) that the CSR row of q-block
 * t / block_m marks visible (FULL block, or MIXED bit set), with
 * kv head h / gqa_group_size.  Same semantics as block_sparse_tree_fwd_kernel
 * (tree_sparse_flashattn.py:163-339) including the -inf/NaN guards: a row
 * with no visible key yields NaN (0/0), as the reference does.
 *
 * q, o      [B, Hq, q_len, D] of `dtype`, last-dim stride 1
 * k, v      [B, Hkv, kv_len, D] of `dtype`, last-dim stride 1
 * strides   int64[16]: q(b,h,n,d), k(b,h,n,d), v(b,h,n,d), o(b,h,n,d) in
 *           elements, the reference's stride arguments in order
 *           (tree_sparse_flashattn.py:174-189); every d stride must be 1
 * metadata  row_ptr/col_idx/blk_type/payload/offset as produced by
 *           prepare_tree_sparse_metadata; meta_seq_stride[5] gives the
 *           per-batch-element stride (elements) of each of the five arrays:
 *           all zero = one tree shared by the batch (the reference's protocol),
 *           non-zero = one tree per sequence (tsfa_meta_build's layout)
 * o is written in `dtype` (one rounding of the fp32 result; the reference
 * stores through float16, tree_sparse_flashattn.py:339).
 * Supported: dtype fp16/bf16 with head_dim 64, 128 or 256, fp32 with head_dim
 * 64, 128 or 256 (the reference's tl.dot takes fp32, tree_sparse_flashattn.py:
 * 269, :278); block_n a positive multiple of 16, block_m >= 1, num_heads %
 * num_kv_heads == 0 with gqa_group_size == num_heads / num_kv_heads <= 256,
 * q_len >= 1, kv_len >= prefix_len >= 0, 16-byte aligned q/k/v/o rows.
 * head_dim 256 and fp32 run a simpler kernel whose split-KV partials are in
 * the input dtype (contiguous K/V only: tsfa_fwd_paged and tsfa_bwd refuse
 * them with TSFA_ERR_UNSUPPORTED); size their workspace with
 * tsfa_fwd_workspace_bytes_for_dtype.
 */
int tsfa_fwd_check_args(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len,
                        int prefix_len, int n_q_blocks, int n_tree_blocks, int gqa_group_size,
                        int block_m, int block_n, int head_dim, int dtype);
size_t tsfa_fwd_workspace_bytes(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len,
                                int prefix_len, int head_dim);
/* tsfa_fwd_workspace_bytes for inputs of `dtype` (tsfa_fwd_workspace_bytes
 * sizes 16-bit inputs; fp32 inputs' fp32 partials need more).  No reference
 * counterpart. */
size_t tsfa_fwd_workspace_bytes_for_dtype(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len,
                                          int prefix_len, int head_dim, int dtype);
int tsfa_fwd(const void* q, const void* k, const void* v, void* o,
             const int32_t* row_ptr, const int32_t* col_idx, const int8_t* blk_type,
             const int32_t* mixed_mask_payload, const int32_t* mixed_mask_offset,
             const int64_t* meta_seq_stride, const int64_t* strides, float sm_scale,
             int batch, int num_heads, int num_kv_heads, int q_len, int kv_len, int prefix_len,
             int n_q_blocks, int n_tree_blocks, int gqa_group_size,
             int block_m, int block_n, int head_dim, int dtype,
             void* workspace, size_t workspace_bytes, tsfa_stream_t stream);

/* tsfa_fwd that also writes the log-sum-exp of every query row:
 * lse[(b*num_heads + h)*q_len + t] = log sum_j exp(sm_scale * q.k_j) over the
 * row's visible keys (natural log, fp32, -inf for a row with no visible key).
 * No counterpart in the reference (its kernel keeps m_i / l_i in registers,
 * tree_sparse_flashattn.py:228-329, and has no backward); tsfa_bwd needs it. */
int tsfa_fwd_lse(const void* q, const void* k, const void* v, void* o, float* lse,
                 const int32_t* row_ptr, const int32_t* col_idx, const int8_t* blk_type,
                 const int32_t* mixed_mask_payload, const int32_t* mixed_mask_offset,
                 const int64_t* meta_seq_stride, const int64_t* strides, float sm_scale,
                 int batch, int num_heads, int num_kv_heads, int q_len, int kv_len, int prefix_len,
                 int n_q_blocks, int n_tree_blocks, int gqa_group_size,
                 int block_m, int block_n, int head_dim, int dtype,
                 void* workspace, size_t workspace_bytes, tsfa_stream_t stream);

/* Backward of tsfa_fwd.  No counterpart in the reference (README.md:198 lists
 * the backward kernel as missing).  Given q, k, v, the forward's o and lse
 * (tsfa_fwd_lse) and dout = dL/dO, writes
 *   dq = sm_scale * dS K,  dk = sm_scale * dS^T Q,  dv = P^T dO
 * with P = softmax of the visible scaled scores and dS = P * (dO V^T -
 * rowsum(dO * O)), dk / dv summed over the gqa_group_size query heads of each
 * kv head.  Rows with no visible key contribute nothing (their dq is 0).
 * strides  int64[32]: q, k, v, o, dout, dq, dk, dv -- (b, h, n, d) each, in
 *          elements, d stride 1, 16-byte aligned rows
 * Every other argument as in tsfa_fwd; workspace of
 * tsfa_bwd_workspace_bytes(..., n_trees) bytes, n_trees = batch when
 * meta_seq_stride is non-zero (one tree per sequence), else 1.  Three or
 * four kernel launches, no host synchronisation: the dQ kernel runs on a
 * library-owned side stream forked from `stream` after the first launch and
 * joined back before the call returns its last launch (one side stream and
 * two events per device and caller stream, kept for the process, at most
 * 64 per device, beyond which calls stay on `stream`; inside a
 * graph capture the fork and join are captured too; TSFA_BWD_CONCURRENT=0
 * keeps every launch on `stream`).  Supported: the
 * shapes tsfa_fwd supports with q_len * gqa_group_size < 2^22; the tree's
 * block-state table of one 32-row tile must fit 8192 entries (otherwise
 * TSFA_ERR_UNSUPPORTED, as tsfa_bwd_workspace_bytes returning 0 signals). */
size_t tsfa_bwd_workspace_bytes(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len,
                                int prefix_len, int block_m, int n_tree_blocks, int head_dim,
                                int n_trees);
int tsfa_bwd(const void* q, const void* k, const void* v, const void* o, const float* lse,
             const void* dout, void* dq, void* dk, void* dv,
             const int32_t* row_ptr, const int32_t* col_idx, const int8_t* blk_type,
             const int32_t* mixed_mask_payload, const int32_t* mixed_mask_offset,
             const int64_t* meta_seq_stride, const int64_t* strides, float sm_scale,
             int batch, int num_heads, int num_kv_heads, int q_len, int kv_len, int prefix_len,
             int n_q_blocks, int n_tree_blocks, int gqa_group_size,
             int block_m, int block_n, int head_dim, int dtype,
             void* workspace, size_t workspace_bytes, tsfa_stream_t stream);

/* tsfa_fwd over a paged K/V cache.  No counterpart in the reference's tree
 * kernel (it reads contiguous [B, Hkv, kv_len, D] tensors); it replaces the
 * gather a serving caller would otherwise run to turn its page pool into
 * that layout -- the FlashInfer cache that benchmark.py:67-91 builds
 * ([max_pages, 2, page_size, Hkv, D]) and hands to the paged decode
 * wrapper with indptr/indices (benchmark.py:114-133).  Same semantics and
 * metadata as tsfa_fwd, with key j of sequence b read from page
 * list_b[j / page_size], row j % page_size (K in slot 0, V in slot 1):
 *
 * kv_cache       pages of `dtype`, addressed by cache_strides
 * cache_strides  int64[5] in elements: page, K/V slot, row in page, kv head,
 *                d (d stride 1).  [pages, 2, page_size, Hkv, D] contiguous
 *                is FlashInfer's NHD layout; HND ([pages, 2, Hkv,
 *                page_size, D]) is the same call with the row and head
 *                strides swapped
 * kv_indptr      int32[batch + 1]: list_b = kv_indices[kv_indptr[b] ...]
 *                (FlashInfer's CSR form), or NULL for a dense table:
 *                list_b = kv_indices[b * page_table_stride ...]
 * kv_indices     int32 page ids, n_indices entries; list_b must hold
 *                ceil(kv_len / page_size) ids
 * n_pages        pages in kv_cache; page ids and list positions are clamped
 *                to the pool and to kv_indices, so no table content reads
 *                outside them (a bad table gives wrong O, never a fault)
 * page_size      keys per page: a power of two, >= 16
 * lse            NULL, or fp32 [B, Hq, q_len]: each row's log-sum-exp, as
 *                tsfa_fwd_lse writes it
 * q_strides, o_strides  int64[4] each: b, h, n, d
 * Every sequence has kv_len keys (prefix_len + tree), as in tsfa_fwd. */
int tsfa_fwd_paged(const void* q, const void* kv_cache, const int32_t* kv_indptr,
                   const int32_t* kv_indices, int64_t n_indices, int64_t page_table_stride,
                   int n_pages, int page_size, void* o, float* lse,
                   const int32_t* row_ptr, const int32_t* col_idx, const int8_t* blk_type,
                   const int32_t* mixed_mask_payload, const int32_t* mixed_mask_offset,
                   const int64_t* meta_seq_stride, const int64_t* q_strides,
                   const int64_t* cache_strides, const int64_t* o_strides, float sm_scale,
                   int batch, int num_heads, int num_kv_heads, int q_len, int kv_len, int prefix_len,
                   int n_q_blocks, int n_tree_blocks, int gqa_group_size,
                   int block_m, int block_n, int head_dim, int dtype,
                   void* workspace, size_t workspace_bytes, tsfa_stream_t stream);

/* run_tree_sparse_kernel(q, k, v, tree_mask) in one call
 * (eagle_tree_sparse_bridge.py:76-159: metadata from the tree mask, then the
 * forward with prefix_len = kv_len - q_len, eagle_tree_sparse_bridge.py:91-117):
 * tsfa_meta_build on the device mask into the front of `workspace`, then
 * tsfa_fwd reading that record, both on `stream`, no host synchronisation.
 * mask      uint8 (nonzero = visible) device memory: n_masks trees of
 *           [q_len, q_len] rows mask_row_stride apart, trees mask_seq_stride
 *           apart; n_masks = 1 (one tree for the batch, as the reference) or
 *           batch (one tree per sequence)
 * strides, dtype, sm_scale, o: as tsfa_fwd.
 * workspace of tsfa_tree_attention_workspace_bytes, 256-byte aligned.
 * Errors as tsfa_fwd / tsfa_meta_build; kv_len < q_len is
 * TSFA_ERR_INVALID_ARGUMENT (the reference's ValueError).  The forward's
 * checks run before anything is launched. */
size_t tsfa_tree_attention_workspace_bytes(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len,
                                           int n_masks, int block_m, int block_n, int head_dim, int dtype);
int tsfa_tree_attention(const void* q, const void* k, const void* v, void* o, const uint8_t* mask,
                        int64_t mask_seq_stride, int64_t mask_row_stride, int n_masks,
                        const int64_t* strides, float sm_scale, int batch, int num_heads,
                        int num_kv_heads, int q_len, int kv_len, int block_m, int block_n, int head_dim,
                        int dtype, void* workspace, size_t workspace_bytes, tsfa_stream_t stream);

/* tsfa_fwd without the workspace argument, for callers that cannot allocate
 * device memory (code under graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference.  The split-KV
 * partials go to a library-owned device array of TSFA_FWD_NOALLOC_MAX_BYTES,
 * one per GPU, held until the process ends; its address is taken once per
 * device (hipGetSymbolAddress) and the call allocates nothing.  Calls whose
 * tsfa_fwd_workspace_bytes exceed the array return TSFA_ERR_WORKSPACE before
 * launching.  All calls on one GPU share the array: calls that overlap in
 * time on one GPU (other streams, other host threads) race on it. */
#define TSFA_FWD_NOALLOC_MAX_BYTES ((size_t)64 << 20)
int tsfa_fwd_noalloc(const void* q, const void* k, const void* v, void* o,
                     const int32_t* row_ptr, const int32_t* col_idx, const int8_t* blk_type,
                     const int32_t* mixed_mask_payload, const int32_t* mixed_mask_offset,
                     const int64_t* meta_seq_stride, const int64_t* strides, float sm_scale,
                     int batch, int num_heads, int num_kv_heads, int q_len, int kv_len, int prefix_len,
                     int n_q_blocks, int n_tree_blocks, int gqa_group_size,
                     int block_m, int block_n, int head_dim, int dtype, tsfa_stream_t stream);

/* tsfa_fwd_plan and tsfa_fwd_workspace_bytes for a device of `cus` compute
 * units and `max_lds` bytes of LDS per workgroup instead of the current one
 * (host-only: size a workspace, or test the planner, with no device).
 * out8 = tsfa_fwd_plan's six values, then the partial slots per row chunk
 * and whether the tree units ride on the last prefix run (1) or run as
 * their own work items (0).  `paged` plans tsfa_fwd_paged.  No counterpart in
 * the reference (its grid is fixed, tree_sparse_flashattn.py:358). */
int tsfa_fwd_plan_for_device(int cus, int max_lds, int batch, int num_heads, int num_kv_heads, int q_len,
                             int kv_len, int prefix_len, int head_dim, int paged, int32_t* out8);
size_t tsfa_fwd_workspace_bytes_for_device(int cus, int max_lds, int batch, int num_heads, int num_kv_heads,
                                           int q_len, int kv_len, int prefix_len, int head_dim);

/* The current device's compute-unit count and LDS bytes per workgroup, as
 * the planner reads them: out2[0] = CUs, out2[1] = max LDS per block (the
 * arguments tsfa_fwd_plan_for_device takes to plan this device).  No
 * counterpart in the reference. */
int tsfa_device_limits(int32_t* out2);

/* Re-read the TSFA_* environment switches (read once, at their first use).
 * Not to be called while a forward or backward of this library runs. */
int tsfa_config_reload(void);

/* Work decomposition tsfa_fwd would use (for reports and tests):
 * out[0] = prefix splits per (batch, kv head, row chunk), out[1] = prefix
 * units (32 keys) per split, out[2] = query rows (token x head of a GQA
 * group) per row chunk, out[3] = row chunks per (batch, kv head),
 * out[4] = workgroups of the main kernel, out[5] = LDS ring stages per wave. */
int tsfa_fwd_plan(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len, int prefix_len,
                  int head_dim, int32_t* out6);

/* Measurement hook (no reference counterpart; for benchmarks and profilers):
 * which kernels tsfa_fwd launches on this host thread -- bit 0 the split-KV
 * kernel, bit 1 the combine (3 = both, the default and the only setting that
 * computes O).  A benchmark times each kernel alone this way; any other mask
 * leaves O unwritten or computed from stale partials, so only a process that
 * sets TSFA_BENCH_HOOKS=1 may select one (else TSFA_ERR_UNSUPPORTED; 3 is
 * always accepted).  Invalid: mask outside 1..3. */
int tsfa_fwd_set_kernel_mask(int mask);

#ifdef __cplusplus
}
#endif

#endif /* TSFA_H_ */
