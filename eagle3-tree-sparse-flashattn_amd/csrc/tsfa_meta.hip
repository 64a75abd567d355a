// Tree-sparse metadata builder on the GPU: tiling, ZERO/FULL/MIXED
// classification, CSR construction and row-major int32 bitset packing.
//
// Output is bit-exact with prepare_tree_sparse_metadata
// (tree_sparse_flashattn.py:67-160) applied per sequence:
//   * blocks are visited row-major (q-block, then tree block; :103-108);
//   * a block with no set bit is ZERO and absent (:113-114);
//   * FULL iff every element of the block CLIPPED to q_len is set (:116-124),
//     with a 0 placeholder in the offset array;
//   * otherwise MIXED: the block zero-padded to block_m x block_n is packed
//     with bit i of word w = flat[32w+i], flat = r*block_n + c (:44-64), and
//     its offset is the running payload cursor (:125-134);
//   * row_ptr is the running nnz count (:136).
//
// Two launches per call: `classify` (one workgroup per block and sequence)
// packs words and counts bits; `compact` (one workgroup per sequence) scans
// the block classes and scatters the CSR arrays and MIXED payload.  A tree
// whose packed words fit in LDS (at most kSmallBlocks blocks and
// kSmallWords words) takes one launch instead: `build_small` packs,
// classifies and compacts a sequence in one workgroup, and `build_tree`
// does so for at most 64 blocks (every EAGLE draft tree) with ballots in
// place of the block-wide scan.

#include <stdlib.h>

#include "tsfa_internal.h"

namespace tsfa {

namespace {

constexpr int kMetaThreads = 256;

enum : int8_t { kZero = 0, kFull = 1, kMixed = 2 };

using meta::MetaGeom;  // tsfa_plan.h
using meta::meta_geom;

constexpr int kSmallBlocks = 256;
constexpr int kSmallWords = 8192;  // 32 KB of packed words in LDS
constexpr int kTreeBlocks = 64;    // one wave's lanes

// Nonzero bytes of x (4 mask bytes, first byte lowest) as bits 0-3: the
// high bit of each byte of (x & 0x7f7f7f7f) + 0x7f7f7f7f | x is set iff the
// byte is nonzero; the multiply moves bits 7, 15, 23, 31 to 28..31 (its other
// partial products land on distinct positions below 28, so no carry reaches
// them).
__device__ inline uint32_t nonzero_nibble(uint32_t x) {
  const uint32_t t = ((((x & 0x7f7f7f7fu) + 0x7f7f7f7fu) | x) & 0x80808080u);
  return (t * 0x00204081u) >> 28;
}

// Bits [32*wi, 32*wi + 32) of block (qb, tb) of the sequence whose mask
// starts at m0, zero-padded past the block's clipped h x w extent (:44-64).
// When the 32 bits are one run of a block row inside the clipped block, the
// 32 mask bytes come in two 16-byte loads (aligned) or 32 independent byte
// loads; otherwise every byte load is issued before any is used (addresses
// clamped to the block's first byte where the bit is padding), so a word
// costs one memory latency.
// (r0, c0): row and column of the word's first bit, flat = 32 * wi.
__device__ inline uint32_t block_word_at(const uint8_t* m0, int64_t row_stride, const MetaGeom& g, int qb, int tb,
                                         int64_t flat, int r0, int c0) {
  const int q0 = qb * g.block_m, k0 = tb * g.block_n;
  const int h = min(g.block_m, g.q_len - q0);
  const int w = min(g.block_n, g.q_len - k0);
  const uint8_t* m = m0 + (int64_t)q0 * row_stride + k0;
  const int64_t n_flat = (int64_t)g.block_m * g.block_n;
  if (r0 < h && c0 + 32 <= w && flat + 32 <= n_flat) {
    const uint8_t* p = m + (int64_t)r0 * row_stride + c0;
    if ((reinterpret_cast<uintptr_t>(p) & 15) == 0) {
      const uint4 a = *reinterpret_cast<const uint4*>(p);
      const uint4 b = *reinterpret_cast<const uint4*>(p + 16);
      return nonzero_nibble(a.x) | nonzero_nibble(a.y) << 4 | nonzero_nibble(a.z) << 8 |
             nonzero_nibble(a.w) << 12 | nonzero_nibble(b.x) << 16 | nonzero_nibble(b.y) << 20 |
             nonzero_nibble(b.z) << 24 | nonzero_nibble(b.w) << 28;
    }
    uint8_t v[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = p[i];
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) word |= (uint32_t)(v[i] != 0) << i;
    return word;
  }
  uint8_t v[32];
  bool in[32];
  int r = r0, c = c0;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    in[i] = flat + i < n_flat && r < h && c < w;
    v[i] = m[in[i] ? (int64_t)r * row_stride + c : 0];
    if (++c == g.block_n) {
      c = 0;
      ++r;
    }
  }
  uint32_t word = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) word |= (uint32_t)(in[i] && v[i] != 0) << i;
  return word;
}

__device__ inline uint32_t block_word(const uint8_t* m0, int64_t row_stride, const MetaGeom& g, int qb, int tb,
                                      int wi) {
  const int64_t flat = (int64_t)wi * 32;
  const int r0 = (int)(flat / g.block_n);
  return block_word_at(m0, row_stride, g, qb, tb, flat, r0, (int)(flat - (int64_t)r0 * g.block_n));
}

// ZERO / FULL / MIXED from the set-bit count of a block (:113-124).
__device__ inline int8_t block_class(const MetaGeom& g, int qb, int tb, int ones) {
  const int h = min(g.block_m, g.q_len - qb * g.block_m);
  const int w = min(g.block_n, g.q_len - tb * g.block_n);
  return ones == 0 ? kZero : (ones == h * w ? kFull : kMixed);
}

__global__ __launch_bounds__(kMetaThreads) void classify_kernel(
    const uint8_t* __restrict__ mask, int64_t seq_stride, int64_t row_stride, MetaGeom g,
    int8_t* __restrict__ cls, int32_t* __restrict__ words) {
  const int blk = blockIdx.x;  // qb * ntb + tb
  const int seq = blockIdx.y;
  const int qb = blk / g.ntb, tb = blk - qb * g.ntb;
  int32_t* out = words + ((int64_t)seq * g.cap + blk) * g.words;

  int ones = 0;
  for (int wi = threadIdx.x; wi < g.words; wi += kMetaThreads) {
    const uint32_t word = block_word(mask + seq * seq_stride, row_stride, g, qb, tb, wi);
    out[wi] = (int32_t)word;
    ones += __popc(word);
  }

  __shared__ int red[kMetaThreads / 64];
  for (int off = 32; off > 0; off >>= 1) ones += __shfl_xor(ones, off);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ones;
  __syncthreads();
  if (threadIdx.x == 0) {
    int total = 0;
    for (int i = 0; i < kMetaThreads / 64; ++i) total += red[i];
    cls[(int64_t)seq * g.cap + blk] = block_class(g, qb, tb, total);
  }
}

// Block-wide exclusive scan of (a, b) pairs; returns the totals.
__device__ inline void scan2(int a, int b, int* ex_a, int* ex_b, int* tot_a, int* tot_b) {
  __shared__ int sa[kMetaThreads], sb[kMetaThreads];
  const int t = threadIdx.x;
  sa[t] = a;
  sb[t] = b;
  __syncthreads();
  for (int off = 1; off < kMetaThreads; off <<= 1) {
    int va = (t >= off) ? sa[t - off] : 0;
    int vb = (t >= off) ? sb[t - off] : 0;
    __syncthreads();
    sa[t] += va;
    sb[t] += vb;
    __syncthreads();
  }
  *ex_a = sa[t] - a;
  *ex_b = sb[t] - b;
  *tot_a = sa[kMetaThreads - 1];
  *tot_b = sb[kMetaThreads - 1];
  __syncthreads();
}

// CSR scatter of sequence seq from its block classes c[], packed words
// wsrc[] and rank scratch sr[] (global memory, or LDS for build_small).
__device__ inline void compact_seq(const MetaGeom& g, int seq, const int8_t* c, const int32_t* wsrc, int32_t* sr,
                                   int32_t* __restrict__ row_ptr, int32_t* __restrict__ col_idx,
                                   int8_t* __restrict__ blk_type, int32_t* __restrict__ payload,
                                   int32_t* __restrict__ offset, int32_t* __restrict__ counts) {
  const int64_t nb = g.cap;
  const int per = (int)((nb + kMetaThreads - 1) / kMetaThreads);
  const int64_t i0 = min((int64_t)threadIdx.x * per, nb);
  const int64_t i1 = min(i0 + per, nb);

  int nz = 0, mx = 0;
  for (int64_t i = i0; i < i1; ++i) {
    nz += c[i] != kZero;
    mx += c[i] == kMixed;
  }
  int nz_base, mx_base, nnz, n_mixed;
  scan2(nz, mx, &nz_base, &mx_base, &nnz, &n_mixed);

  int32_t* rp = row_ptr + (int64_t)seq * (g.nqb + 1);
  int32_t* ci = col_idx + seq * nb;
  int8_t* bt = blk_type + seq * nb;
  int32_t* of = offset + seq * nb;
  for (int64_t i = i0; i < i1; ++i) {
    const int qb = (int)(i / g.ntb), tb = (int)(i - (int64_t)qb * g.ntb);
    if (tb == 0) rp[qb] = nz_base;
    const int8_t k = c[i];
    if (k == kZero) continue;
    ci[nz_base] = tb;
    bt[nz_base] = (k == kFull) ? TSFA_FULL_BLOCK : TSFA_MIXED_BLOCK;
    if (k == kMixed) {
      of[nz_base] = mx_base * g.words;
      sr[mx_base] = (int32_t)i;
      ++mx_base;
    } else {
      of[nz_base] = 0;
    }
    ++nz_base;
  }
  if (threadIdx.x == 0) {
    rp[g.nqb] = nnz;
    counts[2 * seq] = nnz;
    counts[2 * seq + 1] = n_mixed;
  }
  __syncthreads();  // src_of_rank complete (workgroup-scope fence + barrier)

  const int64_t total = (int64_t)n_mixed * g.words;
  int32_t* pl = payload + seq * nb * g.words;
  for (int64_t e = threadIdx.x; e < total; e += kMetaThreads) {
    const int64_t r = e / g.words, wi = e - r * g.words;
    pl[e] = wsrc[(int64_t)sr[r] * g.words + wi];
  }
}

__global__ __launch_bounds__(kMetaThreads) void compact_kernel(
    MetaGeom g, const int8_t* __restrict__ cls, const int32_t* __restrict__ words,
    int32_t* __restrict__ src_of_rank, int32_t* __restrict__ row_ptr, int32_t* __restrict__ col_idx,
    int8_t* __restrict__ blk_type, int32_t* __restrict__ payload, int32_t* __restrict__ offset,
    int32_t* __restrict__ counts) {
  const int seq = blockIdx.x;
  const int64_t nb = g.cap;
  compact_seq(g, seq, cls + seq * nb, words + seq * nb * g.words, src_of_rank + seq * nb, row_ptr, col_idx,
              blk_type, payload, offset, counts);
}

// One workgroup per sequence: packed words and block bit counts in LDS,
// classes, then the same scatter as compact_kernel.
__global__ __launch_bounds__(kMetaThreads) void build_small_kernel(
    const uint8_t* __restrict__ mask, int64_t seq_stride, int64_t row_stride, MetaGeom g,
    int32_t* __restrict__ row_ptr, int32_t* __restrict__ col_idx, int8_t* __restrict__ blk_type,
    int32_t* __restrict__ payload, int32_t* __restrict__ offset, int32_t* __restrict__ counts) {
  __shared__ int32_t s_words[kSmallWords];
  __shared__ int s_ones[kSmallBlocks];
  __shared__ int32_t s_rank[kSmallBlocks];
  __shared__ int8_t s_cls[kSmallBlocks];
  const int seq = blockIdx.x;
  const int nb = (int)g.cap;
  for (int i = threadIdx.x; i < nb; i += kMetaThreads) s_ones[i] = 0;
  __syncthreads();
  const uint8_t* m0 = mask + seq * seq_stride;
  for (int e = threadIdx.x; e < nb * g.words; e += kMetaThreads) {
    const int blk = e / g.words, wi = e - blk * g.words;
    const int qb = blk / g.ntb, tb = blk - qb * g.ntb;
    const uint32_t word = block_word(m0, row_stride, g, qb, tb, wi);
    s_words[e] = (int32_t)word;
    if (word != 0) atomicAdd(&s_ones[blk], __popc(word));
  }
  __syncthreads();
  for (int i = threadIdx.x; i < nb; i += kMetaThreads) {
    const int qb = i / g.ntb;
    s_cls[i] = block_class(g, qb, i - qb * g.ntb, s_ones[i]);
  }
  __syncthreads();
  compact_seq(g, seq, s_cls, s_words, s_rank, row_ptr, col_idx, blk_type, payload, offset, counts);
}

// Arguments of build_tree_kernel, with the divisors its threads use.
struct TreeArgs {
  const uint8_t* mask;
  int64_t seq_stride, row_stride;
  MetaGeom g;
  FastDiv fd_words, fd_ntb, fd_block_n;
  int32_t* row_ptr;
  int32_t* col_idx;
  int8_t* blk_type;
  int32_t* payload;
  int32_t* offset;
  int32_t* counts;
};

__device__ inline void sync_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// One workgroup per sequence of at most kTreeBlocks blocks (an EAGLE draft
// tree): packed words and block bit counts in LDS; then every wave
// classifies the blocks, lane i block i, and ranks the present and the MIXED
// blocks by ballot and popcount of the lanes below, so each thread places
// the packed words it owns from the ballot alone -- no block-wide scan, two
// barriers in all.
__global__ __launch_bounds__(kMetaThreads) void build_tree_kernel(TreeArgs a) {
  __shared__ int32_t s_words[kSmallWords];
  __shared__ int s_ones[kTreeBlocks];
  const MetaGeom& g = a.g;
  const int seq = blockIdx.x;
  const int nb = (int)g.cap, n_words = nb * g.words;
  if (threadIdx.x < kTreeBlocks) s_ones[threadIdx.x] = 0;
  sync_lds();
  const uint8_t* m0 = a.mask + seq * a.seq_stride;
  for (int e = threadIdx.x; e < n_words; e += kMetaThreads) {
    const int blk = (int)fdiv(e, a.fd_words), wi = e - blk * g.words;
    const int qb = (int)fdiv(blk, a.fd_ntb), tb = blk - qb * g.ntb;
    const int flat = wi * 32, r0 = (int)fdiv(flat, a.fd_block_n);
    const uint32_t word = block_word_at(m0, a.row_stride, g, qb, tb, flat, r0, flat - r0 * g.block_n);
    s_words[e] = (int32_t)word;
    if (word != 0) atomicAdd(&s_ones[blk], __popc(word));
  }
  sync_lds();
  const int lane = threadIdx.x & 63;
  const int qb = (int)fdiv(lane, a.fd_ntb), tb = lane - qb * g.ntb;
  const int8_t c = lane < nb ? block_class(g, qb, tb, s_ones[lane]) : kZero;
  const uint64_t nz = __ballot(c != kZero), mx = __ballot(c == kMixed);
  if (threadIdx.x < 64) {
    const int nz_below = __builtin_amdgcn_mbcnt_hi((uint32_t)(nz >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)nz, 0));
    const int mx_below = __builtin_amdgcn_mbcnt_hi((uint32_t)(mx >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mx, 0));
    int32_t* rp = a.row_ptr + (int64_t)seq * (g.nqb + 1);
    if (lane < nb && tb == 0) rp[qb] = nz_below;  // present blocks before row qb
    if (c != kZero) {
      a.col_idx[(int64_t)seq * nb + nz_below] = tb;
      a.blk_type[(int64_t)seq * nb + nz_below] = (c == kFull) ? TSFA_FULL_BLOCK : TSFA_MIXED_BLOCK;
      a.offset[(int64_t)seq * nb + nz_below] = (c == kMixed) ? mx_below * g.words : 0;
    }
    if (lane == 0) {
      rp[g.nqb] = __popcll(nz);
      a.counts[2 * seq] = __popcll(nz);
      a.counts[2 * seq + 1] = __popcll(mx);
    }
  }
  int32_t* pl = a.payload + (int64_t)seq * nb * g.words;
  for (int e = threadIdx.x; e < n_words; e += kMetaThreads) {
    const int blk = (int)fdiv(e, a.fd_words);
    if ((mx >> blk) & 1) {
      const int rank = __popcll(mx & ((1ull << blk) - 1));  // MIXED blocks before blk
      pl[rank * g.words + (e - blk * g.words)] = s_words[e];
    }
  }
}

__global__ void pack_bits_kernel(const uint8_t* __restrict__ bits, int64_t n_bits, int32_t* __restrict__ words,
                                 int64_t n_words) {
  const int64_t wi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (wi >= n_words) return;
  uint32_t word = 0;
  for (int i = 0; i < 32; ++i) {
    const int64_t f = wi * 32 + i;
    if (f < n_bits && bits[f] != 0) word |= 1u << i;
  }
  words[wi] = (int32_t)word;
}

}  // namespace
}  // namespace tsfa

using namespace tsfa;

extern "C" int tsfa_meta_build(const uint8_t* mask, int64_t mask_seq_stride, int64_t mask_row_stride,
                               int n_seq, int q_len, int block_m, int block_n, int32_t* row_ptr,
                               int32_t* col_idx, int8_t* blk_type, int32_t* payload, int32_t* offset,
                               int32_t* counts, void* workspace, size_t workspace_bytes,
                               tsfa_stream_t stream_) {
  int st = tsfa_meta_check_args(n_seq, q_len, block_m, block_n);
  if (st != TSFA_OK) return st;
  if (n_seq == 0) return TSFA_OK;
  if (row_ptr == nullptr || counts == nullptr) return TSFA_ERR_INVALID_ARGUMENT;
  MetaGeom g;
  meta_geom(q_len, block_m, block_n, &g);
  const size_t need = tsfa_meta_workspace_bytes(n_seq, q_len, block_m, block_n);
  if (g.cap > 0 && (workspace == nullptr || workspace_bytes < need)) return TSFA_ERR_WORKSPACE;
  if (g.cap > 0 && (mask == nullptr || col_idx == nullptr || blk_type == nullptr || payload == nullptr ||
                    offset == nullptr))
    return TSFA_ERR_INVALID_ARGUMENT;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  const size_t nb = (size_t)n_seq * g.cap;
  int8_t* cls = static_cast<int8_t*>(workspace);
  int32_t* words = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + align256(nb));
  int32_t* src_of_rank =
      reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + align256(nb) + align256(nb * g.words * 4));
  const bool small = g.cap > 0 && g.cap <= kSmallBlocks && g.cap * g.words <= kSmallWords &&
                     config().meta_small != 0;  // TSFA_META_SMALL=0: always two launches
  if (small && g.cap <= kTreeBlocks) {
    TreeArgs ta;
    ta.mask = mask;
    ta.seq_stride = mask_seq_stride;
    ta.row_stride = mask_row_stride;
    ta.g = g;
    ta.fd_words = make_fastdiv((uint32_t)g.words);
    ta.fd_ntb = make_fastdiv((uint32_t)g.ntb);
    ta.fd_block_n = make_fastdiv((uint32_t)g.block_n);
    ta.row_ptr = row_ptr;
    ta.col_idx = col_idx;
    ta.blk_type = blk_type;
    ta.payload = payload;
    ta.offset = offset;
    ta.counts = counts;
    hipLaunchKernelGGL(build_tree_kernel, dim3((unsigned)n_seq), dim3(kMetaThreads), 0, stream, ta);
    return hipGetLastError() == hipSuccess ? TSFA_OK : TSFA_ERR_LAUNCH;
  }
  if (small) {
    hipLaunchKernelGGL(build_small_kernel, dim3((unsigned)n_seq), dim3(kMetaThreads), 0, stream, mask,
                       mask_seq_stride, mask_row_stride, g, row_ptr, col_idx, blk_type, payload, offset, counts);
    return hipGetLastError() == hipSuccess ? TSFA_OK : TSFA_ERR_LAUNCH;
  }
  if (g.cap > 0) {
    if (g.cap > INT32_MAX) return TSFA_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(classify_kernel, dim3((unsigned)g.cap, (unsigned)n_seq), dim3(kMetaThreads), 0, stream,
                       mask, mask_seq_stride, mask_row_stride, g, cls, words);
    if (hipGetLastError() != hipSuccess) return TSFA_ERR_LAUNCH;
  }
  hipLaunchKernelGGL(compact_kernel, dim3((unsigned)n_seq), dim3(kMetaThreads), 0, stream, g, cls, words,
                     src_of_rank, row_ptr, col_idx, blk_type, payload, offset, counts);
  if (hipGetLastError() != hipSuccess) return TSFA_ERR_LAUNCH;
  return TSFA_OK;
}

extern "C" int tsfa_pack_bits(const uint8_t* bits, int64_t n_bits, int32_t* words, tsfa_stream_t stream_) {
  if (n_bits < 0) return TSFA_ERR_INVALID_ARGUMENT;
  const int64_t n_words = (n_bits + 31) / 32;
  if (n_words == 0) return TSFA_OK;
  if (bits == nullptr || words == nullptr) return TSFA_ERR_INVALID_ARGUMENT;
  if (n_words > ((int64_t)1 << 31)) return TSFA_ERR_UNSUPPORTED;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  const unsigned grid = (unsigned)((n_words + 255) / 256);
  hipLaunchKernelGGL(pack_bits_kernel, dim3(grid), dim3(256), 0, stream, bits, n_bits, words, n_words);
  return hipGetLastError() == hipSuccess ? TSFA_OK : TSFA_ERR_LAUNCH;
}
