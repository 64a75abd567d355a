// Host-side planning and validation of libtsfa, shared by the HIP sources
// (their launch code) and tsfa_plan.cpp, which holds the implementations and
// builds with a plain C++ compiler (no HIP headers): the planners, argument
// validators and workspace sizing can then be built and tested on their own,
// under sanitizers, on a host without a GPU.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "../../include/tsfa.h"

#ifdef __HIPCC__
#define TSFA_HD __host__ __device__
#else
#define TSFA_HD
#endif

namespace tsfa {

// ceil(a / b) for b > 0 without the overflow of (a + b - 1) / b near INT32_MAX
inline int ceil_div(int a, int b) { return a / b + (a % b > 0 ? 1 : 0); }
inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Division by a runtime-invariant divisor d >= 1 for dividends 0 <= n < 2^31:
// n / d == (umulhi(n, m) + n) >> s with s = ceil(log2 d) and
// m = floor(2^32 (2^s - d) / d) + 1 (Granlund and Montgomery, "Division by
// invariant integers using multiplication", 1994, Fig. 4.1; the sum cannot
// wrap because umulhi(n, m) <= n < 2^31).  A kernel's per-wave scalar
// divisions cost ~35 instructions each, on the scalar unit the CU's waves share.
struct FastDiv {
  uint32_t m, s, d;
};
FastDiv make_fastdiv(uint32_t d);  // d >= 1
TSFA_HD inline uint32_t fdiv(uint32_t n, const FastDiv& f) {
  return (uint32_t)((((uint64_t)n * f.m) >> 32) + n) >> f.s;
}
TSFA_HD inline uint32_t frem(uint32_t n, const FastDiv& f) { return n - fdiv(n, f) * f.d; }

// The TSFA_* environment switches, read once at first use (tsfa_config_reload
// reads them again).  -1 / 0 mean "the planner decides" where noted.  Apart
// from TSFA_BENCH_HOOKS they select among kernels and plans the planner picks
// for other shapes anyway, so tests can run each one on any shape.
struct Config {
  int streams;         // TSFA_STREAMS: 1 or 2 key streams, 0 planner
  int prefix_units;    // TSFA_PREFIX_UNITS_PER_SPLIT: > 0 forces the run length
  int fold_tree;       // TSFA_FOLD_TREE: 0/1 forces, -1 planner
  int fast_ring;       // TSFA_FAST_RING: 0 keeps the checked ring steps for full prefix runs
  int direct_out;      // TSFA_DIRECT_OUT: 0 keeps the combine for one-slot plans
  int kv_nt;           // TSFA_KV_NT: 0/1 forces non-temporal K/V loads, -1 planner
  int item_order;      // TSFA_ITEM_ORDER: 0/1/2 forces, -1 planner
  int paged32;         // TSFA_PAGED32: 0 keeps the 64-bit-offset paged kernel
  int meta_small;      // TSFA_META_SMALL: 0 always two metadata launches
  int bwd_concurrent;  // TSFA_BWD_CONCURRENT: 0 keeps the backward on one stream
  int bench_hooks;     // TSFA_BENCH_HOOKS: 1 unlocks tsfa_fwd_set_kernel_mask
  int generation;      // bumped by every reload (keys of memoised plans)
};
// A copy of the switches, taken under the lock that config_reload holds, so
// a call that snapshots them once sees one consistent set even while another
// thread reloads them.
Config config();
void config_reload();

namespace fwd {

constexpr int kWaves = 8;                  // 32 query rows each
constexpr int kMaxRows = 32 * kWaves;      // rows per chunk with one key stream
constexpr int kUnitKeys = 32;
constexpr int kRingBytes = 131072;   // K/V rings of the streams; the merge buffer at the end
constexpr int kMaskWords = 4096;     // per-token 32-bit visibility words of tree units
constexpr int kMaxTreeUnits = 1024;  // tree keys <= 32768
constexpr int kMiscInts = 320;       // LDS scalars: visible-unit count, row_ptr window
// dynamic LDS of the split kernel: ring, mask words, visible-unit list, scalars
constexpr size_t kSplitLdsBytes = (size_t)kRingBytes + kMaskWords * 4 + (kMaxTreeUnits + kMiscInts) * 4;
// paged: the clamped page ids of a prefix run in LDS (plans whose runs span
// more pages read the page table unit by unit)
constexpr int kPageTabInts = 2048;
constexpr size_t kPagedLdsBytes = kSplitLdsBytes + (size_t)kPageTabInts * 4;

// Tokens a chunk of `rows` consecutive rows can touch, and q-blocks those span.
inline int64_t chunk_tokens(int rows, int group) { return (int64_t)(rows - 1) / group + 2; }
inline int64_t chunk_qblocks(int rows, int group, int block_m) {
  return (chunk_tokens(rows, group) - 1) / block_m + 2;
}

struct Plan {
  int streams, rows_per_chunk;
  int n_chunks, n_pu, units_per_split, n_splits, n_slots, n_items, items_per_xcd, grid, ring_stages, fold_tree;
  int vt_max, tree_key_limit;
  size_t lds_bytes, ws_acc_bytes, ws_ml_bytes;
};

// The forward's work decomposition on a device of `cus` compute units and
// `max_lds` bytes of LDS per workgroup.
int make_plan(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len, int prefix_len, int head_dim,
              bool paged, int cus, int max_lds, const Config& cfg, Plan* p);
// Workspace of both the contiguous and the paged plan of a shape (0: invalid).
size_t workspace_bytes(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len, int prefix_len,
                       int head_dim, int cus, int max_lds);

int check_args(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len, int prefix_len, int n_q_blocks,
               int n_tree_blocks, int gqa_group_size, int block_m, int block_n, int head_dim, int dtype);

// Layout checks of one call (contiguous head_dim, 16-byte aligned rows and
// bases, 32-bit lane offsets): TSFA_OK, TSFA_ERR_UNSUPPORTED or
// TSFA_ERR_INVALID_ARGUMENT.  `kv` strides for K and V, or (paged) the
// cache strides [page, slot, row, head, d].
int check_strides(const void* q, const int64_t* q_strides, const void* o, const int64_t* o_strides);
int check_kv_strides(const void* k, const int64_t* k_strides, const void* v, const int64_t* v_strides);
int check_paged(int batch, int kv_len, const void* cache, const int64_t* cache_strides, const int32_t* kv_indptr,
                int64_t pt_stride, int64_t n_indices, int n_pages, int page_size);

// Whether every byte offset the 32-bit-offset paged kernel forms from a kv
// head's base -- page * page_stride + row * row_stride + a row's bytes, all
// in bytes -- stays below 2^32 (strides in elements of 2 bytes).
bool paged_offsets_fit_32(int n_pages, int64_t page_stride, int64_t row_stride, int page_size, int head_dim);

}  // namespace fwd

namespace bwd {

constexpr int kBlockKeys = 128;      // keys per workgroup (32 per key group)
constexpr int kTileRows = 32;        // query rows per tile
constexpr int kMaxStateInts = 8192;  // block-state table of one tile (visibility words)

struct BwdPlan {
  int n_tiles, n_pb, n_tb, n_tkeys, n_trees, nqbc_max;
  size_t rowstat_bytes, dq_bytes, vis_bytes;
};

int make_bwd_plan(int batch, int num_kv_heads, int q_len, int kv_len, int prefix_len, int gqa, int head_dim,
                  int block_m, int n_tree_blocks, int n_trees, BwdPlan* p);

}  // namespace bwd

namespace meta {

struct MetaGeom {
  int q_len, block_m, block_n, nqb, ntb, words;  // words = W per block
  int64_t cap;                                   // nqb * ntb
};

bool meta_geom(int q_len, int block_m, int block_n, MetaGeom* g);

}  // namespace meta

}  // namespace tsfa
