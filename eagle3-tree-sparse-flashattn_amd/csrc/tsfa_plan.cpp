// Host-only part of libtsfa (plain C++, no HIP headers): status strings, the
// environment switches, the forward / backward / metadata planners, argument
// validation, workspace sizing, and the CPU builder of the tree metadata.
// Built into libtsfa.so beside the HIP sources, and on its own with
// -fsanitize=address,undefined by the host sanitizer test.

#include "tsfa_plan.h"

#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>

namespace tsfa {

FastDiv make_fastdiv(uint32_t d) {
  if (d == 0) d = 1;
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;
  const uint64_t m = ((1ull << 32) * ((1ull << s) - d)) / d + 1;
  return FastDiv{(uint32_t)m, s, d};
}

// ------------------------------------------------------------------ config
namespace {

int env_int(const char* name, int dflt) {
  const char* s = getenv(name);
  if (s == nullptr || *s == 0) return dflt;
  return atoi(s);
}

Config read_config() {
  Config c;
  c.streams = env_int("TSFA_STREAMS", 0);
  c.prefix_units = env_int("TSFA_PREFIX_UNITS_PER_SPLIT", 0);
  c.fold_tree = env_int("TSFA_FOLD_TREE", -1);
  c.fast_ring = env_int("TSFA_FAST_RING", 1);
  c.direct_out = env_int("TSFA_DIRECT_OUT", 1);
  c.kv_nt = env_int("TSFA_KV_NT", -1);
  c.item_order = env_int("TSFA_ITEM_ORDER", -1);
  c.paged32 = env_int("TSFA_PAGED32", 1);
  c.meta_small = env_int("TSFA_META_SMALL", 1);
  c.bwd_concurrent = env_int("TSFA_BWD_CONCURRENT", 1);
  c.bench_hooks = env_int("TSFA_BENCH_HOOKS", 0);
  c.generation = 0;
  return c;
}

std::mutex g_config_mu;
bool g_config_loaded = false;  // guarded by g_config_mu
Config g_config;

}  // namespace

Config config() {
  std::lock_guard<std::mutex> lock(g_config_mu);
  if (!g_config_loaded) {
    g_config = read_config();
    g_config_loaded = true;
  }
  return g_config;
}

void config_reload() {
  std::lock_guard<std::mutex> lock(g_config_mu);
  const int gen = g_config.generation + 1;
  g_config = read_config();
  g_config.generation = gen;
  g_config_loaded = true;
}

// -------------------------------------------------------------- forward plan
namespace fwd {

// Kernel, key streams per workgroup, prefix run length (units per split) and
// the grid.  Runs are chosen by the makespan model below, which counts the
// short tree items apart from the prefix runs: one round of 256-unit runs
// with the tree folded in beats 5 splits of 103 on the 1024-token wide tree
// (338 -> 306 us per call), one 1024-unit run beats 8 of 128 on the 70B
// shape (1243 -> 1180 us), one 64-unit run beats 2 of 32 on the 16-sequence
// decode shape (71 -> 66 us; same-box A/B).  Key streams: two, with
// 128-row chunks, below 1024 rows per (batch, kv head); one, with 256-row
// chunks, from 1024 rows on (TSFA_STREAMS=1/2 forces one or two).  One stream
// loads each K/V unit once for 256 rows, halving the loads per MFMA and
// leaving six units in flight instead of two per stream (the 1024-token wide
// tree 391 -> 377 us per call); two streams fill the grid where rows are few
// (the 8B decode shape: 22.9 -> 19.3 us; 16 sequences: 75.1 -> 70.3 us).
int make_plan(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len, int prefix_len, int head_dim,
              bool paged, int cus, int max_lds, const Config& cfg, Plan* p) {
  (void)paged;
  if (batch <= 0 || q_len <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 ||
      prefix_len < 0 || kv_len < prefix_len || (head_dim != 64 && head_dim != 128) || cus <= 0)
    return TSFA_ERR_INVALID_ARGUMENT;
  const int G = num_heads / num_kv_heads;
  const int64_t TG = (int64_t)q_len * G;
  if (TG > INT32_MAX / 2) return TSFA_ERR_UNSUPPORTED;
  p->streams = cfg.streams == 1 || (cfg.streams != 2 && TG >= 1024) ? 1 : 2;
  p->rows_per_chunk = kMaxRows / p->streams;
  p->n_chunks = (int)((TG + p->rows_per_chunk - 1) / p->rows_per_chunk);
  p->n_pu = ceil_div(prefix_len, kUnitKeys);
  const int64_t groups = (int64_t)batch * num_kv_heads * p->n_chunks;
  int ups = 0;
  if (p->n_pu > 0) {
    ups = cfg.prefix_units;
    if (ups <= 0) {
      // Makespan model (microseconds, measured on MI355X): one workgroup per
      // CU, dispatched as CUs free up; a workgroup costs a fixed start/finish
      // plus one step per unit of its stream (a step is the same MFMA work
      // with one or two streams); every slot of partials is written once and
      // read once by the combine.  The prefix runs go out first: after their
      // full rounds, the last partial round of runs and the (shorter) tree
      // items share the CUs.  A tree item runs only its visible units,
      // estimated as 60 % of the tree's.
      const double t_step = 1.15 * head_dim / 128.0, t_fixed = 5.0;
      const double part_bytes = (double)batch * num_heads * q_len * (2.0 * head_dim + 8.0);
      const int64_t tree_units = ceil_div(std::max(0, kv_len - prefix_len), kUnitKeys);
      const double c_tree =
          t_fixed + 0.6 * (double)ceil_div((int)std::min<int64_t>(tree_units, INT32_MAX), p->streams) * t_step;
      double best = 1e300;
      for (int cand = 1; cand <= p->n_pu; ++cand) {
        const int64_t splits = ceil_div(p->n_pu, cand);
        if (cand > 1 && ceil_div(p->n_pu, cand - 1) == splits) continue;
        const double c_run = t_fixed + ceil_div(cand, p->streams) * t_step;
        const int64_t runs = groups * splits, full = runs / cus, rest = runs % cus;
        const double tail = rest > 0 ? std::max(c_run, (double)((groups + cus - rest - 1) / (cus - rest)) * c_tree)
                                     : (double)((groups + cus - 1) / cus) * c_tree;
        const double cost = (double)full * c_run + tail + part_bytes * (double)(splits + 1) * 2.0 / 5.0e6;
        if (cost < best * (1.0 - 1e-9)) {
          best = cost;
          ups = cand;
        }
      }
      // Within one round, a plan with the same steps per stream that keeps
      // more CUs busy is faster despite its extra partials (measured on the
      // Llama-3-8B shape: 256 workgroups of 9 units beat 224 of 10 by ~1 %).
      if (ups > 0 && groups * (ceil_div(p->n_pu, ups) + 1) <= cus) {
        const int steps = ceil_div(ups, p->streams);
        for (int cand = ups - 1; cand >= 1 && ceil_div(cand, p->streams) == steps; --cand)
          if (groups * (ceil_div(p->n_pu, cand) + 1) <= cus) ups = cand;
      }
    }
    ups = std::min(std::max(ups, 1), p->n_pu);
  }
  p->units_per_split = ups;
  p->n_splits = ups > 0 ? ceil_div(p->n_pu, ups) : 0;
  // A separate tree item per chunk costs a round when it does not fit beside
  // the prefix runs; on a plan of at most 4 rounds, if the tree is short next
  // to a run (at most a quarter of its units, or 2), the last run of each
  // chunk takes the tree units too (the 16-sequence decode shape: 3 rounds ->
  // 2, 73.6 -> 66.0 us per call; on the 70B shape, 16 rounds -> 15, folding
  // measured 0.6 % slower).  TSFA_FOLD_TREE=0/1 forces it off/on (on only
  // where there is a prefix run).
  p->fold_tree = 0;
  if (p->n_splits >= 1) {
    const int64_t tree_units = ceil_div(std::max(0, kv_len - prefix_len), kUnitKeys);
    const int64_t rounds_sep = (groups * (p->n_splits + 1) + cus - 1) / cus;
    const int64_t rounds_fold = (groups * p->n_splits + cus - 1) / cus;
    p->fold_tree = cfg.fold_tree >= 0 ? (cfg.fold_tree != 0)
                                      : (rounds_fold < rounds_sep && rounds_sep <= 4 &&
                                                 tree_units <= std::max(2, ups / 4)
                                             ? 1
                                             : 0);
  }
  // A folded tree lengthens the last run of each chunk: the earlier runs of
  // a plan of several splits take the modelled tree cost off it, spread over
  // the splits, while the split count stays (the 1024-token wide tree: 256
  // -> 266 units per split, 270 -> 266-268 us per call in one sweep, within
  // noise of it in a later A/B).
  if (p->fold_tree && p->n_splits >= 2 && cfg.prefix_units <= 0) {
    const int64_t tree_units = ceil_div(std::max(0, kv_len - prefix_len), kUnitKeys);
    const int extra = (int)std::min<int64_t>((int64_t)(0.6 * (double)tree_units / p->streams), p->n_pu);
    const int ups2 = ceil_div(p->n_pu + extra, p->n_splits);
    if (ups2 > ups && ceil_div(p->n_pu, ups2) == p->n_splits) {
      ups = ups2;
      p->units_per_split = ups;
    }
  }
  p->n_slots = p->n_splits + (p->fold_tree ? 0 : 1);
  const int64_t items = groups * p->n_slots;
  if (items > (int64_t)INT32_MAX / 2) return TSFA_ERR_UNSUPPORTED;
  p->n_items = (int)items;
  p->items_per_xcd = ceil_div(p->n_items, 8);
  p->grid = p->items_per_xcd * 8;
  p->lds_bytes = kSplitLdsBytes;  // (the paged page-id table's instances ask for kPagedLdsBytes at launch)
  if (p->lds_bytes > (size_t)max_lds) return TSFA_ERR_UNSUPPORTED;
  p->ring_stages = kRingBytes / p->streams / (2 * kUnitKeys * head_dim * 2);
  p->vt_max = (int)(kMaskWords / chunk_tokens(p->rows_per_chunk, G));
  p->tree_key_limit = kv_len - prefix_len;  // refined by the caller with n_tree_blocks*BN
  const size_t rows = (size_t)batch * num_heads * q_len;
  p->ws_acc_bytes = align256(rows * p->n_slots * head_dim * 2);
  p->ws_ml_bytes = align256(rows * p->n_slots * 8);
  return TSFA_OK;
}

size_t workspace_bytes(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len, int prefix_len,
                       int head_dim, int cus, int max_lds) {
  if (batch <= 0 || q_len <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0) return 0;
  Plan p, pp;
  const Config& cfg = config();
  if (make_plan(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, head_dim, false, cus, max_lds, cfg,
                &p) != TSFA_OK ||
      make_plan(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, head_dim, true, cus, max_lds, cfg,
                &pp) != TSFA_OK)
    return 0;
  return std::max(p.ws_acc_bytes + p.ws_ml_bytes, pp.ws_acc_bytes + pp.ws_ml_bytes);
}

int check_args(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len, int prefix_len, int n_q_blocks,
               int n_tree_blocks, int gqa_group_size, int block_m, int block_n, int head_dim, int dtype) {
  if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || q_len < 0) return TSFA_ERR_INVALID_ARGUMENT;
  if (block_m <= 0 || block_n <= 0) return TSFA_ERR_INVALID_ARGUMENT;          // tree_sparse_flashattn.py:87-88
  if (prefix_len < 0 || kv_len < prefix_len) return TSFA_ERR_INVALID_ARGUMENT;  // eagle_tree_sparse_bridge.py:91-93
  if (gqa_group_size <= 0 || (int64_t)num_heads != (int64_t)gqa_group_size * num_kv_heads)
    return TSFA_ERR_INVALID_ARGUMENT;
  if ((int64_t)n_q_blocks != ((int64_t)q_len + block_m - 1) / block_m ||
      (int64_t)n_tree_blocks != ((int64_t)q_len + block_n - 1) / block_n)
    return TSFA_ERR_INVALID_ARGUMENT;
  if (dtype != TSFA_DTYPE_FP16 && dtype != TSFA_DTYPE_BF16 && dtype != TSFA_DTYPE_FP32) return TSFA_ERR_UNSUPPORTED;
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return TSFA_ERR_UNSUPPORTED;
  if (block_n % 16 != 0) return TSFA_ERR_UNSUPPORTED;
  const int64_t tree_limit = std::min<int64_t>((int64_t)n_tree_blocks * block_n, (int64_t)kv_len - prefix_len);
  if (tree_limit > (int64_t)kMaxTreeUnits * kUnitKeys) return TSFA_ERR_UNSUPPORTED;
  // the tree block-state table [q-blocks of a chunk][n_tree_blocks] lives in
  // the LDS ring and the chunk's row_ptr window in the LDS scalars
  const int64_t nqbc = chunk_qblocks(kMaxRows, gqa_group_size, block_m);
  if (nqbc * n_tree_blocks * 4 > (int64_t)kRingBytes || nqbc + 1 > kMiscInts - 8) return TSFA_ERR_UNSUPPORTED;
  return TSFA_OK;
}

namespace {
// contiguous head_dim, 16-byte aligned rows
bool rows_ok(const int64_t* sd, int n) {
  if (sd[n - 1] != 1) return false;
  for (int j = 0; j < n - 1; ++j)
    if (sd[j] % 8 != 0) return false;
  return true;
}
bool aligned16(const void* ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; }
}  // namespace

int check_strides(const void* q, const int64_t* q_strides, const void* o, const int64_t* o_strides) {
  if (q_strides == nullptr || o_strides == nullptr) return TSFA_ERR_INVALID_ARGUMENT;
  if (!rows_ok(q_strides, 4) || !rows_ok(o_strides, 4) || !aligned16(q) || !aligned16(o))
    return TSFA_ERR_UNSUPPORTED;
  return TSFA_OK;
}

int check_kv_strides(const void* k, const int64_t* k_strides, const void* v, const int64_t* v_strides) {
  if (k == nullptr || v == nullptr || k_strides == nullptr || v_strides == nullptr) return TSFA_ERR_INVALID_ARGUMENT;
  if (!rows_ok(k_strides, 4) || !rows_ok(v_strides, 4) || !aligned16(k) || !aligned16(v))
    return TSFA_ERR_UNSUPPORTED;
  // K/V row strides must keep a 32-bit lane offset of 8 rows
  if (k_strides[2] >= ((int64_t)1 << 26) || v_strides[2] >= ((int64_t)1 << 26)) return TSFA_ERR_UNSUPPORTED;
  return TSFA_OK;
}

int check_paged(int batch, int kv_len, const void* cache, const int64_t* cache_strides, const int32_t* kv_indptr,
                int64_t pt_stride, int64_t n_indices, int n_pages, int page_size) {
  if (cache == nullptr || cache_strides == nullptr) return TSFA_ERR_INVALID_ARGUMENT;
  if (!rows_ok(cache_strides, 5) || !aligned16(cache)) return TSFA_ERR_UNSUPPORTED;
  if (cache_strides[2] >= ((int64_t)1 << 26)) return TSFA_ERR_UNSUPPORTED;  // 32-bit lane offsets
  // pages of 16 keys or more, a power of two: a wave's 16-key DMA share
  // then spans at most two pages
  if (page_size < 16 || (page_size & (page_size - 1)) != 0) return TSFA_ERR_UNSUPPORTED;
  if (pt_stride < 0 || n_indices > INT32_MAX || pt_stride > INT32_MAX ||
      (kv_len > 0 && (n_pages <= 0 || n_indices <= 0)))
    return TSFA_ERR_INVALID_ARGUMENT;
  // a dense page table holds every sequence's ceil(kv_len / page_size) pages
  if (kv_indptr == nullptr && kv_len > 0 &&
      (int64_t)(batch - 1) * pt_stride + ceil_div(kv_len, page_size) > n_indices)
    return TSFA_ERR_INVALID_ARGUMENT;
  return TSFA_OK;
}

bool paged_offsets_fit_32(int n_pages, int64_t page_stride, int64_t row_stride, int page_size, int head_dim) {
  if (n_pages <= 0 || page_stride < 0 || row_stride < 0 || page_size <= 0 || head_dim <= 0) return false;
  // the largest offset one load forms: last page, last row, end of the row
  const unsigned __int128 top = (unsigned __int128)(n_pages - 1) * (uint64_t)page_stride * 2 +
                                (unsigned __int128)(page_size - 1) * (uint64_t)row_stride * 2 +
                                (unsigned __int128)head_dim * 2;
  return top < ((unsigned __int128)1 << 32);
}

}  // namespace fwd

// ------------------------------------------------------------- backward plan
namespace bwd {

int make_bwd_plan(int batch, int num_kv_heads, int q_len, int kv_len, int prefix_len, int gqa, int head_dim,
                  int block_m, int n_tree_blocks, int n_trees, BwdPlan* p) {
  if (batch <= 0 || num_kv_heads <= 0 || q_len <= 0 || gqa <= 0 || block_m <= 0 || n_tree_blocks < 0 ||
      n_trees <= 0 || prefix_len < 0 || kv_len < prefix_len || head_dim <= 0)
    return TSFA_ERR_INVALID_ARGUMENT;
  const int64_t TG = (int64_t)q_len * gqa;
  if (TG >= ((int64_t)1 << 22)) return TSFA_ERR_UNSUPPORTED;  // the kernel's row -> token division is exact below
  p->n_tiles = (int)((TG + kTileRows - 1) / kTileRows);
  p->n_pb = ceil_div(prefix_len, kBlockKeys);
  p->n_tb = ceil_div(kv_len - prefix_len, kBlockKeys);
  if ((int64_t)p->n_tb * kBlockKeys > ((int64_t)1 << 28)) return TSFA_ERR_UNSUPPORTED;  // tree keys of the tables
  p->n_tkeys = p->n_tb * kBlockKeys;
  p->n_trees = n_trees;
  // q-blocks a 32-row tile spans: tokens t_lo .. t_lo + ceil(32/G)
  const int toks = (kTileRows + gqa - 1) / gqa + 1;
  p->nqbc_max = std::min(ceil_div(q_len, block_m), toks / block_m + 2);
  if ((int64_t)p->nqbc_max * n_tree_blocks > kMaxStateInts || p->nqbc_max + 1 > 72) return TSFA_ERR_UNSUPPORTED;
  const int64_t rows = (int64_t)batch * num_kv_heads;
  // the grid (rows x key blocks) and the workspace sizes stay far from
  // int64 overflow: every product below is checked by division first
  const int64_t kblocks = (int64_t)p->n_pb + p->n_tb;
  if (kblocks > 0 && rows > ((int64_t)INT32_MAX / 2) / kblocks) return TSFA_ERR_UNSUPPORTED;
  if (rows > ((int64_t)1 << 40) / ((int64_t)p->n_tiles * kTileRows * head_dim * 4)) return TSFA_ERR_UNSUPPORTED;
  if ((int64_t)n_trees * p->n_tiles * p->n_tkeys > ((int64_t)1 << 28)) return TSFA_ERR_UNSUPPORTED;
  p->rowstat_bytes = align256((size_t)rows * p->n_tiles * kTileRows * 8);
  p->dq_bytes = align256((size_t)rows * p->n_tiles * kTileRows * head_dim * 4);
  p->vis_bytes = align256((size_t)n_trees * p->n_tiles * p->n_tkeys * 4 + 16);
  return TSFA_OK;
}

}  // namespace bwd

// ------------------------------------------------------------------ metadata
namespace meta {

bool meta_geom(int q_len, int block_m, int block_n, MetaGeom* g) {
  if (q_len < 0 || block_m <= 0 || block_n <= 0) return false;
  g->q_len = q_len;
  g->block_m = block_m;
  g->block_n = block_n;
  g->nqb = ceil_div(q_len, block_m);
  g->ntb = ceil_div(q_len, block_n);
  const int64_t words = ((int64_t)block_m * block_n + 31) / 32;
  g->cap = (int64_t)g->nqb * g->ntb;
  if (words > INT32_MAX || g->cap * words > INT32_MAX) return false;  // int32 payload offsets
  g->words = (int)words;
  return true;
}

}  // namespace meta

}  // namespace tsfa

using namespace tsfa;

// ------------------------------------------------------------- C entry points
extern "C" int tsfa_version(void) { return 1; }

extern "C" const char* tsfa_status_string(int status) {
  switch (status) {
    case TSFA_OK: return "ok";
    case TSFA_ERR_INVALID_ARGUMENT: return "invalid argument";
    case TSFA_ERR_UNSUPPORTED: return "unsupported configuration";
    case TSFA_ERR_WORKSPACE: return "workspace missing or too small";
    case TSFA_ERR_LAUNCH: return "kernel launch failed";
    case TSFA_ERR_DEVICE: return "no usable HIP device";
    default: return "unknown status";
  }
}

extern "C" int tsfa_config_reload(void) {
  config_reload();
  return TSFA_OK;
}

extern "C" int tsfa_fwd_check_args(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len,
                                   int prefix_len, int n_q_blocks, int n_tree_blocks, int gqa_group_size,
                                   int block_m, int block_n, int head_dim, int dtype) {
  return fwd::check_args(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, n_q_blocks, n_tree_blocks,
                         gqa_group_size, block_m, block_n, head_dim, dtype);
}

extern "C" int tsfa_fwd_plan_for_device(int cus, int max_lds, int batch, int num_heads, int num_kv_heads, int q_len,
                                        int kv_len, int prefix_len, int head_dim, int paged, int32_t* out8) {
  if (out8 == nullptr || cus <= 0 || max_lds <= 0) return TSFA_ERR_INVALID_ARGUMENT;
  fwd::Plan p;
  const int st = fwd::make_plan(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, head_dim, paged != 0,
                                cus, max_lds, config(), &p);
  if (st != TSFA_OK) return st;
  out8[0] = p.n_splits;
  out8[1] = p.units_per_split;
  out8[2] = p.rows_per_chunk;
  out8[3] = p.n_chunks;
  out8[4] = p.grid;
  out8[5] = p.ring_stages;
  out8[6] = p.n_slots;
  out8[7] = p.fold_tree;
  return TSFA_OK;
}

extern "C" size_t tsfa_fwd_workspace_bytes_for_device(int cus, int max_lds, int batch, int num_heads,
                                                      int num_kv_heads, int q_len, int kv_len, int prefix_len,
                                                      int head_dim) {
  if (cus <= 0 || max_lds <= 0) return 0;
  return fwd::workspace_bytes(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, head_dim, cus, max_lds);
}

extern "C" size_t tsfa_bwd_workspace_bytes(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len,
                                           int prefix_len, int block_m, int n_tree_blocks, int head_dim,
                                           int n_trees) {
  if (batch <= 0 || q_len <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 || block_m <= 0 ||
      kv_len < prefix_len || prefix_len < 0 || n_trees <= 0)
    return 0;
  bwd::BwdPlan p;
  if (bwd::make_bwd_plan(batch, num_kv_heads, q_len, kv_len, prefix_len, num_heads / num_kv_heads, head_dim,
                         block_m, n_tree_blocks, n_trees, &p) != TSFA_OK)
    return 0;
  return p.rowstat_bytes + p.dq_bytes + p.vis_bytes;
}

extern "C" int tsfa_meta_check_args(int n_seq, int q_len, int block_m, int block_n) {
  if (block_m <= 0 || block_n <= 0 || n_seq < 0 || q_len < 0) return TSFA_ERR_INVALID_ARGUMENT;
  meta::MetaGeom g;
  if (!meta::meta_geom(q_len, block_m, block_n, &g)) return TSFA_ERR_UNSUPPORTED;
  if ((int64_t)n_seq * g.cap * g.words > ((int64_t)1 << 40)) return TSFA_ERR_UNSUPPORTED;
  if (n_seq > 65535) return TSFA_ERR_UNSUPPORTED;  // grid.y of the device builder
  return TSFA_OK;
}

extern "C" size_t tsfa_meta_workspace_bytes(int n_seq, int q_len, int block_m, int block_n) {
  if (tsfa_meta_check_args(n_seq, q_len, block_m, block_n) != TSFA_OK) return 0;
  meta::MetaGeom g;
  meta::meta_geom(q_len, block_m, block_n, &g);
  const size_t nb = (size_t)n_seq * g.cap;
  return align256(nb) + align256(nb * g.words * 4) + align256(nb * 4);
}

// The tree metadata of n_seq masks on the host, in tsfa_meta_build's layout
// (every pointer host memory).  Blocks are visited row-major (q-block, then
// tree block; tree_sparse_flashattn.py:103-108); a block with no set bit is
// absent (:113-114); FULL iff every element of the block clipped to q_len is
// set (:116-124), with a 0 offset; otherwise MIXED: the block zero-padded to
// block_m x block_n packed with bit i of word w = flat[32w+i], flat =
// r*block_n + c (:44-64), its offset the running payload word cursor
// (:125-134); row_ptr is the running nnz count (:136).
extern "C" int tsfa_meta_build_host(const uint8_t* mask, int64_t mask_seq_stride, int64_t mask_row_stride,
                                    int n_seq, int q_len, int block_m, int block_n, int32_t* row_ptr,
                                    int32_t* col_idx, int8_t* blk_type, int32_t* payload, int32_t* offset,
                                    int32_t* counts) {
  const int st = tsfa_meta_check_args(n_seq, q_len, block_m, block_n);
  if (st != TSFA_OK) return st;
  if (n_seq == 0) return TSFA_OK;
  meta::MetaGeom g;
  meta::meta_geom(q_len, block_m, block_n, &g);
  if (row_ptr == nullptr || counts == nullptr) return TSFA_ERR_INVALID_ARGUMENT;
  if (g.cap > 0 && (mask == nullptr || col_idx == nullptr || blk_type == nullptr || payload == nullptr ||
                    offset == nullptr || mask_row_stride < q_len || mask_seq_stride < 0))
    return TSFA_ERR_INVALID_ARGUMENT;
  const int W = g.words;
  uint32_t* words = g.cap > 0 ? static_cast<uint32_t*>(calloc((size_t)W, sizeof(uint32_t))) : nullptr;
  if (g.cap > 0 && words == nullptr) return TSFA_ERR_UNSUPPORTED;
  for (int s = 0; s < n_seq; ++s) {
    const uint8_t* m0 = g.cap > 0 ? mask + (int64_t)s * mask_seq_stride : nullptr;
    int32_t* rp = row_ptr + (int64_t)s * (g.nqb + 1);
    int32_t* ci = col_idx + (int64_t)s * g.cap;
    int8_t* bt = blk_type + (int64_t)s * g.cap;
    int32_t* of = offset + (int64_t)s * g.cap;
    int32_t* pl = payload + (int64_t)s * g.cap * W;
    int32_t nnz = 0, n_mixed = 0;
    for (int qb = 0; qb < g.nqb; ++qb) {
      rp[qb] = nnz;
      const int q0 = qb * block_m, h = std::min(block_m, q_len - q0);
      for (int tb = 0; tb < g.ntb; ++tb) {
        const int k0 = tb * block_n, w = std::min(block_n, q_len - k0);
        memset(words, 0, (size_t)W * sizeof(uint32_t));
        int64_t ones = 0;
        for (int r = 0; r < h; ++r) {
          const uint8_t* row = m0 + (int64_t)(q0 + r) * mask_row_stride + k0;
          const int64_t f0 = (int64_t)r * block_n;
          for (int c = 0; c < w; ++c)
            if (row[c] != 0) {
              const int64_t f = f0 + c;
              words[f >> 5] |= 1u << (f & 31);
              ++ones;
            }
        }
        if (ones == 0) continue;
        ci[nnz] = tb;
        if (ones == (int64_t)h * w) {
          bt[nnz] = TSFA_FULL_BLOCK;
          of[nnz] = 0;
        } else {
          bt[nnz] = TSFA_MIXED_BLOCK;
          of[nnz] = n_mixed * W;
          memcpy(pl + (int64_t)n_mixed * W, words, (size_t)W * sizeof(uint32_t));
          ++n_mixed;
        }
        ++nnz;
      }
    }
    rp[g.nqb] = nnz;
    counts[2 * s] = nnz;
    counts[2 * s + 1] = n_mixed;
  }
  free(words);
  return TSFA_OK;
}

// _pack_block_mask_to_int32 on the host: word w bit i = bits[32w + i] != 0
// (tree_sparse_flashattn.py:44-64), the last word zero-padded.
extern "C" int tsfa_pack_bits_host(const uint8_t* bits, int64_t n_bits, int32_t* words) {
  if (n_bits < 0) return TSFA_ERR_INVALID_ARGUMENT;
  const int64_t n_words = (n_bits + 31) / 32;
  if (n_words == 0) return TSFA_OK;
  if (bits == nullptr || words == nullptr) return TSFA_ERR_INVALID_ARGUMENT;
  for (int64_t wi = 0; wi < n_words; ++wi) {
    uint32_t word = 0;
    const int64_t end = std::min<int64_t>(32, n_bits - wi * 32);
    for (int64_t i = 0; i < end; ++i)
      if (bits[wi * 32 + i] != 0) word |= 1u << i;
    words[wi] = (int32_t)word;
  }
  return TSFA_OK;
}
