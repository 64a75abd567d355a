// Randomized sweep of libtsfa's host-only code (csrc/tsfa_plan.cpp), built
// with -fsanitize=address,undefined by tests/test_host_sanitizers.py: the
// invariant-division helper against '/', the forward and backward planners
// against the invariants their kernels rely on, the argument validators on
// random and extreme arguments, the paged 32-bit offset rule on known
// layouts, and the host metadata builder by decoding its output back into
// the mask.  Exits non-zero on the first violated invariant; the sanitizers
// abort on any out-of-bounds access, overflow or undefined shift.

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <random>
#include <vector>

#include "tsfa_plan.h"

extern "C" int tsfa_meta_build_host(const uint8_t* mask, int64_t mask_seq_stride, int64_t mask_row_stride,
                                    int n_seq, int q_len, int block_m, int block_n, int32_t* row_ptr,
                                    int32_t* col_idx, int8_t* blk_type, int32_t* payload, int32_t* offset,
                                    int32_t* counts);
extern "C" int tsfa_pack_bits_host(const uint8_t* bits, int64_t n_bits, int32_t* words);
extern "C" int tsfa_meta_check_args(int n_seq, int q_len, int block_m, int block_n);
extern "C" size_t tsfa_meta_workspace_bytes(int n_seq, int q_len, int block_m, int block_n);
extern "C" size_t tsfa_bwd_workspace_bytes(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len,
                                           int prefix_len, int block_m, int n_tree_blocks, int head_dim,
                                           int n_trees);

using namespace tsfa;

static int g_fail = 0;
#define EXPECT(cond, ...)                                   \
  do {                                                      \
    if (!(cond)) {                                          \
      fprintf(stderr, "FAILED %s:%d: %s: ", __FILE__, __LINE__, #cond); \
      fprintf(stderr, __VA_ARGS__);                         \
      fprintf(stderr, "\n");                                \
      if (++g_fail > 20) exit(1);                           \
    }                                                       \
  } while (0)

static std::mt19937_64 rng(12345);
static int64_t uni(int64_t lo, int64_t hi) { return std::uniform_int_distribution<int64_t>(lo, hi)(rng); }

static void sweep_fastdiv() {
  const uint32_t ds[] = {1, 2, 3, 4, 5, 7, 8, 9, 16, 31, 32, 33, 255, 256, 257, 1000, 65535, 65536, 65537,
                         (1u << 20) + 1, (1u << 30) - 1, 1u << 30, (1u << 31) - 1};
  const uint32_t ns[] = {0, 1, 2, 3, 7, 8, 1000, 65535, 65536, (1u << 30), (1u << 31) - 2, (1u << 31) - 1};
  for (uint32_t d : ds) {
    const FastDiv f = make_fastdiv(d);
    for (uint32_t n : ns) EXPECT(fdiv(n, f) == n / d && frem(n, f) == n % d, "n %u d %u", n, d);
    for (int i = 0; i < 20000; ++i) {
      const uint32_t n = (uint32_t)uni(0, (1ll << 31) - 1);
      EXPECT(fdiv(n, f) == n / d && frem(n, f) == n % d, "n %u d %u", n, d);
    }
  }
  for (int i = 0; i < 200000; ++i) {
    const uint32_t d = (uint32_t)uni(1, (1ll << 31) - 1), n = (uint32_t)uni(0, (1ll << 31) - 1);
    const FastDiv f = make_fastdiv(d);
    EXPECT(fdiv(n, f) == n / d, "n %u d %u", n, d);
  }
}

static void sweep_fwd_plan() {
  const int cus_list[] = {1, 8, 80, 256, 304};
  Config cfg = config();
  for (int it = 0; it < 200000; ++it) {
    const int kvh = (int)uni(1, 16), g = (int)uni(1, 16);
    const int batch = (int)uni(1, 64), heads = kvh * g;
    const int q_len = (int)uni(1, it % 10 == 0 ? 20000 : 1100);
    const int prefix = (int)uni(0, it % 7 == 0 ? 300000 : 70000);
    const int kv_len = prefix + q_len + (int)uni(0, 3) * (it % 13 == 0);
    const int D = uni(0, 1) ? 64 : 128;
    const int cus = cus_list[uni(0, 4)];
    const int max_lds = uni(0, 3) ? 163840 : 65536;
    cfg.streams = (int)uni(0, 2);
    cfg.prefix_units = uni(0, 5) ? 0 : (int)uni(-3, 300);
    cfg.fold_tree = (int)uni(-1, 1);
    fwd::Plan p;
    memset(&p, 0xAB, sizeof(p));
    const int st = fwd::make_plan(batch, heads, kvh, q_len, kv_len, prefix, D, uni(0, 1) != 0, cus, max_lds, cfg, &p);
    if (st != TSFA_OK) {
      EXPECT(st == TSFA_ERR_UNSUPPORTED || st == TSFA_ERR_INVALID_ARGUMENT, "status %d", st);
      continue;
    }
    const int64_t TG = (int64_t)q_len * g;
    EXPECT(p.streams == 1 || p.streams == 2, "streams %d", p.streams);
    EXPECT(p.rows_per_chunk * p.streams == fwd::kMaxRows, "rows %d", p.rows_per_chunk);
    EXPECT((int64_t)p.n_chunks * p.rows_per_chunk >= TG && (int64_t)(p.n_chunks - 1) * p.rows_per_chunk < TG,
           "chunks %d TG %lld", p.n_chunks, (long long)TG);
    EXPECT(p.n_pu == (prefix + 31) / 32, "n_pu %d", p.n_pu);
    if (p.n_pu > 0) {
      EXPECT(p.units_per_split >= 1 && p.units_per_split <= p.n_pu, "ups %d", p.units_per_split);
      EXPECT((int64_t)p.n_splits * p.units_per_split >= p.n_pu &&
                 (int64_t)(p.n_splits - 1) * p.units_per_split < p.n_pu,
             "splits %d ups %d n_pu %d", p.n_splits, p.units_per_split, p.n_pu);
    } else {
      EXPECT(p.n_splits == 0, "splits %d", p.n_splits);
    }
    EXPECT(p.n_slots == p.n_splits + (p.fold_tree ? 0 : 1), "slots %d", p.n_slots);
    EXPECT(!p.fold_tree || p.n_splits >= 1, "fold without a run");
    EXPECT((int64_t)p.n_items == (int64_t)batch * kvh * p.n_chunks * p.n_slots, "items %d", p.n_items);
    EXPECT(p.grid % 8 == 0 && p.grid >= p.n_items && p.grid - p.n_items < 8, "grid %d items %d", p.grid, p.n_items);
    EXPECT(p.lds_bytes <= (size_t)max_lds, "lds");
    const size_t rows = (size_t)batch * heads * q_len;
    EXPECT(p.ws_acc_bytes >= rows * p.n_slots * D * 2 && p.ws_acc_bytes % 256 == 0, "acc");
    EXPECT(p.ws_ml_bytes >= rows * p.n_slots * 8 && p.ws_ml_bytes % 256 == 0, "ml");
    EXPECT(p.vt_max >= 1, "vt_max %d", p.vt_max);
  }
  // invalid shapes come back as errors, never as plans
  fwd::Plan p;
  const Config c0 = config();
  EXPECT(fwd::make_plan(0, 4, 2, 8, 8, 0, 128, false, 256, 163840, c0, &p) != TSFA_OK, "batch 0");
  EXPECT(fwd::make_plan(1, 5, 2, 8, 8, 0, 128, false, 256, 163840, c0, &p) != TSFA_OK, "heads not a multiple of kv heads");
  EXPECT(fwd::make_plan(1, 4, 2, 8, 4, 8, 128, false, 256, 163840, c0, &p) != TSFA_OK, "kv < prefix");
  EXPECT(fwd::make_plan(1, 4, 2, 8, 8, 0, 96, false, 256, 163840, c0, &p) != TSFA_OK, "head_dim");
  EXPECT(fwd::make_plan(1, 4, 2, 8, 8, 0, 128, false, 0, 163840, c0, &p) != TSFA_OK, "no CUs");
  EXPECT(fwd::make_plan(1, 4, 2, 8, 8, 0, 128, false, 256, 1024, c0, &p) == TSFA_ERR_UNSUPPORTED, "small LDS");
  EXPECT(fwd::make_plan(1, 4096, 1, (1 << 30), (1 << 30), 0, 128, false, 256, 163840, c0, &p) ==
             TSFA_ERR_UNSUPPORTED, "huge rows");
}

static void sweep_check_args() {
  const int extremes[] = {INT32_MIN, -1, 0, 1, 2, 15, 16, 17, 64, 128, 1 << 20, INT32_MAX};
  for (int it = 0; it < 300000; ++it) {
    int v[13];
    for (int& x : v) x = uni(0, 3) ? (int)uni(-2, 300) : extremes[uni(0, 11)];
    const int st = fwd::check_args(v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7], v[8], v[9], v[10], v[11], v[12]);
    EXPECT(st == TSFA_OK || st == TSFA_ERR_INVALID_ARGUMENT || st == TSFA_ERR_UNSUPPORTED, "status %d", st);
    const int ms = tsfa_meta_check_args(v[0], v[3], v[9], v[10]);
    EXPECT(ms == TSFA_OK || ms == TSFA_ERR_INVALID_ARGUMENT || ms == TSFA_ERR_UNSUPPORTED, "meta status %d", ms);
    if (ms == TSFA_OK && (int64_t)v[0] * v[3] < (1 << 22))
      EXPECT(tsfa_meta_workspace_bytes(v[0], v[3], v[9], v[10]) > 0 || v[0] == 0 || v[3] == 0, "meta ws");
    (void)tsfa_bwd_workspace_bytes(v[0], v[1], v[2], v[3], v[4], v[5], v[9], v[7], v[11], v[8]);
  }
  // a valid Llama-3-8B call and the reference's rejections of it
  EXPECT(fwd::check_args(1, 32, 8, 64, 4160, 4096, 4, 1, 4, 16, 64, 128, TSFA_DTYPE_BF16) == TSFA_OK, "ok");
  EXPECT(fwd::check_args(1, 32, 8, 64, 4160, 4096, 4, 1, 4, 0, 64, 128, TSFA_DTYPE_BF16) == TSFA_ERR_INVALID_ARGUMENT,
         "block_m 0");
  EXPECT(fwd::check_args(1, 32, 8, 64, 100, 4096, 4, 1, 4, 16, 64, 128, TSFA_DTYPE_BF16) == TSFA_ERR_INVALID_ARGUMENT,
         "kv < prefix");
  EXPECT(fwd::check_args(1, 32, 8, 64, 4160, 4096, 4, 1, 4, 16, 64, 96, TSFA_DTYPE_BF16) == TSFA_ERR_UNSUPPORTED,
         "head_dim 96");
}

static void sweep_layouts() {
  alignas(16) static char buf[64];
  const void* al = buf;
  const void* mis = buf + 8;
  for (int it = 0; it < 100000; ++it) {
    int64_t s4[4], s5[5];
    for (auto& x : s4) x = uni(0, 3) ? uni(0, 1 << 20) * (uni(0, 1) ? 8 : 1) : uni(INT64_MIN / 4, INT64_MAX / 4);
    for (auto& x : s5) x = uni(0, 3) ? uni(0, 1 << 22) * (uni(0, 1) ? 8 : 1) : uni(INT64_MIN / 4, INT64_MAX / 4);
    if (uni(0, 1)) s4[3] = 1;
    if (uni(0, 1)) s5[4] = 1;
    const void* p = uni(0, 1) ? al : mis;
    int st = fwd::check_strides(p, s4, al, uni(0, 9) ? s4 : nullptr);
    EXPECT(st >= 0 && st <= 2, "strides %d", st);
    st = fwd::check_kv_strides(p, s4, al, s4);
    EXPECT(st >= 0 && st <= 2, "kv strides %d", st);
    const int32_t indptr[2] = {0, 1};
    st = fwd::check_paged((int)uni(1, 64), (int)uni(0, 100000), p, uni(0, 9) ? s5 : nullptr,
                          uni(0, 1) ? indptr : nullptr, uni(-2, 1 << 20), uni(-2, 1ll << 33), (int)uni(-2, 1 << 20),
                          (int)uni(-1, 300));
    EXPECT(st >= 0 && st <= 2, "paged %d", st);
    (void)fwd::paged_offsets_fit_32((int)uni(-1, 1 << 24), s5[0], s5[2], (int)uni(-1, 512), (int)uni(-1, 256));
  }
  // the 32-bit paged kernel: FlashInfer's NHD pool of 1000 pages fits; a
  // permuted [page_size, pages, 2, Hkv, D] pool whose row stride spans every
  // page does not, although pages * page_stride alone would (2048-element
  // pages of 200000 pages = 0.8 GB)
  EXPECT(fwd::paged_offsets_fit_32(1000, 2 * 16 * 8 * 128, 8 * 128, 16, 128), "NHD pool");
  EXPECT(!fwd::paged_offsets_fit_32(200000, 2 * 8 * 128, 200000LL * 2 * 8 * 128, 16, 128), "permuted pool");
  EXPECT(!fwd::paged_offsets_fit_32((1 << 17) + 1, 1 << 14, 128, 16, 128), "4 GiB of pages");
  EXPECT(fwd::paged_offsets_fit_32(1, 0, 0, 16, 128), "one page");
}

static void sweep_bwd_plan() {
  for (int it = 0; it < 100000; ++it) {
    const int batch = (int)uni(1, 32), kvh = (int)uni(1, 16), gqa = (int)uni(1, 16);
    const int q_len = (int)uni(1, it % 5 ? 600 : 300000), prefix = (int)uni(0, 70000);
    const int kv_len = prefix + q_len, bm = (int)uni(1, 128), ntb = (int)uni(0, 64), nt = (int)uni(1, batch);
    bwd::BwdPlan p;
    const int st = bwd::make_bwd_plan(batch, kvh, q_len, kv_len, prefix, gqa, uni(0, 1) ? 64 : 128, bm, ntb, nt, &p);
    if (st != TSFA_OK) continue;
    const int64_t TG = (int64_t)q_len * gqa;
    EXPECT((int64_t)p.n_tiles * bwd::kTileRows >= TG, "tiles");
    EXPECT((int64_t)p.n_pb * bwd::kBlockKeys >= prefix && (int64_t)p.n_tb * bwd::kBlockKeys >= kv_len - prefix, "blocks");
    EXPECT((int64_t)p.nqbc_max * ntb <= bwd::kMaxStateInts, "state table");
    EXPECT(p.rowstat_bytes % 256 == 0 && p.dq_bytes % 256 == 0 && p.vis_bytes % 256 == 0, "alignment");
  }
}

static void sweep_meta() {
  for (int it = 0; it < 3000; ++it) {
    const int n_seq = (int)uni(1, 3), q_len = (int)uni(0, 90), bm = (int)uni(1, 40), bn = (int)uni(1, 40);
    const int64_t row_stride = q_len + uni(0, 5), seq_stride = row_stride * q_len + uni(0, 7);
    std::vector<uint8_t> mask((size_t)std::max<int64_t>(1, seq_stride * n_seq), 0);
    const double dens = std::uniform_real_distribution<double>(0, 1)(rng);
    for (int s = 0; s < n_seq; ++s)
      for (int i = 0; i < q_len; ++i)
        for (int j = 0; j < q_len; ++j)
          mask[s * seq_stride + i * row_stride + j] = std::uniform_real_distribution<double>(0, 1)(rng) < dens ? (uint8_t)uni(1, 255) : 0;
    meta::MetaGeom g;
    if (!meta::meta_geom(q_len, bm, bn, &g)) continue;
    const int W = g.words;
    std::vector<int32_t> row_ptr((size_t)n_seq * (g.nqb + 1)), col_idx((size_t)std::max<int64_t>(1, n_seq * g.cap)),
        payload((size_t)std::max<int64_t>(1, n_seq * g.cap * W)), offset(col_idx.size()), counts((size_t)n_seq * 2);
    std::vector<int8_t> blk_type(col_idx.size());
    const int st = tsfa_meta_build_host(mask.data(), seq_stride, row_stride, n_seq, q_len, bm, bn, row_ptr.data(),
                                        col_idx.data(), blk_type.data(), payload.data(), offset.data(), counts.data());
    EXPECT(st == TSFA_OK, "status %d", st);
    if (st != TSFA_OK) continue;
    for (int s = 0; s < n_seq; ++s) {
      const int32_t* rp = &row_ptr[(size_t)s * (g.nqb + 1)];
      const int nnz = counts[2 * s], n_mixed = counts[2 * s + 1];
      EXPECT(rp[0] == 0 && rp[g.nqb] == nnz, "row_ptr ends");
      // decode every listed block and compare it with the mask; every block
      // not listed must be all zero
      std::vector<uint8_t> covered((size_t)std::max<int64_t>(1, g.cap), 0);
      int mixed_seen = 0;
      for (int qb = 0; qb < g.nqb; ++qb) {
        EXPECT(rp[qb] <= rp[qb + 1], "row_ptr monotone");
        for (int e = rp[qb]; e < rp[qb + 1]; ++e) {
          const int tb = col_idx[(size_t)s * g.cap + e];
          EXPECT(tb >= 0 && tb < g.ntb, "col %d", tb);
          if (e > rp[qb]) EXPECT(col_idx[(size_t)s * g.cap + e - 1] < tb, "cols ascending");
          covered[(size_t)qb * g.ntb + tb] = 1;
          const int8_t kind = blk_type[(size_t)s * g.cap + e];
          const int32_t off = offset[(size_t)s * g.cap + e];
          if (kind == TSFA_MIXED_BLOCK) EXPECT(off == mixed_seen++ * W, "offset cursor");
          for (int r = 0; r < bm; ++r)
            for (int c = 0; c < bn; ++c) {
              const int qi = qb * bm + r, kj = tb * bn + c;
              const bool in = qi < q_len && kj < q_len;
              const bool want = in && mask[s * seq_stride + (int64_t)qi * row_stride + kj] != 0;
              bool got;
              if (kind == TSFA_FULL_BLOCK) {
                got = in;
              } else {
                const int64_t f = (int64_t)r * bn + c;
                got = ((uint32_t)payload[(size_t)s * g.cap * W + off + (f >> 5)] >> (f & 31)) & 1u;
              }
              EXPECT(got == want, "seq %d block (%d,%d) r %d c %d", s, qb, tb, r, c);
            }
        }
      }
      EXPECT(mixed_seen == n_mixed, "n_mixed");
      for (int qb = 0; qb < g.nqb; ++qb)
        for (int tb = 0; tb < g.ntb; ++tb) {
          if (covered[(size_t)qb * g.ntb + tb]) continue;
          for (int qi = qb * bm; qi < std::min(q_len, qb * bm + bm); ++qi)
            for (int kj = tb * bn; kj < std::min(q_len, tb * bn + bn); ++kj)
              EXPECT(mask[s * seq_stride + (int64_t)qi * row_stride + kj] == 0, "absent block has a bit");
        }
    }
    // bit packing: word w bit i = bits[32w + i]
    const int64_t nb = uni(0, 200);
    std::vector<uint8_t> bits((size_t)std::max<int64_t>(1, nb));
    for (auto& b : bits) b = (uint8_t)(uni(0, 1) * uni(1, 255));
    std::vector<int32_t> words((size_t)std::max<int64_t>(1, (nb + 31) / 32));
    EXPECT(tsfa_pack_bits_host(bits.data(), nb, words.data()) == TSFA_OK, "pack");
    for (int64_t i = 0; i < nb; ++i) EXPECT((((uint32_t)words[i >> 5] >> (i & 31)) & 1u) == (bits[i] != 0), "bit");
  }
  EXPECT(tsfa_meta_build_host(nullptr, 0, 0, 1, 8, 4, 4, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr) ==
             TSFA_ERR_INVALID_ARGUMENT, "null outputs");
  EXPECT(tsfa_pack_bits_host(nullptr, -1, nullptr) == TSFA_ERR_INVALID_ARGUMENT, "negative bits");
}

int main() {
  sweep_fastdiv();
  sweep_fwd_plan();
  sweep_check_args();
  sweep_layouts();
  sweep_bwd_plan();
  sweep_meta();
  if (g_fail) {
    fprintf(stderr, "%d invariant violations\n", g_fail);
    return 1;
  }
  printf("host sweep: all invariants hold\n");
  return 0;
}
