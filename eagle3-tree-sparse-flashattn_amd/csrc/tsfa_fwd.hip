// Tree-sparse attention forward for gfx950 (MI355X).
//
// Semantics: block_sparse_tree_fwd_kernel (tree_sparse_flashattn.py:163-339).
// For query row (b, h, t): dense prefix keys [0, prefix_len) (:235-279) plus
// the tree keys prefix_len + tb*BN + c (< kv_len) of the CSR row of q-block
// t / BM, filtered by the MIXED bitset (:281-327); kv head h / G (:216);
// online softmax with the -inf guards of :272-279 / :320-327; O = acc / l
// (:329, NaN for a row with no visible key).
//
// Work decomposition (the MI355X design, not the reference's grid):
//   * rows of one (batch, kv head) are packed token-major, r = t*G + g, so the
//     G query heads that share a K/V head share every K/V byte staged in LDS;
//     a workgroup owns a chunk of <= 256 rows (tokens_per_chunk * G);
//   * the prefix is split into runs of 64-key tiles; each (b, kvh, chunk,
//     split) is one workgroup, so a small tree still spreads the prefix over
//     all 256 CUs (split-KV);
//   * one more workgroup per (b, kvh, chunk) runs the tree part: it expands
//     the CSR rows of the chunk's q-blocks into per-token 64-bit visibility
//     words for every 64-key tree tile that holds a visible key, and skips
//     the rest (ZERO blocks are never loaded);
//   * every workgroup writes an fp32 partial (m, l, acc) per row; a second
//     kernel merges the partials (log-sum-exp) and writes O in the input
//     dtype.
// Inside a workgroup: 4 waves x 64 rows; K/V tiles of 64 keys go HBM -> LDS
// with global_load_lds (16 B per lane, no VGPR staging) into a ring of
// NSTAGE stages; S^T = K Q^T and O^T += V^T P^T run on
// v_mfma_f32_16x16x32_{bf16,f16}; V^T operands come from ds_read_b64_tr_b16,
// so V is never transposed in memory.  Scores stay in registers; exp2 with
// sm_scale*log2(e) folded into one FMA.  The running max is only re-based
// when it grows by more than 2^8 (rescaling is exact for any consistent
// reference point), which skips the O rescale on almost every tile.

#include <math.h>
#include <stdlib.h>

#include <algorithm>

#include "tsfa_internal.h"

namespace tsfa {
namespace fwd {

constexpr int kRowsPerChunk = 256;  // rows of one workgroup (all waves)
constexpr int kTileKeys = 64;
constexpr int kMaskBytes = 16384;    // per-token tree visibility words
constexpr int kMaxTreeTiles = 512;   // tree keys <= 32768
constexpr int kMiscInts = 320;       // LDS scalars: visited count, row_ptr window of <= 258 q-blocks
constexpr float kRescaleLog2 = 8.0f;

struct SplitArgs {
  const void* q;
  const void* k;
  const void* v;
  const int32_t* row_ptr;
  const int32_t* col_idx;
  const int8_t* blk_type;
  const int32_t* payload;
  const int32_t* offset;
  int64_t ms_row_ptr, ms_col_idx, ms_blk_type, ms_payload, ms_offset;
  int64_t sqb, sqh, sqm, skb, skh, skn, svb, svh, svn;
  float scale_log2;  // sm_scale * log2(e)
  int num_kv_heads, group, q_len, kv_len, prefix_len, block_m, block_n, n_tree_blocks;
  int tpc, n_chunks, tiles_per_split, n_ptiles, n_slots, n_items, items_per_xcd;
  int tree_key_limit;  // min(n_tree_blocks*BN, kv_len - prefix_len)
  int vt_max;          // tree tiles per mask batch
  void* ws_o;          // [B*Hkv][n_slots][q_len*G][D] partial O / l in the input dtype
  float2* ws_ml;       // [B*Hkv][n_slots][q_len*G] (m, l) of each partial
};

struct CombineArgs {
  void* o;
  int64_t sob, soh, som;
  float scale_log2;
  int batch, num_heads, num_kv_heads, group, q_len, n_slots;
  const void* ws_o;
  const float2* ws_ml;
};

// 16-byte-chunk XOR swizzles of the K and V LDS tiles (row = key in tile).
// K: the 16 keys one MFMA A-operand read touches land on 16 distinct bank
// groups.  V: the 4 keys x 32 bytes of a ds_read_b64_tr_b16 group, and the
// neighbouring group, land on distinct bank groups.
template <int D> __device__ inline int swz_k(int key);
template <> __device__ inline int swz_k<128>(int key) { return (key & 3) | ((key >> 1) & 12); }
template <> __device__ inline int swz_k<64>(int key) { return ((key >> 1) & 1) | ((key >> 2) & 6); }
template <int D> __device__ inline int swz_v(int key);
template <> __device__ inline int swz_v<128>(int key) { return ((key & 3) << 1) | (((key >> 3) & 1) << 3); }
template <> __device__ inline int swz_v<64>(int key) { return (((key >> 1) & 1) << 1) | (((key >> 3) & 1) << 2); }

// 16 bytes per lane HBM -> LDS (global_load_lds_dwordx4): lane i's bytes land
// at LDS address lds_base + 16*i.  Issued as inline asm so the compiler does
// not treat every later LDS read as aliasing the in-flight copy (it would
// insert vmcnt(0) before them and serialise the prefetch); completion is
// ordered explicitly by sync_tiles().
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is reserved; the clobber documents the write
__device__ inline void dma16(const void* src, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(lds_base)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Wait until at most N of this wave's vector-memory loads are in flight, then
// workgroup barrier (LDS writes of every wave complete and visible).
template <int N> __device__ inline void sync_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" : : "n"(N) : "memory");
}

// sync_vm with at most `tiles` ring tiles (LPT loads each) still in flight.
template <int LPT, int NSTAGE> __device__ inline void sync_tiles(int tiles) {
  if constexpr (NSTAGE >= 4) {
    if (tiles >= 2) { sync_vm<2 * LPT>(); return; }
  }
  if constexpr (NSTAGE >= 3) {
    if (tiles >= 1) { sync_vm<LPT>(); return; }
  }
  sync_vm<0>();
}

// Workgroup barrier that also orders LDS accesses (compiler and hardware).
__device__ inline void sync_lds() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ inline uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const TSFA_LDS void*)p;
}

template <typename V, typename U> __device__ inline V bit_cast(U u) { return __builtin_bit_cast(V, u); }

// Max / sum over lanes {l, l^16, l^32, l^48} with the gfx950 row-swap
// permutes (two VALU ops each, no LDS round trip).
__device__ inline float row_max4(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ inline float row_sum4(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// WAVES waves per workgroup, each owning RT row tiles (16 rows) of the 256-row
// chunk: WAVES = 8 gives two waves per SIMD (one wave's softmax overlaps the
// other's MFMAs) at <= 256 registers per lane.
template <typename T, int D, int NSTAGE, int WAVES>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(WAVES / 4, WAVES / 4)))
void split_kernel(const SplitArgs a) {
  typedef typename Mma<T>::vec8 V8;
  constexpr int kThreads = WAVES * 64;
  constexpr int RT = kRowsPerChunk / (WAVES * 16);
  constexpr int kRowsPerWave = RT * 16;
  constexpr int ROWB = D * 2;
  constexpr int CPR = D / 8;
  constexpr int TILEB = kTileKeys * ROWB;
  constexpr int STAGEB = 2 * TILEB;
  constexpr int KLOADS = TILEB / (kThreads * 16);
  constexpr int LPT = 2 * KLOADS;
  constexpr int KSTEPS = D / 32;
  constexpr int DTILES = D / 16;

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  unsigned char* ring = smem;
  uint16_t* masks = reinterpret_cast<uint16_t*>(smem + NSTAGE * STAGEB);
  int* vis = reinterpret_cast<int*>(smem + NSTAGE * STAGEB + kMaskBytes);
  int* misc = vis + kMaxTreeTiles;  // kMiscInts ints

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lg = lane >> 4;

  // XCD-aware item order: consecutive block ids go to different XCDs, so map
  // each XCD to a contiguous range of items (items sharing K/V stay together).
  const int bid = blockIdx.x;
  const int item = (bid & 7) * a.items_per_xcd + (bid >> 3);
  if (item >= a.n_items) return;
  const int slot = item % a.n_slots;
  int rest = item / a.n_slots;
  const int chunk = rest % a.n_chunks;
  rest /= a.n_chunks;
  const int kvh = rest % a.num_kv_heads;
  const int b = rest / a.num_kv_heads;
  const bool is_tree = slot == a.n_slots - 1;

  const int G = a.group;
  const int t_lo = chunk * a.tpc;
  const int t_hi = min(t_lo + a.tpc, a.q_len);
  const int ntok = t_hi - t_lo;
  const int rows = ntok * G;
  const bool active = wave * kRowsPerWave < rows;
  const float sl2 = a.scale_log2;
  const float rescale_raw = kRescaleLog2 / sl2;  // re-base the running max past 2^8 growth

  const T* kbase = static_cast<const T*>(a.k) + b * a.skb + kvh * a.skh;
  const T* vbase = static_cast<const T*>(a.v) + b * a.svb + kvh * a.svh;

  // HBM -> LDS for tile j (keys key0 .. key0+63) into ring stage j % NSTAGE.
  auto issue = [&](int j, int key0) {
    unsigned char* sk = ring + (j % NSTAGE) * STAGEB;
    unsigned char* sv = sk + TILEB;
#pragma unroll
    for (int u = 0; u < KLOADS; ++u) {
      const int sidx = (wave * KLOADS + u) * 64 + lane;
      const int row = sidx / CPR, pos = sidx % CPR;
      const int key = min(key0 + row, a.kv_len - 1);
      const T* src = kbase + (int64_t)key * a.skn + ((pos ^ swz_k<D>(row)) * 8);
      dma16(src, __builtin_amdgcn_readfirstlane(lds_addr(sk + (wave * KLOADS + u) * 1024)));
    }
#pragma unroll
    for (int u = 0; u < KLOADS; ++u) {
      const int sidx = (wave * KLOADS + u) * 64 + lane;
      const int row = sidx / CPR, pos = sidx % CPR;
      const int key = min(key0 + row, a.kv_len - 1);
      const T* src = vbase + (int64_t)key * a.svn + ((pos ^ swz_v<D>(row)) * 8);
      dma16(src, __builtin_amdgcn_readfirstlane(lds_addr(sv + (wave * KLOADS + u) * 1024)));
    }
  };

  // The prefix split's first tile goes out before anything else so the Q
  // loads below overlap its HBM latency.  The rest of the prologue is issued
  // after Q is consumed: the compiler waits for Q with vmcnt(0), which would
  // otherwise also wait for every tile issued before it.
  const int prefix_tile0 = is_tree ? 0 : slot * a.tiles_per_split;
  const int prefix_ntl = is_tree ? 0 : min(a.tiles_per_split, a.n_ptiles - prefix_tile0);
  if (prefix_ntl > 0) issue(0, prefix_tile0 * kTileKeys);

  // Q^T fragments: row r = wave*RT*16 + rt*16 + li, d = ks*32 + lg*8 + [0, 8).
  i16x8 qf[RT][KSTEPS];
  int row_tok[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int r = wave * kRowsPerWave + rt * 16 + li;
    row_tok[rt] = 0;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) qf[rt][ks] = i16x8{0, 0, 0, 0, 0, 0, 0, 0};
    if (r < rows) {
      const int tt = r / G;
      const int g = r - tt * G;
      row_tok[rt] = tt;
      const T* qp = static_cast<const T*>(a.q) + b * a.sqb + (int64_t)(kvh * G + g) * a.sqh +
                    (int64_t)(t_lo + tt) * a.sqm + lg * 8;
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) qf[rt][ks] = *reinterpret_cast<const i16x8*>(qp + ks * 32);
    }
  }

  // Consume the Q loads here: otherwise the compiler waits for them lazily at
  // their first use inside the tile loop, where its vmcnt count would also
  // cover (and stall on) the in-flight K/V prefetch it does not know about.
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) asm volatile("" : : "v"(qf[rt][ks]));
  for (int j = 1; j < NSTAGE - 1 && j < prefix_ntl; ++j) issue(j, (prefix_tile0 + j) * kTileKeys);

  // Running state per lane: rows (rt, li); O^T element d = dt*16 + lg*4 + [0,4).
  f32x4 o[DTILES][RT];
  float m_run[RT], l_run[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m_run[rt] = -INFINITY;
    l_run[rt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DTILES; ++dt) o[dt][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // One 64-key tile for this wave's 64 rows, as two 32-key halves (keeps the
  // live score/probability registers small).  mrow[rt] is the 64-bit key
  // visibility of row tile rt's lane row (read only when `masked`).
  auto compute = [&](int stage, bool masked, const uint64_t (&mrow)[RT]) {
    const unsigned char* sk = ring + stage * STAGEB;
    const unsigned char* sv = sk + TILEB;
#pragma unroll
    for (int hk = 0; hk < 2; ++hk) {
      // S^T sub-tile h: MFMA row li holds key hk*32 + (li/4)*8 + h*4 + li%4, so
      // each lane's 8 scores of this half are 8 consecutive keys.
      f32x4 s[2][RT];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) s[h][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int key = hk * 32 + (li >> 2) * 8 + h * 4 + (li & 3);
          const int chunk = ks * 4 + lg;
          const i16x8 kf = *reinterpret_cast<const i16x8*>(sk + key * ROWB + ((chunk ^ swz_k<D>(key)) << 4));
#pragma unroll
          for (int rt = 0; rt < RT; ++rt)
            s[h][rt] = Mma<T>::run(bit_cast<V8>(kf), bit_cast<V8>(qf[rt][ks]), s[h][rt]);
        }
      }
      if (masked) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const uint32_t bb = (uint32_t)(mrow[rt] >> (hk * 32 + lg * 8)) & 0xffu;
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (!((bb >> (h * 4 + i)) & 1u)) s[h][rt][i] = -INFINITY;
        }
      }
      float m_new[RT];
      bool need = false;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        float mx = fmaxf(s[0][rt][0], s[1][rt][0]);
#pragma unroll
        for (int i = 1; i < 4; ++i) mx = fmaxf(mx, fmaxf(s[0][rt][i], s[1][rt][i]));
        // the row's 64 keys sit in lanes li, li+16, li+32, li+48
        mx = row_max4(mx);
        m_new[rt] = fmaxf(m_run[rt], mx);
        need |= m_new[rt] - m_run[rt] > rescale_raw;  // false for -inf/-inf (NaN)
      }
      if (__ballot(need) != 0) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          // alpha = 1 when both are -inf (tree_sparse_flashattn.py:276, :324)
          const float alpha =
              (m_new[rt] == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f((m_run[rt] - m_new[rt]) * sl2);
          m_run[rt] = m_new[rt];
          l_run[rt] *= alpha;
#pragma unroll
          for (int dt = 0; dt < DTILES; ++dt) o[dt][rt] *= alpha;
        }
      }
      V8 pb[RT];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        // p = 0 where the score is -inf (tree_sparse_flashattn.py:274, :322): with a
        // finite reference point exp2(-inf) = 0; a row with no visible key yet keeps
        // m = -inf and uses reference 0, so every p there is exp2(-inf) = 0 too.
        const float mb = (m_run[rt] == -INFINITY) ? 0.f : m_run[rt] * sl2;
        float lsum = 0.f;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[h][rt][i], sl2, -mb));
            lsum += p;
            pb[rt][h * 4 + i] = (T)p;  // P rounded to the input dtype (:278)
          }
        l_run[rt] += lsum;
      }
#pragma unroll
      for (int dt = 0; dt < DTILES; ++dt) {
        i16x4 half[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int key = hk * 32 + lg * 8 + hh * 4 + (li >> 2);
          const int d = dt * 16 + 4 * (li & 3);
          const int off = key * ROWB + (((d >> 3) ^ swz_v<D>(key)) << 4) + ((d & 7) << 1);
          half[hh] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((TSFA_LDS i16x4*)(sv + off));
        }
        const i16x8 vf = i16x8{half[0][0], half[0][1], half[0][2], half[0][3],
                               half[1][0], half[1][1], half[1][2], half[1][3]};
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) o[dt][rt] = Mma<T>::run(bit_cast<V8>(vf), pb[rt], o[dt][rt]);
      }
    }
  };

  // Pipeline over ntl tiles: NSTAGE-1 tiles in flight ahead of the one in use.
  auto run_tiles = [&](int ntl, bool prologue_issued, auto key0_of, auto masked_of, auto mask_of_tile) {
    if (!prologue_issued)
      for (int j = 0; j < NSTAGE - 1 && j < ntl; ++j) issue(j, key0_of(j));
    for (int j = 0; j < ntl; ++j) {
      // tile j landed for every wave; stage (j-1)%NSTAGE is free
      sync_tiles<LPT, NSTAGE>(min(ntl - 1 - j, NSTAGE - 2));
      if (j + NSTAGE - 1 < ntl) issue(j + NSTAGE - 1, key0_of(j + NSTAGE - 1));
      if (active) {
        const bool masked = masked_of(j);
        uint64_t mrow[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) mrow[rt] = masked ? mask_of_tile(j, rt) : ~0ull;
        compute(j % NSTAGE, masked, mrow);
      }
    }
    sync_lds();  // ring free again
  };

  if (!is_tree) {
    const int P = a.prefix_len;
    const int tile0 = prefix_tile0;
    run_tiles(
        prefix_ntl, true, [&](int j) { return (tile0 + j) * kTileKeys; },
        [&](int j) { return P - (tile0 + j) * kTileKeys < kTileKeys; },
        [&](int j, int) {
          const int valid = P - (tile0 + j) * kTileKeys;
          return valid >= 64 ? ~0ull : ((1ull << valid) - 1ull);
        });
  } else {
    const int P = a.prefix_len, BM = a.block_m, BN = a.block_n, ntb = a.n_tree_blocks;
    const int qb_lo = t_lo / BM, qb_hi = (t_hi - 1) / BM, nqbc = qb_hi - qb_lo + 1;
    const int32_t* rp = a.row_ptr + b * a.ms_row_ptr;
    const int32_t* ci = a.col_idx + b * a.ms_col_idx;
    const int8_t* bt = a.blk_type + b * a.ms_blk_type;
    const int32_t* pl = a.payload + b * a.ms_payload;
    const int32_t* of = a.offset + b * a.ms_offset;
    int* st = reinterpret_cast<int*>(ring);  // [nqbc][ntb]: 0 ZERO, -1 FULL, 1+offset MIXED
    int* rps = misc + 8;                     // row_ptr[qb_lo .. qb_hi+1]
    // Two parallel round trips: the chunk's row_ptr window, then every CSR
    // entry of those rows at once.
    auto build_state = [&]() {
      for (int i = tid; i < nqbc * ntb; i += kThreads) st[i] = 0;
      if (tid <= nqbc) rps[tid] = rp[qb_lo + tid];
      sync_lds();
      const int e_begin = rps[0], e_end = rps[nqbc];
      for (int e = e_begin + tid; e < e_end; e += kThreads) {
        int qq = 0;
        while (qq + 1 < nqbc && rps[qq + 1] <= e) ++qq;
        const int tb = ci[e];
        if (tb >= 0 && tb < ntb) st[qq * ntb + tb] = (bt[e] == TSFA_FULL_BLOCK) ? -1 : (of[e] + 1);
      }
      sync_lds();
    };
    build_state();
    const int n_tt = (a.tree_key_limit + kTileKeys - 1) / kTileKeys;
    for (int i = tid; i < n_tt; i += kThreads) vis[i] = 0;
    sync_lds();
    for (int i = tid; i < nqbc * ntb; i += kThreads) {
      if (st[i] != 0) {
        const int tb = i % ntb;
        const int c_first = tb * BN, c_last = min(tb * BN + BN, a.tree_key_limit) - 1;
        for (int v = c_first / kTileKeys; v <= c_last / kTileKeys; ++v) vis[v] = 1;
      }
    }
    sync_lds();
    if (wave == 0) {
      int n = 0;
      for (int base = 0; base < n_tt; base += 64) {
        const int idx = base + lane;
        const bool f = idx < n_tt && vis[idx] != 0;
        const uint64_t bal = __ballot(f);
        const int pre = __popcll(bal & ((1ull << lane) - 1ull));
        if (f) vis[n + pre] = idx;
        n += __popcll(bal);
      }
      if (lane == 0) misc[0] = n;
    }
    sync_lds();
    const int n_vis = misc[0];
    for (int vb0 = 0; vb0 < n_vis; vb0 += a.vt_max) {
      const int nb = min(a.vt_max, n_vis - vb0);
      if (vb0 > 0) build_state();
      for (int it = tid; it < ntok * nb * 4; it += kThreads) {
        const int q4 = it & 3, jt = it >> 2;
        const int j = jt % nb, tt = jt / nb;
        const int t = t_lo + tt, qb = t / BM, tl = t - qb * BM;
        const int c0 = vis[vb0 + j] * kTileKeys + q4 * 16;
        uint32_t bits = 0;
        if (c0 < a.tree_key_limit) {
          const int tb = c0 / BN;
          const int e = st[(qb - qb_lo) * ntb + tb];
          if (e < 0) {
            bits = 0xffffu;
          } else if (e > 0) {
            const int flat = tl * BN + (c0 - tb * BN);  // multiple of 16: never straddles a word
            bits = ((uint32_t)pl[e - 1 + (flat >> 5)] >> (flat & 31)) & 0xffffu;
          }
          const int valid = a.tree_key_limit - c0;
          if (valid < 16) bits &= (1u << valid) - 1u;
        }
        masks[(tt * a.vt_max + j) * 4 + q4] = (uint16_t)bits;
      }
      sync_lds();
      run_tiles(
          nb, false, [&](int j) { return P + vis[vb0 + j] * kTileKeys; }, [&](int) { return true; },
          [&](int j, int rt) -> uint64_t {
            int tt = row_tok[0];
#pragma unroll
            for (int r2 = 1; r2 < RT; ++r2) tt = (rt == r2) ? row_tok[r2] : tt;
            return *reinterpret_cast<const uint64_t*>(masks + (tt * a.vt_max + j) * 4);
          });
    }
  }

  // Epilogue.  Each wave stages its rows' O/l (input dtype) through its own
  // 8 KB of the (now idle) ring, row-major with a 16-byte-chunk XOR swizzle,
  // then stores whole rows: every store instruction writes 1 KB contiguous.
  if (!active) return;
  const int64_t TG = (int64_t)a.q_len * G;
  const int64_t base =
      ((int64_t)(b * a.num_kv_heads + kvh) * a.n_slots + slot) * TG + (int64_t)t_lo * G;
  unsigned char* stage = ring + wave * (kRowsPerWave * ROWB);
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const float l = row_sum4(l_run[rt]);
    const float inv = l > 0.f ? 1.f / l : 0.f;  // empty partial: O = 0, weight 0 in the combine
    const int r = wave * kRowsPerWave + rt * 16 + li;
    if (lg == 0 && r < rows) a.ws_ml[base + r] = make_float2(m_run[rt], l);
    const int rl = rt * 16 + li;
#pragma unroll
    for (int dt = 0; dt < DTILES; ++dt) {
      typedef T T4 __attribute__((ext_vector_type(4)));
      T4 v4;
#pragma unroll
      for (int i = 0; i < 4; ++i) v4[i] = (T)(o[dt][rt][i] * inv);
      const int chunk = (dt * 2 + (lg >> 1)) ^ (rl & (CPR - 1));
      *reinterpret_cast<T4*>(stage + rl * ROWB + chunk * 16 + (lg & 1) * 8) = v4;
    }
  }
  T* dst = static_cast<T*>(a.ws_o) + (base + wave * kRowsPerWave) * D;
  const int wave_rows = min(kRowsPerWave, rows - wave * kRowsPerWave);
#pragma unroll
  for (int k = 0; k < kRowsPerWave * CPR / 64; ++k) {
    const int idx = k * 64 + lane;
    const int rl = idx / CPR, c = idx % CPR;
    const i16x8 v = *reinterpret_cast<const i16x8*>(stage + rl * ROWB + ((c ^ (rl & (CPR - 1))) << 4));
    if (rl < wave_rows) *reinterpret_cast<i16x8*>(dst + (int64_t)rl * D + c * 8) = v;
  }
}

// Merge the n_slots partials of every row and write O.  Threads walk the
// workspace rows in order (coalesced 16-byte partial loads); 8 outputs per
// thread; the slot loop is branch-free (an empty partial has weight 0) so the
// loads of several slots are in flight together.
template <typename T, int D>
__global__ __launch_bounds__(256) void combine_kernel(const CombineArgs a) {
  constexpr int TPR = D / 8;
  const int64_t gtid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t TG = (int64_t)a.q_len * a.group;
  const int64_t row = gtid / TPR;  // over B*Hkv*TG
  const int part = (int)(gtid % TPR);
  if (row >= (int64_t)a.batch * a.num_kv_heads * TG) return;
  const int64_t bk = row / TG;
  const int R = (int)(row - bk * TG);
  const int t = R / a.group, g = R - t * a.group;
  const int kvh = (int)(bk % a.num_kv_heads), b = (int)(bk / a.num_kv_heads);
  const int h = kvh * a.group + g;
  const int64_t r0 = bk * a.n_slots * TG + R;
  const float2* ml = a.ws_ml + r0;
  const T* src = static_cast<const T*>(a.ws_o) + r0 * D + part * 8;
  const int64_t slot_stride = TG * D;
  typedef T T8 __attribute__((ext_vector_type(8)));

  // Running merge in batches of 8 slots: the 8 (m, l) pairs and 8 partial
  // vectors of a batch are loaded together, then folded into (M, L, acc)
  // with the same re-basing as the online softmax.
  float mx = -INFINITY, l = 0.f;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < a.n_slots; s0 += 8) {
    const int nb = min(8, a.n_slots - s0);
    float2 v[8];
    T8 x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int s = s0 + min(i, nb - 1);  // duplicates of the last slot get weight 0 below
      v[i] = ml[s * TG];
      x[i] = *reinterpret_cast<const T8*>(src + s * slot_stride);
    }
    float bm = mx;
#pragma unroll
    for (int i = 0; i < 8; ++i) bm = (i < nb) ? fmaxf(bm, v[i].x) : bm;
    if (bm != -INFINITY && bm != mx) {  // re-base the running sums on the new max
      const float alpha = (mx == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f((mx - bm) * a.scale_log2);
      l *= alpha;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] *= alpha;
      mx = bm;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // weight of partial s: l_s * 2^((m_s - M) * scale); 0 for an empty partial
      const float w = (i >= nb || v[i].x == -INFINITY) ? 0.f
                                                      : v[i].y * __builtin_amdgcn_exp2f((v[i].x - mx) * a.scale_log2);
      l += w;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += w * (float)x[i][e];
    }
  }
  // l == 0 (no visible key anywhere) gives 0/0 = NaN, as acc / l_i does in the reference.
  T8 out;
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = (T)(acc[i] / l);
  T* dst = static_cast<T*>(a.o) + b * a.sob + (int64_t)h * a.soh + (int64_t)t * a.som + part * 8;
  *reinterpret_cast<T8*>(dst) = out;
}

// ------------------------------------------------------------------- plan
struct Plan {
  int tpc, n_chunks, n_ptiles, tiles_per_split, n_splits, n_slots, n_items, items_per_xcd, grid;
  int nstage, vt_max, tree_key_limit;
  size_t lds_bytes, ws_acc_bytes, ws_ml_bytes;
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t lds_bytes_for(int head_dim, int nstage) {
  return (size_t)nstage * 2 * kTileKeys * head_dim * 2 + kMaskBytes + (kMaxTreeTiles + kMiscInts) * 4;
}

int env_int(const char* name, int dflt) {
  const char* s = getenv(name);
  if (s == nullptr || *s == 0) return dflt;
  return atoi(s);
}

// Decide tokens per chunk, prefix split size and LDS ring depth.
int make_plan(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len, int prefix_len, int head_dim,
              Plan* p) {
  const int G = num_heads / num_kv_heads;
  p->tpc = std::max(1, std::min(q_len, kRowsPerChunk / G));
  p->n_chunks = ceil_div(q_len, p->tpc);
  p->n_ptiles = ceil_div(prefix_len, kTileKeys);
  int cus = 256;
  if (device_cu_count(&cus) != TSFA_OK) return TSFA_ERR_DEVICE;
  const int64_t groups = (int64_t)batch * num_kv_heads * p->n_chunks;
  int tps = 0;
  if (p->n_ptiles > 0) {
    tps = env_int("TSFA_PREFIX_TILES_PER_SPLIT", 0);
    if (tps <= 0) {
      // Makespan model: workgroups run one per CU; a split of tps tiles costs
      // tps + 1 tile-times (tile + prologue/epilogue) and every extra slot of
      // partials costs a little combine traffic.
      double best = 1e30;
      for (int cand = 1; cand <= p->n_ptiles; ++cand) {
        const int64_t splits = ceil_div(p->n_ptiles, cand);
        if (cand > 1 && ceil_div(p->n_ptiles, cand - 1) == splits) continue;
        const int64_t items = groups * (splits + 1);
        const int64_t rounds = (items + cus - 1) / cus;
        const double cost = (double)rounds * (cand + 1) + 0.15 * (double)(splits + 1);
        if (cost < best - 1e-9) {
          best = cost;
          tps = cand;
        }
      }
    }
    tps = std::min(std::max(tps, 1), p->n_ptiles);
  }
  p->tiles_per_split = tps;
  p->n_splits = tps > 0 ? ceil_div(p->n_ptiles, tps) : 0;
  p->n_slots = p->n_splits + 1;
  const int64_t items = groups * p->n_slots;
  if (items > (int64_t)INT32_MAX / 2) return TSFA_ERR_UNSUPPORTED;
  p->n_items = (int)items;
  p->items_per_xcd = ceil_div(p->n_items, 8);
  p->grid = p->items_per_xcd * 8;
  int max_lds = 65536;
  if (device_max_lds_per_block(&max_lds) != TSFA_OK) return TSFA_ERR_DEVICE;
  int nstage = env_int("TSFA_RING_STAGES", 4);
  if (nstage != 2 && nstage != 4) nstage = 4;
  if (lds_bytes_for(head_dim, nstage) > (size_t)max_lds) nstage = 2;
  if (lds_bytes_for(head_dim, nstage) > (size_t)max_lds) return TSFA_ERR_UNSUPPORTED;
  p->nstage = nstage;
  p->lds_bytes = lds_bytes_for(head_dim, nstage);
  p->vt_max = kMaskBytes / (p->tpc * 8);
  p->tree_key_limit = kv_len - prefix_len;  // refined by the caller with n_tree_blocks*BN
  const size_t rows = (size_t)batch * num_heads * q_len;
  p->ws_acc_bytes = align256(rows * p->n_slots * head_dim * 2);
  p->ws_ml_bytes = align256(rows * p->n_slots * 8);
  return TSFA_OK;
}

template <typename T, int D, int NSTAGE>
int launch_split(const SplitArgs& args, const Plan& p, hipStream_t stream) {
  constexpr int WAVES = 8;
  static bool attr_set = false;  // benign race: idempotent attribute write
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&split_kernel<T, D, NSTAGE, WAVES>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)p.lds_bytes) != hipSuccess)
      return TSFA_ERR_LAUNCH;
    attr_set = true;
  }
  hipLaunchKernelGGL((split_kernel<T, D, NSTAGE, WAVES>), dim3(p.grid), dim3(WAVES * 64), p.lds_bytes, stream,
                     args);
  return hipGetLastError() == hipSuccess ? TSFA_OK : TSFA_ERR_LAUNCH;
}

// Measurement hook: events recorded around the split kernel (per thread).
thread_local hipEvent_t g_split_begin = nullptr;
thread_local hipEvent_t g_split_end = nullptr;

template <typename T, int D>
int launch_all(const SplitArgs& sa, const CombineArgs& ca, const Plan& p, hipStream_t stream) {
  if (g_split_begin != nullptr && hipEventRecord(g_split_begin, stream) != hipSuccess) return TSFA_ERR_LAUNCH;
  int st = (p.nstage == 4) ? launch_split<T, D, 4>(sa, p, stream) : launch_split<T, D, 2>(sa, p, stream);
  if (st != TSFA_OK) return st;
  if (g_split_end != nullptr && hipEventRecord(g_split_end, stream) != hipSuccess) return TSFA_ERR_LAUNCH;
  const int64_t threads = (int64_t)ca.batch * ca.num_kv_heads * ca.q_len * ca.group * (D / 8);
  const unsigned blocks = (unsigned)((threads + 255) / 256);
  hipLaunchKernelGGL((combine_kernel<T, D>), dim3(blocks), dim3(256), 0, stream, ca);
  return hipGetLastError() == hipSuccess ? TSFA_OK : TSFA_ERR_LAUNCH;
}

}  // namespace fwd
}  // namespace tsfa

using namespace tsfa;
using namespace tsfa::fwd;

extern "C" int tsfa_fwd_check_args(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len,
                                   int prefix_len, int n_q_blocks, int n_tree_blocks, int gqa_group_size,
                                   int block_m, int block_n, int head_dim, int dtype) {
  if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || q_len < 0) return TSFA_ERR_INVALID_ARGUMENT;
  if (block_m <= 0 || block_n <= 0) return TSFA_ERR_INVALID_ARGUMENT;          // tree_sparse_flashattn.py:87-88
  if (prefix_len < 0 || kv_len < prefix_len) return TSFA_ERR_INVALID_ARGUMENT;  // eagle_tree_sparse_bridge.py:91-93
  if (gqa_group_size <= 0 || num_heads != gqa_group_size * num_kv_heads) return TSFA_ERR_INVALID_ARGUMENT;
  if (n_q_blocks != ceil_div(q_len, block_m) || n_tree_blocks != ceil_div(q_len, block_n))
    return TSFA_ERR_INVALID_ARGUMENT;
  if (dtype != TSFA_DTYPE_FP16 && dtype != TSFA_DTYPE_BF16) return TSFA_ERR_UNSUPPORTED;
  if (head_dim != 64 && head_dim != 128) return TSFA_ERR_UNSUPPORTED;
  if (block_n % 16 != 0) return TSFA_ERR_UNSUPPORTED;
  if (gqa_group_size > kRowsPerChunk) return TSFA_ERR_UNSUPPORTED;
  const int64_t tree_limit = std::min<int64_t>((int64_t)n_tree_blocks * block_n, (int64_t)kv_len - prefix_len);
  if (tree_limit > (int64_t)kMaxTreeTiles * kTileKeys) return TSFA_ERR_UNSUPPORTED;
  // tree state table [q-blocks per chunk][n_tree_blocks] must fit the smallest LDS ring
  const int tpc = std::max(1, std::min(q_len, kRowsPerChunk / gqa_group_size));
  const int64_t nqbc = (int64_t)(tpc > 0 ? (tpc - 1) / block_m : 0) + 2;
  if (nqbc * n_tree_blocks * 4 > (int64_t)2 * 2 * kTileKeys * head_dim * 2) return TSFA_ERR_UNSUPPORTED;
  return TSFA_OK;
}

extern "C" size_t tsfa_fwd_workspace_bytes(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len,
                                           int prefix_len, int head_dim) {
  if (batch <= 0 || q_len <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0) return 0;
  Plan p;
  if (make_plan(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, head_dim, &p) != TSFA_OK) return 0;
  return p.ws_acc_bytes + p.ws_ml_bytes;
}

extern "C" int tsfa_fwd_plan(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len, int prefix_len,
                             int head_dim, int32_t* out6) {
  if (out6 == nullptr || batch <= 0 || q_len <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
    return TSFA_ERR_INVALID_ARGUMENT;
  Plan p;
  const int st = make_plan(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, head_dim, &p);
  if (st != TSFA_OK) return st;
  out6[0] = p.n_splits;
  out6[1] = p.tiles_per_split;
  out6[2] = p.tpc;
  out6[3] = p.n_chunks;
  out6[4] = p.grid;
  out6[5] = p.nstage;
  return TSFA_OK;
}

extern "C" int tsfa_fwd(const void* q, const void* k, const void* v, void* o, const int32_t* row_ptr,
                        const int32_t* col_idx, const int8_t* blk_type, const int32_t* mixed_mask_payload,
                        const int32_t* mixed_mask_offset, const int64_t* meta_seq_stride, const int64_t* strides,
                        float sm_scale, int batch, int num_heads, int num_kv_heads, int q_len, int kv_len,
                        int prefix_len, int n_q_blocks, int n_tree_blocks, int gqa_group_size, int block_m,
                        int block_n, int head_dim, int dtype, void* workspace, size_t workspace_bytes,
                        tsfa_stream_t stream_) {
  int st = tsfa_fwd_check_args(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, n_q_blocks,
                               n_tree_blocks, gqa_group_size, block_m, block_n, head_dim, dtype);
  if (st != TSFA_OK) return st;
  if (batch == 0 || q_len == 0) return TSFA_OK;
  if (strides == nullptr || meta_seq_stride == nullptr) return TSFA_ERR_INVALID_ARGUMENT;
  if (q == nullptr || k == nullptr || v == nullptr || o == nullptr || row_ptr == nullptr)
    return TSFA_ERR_INVALID_ARGUMENT;
  for (int i = 0; i < 4; ++i) {
    if (strides[4 * i + 3] != 1) return TSFA_ERR_UNSUPPORTED;  // contiguous head_dim
    for (int j = 0; j < 3; ++j)
      if (strides[4 * i + j] % 8 != 0) return TSFA_ERR_UNSUPPORTED;  // 16-byte aligned rows
  }
  const void* ptrs[4] = {q, k, v, o};
  for (const void* ptr : ptrs)
    if (reinterpret_cast<uintptr_t>(ptr) % 16 != 0) return TSFA_ERR_UNSUPPORTED;
  for (int i = 0; i < 5; ++i)
    if (meta_seq_stride[i] < 0) return TSFA_ERR_INVALID_ARGUMENT;

  Plan p;
  st = make_plan(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, head_dim, &p);
  if (st != TSFA_OK) return st;
  p.tree_key_limit = (int)std::min<int64_t>((int64_t)n_tree_blocks * block_n, (int64_t)kv_len - prefix_len);
  if (workspace == nullptr || workspace_bytes < p.ws_acc_bytes + p.ws_ml_bytes) return TSFA_ERR_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0) return TSFA_ERR_WORKSPACE;

  SplitArgs sa;
  sa.q = q;
  sa.k = k;
  sa.v = v;
  sa.row_ptr = row_ptr;
  sa.col_idx = col_idx;
  sa.blk_type = blk_type;
  sa.payload = mixed_mask_payload;
  sa.offset = mixed_mask_offset;
  sa.ms_row_ptr = meta_seq_stride[0];
  sa.ms_col_idx = meta_seq_stride[1];
  sa.ms_blk_type = meta_seq_stride[2];
  sa.ms_payload = meta_seq_stride[3];
  sa.ms_offset = meta_seq_stride[4];
  sa.sqb = strides[0];
  sa.sqh = strides[1];
  sa.sqm = strides[2];
  sa.skb = strides[4];
  sa.skh = strides[5];
  sa.skn = strides[6];
  sa.svb = strides[8];
  sa.svh = strides[9];
  sa.svn = strides[10];
  sa.scale_log2 = sm_scale * 1.4426950408889634f;
  sa.num_kv_heads = num_kv_heads;
  sa.group = gqa_group_size;
  sa.q_len = q_len;
  sa.kv_len = kv_len;
  sa.prefix_len = prefix_len;
  sa.block_m = block_m;
  sa.block_n = block_n;
  sa.n_tree_blocks = n_tree_blocks;
  sa.tpc = p.tpc;
  sa.n_chunks = p.n_chunks;
  sa.tiles_per_split = p.tiles_per_split;
  sa.n_ptiles = p.n_ptiles;
  sa.n_slots = p.n_slots;
  sa.n_items = p.n_items;
  sa.items_per_xcd = p.items_per_xcd;
  sa.tree_key_limit = p.tree_key_limit;
  sa.vt_max = p.vt_max;
  sa.ws_o = workspace;
  sa.ws_ml = reinterpret_cast<float2*>(static_cast<char*>(workspace) + p.ws_acc_bytes);

  CombineArgs ca;
  ca.o = o;
  ca.sob = strides[12];
  ca.soh = strides[13];
  ca.som = strides[14];
  ca.scale_log2 = sa.scale_log2;
  ca.batch = batch;
  ca.num_heads = num_heads;
  ca.num_kv_heads = num_kv_heads;
  ca.group = gqa_group_size;
  ca.q_len = q_len;
  ca.n_slots = p.n_slots;
  ca.ws_o = sa.ws_o;
  ca.ws_ml = sa.ws_ml;

  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (dtype == TSFA_DTYPE_BF16)
    return head_dim == 128 ? launch_all<__bf16, 128>(sa, ca, p, stream) : launch_all<__bf16, 64>(sa, ca, p, stream);
  return head_dim == 128 ? launch_all<_Float16, 128>(sa, ca, p, stream) : launch_all<_Float16, 64>(sa, ca, p, stream);
}

extern "C" int tsfa_fwd_set_split_events(void* begin, void* end) {
  if ((begin == nullptr) != (end == nullptr)) return TSFA_ERR_INVALID_ARGUMENT;
  g_split_begin = static_cast<hipEvent_t>(begin);
  g_split_end = static_cast<hipEvent_t>(end);
  return TSFA_OK;
}
