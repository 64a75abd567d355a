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
//     a workgroup owns a chunk of 128 consecutive rows;
//   * keys move in units of 32.  The prefix units are cut into runs (split-KV:
//     a small tree still spreads the prefix over all 256 CUs) and one more
//     workgroup per chunk runs the tree units (or, when that would add a
//     round of workgroups and the tree is short, the chunk's last run does):
//     it expands the CSR rows of the chunk's q-blocks into per-token 32-bit
//     visibility words for every tree unit that holds a visible key, and
//     skips the rest (ZERO blocks are never loaded);
//   * work items map to XCDs in contiguous ranges, so the row chunks that read
//     the same K/V units share an XCD's L2 (K/V loads carry the non-temporal
//     hint when at most two chunks share a unit); plans of a few rounds
//     dispatch each XCD's long items first;
//   * a workgroup is 8 waves, two per SIMD: two key streams x four row groups
//     of 32 rows.  Stream s takes every other unit of the workgroup's run
//     through its own LDS ring, filled by global_load_lds (HBM -> LDS, 16 B
//     per lane, no VGPR staging) with the stream's four waves moving a
//     quarter each; one barrier per step.  The two waves sharing a SIMD
//     belong to different streams, so one's softmax overlaps the other's
//     MFMAs;
//   * S^T = K Q^T and O^T += V^T P^T run on v_mfma_f32_32x32x16_{bf16,f16}:
//     a lane holds one query row in both, so the softmax statistics and the
//     rescale of O never leave the lane; V^T operands come from
//     ds_read_b64_tr_b16, so V is never transposed in memory.  exp2 with
//     sm_scale*log2(e) folded into one FMA; the running max is only re-based
//     when a score exceeds it by more than 2^8 (rescaling is exact for any
//     consistent reference point), which skips the O rescale on almost every
//     unit;
//   * at the end the two streams' (m, l, O) merge in LDS and the workgroup writes
//     one partial per row (O/l in the input dtype, fp32 (m, l)); a second
//     kernel merges the partials (log-sum-exp) and writes O, each XCD merging
//     the chunks its split workgroups wrote (the partials come from its L2).

#include <math.h>
#include <stdlib.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>

#include "tsfa_internal.h"

namespace tsfa {
namespace fwd {

// kWaves, kMaxRows, kUnitKeys, kRingBytes, kMaskWords, kMaxTreeUnits and
// kMiscInts come from tsfa_plan.h (the planner sizes the grid and LDS by them)
constexpr float kRescaleLog2 = 8.0f;

// Per-workgroup timestamps for timeline measurements: compiled in only with
// -DTSFA_STAMPS (a separate measurement build); TSFA_STAMP is empty otherwise.
#ifdef TSFA_STAMPS
__device__ unsigned long long g_stamps[4096 * 64];
#define TSFA_STAMP(k)                                                                      \
  do {                                                                                     \
    if (threadIdx.x == 0) g_stamps[(size_t)blockIdx.x * 64 + (k)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
// slot k + wave, written by lane 0 of every wave
#define TSFA_STAMPW(k)                                                                               \
  do {                                                                                               \
    if ((threadIdx.x & 63) == 0)                                                                     \
      g_stamps[(size_t)blockIdx.x * 64 + (k) + (threadIdx.x >> 6)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
// Per-wave cycle sums of loop phases (s_memtime deltas; each reading waits
// for the wave's outstanding LDS/scalar loads, so the instrumented library perturbs the loop).
__device__ unsigned long long g_cyc[4096 * 32];
#define TSFA_CYC_DECL unsigned long long cyc_prev = __builtin_amdgcn_s_memtime(), cyc_acc[4] = {0, 0, 0, 0};
#define TSFA_CYC(k)                                              \
  do {                                                           \
    const unsigned long long cyc_now = __builtin_amdgcn_s_memtime(); \
    cyc_acc[k] += cyc_now - cyc_prev;                            \
    cyc_prev = cyc_now;                                          \
  } while (0)
#define TSFA_CYC_STORE                                                                         \
  do {                                                                                         \
    if ((threadIdx.x & 63) == 0)                                                               \
      for (int k_ = 0; k_ < 4; ++k_) g_cyc[(size_t)blockIdx.x * 32 + (threadIdx.x >> 6) * 4 + k_] = cyc_acc[k_]; \
  } while (0)
#else
#define TSFA_STAMP(k) \
  do {            \
  } while (0)
#define TSFA_STAMPW(k) \
  do {             \
  } while (0)
#define TSFA_CYC_DECL
#define TSFA_CYC(k) \
  do {          \
  } while (0)
#define TSFA_CYC_STORE \
  do {             \
  } while (0)
#endif

struct CombineArgs {
  void* o;
  int64_t sob, soh, som;
  float* lse;  // optional [B, Hq, q_len] natural-log log-sum-exp of each row's scaled scores
  float scale_log2;
  int batch, num_heads, num_kv_heads, group, q_len, n_slots;
  const void* ws_o;
  const float2* ws_ml;
  // Workspace rows [xcd_row[x], xcd_row[x + 1]) are merged by the blocks of
  // XCD x (block ids with x = id % 8), the XCD whose split workgroups wrote
  // most of their partials.
  int64_t xcd_row[9];
};

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
  float scale_log2;  // |sm_scale| * log2(e), never 0
  int neg_q;         // sm_scale < 0: Q enters negated (scores keep their sign)
  int num_kv_heads, group, q_len, kv_len, prefix_len, block_m, block_n, n_tree_blocks;
  int n_chunks, units_per_split, n_pu, n_slots, n_items, items_per_xcd;
  FastDiv fd_chunks, fd_slots, fd_kvh, fd_group;  // n_chunks, n_slots, num_kv_heads, group
  FastDiv fd_P, fd_Np, fd_Nt;                     // item order: n_chunks*n_slots, its prefix and tree items
  int tree_key_limit;  // min(n_tree_blocks*BN, kv_len - prefix_len)
  int vt_max;          // tree units per mask batch
  void* ws_o;          // [B*Hkv][n_slots][q_len*G][D] partial O / l in the input dtype
  float2* ws_ml;       // [B*Hkv][n_slots][q_len*G] (m, l) of each partial
  // Paged K/V (split_kernel<..., PAGED = true> only; k and v unused).
  const void* kv_cache;
  const int32_t* kv_indptr;   // [B + 1] page-list offsets into kv_indices, or null
  const int32_t* kv_indices;  // page ids
  int64_t cps, css, crs, chs; // cache strides (elements): page, K/V slot, row, kv head
  int pt_stride;              // kv_indptr null: sequence b's list starts at b * pt_stride
  int n_indices;              // entries of kv_indices (< 2^31)
  int page_shift, n_pages;
  int kv_nt;  // K/V loads non-temporal (each unit read by at most two row chunks)
  int cache32;                // paged cache below 4 GB (selects the 32-bit-offset kernel)
  uint32_t cps_b32, crs_b32;  // its page and row strides in bytes
  int item_order;  // within an XCD: 0 natural, 1 prefix runs first, 2 tree items first
  int fold_tree;   // no tree items: the last prefix split of each chunk also runs the tree units
  // One-slot plans with O contiguous [B, Hq, q_len, D] and no LSE asked: the
  // split kernel writes O itself (ws_o is O; split_kernel<..., FAST | 4>)
  // and no combine runs.  Host-side only.
  int direct_out;
};


// 16-byte-chunk XOR swizzles of the K and V LDS tiles (row = key in unit).
// K: the 16 keys of one quarter-wave of an MFMA A-operand read land on 16
// distinct bank groups.  V: the 4 keys x 64 bytes a half-wave of
// ds_read_b64_tr_b16 touches land on 4 distinct 64-byte bank windows.
template <int D> __device__ inline int swz_k(int key) { return D == 128 ? (key & 15) : ((key >> 1) & 7); }
template <int D> __device__ inline int swz_v(int key) { return D == 128 ? ((key & 3) << 2) : (((key >> 1) & 1) << 2); }

// 16 bytes per lane HBM -> LDS (global_load_lds_dwordx4): lane i's bytes land
// at LDS address lds_base + 16*i.  Issued as inline asm so the compiler does
// not treat every later LDS read as aliasing the in-flight copy (it would
// insert vmcnt(0) before them and serialise the prefetch); completion is
// ordered explicitly by wait_units().  dma16_s takes a scalar base and a
// 32-bit lane offset (no per-lane 64-bit address arithmetic); NT marks the
// load non-temporal (streamed K/V that at most one other workgroup reads:
// measured 19.8 -> 18.6 us per call on the Llama-3-8B decode shape, and 2 %
// slower on the 70B shape, where 16 row chunks re-read each K/V line from
// the L2).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is reserved; the clobber documents the write
__device__ inline void dma16(const void* src, uint32_t lds_in) {
  const uint32_t lds_base = __builtin_amdgcn_readfirstlane(lds_in);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(lds_base)
               : "memory", "m0");
}
// 4 bytes per lane HBM -> LDS (global_load_lds_dword): active lane i's dword
// lands at lds_base + 4*i; inactive lanes write nothing.  Small reads
// (page ids) that complete in order with the ring's unit loads.
__device__ inline void dma4(const void* src, uint32_t lds_in) {
  const uint32_t lds_base = __builtin_amdgcn_readfirstlane(lds_in);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
               :
               : "v"(src), "s"(lds_base)
               : "memory", "m0");
}
// A wave-uniform pointer stated as such to the compiler: the "s" operand of
// the loads below must be an SGPR pair, and a base it cannot prove uniform
// would otherwise be handed over in VGPRs (rejected by the assembler).
__device__ inline const void* uniform_ptr(const void* p) {
  const uint64_t u = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo);
}
template <bool NT = false>
__device__ inline void dma16_s(const void* sbase_in, uint32_t voff, uint32_t lds_in) {
  const void* sbase = uniform_ptr(sbase_in);
  const uint32_t lds_base = __builtin_amdgcn_readfirstlane(lds_in);
  if constexpr (NT)
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt"
                 :
                 : "v"(voff), "s"(sbase), "s"(lds_base)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(sbase), "s"(lds_base)
                 : "memory", "m0");
}
// N loads of 1 KB (N = 4, 2 or 1) with one scalar base and one M0: load i goes
// to LDS m0v + i KB and reads global sbase + off[i] + i KB -- the
// instruction's immediate offset applies to the LDS address as well as the
// global one (checked on gfx950), so consecutive LDS KBs need no M0 update.
template <int N, bool NT>
__device__ inline void dma_rows(const void* sbase_in, const uint32_t (&off)[N], uint32_t m0v_in) {
  static_assert(N == 4 || N == 2 || N == 1, "loads per wave and unit");
  const void* sbase = uniform_ptr(sbase_in);
  const uint32_t m0v = __builtin_amdgcn_readfirstlane(m0v_in);
  if constexpr (N == 1 && NT)
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %2 nt"
                 :
                 : "v"(off[0]), "s"(m0v), "s"(sbase)
                 : "memory", "m0");
  else if constexpr (N == 1)
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %2"
                 :
                 : "v"(off[0]), "s"(m0v), "s"(sbase)
                 : "memory", "m0");
  else if constexpr (N == 4 && NT)
    asm volatile("s_mov_b32 m0, %4\n\ts_nop 0\n\t"
                 "global_load_lds_dwordx4 %0, %5 nt\n\tglobal_load_lds_dwordx4 %1, %5 offset:1024 nt\n\t"
                 "global_load_lds_dwordx4 %2, %5 offset:2048 nt\n\tglobal_load_lds_dwordx4 %3, %5 offset:3072 nt"
                 :
                 : "v"(off[0]), "v"(off[1]), "v"(off[2]), "v"(off[3]), "s"(m0v), "s"(sbase)
                 : "memory", "m0");
  else if constexpr (N == 4)
    asm volatile("s_mov_b32 m0, %4\n\ts_nop 0\n\t"
                 "global_load_lds_dwordx4 %0, %5\n\tglobal_load_lds_dwordx4 %1, %5 offset:1024\n\t"
                 "global_load_lds_dwordx4 %2, %5 offset:2048\n\tglobal_load_lds_dwordx4 %3, %5 offset:3072"
                 :
                 : "v"(off[0]), "v"(off[1]), "v"(off[2]), "v"(off[3]), "s"(m0v), "s"(sbase)
                 : "memory", "m0");
  else if constexpr (NT)
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\t"
                 "global_load_lds_dwordx4 %0, %3 nt\n\tglobal_load_lds_dwordx4 %1, %3 offset:1024 nt"
                 :
                 : "v"(off[0]), "v"(off[1]), "s"(m0v), "s"(sbase)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\t"
                 "global_load_lds_dwordx4 %0, %3\n\tglobal_load_lds_dwordx4 %1, %3 offset:1024"
                 :
                 : "v"(off[0]), "v"(off[1]), "s"(m0v), "s"(sbase)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

template <int N> __device__ inline void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// Wait until at most k units (LPU loads each) of this wave are in flight.
template <int LPU, int K> __device__ inline void wait_units(int k) {
  if constexpr (K == 0) {
    vm_wait<0>();
  } else {
    if (k >= K) {
      vm_wait<K * LPU>();
      return;
    }
    wait_units<LPU, K - 1>(k);
  }
}

// Workgroup barrier that also orders LDS accesses (compiler and hardware).
__device__ inline void sync_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ inline void sync_all() { asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ inline uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(const TSFA_LDS void*)p; }
// LDS reads at a 32-bit LDS byte address (no generic-pointer base arithmetic).
template <typename V> __device__ inline V lds_ld(uint32_t addr) { return *(const TSFA_LDS V*)(uintptr_t)addr; }
__device__ inline i16x4 lds_tr(uint32_t addr) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((TSFA_LDS i16x4*)(uintptr_t)addr);
}

template <typename V, typename U> __device__ inline V bit_cast(U u) { return __builtin_bit_cast(V, u); }

// max(a, b, c) in one v_max3_f32.  fmaxf would first quiet each operand the
// compiler cannot prove canonical (an MFMA result), one extra VALU op apiece;
// scores are never signaling NaNs.
__device__ inline float max3f(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Sum over lanes {l, l^32} (one gfx950 row-swap permute, no LDS).
__device__ inline float pair_sum(float x) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

// Loads [u_lo, u_lo + NL) of one half of a unit whose rows may reach past
// kv_len, or whose row stride is below D: per-lane rows clamped to kv_len - 1
// (those keys are masked) from a scalar base at key0 with 32-bit lane
// offsets (a lane's row is at most 31 rows further and row strides stay below
// 2^26 elements).  The lane index passes through an empty asm: this runs at
// most once per run, and lane terms hoisted out of the unit loop would hold
// registers for the whole loop.
template <typename T, int D, bool IS_V, int NL>
__device__ inline void dma_tail(const T* base, int64_t stride, uint32_t lds_dst, int key0, int kv_len, int lane,
                                int u_lo) {
  constexpr int CPR = D / 8;
  constexpr int RPL = 64 / CPR;
  int ln_ = lane;
  asm volatile("" : "+v"(ln_));
  const char* rowp = reinterpret_cast<const char*>(base + (int64_t)key0 * stride);
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int u = u_lo + i;
    const int row = u * RPL + ln_ / CPR, pos = ln_ % CPR;
    const uint32_t rel = (uint32_t)(min(key0 + row, kv_len - 1) - key0);
    const int sw = IS_V ? swz_v<D>(row) : swz_k<D>(row);
    dma16_s(rowp, rel * (uint32_t)stride * 2u + (uint32_t)((pos ^ sw) << 4), lds_dst + u * 1024);
  }
}

// Paged K/V (FlashInfer's [pages, 2, page_size, Hkv, D] cache, the serving
// layout of benchmark.py:67-91, or any other strides): key `key` of sequence
// b lives in page list[key >> page_shift] at row key & (page_size - 1), K in
// slot 0 and V in slot 1 of the page.  The page list of sequence b starts at
// kv_indices[kv_indptr[b]] (CSR, FlashInfer's form) or, without kv_indptr,
// at kv_indices[b * pt_stride] (a dense [B, pages] table).  Page-table reads
// go through the scalar cache (the addresses are wave-uniform) and are
// clamped, index and page id both, so no table content can send a load out
// of the cache.
__device__ inline int ld_uniform(const int32_t* p, int64_t i) {
  typedef const __attribute__((address_space(4))) int32_t CI;
  return ((CI*)p)[i];
}
// Pages of a wave's DMA share of the unit at key0 (keys kw .. kw + 15, kw =
// key0 + u_lo*RPL, clamped to kv_len - 1): list positions pg0 <= pg1 <= pg0+1.
template <int D, int NL>
__device__ inline void share_pages(const SplitArgs& a, int key0, int u_lo, int& pg0, int& pg1) {
  constexpr int RPL = 64 / (D / 8);
  const int kw = key0 + u_lo * RPL;
  pg0 = min(kw, a.kv_len - 1) >> a.page_shift;
  pg1 = min(kw + NL * RPL - 1, a.kv_len - 1) >> a.page_shift;
}
// Raw page-table entry at list position pg (position clamped to kv_indices,
// which the host keeps below 2^31 entries).
__device__ inline int page_entry(const SplitArgs& a, int pt_base, int pg) {
  return ld_uniform(a.kv_indices, min(max(pt_base + pg, 0), a.n_indices - 1));
}
__device__ inline int64_t clamp_page(const SplitArgs& a, int raw) { return (int64_t)min(max(raw, 0), a.n_pages - 1); }

// dma_half over the paged cache (hbase: the kv head's K or V at page 0, row
// 0; pid0/pid1: the pages at list positions pg0/pg1 of share_pages).  The
// loads of one wave cover NL*RPL <= 16 consecutive keys, so with pages of
// 16 keys or more they touch at most two pages.  A share inside one page and
// below kv_len (every prefix unit with page_size >= 16) is addressed like
// the contiguous fast path: one scalar row base, the lane offsets built from
// the cache's row stride.  Otherwise each 1 KB load takes a scalar base when
// its RPL rows sit in one page below kv_len and per-lane clamped addresses
// when it straddles a page boundary or reaches past kv_len (those keys are
// masked).
template <typename T, int D, bool IS_V, int NL, bool C32>
__device__ inline void dma_half_paged(const T* hbase, const SplitArgs& a, int64_t pid0, int64_t pid1, int pg0,
                                      uint32_t lds_dst, int key0, int lane, int u_lo, const uint32_t* loff,
                                      bool nt) {
  constexpr int CPR = D / 8;
  constexpr int RPL = 64 / CPR;
  constexpr int NOFF = IS_V ? 1 : (D == 128 ? 4 : 2);
  static_assert(NL * RPL <= 16, "a wave's share of a unit spans at most two pages of 16+ keys");
  const int kv_len = a.kv_len, ps = a.page_shift, pmask = (1 << ps) - 1;
  const int kw = key0 + u_lo * RPL;  // first key of the wave's share
  auto row_ptr = [&](int64_t pid, int key) { return hbase + pid * a.cps + (int64_t)(key & pmask) * a.crs; };
  if (kw + NL * RPL <= kv_len && (kw & pmask) + NL * RPL <= pmask + 1) {
    // C32 (a cache below 4 GB): 32-bit byte offsets from the head's base,
    // fewer scalar products and live 64-bit values in the issue path
    const char* rowp;
    int64_t step;
    if constexpr (C32) {
      rowp = reinterpret_cast<const char*>(hbase) + ((uint32_t)pid0 * a.cps_b32 + (uint32_t)(kw & pmask) * a.crs_b32);
      step = (int64_t)(RPL * a.crs_b32);
    } else {
      rowp = reinterpret_cast<const char*>(row_ptr(pid0, kw));
      step = (int64_t)RPL * a.crs * 2;
    }
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int u = u_lo + i;
      if (nt)
        dma16_s<true>(rowp, loff[u % NOFF], lds_dst + u * 1024);
      else
        dma16_s<false>(rowp, loff[u % NOFF], lds_dst + u * 1024);
      rowp += step;
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int u = u_lo + i;
    const int r0 = kw + i * RPL;  // first key of this load
    if (r0 + RPL <= kv_len && (r0 & pmask) + RPL <= pmask + 1) {
      dma16_s(row_ptr((r0 >> ps) == pg0 ? pid0 : pid1, r0), loff[u % NOFF], lds_dst + u * 1024);
    } else {
      const int row = u * RPL + lane / CPR, pos = lane % CPR;
      const int key = min(key0 + row, kv_len - 1);
      const int sw = IS_V ? swz_v<D>(row) : swz_k<D>(row);
      dma16(row_ptr((key >> ps) == pg0 ? pid0 : pid1, key) + ((pos ^ sw) << 3), lds_dst + u * 1024);
    }
  }
}

// Lane offsets (bytes from the load's first key row) of dma_half's fast path.
template <int D, bool IS_V> __device__ inline uint32_t dma_lane_off(int u, int64_t stride, int lane) {
  constexpr int CPR = D / 8;
  constexpr int RPL = 64 / CPR;
  const int lr = lane / CPR, pos = lane % CPR;
  const int sw = IS_V ? swz_v<D>(u * RPL + lr) : swz_k<D>(u * RPL + lr);
  return (uint32_t)(lr * stride * 2 + ((pos ^ sw) << 4));
}


// Work item of this workgroup.  XCD x (block id % 8) owns the items
// [x*ipx, (x+1)*ipx) of the natural order item = chunk + n_chunks * (slot +
// n_slots * bk) (so the row chunks sharing K/V units share the XCD's L2).
// With item_order 1 the workgroups of an XCD take its prefix runs first and
// its tree items last (2: the reverse): with few rounds, like items then
// run side by side and the rounds pack (the 16-sequence decode shape, 3
// rounds: 86.6 -> 78.6 us per call); with many rounds the natural order,
// which spreads the tree items over the rounds, measured ~1 % faster.
// Returns -1 for the padding blocks of the last XCD.
__device__ inline int work_item(const SplitArgs& a) {
  const int x = blockIdx.x & 7, j = blockIdx.x >> 3;
  const int lo = x * a.items_per_xcd, hi = min(lo + a.items_per_xcd, a.n_items);
  if (lo + j >= hi) return -1;
  if (a.n_slots < 2 || a.item_order == 0) return lo + j;
  const int P = a.n_chunks * a.n_slots, Nt = a.n_chunks, Np = P - Nt;
  auto before = [&](int i) { return (int)fdiv(i, a.fd_P) * Np + min((int)frem(i, a.fd_P), Np); };  // prefix items before item i
  auto kth_prefix = [&](int k) { return (int)fdiv(k, a.fd_Np) * P + (int)frem(k, a.fd_Np); };
  auto kth_tree = [&](int k) { return (int)fdiv(k, a.fd_Nt) * P + Np + (int)frem(k, a.fd_Nt); };
  const int plo = before(lo), np = before(hi) - plo, nt = hi - lo - np;
  if (a.item_order == 2) return j < nt ? kth_tree(lo - plo + j) : kth_prefix(plo + j - nt);
  return j < np ? kth_prefix(plo + j) : kth_tree(lo - plo + j - np);
}

// The steady refills of a run with unchecked ring steps (FastSeq<true>):
// init(t) points at the stream's t-th unit, next() requests it and moves to
// the following one.  FastSeq<false> marks runs without them.
template <bool V, typename I = int, typename N = int> struct FastSeq {
  static constexpr bool value = V;
  I init;
  N next;
};

// S key streams of kWaves/S waves: a chunk is 32*kWaves/S rows.  FAST (every
// prefix unit within kv_len; 1: plain loads, 2: non-temporal K/V loads; paged
// runs choose the hint at run time and take 1): prefix runs skip the per-unit
// mask test (only a run's last unit can be the prefix's partial one, tested
// once after the loop), contiguous ring runs issue every unit by the
// run-base path, and the steady ring steps use a fixed wait count.
template <typename T, int D, int S, bool PAGED, bool C32 = false, int FAST = 0>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void split_kernel(const SplitArgs a) {
  constexpr int FM = FAST & 3;              // unchecked ring steps: 0 off, 1 plain, 2 non-temporal loads
  constexpr bool DIRECT = (FAST & 4) != 0;  // one-slot plan: write O, no combine
  constexpr bool PTAB = PAGED && FM != 0 && (FAST & 8) != 0;  // paged: steady refills from the LDS page-id table
  typedef typename Mma<T>::vec8 V8;
  constexpr int RG = kWaves / S;             // row groups (waves per stream)
  constexpr int ROWS = 32 * RG;              // rows per chunk
  constexpr int ROWB = D * 2;                // bytes of one key row
  constexpr int HALF = kUnitKeys * ROWB;     // K (or V) bytes of one unit
  constexpr int SB = 2 * HALF;               // ring stage
  constexpr int RB = kRingBytes / S;         // ring of one stream
  constexpr int NS = RB / SB;                // stages per stream
  constexpr int LPH = HALF / 1024;           // 1 KB loads per half
  constexpr int LPU = 2 * LPH / RG;          // loads per unit per wave
  constexpr int QROWS = ROWS / S;            // Q rows staged in each stream's ring
  constexpr int QS = QROWS * ROWB / SB;      // ring stages they occupy at start
  constexpr int KSTEPS = D / 16;
  constexpr int DT = D / 32;
  static_assert(S == 1 || S == 2, "streams");
  static_assert(kWaves == 8, "two waves per SIMD: w and w + 4");
  static_assert(NS >= 4 && (NS & (NS - 1)) == 0 && LPU >= 1 && LPU * (NS - 2) < 64 && LPH % (RG / 2) == 0,
                "ring geometry");
  static_assert(QS >= 1 && QS < NS && QROWS * ROWB == QS * SB, "Q staging");
  static_assert(S == 1 || (kWaves * (DT / 2) * 4 * 64 * 16 <= kRingBytes && S * ROWS * 8 <= kMaskWords * 4),
                "stream merge buffers");

  extern __shared__ __attribute__((aligned(256))) unsigned char smem[];  // stage bases keep bits 0-7 clear
  unsigned char* ring = smem;
  uint32_t* masks = reinterpret_cast<uint32_t*>(smem + kRingBytes);
  int* vis = reinterpret_cast<int*>(masks + kMaskWords);
  int* misc = vis + kMaxTreeUnits;  // kMiscInts ints

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rg = wave % RG, ks = wave / RG;  // with S = 2, SIMD rg%4 holds one wave of each stream
  const int ln = lane & 31, lh = lane >> 5;

  const int item = work_item(a);
  if (item < 0) return;
  TSFA_STAMP(0);
  TSFA_STAMPW(52);
#ifdef TSFA_STAMPS
  if (threadIdx.x == 0) g_stamps[(size_t)blockIdx.x * 64 + 63] = (unsigned long long)item;
#endif
  const int rest = fdiv(item, a.fd_chunks);
  const int chunk = item - rest * a.n_chunks;
  const int bk = fdiv(rest, a.fd_slots);
  const int slot = rest - bk * a.n_slots;
  const int b = fdiv(bk, a.fd_kvh);
  const int kvh = bk - b * a.num_kv_heads;
  // roles: a prefix run (slots below n_slots - 1), the tree units (the last
  // slot), or with fold_tree both in the last slot
  const bool is_tree = !a.fold_tree && slot == a.n_slots - 1;
  const bool do_tree = slot == a.n_slots - 1;

  const int G = a.group;
  const int TG = a.q_len * G;
  const int row0 = chunk * ROWS;
  const int rows_chunk = min(ROWS, TG - row0);
  const bool active = rg * 32 < rows_chunk;
  const int tok_lo = (int)fdiv(row0, a.fd_group);
  const float sl2 = a.scale_log2;
  const float thr_raw = kRescaleLog2 / sl2;  // re-base the running max past 2^8 growth

  const T* kbase = PAGED ? static_cast<const T*>(a.kv_cache) + kvh * a.chs
                        : static_cast<const T*>(a.k) + b * a.skb + kvh * a.skh;
  const T* vbase = PAGED ? kbase + a.css : static_cast<const T*>(a.v) + b * a.svb + kvh * a.svh;
  const int64_t kstride = PAGED ? a.crs : a.skn, vstride = PAGED ? a.crs : a.svn;
  int pt_base = 0;  // sequence b's page list in kv_indices (b * pt_stride < n_indices by the host check)
  if (PAGED) pt_base = a.kv_indptr ? ld_uniform(a.kv_indptr, b) : b * a.pt_stride;
  unsigned char* sring = ring + ks * RB;
  const uint32_t sring_lds = __builtin_amdgcn_readfirstlane(lds_addr(sring));
  const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(lds_addr(ring));
  constexpr bool RING2 = NS >= 8;  // ring loop meets every other step
  // LDS address of the ring stage of the stream's unit j
  auto stage = [&](int j) { return sring_lds + (uint32_t)((j & (NS - 1)) * SB); };
  TSFA_CYC_DECL

  // The stream's RG waves move equal shares of each unit: the first half of
  // them K, the second half V.
  const bool dma_v = rg >= RG / 2;
  const int dma_u0 = (rg % (RG / 2)) * LPU;
  uint32_t loff[D == 128 ? 4 : 2];  // paged: lane offsets of the loads (by load index mod NOFF)
  if constexpr (PAGED) {
#pragma unroll
    for (int u = 0; u < (D == 128 ? 4 : 2); ++u)
      loff[u] = dma_v ? dma_lane_off<D, true>(u, vstride, lane) : dma_lane_off<D, false>(u, kstride, lane);
  }
  // Contiguous K/V: this wave's half (K or V), its row stride and LDS offset,
  // chosen once.  With a row stride of at least D a unit's LPU loads take one
  // scalar row base and one M0 (dma_rows): load i reads i KB past the base by
  // its immediate offset plus the rest of its global step (RPL rows) by its
  // lane offset doff[i]; smaller strides take the clamped per-lane path.
  constexpr int DRPL = 64 / (D / 8);  // key rows per 1 KB load
  const T* dbase = dma_v ? vbase : kbase;
  const int64_t dstride = dma_v ? vstride : kstride;
  const uint32_t dlds = dma_v ? (uint32_t)HALF : 0u;
  const bool rows_fast = __builtin_amdgcn_readfirstlane(dstride >= D ? 1 : 0) != 0;
  uint32_t doff[LPU];
#pragma unroll
  for (int i = 0; i < LPU; ++i)
    doff[i] = (dma_v ? dma_lane_off<D, true>(dma_u0 + i, dstride, lane)
                     : dma_lane_off<D, false>(dma_u0 + i, dstride, lane)) +
              (uint32_t)((int64_t)i * (DRPL * dstride * 2 - 1024));

  // Paged: the raw page-table entries of the next unit this wave issues,
  // read one step early (prefetch) so their scalar loads land behind the
  // step's compute.  A lookup is a function of key0 alone, so a stale or
  // missing prefetch only costs a fresh lookup.
  int pf_key = -1, pf_raw0 = 0, pf_raw1 = 0;
  auto prefetch = [&](int key0) {
    if (PAGED) {
      int pg0, pg1;
      share_pages<D, LPU>(a, key0, dma_u0, pg0, pg1);
      pf_key = key0;
      pf_raw0 = page_entry(a, pt_base, pg0);
      pf_raw1 = page_entry(a, pt_base, pg1);
    }
  };

  // HBM -> LDS: this wave's share of one unit (keys key0 .. key0+31) into
  // stage st of its stream's ring.
  const bool kv_nt = __builtin_amdgcn_readfirstlane(a.kv_nt) != 0;
  auto issue_at = [&](uint32_t sb, int key0) {
    if (PAGED) {
      int pg0, pg1;
      share_pages<D, LPU>(a, key0, dma_u0, pg0, pg1);
      int raw0 = pf_raw0, raw1 = pf_raw1;
      if (key0 != pf_key) {
        raw0 = page_entry(a, pt_base, pg0);
        raw1 = page_entry(a, pt_base, pg1);
      }
      const int64_t pid0 = clamp_page(a, raw0), pid1 = clamp_page(a, raw1);
      if (dma_v)
        dma_half_paged<T, D, true, LPU, C32>(vbase, a, pid0, pid1, pg0, sb + HALF, key0, lane, dma_u0, loff, kv_nt);
      else
        dma_half_paged<T, D, false, LPU, C32>(kbase, a, pid0, pid1, pg0, sb, key0, lane, dma_u0, loff, kv_nt);
    } else if (rows_fast && key0 + kUnitKeys <= a.kv_len) {
      const char* rowp = reinterpret_cast<const char*>(dbase + (int64_t)(key0 + dma_u0 * DRPL) * dstride);
      const uint32_t m0v = sb + dlds + dma_u0 * 1024;
      if (kv_nt) dma_rows<LPU, true>(rowp, doff, m0v);
      else dma_rows<LPU, false>(rowp, doff, m0v);
    } else if (dma_v) {
      dma_tail<T, D, true, LPU>(dbase, dstride, sb + HALF, key0, a.kv_len, lane, dma_u0);
    } else {
      dma_tail<T, D, false, LPU>(dbase, dstride, sb, key0, a.kv_len, lane, dma_u0);
    }
  };

  // Q^T operand fragments of the wave's row tile: row r = row0 + rg*32 + ln,
  // d = kk*16 + lh*8 + [0, 8); Q is negated for a negative scale.
  i16x8 qf[KSTEPS];
  const int qrow = row0 + rg * 32 + ln;
  const int row_tt = qrow < TG ? (int)fdiv(qrow, a.fd_group) - tok_lo : 0;  // token of the lane's row, chunk-relative
  const short qsgn = a.neg_q ? (short)0x8000 : (short)0;
  // Q straight into registers (rows past the end load zeros).
  auto load_q = [&]() {
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) qf[kk] = i16x8{0, 0, 0, 0, 0, 0, 0, 0};
    if (qrow < TG) {
      const int t = (int)fdiv(qrow, a.fd_group);
      const int g = qrow - t * G;
      const T* qp = static_cast<const T*>(a.q) + b * a.sqb + (int64_t)(kvh * G + g) * a.sqh + (int64_t)t * a.sqm +
                    lh * 8;
#pragma unroll
      for (int kk = 0; kk < KSTEPS; ++kk) qf[kk] = *reinterpret_cast<const i16x8*>(qp + kk * 16) ^ qsgn;
    }
    // Consume the Q loads here: otherwise the compiler waits for them lazily
    // at their first use inside the unit loop, where its vmcnt count would
    // also cover (and stall on) the in-flight K/V prefetch it does not know of.
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) asm volatile("" : : "v"(qf[kk]));
  };
  // Q through LDS instead: the chunk's rows go HBM -> LDS into the last QS
  // ring stages of the stream whose row groups use them (QROWS rows per
  // stream), as global_load_lds issued ahead of the first K/V units, so the
  // prologue need not wait for Q before filling the ring.  Rows past the end
  // repeat the last row (their outputs are never stored).
  // Q stage of the stream holding chunk rows [s*QROWS, (s+1)*QROWS): the last
  // QS stages of its ring.
  auto q_stage = [&](int s) { return ring + s * RB + (NS - QS) * SB; };
  auto issue_q = [&]() {
    constexpr int RPL = 1024 / ROWB, CPR = D / 8;
    constexpr int QL = ROWS / RPL / kWaves;  // 1 KB loads per wave
#pragma unroll
    for (int i = 0; i < QL; ++i) {
      const int l0 = (wave * QL + i) * RPL;  // first chunk row of the load
      const int row = l0 + lane / CPR, pos = lane % CPR, tr = row % QROWS;
      const int R = min(row0 + row, TG - 1);
      const int t = (int)fdiv(R, a.fd_group);
      const int g = R - t * G;
      const T* src = static_cast<const T*>(a.q) + b * a.sqb + (int64_t)(kvh * G + g) * a.sqh + (int64_t)t * a.sqm +
                     ((pos ^ swz_k<D>(tr)) << 3);
      dma16(src, __builtin_amdgcn_readfirstlane(lds_addr(q_stage(l0 / QROWS) + (l0 % QROWS) * ROWB)));
    }
  };
  auto read_q = [&]() {
    const unsigned char* qs = q_stage(rg * 32 / QROWS) + ((rg * 32) % QROWS) * ROWB;
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk)
      qf[kk] = *reinterpret_cast<const i16x8*>(qs + ln * ROWB + (((2 * kk + lh) ^ swz_k<D>(ln)) << 4)) ^ qsgn;
  };

  // Running state per lane (query row ln of the row tile): O^T element i of
  // d-tile dt is d = dt*32 + 8*(i/4) + 4*lh + i%4.  l_run is this lane's half
  // of the row sum (keys 4*lh + [0,4) of every 8).
  f32x16 o[DT];
  float m_run = -INFINITY, m_lim = -INFINITY, mb = 0.f, l_run = 0.f;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[dt][i] = 0.f;

  // LDS byte offsets of this lane's operand reads within a stage.
  // V^T: 16-lane group x = (h, d-half); lane i of the group reads 8 bytes of
  // key row 4*h + i/4 (+16*s2 + 8*jj, which keeps the swizzle) at d = dt*32 +
  // 16*(x&1) + 4*(i%4); the transpose read hands lane i keys +[0,4) of d = i.
  // K: lane (ln, lh) reads 16 bytes of key row ln at d = kk*16 + 8*lh.
  // The chunk XOR swizzles only move offset bits 5-7 (K, per k-step) and 6-7
  // (V^T, per d-tile), so k-step kk reads at k_off0 ^ (kk << 5) and d-tile dt
  // at v_off0 ^ (dt << 6); stage bases are multiples of 4 KB, so the XOR
  // commutes with adding them (one base register per operand instead of one
  // per k-step / d-tile).
  const int vx = lane >> 4, vi = lane & 15;
  const int vkey = 4 * (vx >> 1) + (vi >> 2);
  const int v_off0 = vkey * ROWB + ((((16 * (vx & 1) + 4 * (vi & 3)) >> 3) ^ swz_v<D>(vkey)) << 4) + ((4 * (vi & 3) & 7) << 1);
  const int k_off0 = ln * ROWB + ((lh ^ swz_k<D>(ln)) << 4);

  // S^T of one 32-key unit for the wave's 32 rows: MFMA row m = key, column =
  // query row; lane (ln, lh) holds keys 8*(i/4) + 4*lh + i%4 of row ln.
  auto read_k = [&](const unsigned char* sk, i16x8 (&kf)[KSTEPS]) {
    const int base = (int)(sk - smem) + k_off0;
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) kf[kk] = *reinterpret_cast<const i16x8*>(smem + (base ^ (kk << 5)));
  };
  auto qk = [&](const i16x8 (&kf)[KSTEPS]) {
    f32x16 s;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = 0.f;
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) s = Mma<T>::run(bit_cast<V8>(kf[kk]), bit_cast<V8>(qf[kk]), s);
    return s;
  };

  // ---- the unit loop (software-pipelined) ----
  // Iteration j of a wave: the mask and row statistics of unit j (whose S^T
  // the previous iteration computed), then group 1 -- the S^T MFMAs of unit
  // j+1 with the exponentials and rounded P of unit j between them -- then
  // the rare O re-base, then group 2 -- O^T += V^T P^T of unit j with the row
  // sum of unit j between them.  A wave keeps its own matrix core busy while
  // its softmax runs, and every VALU read of an MFMA result (S^T by the mask
  // and statistics, O^T by the re-base) happens an MFMA group and a barrier
  // after the MFMAs that wrote it.  The running max moves without a branch
  // (a re-based row takes the unit's row max and scales l at once).  The ring
  // is used this way: iteration j reads K of unit j+1 and V of unit j after
  // barrier j, and both finish reading unit j-1 before it, so the barrier
  // orders the ring.
  auto apply_mask = [&](f32x16& s, uint32_t mask) {
    const uint32_t w = mask >> (4 * lh);
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (!((w >> (8 * (i >> 2) + (i & 3))) & 1u)) s[i] = -INFINITY;
  };
  // Row statistics of one unit's S^T (tree_sparse_flashattn.py:272-276,
  // :320-324): returns whether the row re-based; alpha scales O and l.
  auto stats = [&](const f32x16& s, float& alpha) {
    const float mx = max3f(max3f(max3f(s[0], s[1], s[2]), max3f(s[3], s[4], s[5]), max3f(s[6], s[7], s[8])),
                           max3f(max3f(s[9], s[10], s[11]), max3f(s[12], s[13], s[14]), s[15]), -INFINITY);
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    const float rmax = max3f(__uint_as_float(sw[0]), __uint_as_float(sw[1]), -INFINITY);
    // rmax > m_lim >= m_run, so a re-based row takes rmax; false while both are -inf
    const bool need = rmax > m_lim;
    const float m_new = need ? rmax : m_run;
    // m_run = -inf gives alpha = 0 (O and l are still 0) (tree_sparse_flashattn.py:276, :324)
    alpha = need ? __builtin_amdgcn_exp2f((m_run - m_new) * sl2) : 1.f;
    m_run = m_new;
    mb = (m_new == -INFINITY) ? 0.f : m_new * sl2;
    m_lim = m_new + thr_raw;
    l_run *= alpha;
    return need;
  };
  // Unit j of the stream (u: its index in the run; s_in: its S^T; s_out:
  // S^T of unit j+1 when NEXT): the first KA K fragments of unit j+1
  // requested, mask and statistics, group 1 when NEXT (the S^T MFMAs of unit
  // j+1 with the exponentials and rounded P of unit j between them), the O
  // re-base, group 2 (O^T += V^T P^T of unit j, V^T read VA MFMAs ahead, the
  // row sum between them).  Requesting K at the top, fenced so the compiler
  // cannot sink it behind the statistics, lets the first S^T MFMA wait for
  // one LDS read instead of the scheduler's last-moment two (and VA = 4
  // instead of 2 the same for group 2): 1 % at the 8B decode shape and the
  // 1024-token tree, same-box A/B.
  auto pipe_iter = [&](int j, int u, auto next_c, f32x16& s_in, f32x16& s_out, auto masked_of, auto mask_of) {
    constexpr bool NEXT = decltype(next_c)::value;
    constexpr int NPV = 2 * DT;  // P V MFMAs
    i16x4 vh[DT][2][2];
    float p[16];
    V8 pb[2];
    constexpr int KA = KSTEPS < 4 ? KSTEPS : 4;  // K fragments requested before the statistics
    constexpr int VA = NPV < 4 ? NPV : 4;        // P V MFMAs whose V^T is read ahead
    const uint32_t vb = stage(j) + (uint32_t)(HALF + v_off0);
    i16x8 kf[KSTEPS];
    const uint32_t kb = stage(j + 1) + (uint32_t)k_off0;
    auto rk = [&](int kk) { return lds_ld<i16x8>(kb ^ (uint32_t)(kk << 5)); };
    if constexpr (NEXT) {
#pragma unroll
      for (int kk = 0; kk < KA; ++kk) kf[kk] = rk(kk);
      __builtin_amdgcn_sched_barrier(0);
    }
    auto rv = [&](int idx) {  // V^T fragment idx = (dt, s2, jj); P V MFMA g reads 2g and 2g+1
      const int dt = idx >> 2, s2 = (idx >> 1) & 1, jj = idx & 1;
      vh[dt][s2][jj] = lds_tr((vb ^ (uint32_t)(dt << 6)) + (uint32_t)((16 * s2 + 8 * jj) * ROWB));
    };
    if (masked_of(u)) {
      asm volatile("" ::: "memory");
      apply_mask(s_in, mask_of(u));
    }
    float alpha;
    const bool need = stats(s_in, alpha);
    // exponential, rounding and register pin of the pair (e, e+1) of unit j
    auto expo2 = [&](int e) {
      p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s_in[e], sl2, -mb));
      p[e + 1] = __builtin_amdgcn_exp2f(__builtin_fmaf(s_in[e + 1], sl2, -mb));
      pb[e >> 3][e & 7] = (T)p[e];
      pb[e >> 3][(e & 7) + 1] = (T)p[e + 1];
    };
    // P V MFMA g of group 2: d-tile and k-step, ordered by k-step (keys 0-15
    // of every d-tile, then keys 16-31), so the second half of the
    // exponentials (P^T of keys 16-31) runs under the first half of the P V
    // MFMAs instead of all of them under the S^T MFMAs (2 % at the 8B shape,
    // 1 % at the 1024-token tree in one A/B; the same sums in the same order)
    auto pv_dt = [&](int g) { return g % DT; };
    auto pv_s2 = [&](int g) { return g / DT; };
    auto rv2 = [&](int g) {  // V^T fragments of P V MFMA g
      rv(pv_dt(g) * 4 + pv_s2(g) * 2);
      rv(pv_dt(g) * 4 + pv_s2(g) * 2 + 1);
    };
    constexpr int NG1 = 4;  // exponential pairs in group 1 (keys 0-15)
    if constexpr (NEXT) {
      // group 1 in explicit order: K of unit j+1 read KA k-steps ahead of
      // its MFMAs; the statistics above and then the exponentials and
      // rounded P of unit j between the MFMAs; V^T of the first VA P V
      // MFMAs at the end
#pragma unroll
      for (int i = 0; i < 16; ++i) s_out[i] = 0.f;
      constexpr int K0 = KSTEPS / 4;  // steps that carry the statistics; the exponential pairs spread over the rest
#pragma unroll
      for (int kk = 0; kk < KSTEPS; ++kk) {
        if (kk + KA < KSTEPS) kf[kk + KA] = rk(kk + KA);
        s_out = Mma<T>::run(bit_cast<V8>(kf[kk]), bit_cast<V8>(qf[kk]), s_out);
        if (kk >= K0) {
#pragma unroll
          for (int pr = (kk - K0) * NG1 / (KSTEPS - K0); pr < (kk - K0 + 1) * NG1 / (KSTEPS - K0); ++pr) expo2(2 * pr);
        }
        if (kk == KSTEPS - 1) {
#pragma unroll
          for (int g = 0; g < VA; ++g) rv2(g);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      // P (its group-1 half) exists here: the exponentials and conversions
      // stay in group 1 (its block ends at the mask branch) instead of
      // sinking into group 2
      asm volatile("" : "+v"(pb[0]));
      TSFA_CYC(0);
    } else {
#pragma unroll
      for (int g = 0; g < VA; ++g) rv2(g);
#pragma unroll
      for (int pr = 0; pr < NG1; ++pr) expo2(2 * pr);
    }
    // O re-base for unit j: after P V of unit j-1 (issued an iteration ago),
    // before that of unit j
    if (__ballot(need) != 0) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
    }
    if constexpr (NEXT) TSFA_CYC(3);
    // group 2 in explicit order: MFMA g with V^T of MFMA g+VA read behind it,
    // the remaining exponentials under the k-step-0 MFMAs and the row sum
    // of unit j under the k-step-1 MFMAs
#pragma unroll
    for (int g = 0; g < NPV; ++g) {
      if (g + VA < NPV) rv2(g + VA);
      const int dt = pv_dt(g), s2 = pv_s2(g);
      const i16x8 vf = __builtin_shufflevector(vh[dt][s2][0], vh[dt][s2][1], 0, 1, 2, 3, 4, 5, 6, 7);
      o[dt] = Mma<T>::run(bit_cast<V8>(vf), pb[s2], o[dt]);
      if (g < DT) {
#pragma unroll
        for (int pr = NG1 + g * (8 - NG1) / DT; pr < NG1 + (g + 1) * (8 - NG1) / DT; ++pr) expo2(2 * pr);
        if (g == DT - 1) asm volatile("" : "+v"(pb[1]));
      }
      // tree sum of p: 8 + 4 + 2 + 1 adds over the k-step-1 MFMAs
      const int h = g - DT;
      if (h == 0)
#pragma unroll
        for (int i = 0; i < 8; ++i) p[i] = p[i] + p[i + 8];
      if (h == DT / 2)
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = p[i] + p[i + 4];
      if (h == DT - 1) {
        p[0] = p[0] + p[2];
        p[1] = p[1] + p[3];
        l_run += p[0] + p[1];
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (NEXT) TSFA_CYC(1);
  };
  // (requests address their stages as j * SB and (j % NS) * SB: the masked
  // form of stage() there left the two-stream paged kernels 105-125
  // spilled SGPRs instead of 38-42)
  // masked_last_of tests the stream's last unit, which the loops below never
  // process (a prefix run's partial last unit, on the unchecked steps too)
  auto run_units_pipe = [&](int n, int pre, auto key0_of, auto masked_of, auto mask_of, auto issue_of, auto fast_c,
                            auto masked_last_of) {
    const int mine = n > ks ? (n - ks + S - 1) / S : 0;
    const int steps = (n + S - 1) / S;
    {
      // RING2: NS-2 units ahead, two issued at every other step
      constexpr int AHEAD = RING2 ? NS - 2 : NS - 1;
      for (int j = pre; j < AHEAD && j < mine; ++j) issue_of(sring_lds + j * SB, ks + S * j);
      if constexpr (decltype(fast_c)::value) fast_c.init(AHEAD);  // the steady refills start there
      if (PAGED && AHEAD < mine) prefetch(key0_of(ks + S * AHEAD));
      if (mine > 0) wait_units<LPU, NS - 2>(min(mine, AHEAD) - 1);  // unit 0 landed
      sync_lds();
    }
    TSFA_STAMP(2);
    f32x16 s_cur, s_next;  // S^T of unit j and of unit j+1
    if (mine > 0 && active) {
      i16x8 kf[KSTEPS];
      read_k(ring + (stage(0) - ring_lds), kf);
      s_cur = qk(kf);
    }
    // Ring: unit j+1 landed for every wave of the stream; ring stage
    // (j-1)%NS is free.
    // RING2 (rings of at least 8 stages): the same with the waves meeting
    // every other step, units up to j+2 landed and stages (j-2)%NS and
    // (j-1)%NS refilled at even steps j.
    auto ring_step = [&](int j) {
      if constexpr (RING2) {
        if (j & 1) return;
        if constexpr (decltype(fast_c)::value) {
          // steady state (both refill units exist): fixed wait, unchecked
          // refills -- scalar work and branches here stall the wave's
          // MFMA issue (measured ~8 cycles per scalar instruction and
          // ~35 per taken branch per unit in a replica of this loop)
          if (j + NS - 1 < mine) {
            vm_wait<(NS - 5) * LPU>();
            __builtin_amdgcn_sched_barrier(0);
            sync_lds();
            __builtin_amdgcn_sched_barrier(0);
            if (j < 40) TSFA_STAMP(3 + j);
            TSFA_CYC(2);
            fast_c.next(mine);  // units j + NS - 2 and j + NS - 1 of the stream
            fast_c.next(mine);
            __builtin_amdgcn_sched_barrier(0);
            return;
          }
        }
        // issued: units below min(mine, j + NS - 2)
        if (j + 1 < mine) wait_units<LPU, NS - 5>(max(min(mine - j - 3, NS - 5), 0));
      } else {
        if constexpr (decltype(fast_c)::value) {
          // steady state (the refill unit exists): fixed wait, unchecked refill
          if (j + NS - 1 < mine) {
            vm_wait<(NS - 3) * LPU>();
            __builtin_amdgcn_sched_barrier(0);
            sync_lds();
            __builtin_amdgcn_sched_barrier(0);
            if (j < 40) TSFA_STAMP(3 + j);
            TSFA_CYC(2);
            fast_c.next(mine);  // unit j + NS - 1 of the stream
            __builtin_amdgcn_sched_barrier(0);
            return;
          }
        }
        if (j + 1 < mine) wait_units<LPU, NS - 3>(min(mine - 2 - j, NS - 3));
      }
      __builtin_amdgcn_sched_barrier(0);
      sync_lds();
      __builtin_amdgcn_sched_barrier(0);
      if (j < 40) TSFA_STAMP(3 + j);
      TSFA_CYC(2);
      if constexpr (RING2) {
        if (j + NS - 2 < mine) issue_of(sring_lds + ((j + NS - 2) % NS) * SB, ks + S * (j + NS - 2));
        if (j + NS - 1 < mine) issue_of(sring_lds + ((j + NS - 1) % NS) * SB, ks + S * (j + NS - 1));
      } else if (j + NS - 1 < mine) {
        issue_of(sring_lds + ((j + NS - 1) % NS) * SB, ks + S * (j + NS - 1));
      }
      if (PAGED && j + NS < mine) prefetch(key0_of(ks + S * (j + NS)));
      __builtin_amdgcn_sched_barrier(0);
    };
    // (unrolling by two to alternate the S^T registers instead of copying
    // them made the allocator shuffle the O accumulators: 281 copies)
    int j0 = 0;
    if constexpr (RING2 && decltype(fast_c)::value) {
      // Unchecked steady state in pairs of steps (the even one meets and
      // refills two units): no parity test and one loop test per two units;
      // the scheduling fences keep the two iterations' registers apart (the
      // 2x unrolled body spills without them).  1024-token wide tree -2 %,
      // 70B shape -3 to -6 % (same-call A/B).
      if (active) {
        for (; j0 + NS - 1 < mine; j0 += 2) {
          vm_wait<(NS - 5) * LPU>();
          __builtin_amdgcn_sched_barrier(0);
          sync_lds();
          __builtin_amdgcn_sched_barrier(0);
          if (j0 < 40) TSFA_STAMP(3 + j0);
          TSFA_CYC(2);
          fast_c.next(mine);  // units j0 + NS - 2 and j0 + NS - 1 of the stream
          fast_c.next(mine);
          __builtin_amdgcn_sched_barrier(0);
          pipe_iter(j0, ks + S * j0, std::true_type{}, s_cur, s_next, masked_of, mask_of);
          s_cur = s_next;
          __builtin_amdgcn_sched_barrier(0);
          pipe_iter(j0 + 1, ks + S * (j0 + 1), std::true_type{}, s_cur, s_next, masked_of, mask_of);
          s_cur = s_next;
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    } else if constexpr (decltype(fast_c)::value) {
      // the same for rings that meet and refill at every step
      if (active) {
        for (; j0 + NS < mine; j0 += 2) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            vm_wait<(NS - 3) * LPU>();
            __builtin_amdgcn_sched_barrier(0);
            sync_lds();
            __builtin_amdgcn_sched_barrier(0);
            if (j0 + h < 32) TSFA_STAMP(3 + j0 + h);
            TSFA_CYC(2);
            fast_c.next(mine);  // unit j0 + h + NS - 1 of the stream
            __builtin_amdgcn_sched_barrier(0);
            pipe_iter(j0 + h, ks + S * (j0 + h), std::true_type{}, s_cur, s_next, masked_of, mask_of);
            s_cur = s_next;
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
    }
    for (int j = j0; j < steps; ++j) {
      ring_step(j);
      if (j + 1 < mine && active) {
        pipe_iter(j, ks + S * j, std::true_type{}, s_cur, s_next, masked_of, mask_of);
        s_cur = s_next;
      }
    }
    // The stream's last unit: its V^T stage landed before barrier mine-2 and
    // no later load targets it (a load into it would be of unit >= mine).
    if (mine > 0 && active)
      pipe_iter(mine - 1, ks + S * (mine - 1), std::false_type{}, s_cur, s_cur, masked_last_of, mask_of);
  };
  // issue_of(lds stage, i) requests run unit i (keys key0_of(i)) into a stage
  auto units = [&](int n, int pre, auto key0_of, auto masked_of, auto mask_of, auto issue_of, auto fast_c,
                   auto masked_last_of) {
    run_units_pipe(n, pre, key0_of, masked_of, mask_of, issue_of, fast_c, masked_last_of);
  };

  if (!is_tree) {
    // Prefix run: units [u_lo, u_lo + n) of keys [0, prefix_len); the last
    // unit of the prefix may be partial.
    const int P = a.prefix_len;
    const int u_lo = slot * a.units_per_split;
    const int n = min(a.units_per_split, a.n_pu - u_lo);
    auto key0_of = [&](int i) { return (u_lo + i) * kUnitKeys; };
    // Contiguous K/V: run unit i's row pointer is this wave's base for the
    // run plus one product (the general path rebuilds it from the key with
    // 64-bit scalar arithmetic and range checks, on the scalar unit the
    // workgroup's waves share); units reaching past kv_len take that path.
    const int64_t unit_bytes = (int64_t)kUnitKeys * dstride * (int64_t)sizeof(T);
    const char* run_rows =
        reinterpret_cast<const char*>(dbase + ((int64_t)u_lo * kUnitKeys + dma_u0 * DRPL) * dstride);
    const int n_fast = rows_fast ? max(0, min(n, a.kv_len / kUnitKeys - u_lo)) : 0;
    const uint32_t m0_off = dlds + (uint32_t)dma_u0 * 1024u;
    auto issue_prefix = [&](uint32_t sb, int i) {
      if constexpr (FM != 0 && !PAGED) {
        dma_rows<LPU, FM == 2>(run_rows + (int64_t)i * unit_bytes, doff, sb + m0_off);
      } else if (!PAGED && i < n_fast) {
        const char* rowp = run_rows + i * unit_bytes;
        if (kv_nt) dma_rows<LPU, true>(rowp, doff, sb + m0_off);
        else dma_rows<LPU, false>(rowp, doff, sb + m0_off);
      } else {
        issue_at(sb, key0_of(i));
      }
    };
    // Q and the first two units of each stream leave together; wait for Q
    // only (loads complete in order), then every wave reads its fragments
    // and the ring prologue requests the rest of its NS - 1 units ahead.
    // With QS > 1 the ring prologue reuses Q stages: one more barrier first.
    // Every workgroup starts at once, so the opening requests of the whole
    // grid queue in HBM together: the fewer units beside Q, the sooner every
    // CU's Q and unit 0 arrive.  Requesting a short run's units all at once
    // (every run of the Llama-3-8B decode shape fits in LDS) measured 16.0
    // against 15.4-15.6 us per call; two units with Q instead of NS - QS
    // (3 with two streams, 4 with one): the 8B shape 15.6 -> 15.3 us, the
    // 16-sequence shape 49.7 -> 47.8-48.3 us, the 1024-token tree unchanged
    // (same-box A/B; one unit: in between).
    const int mine = n > ks ? (n - ks + S - 1) / S : 0;
    const int pre = min(mine, min(NS - QS, 2));
    // Paged runs on the unchecked steps: the run's page ids (list positions
    // pg_lo .. pg_lo + n_pg - 1, clamped like page_entry / clamp_page) leave
    // HBM with Q into an LDS table, so a steady refill takes its page from
    // one LDS read a step ahead and a product, instead of the page-table
    // scalar loads, clamps and 64-bit address checks of the general path.
    // Each wave clamps the entries it requested once its Q landed; the Q
    // barrier publishes them.  Its own instance (FAST & 8): the general
    // path's variables beside the table's spilled SGPRs in the loop of the
    // two-stream kernels (the Llama-3-8B decode shape's paged call 19.9 ->
    // 22.3 us with both paths in one instance; 19.4 -> 19.1 us as its own).
    int* ptab = misc + kMiscInts;  // kPageTabInts entries (paged instances only)
    const int pg_lo = PAGED ? (int)(((int64_t)u_lo * kUnitKeys) >> a.page_shift) : 0;
    const int n_pg = PAGED ? (int)((((int64_t)(u_lo + n) * kUnitKeys - 1) >> a.page_shift) - pg_lo + 1) : 0;
    // (the host chose the instance: every run within the table, rows_fast;
    // the table's reads are clamped to it all the same)
    const bool ptab_ok = PTAB && n > 0;
    if (ptab_ok) {
      for (int i0 = wave * 64; i0 < min(n_pg, kPageTabInts); i0 += kWaves * 64)
        if (i0 + lane < min(n_pg, kPageTabInts))
          dma4(a.kv_indices + min(max(pt_base + pg_lo + i0 + lane, 0), a.n_indices - 1), lds_addr(ptab + i0));
    }
    TSFA_STAMP(62);
    issue_q();
    for (int j = 0; j < pre; ++j) issue_prefix(sring_lds + j * SB, ks + S * j);
    TSFA_STAMP(60);
    wait_units<LPU, NS - QS>(pre);
    if (ptab_ok) {
      for (int i = wave * 64 + lane; i < min(n_pg, kPageTabInts); i += kWaves * 64)
        ptab[i] = min(max(ptab[i], 0), a.n_pages - 1);
    }
    sync_lds();
    TSFA_STAMP(1);
    read_q();
    if (QS > 1) sync_lds();
    // Steady refills (FAST, rotation off): the next unit's row pointer and
    // ring stage advance by S units and one stage per refill.
    const char* seq_rows = nullptr;
    uint32_t seq_stage = 0;
    int seq_t = 0;  // paged: the stream's next unit
    // paged with the LDS page table: the wave's first key of the next unit
    // and that key's page id, read from the table one refill ahead (its rows
    // sit in one page: a share of 8 or 16 aligned keys, pages of 16 or more)
    int seq_kw = 0, seq_pid = 0;
    const int pmask = PAGED ? (1 << a.page_shift) - 1 : 0;
    auto seq_init = [&](int t) {
      if constexpr (PTAB) {
        seq_stage = (uint32_t)(t % NS) * SB;
        seq_kw = key0_of(ks + S * t) + dma_u0 * DRPL;
        if (t < mine) seq_pid = ptab[min((seq_kw >> a.page_shift) - pg_lo, kPageTabInts - 1)];
      } else if constexpr (PAGED) {
        seq_t = t;
      } else {
        seq_rows = run_rows + (int64_t)(ks + S * t) * unit_bytes;
        seq_stage = (uint32_t)(t % NS) * SB;
      }
    };
    auto seq_next = [&](int mine_units) {
      if constexpr (PTAB) {
        const int pid = __builtin_amdgcn_readfirstlane(seq_pid);
        const char* rowp;
        if constexpr (C32)
          rowp = reinterpret_cast<const char*>(dbase) + ((uint32_t)pid * a.cps_b32 + (uint32_t)(seq_kw & pmask) * a.crs_b32);
        else  // 64-bit page offset, 32-bit strides (the host checked that they fit)
          rowp = reinterpret_cast<const char*>(dbase) + ((uint64_t)(uint32_t)pid * a.cps_b32 +
                                                         (uint32_t)(seq_kw & pmask) * a.crs_b32);
        if (kv_nt) dma_rows<LPU, true>(rowp, doff, sring_lds + seq_stage + m0_off);
        else dma_rows<LPU, false>(rowp, doff, sring_lds + seq_stage + m0_off);
        seq_stage = (seq_stage + SB) & (uint32_t)(NS * SB - 1);
        seq_kw += S * kUnitKeys;
        // the unit after it (its key is past the run's pages when none follows)
        if (seq_kw < (u_lo + n) * kUnitKeys) seq_pid = ptab[min((seq_kw >> a.page_shift) - pg_lo, kPageTabInts - 1)];
        (void)mine_units;
      } else if constexpr (PAGED) {
        // the page-table path, then the lookup of the unit after it
        issue_prefix(sring_lds + (uint32_t)(seq_t % NS) * SB, ks + S * seq_t);
        ++seq_t;
        if (seq_t < mine_units) prefetch(key0_of(ks + S * seq_t));
      } else {
        dma_rows<LPU, FM == 2>(seq_rows, doff, sring_lds + seq_stage + m0_off);
        seq_rows += S * unit_bytes;
        seq_stage = (seq_stage + SB) & (uint32_t)(NS * SB - 1);
      }
    };
    units(
        n, pre, key0_of,
        [&](int i) {
          if constexpr (FM != 0) return false;
          else return P - key0_of(i) < kUnitKeys;
        },
        [&](int i) { return (1u << (P - key0_of(i))) - 1u; }, issue_prefix,
        FastSeq<FM != 0, decltype(seq_init), decltype(seq_next)>{seq_init, seq_next},
        // the prefix's partial last unit (the last unit of its run: with the
        // unchecked steps too, its keys past the prefix are masked here)
        [&](int i) { return P - key0_of(i) < kUnitKeys; });
  }
  if (do_tree) {
    // Tree units, after a prefix run (its ring reads and loads done: the
    // block states reuse the ring; Q already in registers) or as a tree
    // item: the chunk's block states, its visible tree units, then the mask
    // words (word token * vt_max + unit of the batch) batch by batch.
    if (is_tree) load_q();
    else sync_all();
    TSFA_STAMP(43);
    const int P = a.prefix_len, BM = a.block_m, BN = a.block_n, ntb = a.n_tree_blocks;
    const int tok_hi = (int)fdiv(row0 + rows_chunk - 1, a.fd_group);  // tokens tok_lo .. tok_hi
    const int ntok = tok_hi - tok_lo + 1;
    const int qb_lo = tok_lo / BM, qb_hi = tok_hi / BM, nqbc = qb_hi - qb_lo + 1;
    const int32_t* rp = a.row_ptr + b * a.ms_row_ptr;
    const int32_t* ci = a.col_idx + b * a.ms_col_idx;
    const int8_t* bt = a.blk_type + b * a.ms_blk_type;
    const int32_t* pl = a.payload + b * a.ms_payload;
    const int32_t* of = a.offset + b * a.ms_offset;
    int* st = reinterpret_cast<int*>(ring);  // [nqbc][ntb]: 0 ZERO, -1 FULL, 1+offset MIXED
    int* rps = misc + 8;                     // row_ptr[qb_lo .. qb_hi+1]
    // Block states of the chunk's q-blocks in two parallel round trips: the
    // row_ptr window, then every CSR entry of those rows at once.
    auto build_state = [&]() {
      for (int i = tid; i < nqbc * ntb; i += kWaves * 64) st[i] = 0;
      if (tid <= nqbc) rps[tid] = rp[qb_lo + tid];
      sync_lds();
      const int e_begin = rps[0], e_end = rps[nqbc];
      for (int e = e_begin + tid; e < e_end; e += kWaves * 64) {
        int qq = 0;
        while (qq + 1 < nqbc && rps[qq + 1] <= e) ++qq;
        const int tb = ci[e];
        if (tb >= 0 && tb < ntb) st[qq * ntb + tb] = (bt[e] != TSFA_MIXED_BLOCK) ? -1 : (of[e] + 1);
      }
      sync_lds();
    };
    build_state();
    TSFA_STAMP(44);
    // Tree units holding a key some row of the chunk can see, compacted.
    const int n_tu = (a.tree_key_limit + kUnitKeys - 1) / kUnitKeys;
    for (int i = tid; i < n_tu; i += kWaves * 64) vis[i] = 0;
    sync_lds();
    for (int i = tid; i < nqbc * ntb; i += kWaves * 64) {
      if (st[i] != 0) {
        const int tb = i % ntb;
        const int c_first = tb * BN, c_last = min(tb * BN + BN, a.tree_key_limit) - 1;
        for (int u = c_first / kUnitKeys; u <= c_last / kUnitKeys; ++u) vis[u] = 1;
      }
    }
    sync_lds();
    if (wave == 0) {
      int nv = 0;
      for (int base = 0; base < n_tu; base += 64) {
        const int idx = base + lane;
        const bool f = idx < n_tu && vis[idx] != 0;
        const uint64_t bal = __ballot(f);
        const int pre = __popcll(bal & ((1ull << lane) - 1ull));
        if (f) vis[nv + pre] = idx;
        nv += __popcll(bal);
      }
      if (lane == 0) misc[0] = nv;
    }
    sync_lds();
    TSFA_STAMP(45);
    const int n_vis = misc[0];
    for (int vb0 = 0; vb0 < n_vis; vb0 += a.vt_max) {
      const int nb = min(a.vt_max, n_vis - vb0);
      if (vb0 > 0) build_state();
      // Per-token visibility word of each unit of the batch, from two 16-key
      // groups (BN is a multiple of 16, so a group never straddles blocks).
      for (int it = tid; it < ntok * nb * 2; it += kWaves * 64) {
        const int q2 = it & 1, jt = it >> 1;
        const int j = jt % nb, tt = jt / nb;
        const int t = tok_lo + tt, qb = t / BM, tl = t - qb * BM;
        const int c0 = vis[vb0 + j] * kUnitKeys + q2 * 16;
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
        // two 16-bit halves assembled through LDS: the q2 = 1 half lands in the high bits
        reinterpret_cast<uint16_t*>(masks)[(tt * a.vt_max + j) * 2 + q2] = (uint16_t)bits;
      }
      sync_lds();
      TSFA_STAMP(46);
      auto tree_key0 = [&](int i) { return P + vis[vb0 + i] * kUnitKeys; };
      units(
          nb, 0, tree_key0, [&](int) { return true; }, [&](int i) { return masks[row_tt * a.vt_max + i]; },
          [&](uint32_t sb, int i) { issue_at(sb, tree_key0(i)); }, FastSeq<false>{}, [&](int) { return true; });
      sync_all();  // ring and masks free for the next batch
      TSFA_STAMP(47);
    }
  }

  // Epilogue.  With two streams, each stream merges (log-sum-exp) half the
  // d-tiles of its rows: it leaves (m, l) and O^T of the other half in LDS
  // for the other stream, then folds in the other stream's.  Every lane then
  // normalises its own O^T elements and stores them straight into the
  // partial row (8 bytes per element quad; a row's 16-byte pieces come from
  // lanes l and l+32 of one instruction), so the partial needs no LDS
  // staging pass.
  sync_all();
  TSFA_STAMP(50);
  typedef T T4 __attribute__((ext_vector_type(4)));
  const int64_t part_row0 = ((int64_t)bk * a.n_slots + slot) * TG + row0;
  const int r = rg * 32 + ln;  // the lane's chunk row
  const bool row_ok = r < rows_chunk;
  // One-slot plans write the lane's row of O itself: token t, head kvh*G+g
  // (rows past the chunk's end store nothing).  A row that saw no key gets
  // NaN (0/0, as the combine and the reference give) instead of a partial
  // of weight 0.
  constexpr bool direct = DIRECT;
  T* dst;
  if constexpr (direct) {
    // row (token t, head kvh*G + g) of O [B, Hq, q_len, D]
    const int R = min(row0 + r, TG - 1);
    const int t = (int)fdiv((uint32_t)R, a.fd_group);
    const int64_t h = (int64_t)kvh * G + (R - t * G);
    dst = static_cast<T*>(a.ws_o) + (((int64_t)b * a.num_kv_heads * G + h) * a.q_len + t) * D;
  } else {
    dst = static_cast<T*>(a.ws_o) + (part_row0 + r) * D;
  }
  const float empty_inv = direct ? __builtin_nanf("") : 0.f;  // (compile-time)
  // (m, l) of the lane's row into the workspace (none when writing O)
  auto put_ml = [&](float m, float l) {
    if constexpr (!direct) a.ws_ml[part_row0 + r] = make_float2(m, l);
  };
  // Quads e (d = 8q + 4lh + [0,4), q = 2p) and f (q = 2p+1) of one row in
  // lanes l and l+32 become 16 contiguous bytes per lane: lane l takes
  // d = 16p + [0,8) (its e and the partner's), lane l+32 d = 16p + [8,16)
  // (the partner's f and its own), by one row-swap per dword.
  auto store16 = [&](T* row_p16, const T4& e, const T4& f) {
    const auto w0 = __builtin_amdgcn_permlane32_swap(bit_cast<uint2>(e).x, bit_cast<uint2>(f).x, false, false);
    const auto w1 = __builtin_amdgcn_permlane32_swap(bit_cast<uint2>(e).y, bit_cast<uint2>(f).y, false, false);
    if (row_ok) *reinterpret_cast<uint4*>(row_p16 + 8 * lh) = uint4{w0[0], w1[0], w0[1], w1[1]};
  };
  const float lt = pair_sum(l_run);
  if constexpr (S == 2) {
    constexpr int DH = DT / 2;
    float2* mls = reinterpret_cast<float2*>(masks);  // [stream][row]
    // O^T of d-tiles [DH*(1-ks), DH*(1-ks) + DH), lane-major: the other
    // stream's wave of row group rg reads the same lane positions
    auto xbuf = [&](int src_ks, int dl, int q) {
      return ring + ((((src_ks * RG + rg) * DH + dl) * 4 + q) * 64 + lane) * 16;
    };
    if (lh == 0) mls[ks * ROWS + r] = make_float2(m_run, lt);
    // stream KS keeps d-tiles [DH*KS, DH*KS + DH) (compile-time indices:
    // a runtime index into o[] would move the accumulators to scratch)
    auto merge = [&](auto ks_c) {
      constexpr int KS = decltype(ks_c)::value, GIVE = DH * (1 - KS), KEEP = DH * KS;
#pragma unroll
      for (int dl = 0; dl < DH; ++dl)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<f32x4*>(xbuf(KS, dl, q)) =
              f32x4{o[GIVE + dl][4 * q], o[GIVE + dl][4 * q + 1], o[GIVE + dl][4 * q + 2], o[GIVE + dl][4 * q + 3]};
      sync_lds();
      const float2 other = mls[(1 - KS) * ROWS + r];
      f32x4 xo[DH][4];
#pragma unroll
      for (int dl = 0; dl < DH; ++dl)
#pragma unroll
        for (int q = 0; q < 4; ++q) xo[dl][q] = *reinterpret_cast<const f32x4*>(xbuf(1 - KS, dl, q));
      const float M = fmaxf(m_run, other.x);
      // weights 2^((m_s - M) * scale); 0 for a stream that saw no key
      const float w0 = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f((m_run - M) * sl2);
      const float w1 = (other.x == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f((other.x - M) * sl2);
      const float L = w0 * lt + w1 * other.y;
      const float inv = L > 0.f ? 1.f / L : empty_inv;  // empty partial: O = 0, weight 0 in the combine
      const float a0 = w0 * inv, a1 = w1 * inv;
#pragma unroll
      for (int dl = 0; dl < DH; ++dl)
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          T4 e, f;  // element quads q = 2p, 2p+1
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            e[i] = (T)(a0 * o[KEEP + dl][8 * p + i] + a1 * xo[dl][2 * p][i]);
            f[i] = (T)(a0 * o[KEEP + dl][8 * p + 4 + i] + a1 * xo[dl][2 * p + 1][i]);
          }
          store16(dst + (KEEP + dl) * 32 + 16 * p, e, f);
        }
      if (KS == 0 && lh == 0 && row_ok) put_ml(M, L);
    };
    if (ks == 0) merge(std::integral_constant<int, 0>{});
    else merge(std::integral_constant<int, 1>{});
  } else {
    const float inv = lt > 0.f ? 1.f / lt : empty_inv;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        T4 e, f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          e[i] = (T)(o[dt][8 * p + i] * inv);
          f[i] = (T)(o[dt][8 * p + 4 + i] * inv);
        }
        store16(dst + dt * 32 + 16 * p, e, f);
      }
    if (lh == 0 && row_ok) put_ml(m_run, lt);
  }
  TSFA_STAMP(51);
  TSFA_CYC_STORE;
}

// Merge of the n_slots partials of workspace row R of (batch, kv head) bk
// into O (and the row's LSE when asked): kEpt outputs per thread, part
// selects them.  16-byte loads and stores (measured 19.0 -> 12.8 us at B=16
// against 8-byte accesses, no change at B=1); up to NB slots are loaded
// together (one memory round trip for the usual slot counts) and folded in
// branch-free (an empty partial has weight 0).  NB is the smallest of 2, 4,
// 8, 16 that covers n_slots (a batch past n_slots repeats the last slot's
// loads: 16-slot batches on the 2-slot plan of the 16-sequence decode shape
// cost 17.0 us per combine against 7.0).
constexpr int kEpt = 8;
constexpr int kCombineThreads = 128;

// GR > 1: the row's slots are split between GR groups of D/kEpt threads
// (group h takes slots h, h+GR, ...), merged through lane exchanges, and
// group 0 writes the row: GR times the threads for the same 16-byte loads,
// 1/GR of the conversions and multiply-adds per thread (the combine is bound
// by those VALU instructions at one or two waves per SIMD, not by its loads).
template <typename T, int D, int NB, int GR = 1, typename PT = T>
__device__ inline void merge_row(const CombineArgs& a, int64_t bk, int R, int part, int half = 0) {
  const int64_t TG = (int64_t)a.q_len * a.group;
  const int t = R / a.group, g = R - t * a.group;
  const int kvh = (int)(bk % a.num_kv_heads), b = (int)(bk / a.num_kv_heads);
  const int h = kvh * a.group + g;
  const int64_t r0 = bk * a.n_slots * TG + R;
  const float2* ml = a.ws_ml + r0;
  const PT* src = static_cast<const PT*>(a.ws_o) + r0 * D + part * kEpt;
  const int64_t slot_stride = TG * D;
  typedef T TV __attribute__((ext_vector_type(kEpt)));
  typedef PT PV __attribute__((ext_vector_type(kEpt)));

  // Running merge over batches of slots: a batch's (m, l) pairs and partial
  // vectors are loaded together, then folded into (M, L, acc) with the same
  // re-basing as the online softmax.
  float mx = -INFINITY, l = 0.f;
  float acc[kEpt];
#pragma unroll
  for (int e = 0; e < kEpt; ++e) acc[e] = 0.f;
  constexpr int SS = GR;  // slot step of this thread
  for (int s0 = half; s0 < a.n_slots; s0 += SS * NB) {
    const int nb = min(NB, (a.n_slots - s0 + SS - 1) / SS);
    float2 v[NB];
    PV x[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int s = s0 + SS * min(i, nb - 1);  // duplicates of the last slot get weight 0 below
      v[i] = ml[s * TG];
      x[i] = *reinterpret_cast<const PV*>(src + s * slot_stride);
    }
    float bm = mx;
#pragma unroll
    for (int i = 0; i < NB; ++i) bm = (i < nb) ? fmaxf(bm, v[i].x) : bm;
    if (bm != -INFINITY && bm != mx) {  // re-base the running sums on the new max
      const float alpha = (mx == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f((mx - bm) * a.scale_log2);
      l *= alpha;
#pragma unroll
      for (int e = 0; e < kEpt; ++e) acc[e] *= alpha;
      mx = bm;
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      // weight of partial s: l_s * 2^((m_s - M) * scale); 0 for an empty partial
      const float w = (i >= nb || v[i].x == -INFINITY) ? 0.f
                                                      : v[i].y * __builtin_amdgcn_exp2f((v[i].x - mx) * a.scale_log2);
      l += w;
#pragma unroll
      for (int e = 0; e < kEpt; ++e) acc[e] += w * (float)x[i][e];
    }
  }
  if constexpr (GR > 1) {
    // the other groups' (M, L, acc) from lane ^ off (off = D/kEpt, 2*D/kEpt,
    // ...); an empty group (M = -inf) weighs 0, and all empty leave l = 0
#pragma unroll
    for (int off = D / kEpt; off < GR * (D / kEpt); off *= 2) {
      const float pm = __shfl_xor(mx, off), pl = __shfl_xor(l, off);
      float pacc[kEpt];
#pragma unroll
      for (int e = 0; e < kEpt; ++e) pacc[e] = __shfl_xor(acc[e], off);
      const float M = fmaxf(mx, pm);
      const float w0 = (mx == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f((mx - M) * a.scale_log2);
      const float w1 = (pm == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f((pm - M) * a.scale_log2);
      l = w0 * l + w1 * pl;
#pragma unroll
      for (int e = 0; e < kEpt; ++e) acc[e] = w0 * acc[e] + w1 * pacc[e];
      mx = M;
    }
    if (half != 0) return;
  }
  // l == 0 (no visible key anywhere) gives 0 * inf = NaN, as acc / l_i does in
  // the reference (one reciprocal instead of kEpt divisions).
  const float inv_l = 1.f / l;
  TV out;
#pragma unroll
  for (int i = 0; i < kEpt; ++i) out[i] = (T)(acc[i] * inv_l);
  if (a.lse != nullptr && part == 0) {
    // log-sum-exp of sm_scale * q.k over the row's visible keys: M and l are
    // in the exp2 domain of |sm_scale| * log2(e); -inf for a row with no key
    const float lse2 = (l > 0.f) ? mx * a.scale_log2 + __log2f(l) : -INFINITY;
    a.lse[((int64_t)b * a.num_heads + h) * a.q_len + t] = lse2 * 0.69314718055994531f;
  }
  // O leaves by non-temporal stores: no dirty O lines stay in the L2 for the
  // end-of-kernel write-back (the Llama-3-8B decode shape: 16.5-16.9 ->
  // 16.2-16.5 us per call, same-box A/B; the combine alone is unchanged)
  T* dst = static_cast<T*>(a.o) + b * a.sob + (int64_t)h * a.soh + (int64_t)t * a.som + part * kEpt;
  __builtin_nontemporal_store(out, reinterpret_cast<TV*>(dst));
}

// Merge the n_slots partials of every row and write O.  Threads walk the
// workspace rows in order (coalesced partial loads).
template <typename T, int D, int NB, int GR = 1, typename PT = T>
__global__ __launch_bounds__(kCombineThreads) void combine_kernel(const CombineArgs a) {
  constexpr int TPR = D / kEpt;
  static_assert(GR * TPR <= 64 && kCombineThreads % (GR * TPR) == 0, "a row's groups share one wave");
  constexpr int RPB = kCombineThreads / (TPR * GR);  // rows per block
  const int x = blockIdx.x & 7;
  const int64_t TG = (int64_t)a.q_len * a.group;
  const int64_t row = a.xcd_row[x] + (int64_t)(blockIdx.x >> 3) * RPB + threadIdx.x / (GR * TPR);  // over B*Hkv*TG
  // (a whole row's threads leave together: its groups exchange within it)
  if (row >= a.xcd_row[x + 1]) return;
  const int64_t bk = row / TG;
  merge_row<T, D, NB, GR, PT>(a, bk, (int)(row - bk * TG), (int)(threadIdx.x % TPR), (int)(threadIdx.x / TPR) % GR);
}

template <typename T, int D, int S, bool PAGED, bool C32 = false, int FAST = 0>
int launch_split(const SplitArgs& args, const Plan& p, hipStream_t stream) {
  // The LDS limit attribute is set once per device (the first call on a
  // device, before any graph capture that replays it).
  static std::atomic<uint64_t> attr_set{0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return TSFA_ERR_DEVICE;
  const uint64_t bit = 1ull << (dev & 63);
  if ((attr_set.load(std::memory_order_acquire) & bit) == 0) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&split_kernel<T, D, S, PAGED, C32, FAST>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)p.lds_bytes) != hipSuccess)
      return TSFA_ERR_LAUNCH;
    attr_set.fetch_or(bit, std::memory_order_acq_rel);
  }
  hipLaunchKernelGGL((split_kernel<T, D, S, PAGED, C32, FAST>), dim3(p.grid), dim3(kWaves * 64), p.lds_bytes, stream,
                     args);
  return hipGetLastError() == hipSuccess ? TSFA_OK : TSFA_ERR_LAUNCH;
}

// Measurement hook (per host thread): which of the two kernels a call
// launches (bit 0 split-KV, bit 1 combine).
thread_local int g_kernel_mask = 3;

// The unchecked prefix ring steps load every prefix unit whole: the last,
// partial one too (its keys past the prefix are masked at the end of its
// run), so they need the prefix rounded up to whole units within kv_len.
inline bool prefix_units_in_kv(const SplitArgs& sa) {
  return ((int64_t)sa.prefix_len + kUnitKeys - 1) / kUnitKeys * kUnitKeys <= (int64_t)sa.kv_len;
}

// Contiguous calls whose prefix units lie within kv_len take the kernel with
// the unchecked prefix ring steps (split_kernel<..., FAST>): 1 with plain K/V
// loads, 2 with non-temporal ones (instantiated for two streams, where the
// planner asks for them); 0 keeps the checked steps.  The run-base path
// needs a row stride of at least D in both K and V.
template <int D> inline int fast_ring(const SplitArgs& sa, const Plan& p, const Config& cfg) {
  if (cfg.fast_ring == 0 || !prefix_units_in_kv(sa) || sa.skn < D || sa.svn < D) return 0;
  if (!sa.kv_nt) return 1;
  return p.streams == 2 ? 2 : 0;
}

// The kernels of one call, for the switches of one configuration snapshot
// (cfg, read once by the caller).
template <typename T, int D, bool PAGED>
int launch_all(const SplitArgs& sa_in, const CombineArgs& ca, const Plan& p, const Config& cfg,
               hipStream_t stream) {
  // contiguous: the unchecked-step flavour, +4 for the kernel that writes O
  // itself (one-slot plans, with the unchecked steps only): then its
  // "partial" goes straight to O and the combine is not launched
  const bool fp = cfg.fast_ring != 0 && prefix_units_in_kv(sa_in);
  const int fm0 = PAGED ? (fp ? 1 : 0) : fast_ring<D>(sa_in, p, cfg);
  const int fm = fm0 != 0 && sa_in.direct_out ? fm0 | 4 : fm0;
  SplitArgs sa = sa_in;
  if (fm & 4) sa.ws_o = ca.o;
  // paged, head_dim 128, unchecked steps, one key stream (or two with a
  // cache below 4 GB, or two writing O): the instance that takes the steady
  // refills' pages from an LDS table of the run's page ids (FAST | 8), when
  // every run spans at most kPageTabInts pages and the cache's rows take the
  // row-base path.  (Two streams over a larger cache with partials: that
  // instance spilled 107 SGPRs, 589 reloads in its checked-step loop.)
  bool ptab = false;
  Plan pt = p;
  if constexpr (PAGED && D == 128) {
    int max_lds = 0;
    // a run starts on a 32-key boundary: page-aligned for pages of 16 or 32
    // keys, so it spans ceil(keys / page) pages, one more with larger pages
    const int64_t ps = (int64_t)1 << sa.page_shift;
    const int64_t run_pages = ((int64_t)p.units_per_split * kUnitKeys + ps - 1) / ps + (ps > kUnitKeys ? 1 : 0);
    // (its 64-bit refills take the page and row strides in 32-bit bytes)
    const bool strides32 = sa.cache32 || ((uint64_t)sa.cps * 2 < (1ull << 32) &&
                                          (uint64_t)ps * (uint64_t)sa.crs * 2 < (1ull << 32));
    ptab = (p.streams == 1 || sa.cache32 || fm == 5) && strides32 && fm != 0 && run_pages <= kPageTabInts &&
           sa.crs >= D && device_max_lds_per_block(&max_lds) == TSFA_OK && (size_t)max_lds >= kPagedLdsBytes;
    pt.lds_bytes = kPagedLdsBytes;
  }
  if (g_kernel_mask & 1) {
    int st;
    // paged: the unchecked steps need only the prefix units within kv_len
    // (the page-table path serves every refill); FAST 5 also writes O
    // (one-slot plans)
    if constexpr (PAGED)
      st = (sa.cache32 && p.streams == 2)
               ? (fm == 5   ? (ptab ? launch_split<T, D, 2, true, true, D == 128 ? 13 : 5>(sa, pt, stream)
                                    : launch_split<T, D, 2, true, true, 5>(sa, p, stream))
                  : fm == 1 ? (ptab ? launch_split<T, D, 2, true, true, D == 128 ? 9 : 1>(sa, pt, stream)
                                    : launch_split<T, D, 2, true, true, 1>(sa, p, stream))
                            : launch_split<T, D, 2, true, true>(sa, p, stream))
           : p.streams == 2 ? (fm == 5   ? (ptab ? launch_split<T, D, 2, true, false, D == 128 ? 13 : 5>(sa, pt, stream)
                                                 : launch_split<T, D, 2, true, false, 5>(sa, p, stream))
                               : fm == 1 ? launch_split<T, D, 2, true, false, 1>(sa, p, stream)
                                         : launch_split<T, D, 2, true, false>(sa, p, stream))
                            : (fm == 5   ? (ptab ? launch_split<T, D, 1, true, false, D == 128 ? 13 : 5>(sa, pt, stream)
                                                 : launch_split<T, D, 1, true, false, 5>(sa, p, stream))
                               : fm == 1 ? (ptab ? launch_split<T, D, 1, true, false, D == 128 ? 9 : 1>(sa, pt, stream)
                                                 : launch_split<T, D, 1, true, false, 1>(sa, p, stream))
                                         : launch_split<T, D, 1, true, false>(sa, p, stream));
    else
      st = p.streams == 2 ? (fm == 6   ? launch_split<T, D, 2, false, false, 6>(sa, p, stream)
                             : fm == 5 ? launch_split<T, D, 2, false, false, 5>(sa, p, stream)
                             : fm == 2 ? launch_split<T, D, 2, false, false, 2>(sa, p, stream)
                             : fm == 1 ? launch_split<T, D, 2, false, false, 1>(sa, p, stream)
                                       : launch_split<T, D, 2, false, false>(sa, p, stream))
                          : (fm == 5   ? launch_split<T, D, 1, false, false, 5>(sa, p, stream)
                             : fm == 1 ? launch_split<T, D, 1, false, false, 1>(sa, p, stream)
                                       : launch_split<T, D, 1, false, false>(sa, p, stream));
    if (st != TSFA_OK) return st;
  }
  // no combine when the split kernel wrote O
  if ((g_kernel_mask & 2) == 0 || (fm & 4)) return TSFA_OK;
  // Each XCD merges the rows of the chunks its split workgroups ran (item i
  // runs on XCD i / items_per_xcd; a chunk's rows go to the XCD of its middle
  // slot), so the partials are read from the L2 they were written to and the
  // next call's partial stores find no copies in other XCDs' L2s.
  CombineArgs c = ca;
  // more than 4 slots: 2 groups of threads per row; more than 8: 4 groups
  // (16 slots at the Llama-3-8B decode shape: 3.86 us per combine with one
  // group, 3.60 with two, 3.19 with four; same-call A/B)
  const int gr = ca.n_slots > 8 ? 4 : ca.n_slots > 4 ? 2 : 1;
  const int RPB = kCombineThreads / (D / kEpt) / gr;
  const int64_t TG = (int64_t)ca.q_len * ca.group;
  const int64_t groups = (int64_t)ca.batch * ca.num_kv_heads * p.n_chunks;
  auto first_row = [&](int64_t g) { return (g / p.n_chunks) * TG + (g % p.n_chunks) * p.rows_per_chunk; };
  auto mid_item = [&](int64_t g) {
    return g % p.n_chunks + (int64_t)p.n_chunks * (p.n_slots / 2 + (int64_t)p.n_slots * (g / p.n_chunks));
  };
  int64_t most = 0, g = 0;
  for (int x = 0; x < 8; ++x) {
    c.xcd_row[x] = first_row(g);
    // first group past XCD x (mid_item is increasing in g)
    int64_t lo = g, hi = groups;
    while (lo < hi) {
      const int64_t m = (lo + hi) / 2;
      if (mid_item(m) / p.items_per_xcd > x) hi = m; else lo = m + 1;
    }
    g = lo;
    most = std::max(most, (first_row(g) - c.xcd_row[x] + RPB - 1) / RPB);
  }
  c.xcd_row[8] = (int64_t)ca.batch * ca.num_kv_heads * TG;
  const unsigned blocks = (unsigned)(8 * most);
  if (blocks == 0) return TSFA_OK;
  const int ns = ca.n_slots;
  if (ns <= 2)
    hipLaunchKernelGGL((combine_kernel<T, D, 2>), dim3(blocks), dim3(kCombineThreads), 0, stream, c);
  else if (ns <= 4)
    hipLaunchKernelGGL((combine_kernel<T, D, 4>), dim3(blocks), dim3(kCombineThreads), 0, stream, c);
  else if (ns <= 8)
    hipLaunchKernelGGL((combine_kernel<T, D, 4, 2>), dim3(blocks), dim3(kCombineThreads), 0, stream, c);
  else
    hipLaunchKernelGGL((combine_kernel<T, D, 4, 4>), dim3(blocks), dim3(kCombineThreads), 0, stream, c);
  return hipGetLastError() == hipSuccess ? TSFA_OK : TSFA_ERR_LAUNCH;
}

// ------------------------------------------------------------ generic kernel
// Head dims above 128 (bf16 / fp16) and fp32 inputs.  The same semantics as
// split_kernel (tree_sparse_flashattn.py:211-339) with a simpler structure:
// a workgroup is 4 waves of 32 packed query rows (a 128-row chunk, r = t*G +
// g) over one split of the key axis in units of 32 keys; prefix keys are
// visible, tree keys by the CSR record of the row's q-block (FULL, or the
// MIXED bit).  S^T = K Q^T and O^T += V^T P^T on
// v_mfma_f32_32x32x16_{bf16,f16} (V^T from ds_read_b64_tr_b16) or
// v_mfma_f32_32x32x2_f32, with the key order of the P V product permuted so
// that P^T comes straight from the S^T accumulator.  Every split writes a
// partial (O / l in the input dtype, fp32 (m, l)) that combine_kernel merges.
// Units stream HBM -> LDS through a ring of kGenStages(stage bytes) stages
// (global_load_lds, NSTG - 1 units ahead).  In the 16-bit instances 16-byte
// chunk c of key row k sits at chunk position c ^ (k & 15) in the K tile and
// c ^ ((k & 3) << 2) in the V tile, so the 16 key rows of a K operand read
// and the 4 rows x 4 chunks of a transposing V^T read spread over the LDS
// banks (a 512-byte row stride maps every row to the same banks; XOR with
// k & 15 on V only permutes chunks inside their group of 4, which measured
// bank conflicts on half of the LDS cycles).  The fp32 instances keep
// rows unswizzled: their 4-byte operand reads then use immediate offsets
// (with the XOR, one address register per read spills the head_dim 256
// instance), and their 32x32x2 MFMAs, at 1/16 of the 16-bit rate, bound
// the loop anyway.
struct GenArgs {
  const void* q;
  const void* k;
  const void* v;
  const int32_t* row_ptr;
  const int32_t* col_idx;
  const int8_t* blk_type;
  const int32_t* payload;
  const int32_t* offset;
  int64_t ms[5];  // per-sequence strides of the five metadata arrays (0: one tree)
  int64_t sqb, sqh, sqm, skb, skh, skn, svb, svh, svn;
  float scale_log2;  // |sm_scale| * log2(e), never 0
  int neg_q;         // sm_scale < 0: Q enters negated
  int num_kv_heads, group, q_len, kv_len, prefix_len, block_m, block_n;
  int n_chunks, n_units, units_per_split, n_slots;
  void* ws_o;      // [B*Hkv][n_slots][q_len*G][D] partial O / l: the input dtype (fp32 for fp32)
  float2* ws_ml;   // [B*Hkv][n_slots][q_len*G] (m, l)
  void* out;       // direct: O [B, Hq, q_len, D] (strides sob, soh, som; d stride 1)
  int64_t sob, soh, som;
  int direct;      // one split and no LSE: the kernel writes O, no partials, no combine
};

// 128-row chunks: 4 row groups of 32.  The 16-bit instances (head_dim 256)
// run 8 waves, waves w and w + 4 sharing row group w % 4 and each owning
// half of O's columns: both compute the group's S^T and softmax (1.5x the
// MFMAs of one wave per group), but a wave then holds 64 O accumulators
// instead of 128 and everything fits the 256 VGPRs, two waves per SIMD
// (with 128 accumulators, Q and the temporaries the compiler parked O in
// AGPRs and copied all of it to VGPRs on every unit).  fp32 keeps 4 waves.
constexpr int kGenRows = 128;
template <typename T> constexpr int gen_waves() { return sizeof(T) == 2 ? 8 : 4; }
// Tree units per split whose visibility words the prologue builds into LDS
// (kGenTreeUnits x 128 rows x 4 bytes after the ring).  Splits with more take
// the gen_kernel<..., TW = false> instance, which builds each unit's words in
// the loop: its global loads then make the compiler wait for every vector
// load in flight (vmcnt(0), which counts the ring's DMA) on every unit, so
// the ring drains each step.
constexpr int kGenTreeUnits = 32;
constexpr size_t kGenTreeBytes = (size_t)kGenTreeUnits * kGenRows * 4;
// Ring stages for a stage of K+V bytes: as many as fit 128 KB, at least 2,
// at most 4 (head_dim 256 and fp32 head_dim 128 hold one workgroup per CU by
// their registers; fp32 head_dim 64 fits two at 64 KB each).
constexpr int kGenStages(int stage_bytes) {
  return 131072 / stage_bytes < 2 ? 2 : (131072 / stage_bytes > 4 ? 4 : 131072 / stage_bytes);
}

template <typename T, int D, bool TW>
__global__ __launch_bounds__(gen_waves<T>() * 64) void gen_kernel(const GenArgs a) {
  constexpr bool F32 = std::is_same<T, float>::value;
  constexpr int NW = gen_waves<T>();  // waves
  constexpr int DS = NW / 4;          // column parts of O (waves per row group)
  constexpr int ROWB = D * (int)sizeof(T);  // bytes of one key row
  constexpr int CPR = ROWB / 16;            // 16-byte chunks per row
  constexpr int TILE = 32 * ROWB;           // bytes of one unit's K (or V)
  constexpr int SB = 2 * TILE;              // ring stage: K then V
  constexpr int NSTG = kGenStages(SB);
  constexpr int LPW = SB / 1024 / NW;  // 1 KB loads per wave per unit
  constexpr int DT = D / 32 / DS;      // O d-tiles of a wave
  constexpr int KS = F32 ? D / 2 : D / 16;  // k-steps of S^T
  // chunk c of row k at c ^ (k & SWZ) in K, c ^ ((k & SWV) << 2) in V
  constexpr int SWZ = F32 ? 0 : 15, SWV = F32 ? 0 : 3;
  static_assert(CPR >= 16 && LPW >= 1 && LPW * (NSTG - 2) < 64 && SB % (1024 * NW) == 0, "generic ring");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 31, lh = lane >> 5;
  const int rg = wave % 4, dh = wave / 4;  // row group; O columns [dh * D/DS, (dh+1) * D/DS)
  const int chunk = blockIdx.x % a.n_chunks;
  const int rest = blockIdx.x / a.n_chunks;
  const int slot = rest % a.n_slots, bk = rest / a.n_slots;
  const int b = bk / a.num_kv_heads, kvh = bk % a.num_kv_heads;
  const int G = a.group, TG = a.q_len * G;
  const int r = chunk * kGenRows + rg * 32 + ln;  // the lane's packed row
  const bool row_ok = r < TG;
  const int R = min(r, TG - 1);
  const int t = R / G, g = R - t * G;
  const float sl2 = a.scale_log2;

  const T* kbase = static_cast<const T*>(a.k) + b * a.skb + kvh * a.skh;
  const T* vbase = static_cast<const T*>(a.v) + b * a.svb + kvh * a.svh;
  const T* qrow = static_cast<const T*>(a.q) + b * a.sqb + (int64_t)(kvh * G + g) * a.sqh + (int64_t)t * a.sqm;

  // Q^T operand: 16-bit, lane (ln, lh) holds d = 16kk + 8lh + [0, 8) of its
  // row; fp32, d = 2kk + lh (16-byte loads, the lane keeps its two words of
  // each).  Q is negated for a negative scale.
  typedef typename std::conditional<F32, float, i16x8>::type QF;
  QF qf[KS];
#pragma unroll
  for (int kk = 0; kk < KS; kk += (F32 ? 2 : 1)) {
    if constexpr (F32) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(qrow + 2 * kk);
      qf[kk] = a.neg_q ? -(lh ? x[1] : x[0]) : (lh ? x[1] : x[0]);
      qf[kk + 1] = a.neg_q ? -(lh ? x[3] : x[2]) : (lh ? x[3] : x[2]);
    } else {
      qf[kk] = *reinterpret_cast<const i16x8*>(qrow + 16 * kk + 8 * lh) ^ (short)(a.neg_q ? 0x8000 : 0);
    }
  }

  // The lane's row in the tree record: token t, q-block t / BM.
  const int32_t* rp = a.row_ptr + b * a.ms[0];
  const int32_t* ci = a.col_idx + b * a.ms[1];
  const int8_t* bt = a.blk_type + b * a.ms[2];
  const int32_t* pl = a.payload + b * a.ms[3];
  const int32_t* of = a.offset + b * a.ms[4];
  const int qb = t / a.block_m, tl = t - qb * a.block_m;
  const int e_lo = rp[qb], e_hi = rp[qb + 1];
  // Visibility of keys k0 .. k0+31 for the lane's row: prefix keys, then the
  // tree keys of the row's FULL and MIXED blocks (tree_sparse_flashattn.py:
  // 266-270, :307-318); keys past kv_len are not visible.
  auto vis_word = [&](int k0) {
    const int P = a.prefix_len, BN = a.block_n;
    const int np = min(max(P - k0, 0), 32);
    uint32_t w = np >= 32 ? 0xffffffffu : ((1u << np) - 1u);
    const int c_lo = max(k0, P) - P, c_hi = min(k0 + 32, a.kv_len) - P;  // tree columns of the unit
    if (c_lo < c_hi) {
      for (int e = e_lo; e < e_hi; ++e) {
        const int cb = ci[e] * BN;
        const int lo = max(cb, c_lo), hi = min(cb + BN, c_hi);
        if (lo >= hi) continue;
        const bool full = bt[e] != TSFA_MIXED_BLOCK;  // any kind but MIXED (tree_sparse_flashattn.py:313-318)
        const int off = full ? 0 : of[e];
        // columns lo .. hi-1 are flat bits f0 .. f1-1 of the block's row-major
        // bitset: one payload word per run of bits inside a word
        const int f0 = tl * BN + (lo - cb), f1 = tl * BN + (hi - cb);
        for (int f = f0; f < f1;) {
          const int b0 = f & 31, nb = min(32 - b0, f1 - f);
          const uint32_t word = full ? 0xffffffffu : (uint32_t)pl[off + (f >> 5)];
          const uint32_t bits = (word >> b0) & (nb == 32 ? 0xffffffffu : ((1u << nb) - 1u));
          w |= bits << (cb + (f - tl * BN) + P - k0);
          f += nb;
        }
      }
    }
    return w;
  };

  // The wave's DMA share of a unit: the first NW/2 waves move the K tile,
  // the others the V tile (LPW loads of 1 KB each, NW/2 * LPW KB = one
  // tile).  Load i of wave w moves tile chunks x = ((w % (NW/2))*LPW + i)*64
  // + lane, landing at tile + 16x: key row x / CPR, chunk position x % CPR,
  // which holds the row's chunk (x % CPR) ^ (row & SWZ) (K) or
  // (x % CPR) ^ ((row & SWV) << 2) (V).  Rows past kv_len repeat the last
  // key (never visible).
  constexpr int HW = NW / 2;
  static_assert(HW * LPW * 1024 == TILE, "one tile per half of the waves");
  const bool dma_v = wave >= HW;
  const T* dbase = dma_v ? vbase : kbase;
  const int64_t dstride = dma_v ? a.svn : a.skn;
  const uint32_t ring = lds_addr(smem);
  const int u_lo = slot * a.units_per_split;
  const int n = min(a.units_per_split, a.n_units - u_lo);
  auto issue = [&](int j) {  // run unit j into stage j % NSTG
    const int k0 = (u_lo + j) * 32;
    const uint32_t st = ring + (uint32_t)((j % NSTG) * SB + (dma_v ? TILE : 0) + (wave % HW) * LPW * 1024);
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int x = ((wave % HW) * LPW + i) * 64 + lane;
      const int row = x / CPR;
      const int col = ((x % CPR) ^ (dma_v ? (row & SWV) << 2 : (row & SWZ))) * (16 / (int)sizeof(T));
      const int64_t key = min(k0 + row, a.kv_len - 1);
      dma16(dbase + key * dstride + col, st + (uint32_t)i * 1024u);
    }
  };
  // LDS byte offset of chunk c (16 B) of key row k within the K / V tile
  auto swz = [](int k, int c) { return k * ROWB + ((c ^ (k & SWZ)) << 4); };
  auto swv = [](int k, int c) { return k * ROWB + ((c ^ ((k & SWV) << 2)) << 4); };

  f32x16 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[dt][i] = 0.f;
  float m_run = -INFINITY, m_lim = -INFINITY, l_run = 0.f;
  const float thr_raw = kRescaleLog2 / sl2;  // re-base past 2^8 growth

  // Units holding a tree column: u >= P / 32 (the unit at P / 32 may also
  // hold prefix keys).  TW: their visibility words of the chunk's rows,
  // built once below into tw[unit - ut0][row].
  const int ut0 = max(u_lo, a.prefix_len / 32);
  const int nt = max(0, u_lo + n - ut0);
  uint32_t* tw = reinterpret_cast<uint32_t*>(smem + NSTG * SB);

  // ring prologue: Q (compiler-tracked loads, consumed here so the compiler's
  // own waits never count the ring's), the first NSTG - 1 units, and with TW
  // the tree words (their loads land behind the units')
  for (int j = 0; j < NSTG - 1 && j < n; ++j) issue(j);
  if constexpr (TW) {
    for (int i = 0; i < nt; ++i) {
      const uint32_t w = row_ok ? vis_word((ut0 + i) * 32) : 0u;
      if (lh == 0 && dh == 0) tw[i * kGenRows + rg * 32 + ln] = w;
    }
  }
  vm_wait<0>();
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) asm volatile("" : : "v"(qf[kk]));
  for (int j = 0; j < n; ++j) {
    // unit j landed for every wave; stage (j - 1) % NSTG is free
    wait_units<LPW, NSTG - 2>(min(n - 1 - j, NSTG - 2));
    sync_lds();
    if (j + NSTG - 1 < n) issue(j + NSTG - 1);
    const unsigned char* kt = smem + (j % NSTG) * SB;
    const unsigned char* vt = kt + TILE;
    const int k0 = (u_lo + j) * 32;
    // S^T: MFMA row = key, column = query row; lane (ln, lh) element i is key
    // 8*(i/4) + 4*lh + i%4 of row ln
    // (K read KA k-steps ahead of its MFMA, fenced: left to itself the
    // scheduler reads one step ahead and every MFMA waits an LDS latency)
    f32x16 s;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = 0.f;
    constexpr int KA = F32 ? 8 : 4;
    typedef typename std::conditional<F32, float, i16x8>::type KF;
    KF kf[KS];
    auto rk = [&](int kk) {
      if constexpr (F32) {
        const int wd = 2 * kk + lh;  // word of the row
        kf[kk] = *reinterpret_cast<const float*>(kt + swz(ln, wd >> 2) + (wd & 3) * 4);
      } else {
        kf[kk] = *reinterpret_cast<const i16x8*>(kt + swz(ln, 2 * kk + lh));
      }
    };
#pragma unroll
    for (int kk = 0; kk < KA; ++kk) rk(kk);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      if (kk + KA < KS) rk(kk + KA);
      if constexpr (F32) {
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[kk], qf[kk], s, 0, 0, 0);
      } else {
        s = Mma<T>::run(bit_cast<typename Mma<T>::vec8>(kf[kk]), bit_cast<typename Mma<T>::vec8>(qf[kk]), s);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // mask (units with a tree column only: every key of the others is a
    // visible prefix key), online softmax (tree_sparse_flashattn.py:272-279,
    // :320-327)
    if (u_lo + j >= ut0) {
      uint32_t w;
      if constexpr (TW) w = tw[(u_lo + j - ut0) * kGenRows + rg * 32 + ln];
      else w = row_ok ? vis_word(k0) : 0u;
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (!((w >> (8 * (i >> 2) + 4 * lh + (i & 3))) & 1u)) s[i] = -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[i]);
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    const float rmax = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    // The reference point m_run moves only when a score passes it by more
    // than 2^kRescaleLog2 (or on the row's first visible key: m_lim is -inf
    // until then), so p <= 2^8 and O is rescaled on few units: with 32 rows
    // per wave some row's exact maximum moves on almost every unit, and each
    // rescale moves the D / 2 accumulators of a lane through the VALU.
    // Exact for any consistent reference point (tree_sparse_flashattn.py:
    // 272-279 rescales at every block); a row that sees one key still gets
    // p = 2^0 = 1, O = V bit for bit.
    const bool need = rmax > m_lim;
    const float m_new = need ? rmax : m_run;
    // alpha = 0 on the first visible key (O and l are still 0)
    const float alpha = need ? __builtin_amdgcn_exp2f((m_run - m_new) * sl2) : 1.f;
    m_run = m_new;
    m_lim = m_new + thr_raw;
    // p = 2^((s - m_run) * scale); 0 for masked keys and while no key is visible
    float p[16], ps = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      p[i] = (m_new == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f((s[i] - m_new) * sl2);
      ps += p[i];
    }
    l_run = l_run * alpha + ps;
    if (__ballot(need) != 0) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
    }
    // O^T += V^T P^T, P rounded to the input dtype (tree_sparse_flashattn.py:278)
    if constexpr (F32) {
      // k-step i: keys 8*(i/4) + 4*k + i%4 (k = 0, 1), lane (ln, lh) gives its
      // element i of P^T and V[key 8*(i/4) + 4*lh + i%4][32*dt + ln] of V^T
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = 8 * (i >> 2) + 4 * lh + (i & 3);
          const int wd = 32 * (dh * DT + dt) + ln;
          const float vv = *reinterpret_cast<const float*>(vt + swv(key, wd >> 2) + (wd & 3) * 4);
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv, p[i], o[dt], 0, 0, 0);
        }
    } else {
      typedef typename Mma<T>::vec8 V8;
      V8 pb[2];
#pragma unroll
      for (int i = 0; i < 16; ++i) pb[i >> 3][i & 7] = (T)p[i];
      // V^T fragments by the transposing LDS read: lane i of 16-lane group x
      // gets keys 16*s2 + 8*jj + 4*(x>>1) + [0,4) of d = 32*gt + 16*(x&1) + i,
      // gt = dh*DT + dt the d-tile (bytes 64*gt + 2*(16*(x&1) + 4*(i&3)) of the
      // key row: chunk 4*gt + 2*(x&1) + (i&3)/2, 8-byte half (i&3)&1)
      const int vx = lane >> 4, vi = lane & 15;
      const int vrow = 4 * (vx >> 1) + (vi >> 2);
      const int vch = 2 * (vx & 1) + ((vi & 3) >> 1), vhalf = 8 * (vi & 1);
      // P V MFMA g = (dt, s2) = (g / 2, g % 2), its V^T read VA MFMAs ahead
      constexpr int NPV = 2 * DT, VA = 3;
      i16x4 vh[NPV][2];
      auto rv = [&](int g) {
        const int dt = g >> 1, s2 = g & 1;
        const int k0r = 16 * s2 + vrow, k1r = 16 * s2 + 8 + vrow;
        vh[g][0] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (TSFA_LDS i16x4*)(vt + swv(k0r, 4 * (dh * DT + dt) + vch) + vhalf));
        vh[g][1] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (TSFA_LDS i16x4*)(vt + swv(k1r, 4 * (dh * DT + dt) + vch) + vhalf));
      };
#pragma unroll
      for (int g = 0; g < VA && g < NPV; ++g) rv(g);
#pragma unroll
      for (int g = 0; g < NPV; ++g) {
        if (g + VA < NPV) rv(g + VA);
        const i16x8 vf = __builtin_shufflevector(vh[g][0], vh[g][1], 0, 1, 2, 3, 4, 5, 6, 7);
        o[g >> 1] = Mma<T>::run(bit_cast<V8>(vf), pb[g & 1], o[g >> 1]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  const float lt = pair_sum(l_run);
  if (a.direct) {
    // a one-split plan writes the lane's row of O (token t, head kvh*G + g)
    // in the input dtype: one rounding of the fp32 result; a row that saw no
    // key gets NaN (0/0, as the reference and the combine give)
    if (row_ok) {
      typedef T T4 __attribute__((ext_vector_type(4)));
      const float inv_o = lt > 0.f ? 1.f / lt : __builtin_nanf("");
      T* dst = static_cast<T*>(a.out) + b * a.sob + (int64_t)(kvh * G + g) * a.soh + (int64_t)t * a.som +
               32 * DT * dh;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          *reinterpret_cast<T4*>(dst + 32 * dt + 8 * j + 4 * lh) =
              T4{(T)(o[dt][4 * j] * inv_o), (T)(o[dt][4 * j + 1] * inv_o), (T)(o[dt][4 * j + 2] * inv_o),
                 (T)(o[dt][4 * j + 3] * inv_o)};
    }
    return;
  }
  // partial of the lane's row: O / l in the input dtype (as the split
  // kernel's; half the bytes written here and read by the combine of fp32
  // ones) and (m, l); a split that saw no key stores O = 0 with m = -inf
  // (weight 0 in the combine)
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  const int64_t prow = ((int64_t)bk * a.n_slots + slot) * TG + r;
  if (row_ok) {
    typedef T T4 __attribute__((ext_vector_type(4)));
    T* dst = static_cast<T*>(a.ws_o) + prow * D + 32 * DT * dh;  // the wave's columns
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *reinterpret_cast<T4*>(dst + 32 * dt + 8 * j + 4 * lh) =
            T4{(T)(o[dt][4 * j] * inv), (T)(o[dt][4 * j + 1] * inv), (T)(o[dt][4 * j + 2] * inv),
               (T)(o[dt][4 * j + 3] * inv)};
    if (lh == 0 && dh == 0) a.ws_ml[prow] = make_float2(m_run, lt);
  }
}

// The generic kernel's plan: 128-row chunks, the key axis cut into n_slots
// splits of whole 32-key units: about one workgroup per compute unit, with
// the partials (written once, read once by the combine) held to at most
// the K/V bytes or 8 MB, whichever is larger (the 8B decode shape at
// head_dim 256 with fp32 partials: 16 splits, 36.8 us per call, against 40.5
// with half the K/V bytes (8 splits, half the CUs idle); twice the K/V
// bytes: the same 16).
struct GenPlan {
  int n_chunks, n_units, units_per_split, n_slots, grid;
  size_t lds_bytes, ws_acc_bytes, ws_ml_bytes;
};

inline bool gen_path(int head_dim, int dtype) { return head_dim > 128 || dtype == TSFA_DTYPE_FP32; }

inline int gen_plan(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len, int head_dim, int dtype,
                    int cus, GenPlan* p) {
  if (batch <= 0 || q_len <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 || kv_len < 1 || cus <= 0)
    return TSFA_ERR_INVALID_ARGUMENT;
  const int64_t TG = (int64_t)q_len * (num_heads / num_kv_heads);
  if (TG > INT32_MAX / 2) return TSFA_ERR_UNSUPPORTED;
  p->n_chunks = (int)((TG + kGenRows - 1) / kGenRows);
  p->n_units = ceil_div(kv_len, 32);
  const int64_t groups = (int64_t)batch * num_kv_heads * p->n_chunks;
  const size_t es = dtype == TSFA_DTYPE_FP32 ? 4 : 2;
  const double kv_bytes = 2.0 * batch * num_kv_heads * (double)kv_len * head_dim * es;
  const double slot_bytes = (double)batch * num_heads * q_len * ((double)es * head_dim + 8.0);
  const int64_t want = std::max<int64_t>(1, ((int64_t)cus + groups - 1) / groups);
  const int64_t cap = std::max<int64_t>(1, (int64_t)(std::max(kv_bytes, 8.0 * (1 << 20)) / slot_bytes));
  const int slots = (int)std::min<int64_t>(p->n_units, std::min(want, cap));
  p->units_per_split = ceil_div(p->n_units, slots);
  p->n_slots = ceil_div(p->n_units, p->units_per_split);
  const int64_t grid = groups * p->n_slots;
  if (grid > INT32_MAX / 2) return TSFA_ERR_UNSUPPORTED;
  p->grid = (int)grid;
  const int stage = 2 * 32 * head_dim * (int)es;
  p->lds_bytes = (size_t)kGenStages(stage) * stage + kGenTreeBytes;
  const size_t rows = (size_t)batch * num_heads * q_len;
  p->ws_acc_bytes = align256(rows * p->n_slots * head_dim * es);
  p->ws_ml_bytes = align256(rows * p->n_slots * 8);
  return TSFA_OK;
}

template <typename T, int D, bool TW>
int launch_gen_kernel(const GenArgs& ga, const GenPlan& p, hipStream_t stream) {
  static std::atomic<uint64_t> attr_set{0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return TSFA_ERR_DEVICE;
  const uint64_t bit = 1ull << (dev & 63);
  if (p.lds_bytes > 65536 && (attr_set.load(std::memory_order_acquire) & bit) == 0) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&gen_kernel<T, D, TW>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)p.lds_bytes) != hipSuccess)
      return TSFA_ERR_LAUNCH;
    attr_set.fetch_or(bit, std::memory_order_acq_rel);
  }
  hipLaunchKernelGGL((gen_kernel<T, D, TW>), dim3(p.grid), dim3(gen_waves<T>() * 64), p.lds_bytes, stream, ga);
  return hipGetLastError() == hipSuccess ? TSFA_OK : TSFA_ERR_LAUNCH;
}

template <typename T, int D>
int launch_gen(const GenArgs& ga, const CombineArgs& ca, const GenPlan& p, hipStream_t stream) {
  if (g_kernel_mask & 1) {
    // tree units of the fullest split: their words fit the LDS table?
    const bool tw = std::min(p.units_per_split, p.n_units - ga.prefix_len / 32) <= kGenTreeUnits;
    const int st = tw ? launch_gen_kernel<T, D, true>(ga, p, stream) : launch_gen_kernel<T, D, false>(ga, p, stream);
    if (st != TSFA_OK) return st;
  }
  if ((g_kernel_mask & 2) == 0 || ga.direct) return TSFA_OK;
  // the partials of every row merged: rows cut into 8 equal ranges, one
  // per XCD slot of the combine's block ids (no placement to follow: the
  // splits of a chunk spread over the grid)
  CombineArgs c = ca;
  constexpr int TPR = D / kEpt;
  const int gr = (ca.n_slots > 4 && 2 * TPR <= 64) ? 2 : 1;
  const int RPB = kCombineThreads / TPR / gr;
  const int64_t rows = (int64_t)ca.batch * ca.num_kv_heads * ca.q_len * ca.group;
  const int64_t per = (rows + 7) / 8;
  for (int x = 0; x <= 8; ++x) c.xcd_row[x] = std::min<int64_t>(x * per, rows);
  const int64_t blocks = 8 * ((per + RPB - 1) / RPB);
  if (blocks > INT32_MAX) return TSFA_ERR_UNSUPPORTED;
  const int ns = ca.n_slots;
  if (ns <= 2)
    hipLaunchKernelGGL((combine_kernel<T, D, 2, 1, T>), dim3((unsigned)blocks), dim3(kCombineThreads), 0, stream, c);
  else if (ns <= 4)
    hipLaunchKernelGGL((combine_kernel<T, D, 4, 1, T>), dim3((unsigned)blocks), dim3(kCombineThreads), 0, stream, c);
  else if (gr == 2)
    hipLaunchKernelGGL((combine_kernel<T, D, 4, 2, T>), dim3((unsigned)blocks), dim3(kCombineThreads), 0, stream, c);
  else
    hipLaunchKernelGGL((combine_kernel<T, D, 4, 1, T>), dim3((unsigned)blocks), dim3(kCombineThreads), 0, stream, c);
  return hipGetLastError() == hipSuccess ? TSFA_OK : TSFA_ERR_LAUNCH;
}

}  // namespace fwd
}  // namespace tsfa

using namespace tsfa;
using namespace tsfa::fwd;

namespace {

// The plan of a shape on the current device (its CU count and LDS limit),
// memoised per host thread: a call's workspace query and its launch plan the
// same shape once.
int device_plan(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len, int prefix_len, int head_dim,
                bool paged, const Config& cfg, Plan* p) {
  int cus = 0, max_lds = 0;
  if (device_cu_count(&cus) != TSFA_OK || device_max_lds_per_block(&max_lds) != TSFA_OK) return TSFA_ERR_DEVICE;
  struct Entry {
    int key[12];
    Plan plan;
    int status;
  };
  constexpr int kEntries = 4;
  thread_local Entry cache[kEntries];
  thread_local int n_cached = 0, next = 0;
  const int key[12] = {batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, head_dim, paged ? 1 : 0, cus,
                       max_lds, cfg.generation, 1};
  for (int e = 0; e < n_cached; ++e)
    if (std::equal(key, key + 12, cache[e].key)) {
      *p = cache[e].plan;
      return cache[e].status;
    }
  Entry& ent = cache[next];
  next = (next + 1) % kEntries;
  n_cached = std::min(n_cached + 1, kEntries);
  std::copy(key, key + 12, ent.key);
  ent.status = make_plan(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, head_dim, paged, cus, max_lds,
                         cfg, &ent.plan);
  *p = ent.plan;
  return ent.status;
}

}  // namespace

extern "C" size_t tsfa_fwd_workspace_bytes_for_dtype(int batch, int num_heads, int num_kv_heads, int q_len,
                                                     int kv_len, int prefix_len, int head_dim, int dtype) {
  if (batch <= 0 || q_len <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0) return 0;
  if (gen_path(head_dim, dtype)) {
    int cus = 0;
    GenPlan gp;
    if (device_cu_count(&cus) != TSFA_OK ||
        gen_plan(batch, num_heads, num_kv_heads, q_len, kv_len, head_dim, dtype, cus, &gp) != TSFA_OK)
      return 0;
    return gp.ws_acc_bytes + gp.ws_ml_bytes;
  }
  // enough for both the contiguous and the paged plan of the shape
  const Config cfg = config();
  Plan p, pp;
  if (device_plan(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, head_dim, false, cfg, &p) != TSFA_OK ||
      device_plan(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, head_dim, true, cfg, &pp) != TSFA_OK)
    return 0;
  return std::max(p.ws_acc_bytes + p.ws_ml_bytes, pp.ws_acc_bytes + pp.ws_ml_bytes);
}

extern "C" size_t tsfa_fwd_workspace_bytes(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len,
                                           int prefix_len, int head_dim) {
  return tsfa_fwd_workspace_bytes_for_dtype(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, head_dim,
                                            TSFA_DTYPE_BF16);
}

extern "C" int tsfa_fwd_plan(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len, int prefix_len,
                             int head_dim, int32_t* out6) {
  if (out6 == nullptr || batch <= 0 || q_len <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
    return TSFA_ERR_INVALID_ARGUMENT;
  Plan p;
  const int st = device_plan(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, head_dim, false, config(), &p);
  if (st != TSFA_OK) return st;
  out6[0] = p.n_splits;
  out6[1] = p.units_per_split;
  out6[2] = p.rows_per_chunk;
  out6[3] = p.n_chunks;
  out6[4] = p.grid;
  out6[5] = p.ring_stages;
  return TSFA_OK;
}

namespace {

// K/V of one call: contiguous per-head tensors, or the paged cache.
struct KvSource {
  const void* k = nullptr;
  const void* v = nullptr;
  const int64_t* k_strides = nullptr;  // [4]: b, h, n, d
  const int64_t* v_strides = nullptr;
  const void* cache = nullptr;  // paged: [pages, 2, page_size, Hkv, D] by cache_strides
  const int64_t* cache_strides = nullptr;  // [5]: page, slot, row, head, d
  const int32_t* kv_indptr = nullptr;
  const int32_t* kv_indices = nullptr;
  int64_t pt_stride = 0, n_indices = 0;
  int n_pages = 0, page_size = 0;
  bool paged() const { return cache != nullptr; }
};

// The generic kernel's call (head_dim 256, fp32): contiguous K/V only.
int gen_impl(const void* q, const KvSource& kv, void* o, float* lse, const int32_t* row_ptr, const int32_t* col_idx,
             const int8_t* blk_type, const int32_t* payload, const int32_t* offset, const int64_t* meta_seq_stride,
             const int64_t* o_strides, float sm_scale, int batch, int num_heads, int num_kv_heads, int q_len,
             int kv_len, int prefix_len, int gqa_group_size, int block_m, int block_n, int head_dim, int dtype,
             void* workspace, size_t workspace_bytes, hipStream_t stream, const int64_t* q_strides) {
  if (kv.paged()) return TSFA_ERR_UNSUPPORTED;
  int cus = 0;
  if (device_cu_count(&cus) != TSFA_OK) return TSFA_ERR_DEVICE;
  GenPlan p;
  int st = gen_plan(batch, num_heads, num_kv_heads, q_len, kv_len, head_dim, dtype, cus, &p);
  if (st != TSFA_OK) return st;
  if (workspace == nullptr || workspace_bytes < p.ws_acc_bytes + p.ws_ml_bytes ||
      reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
    return TSFA_ERR_WORKSPACE;
  // fp32 rows are addressed as 16-byte pieces too: q/k/v/o row strides and
  // bases are multiples of 16 bytes (check_strides asks 8 elements of 2 bytes)
  GenArgs ga = {};
  ga.q = q;
  ga.k = kv.k;
  ga.v = kv.v;
  ga.row_ptr = row_ptr;
  ga.col_idx = col_idx;
  ga.blk_type = blk_type;
  ga.payload = payload;
  ga.offset = offset;
  for (int i = 0; i < 5; ++i) ga.ms[i] = meta_seq_stride[i];
  ga.sqb = q_strides[0];
  ga.sqh = q_strides[1];
  ga.sqm = q_strides[2];
  ga.skb = kv.k_strides[0];
  ga.skh = kv.k_strides[1];
  ga.skn = kv.k_strides[2];
  ga.svb = kv.v_strides[0];
  ga.svh = kv.v_strides[1];
  ga.svn = kv.v_strides[2];
  float sl2 = fabsf(sm_scale) * 1.4426950408889634f;
  if (sl2 == 0.f) sl2 = 1e-30f;
  ga.scale_log2 = sl2;
  ga.neg_q = sm_scale < 0.f ? 1 : 0;
  ga.num_kv_heads = num_kv_heads;
  ga.group = gqa_group_size;
  ga.q_len = q_len;
  ga.kv_len = kv_len;
  ga.prefix_len = prefix_len;
  ga.block_m = block_m;
  ga.block_n = block_n;
  ga.n_chunks = p.n_chunks;
  ga.n_units = p.n_units;
  ga.units_per_split = p.units_per_split;
  ga.n_slots = p.n_slots;
  ga.ws_o = workspace;
  ga.ws_ml = reinterpret_cast<float2*>(static_cast<char*>(workspace) + p.ws_acc_bytes);
  // One split and no LSE: the kernel writes O itself (TSFA_DIRECT_OUT=0
  // keeps the partials and the combine)
  ga.out = o;
  ga.sob = o_strides[0];
  ga.soh = o_strides[1];
  ga.som = o_strides[2];
  ga.direct = (config().direct_out != 0 && p.n_slots == 1 && lse == nullptr) ? 1 : 0;
  CombineArgs ca;
  ca.o = o;
  ca.lse = lse;
  ca.sob = o_strides[0];
  ca.soh = o_strides[1];
  ca.som = o_strides[2];
  ca.scale_log2 = sl2;
  ca.batch = batch;
  ca.num_heads = num_heads;
  ca.num_kv_heads = num_kv_heads;
  ca.group = gqa_group_size;
  ca.q_len = q_len;
  ca.n_slots = p.n_slots;
  ca.ws_o = ga.ws_o;
  ca.ws_ml = ga.ws_ml;
  if (dtype == TSFA_DTYPE_FP32) {
    if (head_dim == 64) return launch_gen<float, 64>(ga, ca, p, stream);
    if (head_dim == 128) return launch_gen<float, 128>(ga, ca, p, stream);
    return launch_gen<float, 256>(ga, ca, p, stream);
  }
  if (head_dim != 256) return TSFA_ERR_UNSUPPORTED;
  return dtype == TSFA_DTYPE_BF16 ? launch_gen<__bf16, 256>(ga, ca, p, stream)
                                  : launch_gen<_Float16, 256>(ga, ca, p, stream);
}

int fwd_impl(const void* q, const KvSource& kv, void* o, float* lse, const int32_t* row_ptr, const int32_t* col_idx,
             const int8_t* blk_type, const int32_t* mixed_mask_payload, const int32_t* mixed_mask_offset,
             const int64_t* meta_seq_stride, const int64_t* q_strides, const int64_t* o_strides, float sm_scale,
             int batch, int num_heads, int num_kv_heads, int q_len, int kv_len, int prefix_len, int n_q_blocks,
             int n_tree_blocks, int gqa_group_size, int block_m, int block_n, int head_dim, int dtype,
             void* workspace, size_t workspace_bytes, tsfa_stream_t stream_) {
  int st = tsfa_fwd_check_args(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, n_q_blocks,
                               n_tree_blocks, gqa_group_size, block_m, block_n, head_dim, dtype);
  if (st != TSFA_OK) return st;
  if (batch == 0 || q_len == 0) return TSFA_OK;
  if (q_strides == nullptr || o_strides == nullptr || meta_seq_stride == nullptr) return TSFA_ERR_INVALID_ARGUMENT;
  if (q == nullptr || o == nullptr || row_ptr == nullptr) return TSFA_ERR_INVALID_ARGUMENT;
  if (kv.paged() && kv.kv_indices == nullptr) return TSFA_ERR_INVALID_ARGUMENT;
  if (kv.paged() && (kv.cache == nullptr || kv.cache_strides == nullptr)) return TSFA_ERR_INVALID_ARGUMENT;
  st = check_strides(q, q_strides, o, o_strides);
  if (st != TSFA_OK) return st;
  st = kv.paged() ? check_paged(batch, kv_len, kv.cache, kv.cache_strides, kv.kv_indptr, kv.pt_stride, kv.n_indices,
                                kv.n_pages, kv.page_size)
                  : check_kv_strides(kv.k, kv.k_strides, kv.v, kv.v_strides);
  if (st != TSFA_OK) return st;
  for (int i = 0; i < 5; ++i)
    if (meta_seq_stride[i] < 0) return TSFA_ERR_INVALID_ARGUMENT;
  if (gen_path(head_dim, dtype))
    return gen_impl(q, kv, o, lse, row_ptr, col_idx, blk_type, mixed_mask_payload, mixed_mask_offset,
                    meta_seq_stride, o_strides, sm_scale, batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len,
                    gqa_group_size, block_m, block_n, head_dim, dtype, workspace, workspace_bytes,
                    reinterpret_cast<hipStream_t>(stream_), q_strides);

  // one snapshot of the TSFA_* switches for the whole call
  const Config cfg = config();
  Plan p;
  st = device_plan(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, head_dim, kv.paged(), cfg, &p);
  if (st != TSFA_OK) return st;
  p.tree_key_limit = (int)std::min<int64_t>((int64_t)n_tree_blocks * block_n, (int64_t)kv_len - prefix_len);
  if (workspace == nullptr || workspace_bytes < p.ws_acc_bytes + p.ws_ml_bytes) return TSFA_ERR_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0) return TSFA_ERR_WORKSPACE;

  SplitArgs sa = {};
  sa.q = q;
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
  sa.sqb = q_strides[0];
  sa.sqh = q_strides[1];
  sa.sqm = q_strides[2];
  if (kv.paged()) {
    sa.kv_cache = kv.cache;
    sa.kv_indptr = kv.kv_indptr;
    sa.kv_indices = kv.kv_indices;
    sa.pt_stride = (int)kv.pt_stride;
    sa.n_indices = (int)kv.n_indices;
    sa.cps = kv.cache_strides[0];
    sa.css = kv.cache_strides[1];
    sa.crs = kv.cache_strides[2];
    sa.chs = kv.cache_strides[3];
    sa.n_pages = kv.n_pages;
    int shift = 0;
    while ((1 << shift) < kv.page_size) ++shift;
    sa.page_shift = shift;
    // the 32-bit-offset kernel when every byte offset it forms from a kv
    // head's base fits (TSFA_PAGED32=0 keeps the 64-bit kernel)
    sa.cache32 = (cfg.paged32 != 0 && paged_offsets_fit_32(kv.n_pages, kv.cache_strides[0], kv.cache_strides[2],
                                                                 kv.page_size, head_dim))
                     ? 1 : 0;
    sa.cps_b32 = (uint32_t)(kv.cache_strides[0] * 2);
    sa.crs_b32 = (uint32_t)(kv.cache_strides[2] * 2);
  } else {
    sa.k = kv.k;
    sa.v = kv.v;
    sa.skb = kv.k_strides[0];
    sa.skh = kv.k_strides[1];
    sa.skn = kv.k_strides[2];
    sa.svb = kv.v_strides[0];
    sa.svh = kv.v_strides[1];
    sa.svn = kv.v_strides[2];
  }
  // Scores enter the exponent as s * |sm_scale| * log2(e) with Q negated for a
  // negative scale; a zero scale becomes a vanishing one (every visible p = 1
  // and masked keys still get p = 0).
  float sl2 = fabsf(sm_scale) * 1.4426950408889634f;
  if (sl2 == 0.f) sl2 = 1e-30f;
  sa.scale_log2 = sl2;
  sa.neg_q = sm_scale < 0.f ? 1 : 0;
  sa.num_kv_heads = num_kv_heads;
  sa.group = gqa_group_size;
  sa.q_len = q_len;
  sa.kv_len = kv_len;
  sa.prefix_len = prefix_len;
  sa.block_m = block_m;
  sa.block_n = block_n;
  sa.n_tree_blocks = n_tree_blocks;
  sa.n_chunks = p.n_chunks;
  sa.units_per_split = p.units_per_split;
  sa.n_pu = p.n_pu;
  sa.n_slots = p.n_slots;
  sa.n_items = p.n_items;
  sa.items_per_xcd = p.items_per_xcd;
  sa.fd_chunks = make_fastdiv(p.n_chunks);
  sa.fd_slots = make_fastdiv(p.n_slots);
  sa.fd_kvh = make_fastdiv(num_kv_heads);
  sa.fd_group = make_fastdiv(gqa_group_size);
  sa.fd_P = make_fastdiv(p.n_chunks * p.n_slots);
  sa.fd_Np = make_fastdiv(std::max(1, p.n_chunks * (p.n_slots - 1)));
  sa.fd_Nt = make_fastdiv(p.n_chunks);
  sa.tree_key_limit = p.tree_key_limit;
  sa.vt_max = p.vt_max;
  sa.ws_o = workspace;
  sa.ws_ml = reinterpret_cast<float2*>(static_cast<char*>(workspace) + p.ws_acc_bytes);
  // Non-temporal K/V loads when little L2 reuse is at stake (TSFA_KV_NT=0/1
  // forces them off/on).
  const int kv_nt = cfg.kv_nt;
  sa.kv_nt = kv_nt >= 0 ? (kv_nt != 0) : (p.n_chunks <= 2);
  // Prefix runs first when the grid has at most 4 rounds (TSFA_ITEM_ORDER=0/1/2
  // forces natural / prefix first / tree first).
  int cus = 256;
  if (device_cu_count(&cus) != TSFA_OK) return TSFA_ERR_DEVICE;
  const int order = cfg.item_order;
  sa.item_order = order >= 0 && order <= 2 ? order : ((int64_t)p.n_items <= 4LL * cus ? 1 : 0);
  sa.fold_tree = p.fold_tree;
  // folded: the last run of each chunk carries the tree units, the longest
  // items, so those go first (longest first)
  if (p.fold_tree && order < 0) sa.item_order = sa.item_order ? 2 : 0;
  // one round (every XCD's items start together): the order cannot matter,
  // and the natural one costs each wave no scalar divisions to decode
  if (order < 0 && (int64_t)p.items_per_xcd * 8 <= cus) sa.item_order = 0;

  // One slot (one prefix run per chunk with the tree folded in, or a tree
  // alone): the split kernel's partial is O itself, so with O contiguous
  // [B, Hq, q_len, D] and no LSE asked it writes O and the combine is
  // skipped (the 16-sequence decode shape: its ~5 us combine of ~55 us).
  const bool o_dense = o_strides[3] == 1 && o_strides[2] == head_dim && o_strides[1] == (int64_t)q_len * head_dim &&
                       o_strides[0] == (int64_t)num_heads * q_len * head_dim;
  sa.direct_out = p.n_slots == 1 && lse == nullptr && o_dense && cfg.direct_out != 0 ? 1 : 0;

  CombineArgs ca;
  ca.o = o;
  ca.lse = lse;
  ca.sob = o_strides[0];
  ca.soh = o_strides[1];
  ca.som = o_strides[2];
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
  const bool bf = dtype == TSFA_DTYPE_BF16, d128 = head_dim == 128;
  if (kv.paged()) {
    if (bf) return d128 ? launch_all<__bf16, 128, true>(sa, ca, p, cfg, stream) : launch_all<__bf16, 64, true>(sa, ca, p, cfg, stream);
    return d128 ? launch_all<_Float16, 128, true>(sa, ca, p, cfg, stream) : launch_all<_Float16, 64, true>(sa, ca, p, cfg, stream);
  }
  if (bf) return d128 ? launch_all<__bf16, 128, false>(sa, ca, p, cfg, stream) : launch_all<__bf16, 64, false>(sa, ca, p, cfg, stream);
  return d128 ? launch_all<_Float16, 128, false>(sa, ca, p, cfg, stream) : launch_all<_Float16, 64, false>(sa, ca, p, cfg, stream);
}

}  // namespace

extern "C" int tsfa_fwd(const void* q, const void* k, const void* v, void* o, const int32_t* row_ptr,
                        const int32_t* col_idx, const int8_t* blk_type, const int32_t* mixed_mask_payload,
                        const int32_t* mixed_mask_offset, const int64_t* meta_seq_stride, const int64_t* strides,
                        float sm_scale, int batch, int num_heads, int num_kv_heads, int q_len, int kv_len,
                        int prefix_len, int n_q_blocks, int n_tree_blocks, int gqa_group_size, int block_m,
                        int block_n, int head_dim, int dtype, void* workspace, size_t workspace_bytes,
                        tsfa_stream_t stream_) {
  KvSource kv;
  kv.k = k;
  kv.v = v;
  kv.k_strides = strides ? strides + 4 : nullptr;
  kv.v_strides = strides ? strides + 8 : nullptr;
  return fwd_impl(q, kv, o, nullptr, row_ptr, col_idx, blk_type, mixed_mask_payload, mixed_mask_offset,
                  meta_seq_stride, strides, strides ? strides + 12 : nullptr, sm_scale, batch, num_heads, num_kv_heads, q_len,
                  kv_len, prefix_len, n_q_blocks, n_tree_blocks, gqa_group_size, block_m, block_n, head_dim, dtype,
                  workspace, workspace_bytes, stream_);
}

// ------------------------------------- metadata build + forward in one call
// run_tree_sparse_kernel(q, k, v, tree_mask) as one C call: the device
// metadata builder (tsfa_meta_build) writes the capacity-layout tree record
// into the front of the workspace and the forward reads it there, in stream
// order, with no host synchronisation.  Workspace layout (each section
// 256-byte aligned): row_ptr, col_idx, blk_type, payload, offset, counts of
// n_masks trees, the builder's scratch, the forward's split-KV partials.
namespace {

struct TreeCallLayout {
  size_t off[8];  // row_ptr col_idx blk_type payload offset counts meta_ws fwd_ws
  size_t total, fwd_bytes;
  int nqb, ntb, words;
  int64_t cap;
};

int tree_call_layout(int batch, int num_heads, int num_kv_heads, int q_len, int kv_len, int n_masks,
                     int block_m, int block_n, int head_dim, int dtype, TreeCallLayout* L) {
  if (batch <= 0 || q_len <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 || kv_len < q_len ||
      (n_masks != 1 && n_masks != batch))
    return TSFA_ERR_INVALID_ARGUMENT;
  const int st = tsfa_meta_check_args(n_masks, q_len, block_m, block_n);
  if (st != TSFA_OK) return st;
  meta::MetaGeom g;
  if (!meta::meta_geom(q_len, block_m, block_n, &g)) return TSFA_ERR_UNSUPPORTED;
  L->nqb = g.nqb;
  L->ntb = g.ntb;
  L->words = g.words;
  L->cap = g.cap;
  const size_t n = (size_t)n_masks;
  const size_t sizes[7] = {n * (g.nqb + 1) * 4, n * g.cap * 4, n * g.cap, n * g.cap * g.words * 4, n * g.cap * 4,
                           n * 2 * 4, tsfa_meta_workspace_bytes(n_masks, q_len, block_m, block_n)};
  size_t at = 0;
  for (int i = 0; i < 7; ++i) {
    L->off[i] = at;
    at += align256(std::max<size_t>(sizes[i], 1));
  }
  L->off[7] = at;
  L->fwd_bytes = tsfa_fwd_workspace_bytes_for_dtype(batch, num_heads, num_kv_heads, q_len, kv_len, kv_len - q_len,
                                                    head_dim, dtype);
  if (L->fwd_bytes == 0) return TSFA_ERR_UNSUPPORTED;
  L->total = at + L->fwd_bytes;
  return TSFA_OK;
}

}  // namespace

extern "C" size_t tsfa_tree_attention_workspace_bytes(int batch, int num_heads, int num_kv_heads, int q_len,
                                                      int kv_len, int n_masks, int block_m, int block_n,
                                                      int head_dim, int dtype) {
  TreeCallLayout L;
  if (tree_call_layout(batch, num_heads, num_kv_heads, q_len, kv_len, n_masks, block_m, block_n, head_dim, dtype,
                       &L) != TSFA_OK)
    return 0;
  return L.total;
}

extern "C" int tsfa_tree_attention(const void* q, const void* k, const void* v, void* o, const uint8_t* mask,
                                   int64_t mask_seq_stride, int64_t mask_row_stride, int n_masks,
                                   const int64_t* strides, float sm_scale, int batch, int num_heads,
                                   int num_kv_heads, int q_len, int kv_len, int block_m, int block_n, int head_dim,
                                   int dtype, void* workspace, size_t workspace_bytes, tsfa_stream_t stream) {
  if (kv_len < q_len) return TSFA_ERR_INVALID_ARGUMENT;  // eagle_tree_sparse_bridge.py:91-93
  if (batch == 0) return TSFA_OK;
  TreeCallLayout L;
  int st = tree_call_layout(batch, num_heads, num_kv_heads, q_len, kv_len, n_masks, block_m, block_n, head_dim,
                            dtype, &L);
  if (st != TSFA_OK) return st;
  const int prefix_len = kv_len - q_len;
  // the forward's own checks first: nothing is launched for a call it refuses
  st = tsfa_fwd_check_args(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, L.nqb, L.ntb,
                           num_heads / num_kv_heads, block_m, block_n, head_dim, dtype);
  if (st != TSFA_OK) return st;
  if (mask == nullptr || strides == nullptr || mask_row_stride < 1 || mask_seq_stride < 0)
    return TSFA_ERR_INVALID_ARGUMENT;
  if (q == nullptr || o == nullptr) return TSFA_ERR_INVALID_ARGUMENT;
  st = check_strides(q, strides, o, strides + 12);
  if (st == TSFA_OK) st = check_kv_strides(k, strides + 4, v, strides + 8);
  if (st != TSFA_OK) return st;
  if (workspace == nullptr || workspace_bytes < L.total || reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
    return TSFA_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  int32_t* row_ptr = reinterpret_cast<int32_t*>(ws + L.off[0]);
  int32_t* col_idx = reinterpret_cast<int32_t*>(ws + L.off[1]);
  int8_t* blk_type = reinterpret_cast<int8_t*>(ws + L.off[2]);
  int32_t* payload = reinterpret_cast<int32_t*>(ws + L.off[3]);
  int32_t* offset = reinterpret_cast<int32_t*>(ws + L.off[4]);
  int32_t* counts = reinterpret_cast<int32_t*>(ws + L.off[5]);
  st = tsfa_meta_build(mask, mask_seq_stride, mask_row_stride, n_masks, q_len, block_m, block_n, row_ptr, col_idx,
                       blk_type, payload, offset, counts, ws + L.off[6], L.off[7] - L.off[6], stream);
  if (st != TSFA_OK) return st;
  // one tree for the batch: stride 0; one per sequence: the capacity layout
  const int64_t ms[5] = {n_masks > 1 ? (int64_t)L.nqb + 1 : 0, n_masks > 1 ? L.cap : 0, n_masks > 1 ? L.cap : 0,
                         n_masks > 1 ? L.cap * L.words : 0, n_masks > 1 ? L.cap : 0};
  return tsfa_fwd(q, k, v, o, row_ptr, col_idx, blk_type, payload, offset, ms, strides, sm_scale, batch, num_heads,
                  num_kv_heads, q_len, kv_len, prefix_len, L.nqb, L.ntb, num_heads / num_kv_heads, block_m, block_n,
                  head_dim, dtype, ws + L.off[7], L.fwd_bytes, stream);
}

// ------------------------------------------------- allocation-free forward
// The split-KV partials of tsfa_fwd_noalloc live in this file-scope device
// array: each GPU the library runs on holds its own copy (kNoAllocBytes) until
// the process ends.  Its address on a device comes from hipGetSymbolAddress,
// taken once per device with that device current; host code passes that
// address, never the array's name, to kernels.  The split kernel writes every
// partial the combine reads, so nothing needs clearing between calls.  All
// calls on one GPU share the array: calls that overlap in time on one GPU
// (different streams, or host threads) race on it.
constexpr size_t kNoAllocBytes = TSFA_FWD_NOALLOC_MAX_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// The device of `stream` (the current device for the null stream) and the
// scratch array's address there.
int noalloc_scratch(hipStream_t stream, void** out) {
  int dev = -1;
  if (stream != nullptr) {
    if (hipStreamGetDevice(stream, &dev) != hipSuccess) return TSFA_ERR_DEVICE;
  } else if (hipGetDevice(&dev) != hipSuccess) {
    return TSFA_ERR_DEVICE;
  }
  if (dev < 0 || dev >= kMaxDevices) return TSFA_ERR_DEVICE;
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      int cur = -1;
      if (hipGetDevice(&cur) != hipSuccess) return TSFA_ERR_DEVICE;
      if (cur != dev && hipSetDevice(dev) != hipSuccess) return TSFA_ERR_DEVICE;
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (cur != dev) (void)hipSetDevice(cur);
      if (e != hipSuccess || p == nullptr) return TSFA_ERR_DEVICE;
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return TSFA_OK;
}
}  // namespace

extern "C" int tsfa_fwd_noalloc(const void* q, const void* k, const void* v, void* o, const int32_t* row_ptr,
                                const int32_t* col_idx, const int8_t* blk_type, const int32_t* mixed_mask_payload,
                                const int32_t* mixed_mask_offset, const int64_t* meta_seq_stride,
                                const int64_t* strides, float sm_scale, int batch, int num_heads, int num_kv_heads,
                                int q_len, int kv_len, int prefix_len, int n_q_blocks, int n_tree_blocks,
                                int gqa_group_size, int block_m, int block_n, int head_dim, int dtype,
                                tsfa_stream_t stream_) {
  // the same checks and kernels as tsfa_fwd; a call whose partials exceed
  // the array is refused before anything runs
  const int st = tsfa_fwd_check_args(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, n_q_blocks,
                                     n_tree_blocks, gqa_group_size, block_m, block_n, head_dim, dtype);
  if (st != TSFA_OK) return st;
  if (tsfa_fwd_workspace_bytes_for_dtype(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, head_dim,
                                         dtype) > kNoAllocBytes)
    return TSFA_ERR_WORKSPACE;
  void* ws = nullptr;
  const int sst = noalloc_scratch(reinterpret_cast<hipStream_t>(stream_), &ws);
  if (sst != TSFA_OK) return sst;
  return tsfa_fwd(q, k, v, o, row_ptr, col_idx, blk_type, mixed_mask_payload, mixed_mask_offset, meta_seq_stride,
                  strides, sm_scale, batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, n_q_blocks,
                  n_tree_blocks, gqa_group_size, block_m, block_n, head_dim, dtype, ws, kNoAllocBytes, stream_);
}

extern "C" int tsfa_fwd_lse(const void* q, const void* k, const void* v, void* o, float* lse,
                            const int32_t* row_ptr, const int32_t* col_idx, const int8_t* blk_type,
                            const int32_t* mixed_mask_payload, const int32_t* mixed_mask_offset,
                            const int64_t* meta_seq_stride, const int64_t* strides, float sm_scale, int batch,
                            int num_heads, int num_kv_heads, int q_len, int kv_len, int prefix_len, int n_q_blocks,
                            int n_tree_blocks, int gqa_group_size, int block_m, int block_n, int head_dim, int dtype,
                            void* workspace, size_t workspace_bytes, tsfa_stream_t stream_) {
  if (lse == nullptr && batch > 0 && q_len > 0) return TSFA_ERR_INVALID_ARGUMENT;
  KvSource kv;
  kv.k = k;
  kv.v = v;
  kv.k_strides = strides ? strides + 4 : nullptr;
  kv.v_strides = strides ? strides + 8 : nullptr;
  return fwd_impl(q, kv, o, lse, row_ptr, col_idx, blk_type, mixed_mask_payload, mixed_mask_offset,
                  meta_seq_stride, strides, strides ? strides + 12 : nullptr, sm_scale, batch, num_heads,
                  num_kv_heads, q_len, kv_len, prefix_len, n_q_blocks, n_tree_blocks, gqa_group_size, block_m,
                  block_n, head_dim, dtype, workspace, workspace_bytes, stream_);
}

extern "C" int tsfa_fwd_paged(const void* q, const void* kv_cache, const int32_t* kv_indptr,
                              const int32_t* kv_indices, int64_t n_indices, int64_t page_table_stride, int n_pages,
                              int page_size, void* o, float* lse, const int32_t* row_ptr, const int32_t* col_idx,
                              const int8_t* blk_type, const int32_t* mixed_mask_payload,
                              const int32_t* mixed_mask_offset, const int64_t* meta_seq_stride,
                              const int64_t* q_strides, const int64_t* cache_strides, const int64_t* o_strides,
                              float sm_scale, int batch, int num_heads, int num_kv_heads, int q_len, int kv_len,
                              int prefix_len, int n_q_blocks, int n_tree_blocks, int gqa_group_size, int block_m,
                              int block_n, int head_dim, int dtype, void* workspace, size_t workspace_bytes,
                              tsfa_stream_t stream_) {
  if (kv_cache == nullptr) return TSFA_ERR_INVALID_ARGUMENT;
  KvSource kv;
  kv.cache = kv_cache;
  kv.cache_strides = cache_strides;
  kv.kv_indptr = kv_indptr;
  kv.kv_indices = kv_indices;
  kv.n_indices = n_indices;
  kv.pt_stride = page_table_stride;
  kv.n_pages = n_pages;
  kv.page_size = page_size;
  return fwd_impl(q, kv, o, lse, row_ptr, col_idx, blk_type, mixed_mask_payload, mixed_mask_offset,
                  meta_seq_stride, q_strides, o_strides, sm_scale, batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len,
                  n_q_blocks, n_tree_blocks, gqa_group_size, block_m, block_n, head_dim, dtype, workspace,
                  workspace_bytes, stream_);
}

extern "C" int tsfa_fwd_set_kernel_mask(int mask) {
  if (mask < 1 || mask > 3) return TSFA_ERR_INVALID_ARGUMENT;
  // measurement builds of a process only: TSFA_BENCH_HOOKS=1 unlocks it
  if (mask != 3 && config().bench_hooks == 0) return TSFA_ERR_UNSUPPORTED;
  g_kernel_mask = mask;
  return TSFA_OK;
}

#ifdef TSFA_STAMPS
extern "C" int tsfa_stamps_copy(void* dst, size_t bytes) {
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_stamps), bytes, 0, hipMemcpyDeviceToHost) == hipSuccess ? 0 : 4;
}
extern "C" int tsfa_cyc_copy(void* dst, size_t bytes) {
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_cyc), bytes, 0, hipMemcpyDeviceToHost) == hipSuccess ? 0 : 4;
}
#endif
