// Tree-sparse attention backward for gfx950 (MI355X).
//
// The reference has no backward (README.md:198 lists it as missing).  This is
// the gradient of the function its forward computes
// (block_sparse_tree_fwd_kernel, tree_sparse_flashattn.py:163-339): with
// z = sm_scale * q.k over a row's visible keys (the dense prefix [0, P) and the
// tree keys its CSR row marks), P = softmax(z), O = P V,
//   dV = P^T dO,  dP = dO V^T,  dS = P * (dP - rowsum(dO * O)),
//   dQ = sm_scale * dS K,  dK = sm_scale * dS^T Q,
// summed over the G query heads of each kv head.  P is recomputed from the
// forward's per-row log-sum-exp (tsfa_fwd_lse).
//
// Kernels (one call = three or four launches, no host synchronisation):
//   * bwd_prep_vis_kernel, two jobs in one launch:
//     prep -- per query row (16 lanes): Dv = rowsum(dO * O) in fp32, the
//     log2-domain LSE, and (when the dQ pass is split) the row of the fp32 dQ
//     accumulator cleared.  Rows with no visible key (LSE = -inf) and the
//     padding rows of the last 32-row tile get LSE = +inf and Dv = 0, so their
//     P and dS are exactly 0;
//     visibility -- per (32-row tile, tree key) a word (bit m: row 32*tile + m
//     sees the key), from the CSR metadata;
//   * bwd_kv_kernel (key-parallel, dK and dV): a workgroup owns 128 keys of
//     one (batch, kv head) -- prefix keys and tree keys in separate blocks --
//     as 4 key groups x 2 row groups of waves; each wave keeps dK^T and dV^T
//     of its 32 keys in registers while its row group walks every other
//     32-row tile of the (batch, kv head) (rows token-major, r = t*G + g, as
//     in the forward).  Per tile, on v_mfma_f32_32x32x16: S = Q K^T and dP =
//     dO V^T (a lane holds one key), then dV^T += dO^T P and dK^T += Q^T dS
//     with P and dS taken straight from the S / dP accumulators (the MFMA k
//     order is permuted to the order the accumulator holds rows in; the dO^T
//     / Q^T operands come from ds_read_b64_tr_b16 in the same order).  Q / dO
//     tiles, their row statistics and the tree block's mask words move HBM
//     -> LDS with global_load_lds, double-buffered per row group; one LDS
//     copy of each tile serves both the row reads and the transposed reads
//     (a swizzle that is conflict-free for both patterns).  The row groups
//     merge their sums through LDS at the end;
//   * bwd_dq_main_kernel (row-parallel, dQ): a workgroup owns 128 rows and a
//     split of the 32-key units; S^T, dP^T, dS^T recomputed per unit and dQ^T
//     += K^T dS^T accumulated in registers; an unsplit chunk writes dQ
//     directly, split chunks add once per workgroup to the fp32 accumulator;
//   * bwd_dq_kernel (split chunks only): dQ = sm_scale * accumulator in the
//     input dtype.
// bwd_kv_kernel and bwd_dq_main_kernel are independent once the first launch
// has run; the dQ kernel goes to a side stream so its workgroups fill the CUs
// the dK/dV grid leaves idle (70 -> 63 us per call at the Llama-3-8B shape,
// where 264 dK/dV workgroups of one per CU leave a second round of 8).

#include <math.h>
#include <stdlib.h>

#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <utility>

#include "tsfa_internal.h"

namespace tsfa {
namespace bwd {

constexpr int kWaves = 8;                 // 4 key groups x 2 row groups
// kBlockKeys, kTileRows, kMaxStateInts: tsfa_plan.h
constexpr int kBufs = 2;                  // Q / dO tile buffers per row group: loads run one step ahead

// 16-byte-chunk XOR swizzle of a row-major [rows][D] LDS tile (row period
// 16), conflict-free for both read patterns of the kernel:
//   * row reads (ds_read_b128, a quarter-wave reads chunk c of 16 rows): the
//     16 rows land on 16 distinct 16-byte bank slots;
//   * transposed reads (ds_read_b64_tr_b16, a half-wave reads 4 consecutive
//     rows x 64 bytes): the 4 rows land on 4 distinct 64-byte bank windows.
template <int D> __device__ inline int swz(int row) {
  if constexpr (D == 128) {
    return ((row & 3) << 2) | ((row >> 2) & 3);
  } else {
    const int j = row >> 1;
    return ((j & 1) << 2) | ((j >> 1) & 3);
  }
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is reserved; the clobber documents the write
// 16 bytes per active lane HBM -> LDS: lane i's bytes land at lds_base + 16*i.
__device__ inline void dma16(const void* src, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(lds_base)
               : "memory", "m0");
}
// The same with a scalar base and a 32-bit lane offset (no per-lane 64-bit
// address held in registers).
__device__ inline void dma16_s(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(sbase), "s"(lds_base)
               : "memory", "m0");
}
#pragma clang diagnostic pop

template <int N> __device__ inline void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}
__device__ inline void sync_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ inline uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(const TSFA_LDS void*)p; }
template <typename V, typename U> __device__ inline V bit_cast(U u) { return __builtin_bit_cast(V, u); }

struct BwdArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* dout;
  void* dk;
  void* dv;
  float* dq_acc;            // [B*Hkv][D][n_tiles*32] fp32 (d-major: a wave's atomics cover whole lines)
  const float2* rowstat;    // [B*Hkv][n_tiles*32] (log2 LSE, Dv)
  const uint32_t* vis;      // [n_trees][n_tiles][n_tkeys] visibility words of tree keys
  int64_t sqb, sqh, sqm, skb, skh, skn, svb, svh, svn, sdob, sdoh, sdom, sdkb, sdkh, sdkn, sdvb, sdvh, sdvn;
  int64_t vis_tree_stride;  // 0: one tree for the batch
  float scale_log2;         // sm_scale * log2(e) (signed), never 0
  float dk_scale;           // sm_scale
  int num_kv_heads, group, q_len, kv_len, prefix_len;
  int n_tiles, n_pb, n_tb, n_tkeys;
  int n_items, items_per_xcd;
  uint32_t group_magic;     // floor(2^32 / group) + 1 (group > 1): R / group = umulhi(R, magic) for R < 2^21
  // row-parallel dQ kernel
  void* dq;                 // dq_direct: the kernel writes sm_scale * dQ here (one split per chunk)
  int64_t sdqb, sdqh, sdqm;
  float dq_scale;
  int dq_direct;
  int n_pu, n_tu;           // prefix / tree units of 32 keys
  int n_chunks, n_splits, units_per_split, q_items, q_items_per_xcd;
};

template <int D> constexpr size_t kv_lds_bytes() {
  // K block | V block | 2 groups x kBufs x (Q tile, dO tile) | 2 x kBufs x 32 row stats |
  // 2 x kBufs x 128 mask words | 64 bytes of dummy load targets
  return 2 * (size_t)kBlockKeys * D * 2 + 2 * 2 * kBufs * (size_t)kTileRows * D * 2 + 2 * kBufs * kTileRows * 8 +
         2 * kBufs * kBlockKeys * 4 + 64;
}

// Workgroup = 8 waves: key group kg = wave & 3 owns keys key0 + 32kg + [0, 32);
// row group rg = wave >> 2 takes every other 32-row tile.  Each SIMD runs one
// wave of each row group, so one wave's softmax-like VALU work and LDS waits
// overlap the other's MFMAs.  Both groups accumulate dK^T / dV^T of the same
// keys; group 1 hands its sums to group 0 through LDS at the end.
template <typename T, int D>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void bwd_kv_kernel(const BwdArgs a) {
  typedef typename Mma<T>::vec8 V8;
  constexpr int ROWB = D * 2;                 // bytes of one row
  constexpr int KSTEPS = D / 16;
  constexpr int DT = D / 32;
  constexpr int CPR = D / 8;                  // 16-byte chunks per row
  constexpr int RPL = 64 / CPR;               // rows per 1 KB load
  constexpr int TILE_B = kTileRows * ROWB;
  constexpr int KBLK_B = kBlockKeys * ROWB;
  constexpr int LPT = TILE_B / 1024;          // 1 KB loads per Q (or dO) tile
  constexpr int TPW = 2 * LPT / 4;            // tile loads per wave (4 waves per row group)
  constexpr int KPW = 2 * KBLK_B / 1024 / kWaves;  // K + V block loads per wave
  constexpr int LPW = TPW + 1;                // vector-memory instructions a wave issues per tile
  static_assert(kBufs == 2, "the exchange at the end reuses the K, V and tile areas");
  static_assert(TPW >= 1 && KPW >= 1 && 2 * LPT == TPW * 4, "load split");

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  unsigned char* kblk = smem;
  unsigned char* vblk = kblk + KBLK_B;
  unsigned char* tiles = vblk + KBLK_B;  // group g, buffer s: Q at tiles + 2*(g*kBufs + s)*TILE_B, dO after
  float2* rs = reinterpret_cast<float2*>(tiles + 2 * 2 * kBufs * TILE_B);          // [g][s][32]
  uint32_t* visw = reinterpret_cast<uint32_t*>(rs + 2 * kBufs * kTileRows);        // [g][s][128]
  unsigned char* dummy = reinterpret_cast<unsigned char*>(visw + 2 * kBufs * kBlockKeys);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kg = wave & 3, rg = wave >> 2;
  const int ln = lane & 31, lh = lane >> 5;

  // XCD-aware item order: consecutive block ids go to different XCDs and each
  // XCD gets a contiguous item range, so the key blocks of one (b, kv head),
  // which read the same Q / dO tiles, share an L2.
  const int item = (blockIdx.x & 7) * a.items_per_xcd + (blockIdx.x >> 3);
  if (item >= a.n_items) return;
  const int nkb = a.n_pb + a.n_tb;
  const int kb = item % nkb;
  const int bk = item / nkb;
  const int kvh = bk % a.num_kv_heads, b = bk / a.num_kv_heads;
  const bool tree_blk = kb >= a.n_pb;
  const int tkb = kb - a.n_pb;
  const int key0 = tree_blk ? a.prefix_len + tkb * kBlockKeys : kb * kBlockKeys;
  const int key_end = tree_blk ? a.kv_len : a.prefix_len;  // keys of this block: [key0, min(key0 + 128, key_end))
  const int G = a.group;
  const int TG = a.q_len * G;
  const int TGP = a.n_tiles * kTileRows;
  const float sl2 = a.scale_log2;  // signed: exp2(s * sl2 - lse2) for either sign of sm_scale

  const T* kbase = static_cast<const T*>(a.k) + b * a.skb + kvh * a.skh;
  const T* vbase = static_cast<const T*>(a.v) + b * a.svb + kvh * a.svh;
  const T* qbase = static_cast<const T*>(a.q) + b * a.sqb + (int64_t)kvh * G * a.sqh;
  const T* dobase = static_cast<const T*>(a.dout) + b * a.sdob + (int64_t)kvh * G * a.sdoh;
  const float2* rsbase = a.rowstat + (int64_t)bk * TGP;
  const uint32_t* visbase =
      a.vis + (int64_t)b * a.vis_tree_stride + (tree_blk ? (int64_t)tkb * kBlockKeys : 0);

  // K and V blocks HBM -> LDS (keys past the end repeat the last key; masked).
#pragma unroll
  for (int i = 0; i < KPW; ++i) {
    const int u = wave * KPW + i;  // 0 .. 2*KBLK_B/1024 - 1: K loads, then V loads
    const bool is_v = u >= KBLK_B / 1024;
    const int ul = is_v ? u - KBLK_B / 1024 : u;
    const int row = ul * RPL + lane / CPR, pos = lane % CPR;
    const int key = min(key0 + row, a.kv_len - 1);
    const T* src = (is_v ? vbase + (int64_t)key * a.svn : kbase + (int64_t)key * a.skn) + ((pos ^ swz<D>(row)) << 3);
    dma16(src, lds_addr((is_v ? vblk : kblk) + ul * 1024));
  }

  // The tiles of row group rg: step n handles tile tile_at(2n + rg).  The key
  // blocks of one (b, kv head) start their walk at different tiles (block kb
  // at tile kb * n_tiles / nkb), so the dQ atomics of concurrent blocks land
  // on different rows.
  const int j0 = (int)((int64_t)kb * a.n_tiles / nkb);
  auto tile_at = [&](int i) {
    const int j = j0 + i;
    return j >= a.n_tiles ? j - a.n_tiles : j;
  };
  const int n_steps = (a.n_tiles + 1) >> 1;
  const int my_tiles = (a.n_tiles + 1 - rg) >> 1;  // steps with a tile for this group

  // Q / dO tile j -> this group's buffer s, with its row statistics and (tree
  // blocks) the 128 keys' mask words.  Every wave issues exactly LPW loads
  // per tile: its share of Q and dO plus one more (the row statistics for key
  // group 0, the mask words for key group 1 of a tree block, else one lane
  // into a dummy LDS slot), so the waits below are compile-time counts.
  // Rows past the end repeat the last row; their statistics make P = dS = 0.
  auto issue_tile = [&](int j, int s) {
    unsigned char* qt = tiles + 2 * (rg * kBufs + s) * TILE_B;
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int u = kg * TPW + i;  // 0 .. 2*LPT-1: Q loads, then dO loads
      const bool is_do = u >= LPT;
      const int ul = is_do ? u - LPT : u;
      const int row = ul * RPL + lane / CPR, pos = lane % CPR;
      const int R = min(j * kTileRows + row, TG - 1);
      const int t = G == 1 ? R : (int)__umulhi((uint32_t)R, a.group_magic);
      const int g = R - t * G;
      const T* src = is_do ? dobase + g * a.sdoh + (int64_t)t * a.sdom : qbase + g * a.sqh + (int64_t)t * a.sqm;
      dma16(src + ((pos ^ swz<D>(row)) << 3), lds_addr(qt + (is_do ? TILE_B : 0) + ul * 1024));
    }
    if (kg == 0) {
      if (lane < kTileRows * 8 / 16)
        dma16_s(rsbase + j * kTileRows, 16u * lane, lds_addr(rs + (rg * kBufs + s) * kTileRows));
    } else if (kg == 1 && tree_blk) {
      if (lane < kBlockKeys * 4 / 16)
        dma16_s(visbase + (int64_t)j * a.n_tkeys, 16u * lane, lds_addr(visw + (rg * kBufs + s) * kBlockKeys));
    } else if (lane == 0) {
      dma16_s(rsbase, 0u, lds_addr(dummy + 16 * (wave & 3)));
    }
  };
  for (int i = 0; i < kBufs - 1 && i < my_tiles; ++i) issue_tile(tile_at(2 * i + rg), i);

  const int mykey = key0 + 32 * kg + ln;
  const bool key_ok = mykey < key_end && mykey < key0 + kBlockKeys;

  // LDS offsets (bytes).  Row reads: lane (row ln, lh) reads chunk 2kk + lh.
  // Transposed reads: lane (x = lane>>4, i = lane&15) reads 8 bytes of row
  // 8jj + 4(x>>1) + (i>>2) (+16 per k-step) at d = dt*32 + 16(x&1) + 4(i&3);
  // after the transpose it holds rows +[0,4) of d = dt*32 + 16(x&1) + i.
  const int vx = lane >> 4, vi = lane & 15;
  auto r_off = [&](int kk) { return ln * ROWB + (((2 * kk + lh) ^ swz<D>(ln)) << 4); };
  auto t_off = [&](int dt, int jj) {
    const int r = 8 * jj + 4 * (vx >> 1) + (vi >> 2);
    const int d = dt * 32 + 16 * (vx & 1) + 4 * (vi & 3);
    return r * ROWB + (((d >> 3) ^ swz<D>(r)) << 4) + ((d & 7) << 1);
  };
  const unsigned char* kmine = kblk + 32 * kg * ROWB;
  const unsigned char* vmine = vblk + 32 * kg * ROWB;

  f32x16 dk[DT], dv[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) dk[dt][i] = dv[dt][i] = 0.f;

  // rows (keys) +0..3 and +8..11 of a transposed read: the two halves of
  // one operand (jj = 0, 1; the swizzle differs between them)
  auto tr_pair = [&](const unsigned char* base, int dt) {
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((TSFA_LDS i16x4*)(base + t_off(dt, 0)));
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((TSFA_LDS i16x4*)(base + t_off(dt, 1)));
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  };

  for (int n = 0; n < n_steps; ++n) {
    const int s = n & (kBufs - 1);
    const bool has = n < my_tiles;  // group 1 has no tile on the last step of an odd count
    // Wait for this group's tile of step n (and on the first step the K / V
    // blocks): vector memory completes in issue order, and in the steady
    // state issued after this tile's loads are the next kBufs-2 tiles' loads.
    if (n >= kBufs - 1 && n + kBufs - 2 < my_tiles)
      vm_wait<(kBufs - 2) * LPW>();
    else
      vm_wait<0>();
    // every wave is done with step n-1: its buffers (the ones step n+kBufs-1
    // loads into) are free
    sync_lds();
    if (n + kBufs - 1 < my_tiles) issue_tile(tile_at(2 * (n + kBufs - 1) + rg), (n + kBufs - 1) & (kBufs - 1));
    const unsigned char* qt = tiles + 2 * (rg * kBufs + s) * TILE_B;
    const unsigned char* dot = qt + TILE_B;

    if (has) {
      // S = Q K^T, dP = dO V^T: M = rows, N = keys; lane (key ln, lh) holds
      // rows 8(i/4) + 4lh + i%4 of its key.
      f32x16 sc, dp;
#pragma unroll
      for (int i = 0; i < 16; ++i) sc[i] = dp[i] = 0.f;
#pragma unroll
      for (int kk = 0; kk < KSTEPS; ++kk) {
        const int ro = r_off(kk);
        const i16x8 qa = *reinterpret_cast<const i16x8*>(qt + ro);
        const i16x8 kf = *reinterpret_cast<const i16x8*>(kmine + ro);
        const i16x8 da = *reinterpret_cast<const i16x8*>(dot + ro);
        const i16x8 vf = *reinterpret_cast<const i16x8*>(vmine + ro);
        sc = Mma<T>::run(bit_cast<V8>(qa), bit_cast<V8>(kf), sc);
        dp = Mma<T>::run(bit_cast<V8>(da), bit_cast<V8>(vf), dp);
      }
      // P and dS from the row statistics of the lane's 16 rows (one group of
      // 4 rows at a time) and its key's mask word.
      uint32_t w = key_ok ? 0xffffffffu : 0u;
      if (tree_blk) w &= visw[(rg * kBufs + s) * kBlockKeys + 32 * kg + ln];
      V8 pb[2], db[2];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4* rp = reinterpret_cast<const float4*>(rs + (rg * kBufs + s) * kTileRows + 8 * q + 4 * lh);
        const float4 st0 = rp[0], st1 = rp[1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * q + e, m = 8 * q + 4 * lh + e;
          const float4 pr = (e < 2) ? st0 : st1;
          const float lse2 = (e & 1) ? pr.z : pr.x;
          const float dvr = (e & 1) ? pr.w : pr.y;
          const float p = ((w >> m) & 1u) ? __builtin_amdgcn_exp2f(__builtin_fmaf(sc[i], sl2, -lse2)) : 0.f;
          pb[i >> 3][i & 7] = (T)p;
          db[i >> 3][i & 7] = (T)(p * (dp[i] - dvr));
        }
      }
      // dV^T += dO^T P, dK^T += Q^T dS: M = d, N = keys, k-step s2 covers rows
      // 16s2 + 8(e/4) + 4lh + e%4 -- elements 8s2 .. 8s2+7 of the accumulator.
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const i16x8 doT = tr_pair(dot + 16 * s2 * ROWB, dt);
          const i16x8 qT = tr_pair(qt + 16 * s2 * ROWB, dt);
          dv[dt] = Mma<T>::run(bit_cast<V8>(doT), pb[s2], dv[dt]);
          dk[dt] = Mma<T>::run(bit_cast<V8>(qT), db[s2], dk[dt]);
        }
    }
  }

  // Row group 1 hands dK^T / dV^T to row group 0 through LDS (the K / V
  // blocks and tile buffers at the start of LDS are free now): register r of
  // lane l at xch[kg][r][l].
  vm_wait<0>();
  sync_lds();
  float* xch = reinterpret_cast<float*>(smem);
  static_assert(4 * 2 * DT * 16 * 64 * 4 <= 2 * KBLK_B + 2 * 2 * kBufs * TILE_B, "exchange fits in K, V and tiles");
  float* xw = xch + kg * (2 * DT * 16 * 64);
  if (rg == 1) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        xw[((2 * dt) * 16 + i) * 64 + lane] = dk[dt][i];
        xw[((2 * dt + 1) * 16 + i) * 64 + lane] = dv[dt][i];
      }
  }
  sync_lds();
  if (rg == 1) return;

  // dK = sm_scale dK^T, dV = dV^T: lane (key ln, lh) holds d = dt*32 +
  // 8(i/4) + 4lh + i%4 of its key.
  if (key_ok) {
    T* dkp = static_cast<T*>(a.dk) + b * a.sdkb + kvh * a.sdkh + (int64_t)mykey * a.sdkn + 4 * lh;
    T* dvp = static_cast<T*>(a.dv) + b * a.sdvb + kvh * a.sdvh + (int64_t)mykey * a.sdvn + 4 * lh;
    typedef T T4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        T4 x, y;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * q + e;
          x[e] = (T)((dk[dt][i] + xw[((2 * dt) * 16 + i) * 64 + lane]) * a.dk_scale);
          y[e] = (T)(dv[dt][i] + xw[((2 * dt + 1) * 16 + i) * 64 + lane]);
        }
        *reinterpret_cast<T4*>(dkp + dt * 32 + 8 * q) = x;
        *reinterpret_cast<T4*>(dvp + dt * 32 + 8 * q) = y;
      }
  }
}

// ------------------------------------------------------------- dQ kernel
constexpr int kQWaves = 4;   // 32 rows each: 128-row chunks
constexpr int kRing = 4;     // LDS ring stages of 32-key units
constexpr int kMaxDqSplits = 16;

template <int D> constexpr size_t dq_lds_bytes() {
  // kRing x (K unit, V unit, mask words of the chunk's 4 row tiles x 32 keys) | dummy load targets
  return (size_t)kRing * (2 * 32 * D * 2 + 4 * 32 * 4) + 64;
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

// Row-parallel dQ: a workgroup owns a 128-row chunk of one (b, kv head) (one
// 32-row tile per wave, Q and dO fragments in registers) and one split of its
// 32-key units (prefix units, then the tree units), streamed through a
// 4-stage LDS ring.  Per unit, on v_mfma_f32_32x32x16:
//   S^T = K Q^T and dP^T = V dO^T (a lane holds one row, so its LSE and Dv
//   are scalars), P^T and dS^T on the VALU, then dQ^T += K^T dS^T with dS^T
//   taken straight from the accumulator (k order permuted to the order it
//   holds keys in; K^T from ds_read_b64_tr_b16 in the same order).
// The workgroup's dQ^T adds to the fp32 accumulator once at the end
// (atomics: several splits of one chunk add to the same rows).
template <typename T, int D>
__global__ __launch_bounds__(kQWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void bwd_dq_main_kernel(const BwdArgs a) {
  typedef typename Mma<T>::vec8 V8;
  constexpr int ROWB = D * 2;
  constexpr int KSTEPS = D / 16;
  constexpr int DT = D / 32;
  constexpr int CPR = D / 8;
  constexpr int RPL = 64 / CPR;
  constexpr int HALF = 32 * ROWB;          // K (or V) bytes of one unit
  constexpr int VISB = 4 * 32 * 4;         // mask words of the chunk's 4 row tiles for the unit's 32 keys
  constexpr int SB = 2 * HALF + VISB;      // ring stage
  constexpr int LPH = HALF / 1024;         // 1 KB loads per half
  constexpr int UPW = 2 * LPH / kQWaves;   // K + V loads per wave per unit
  constexpr int LPU = UPW + 1;             // + the mask words (wave 0, tree units) or a dummy load
  static_assert(UPW >= 1 && UPW * kQWaves == 2 * LPH, "load split");

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  unsigned char* ring = smem;
  unsigned char* dummy = ring + kRing * SB;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 31, lh = lane >> 5;

  // item order: chunk fastest (the chunks of one (b, kv head) read the same
  // K / V units), XCD-aware as in the forward
  const int item = (blockIdx.x & 7) * a.q_items_per_xcd + (blockIdx.x >> 3);
  if (item >= a.q_items) return;
  const int chunk = item % a.n_chunks;
  int rest = item / a.n_chunks;
  const int sp = rest % a.n_splits;
  const int bk = rest / a.n_splits;
  const int kvh = bk % a.num_kv_heads, b = bk / a.num_kv_heads;
  const int G = a.group;
  const int TG = a.q_len * G;
  const int TGP = a.n_tiles * kTileRows;
  const int P = a.prefix_len;
  const float sl2 = a.scale_log2;
  const int tile = chunk * kQWaves + wave;     // this wave's 32-row tile
  const bool active = tile < a.n_tiles;
  const int r = tile * kTileRows + ln;         // this lane's row
  const int n_units = a.n_pu + a.n_tu;
  const int u_lo = sp * a.units_per_split;
  const int mine = max(0, min(a.units_per_split, n_units - u_lo));

  const T* kbase = static_cast<const T*>(a.k) + b * a.skb + kvh * a.skh;
  const T* vbase = static_cast<const T*>(a.v) + b * a.svb + kvh * a.svh;
  const uint32_t* visbase = a.vis + (int64_t)b * a.vis_tree_stride;

  // Q^T and dO^T operands (B[d][row]: lane (row ln, lh) holds d = 16kk + 8lh
  // + [0, 8)) and the row's statistics, in registers for the whole walk.
  // Loaded before any ring load and consumed at once, so the compiler's wait
  // for them covers nothing else.
  i16x8 qf[KSTEPS], df[KSTEPS];
  float lse2 = INFINITY, dvr = 0.f;
  {
    const int R = min(r, TG - 1);
    const int t = R / G, g = R - t * G;
    const T* qp = static_cast<const T*>(a.q) + b * a.sqb + (int64_t)(kvh * G + g) * a.sqh + (int64_t)t * a.sqm + 8 * lh;
    const T* dp = static_cast<const T*>(a.dout) + b * a.sdob + (int64_t)(kvh * G + g) * a.sdoh +
                  (int64_t)t * a.sdom + 8 * lh;
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
      qf[kk] = *reinterpret_cast<const i16x8*>(qp + 16 * kk);
      df[kk] = *reinterpret_cast<const i16x8*>(dp + 16 * kk);
    }
    if (active) {
      const float2 st = a.rowstat[(int64_t)bk * TGP + r];  // padding rows: (+inf, 0)
      lse2 = st.x;
      dvr = st.y;
    }
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) asm volatile("" : : "v"(qf[kk]), "v"(df[kk]));
    asm volatile("" : : "v"(lse2), "v"(dvr));
  }

  auto key0_of = [&](int u) { return u < a.n_pu ? 32 * u : P + 32 * (u - a.n_pu); };
  // HBM -> LDS: this wave's share of unit u into stage st.
  auto issue = [&](int st, int u) {
    unsigned char* sb = ring + st * SB;
    const int key0 = key0_of(u);
#pragma unroll
    for (int i = 0; i < UPW; ++i) {
      const int v = wave * UPW + i;  // 0 .. 2*LPH-1: K loads, then V loads
      const bool is_v = v >= LPH;
      const int vl = is_v ? v - LPH : v;
      const int row = vl * RPL + lane / CPR, pos = lane % CPR;
      const int key = min(key0 + row, a.kv_len - 1);
      const T* src = (is_v ? vbase + (int64_t)key * a.svn : kbase + (int64_t)key * a.skn) + ((pos ^ swz<D>(row)) << 3);
      dma16(src, lds_addr(sb + (is_v ? HALF : 0) + vl * 1024));
    }
    if (wave == 0 && u >= a.n_pu) {
      // words [tile][tree key]: 4 tiles x 32 keys x 4 B, 8 lanes per tile
      if (lane < 32) {
        const int jt = min(chunk * kQWaves + (lane >> 3), a.n_tiles - 1);
        dma16(visbase + (int64_t)jt * a.n_tkeys + 32 * (u - a.n_pu) + 4 * (lane & 7), lds_addr(sb + 2 * HALF));
      }
    } else if (lane == 0) {
      dma16(a.rowstat, lds_addr(dummy + 16 * wave));
    }
  };

  // LDS offsets: row reads of K / V (lane (key ln, lh), chunk 2kk + lh) and
  // transposed reads of K (rows 8jj + 4(x>>1) + (i>>2), d = dt*32 + 16(x&1) +
  // 4(i&3)); the tiles use the same swizzle as the dK / dV kernel.
  const int vx = lane >> 4, vi = lane & 15;
  auto r_off = [&](int kk) { return ln * ROWB + (((2 * kk + lh) ^ swz<D>(ln)) << 4); };
  auto t_off = [&](int dt, int jj) {
    const int rr = 8 * jj + 4 * (vx >> 1) + (vi >> 2);
    const int d = dt * 32 + 16 * (vx & 1) + 4 * (vi & 3);
    return rr * ROWB + (((d >> 3) ^ swz<D>(rr)) << 4) + ((d & 7) << 1);
  };

  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[dt][i] = 0.f;

  for (int j = 0; j < kRing - 1 && j < mine; ++j) issue(j, u_lo + j);
  for (int j = 0; j < mine; ++j) {
    // unit j landed for every wave (later units in flight: up to kRing-2);
    // every wave is done with unit j-1, whose stage unit j+kRing-1 reuses
    wait_units<LPU, kRing - 2>(min(mine - 1 - j, kRing - 2));
    sync_lds();
    if (j + kRing - 1 < mine) issue((j + kRing - 1) % kRing, u_lo + j + kRing - 1);
    if (!active) continue;
    const unsigned char* sb = ring + (j % kRing) * SB;
    const int u = u_lo + j;
    const bool tree_u = u >= a.n_pu;
    // S^T = K Q^T, dP^T = V dO^T: M = keys, N = rows; lane (row ln, lh)
    // holds keys 8(i/4) + 4lh + i%4.
    f32x16 sc, dp;
#pragma unroll
    for (int i = 0; i < 16; ++i) sc[i] = dp[i] = 0.f;
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
      const int ro = r_off(kk);
      const i16x8 kf = *reinterpret_cast<const i16x8*>(sb + ro);
      const i16x8 vf = *reinterpret_cast<const i16x8*>(sb + HALF + ro);
      sc = Mma<T>::run(bit_cast<V8>(kf), bit_cast<V8>(qf[kk]), sc);
      dp = Mma<T>::run(bit_cast<V8>(vf), bit_cast<V8>(df[kk]), dp);
    }
    // visibility of the lane's 16 keys from its row: prefix keys below P;
    // tree keys: bit ln of each key's word for this wave's tile
    uint32_t vis16 = 0;
    if (tree_u) {
      const uint32_t* wv = reinterpret_cast<const uint32_t*>(sb + 2 * HALF) + wave * 32;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint4 w4 = *reinterpret_cast<const uint4*>(wv + 8 * q + 4 * lh);
        vis16 |= ((w4.x >> ln) & 1u) << (4 * q + 0);
        vis16 |= ((w4.y >> ln) & 1u) << (4 * q + 1);
        vis16 |= ((w4.z >> ln) & 1u) << (4 * q + 2);
        vis16 |= ((w4.w >> ln) & 1u) << (4 * q + 3);
      }
    } else {
      const int key0 = 32 * u;
#pragma unroll
      for (int i = 0; i < 16; ++i) vis16 |= (uint32_t)(key0 + 8 * (i >> 2) + 4 * lh + (i & 3) < P) << i;
    }
    V8 db[2];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float p = ((vis16 >> i) & 1u) ? __builtin_amdgcn_exp2f(__builtin_fmaf(sc[i], sl2, -lse2)) : 0.f;
      db[i >> 3][i & 7] = (T)(p * (dp[i] - dvr));
    }
    // dQ^T += K^T dS^T: M = d, N = rows, k-step s2 covers keys 16s2 + 8(e/4)
    // + 4lh + e%4 -- elements 8s2 .. 8s2+7 of the accumulator.
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (TSFA_LDS i16x4*)(sb + 16 * s2 * ROWB + t_off(dt, 0)));
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (TSFA_LDS i16x4*)(sb + 16 * s2 * ROWB + t_off(dt, 1)));
        const i16x8 kT = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        acc[dt] = Mma<T>::run(bit_cast<V8>(kT), db[s2], acc[dt]);
      }
  }
  // lane (row ln, lh) holds d = dt*32 + 8(i/4) + 4lh + i%4.  One split per
  // chunk: the workgroup owns its rows' dQ and writes it in the input dtype.
  // Otherwise it adds to the d-major fp32 accumulator (each instruction's 64
  // lanes cover two whole 128-byte lines).
  if (active && mine > 0) {
    if (a.dq_direct) {
      if (r < TG) {
        const int t = r / G, g = r - t * G;
        T* dst = static_cast<T*>(a.dq) + b * a.sdqb + (int64_t)(kvh * G + g) * a.sdqh + (int64_t)t * a.sdqm + 4 * lh;
        typedef T T4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            T4 x;
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = (T)(acc[dt][4 * q + e] * a.dq_scale);
            *reinterpret_cast<T4*>(dst + dt * 32 + 8 * q) = x;
          }
      }
    } else {
      float* dq = a.dq_acc + ((int64_t)bk * D + 4 * lh) * TGP + r;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          atomicAdd(dq + (int64_t)(dt * 32 + 8 * (i >> 2) + (i & 3)) * TGP, acc[dt][i]);
    }
  }
}

// ------------------------------------------------------------ prep / dq / vis
struct PrepArgs {
  const void* o;
  const void* dout;
  const float* lse;  // [B, Hq, q_len]
  float2* rowstat;   // [B*Hkv][n_tiles*32]
  float* dq_acc;     // [B*Hkv][D][TGP]
  int64_t sob, soh, som, sdob, sdoh, sdom;
  int batch, num_heads, num_kv_heads, group, q_len, n_tiles;
  int zero_dq;       // clear the accumulator (the dQ kernel adds into it)
};

// 16 lanes per row of the padded row space B*Hkv*TGP (workgroup `blk` of the
// prep range).
template <typename T, int D>
__device__ inline void bwd_prep(const PrepArgs& a, int blk) {
  constexpr int EPL = D / 16;  // elements per lane
  const int64_t gid = (int64_t)blk * 256 + threadIdx.x;
  const int64_t row = gid >> 4;
  const int part = (int)(gid & 15);
  const int TG = a.q_len * a.group;
  const int TGP = a.n_tiles * kTileRows;
  const int64_t nrows = (int64_t)a.batch * a.num_kv_heads * TGP;
  const bool live = row < nrows;
  const int64_t bk = live ? row / TGP : 0;
  const int R = live ? (int)(row - bk * TGP) : 0;
  const bool real = live && R < TG;
  float acc = 0.f, lse = -INFINITY;
  if (real) {
    const int t = R / a.group, g = R - t * a.group;
    const int kvh = (int)(bk % a.num_kv_heads), b = (int)(bk / a.num_kv_heads);
    const int h = kvh * a.group + g;
    typedef T TV __attribute__((ext_vector_type(EPL)));
    const TV ov = *reinterpret_cast<const TV*>(static_cast<const T*>(a.o) + b * a.sob + (int64_t)h * a.soh +
                                               (int64_t)t * a.som + part * EPL);
    const TV dv = *reinterpret_cast<const TV*>(static_cast<const T*>(a.dout) + b * a.sdob + (int64_t)h * a.sdoh +
                                               (int64_t)t * a.sdom + part * EPL);
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc += (float)ov[e] * (float)dv[e];
    lse = a.lse[((int64_t)b * a.num_heads + h) * a.q_len + t];
  }
  if (live && a.zero_dq) {
    float* dq = a.dq_acc + ((int64_t)bk * D + part * EPL) * TGP + R;
#pragma unroll
    for (int e = 0; e < EPL; ++e) dq[(int64_t)e * TGP] = 0.f;
  }
#pragma unroll
  for (int off = 8; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 16);
  if (live && part == 0) {
    const bool empty = !(lse > -INFINITY);  // no visible key (or a padding row)
    a.rowstat[row] = empty ? make_float2(INFINITY, 0.f) : make_float2(lse * 1.4426950408889634f, acc);
  }
}

struct DqArgs {
  const float* dq_acc;  // [B*Hkv][D][tgp]
  void* dq;
  int64_t sqb, sqh, sqm;
  float scale;
  int batch, num_kv_heads, group, q_len, tgp;
};

// Thread (bk, part, R), R fastest: 8 d of one row, read d-major (coalesced
// across the threads of a part).
template <typename T, int D>
__global__ __launch_bounds__(256) void bwd_dq_kernel(const DqArgs a) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int TG = a.q_len * a.group;
  const int64_t per_bk = (int64_t)(D / 8) * TG;
  if (gid >= (int64_t)a.batch * a.num_kv_heads * per_bk) return;
  const int64_t bk = gid / per_bk;
  const int rem = (int)(gid - bk * per_bk);
  const int part = rem / TG, R = rem - part * TG;
  const int t = R / a.group, g = R - t * a.group;
  const int kvh = (int)(bk % a.num_kv_heads), b = (int)(bk / a.num_kv_heads);
  const float* src = a.dq_acc + ((int64_t)bk * D + part * 8) * a.tgp + R;
  typedef T T8 __attribute__((ext_vector_type(8)));
  T8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = (T)(src[(int64_t)e * a.tgp] * a.scale);
  *reinterpret_cast<T8*>(static_cast<T*>(a.dq) + b * a.sqb + (int64_t)(kvh * a.group + g) * a.sqh +
                         (int64_t)t * a.sqm + part * 8) = o;
}

struct VisArgs {
  const int32_t* row_ptr;
  const int32_t* col_idx;
  const int8_t* blk_type;
  const int32_t* payload;
  const int32_t* offset;
  int64_t ms_row_ptr, ms_col_idx, ms_blk_type, ms_payload, ms_offset;
  uint32_t* vis;  // [n_trees][n_tiles][n_tkeys]
  int64_t tree_stride;
  int group, q_len, block_m, block_n, n_tree_blocks, tree_key_limit, n_tiles, n_tkeys;
};

// One workgroup per (tile, tree, 64 tree keys): the block states of the
// tile's q-blocks (0 ZERO, -1 FULL, 1 + offset MIXED) expand into LDS, then
// each thread decides one (key, row) bit and a ballot assembles the 32-row
// words (lanes 0-31: one key, lanes 32-63: the next).
__device__ inline void bwd_vis(const VisArgs& a, int tile, int tree, int zc, int* st, int* rps) {
  const int c0 = zc * 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = a.group, BM = a.block_m, BN = a.block_n, ntb = a.n_tree_blocks;
  const int TG = a.q_len * G;
  const int r_lo = tile * kTileRows;
  const int r_hi = min(r_lo + kTileRows, TG) - 1;
  uint32_t* out = a.vis + (int64_t)tree * a.tree_stride + (int64_t)tile * a.n_tkeys;
  const int qb_lo = (r_lo / G) / BM, qb_hi = (r_hi / G) / BM, nqbc = qb_hi - qb_lo + 1;
  const int32_t* rp = a.row_ptr + tree * a.ms_row_ptr;
  const int32_t* ci = a.col_idx + tree * a.ms_col_idx;
  const int8_t* bt = a.blk_type + tree * a.ms_blk_type;
  const int32_t* pl = a.payload + tree * a.ms_payload;
  const int32_t* of = a.offset + tree * a.ms_offset;
  for (int i = tid; i < nqbc * ntb; i += 256) st[i] = 0;
  if (tid <= nqbc) rps[tid] = rp[qb_lo + tid];
  __syncthreads();
  for (int e = rps[0] + tid; e < rps[nqbc]; e += 256) {
    int qq = 0;
    while (qq + 1 < nqbc && rps[qq + 1] <= e) ++qq;
    const int tb = ci[e];
    // a block of any kind but MIXED is FULL (tree_sparse_flashattn.py:313-318)
    if (tb >= 0 && tb < ntb) st[qq * ntb + tb] = (bt[e] != TSFA_MIXED_BLOCK) ? -1 : (of[e] + 1);
  }
  __syncthreads();
  const int R = r_lo + (lane & 31);
  const int t = R / G, qb = t / BM;
#pragma unroll
  for (int pass = 0; pass < 8; ++pass) {
    const int c = c0 + pass * 8 + wave * 2 + (lane >> 5);  // this thread's tree key
    bool bit = false;
    if (R <= r_hi && c < a.tree_key_limit) {
      const int tb = c / BN;
      const int e = st[(qb - qb_lo) * ntb + tb];
      bit = e < 0;
      if (e > 0) {
        const int flat = (t - qb * BM) * BN + (c - tb * BN);
        bit = ((uint32_t)pl[e - 1 + (flat >> 5)] >> (flat & 31)) & 1u;
      }
    }
    const uint64_t bal = __ballot(bit);
    if ((lane & 31) == 0 && c < a.n_tkeys) out[c] = (uint32_t)(bal >> (lane & 32));
  }
}

// Prep and visibility words in one launch: blocks [0, prep_blocks) run the
// prep, the rest one (tile, tree, 64-key chunk) of the visibility words each.
template <typename T, int D>
__global__ __launch_bounds__(256) void bwd_prep_vis_kernel(const PrepArgs pa, const VisArgs va, int prep_blocks,
                                                           int vis_chunks) {
  __shared__ int st[kMaxStateInts];
  __shared__ int rps[72];
  const int blk = blockIdx.x;
  if (blk < prep_blocks) {
    bwd_prep<T, D>(pa, blk);
    return;
  }
  const int v = blk - prep_blocks;
  const int zc = v % vis_chunks, rest = v / vis_chunks;
  bwd_vis(va, rest % va.n_tiles, rest / va.n_tiles, zc, st, rps);
}

// ------------------------------------------------------------------- host
// A side stream and fork/join events per (device, caller stream): the dQ
// kernel runs beside the dK/dV kernel, so its workgroups fill the CUs that
// the dK/dV grid leaves idle (a partial last round: 264 workgroups of one
// per CU on 256 CUs at the Llama-3-8B shape).  Default priority; the side
// stream does not synchronise with the null stream.  A call captured into a
// graph forks and joins inside the capture.
constexpr int kMaxSideStreams = 64;

struct SideStream {
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};

const SideStream* side_stream(hipStream_t stream) {
  static std::mutex mu;
  static std::map<std::pair<int, uintptr_t>, SideStream> sides;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_pair(dev, reinterpret_cast<uintptr_t>(stream));
  auto it = sides.find(key);
  if (it != sides.end()) return &it->second;
  // at most kMaxSideStreams per device; callers past that run on one stream
  static int per_dev[64] = {};
  if (dev < 0 || dev >= 64 || per_dev[dev] >= kMaxSideStreams) return nullptr;
  SideStream ss;
  if (hipStreamCreateWithFlags(&ss.s, hipStreamNonBlocking) != hipSuccess) return nullptr;
  if (hipEventCreateWithFlags(&ss.fork, hipEventDisableTiming) != hipSuccess) {
    (void)hipStreamDestroy(ss.s);
    return nullptr;
  }
  if (hipEventCreateWithFlags(&ss.join, hipEventDisableTiming) != hipSuccess) {
    (void)hipEventDestroy(ss.fork);
    (void)hipStreamDestroy(ss.s);
    return nullptr;
  }
  ++per_dev[dev];
  return &sides.emplace(key, ss).first->second;
}

template <typename T, int D>
int launch_bwd(const BwdArgs& ba, const PrepArgs& pa, const VisArgs& va, const DqArgs& da, const BwdPlan& p,
               bool has_tree, hipStream_t stream) {
  static std::atomic<uint64_t> attr_set{0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return TSFA_ERR_DEVICE;
  const uint64_t bit = 1ull << (dev & 63);
  if ((attr_set.load(std::memory_order_acquire) & bit) == 0) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&bwd_kv_kernel<T, D>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)kv_lds_bytes<D>()) != hipSuccess)
      return TSFA_ERR_LAUNCH;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&bwd_dq_main_kernel<T, D>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)dq_lds_bytes<D>()) != hipSuccess)
      return TSFA_ERR_LAUNCH;
    attr_set.fetch_or(bit, std::memory_order_acq_rel);
  }
  const int64_t prep_threads = (int64_t)pa.batch * pa.num_kv_heads * p.n_tiles * kTileRows * 16;
  const int64_t prep_blocks = (prep_threads + 255) / 256;
  const int vis_chunks = p.n_tkeys / 64;
  const int64_t vis_blocks = has_tree ? (int64_t)p.n_tiles * p.n_trees * vis_chunks : 0;
  if (prep_blocks + vis_blocks > INT32_MAX) return TSFA_ERR_UNSUPPORTED;
  hipLaunchKernelGGL((bwd_prep_vis_kernel<T, D>), dim3((unsigned)(prep_blocks + vis_blocks)), dim3(256), 0, stream,
                     pa, va, (int)prep_blocks, std::max(1, vis_chunks));
  if (hipGetLastError() != hipSuccess) return TSFA_ERR_LAUNCH;
  const unsigned grid = (unsigned)ba.items_per_xcd * 8;
  const bool concurrent = config().bwd_concurrent != 0;  // TSFA_BWD_CONCURRENT=0: one stream (measurements)
  const SideStream* side = (ba.q_items > 0 && concurrent) ? side_stream(stream) : nullptr;
  if (side != nullptr && (hipEventRecord(side->fork, stream) != hipSuccess ||
                          hipStreamWaitEvent(side->s, side->fork, 0) != hipSuccess))
    return TSFA_ERR_LAUNCH;
  hipLaunchKernelGGL((bwd_kv_kernel<T, D>), dim3(grid), dim3(kWaves * 64), kv_lds_bytes<D>(), stream, ba);
  if (hipGetLastError() != hipSuccess) return TSFA_ERR_LAUNCH;
  if (ba.q_items > 0) {
    const unsigned qgrid = (unsigned)ba.q_items_per_xcd * 8;
    hipLaunchKernelGGL((bwd_dq_main_kernel<T, D>), dim3(qgrid), dim3(kQWaves * 64), dq_lds_bytes<D>(),
                       side != nullptr ? side->s : stream, ba);
    if (hipGetLastError() != hipSuccess) return TSFA_ERR_LAUNCH;
    if (side != nullptr && (hipEventRecord(side->join, side->s) != hipSuccess ||
                            hipStreamWaitEvent(stream, side->join, 0) != hipSuccess))
      return TSFA_ERR_LAUNCH;
  }
  if (ba.dq_direct) return TSFA_OK;
  const int64_t dq_threads = (int64_t)da.batch * da.num_kv_heads * da.q_len * da.group * (D / 8);
  hipLaunchKernelGGL((bwd_dq_kernel<T, D>), dim3((unsigned)((dq_threads + 255) / 256)), dim3(256), 0, stream, da);
  return hipGetLastError() == hipSuccess ? TSFA_OK : TSFA_ERR_LAUNCH;
}

}  // namespace bwd
}  // namespace tsfa

using namespace tsfa;
using namespace tsfa::bwd;

extern "C" int tsfa_bwd(const void* q, const void* k, const void* v, const void* o, const float* lse,
                        const void* dout, void* dq, void* dk, void* dv, const int32_t* row_ptr,
                        const int32_t* col_idx, const int8_t* blk_type, const int32_t* mixed_mask_payload,
                        const int32_t* mixed_mask_offset, const int64_t* meta_seq_stride, const int64_t* strides,
                        float sm_scale, int batch, int num_heads, int num_kv_heads, int q_len, int kv_len,
                        int prefix_len, int n_q_blocks, int n_tree_blocks, int gqa_group_size, int block_m,
                        int block_n, int head_dim, int dtype, void* workspace, size_t workspace_bytes,
                        tsfa_stream_t stream_) {
  int st = tsfa_fwd_check_args(batch, num_heads, num_kv_heads, q_len, kv_len, prefix_len, n_q_blocks,
                               n_tree_blocks, gqa_group_size, block_m, block_n, head_dim, dtype);
  if (st != TSFA_OK) return st;
  // the backward kernels: 16-bit inputs, head_dim 64 or 128
  if ((dtype != TSFA_DTYPE_FP16 && dtype != TSFA_DTYPE_BF16) || (head_dim != 64 && head_dim != 128))
    return TSFA_ERR_UNSUPPORTED;
  if (batch == 0 || q_len == 0) return TSFA_OK;
  if (strides == nullptr || meta_seq_stride == nullptr) return TSFA_ERR_INVALID_ARGUMENT;
  const void* ptrs[9] = {q, k, v, o, dout, dq, dk, dv, lse};
  for (const void* ptr : ptrs)
    if (ptr == nullptr) return TSFA_ERR_INVALID_ARGUMENT;
  if (row_ptr == nullptr) return TSFA_ERR_INVALID_ARGUMENT;
  // strides: q, k, v, o, dout, dq, dk, dv -- (b, h, n, d) each
  for (int i = 0; i < 8; ++i) {
    if (strides[4 * i + 3] != 1) return TSFA_ERR_UNSUPPORTED;
    for (int j = 0; j < 3; ++j)
      if (strides[4 * i + j] % 8 != 0) return TSFA_ERR_UNSUPPORTED;
  }
  for (int i = 0; i < 8; ++i)
    if (reinterpret_cast<uintptr_t>(ptrs[i]) % 16 != 0) return TSFA_ERR_UNSUPPORTED;
  bool per_seq = false;
  for (int i = 0; i < 5; ++i) {
    if (meta_seq_stride[i] < 0) return TSFA_ERR_INVALID_ARGUMENT;
    per_seq = per_seq || meta_seq_stride[i] != 0;
  }
  const int n_trees = per_seq ? batch : 1;
  BwdPlan p;
  st = make_bwd_plan(batch, num_kv_heads, q_len, kv_len, prefix_len, gqa_group_size, head_dim, block_m,
                     n_tree_blocks, n_trees, &p);
  if (st != TSFA_OK) return st;
  if (workspace == nullptr || workspace_bytes < p.rowstat_bytes + p.dq_bytes + p.vis_bytes)
    return TSFA_ERR_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0) return TSFA_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  float2* rowstat = reinterpret_cast<float2*>(ws);
  float* dq_acc = reinterpret_cast<float*>(ws + p.rowstat_bytes);
  uint32_t* vis = reinterpret_cast<uint32_t*>(ws + p.rowstat_bytes + p.dq_bytes);
  const int tree_key_limit =
      (int)std::min<int64_t>((int64_t)n_tree_blocks * block_n, (int64_t)kv_len - prefix_len);

  // signed: P = exp2(q.k * sl2 - lse2); a zero scale becomes a vanishing one
  float sl2 = sm_scale * 1.4426950408889634f;
  if (sl2 == 0.f) sl2 = 1e-30f;

  PrepArgs pa;
  pa.o = o;
  pa.dout = dout;
  pa.lse = lse;
  pa.rowstat = rowstat;
  pa.dq_acc = dq_acc;
  pa.sob = strides[12];
  pa.soh = strides[13];
  pa.som = strides[14];
  pa.sdob = strides[16];
  pa.sdoh = strides[17];
  pa.sdom = strides[18];
  pa.batch = batch;
  pa.num_heads = num_heads;
  pa.num_kv_heads = num_kv_heads;
  pa.group = gqa_group_size;
  pa.q_len = q_len;
  pa.n_tiles = p.n_tiles;

  VisArgs va;
  va.row_ptr = row_ptr;
  va.col_idx = col_idx;
  va.blk_type = blk_type;
  va.payload = mixed_mask_payload;
  va.offset = mixed_mask_offset;
  va.ms_row_ptr = meta_seq_stride[0];
  va.ms_col_idx = meta_seq_stride[1];
  va.ms_blk_type = meta_seq_stride[2];
  va.ms_payload = meta_seq_stride[3];
  va.ms_offset = meta_seq_stride[4];
  va.vis = vis;
  va.tree_stride = (int64_t)p.n_tiles * p.n_tkeys;
  va.group = gqa_group_size;
  va.q_len = q_len;
  va.block_m = block_m;
  va.block_n = block_n;
  va.n_tree_blocks = n_tree_blocks;
  va.tree_key_limit = tree_key_limit;
  va.n_tiles = p.n_tiles;
  va.n_tkeys = p.n_tkeys;

  BwdArgs ba;
  ba.q = q;
  ba.k = k;
  ba.v = v;
  ba.dout = dout;
  ba.dk = dk;
  ba.dv = dv;
  ba.dq_acc = dq_acc;
  ba.rowstat = rowstat;
  ba.vis = vis;
  ba.sqb = strides[0];
  ba.sqh = strides[1];
  ba.sqm = strides[2];
  ba.skb = strides[4];
  ba.skh = strides[5];
  ba.skn = strides[6];
  ba.svb = strides[8];
  ba.svh = strides[9];
  ba.svn = strides[10];
  ba.sdob = strides[16];
  ba.sdoh = strides[17];
  ba.sdom = strides[18];
  ba.sdkb = strides[24];
  ba.sdkh = strides[25];
  ba.sdkn = strides[26];
  ba.sdvb = strides[28];
  ba.sdvh = strides[29];
  ba.sdvn = strides[30];
  ba.vis_tree_stride = n_trees > 1 ? va.tree_stride : 0;
  ba.scale_log2 = sl2;
  ba.dk_scale = sm_scale;
  ba.num_kv_heads = num_kv_heads;
  ba.group = gqa_group_size;
  ba.q_len = q_len;
  ba.kv_len = kv_len;
  ba.prefix_len = prefix_len;
  ba.n_tiles = p.n_tiles;
  ba.n_pb = p.n_pb;
  ba.n_tb = p.n_tb;
  ba.n_tkeys = p.n_tkeys;
  ba.n_items = batch * num_kv_heads * (p.n_pb + p.n_tb);
  // row-parallel dQ: 128-row chunks; the 32-key units (prefix, then the tree
  // keys up to tree_key_limit) split so the grid covers about two workgroups
  // per CU (two fit, and their waves interleave), at most kMaxDqSplits ways
  // (each split adds its chunk's dQ once with atomics: splits x rows x D x 4
  // bytes of atomic traffic; an unsplit chunk writes dQ directly)
  ba.n_pu = ceil_div(prefix_len, 32);
  ba.n_tu = ceil_div(tree_key_limit, 32);
  ba.n_chunks = ceil_div(p.n_tiles, kQWaves);
  {
    int cus = 256;
    if (device_cu_count(&cus) != TSFA_OK) return TSFA_ERR_DEVICE;
    const int n_units = ba.n_pu + ba.n_tu;
    const int64_t base = (int64_t)batch * num_kv_heads * ba.n_chunks;
    const int64_t want = std::min<int64_t>(kMaxDqSplits, std::max<int64_t>(1, (2 * cus + base - 1) / base));
    int splits = (int)std::min<int64_t>(want, std::max(1, n_units));
    ba.units_per_split = std::max(1, ceil_div(n_units, splits));
    ba.n_splits = std::max(1, ceil_div(n_units, ba.units_per_split));
    const int64_t q_items = n_units > 0 ? base * ba.n_splits : 0;
    if (q_items > INT32_MAX / 2) return TSFA_ERR_UNSUPPORTED;
    ba.q_items = (int)q_items;
    ba.q_items_per_xcd = (ba.q_items + 7) / 8;
  }
  ba.dq = dq;
  ba.sdqb = strides[20];
  ba.sdqh = strides[21];
  ba.sdqm = strides[22];
  ba.dq_scale = sm_scale;
  ba.dq_direct = (ba.n_splits == 1 && ba.q_items > 0) ? 1 : 0;
  pa.zero_dq = ba.dq_direct ? 0 : 1;
  ba.group_magic = gqa_group_size > 1 ? (uint32_t)((((uint64_t)1) << 32) / (uint64_t)gqa_group_size + 1) : 0u;
  ba.items_per_xcd = (ba.n_items + 7) / 8;

  DqArgs da;
  da.dq_acc = dq_acc;
  da.dq = dq;
  da.sqb = strides[20];
  da.sqh = strides[21];
  da.sqm = strides[22];
  da.scale = sm_scale;
  da.batch = batch;
  da.num_kv_heads = num_kv_heads;
  da.group = gqa_group_size;
  da.q_len = q_len;
  da.tgp = p.n_tiles * kTileRows;

  const bool has_tree = p.n_tb > 0;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  if (dtype == TSFA_DTYPE_BF16)
    return head_dim == 128 ? launch_bwd<__bf16, 128>(ba, pa, va, da, p, has_tree, stream)
                           : launch_bwd<__bf16, 64>(ba, pa, va, da, p, has_tree, stream);
  return head_dim == 128 ? launch_bwd<_Float16, 128>(ba, pa, va, da, p, has_tree, stream)
                         : launch_bwd<_Float16, 64>(ba, pa, va, da, p, has_tree, stream);
}
