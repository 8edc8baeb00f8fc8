// Greedy next-token selection fused with the lm_head projection:
//   ids[b] = argmax_v round(hidden[b] . weight[v])
// where round() is the rounding of the fp32 dot product to the model dtype (the
// reference compares the lm_head's output logits, which are in that dtype), NaN
// counts as the largest value, and ties go to the smallest index (torch.argmax).
// Replaces self.lm_head(hidden_states) (models/llama3/model.py:156 of the
// reference) followed by torch.argmax(logits[:, -1, :]) (model.py:214) for the
// last position, without writing the [B, V] logits.
//
// Kernels:
//   * lm_head_argmax_mfma_kernel (bf16/f16, K % 128 == 0, up to 32 hidden rows
//     per launch): one workgroup per CU, each owning a contiguous range of
//     vocab rows (V / grid, balanced to one row), which it walks in blocks of
//     64 rows; with the counters, k whole blocks each and then single blocks
//     drawn from a pool by a ticket, so the faster XCDs take more of them. Weight rows stream through LDS in 256-column tiles (buffer-to-
//     LDS DMA, 512-byte runs per row, a three-stage ring with two tiles in
//     flight) together with the matching 256 columns of the hidden rows; the
//     ring runs on across block boundaries, so a block's start and finish
//     overlap the neighbouring blocks' streams. Its 4 waves are 2 row groups x
//     2 column halves; each computes
//     logits^T[32 vocab x 32 batch] += W[32 x 16] hidden^T[16 x 32] on
//     v_mfma_f32_32x32x16 over its half; at a block's end the halves are
//     added through LDS, rounded, and folded into each lane's running best
//     (value, index). At the end the workgroup's best per batch row is either
//     merged into packed 64-bit (value, index) keys with atomic max, the last
//     workgroup (ticket) writing the ids and returning keys and ticket to zero
//     (with a counters buffer), or written as a partial for the reduce kernel.
//   * lm_head_argmax_generic_kernel (any dtype / K): one lane per vocab row.
//   * lm_head_argmax_reduce_kernel: one workgroup per batch row reduces the
//     partials to the final id (int64) and, optionally, the winning logit.
// HBM-bound: the weight (V x K x 2 bytes, 1.05 GB for Llama-3-8B) is read once.
#include <limits.h>
#include <algorithm>
#include <math.h>

#include <type_traits>

#include "attn_tiles.h"
#include "lc_common.h"

namespace {

using namespace lc_attn;

// A workgroup: 2 row groups of 32 vocab rows x 2 halves of each tile's
// columns, one wave each. 512-byte runs per row: at one workgroup per CU a
// stream of 64 rows x 512 B tiles measured 5.85 TB/s against 5.49 TB/s for
// 128 rows x 256 B (same bytes per tile).
constexpr int kLhWaves = 4;
constexpr int kLhRowWaves = 2;
constexpr int kLhRows = 32 * kLhRowWaves;  // vocab rows per workgroup
constexpr int kLhKc = 256;              // hidden columns per tile (512-byte runs per row)
constexpr int kLhKHalf = kLhKc / 2;     // columns of a tile per wave
constexpr int kLhStages = 3;            // LDS ring depth: two tiles in flight
// (deeper rings, and 64-column tiles, measured no faster)
// Cache policy of the weight loads: non-temporal. Each weight byte is read
// once; streaming it past the caches measured 11% faster (230 -> 207 us at
// the Llama-3-8B vocab) than the default policy. The hidden rows, re-read by
// every workgroup, keep the default policy.
constexpr bool kLhWeightNt = true;
constexpr int kLhBatch = 32;            // hidden rows per launch
constexpr int kLhGenRows = 256;         // vocab rows per generic workgroup

// (value, index) order of torch.argmax: NaN above everything (first NaN wins),
// then larger value, then smaller index.
__device__ __forceinline__ bool lh_better(float xa, int ia, float xb, int ib) {
  const bool na = xa != xa, nb = xb != xb;
  if (na || nb) return na && (!nb || ia < ib);
  if (xa != xb) return xa > xb;
  return ia < ib;
}

__device__ __forceinline__ void lh_take(float& bv, int& bi, float xv, int xi) {
  if (lh_better(xv, xi, bv, bi)) {
    bv = xv;
    bi = xi;
  }
}

// LDS swizzle of the 512-byte tile rows: 16-byte chunk c of row r sits at
// c ^ s(r), s a permutation of 0..15 over 16 consecutive rows (the 256-byte
// rows' swizzle), so the 16 lanes of an operand read (16 rows, one chunk) hit
// 16 different 16-byte bank groups.
__device__ __forceinline__ int lh_swz(int r) { return pf_swz<16>(r); }

// s_waitcnt immediate: vmcnt(vm) lgkmcnt(lgkm), expcnt not waited on.
constexpr int lh_waitcnt(int vm, int lgkm) {
  return (vm & 0xF) | ((vm >> 4) << 14) | (7 << 4) | (lgkm << 8);
}

struct LhArgs {
  const void* hidden;
  const void* weight;
  float* part_val;  // [n_wg][pstride]
  int* part_idx;
  // Packed best keys [kLhBatch] followed by the ticket (zero at entry, left
  // zero), or null: partials for the reduce kernel.
  unsigned long long* keys;
  // Block pool (with the counters): the vocab blocks from pool_begin on are
  // handed out by a ticket; null: every workgroup owns a contiguous range.
  int* pool_ticket;
  int pool_begin, pool_blocks;
  int64_t* ids;
  float* max_out;
  int64_t hs, ws;  // row strides (elements)
  int B, K, V, pstride;
};

// (value, index) as one unsigned 64-bit key whose order is lh_better's: the
// high word orders the values (NaN above +inf, -0 taken as +0), the low word
// is ~index, so among equal values the smaller index is larger. Key 0 is
// below every (value, index) pair.
__device__ __forceinline__ unsigned long long lh_pack(float x, int idx) {
  // x + 0 turns -0 into +0 (round to nearest) and keeps every other value;
  // negative values flip every bit, others only the sign bit. Branch-free.
  const uint32_t b = __float_as_uint(x + 0.f);
  const uint32_t m = static_cast<uint32_t>(static_cast<int32_t>(b) >> 31);
  const uint32_t hi = x != x ? 0xFFFFFFFFu : (b ^ (m | 0x80000000u));
  return (static_cast<unsigned long long>(hi) << 32) | static_cast<uint32_t>(~idx);
}
__device__ __forceinline__ unsigned long long lh_max_key(unsigned long long a,
                                                         unsigned long long b) {
  return a > b ? a : b;
}
__device__ __forceinline__ float lh_unpack_value(unsigned long long key) {
  const uint32_t hi = static_cast<uint32_t>(key >> 32);
  if (hi == 0xFFFFFFFFu) return __uint_as_float(0x7FC00000u);
  return __uint_as_float((hi & 0x80000000u) ? (hi & 0x7FFFFFFFu) : ~hi);
}
__device__ __forceinline__ int lh_unpack_index(unsigned long long key) {
  return static_cast<int>(~static_cast<uint32_t>(key));
}
constexpr int kLhCounterInts = (kLhBatch * 8 + 16) / 4;  // keys + ticket (+ padding)
constexpr int kLhPoolTicket = kLhBatch * 2 + 2;  // int index of the block pool's ticket

template <typename T>
__global__ __launch_bounds__(64 * kLhWaves) void lm_head_argmax_mfma_kernel(LhArgs a) {
  typedef Mfma32<T> Ops;
  typedef typename Ops::v8 v8;
  constexpr int ROW_B = kLhKc * (int)sizeof(T);  // bytes per row per tile
  constexpr int KS = kLhKHalf / 16;               // MFMA k-steps per wave per tile
  constexpr int CPR = ROW_B / 16;
  constexpr int RPI = 64 / CPR;                   // rows per 1 KB DMA instruction
  constexpr int NIW_W = kLhRows / (RPI * kLhWaves);
  constexpr int NIW_H = kLhBatch / (RPI * kLhWaves);
  constexpr int W_B = kLhRows * ROW_B;
  constexpr int H_B = kLhBatch * ROW_B;
  constexpr int XCH = kLhRowWaves * 16 * 64;      // floats per half-sum exchange buffer
  // Three-stage rings for the weight and hidden tiles, addressed by a
  // run-time stage (the DMA is issued as untracked assembly, so the compiler
  // does not order LDS reads after it: the loop's waits and barriers do).
  __shared__ __align__(16) char wring[kLhStages][W_B];
  __shared__ __align__(16) char hring[kLhStages][H_B];
  // Two exchange buffers (block parity) for the column halves' sums; the
  // final per-workgroup reduction reuses the one the last block left free.
  __shared__ __align__(16) float xch[2][XCH];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  const int rw = wave_s % kLhRowWaves;  // row group
  const int kh = wave_s / kLhRowWaves;  // column half of each tile
  // This workgroup's vocab rows [r_begin, r_end), in blocks of kLhRows.
  const int nwg = gridDim.x;
  // With a block pool, the first range is pool_begin / nwg whole blocks and
  // later ranges are single blocks drawn from the pool.
  const int sb = a.pool_ticket != nullptr ? a.pool_begin / kLhRows / nwg : 0;
  int rb_next = a.pool_ticket != nullptr ? static_cast<int>(blockIdx.x) * sb * kLhRows
                                         : static_cast<int>((int64_t)a.V * blockIdx.x / nwg);
  int re_next = a.pool_ticket != nullptr ? min(a.V, rb_next + sb * kLhRows)
                                         : static_cast<int>((int64_t)a.V * (blockIdx.x + 1) / nwg);
  const int n_tiles = (a.K + kLhKc - 1) / kLhKc;
  const T* wbase = static_cast<const T*>(a.weight);
  // Rows past the range (and hidden rows past B) are out of the descriptors'
  // range and land in LDS as zeros.
  const int hbytes = static_cast<int>(((int64_t)(a.B - 1) * a.hs + a.K) * sizeof(T));
  const PfLoadOffsets<NIW_W> woff = [&] {
    PfLoadOffsets<NIW_W> o;
#pragma unroll
    for (int u = 0; u < NIW_W; ++u) {
      const int row = (wave * NIW_W + u) * RPI + lane / CPR;
      const int ch = (lane % CPR) ^ lh_swz(row);
      o.o[u] = static_cast<int>(((int64_t)row * a.ws + ch * 8) * sizeof(T));
    }
    return o;
  }();
  const PfLoadOffsets<NIW_H> hoff = [&] {
    PfLoadOffsets<NIW_H> o;
#pragma unroll
    for (int u = 0; u < NIW_H; ++u) {
      const int row = (wave * NIW_H + u) * RPI + lane / CPR;
      const int ch = (lane % CPR) ^ lh_swz(row);
      // Rows past B get an offset of 2^31 bytes: beyond the descriptor's
      // range (< 2^31) with any tile offset added, so they load zeros, and
      // their row * stride is never formed (it may not fit 32 bits).
      o.o[u] = row < a.B ? static_cast<int>(((int64_t)row * a.hs + ch * 8) * sizeof(T))
                         : INT_MIN;
    }
    return o;
  }();
  // Operand reads: row l32 (of the wave's 32 vocab rows, or of the hidden
  // rows), 16-byte chunk kh*16 + hh*8 + s of the tile row at k-step s.
  int raddr[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s)
    raddr[s] = l32 * ROW_B + (((kh * (CPR / 2) + hh * (CPR / 4) + s) ^ lh_swz(l32)) << 4);
  const int wrow0 = rw * 32 * ROW_B;

  // Tile ft of block fb into ring stage st.
  auto fetch = [&](int fb, int ft, int st, int r_begin, int r_end) __attribute__((always_inline)) {
    const int row0 = r_begin + fb * kLhRows;
    const int valid = min(kLhRows, r_end - row0);
    const int wbytes = static_cast<int>(((int64_t)(valid - 1) * a.ws + a.K) * sizeof(T));
    pf_dma_tile_untracked<NIW_W, RPI, ROW_B, kLhWeightNt>(
        wbase + (int64_t)row0 * a.ws, wbytes, (LC_LDS char*)wring[st], wave_s, woff, ft * ROW_B);
    pf_dma_tile_untracked<NIW_H, RPI, ROW_B, false>(a.hidden, hbytes, (LC_LDS char*)hring[st],
                                                    wave_s, hoff, ft * ROW_B);
  };

  f32x16_t acc[2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
  auto compute = [&](int st) __attribute__((always_inline)) {
    LC_LDS const char* wl = (LC_LDS const char*)wring[st] + wrow0;
    LC_LDS const char* hl = (LC_LDS const char*)hring[st];
#pragma unroll
    for (int s = 0; s < KS; ++s)
      acc[s & 1] = Ops::mma(*reinterpret_cast<LC_LDS const v8*>(wl + raddr[s]),
                            *reinterpret_cast<LC_LDS const v8*>(hl + raddr[s]), acc[s & 1]);
  };

  // At a block's end the second column half stores its sums in xch[block & 1]
  // and the first half keeps its own in `keep`; after the next barrier the
  // first half adds them up, rounds, and folds them into the lane's running
  // best (batch row l32; the lane's vocab rows 8j + 4hh + i of its row group)
  // as a packed key (lh_pack; 0 = none yet). Branch-free.
  float keep[16];
  unsigned long long best = 0;
  auto block_epilogue = [&](int blk, int r_begin, int r_end) __attribute__((always_inline)) {
    if (kh == 0) {
      const int row0 = r_begin + blk * kLhRows;
      const int valid = min(kLhRows, r_end - row0);
      const float* other = xch[blk & 1] + rw * 16 * 64 + lane;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = rw * 32 + (r >> 2) * 8 + hh * 4 + (r & 3);
        const float x = lc_to_f32(lc_from_f32<T>(keep[r] + other[r * 64]));
        const unsigned long long k = lh_pack(x, row0 + row);
        best = lh_max_key(best, row < valid ? k : 0ull);
      }
    }
  };
  auto block_end = [&](int blk) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[0][r] += acc[1][r];
    if (kh == 1) {
      float* mine = xch[blk & 1] + rw * 16 * 64 + lane;
#pragma unroll
      for (int r = 0; r < 16; ++r) mine[r * 64] = acc[0][r];
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) keep[r] = acc[0][r];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
  };

  // Tile g = blk * n_tiles + t: wait for tile g (this wave's DMA; tile g+1
  // may still be in flight), barrier (every wave's part of tile g landed,
  // every wave done with tile g-1, the previous block's half sums stored),
  // finish the previous block at its first tile, refill tile g-1's stage with
  // tile g+2, compute tile g.
  static_assert(kLhStages == 3, "the loop below is written for a three-stage ring");
  // K a multiple of 128: with an odd number of half tiles each block's last
  // tile's second half is past K, and its waves skip that tile's products.
  const bool skip_last = kh == 1 && (a.K % kLhKc) != 0;
  constexpr int kNi = NIW_W + NIW_H;  // DMA instructions per wave per tile
  // Ranges of rows, one after another: the workgroup's own range, then (with
  // a block pool) one block at a time drawn from the pool until it is empty.
  // Every workgroup draws once per pool block it takes plus one final draw,
  // so the draws number pool_blocks + nwg and the last one returns the ticket
  // to zero. The running best carries over from range to range.
  int last_nb = 0;
  for (;;) {
    const int r_begin = __builtin_amdgcn_readfirstlane(rb_next);
    const int r_end = __builtin_amdgcn_readfirstlane(re_next);
    const int nb = (r_end - r_begin + kLhRows - 1) / kLhRows;
    const int G = nb * n_tiles;  // tiles of the range
    if (G > 0) fetch(0, 0, 0, r_begin, r_end);
    if (G > 1) fetch(n_tiles > 1 ? 0 : 1, n_tiles > 1 ? 1 : 0, 1, r_begin, r_end);
    int fb = n_tiles > 2 ? 0 : (n_tiles == 2 ? 1 : 2);  // tile 2 of the range
    int ft = n_tiles > 2 ? 2 : 0;
    int st = 0;
    int g = 0;
    for (int blk = 0; blk < nb; ++blk) {
      for (int t = 0; t < n_tiles; ++t, ++g) {
        if (g + 1 < G)
          __builtin_amdgcn_s_waitcnt(lh_waitcnt(kNi, 0));
        else
          __builtin_amdgcn_s_waitcnt(lh_waitcnt(0, 0));
        lc_compiler_fence();
        __builtin_amdgcn_s_barrier();
        lc_compiler_fence();
        if (t == 0 && blk > 0) block_epilogue(blk - 1, r_begin, r_end);
        if (g + 2 < G) {
          fetch(fb, ft, st == 0 ? 2 : st - 1, r_begin, r_end);
          if (++ft == n_tiles) {
            ft = 0;
            ++fb;
          }
        }
        if (!(skip_last && t == n_tiles - 1)) compute(st);
        st = st == 2 ? 0 : st + 1;
      }
      block_end(blk);
    }
    __syncthreads();  // the last block's second-half sums are in LDS
    if (nb > 0) block_epilogue(nb - 1, r_begin, r_end);
    last_nb = nb;
    if (a.pool_ticket == nullptr) break;
    // The draw goes through the exchange buffer this range's last block left
    // free (the next range writes it only after its first block's barriers).
    int* s_draw = reinterpret_cast<int*>(xch[nb & 1]) + (XCH - 1);
    if (tid == 0) {
      const int t = __hip_atomic_fetch_add(a.pool_ticket, 1, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
      if (t == a.pool_blocks + nwg - 1)
        __hip_atomic_store(a.pool_ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *s_draw = t;
    }
    __syncthreads();
    const int t = __builtin_amdgcn_readfirstlane(*s_draw);
    __syncthreads();
    if (t >= a.pool_blocks) break;
    rb_next = a.pool_begin + t * kLhRows;
    re_next = min(a.V, rb_next + kLhRows);
  }
  // Workgroup best per batch row: the two lane halves, then the row groups
  // through the exchange buffer the last block did not use (xch[last_nb & 1],
  // free since the last barrier).
  unsigned long long* red = reinterpret_cast<unsigned long long*>(xch[last_nb & 1]);
  if (kh == 0) {
    const uint32_t lo = static_cast<uint32_t>(best), hi = static_cast<uint32_t>(best >> 32);
    best = lh_max_key(best, (static_cast<unsigned long long>(__shfl_xor(hi, 32, 64)) << 32) |
                                __shfl_xor(lo, 32, 64));
    if (hh == 0) red[rw * 32 + l32] = best;
  }
  __syncthreads();
  if (wave == 0 && hh == 0) {
#pragma unroll
    for (int w = 1; w < kLhRowWaves; ++w) best = lh_max_key(best, red[w * 32 + l32]);
  }
  if (a.keys == nullptr) {
    if (wave == 0 && hh == 0 && l32 < a.B) {
      a.part_val[(int64_t)blockIdx.x * a.pstride + l32] = lh_unpack_value(best);
      a.part_idx[(int64_t)blockIdx.x * a.pstride + l32] = lh_unpack_index(best);
    }
    return;
  }
  // Merge into the packed keys; the workgroup that draws the last ticket
  // (after every other workgroup's merges have been performed: returning
  // atomics, waited for before the ticket) reads the keys back, resetting
  // them, writes the ids, and returns the ticket to zero.
  int& s_last = reinterpret_cast<int*>(red)[256];
  if (wave == 0 && hh == 0 && l32 < a.B) {
    const unsigned long long old = __hip_atomic_fetch_max(
        a.keys + l32, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    (void)old;
  }
  __builtin_amdgcn_s_waitcnt(lh_waitcnt(0, 0));
  __syncthreads();
  if (tid == 0) {
    unsigned* ticket = reinterpret_cast<unsigned*>(a.keys + kLhBatch);
    const unsigned t = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
    s_last = t == static_cast<unsigned>(nwg - 1);
  }
  __syncthreads();
  if (!s_last) return;
  if (wave == 0 && hh == 0) {
    const unsigned long long k =
        __hip_atomic_exchange(a.keys + l32, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (l32 < a.B) {
      a.ids[l32] = lh_unpack_index(k);
      if (a.max_out != nullptr) a.max_out[l32] = lh_unpack_value(k);
    }
  }
  if (tid == 0)
    __hip_atomic_store(reinterpret_cast<unsigned*>(a.keys + kLhBatch), 0u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// One lane per vocab row; the hidden rows are read through the cache.
template <typename T>
__global__ __launch_bounds__(kLhGenRows) void lm_head_argmax_generic_kernel(LhArgs a) {
  __shared__ float red_v[kLhGenRows / 64];
  __shared__ int red_i[kLhGenRows / 64];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int v = blockIdx.x * kLhGenRows + tid;
  const bool ok = v < a.V;
  const T* wrow = static_cast<const T*>(a.weight) + (int64_t)(ok ? v : 0) * a.ws;
  for (int b = 0; b < a.B; ++b) {
    const T* hrow = static_cast<const T*>(a.hidden) + (int64_t)b * a.hs;
    float acc = 0.f;
    if (ok)
      for (int k = 0; k < a.K; ++k) acc = fmaf(lc_to_f32(wrow[k]), lc_to_f32(hrow[k]), acc);
    float bv = ok ? lc_to_f32(lc_from_f32<T>(acc)) : -INFINITY;
    int bi = ok ? v : INT_MAX;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) lh_take(bv, bi, __shfl_xor(bv, o, 64), __shfl_xor(bi, o, 64));
    __syncthreads();  // red_* of the previous row has been read
    if (lane == 0) {
      red_v[wave] = bv;
      red_i[wave] = bi;
    }
    __syncthreads();
    if (tid == 0) {
      for (int w = 1; w < kLhGenRows / 64; ++w) lh_take(bv, bi, red_v[w], red_i[w]);
      a.part_val[(int64_t)blockIdx.x * a.pstride + b] = bv;
      a.part_idx[(int64_t)blockIdx.x * a.pstride + b] = bi;
    }
  }
}

// One workgroup per batch row; thread p takes partials p, p + 1024, ... (one
// load each at the Llama-3 vocab: the reduction is latency-bound, so all of a
// row's partials are fetched in one round), then a wave and a workgroup
// reduction.
__global__ __launch_bounds__(1024) void lm_head_argmax_reduce_kernel(const float* __restrict__ pv,
                                                                     const int* __restrict__ pi,
                                                                     int n_part, int pstride,
                                                                     int64_t* __restrict__ ids,
                                                                     float* __restrict__ max_out) {
  __shared__ float red_v[16];
  __shared__ int red_i[16];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  float bv = -INFINITY;
  int bi = INT_MAX;
  for (int p = tid; p < n_part; p += 1024)
    lh_take(bv, bi, pv[(int64_t)p * pstride + b], pi[(int64_t)p * pstride + b]);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) lh_take(bv, bi, __shfl_xor(bv, o, 64), __shfl_xor(bi, o, 64));
  if ((tid & 63) == 0) {
    red_v[tid >> 6] = bv;
    red_i[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 16; ++w) lh_take(bv, bi, red_v[w], red_i[w]);
    ids[b] = bi;
    if (max_out != nullptr) max_out[b] = bv;
  }
}

template <typename T>
int run_lm_head_mfma(LhArgs a, int64_t* ids, float* max_out, hipStream_t st);

template <typename T>
int run_lm_head(LhArgs a, bool mfma, int64_t* ids, float* max_out, hipStream_t st) {
  if constexpr (!std::is_same<T, float>::value) {
    if (mfma) return run_lm_head_mfma<T>(a, ids, max_out, st);
  }
  {
    const int n_wg = (a.V + kLhGenRows - 1) / kLhGenRows;
    a.pstride = a.B;
    lm_head_argmax_generic_kernel<T><<<n_wg, kLhGenRows, 0, st>>>(a);
    lm_head_argmax_reduce_kernel<<<a.B, 1024, 0, st>>>(a.part_val, a.part_idx, n_wg, a.pstride,
                                                        ids, max_out);
  }
  return lc_check_launch("lc_lm_head_argmax");
}

template <typename T>
int run_lm_head_mfma(LhArgs a, int64_t* ids, float* max_out, hipStream_t st) {
  // One workgroup per CU (its 160 KiB of LDS), each over V / grid rows.
  const int n_wg = static_cast<int>(std::min<int64_t>((a.V + kLhRows - 1) / kLhRows,
                                                      lc_cu_count()));
  const T* hidden = static_cast<const T*>(a.hidden);
  const int B = a.B;
  a.pstride = kLhBatch;
  // Block pool (fused selection only, it needs the counters): each workgroup
  // first takes k whole 64-row blocks, k leaving at least half a block per
  // workgroup to the pool; the rest go to whichever workgroups finish first
  // (the XCDs stream at different rates). At the Llama-3-8B vocab (2004
  // blocks, 256 workgroups) k = 7: 152.8-153.0 us against 164.7-165.0 us for
  // contiguous ranges in an A/B on one box (k = 6 153-154, 5 157-158, 4 161).
  a.pool_ticket = nullptr;
  {
    const int nblk = static_cast<int>((a.V + kLhRows - 1) / kLhRows);
    const int k = (nblk - n_wg / 2) / n_wg;
    if (a.keys != nullptr && k >= 1 && k * n_wg < nblk) {
      a.pool_ticket = reinterpret_cast<int*>(a.keys) + kLhPoolTicket;
      a.pool_begin = k * n_wg * kLhRows;
      a.pool_blocks = nblk - k * n_wg;
    }
  }
  for (int b0 = 0; b0 < B; b0 += kLhBatch) {
    a.hidden = hidden + (int64_t)b0 * a.hs;
    a.B = min(kLhBatch, B - b0);
    a.ids = ids + b0;
    a.max_out = max_out ? max_out + b0 : nullptr;
    lm_head_argmax_mfma_kernel<T><<<n_wg, 64 * kLhWaves, 0, st>>>(a);
    if (a.keys == nullptr)
      lm_head_argmax_reduce_kernel<<<a.B, 1024, 0, st>>>(a.part_val, a.part_idx, n_wg, a.pstride,
                                                          a.ids, a.max_out);
  }
  return lc_check_launch("lc_lm_head_argmax");
}

}  // namespace

extern "C" {

int64_t lc_lm_head_argmax_counter_count() { return kLhCounterInts; }

int64_t lc_lm_head_argmax_workspace_bytes(int64_t B, int64_t V) {
  if (B < 0 || V < 0) return -1;
  const int64_t parts = (V + kLhRows - 1) / kLhRows;
  const int64_t cols = B > kLhBatch ? B : kLhBatch;
  return (parts * cols * 8 + 255) / 256 * 256;
}

int lc_lm_head_argmax(const void* hidden, int64_t hidden_row_stride, const void* weight,
                      int64_t weight_row_stride, int64_t B, int64_t K, int64_t V, int64_t* ids,
                      float* max_logit, void* workspace, int64_t workspace_bytes,
                      int32_t* counters, int dtype, void* stream) {
  if (B == 0) return LC_OK;  // no rows (pointers may be null)
  LC_REQUIRE(hidden && weight && ids && workspace, "lc_lm_head_argmax: null pointer");
  LC_REQUIRE(B >= 0 && B < 65536, "lc_lm_head_argmax: batch %lld out of range", (long long)B);
  LC_REQUIRE(K > 0 && V > 0 && V < (1LL << 31) - kLhGenRows && K < (1LL << 30),
             "lc_lm_head_argmax: bad sizes K=%lld V=%lld", (long long)K, (long long)V);
  LC_REQUIRE(hidden_row_stride >= K && weight_row_stride >= K,
             "lc_lm_head_argmax: row strides must be >= K");
  const int64_t need = lc_lm_head_argmax_workspace_bytes(B, V);
  LC_REQUIRE(workspace_bytes >= need, "lc_lm_head_argmax: workspace %lld < %lld bytes",
             (long long)workspace_bytes, (long long)need);
  LC_REQUIRE(lc_aligned(workspace, 16), "lc_lm_head_argmax: workspace not 16-byte aligned");
  LC_REQUIRE(counters == nullptr || lc_aligned(counters, 8),
             "lc_lm_head_argmax: counters not 8-byte aligned");
  if (B == 0) return LC_OK;
  const int64_t parts = (V + kLhRows - 1) / kLhRows;
  LhArgs a{};
  a.hidden = hidden;
  a.weight = weight;
  a.part_val = static_cast<float*>(workspace);
  a.part_idx = reinterpret_cast<int*>(static_cast<char*>(workspace) +
                                      parts * (B > kLhBatch ? B : kLhBatch) * 4);
  // The fused argmax (packed keys + ticket) runs on the MFMA path only; the
  // generic kernel always hands partials to the reduce kernel.
  a.keys = reinterpret_cast<unsigned long long*>(counters);
  a.hs = hidden_row_stride;
  a.ws = weight_row_stride;
  a.B = (int)B;
  a.K = (int)K;
  a.V = (int)V;
  const int64_t esz = lc_dtype_size(dtype);
  const bool mfma = (dtype == LC_DTYPE_BF16 || dtype == LC_DTYPE_F16) && K % kLhKHalf == 0 &&
                    lc_aligned(hidden, 16) && lc_aligned(weight, 16) &&
                    hidden_row_stride % 8 == 0 && weight_row_stride % 8 == 0 &&
                    ((int64_t)kLhRows * weight_row_stride) * esz < (1LL << 31) &&
                    ((int64_t)(std::min<int64_t>(B, kLhBatch) - 1) * hidden_row_stride + K) *
                            esz < (1LL << 31);
  hipStream_t st = lc_stream(stream);
  switch (dtype) {
    case LC_DTYPE_F32:
      return run_lm_head<float>(a, false, ids, max_logit, st);
    case LC_DTYPE_BF16:
      return run_lm_head<bf16_t>(a, mfma, ids, max_logit, st);
    case LC_DTYPE_F16:
      return run_lm_head<f16_t>(a, mfma, ids, max_logit, st);
    default:
      return lc_fail(LC_EINVAL, "lc_lm_head_argmax: unknown dtype %d", dtype);
  }
}

}  // extern "C"
