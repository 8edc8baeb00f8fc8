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
//     per launch): a workgroup owns 64 vocab rows and streams their weight rows
//     through LDS in 256-column tiles (buffer-to-LDS DMA, 512-byte runs per
//     row, a three-stage ring with two tiles in flight), together with the
//     matching 256 columns of the hidden rows. Its 4 waves are 2 row groups x
//     2 column halves; each computes
//     logits^T[32 vocab x 32 batch] += W[32 x 16] hidden^T[16 x 32] on
//     v_mfma_f32_32x32x16 over its half, the halves are added through LDS, and
//     the epilogue rounds, takes each batch row's best (value, index) over the
//     workgroup's 64 rows and writes it as a partial.
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
  int64_t hs, ws;  // row strides (elements)
  int B, K, V, pstride;
};

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
  __shared__ __align__(16) char w0[W_B];
  __shared__ __align__(16) char w1[W_B];
  __shared__ __align__(16) char w2[W_B];
  __shared__ __align__(16) char h0[H_B];
  __shared__ __align__(16) char h1[H_B];
  __shared__ __align__(16) char h2[H_B];
  __shared__ float red_v[kLhRowWaves][32];
  __shared__ int red_i[kLhRowWaves][32];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  const int rw = wave_s % kLhRowWaves;  // row group
  const int kh = wave_s / kLhRowWaves;  // column half of each tile
  const int v0 = blockIdx.x * kLhRows;
  const int rows_valid = min(kLhRows, a.V - v0);
  const T* wbase = static_cast<const T*>(a.weight) + (int64_t)v0 * a.ws;
  // Rows past the vocabulary (and hidden rows past B) are out of the
  // descriptors' range and land in LDS as zeros.
  const int wbytes = static_cast<int>(((int64_t)(rows_valid - 1) * a.ws + a.K) * sizeof(T));
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

  auto wbuf = [&](auto st_c) __attribute__((always_inline)) -> LC_LDS char* {
    constexpr int S = decltype(st_c)::value;
    if constexpr (S == 0) return (LC_LDS char*)w0;
    else if constexpr (S == 1) return (LC_LDS char*)w1;
    else return (LC_LDS char*)w2;
  };
  auto hbuf = [&](auto st_c) __attribute__((always_inline)) -> LC_LDS char* {
    constexpr int S = decltype(st_c)::value;
    if constexpr (S == 0) return (LC_LDS char*)h0;
    else if constexpr (S == 1) return (LC_LDS char*)h1;
    else return (LC_LDS char*)h2;
  };
  auto fetch = [&](int t, auto st_c) __attribute__((always_inline)) {
    pf_dma_tile_untracked<NIW_W, RPI, ROW_B, kLhWeightNt>(wbase, wbytes, wbuf(st_c), wave_s, woff,
                                                   t * ROW_B);
    pf_dma_tile_untracked<NIW_H, RPI, ROW_B, false>(a.hidden, hbytes, hbuf(st_c), wave_s, hoff,
                                                    t * ROW_B);
  };

  f32x16_t acc[2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
  auto compute = [&](auto st_c) __attribute__((always_inline)) {
    LC_LDS const char* wl = wbuf(st_c) + wrow0;
    LC_LDS const char* hl = hbuf(st_c);
#pragma unroll
    for (int s = 0; s < KS; ++s)
      acc[s & 1] = Ops::mma(*reinterpret_cast<LC_LDS const v8*>(wl + raddr[s]),
                            *reinterpret_cast<LC_LDS const v8*>(hl + raddr[s]), acc[s & 1]);
  };

  // Iteration t: wait for tile t (this wave's DMA; tile t+1 may still be in
  // flight), barrier (every wave's part of tile t landed, every wave done with
  // tile t-1), refill tile t-1's stage with tile t+2, compute tile t.
  static_assert(kLhStages == 3, "the loop below is written for a three-stage ring");
  // K a multiple of 128: with an odd number of half tiles the last tile's
  // second half is past K, and its waves skip that tile's products.
  const int n_tiles = (a.K + kLhKc - 1) / kLhKc;
  const bool skip_last = kh == 1 && (a.K % kLhKc) != 0;
  constexpr int kNi = NIW_W + NIW_H;  // DMA instructions per wave per tile
  auto iteration = [&](int t, auto st_c) __attribute__((always_inline)) {
    constexpr int S = decltype(st_c)::value;
    if (t + 1 < n_tiles)
      __builtin_amdgcn_s_waitcnt(lh_waitcnt(kNi, 0));
    else
      __builtin_amdgcn_s_waitcnt(lh_waitcnt(0, 0));
    lc_compiler_fence();
    __builtin_amdgcn_s_barrier();
    lc_compiler_fence();
    if (t + 2 < n_tiles) fetch(t + 2, std::integral_constant<int, (S + 2) % 3>{});
    if (!(skip_last && t + 1 == n_tiles)) compute(st_c);
  };

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  fetch(0, I0{});
  if (n_tiles > 1) fetch(1, I1{});
  for (int t = 0; t < n_tiles; t += 3) {
    iteration(t, I0{});
    if (t + 1 < n_tiles) iteration(t + 1, I1{});
    if (t + 2 < n_tiles) iteration(t + 2, I2{});
  }

  // The second column half hands its sums to the first through LDS (the W
  // ring is free after the barrier), added in a fixed order.
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[0][r] += acc[1][r];
  __syncthreads();
  float* half = reinterpret_cast<float*>(w0);
  if (kh == 1) {
#pragma unroll
    for (int r = 0; r < 16; ++r) half[(rw * 16 + r) * 64 + lane] = acc[0][r];
  }
  __syncthreads();
  // Epilogue (first-half waves): lane (l32, hh) holds batch row l32 and vocab
  // rows v0 + rw*32 + 8j + 4hh + i for register 4j + i.
  float bv = -INFINITY;
  int bi = INT_MAX;
  if (kh == 0) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = rw * 32 + (r >> 2) * 8 + hh * 4 + (r & 3);
      const float x = lc_to_f32(lc_from_f32<T>(acc[0][r] + half[(rw * 16 + r) * 64 + lane]));
      if (row < rows_valid) lh_take(bv, bi, x, v0 + row);
    }
    lh_take(bv, bi, __shfl_xor(bv, 32, 64), __shfl_xor(bi, 32, 64));
    if (hh == 0) {
      red_v[rw][l32] = bv;
      red_i[rw][l32] = bi;
    }
  }
  __syncthreads();
  if (wave == 0 && hh == 0) {
#pragma unroll
    for (int w = 1; w < kLhRowWaves; ++w) lh_take(bv, bi, red_v[w][l32], red_i[w][l32]);
    if (l32 < a.B) {
      a.part_val[(int64_t)blockIdx.x * a.pstride + l32] = bv;
      a.part_idx[(int64_t)blockIdx.x * a.pstride + l32] = bi;
    }
  }
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
  {
    const int n_wg = (a.V + kLhRows - 1) / kLhRows;
    const T* hidden = static_cast<const T*>(a.hidden);
    const int B = a.B;
    a.pstride = kLhBatch;
    for (int b0 = 0; b0 < B; b0 += kLhBatch) {
      a.hidden = hidden + (int64_t)b0 * a.hs;
      a.B = min(kLhBatch, B - b0);
      lm_head_argmax_mfma_kernel<T><<<n_wg, 64 * kLhWaves, 0, st>>>(a);
      lm_head_argmax_reduce_kernel<<<a.B, 1024, 0, st>>>(a.part_val, a.part_idx, n_wg, a.pstride,
                                                          ids + b0,
                                                          max_out ? max_out + b0 : nullptr);
    }
  }
  return lc_check_launch("lc_lm_head_argmax");
}

}  // namespace

extern "C" {

int64_t lc_lm_head_argmax_workspace_bytes(int64_t B, int64_t V) {
  if (B < 0 || V < 0) return -1;
  const int64_t parts = (V + kLhRows - 1) / kLhRows;
  const int64_t cols = B > kLhBatch ? B : kLhBatch;
  return (parts * cols * 8 + 255) / 256 * 256;
}

int lc_lm_head_argmax(const void* hidden, int64_t hidden_row_stride, const void* weight,
                      int64_t weight_row_stride, int64_t B, int64_t K, int64_t V, int64_t* ids,
                      float* max_logit, void* workspace, int64_t workspace_bytes, int dtype,
                      void* stream) {
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
  if (B == 0) return LC_OK;
  const int64_t parts = (V + kLhRows - 1) / kLhRows;
  LhArgs a{};
  a.hidden = hidden;
  a.weight = weight;
  a.part_val = static_cast<float*>(workspace);
  a.part_idx = reinterpret_cast<int*>(static_cast<char*>(workspace) +
                                      parts * (B > kLhBatch ? B : kLhBatch) * 4);
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
