// Projection of a few rows (the decode step's batch) by a weight matrix that
// is streamed once from HBM:
//   mode 0 (plain):  y[m, n] = round(sum_k x[m, k] w[n, k])              n < N
//   mode 1 (SwiGLU): y[m, n] = round(silu(g) u),  g = round(x[m] . w[n]),
//                    u = round(x[m] . w[N + n])                          n < N
// for M <= 32 rows, w row-major [N or 2N, K] (nn.Linear's weight layout),
// fp32 accumulation, round() to the data type. Mode 0 is F.linear(x, w)
// (models/llama3/attention.py:100-102,154 and mlp.py:35-37 of the reference);
// mode 1 is down_proj's input swiglu(gate_proj(x), up_proj(x)) (mlp.py:39-43,
// kernels/triton/swiglu.py:15-42) over the concatenated [gate; up] weight,
// with the same roundings: g and u are rounded as the two projections'
// outputs before the SwiGLU, which is computed in fp32.
//
// Kernel: a workgroup of 4 waves owns 128 weight rows (mode 1: 64 gate rows
// and the 64 matching up rows) and streams them through LDS in 128-column
// tiles (buffer-to-LDS DMA, 256-byte runs per row, non-temporal, a
// three-stage ring with two tiles in flight), with the matching columns of the
// x rows. Each wave computes y^T[32 weight rows x 32 x rows] on
// v_mfma_f32_32x32x16. HBM-bound: the weight is read once; x (<= 256 KiB at
// K 4096) is re-read from L2 by every workgroup.
//
// Split-K: with few row blocks (N = 4096 gives 32) the K tiles are divided
// over grid.y splits so that the grid fills the CUs. Each split writes its
// fp32 partial to the workspace; a per-row-block ticket picks the last split
// to arrive, which sums the partials in split order (the result does not
// depend on which split came last), runs the epilogue and returns the ticket
// counter to zero. No second launch.
#include <limits.h>
#include <algorithm>
#include <math.h>

#include <type_traits>

#include "attn_tiles.h"
#include "lc_common.h"

namespace {

using namespace lc_attn;

// (Two-wave workgroups for mode 1 -- 448 row blocks of 32 columns, two per
// CU, instead of 224 blocks on 256 CUs -- measured slower.)
constexpr int kDlWaves = 4;
constexpr int kDlRows = 32 * kDlWaves;  // weight rows per workgroup
constexpr int kDlKc = 128;              // K columns per tile (256-byte runs per row)
constexpr int kDlBatch = 32;            // x rows per launch (the MFMA's N)
constexpr int kDlPartFloats = kDlRows * kDlBatch;  // fp32 partial of one split (16 per thread)
// Output columns per row block.
constexpr int dl_out_cols(int mode) { return mode == 1 ? kDlRows / 2 : kDlRows; }
constexpr int kDlWeightAux = 2;         // non-temporal weight loads (read once)
constexpr int kDlMaxBlocks = 1 << 16;   // row blocks per launch (ticket counters)
constexpr int kDlMaxSplits = 16;        // K-splits per launch
constexpr int kDlCoherent = 16;         // buffer cache policy sc1: agent-coherent access

__device__ __forceinline__ float dl_silu_mul(float g, float u) {
  const float e = lc_exp2(-g * kLog2e);
  const float sig = 1.0f / (1.0f + e);
  return (g * sig) * u;
}

// s_waitcnt immediate: vmcnt(vm) lgkmcnt(lgkm), expcnt not waited on.
constexpr int dl_waitcnt(int vm, int lgkm) {
  return (vm & 0xF) | ((vm >> 4) << 14) | (7 << 4) | (lgkm << 8);
}

struct DlArgs {
  const void* x;
  const void* w;
  void* y;
  float* part;    // [n_blocks][splits][kDlPartFloats]
  int* counters;  // [n_blocks], zero between calls
  int64_t xs, ws, ys;  // row strides (elements)
  int M, K, N;         // N = output columns
  int tiles_per_split, splits;
};

template <typename T, int MODE>
__global__ __launch_bounds__(64 * kDlWaves) void decode_linear_kernel(DlArgs a) {
  typedef Mfma32<T> Ops;
  typedef typename Ops::v8 v8;
  constexpr int ROW_B = kDlKc * (int)sizeof(T);
  constexpr int KS = kDlKc / 16;
  constexpr int CPR = ROW_B / 16;
  constexpr int RPI = 64 / CPR;
  constexpr int NIW_W = kDlRows / (RPI * kDlWaves);
  constexpr int NIW_H = kDlBatch / (RPI * kDlWaves);
  constexpr int W_B = kDlRows * ROW_B;
  constexpr int H_B = kDlBatch * ROW_B;
  constexpr int OUT_COLS = dl_out_cols(MODE);  // output columns per block
  __shared__ __align__(16) char w0[W_B];
  __shared__ __align__(16) char w1[W_B];
  __shared__ __align__(16) char w2[W_B];
  __shared__ __align__(16) char h0[H_B];
  __shared__ __align__(16) char h1[H_B];
  __shared__ __align__(16) char h2[H_B];
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  const int blk = blockIdx.x;
  const int split = blockIdx.y;
  const int c0 = blk * OUT_COLS;  // first output column of the block
  const int cols_valid = min(OUT_COLS, a.N - c0);
  const int t_begin = split * a.tiles_per_split;
  const int n_tiles = min(a.tiles_per_split, a.K / kDlKc - t_begin);

  // Weight rows of the block: mode 0 rows c0 .. c0 + 127; mode 1 gate rows
  // c0 .. c0 + 63 (block rows 0-63) and up rows N + c0 .. (block rows 64-127).
  // Offsets are taken from row c0. Rows past the matrix are past the
  // descriptor's range and land in LDS as zeros; gate rows past N read up
  // rows (their outputs are not stored).
  const T* wbase = static_cast<const T*>(a.w) + (int64_t)c0 * a.ws + (int64_t)t_begin * kDlKc;
  const int64_t last_row = MODE == 1 ? (int64_t)a.N + cols_valid - 1 : (int64_t)cols_valid - 1;
  const int wbytes = static_cast<int>((last_row * a.ws + (int64_t)(a.K - t_begin * kDlKc)) * sizeof(T));
  const T* xbase = static_cast<const T*>(a.x) + (int64_t)t_begin * kDlKc;
  const int xbytes = static_cast<int>(((int64_t)(a.M - 1) * a.xs + (a.K - t_begin * kDlKc)) * sizeof(T));
  const PfLoadOffsets<NIW_W> woff = [&] {
    PfLoadOffsets<NIW_W> o;
#pragma unroll
    for (int u = 0; u < NIW_W; ++u) {
      const int row = (wave * NIW_W + u) * RPI + lane / CPR;
      const int ch = (lane % CPR) ^ pf_swz<CPR>(row);
      const int64_t wrow = MODE == 1 && row >= kDlRows / 2 ? (int64_t)a.N + row - kDlRows / 2 : row;
      o.o[u] = static_cast<int>((wrow * a.ws + ch * 8) * sizeof(T));
    }
    return o;
  }();
  const PfLoadOffsets<NIW_H> hoff = [&] {
    PfLoadOffsets<NIW_H> o;
#pragma unroll
    for (int u = 0; u < NIW_H; ++u) {
      const int row = (wave * NIW_H + u) * RPI + lane / CPR;
      const int ch = (lane % CPR) ^ pf_swz<CPR>(row);
      // Rows past M: an offset past the descriptor's range (< 2^31) with any
      // tile offset added, so they load zeros.
      o.o[u] = row < a.M ? static_cast<int>(((int64_t)row * a.xs + ch * 8) * sizeof(T)) : INT_MIN;
    }
    return o;
  }();
  int raddr[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) raddr[s] = l32 * ROW_B + (((hh * (CPR / 2) + s) ^ pf_swz<CPR>(l32)) << 4);
  const int wrow0 = wave * 32 * ROW_B;

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
    pf_dma_tile<NIW_W, RPI, ROW_B, kDlWeightAux>(wbase, wbytes, wbuf(st_c), wave_s, woff, t * ROW_B);
    pf_dma_tile<NIW_H, RPI, ROW_B>(xbase, xbytes, hbuf(st_c), wave_s, hoff, t * ROW_B);
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
  constexpr int kNi = NIW_W + NIW_H;  // DMA instructions per wave per tile
  auto iteration = [&](int t, auto st_c) __attribute__((always_inline)) {
    constexpr int S = decltype(st_c)::value;
    if (t + 1 < n_tiles)
      __builtin_amdgcn_s_waitcnt(dl_waitcnt(kNi, 0));
    else
      __builtin_amdgcn_s_waitcnt(dl_waitcnt(0, 0));
    lc_compiler_fence();
    __builtin_amdgcn_s_barrier();
    lc_compiler_fence();
    if (t + 2 < n_tiles) fetch(t + 2, std::integral_constant<int, (S + 2) % 3>{});
    compute(st_c);
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
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[0][r] += acc[1][r];

  if (a.splits > 1) {
    // Partial of this split: register r of lane (wave, lane) at r*256 + tid,
    // so the reading workgroup's thread tid gets the same (row, x row) back.
    // The partials travel through stores and loads with the sc1 cache policy
    // (agent-coherent: performed past the per-XCD L2s, as agent-scope
    // atomics are), so no cache-wide write-back or invalidate is needed: each
    // lane waits for its stores to be acknowledged before the workgroup takes
    // its ticket. Thread tid's 16 values sit at [tid][16] (four 16-byte runs).
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
        a.part + (int64_t)blk * a.splits * kDlPartFloats, 0, a.splits * kDlPartFloats * 4,
        0x00020000);
    const int my_off = (split * kDlPartFloats + tid * 16) * 4;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x4_t v = {acc[0][4 * q], acc[0][4 * q + 1], acc[0][4 * q + 2], acc[0][4 * q + 3]};
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), prs, my_off + 16 * q, 0,
                                             kDlCoherent);
    }
    __builtin_amdgcn_s_waitcnt(dl_waitcnt(0, 0));
    __syncthreads();
    if (tid == 0) {
      const int ticket = __hip_atomic_fetch_add(a.counters + blk, 1, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
      s_last = ticket == a.splits - 1;
    }
    __syncthreads();
    if (!s_last) return;
    // Every split's loads are issued before the first is waited for (up to
    // kDlMaxSplits splits), then summed in split order.
    u32x4_t pv[kDlMaxSplits][4];
#pragma unroll
    for (int sp = 0; sp < kDlMaxSplits; ++sp)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (sp < a.splits)
          pv[sp][q] = __builtin_amdgcn_raw_buffer_load_b128(
              prs, (sp * kDlPartFloats + tid * 16) * 4 + 16 * q, 0, kDlCoherent);
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[0][r] = 0.f;
#pragma unroll
    for (int sp = 0; sp < kDlMaxSplits; ++sp)
      if (sp < a.splits) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4_t v = __builtin_bit_cast(f32x4_t, pv[sp][q]);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[0][4 * q + e] += v[e];
        }
      }
    if (tid == 0)
      __hip_atomic_store(a.counters + blk, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // Epilogue. Lane (l32, hh) of wave w holds x row l32 and block rows
  // w*32 + 8j + 4hh + i (register 4j + i).
  typedef T t4 __attribute__((ext_vector_type(4)));
  T* yrow = static_cast<T*>(a.y) + (int64_t)l32 * a.ys;
  if constexpr (MODE == 0) {
    if (l32 >= a.M) return;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = wave * 32 + j * 8 + hh * 4;
      t4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = lc_from_f32<T>(acc[0][j * 4 + i]);
      if (col + 4 <= cols_valid) {
        *reinterpret_cast<t4*>(yrow + c0 + col) = o;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (col + i < cols_valid) yrow[c0 + col + i] = o[i];
      }
    }
  } else {
    // The upper half of the waves holds the up rows of the columns the lower
    // half holds the gate rows of; the rounded up values go through LDS (the
    // W ring is free now).
    __syncthreads();
    float* ux = reinterpret_cast<float*>(w0);
    constexpr int HALF = kDlWaves / 2;
    if (wave >= HALF) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        ux[((wave - HALF) * 16 + r) * 64 + lane] = lc_to_f32(lc_from_f32<T>(acc[0][r]));
    }
    __syncthreads();
    if (wave >= HALF || l32 >= a.M) return;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = wave * 32 + j * 8 + hh * 4;
      t4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = j * 4 + i;
        const float g = lc_to_f32(lc_from_f32<T>(acc[0][r]));
        o[i] = lc_from_f32<T>(dl_silu_mul(g, ux[(wave * 16 + r) * 64 + lane]));
      }
      if (col + 4 <= cols_valid) {
        *reinterpret_cast<t4*>(yrow + c0 + col) = o;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (col + i < cols_valid) yrow[c0 + col + i] = o[i];
      }
    }
  }
}

// Split count: enough workgroups to cover the CUs once, at most one split per
// K tile. A request > 0 is honoured (clamped to the tile count).
int dl_splits(int n_blocks, int k_tiles, int requested, int n_cu) {
  int s = requested > 0 ? requested : std::max(1, n_cu / std::max(1, n_blocks));
  s = std::min(std::min(s, k_tiles), kDlMaxSplits);
  const int tps = (k_tiles + s - 1) / s;
  return (k_tiles + tps - 1) / tps;
}

int dl_n_cu() {
  static int cached = 0;
  if (cached == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cached = n;
    else
      cached = 256;
  }
  return cached;
}

}  // namespace

extern "C" {

int64_t lc_decode_linear_workspace_bytes(int64_t M, int64_t N, int64_t K, int mode, int splits) {
  if (M < 0 || N <= 0 || K <= 0 || (mode != 0 && mode != 1) || splits < 0) return -1;
  const int64_t out_cols = dl_out_cols(mode);
  const int64_t n_blocks = (N + out_cols - 1) / out_cols;
  if (n_blocks > kDlMaxBlocks) return -1;
  const int k_tiles = (int)std::max<int64_t>(1, K / kDlKc);
  const int s = dl_splits((int)n_blocks, k_tiles, splits, dl_n_cu());
  if (s <= 1) return 256;
  return (n_blocks * s * kDlPartFloats * 4 + 255) / 256 * 256;
}

int64_t lc_decode_linear_counter_count(int64_t N, int mode) {
  if (N <= 0 || (mode != 0 && mode != 1)) return -1;
  const int64_t out_cols = dl_out_cols(mode);
  return (N + out_cols - 1) / out_cols;
}

int lc_decode_linear(const void* x, int64_t x_row_stride, const void* weight,
                     int64_t weight_row_stride, void* y, int64_t y_row_stride, int64_t M,
                     int64_t N, int64_t K, int mode, int splits, void* workspace,
                     int64_t workspace_bytes, int* counters, int dtype, void* stream) {
  LC_REQUIRE(mode == 0 || mode == 1, "lc_decode_linear: mode %d is not 0 (plain) or 1 (swiglu)",
             mode);
  LC_REQUIRE(dtype == LC_DTYPE_BF16 || dtype == LC_DTYPE_F16,
             "lc_decode_linear: dtype %d (bf16 or f16 only)", dtype);
  LC_REQUIRE(M >= 0 && M <= kDlBatch, "lc_decode_linear: M=%lld rows (1..%d)", (long long)M,
             kDlBatch);
  if (M == 0) return LC_OK;
  LC_REQUIRE(x && weight && y && workspace && counters, "lc_decode_linear: null pointer");
  LC_REQUIRE(N > 0 && K > 0 && K % kDlKc == 0 && K < (1LL << 30) && N < (1LL << 30),
             "lc_decode_linear: N=%lld K=%lld (K must be a positive multiple of %d)",
             (long long)N, (long long)K, kDlKc);
  LC_REQUIRE(splits >= 0, "lc_decode_linear: splits %d < 0", splits);
  LC_REQUIRE(x_row_stride >= K && weight_row_stride >= K && y_row_stride >= N,
             "lc_decode_linear: row strides too small");
  LC_REQUIRE(lc_aligned(x, 16) && lc_aligned(weight, 16) && x_row_stride % 8 == 0 &&
                 weight_row_stride % 8 == 0,
             "lc_decode_linear: x and weight need 16-byte aligned rows");
  LC_REQUIRE(lc_aligned(y, 8) && y_row_stride % 4 == 0,
             "lc_decode_linear: y needs 8-byte aligned rows");
  LC_REQUIRE(lc_aligned(workspace, 16), "lc_decode_linear: workspace not 16-byte aligned");
  const int64_t esz = 2;
  const int64_t w_rows = mode == 1 ? 2 * N : N;
  LC_REQUIRE(w_rows * weight_row_stride * esz < (1LL << 31) &&
                 ((M - 1) * x_row_stride + K) * esz < (1LL << 31),
             "lc_decode_linear: weight or x spans 2 GiB or more");
  const int64_t out_cols = dl_out_cols(mode);
  const int64_t n_blocks = (N + out_cols - 1) / out_cols;
  LC_REQUIRE(n_blocks <= kDlMaxBlocks, "lc_decode_linear: N=%lld too large", (long long)N);
  const int k_tiles = (int)(K / kDlKc);
  const int s = dl_splits((int)n_blocks, k_tiles, splits, dl_n_cu());
  const int64_t need = lc_decode_linear_workspace_bytes(M, N, K, mode, splits);
  LC_REQUIRE(workspace_bytes >= need, "lc_decode_linear: workspace %lld < %lld bytes",
             (long long)workspace_bytes, (long long)need);
  DlArgs a{};
  a.x = x;
  a.w = weight;
  a.y = y;
  a.part = static_cast<float*>(workspace);
  a.counters = counters;
  a.xs = x_row_stride;
  a.ws = weight_row_stride;
  a.ys = y_row_stride;
  a.M = (int)M;
  a.K = (int)K;
  a.N = (int)N;
  a.tiles_per_split = (k_tiles + s - 1) / s;
  a.splits = s;
  hipStream_t st = lc_stream(stream);
  const dim3 grid((unsigned)n_blocks, (unsigned)s);
  if (dtype == LC_DTYPE_BF16) {
    if (mode == 0)
      decode_linear_kernel<bf16_t, 0><<<grid, 64 * kDlWaves, 0, st>>>(a);
    else
      decode_linear_kernel<bf16_t, 1><<<grid, 64 * kDlWaves, 0, st>>>(a);
  } else {
    if (mode == 0)
      decode_linear_kernel<f16_t, 0><<<grid, 64 * kDlWaves, 0, st>>>(a);
    else
      decode_linear_kernel<f16_t, 1><<<grid, 64 * kDlWaves, 0, st>>>(a);
  }
  return lc_check_launch("lc_decode_linear");
}

}  // extern "C"
