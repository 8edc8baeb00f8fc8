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
// Work: the weight is cut into row blocks of ROWS rows (mode 1: ROWS/2 gate
// rows and the ROWS/2 matching up rows) and each block into K tiles of
// 16384 / ROWS columns (32 KiB of weight per tile). The (block, tile) units,
// block-major, are dealt out in equal contiguous runs to the workgroups of a
// one-dimensional grid (stream-K): every workgroup streams the same number of
// tiles, whatever the block count, so a grid of one workgroup per CU finishes
// together.
//
// Kernel: 4 waves. ROWS = 128: wave w owns block rows 32w .. 32w + 31 over a
// 128-column tile (256-byte runs per row). ROWS = 64 (K % 256 == 0): wave w
// owns rows 32 (w % 2) .. + 31 over columns 128 (w / 2) .. + 127 of a
// 256-column tile (512-byte runs per row), and the two column halves are
// added through LDS when a block's run ends. Tiles stream through LDS
// (buffer-to-LDS DMA, non-temporal weight loads, a three-stage ring with two
// tiles in flight, kept running across block boundaries) with the matching
// columns of the x rows; each wave computes y^T[32 weight rows x 32 x rows]
// on v_mfma_f32_32x32x16. HBM-bound: the weight is read once; x (<= 1 MiB) is
// re-read from L2 by every workgroup.
//
// A block whose units are split over several workgroups: each writes its fp32
// partial to the workspace, slot (workgroup, 0) for the first block of its run
// and (workgroup, 1) for the last. A per-block ticket picks the last to
// arrive, which sums the partials in workgroup order (the result does not
// depend on which came last), runs the epilogue and returns the ticket counter
// to zero. No second launch, and no workgroup waits for another.
//
// Partial output (lc_decode_linear_partials, mode 0): a grid of whole shares,
// each writing its fp32 partial to [share][M][N] with no hand-off; the
// consumer adds the shares (lc_add_rmsnorm_partials_fwd).
#include <limits.h>
#include <algorithm>
#include <math.h>

#include <type_traits>

#include "attn_tiles.h"
#include "lc_common.h"

namespace {

using namespace lc_attn;

// Four waves, one workgroup per CU (the LDS ring takes 120-156 KiB). (Two-wave
// workgroups, two per CU, measured slower in an earlier whole-block layout.)
constexpr int kDlWaves = 4;
constexpr int kDlBatch = 32;            // x rows per launch (the MFMA's N)
constexpr int kDlTileElems = 16384;     // weight elements per tile: ROWS x columns
constexpr int kDlKc = 128;              // K granularity: columns per wave per tile
// Output columns per row block.
constexpr int dl_out_cols(int mode, int rows) { return mode == 1 ? rows / 2 : rows; }
constexpr int kDlMaxBlocks = 1 << 17;   // row blocks per launch (ticket counters)
constexpr int kDlSumBatch = 8;          // partials loaded per batch by the summing workgroup
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
  float* part;    // [grid][2][ROWS * 32] partials of a workgroup's first / last block
  int* counters;  // [n_blocks], zero between calls
  int64_t xs, ws, ys;  // row strides (elements)
  int M, K, N;         // N = output columns
  int kt;              // K tiles per row block
  int n_blocks;
  // Partial output (OUTP): share s of every row block writes its fp32 sum to
  // pout[(s * M + m) * N + n]; there are `shares` equal shares per block.
  float* pout;
  int shares;
};

// First unit of workgroup g's run when U units are dealt to G workgroups.
__device__ __forceinline__ int dl_run_begin(int64_t g, int64_t U, int64_t G) {
  return static_cast<int>(g * U / G);
}
// The workgroup whose run holds unit u.
__device__ __forceinline__ int dl_owner(int64_t u, int64_t U, int64_t G) {
  return static_cast<int>(((u + 1) * G - 1) / U);
}

template <typename T, int MODE, int ROWS, bool OUTP = false>
__global__ __launch_bounds__(64 * kDlWaves) void decode_linear_kernel(DlArgs a) {
  typedef Mfma32<T> Ops;
  typedef typename Ops::v8 v8;
  constexpr int KC = kDlTileElems / ROWS;       // columns per tile
  constexpr int ROW_B = KC * (int)sizeof(T);    // bytes per row per tile
  constexpr int RW = ROWS / 32;                 // waves along the rows
  constexpr int KP = kDlWaves / RW;             // waves along K (kDlKc columns each)
  constexpr int KS = kDlKc / 16;                // MFMA k-steps per wave per tile
  constexpr int CPR = ROW_B / 16;
  constexpr int RPI = 64 / CPR;
  constexpr int NIW_W = ROWS / (RPI * kDlWaves);
  constexpr int NIW_H = kDlBatch / (RPI * kDlWaves);
  constexpr int W_B = ROWS * ROW_B;
  constexpr int H_B = kDlBatch * ROW_B;
  constexpr int STAGE_B = W_B + H_B;
  constexpr int OUTC = dl_out_cols(MODE, ROWS);  // output columns per block
  constexpr int PF = ROWS * kDlBatch;            // floats of one partial (16 per holding thread)
  constexpr int XK_B = KP > 1 ? (kDlWaves - RW) * 16 * 64 * 4 : 0;  // column-half exchange
  constexpr int XU_B = MODE == 1 ? (RW / 2) * 16 * 64 * 4 : 0;       // up-value exchange
  static_assert(KP * RW == kDlWaves && KC == KP * kDlKc && KP <= 2, "tile geometry");
  __shared__ __align__(16) char lds[3 * STAGE_B + XK_B + XU_B];
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  const int rw = wave % RW;  // row group: block rows 32 rw .. 32 rw + 31
  const int kh = wave / RW;  // column part: tile columns kDlKc kh .. + kDlKc - 1
  // Waves of column part 0 hold a block's sums once the parts are added.
  const bool holder = kh == 0;
  const int kt = a.kt;
  const int64_t U = (int64_t)a.n_blocks * kt;
  const int64_t G = gridDim.x;
  const int g = blockIdx.x;
  const int u_begin = dl_run_begin(g, U, G);
  const int n = dl_run_begin(g + 1, U, G) - u_begin;
  const int first_blk = u_begin / kt;

  // Per-lane DMA offsets from a block's first weight row: mode 0 rows
  // 0 .. ROWS-1; mode 1 gate rows 0 .. ROWS/2-1 (block rows 0 .. ROWS/2-1)
  // and up rows N .. N+ROWS/2-1. Rows past the matrix are past the
  // descriptor's range and land in LDS as zeros; gate rows past N read up
  // rows (their outputs are not stored).
  const PfLoadOffsets<NIW_W> woff = [&] {
    PfLoadOffsets<NIW_W> o;
#pragma unroll
    for (int u = 0; u < NIW_W; ++u) {
      const int row = (wave * NIW_W + u) * RPI + lane / CPR;
      const int ch = (lane % CPR) ^ pf_swz<16>(row);
      const int64_t wrow = MODE == 1 && row >= ROWS / 2 ? (int64_t)a.N + row - ROWS / 2 : row;
      o.o[u] = static_cast<int>((wrow * a.ws + ch * 8) * sizeof(T));
    }
    return o;
  }();
  const PfLoadOffsets<NIW_H> hoff = [&] {
    PfLoadOffsets<NIW_H> o;
#pragma unroll
    for (int u = 0; u < NIW_H; ++u) {
      const int row = (wave * NIW_H + u) * RPI + lane / CPR;
      const int ch = (lane % CPR) ^ pf_swz<16>(row);
      // Rows past M: an offset past the descriptor's range (< 2^31) with any
      // tile offset added, so they load zeros.
      o.o[u] = row < a.M ? static_cast<int>(((int64_t)row * a.xs + ch * 8) * sizeof(T)) : INT_MIN;
    }
    return o;
  }();
  const int xbytes = static_cast<int>(((int64_t)(a.M - 1) * a.xs + a.K) * sizeof(T));
  // LDS chunk c of row r sits at position c ^ pf_swz<16>(r); lane (l32, hh)
  // reads chunks kh*16 + hh*8 + s (k-step s) of row l32 -- the same k order
  // for the weight rows and the x rows.
  int raddr[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s)
    raddr[s] = l32 * ROW_B + (((kh * 16 + hh * 8 + s) ^ pf_swz<16>(l32)) << 4);
  const int wrow0 = rw * 32 * ROW_B;

  // DMA cursor: the block and tile of the next unit to fetch.
  int f_blk = first_blk;
  int f_t = u_begin - first_blk * kt;
  auto fetch = [&](int stage) __attribute__((always_inline)) {
    const int c0 = f_blk * OUTC;
    const int cols_valid = min(OUTC, a.N - c0);
    const int64_t last_row = MODE == 1 ? (int64_t)a.N + cols_valid - 1 : (int64_t)cols_valid - 1;
    const T* wbase = static_cast<const T*>(a.w) + (int64_t)c0 * a.ws;
    const int wbytes = static_cast<int>((last_row * a.ws + a.K) * sizeof(T));
    LC_LDS char* dst = (LC_LDS char*)lds + stage * STAGE_B;
    pf_dma_tile_untracked<NIW_W, RPI, ROW_B, true>(wbase, wbytes, dst, wave_s, woff, f_t * ROW_B);
    pf_dma_tile_untracked<NIW_H, RPI, ROW_B, false>(a.x, xbytes, dst + W_B, wave_s, hoff, f_t * ROW_B);
    if (++f_t == kt) {
      f_t = 0;
      ++f_blk;
    }
  };

  f32x16_t acc[2];
  auto zero_acc = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
  };
  zero_acc();
  auto compute = [&](int stage) __attribute__((always_inline)) {
    LC_LDS const char* wl = (LC_LDS const char*)lds + stage * STAGE_B + wrow0;
    LC_LDS const char* hl = (LC_LDS const char*)lds + stage * STAGE_B + W_B;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      acc[s & 1] = Ops::mma(*reinterpret_cast<LC_LDS const v8*>(wl + raddr[s]),
                            *reinterpret_cast<LC_LDS const v8*>(hl + raddr[s]), acc[s & 1]);
  };

  // End of a block's run in this workgroup: add the column parts, combine
  // with the block's other workgroups if it is split, and (in the workgroup
  // that completes it) store the block's outputs. Every wave takes the same
  // path through the barriers (s_last is read by all after a barrier).
  auto finish_block = [&](int blk) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[0][r] += acc[1][r];
    if constexpr (KP > 1) {
      // (The exchange area is not touched again before every wave has passed
      // the next tile's barrier.)
      float* xk = reinterpret_cast<float*>(lds + 3 * STAGE_B);
      if (!holder) {
#pragma unroll
        for (int r = 0; r < 16; ++r) xk[(((kh - 1) * RW + rw) * 16 + r) * 64 + lane] = acc[0][r];
      }
      __syncthreads();
      if (holder) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[0][r] += xk[(rw * 16 + r) * 64 + lane];
      }
    }
    if constexpr (OUTP) {
      // The grid is n_blocks x shares workgroups, one share each (block g /
      // shares, share g % shares): the share's fp32 sum goes out as it is,
      // for the consumer to add up. Holding lane (l32, hh) of row group rw:
      // x row l32, columns rw*32 + 8j + 4hh + i (register 4j + i). N % 4 == 0.
      if (!holder || l32 >= a.M) return;
      const int c0 = blk * OUTC;
      const int cols_valid = min(OUTC, a.N - c0);
      float* prow = a.pout + ((int64_t)(g % a.shares) * a.M + l32) * a.N + c0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int col = rw * 32 + j * 8 + hh * 4;
        if (col < cols_valid) {
          const f32x4_t v = {acc[0][4 * j], acc[0][4 * j + 1], acc[0][4 * j + 2], acc[0][4 * j + 3]};
          *reinterpret_cast<f32x4_t*>(prow + col) = v;
        }
      }
      return;
    }
    const int blk_lo = blk * kt;
    const int run_lo = u_begin;
    const int run_hi = u_begin + n;
    if (run_lo > blk_lo || run_hi < blk_lo + kt) {
      // Partial of this run: register r of holding thread tid at
      // [slot][tid][16] (four 16-byte runs), so the summing workgroup's
      // thread tid gets the same (row, x row) back. The partials travel
      // through stores and loads with the sc1 cache policy (agent-coherent:
      // performed past the per-XCD L2s, as agent-scope atomics are), so no
      // cache-wide write-back or invalidate is needed: each lane waits for
      // its stores to be acknowledged before the workgroup takes its ticket.
      const int slot = g * 2 + (blk == first_blk ? 0 : 1);
      if (holder) {
        const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
            a.part + (int64_t)slot * PF, 0, PF * 4, 0x00020000);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4_t v = {acc[0][4 * q], acc[0][4 * q + 1], acc[0][4 * q + 2], acc[0][4 * q + 3]};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), prs, tid * 64 + 16 * q,
                                                 0, kDlCoherent);
        }
      }
      const int g_first = dl_owner(blk_lo, U, G);
      const int g_last = dl_owner(blk_lo + kt - 1, U, G);
      // Hand-off invariant (the ticket itself is relaxed): every partial store
      // above is sc1 (agent-coherent, written through to L2) and has been
      // acknowledged (the s_waitcnt) by every wave (the barrier) before the
      // ticket is taken; the last workgroup's loads of the partials are sc1
      // too and control-dependent on s_last, so they cannot be served from a
      // stale L1 line or issued before the ticket. Dropping the wait, or a
      // partial store without sc1, breaks the hand-off.
      __builtin_amdgcn_s_waitcnt(dl_waitcnt(0, 0));
      __syncthreads();
      if (tid == 0) {
        const int ticket = __hip_atomic_fetch_add(a.counters + blk, 1, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
        s_last = ticket == g_last - g_first;
      }
      __syncthreads();
      if (!s_last) return;
      if (holder) {
        // The block's partials in workgroup order: the first workgroup's is
        // its last-block slot unless its run starts at this block.
        const int first_slot =
            g_first * 2 + (dl_run_begin(g_first, U, G) < blk_lo ? 1 : 0);
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[0][r] = 0.f;
        for (int gb = g_first; gb <= g_last; gb += kDlSumBatch) {
          u32x4_t pv[kDlSumBatch][4];
#pragma unroll
          for (int i = 0; i < kDlSumBatch; ++i)
            if (gb + i <= g_last) {
              const int sl = gb + i == g_first ? first_slot : (gb + i) * 2;
              const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
                  a.part + (int64_t)sl * PF, 0, PF * 4, 0x00020000);
#pragma unroll
              for (int q = 0; q < 4; ++q)
                pv[i][q] = __builtin_amdgcn_raw_buffer_load_b128(prs, tid * 64 + 16 * q, 0,
                                                                 kDlCoherent);
            }
#pragma unroll
          for (int i = 0; i < kDlSumBatch; ++i)
            if (gb + i <= g_last) {
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const f32x4_t v = __builtin_bit_cast(f32x4_t, pv[i][q]);
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[0][4 * q + e] += v[e];
              }
            }
        }
      }
      if (tid == 0)
        __hip_atomic_store(a.counters + blk, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // Epilogue. Holding lane (l32, hh) of row group rw holds x row l32 and
    // block rows rw*32 + 8j + 4hh + i (register 4j + i).
    typedef T t4 __attribute__((ext_vector_type(4)));
    const int c0 = blk * OUTC;
    const int cols_valid = min(OUTC, a.N - c0);
    T* yrow = static_cast<T*>(a.y) + (int64_t)l32 * a.ys + c0;
    if constexpr (MODE == 0) {
      if (!holder || l32 >= a.M) return;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int col = rw * 32 + j * 8 + hh * 4;
        t4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = lc_from_f32<T>(acc[0][j * 4 + i]);
        if (col + 4 <= cols_valid) {
          *reinterpret_cast<t4*>(yrow + col) = o;
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (col + i < cols_valid) yrow[col + i] = o[i];
        }
      }
    } else {
      // The upper row groups hold the up rows of the columns the lower ones
      // hold the gate rows of; the rounded up values go through LDS.
      constexpr int HALF = RW / 2;
      float* ux = reinterpret_cast<float*>(lds + 3 * STAGE_B + XK_B);
      if (holder && rw >= HALF) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          ux[((rw - HALF) * 16 + r) * 64 + lane] = lc_to_f32(lc_from_f32<T>(acc[0][r]));
      }
      __syncthreads();
      if (!holder || rw >= HALF || l32 >= a.M) return;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int col = rw * 32 + j * 8 + hh * 4;
        t4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = j * 4 + i;
          const float gv = lc_to_f32(lc_from_f32<T>(acc[0][r]));
          o[i] = lc_from_f32<T>(dl_silu_mul(gv, ux[(rw * 16 + r) * 64 + lane]));
        }
        if (col + 4 <= cols_valid) {
          *reinterpret_cast<t4*>(yrow + col) = o;
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (col + i < cols_valid) yrow[col + i] = o[i];
        }
      }
    }
  };

  // Iteration i: wait for tile i (this wave's DMA; tile i+1 may still be in
  // flight), barrier (every wave's part of tile i landed, every wave done with
  // tile i-1 and with the exchange areas), refill tile i-1's stage with tile
  // i+2, compute tile i; at the last tile of a block's run, finish the block.
  constexpr int kNi = NIW_W + NIW_H;  // DMA instructions per wave per tile
  fetch(0);
  if (n > 1) fetch(1);
  int stage = 0;
  int c_blk = first_blk;
  int c_t = u_begin - first_blk * kt;
  for (int i = 0; i < n; ++i) {
    if (i + 1 < n)
      __builtin_amdgcn_s_waitcnt(dl_waitcnt(kNi, 0));
    else
      __builtin_amdgcn_s_waitcnt(dl_waitcnt(0, 0));
    lc_compiler_fence();
    __builtin_amdgcn_s_barrier();
    lc_compiler_fence();
    if (i + 2 < n) fetch(stage == 0 ? 2 : stage - 1);
    compute(stage);
    stage = stage == 2 ? 0 : stage + 1;
    if (c_t == kt - 1 || i == n - 1) {
      finish_block(c_blk);
      zero_acc();
    }
    if (++c_t == kt) {
      c_t = 0;
      ++c_blk;
    }
  }
}

// Workgroups for U = n_blocks * k_tiles units: with a request, `requested`
// per row block (at most one per unit). Otherwise shares of per0 units, an
// even spread over the CUs -- or of up to two units more where that lines
// the shares up with the blocks (per divides k_tiles, or is a multiple of
// it). A share that ends a partial block before its own end publishes that
// partial while tiles are in flight (waits for its stores, takes a ticket),
// which measured about three tiles' streaming time: at [32, 4096] x
// [4096, 6144] shares of 8 on 192 workgroups beat shares of 6 on 256
// (15.2 vs 16.6 us); at 28 vs 32 tiles per share the even spread wins.
int64_t dl_grid(int64_t n_blocks, int64_t k_tiles, int requested, int n_cu) {
  const int64_t U = n_blocks * k_tiles;
  if (requested > 0) return std::min<int64_t>(U, n_blocks * requested);
  const int64_t per0 = (U + n_cu - 1) / n_cu;
  for (int64_t per = per0; per <= per0 + 2; ++per)
    if (U % per == 0 && (k_tiles % per == 0 || per % k_tiles == 0)) return U / per;
  return (U + per0 - 1) / per0;
}

// Rows per block: 64 (512-byte runs per row) where K allows 256-column
// tiles, else 128.
int dl_rows(int64_t K) { return K % (2 * kDlKc) == 0 ? 64 : 128; }

// Shares per row block for partial output. Where lc_decode_linear's own grid
// deals each block out in equal whole shares, the same shares (so the two
// paths add the same partials in the same order); otherwise the fewest that
// divide the block's tiles and keep at least 3/4 of the CUs busy (every share
// is one workgroup), else one per tile.
int64_t dl_shares(int64_t n_blocks, int64_t k_tiles, int n_cu) {
  const int64_t U = n_blocks * k_tiles;
  const int64_t g = dl_grid(n_blocks, k_tiles, 0, n_cu);
  if (U % g == 0 && k_tiles % (U / g) == 0) return k_tiles / (U / g);
  for (int64_t d = 1; d <= k_tiles; ++d)
    if (k_tiles % d == 0 && 4 * n_blocks * d >= 3 * (int64_t)n_cu) return d;
  return k_tiles;
}

struct DlPlan {
  int rows;
  int64_t n_blocks, k_tiles, grid, workspace;
};

bool dl_plan(int64_t N, int64_t K, int mode, int splits, DlPlan* p) {
  if (N <= 0 || K <= 0 || K % kDlKc || (mode != 0 && mode != 1) || splits < 0) return false;
  p->rows = dl_rows(K);
  const int64_t out_cols = dl_out_cols(mode, p->rows);
  p->n_blocks = (N + out_cols - 1) / out_cols;
  if (p->n_blocks > kDlMaxBlocks) return false;
  p->k_tiles = K / (kDlTileElems / p->rows);
  p->grid = dl_grid(p->n_blocks, p->k_tiles, splits, lc_cu_count());
  const int64_t U = p->n_blocks * p->k_tiles;
  // No partials when every run is a whole number of whole blocks.
  const bool whole = U % p->grid == 0 && (U / p->grid) % p->k_tiles == 0;
  p->workspace = whole ? 256 : (p->grid * 2 * p->rows * kDlBatch * 4 + 255) / 256 * 256;
  return true;
}

}  // namespace

extern "C" {

int64_t lc_decode_linear_workspace_bytes(int64_t M, int64_t N, int64_t K, int mode, int splits) {
  DlPlan p;
  if (M < 0 || !dl_plan(N, K, mode, splits, &p)) return -1;
  return p.workspace;
}

int64_t lc_decode_linear_counter_count(int64_t N, int mode) {
  if (N <= 0 || (mode != 0 && mode != 1)) return -1;
  // Enough for the smaller row block (64 rows).
  const int64_t out_cols = dl_out_cols(mode, 64);
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
  DlPlan p;
  LC_REQUIRE(dl_plan(N, K, mode, splits, &p), "lc_decode_linear: N=%lld too large", (long long)N);
  // Unit indices and the owner arithmetic ((u + 1) * grid) stay in 64 bits;
  // the unit count itself must fit an int.
  LC_REQUIRE(p.n_blocks * p.k_tiles < (1LL << 31), "lc_decode_linear: too many tiles");
  LC_REQUIRE(workspace_bytes >= p.workspace, "lc_decode_linear: workspace %lld < %lld bytes",
             (long long)workspace_bytes, (long long)p.workspace);
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
  a.kt = (int)p.k_tiles;
  a.n_blocks = (int)p.n_blocks;
  hipStream_t st = lc_stream(stream);
  const dim3 grid((unsigned)p.grid);
  const bool bf = dtype == LC_DTYPE_BF16;
  const dim3 block(64 * kDlWaves);
  if (p.rows == 64) {
    if (mode == 0) {
      if (bf) decode_linear_kernel<bf16_t, 0, 64><<<grid, block, 0, st>>>(a);
      else decode_linear_kernel<f16_t, 0, 64><<<grid, block, 0, st>>>(a);
    } else {
      if (bf) decode_linear_kernel<bf16_t, 1, 64><<<grid, block, 0, st>>>(a);
      else decode_linear_kernel<f16_t, 1, 64><<<grid, block, 0, st>>>(a);
    }
  } else {
    if (mode == 0) {
      if (bf) decode_linear_kernel<bf16_t, 0, 128><<<grid, block, 0, st>>>(a);
      else decode_linear_kernel<f16_t, 0, 128><<<grid, block, 0, st>>>(a);
    } else {
      if (bf) decode_linear_kernel<bf16_t, 1, 128><<<grid, block, 0, st>>>(a);
      else decode_linear_kernel<f16_t, 1, 128><<<grid, block, 0, st>>>(a);
    }
  }
  return lc_check_launch("lc_decode_linear");
}

int64_t lc_decode_linear_partial_count(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0 || K % kDlKc) return -1;
  const int rows = dl_rows(K);
  const int64_t n_blocks = (N + rows - 1) / rows;
  if (n_blocks > kDlMaxBlocks) return -1;
  return dl_shares(n_blocks, K / (kDlTileElems / rows), lc_cu_count());
}

int lc_decode_linear_partials(const void* x, int64_t x_row_stride, const void* weight,
                              int64_t weight_row_stride, float* partials, int64_t M, int64_t N,
                              int64_t K, int shares, int dtype, void* stream) {
  LC_REQUIRE(dtype == LC_DTYPE_BF16 || dtype == LC_DTYPE_F16,
             "lc_decode_linear_partials: dtype %d (bf16 or f16 only)", dtype);
  LC_REQUIRE(M >= 0 && M <= kDlBatch, "lc_decode_linear_partials: M=%lld rows (1..%d)",
             (long long)M, kDlBatch);
  if (M == 0) return LC_OK;
  LC_REQUIRE(x && weight && partials, "lc_decode_linear_partials: null pointer");
  LC_REQUIRE(N > 0 && K > 0 && K % kDlKc == 0 && K < (1LL << 30) && N < (1LL << 30) && N % 4 == 0,
             "lc_decode_linear_partials: N=%lld K=%lld (K a positive multiple of %d, N of 4)",
             (long long)N, (long long)K, kDlKc);
  LC_REQUIRE(x_row_stride >= K && weight_row_stride >= K,
             "lc_decode_linear_partials: row strides too small");
  LC_REQUIRE(lc_aligned(x, 16) && lc_aligned(weight, 16) && x_row_stride % 8 == 0 &&
                 weight_row_stride % 8 == 0,
             "lc_decode_linear_partials: x and weight need 16-byte aligned rows");
  LC_REQUIRE(lc_aligned(partials, 16), "lc_decode_linear_partials: partials not 16-byte aligned");
  LC_REQUIRE(N * weight_row_stride * 2 < (1LL << 31) && ((M - 1) * x_row_stride + K) * 2 < (1LL << 31),
             "lc_decode_linear_partials: weight or x spans 2 GiB or more");
  const int rows = dl_rows(K);
  const int64_t n_blocks = (N + rows - 1) / rows;
  LC_REQUIRE(n_blocks <= kDlMaxBlocks, "lc_decode_linear_partials: N=%lld too large",
             (long long)N);
  const int64_t kt = K / (kDlTileElems / rows);
  const int64_t s = shares > 0 ? shares : dl_shares(n_blocks, kt, lc_cu_count());
  LC_REQUIRE(kt % s == 0, "lc_decode_linear_partials: %lld shares do not divide the %lld tiles "
             "of a row block", (long long)s, (long long)kt);
  LC_REQUIRE(n_blocks * kt < (1LL << 31), "lc_decode_linear_partials: too many tiles");
  DlArgs a{};
  a.x = x;
  a.w = weight;
  a.xs = x_row_stride;
  a.ws = weight_row_stride;
  a.M = (int)M;
  a.K = (int)K;
  a.N = (int)N;
  a.kt = (int)kt;
  a.n_blocks = (int)n_blocks;
  a.pout = partials;
  a.shares = (int)s;
  hipStream_t st = lc_stream(stream);
  const dim3 grid((unsigned)(n_blocks * s));
  const dim3 block(64 * kDlWaves);
  const bool bf = dtype == LC_DTYPE_BF16;
  if (rows == 64) {
    if (bf) decode_linear_kernel<bf16_t, 0, 64, true><<<grid, block, 0, st>>>(a);
    else decode_linear_kernel<f16_t, 0, 64, true><<<grid, block, 0, st>>>(a);
  } else {
    if (bf) decode_linear_kernel<bf16_t, 0, 128, true><<<grid, block, 0, st>>>(a);
    else decode_linear_kernel<f16_t, 0, 128, true><<<grid, block, 0, st>>>(a);
  }
  return lc_check_launch("lc_decode_linear_partials");
}

}  // extern "C"
