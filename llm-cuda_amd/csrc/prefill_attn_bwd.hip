// Causal attention backward (dQ, dK, dV) with native GQA, no atomics.
//
// Given the forward's output O and natural-log logsumexp L, and dO:
//   delta_i = sum_d dO_id O_id                      (in the MFMA dQ kernel, or
//                                                    attn_bwd_delta_kernel)
//   P_ij    = exp(s_ij - L_i),  s_ij = q_i.k_j * scale + bias_ij
//             (keys j <= i + q_offset; bias: the optional additive mask)
//   dS_ij   = P_ij (dO_i.v_j - delta_i)
//   dQ_i    = scale * sum_j dS_ij k_j                (one pass over key tiles)
//   dK_j    = scale * sum_{h in group, i} dS_ij q_i  (one pass over query tiles,
//   dV_j    =         sum_{h in group, i} P_ij dO_i   summed over the G heads)
// (kernels/triton/attention.py:180-320,380-454 of the reference, which runs one
// program per query row and accumulates dK/dV with atomics.)
//
// Kernels, chosen like the forward's:
//   * bf16/f16 with D a multiple of 8 up to 128: MFMA kernels. The dQ kernel
//     keeps the forward's layout (K/V tiles in LDS, Q^T and dO^T operands in
//     registers, keys on accumulator rows); the dK/dV kernel swaps the roles
//     (Q/dO tiles in LDS, K^T and V^T operands in registers, queries on
//     accumulator rows, keys on lanes), so in both the probabilities and dS
//     feed the next product straight from the accumulator registers.
//   * everything else: lane-per-row fp32 kernels.
#include <math.h>

#include <type_traits>

#include "attn_tiles.h"
#include "lc_common.h"

namespace {

using namespace lc_attn;

struct BwdArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* dout;
  const float* lse;    // [B, Hq, Sq], natural log
  const float* delta;  // [B, Hq, Sq]
  const float* lse2;   // [B, Hq, Sq], lse * log2(e), +inf where lse = -inf
  // The forward's output: the MFMA dQ kernel forms delta and lse2 itself and
  // writes them for the dK/dV kernel (the generic path runs the delta kernel).
  const void* o;
  int64_t os[4];
  void* dq;
  void* dk;
  void* dv;
  int64_t qs[4], ks[4], vs[4], dos[4], dqs[4], dks[4], dvs[4];
  int B, Hq, Hkv, G, Sq, Skv, D, q_offset;
  float scale, scale_log2;
  // Additive bias [B, Hq, Sq, Skv] with element strides bs (0 = broadcast),
  // dtype bias_dtype (LC_DTYPE_*); null: none. bias_vec as in the forward.
  const void* bias;
  int64_t bs[4];
  int bias_dtype;
  int bias_vec;
};

// ---------------------------------------------------------------------------
// delta = rowsum(dO * O) in fp32: 16 lanes per row.
// ---------------------------------------------------------------------------
// Also writes lse2 = lse * log2(e) (+inf for rows that saw no key, so that
// their probabilities come out as exactly zero) for the MFMA kernels.
// 16 lanes per row; VEC: lane c reads elements 8c .. 8c+7 of both rows as one
// 16-byte load (D a multiple of 8, at most 128).
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void attn_bwd_delta_kernel(const T* __restrict__ o,
                                                             const T* __restrict__ dout,
                                                             const float* __restrict__ lse,
                                                             float* __restrict__ delta,
                                                             float* __restrict__ lse2,
                                                             int64_t os0, int64_t os1,
                                                             int64_t os2, int64_t ds0,
                                                             int64_t ds1, int64_t ds2, int Hq,
                                                             int Sq, int D, int64_t rows) {
  const int64_t row = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 4;
  const int sub = threadIdx.x & 15;
  float acc = 0.f;
  if (row < rows) {
    const int i = static_cast<int>(row % Sq);
    const int64_t bh = row / Sq;
    const int h = static_cast<int>(bh % Hq);
    const int64_t b = bh / Hq;
    const T* orow = o + b * os0 + h * os1 + (int64_t)i * os2;
    const T* drow = dout + b * ds0 + h * ds1 + (int64_t)i * ds2;
    if constexpr (VEC) {
      typedef T t8 __attribute__((ext_vector_type(8)));
      if (sub * 8 < D) {
        const t8 ov = *reinterpret_cast<const t8*>(orow + sub * 8);
        const t8 dv = *reinterpret_cast<const t8*>(drow + sub * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc = fmaf(lc_to_f32(ov[e]), lc_to_f32(dv[e]), acc);
      }
    } else {
      for (int d = sub; d < D; d += 16) acc = fmaf(lc_to_f32(orow[d]), lc_to_f32(drow[d]), acc);
    }
  }
#pragma unroll
  for (int w = 8; w >= 1; w >>= 1) acc += __shfl_xor(acc, w, 64);
  if (row < rows && sub == 0) {
    delta[row] = acc;
    const float l = lse[row];
    lse2[row] = l == -INFINITY ? INFINITY : l * kLog2e;
  }
}

// ---------------------------------------------------------------------------
// Generic kernels (any dtype, any D <= 256). A row (query row for dQ, key row
// for dK/dV) belongs to LPR = DMAX/32 adjacent lanes; lane `sub` of a row holds
// dims d = t*LPR + sub, t < 32, so a row's dot products end in a log2(LPR)-step
// shuffle reduction. Operand tiles of 16 rows are staged in LDS as fp32.
// ---------------------------------------------------------------------------
template <int LPR>
__device__ __forceinline__ float row_sum(float x) {
#pragma unroll
  for (int w = 1; w < LPR; w <<= 1) x += __shfl_xor(x, w, 64);
  return x;
}

template <typename T, int DMAX>
__global__ __launch_bounds__(64) void attn_bwd_dq_generic_kernel(BwdArgs a) {
  constexpr int KT = 16, LPR = DMAX / 32, RPW = 64 / LPR;
  __shared__ float ks[KT][DMAX];
  __shared__ float vs[KT][DMAX];
  const int lane = threadIdx.x;
  const int sub = lane % LPR;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int i = blockIdx.x * RPW + lane / LPR;
  const int kvh = h / a.G;
  const bool row_ok = i < a.Sq;
  const T* qp = static_cast<const T*>(a.q) + b * a.qs[0] + h * a.qs[1] + (int64_t)i * a.qs[2];
  const T* dop = static_cast<const T*>(a.dout) + b * a.dos[0] + h * a.dos[1] + (int64_t)i * a.dos[2];
  const T* kp = static_cast<const T*>(a.k) + b * a.ks[0] + kvh * a.ks[1];
  const T* vp = static_cast<const T*>(a.v) + b * a.vs[0] + kvh * a.vs[1];
  float qr[32], dor[32], acc[32];
#pragma unroll
  for (int t = 0; t < 32; ++t) {
    const int d = t * LPR + sub;
    qr[t] = (row_ok && d < a.D) ? lc_to_f32(qp[d]) : 0.f;
    dor[t] = (row_ok && d < a.D) ? lc_to_f32(dop[d]) : 0.f;
    acc[t] = 0.f;
  }
  const int64_t ridx = ((int64_t)b * a.Hq + h) * a.Sq + i;
  const float lse = row_ok ? a.lse[ridx] : -INFINITY;
  const float lse2 = lse * kLog2e;
  const float dl = row_ok ? a.delta[ridx] : 0.f;
  const int last_row = min(a.Sq - 1, (int)blockIdx.x * RPW + RPW - 1);
  const int kv_hi = min(a.Skv, last_row + a.q_offset + 1);
  // A row with lse = -inf saw no key: its gradient is zero.
  const int my_hi = (row_ok && lse != -INFINITY) ? min(a.Skv, i + a.q_offset + 1) : 0;
  const int64_t brow = b * a.bs[0] + h * a.bs[1] + (int64_t)i * a.bs[2];
  for (int j0 = 0; j0 < kv_hi; j0 += KT) {
    __syncthreads();
    for (int e = lane; e < KT * DMAX; e += 64) {
      const int r = e / DMAX, d = e - r * DMAX;
      const int j = j0 + r;
      const bool ok = j < a.Skv && d < a.D;
      ks[r][d] = ok ? lc_to_f32(kp[(int64_t)j * a.ks[2] + d]) : 0.f;
      vs[r][d] = ok ? lc_to_f32(vp[(int64_t)j * a.vs[2] + d]) : 0.f;
    }
    __syncthreads();
    // All lanes of a row share jn, so the shuffles below see whole rows.
    const int jn = min(KT, my_hi - j0);
    for (int r = 0; r < jn; ++r) {
      float s = 0.f, dp = 0.f;
#pragma unroll
      for (int t = 0; t < 32; ++t) {
        s = fmaf(qr[t], ks[r][t * LPR + sub], s);
        dp = fmaf(dor[t], vs[r][t * LPR + sub], dp);
      }
      s = row_sum<LPR>(s);
      dp = row_sum<LPR>(dp);
      float x = s * a.scale_log2 - lse2;
      if (a.bias != nullptr)
        x += lc_bias_log2(lc_load_bias(a.bias, brow + (int64_t)(j0 + r) * a.bs[3], a.bias_dtype));
      const float p = lc_exp2(x);
      const float ds = p * (dp - dl);
#pragma unroll
      for (int t = 0; t < 32; ++t) acc[t] = fmaf(ds, ks[r][t * LPR + sub], acc[t]);
    }
  }
  if (!row_ok) return;
  T* out = static_cast<T*>(a.dq) + b * a.dqs[0] + h * a.dqs[1] + (int64_t)i * a.dqs[2];
#pragma unroll
  for (int t = 0; t < 32; ++t) {
    const int d = t * LPR + sub;
    if (d < a.D) out[d] = lc_from_f32<T>(acc[t] * a.scale);
  }
}

template <typename T, int DMAX>
__global__ __launch_bounds__(64) void attn_bwd_dkv_generic_kernel(BwdArgs a) {
  constexpr int QT = 16, LPR = DMAX / 32, RPW = 64 / LPR;
  __shared__ float qs[QT][DMAX];
  __shared__ float dos[QT][DMAX];
  __shared__ float lse_t[QT], dl_t[QT];
  const int lane = threadIdx.x;
  const int sub = lane % LPR;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int j = blockIdx.x * RPW + lane / LPR;
  const bool key_ok = j < a.Skv;
  const T* kp = static_cast<const T*>(a.k) + b * a.ks[0] + kvh * a.ks[1] + (int64_t)j * a.ks[2];
  const T* vp = static_cast<const T*>(a.v) + b * a.vs[0] + kvh * a.vs[1] + (int64_t)j * a.vs[2];
  float kr[32], vr[32], dk[32], dv[32];
#pragma unroll
  for (int t = 0; t < 32; ++t) {
    const int d = t * LPR + sub;
    kr[t] = (key_ok && d < a.D) ? lc_to_f32(kp[d]) : 0.f;
    vr[t] = (key_ok && d < a.D) ? lc_to_f32(vp[d]) : 0.f;
    dk[t] = 0.f;
    dv[t] = 0.f;
  }
  // Query row i sees key j iff j <= i + q_offset; the workgroup's first key
  // bounds the first query tile.
  const int i_begin = max(0, (int)blockIdx.x * RPW - a.q_offset);
  for (int g = 0; g < a.G; ++g) {
    const int h = kvh * a.G + g;
    const T* qb = static_cast<const T*>(a.q) + b * a.qs[0] + h * a.qs[1];
    const T* db = static_cast<const T*>(a.dout) + b * a.dos[0] + h * a.dos[1];
    const int64_t rbase = ((int64_t)b * a.Hq + h) * a.Sq;
    for (int i0 = i_begin / QT * QT; i0 < a.Sq; i0 += QT) {
      __syncthreads();
      for (int e = lane; e < QT * DMAX; e += 64) {
        const int r = e / DMAX, d = e - r * DMAX;
        const int i = i0 + r;
        const bool ok = i < a.Sq && d < a.D;
        qs[r][d] = ok ? lc_to_f32(qb[(int64_t)i * a.qs[2] + d]) : 0.f;
        dos[r][d] = ok ? lc_to_f32(db[(int64_t)i * a.dos[2] + d]) : 0.f;
      }
      if (lane < QT) {
        const int i = i0 + lane;
        const float lse = i < a.Sq ? a.lse[rbase + i] : -INFINITY;
        // +inf for rows without keys (and past the end) makes their P zero.
        lse_t[lane] = lse == -INFINITY ? INFINITY : lse * kLog2e;
        dl_t[lane] = i < a.Sq ? a.delta[rbase + i] : 0.f;
      }
      __syncthreads();
      // Per-row conditions depend on j only through the row's key, which all
      // LPR lanes of the row share, so the shuffles below see whole rows.
      for (int r = 0; r < QT; ++r) {
        const int i = i0 + r;
        if (!key_ok || i >= a.Sq || j > i + a.q_offset) continue;
        float s = 0.f, dp = 0.f;
#pragma unroll
        for (int t = 0; t < 32; ++t) {
          s = fmaf(qs[r][t * LPR + sub], kr[t], s);
          dp = fmaf(dos[r][t * LPR + sub], vr[t], dp);
        }
        s = row_sum<LPR>(s);
        dp = row_sum<LPR>(dp);
        float x = s * a.scale_log2 - lse_t[r];
        if (a.bias != nullptr)
          x += lc_bias_log2(lc_load_bias(
              a.bias, b * a.bs[0] + h * a.bs[1] + (int64_t)i * a.bs[2] + (int64_t)j * a.bs[3],
              a.bias_dtype));
        const float p = lc_exp2(x);
        const float ds = p * (dp - dl_t[r]);
#pragma unroll
        for (int t = 0; t < 32; ++t) {
          dk[t] = fmaf(ds, qs[r][t * LPR + sub], dk[t]);
          dv[t] = fmaf(p, dos[r][t * LPR + sub], dv[t]);
        }
      }
    }
  }
  if (!key_ok) return;
  T* dkp = static_cast<T*>(a.dk) + b * a.dks[0] + kvh * a.dks[1] + (int64_t)j * a.dks[2];
  T* dvp = static_cast<T*>(a.dv) + b * a.dvs[0] + kvh * a.dvs[1] + (int64_t)j * a.dvs[2];
#pragma unroll
  for (int t = 0; t < 32; ++t) {
    const int d = t * LPR + sub;
    if (d < a.D) {
      dkp[d] = lc_from_f32<T>(dk[t] * a.scale);
      dvp[d] = lc_from_f32<T>(dv[t]);
    }
  }
}

template <typename T>
int launch_bwd_generic(const BwdArgs& a, hipStream_t st) {
#define LC_BWD_GEN(DM)                                                                  \
  do {                                                                                  \
    constexpr int rpw = 64 / ((DM) / 32);                                               \
    if (a.Sq > 0)                                                                       \
      attn_bwd_dq_generic_kernel<T, DM>                                                 \
          <<<dim3((a.Sq + rpw - 1) / rpw, a.Hq, a.B), 64, 0, st>>>(a);                 \
    if (a.Skv > 0)                                                                      \
      attn_bwd_dkv_generic_kernel<T, DM>                                                \
          <<<dim3((a.Skv + rpw - 1) / rpw, a.Hkv, a.B), 64, 0, st>>>(a);               \
  } while (0)
  if (a.D <= 32)
    LC_BWD_GEN(32);
  else if (a.D <= 64)
    LC_BWD_GEN(64);
  else if (a.D <= 128)
    LC_BWD_GEN(128);
  else
    LC_BWD_GEN(256);
#undef LC_BWD_GEN
  return lc_check_launch("lc_prefill_attn_bwd (generic)");
}

// ---------------------------------------------------------------------------
// MFMA kernels (bf16/f16, D a multiple of 8 up to 128, padded to DPAD 64/128).
//
// v_mfma_f32_32x32x16 operand layout used throughout: an A operand lane holds
// row l % 32 and 8 consecutive k; a B operand lane holds column l % 32 and the
// same 8 k; accumulator register r of lane l holds column l % 32, row
// 8 (r / 4) + 4 (l / 32) + r % 4. In a product whose B operand is an
// accumulator of the previous product (P or dS), k index 8 (l / 32) + e is
// mapped to row 16 jp + 8 (e / 4) + 4 (l / 32) + e % 4 of that accumulator for
// k-step jp, so a lane's B operand is its own registers 8 jp .. 8 jp + 7; the
// A operand then comes from ds_read_b64_tr_b16 (4 rows x 16 columns per
// 16-lane group) over the same rows.
// ---------------------------------------------------------------------------
constexpr int kBwWaves = 4;   // dQ kernel: waves per workgroup
constexpr int kBwRows = 32;   // dQ kernel: query rows per wave
constexpr int kBwTile = 64;   // rows per LDS tile (keys for dQ, queries for dK/dV)
constexpr int kBkWaves = 4;             // dK/dV kernel: waves per workgroup (32 keys each)
constexpr int kBkKeys = 32 * kBkWaves;  // keys per dK/dV workgroup
// Depth of the dK/dV pipeline's LDS operand ring (MFMA slots read ahead).
constexpr int kBkRing = 8;
// Mask selector for the dK/dV loop: decide per tile at run time.
constexpr int kRuntimeMask = 2;

// LDS offsets shared by both kernels for a tile of 64 rows x DPAD.
template <int DPAD, int T_SIZE>
struct TileAddr {
  static constexpr int KS = DPAD / 16;
  static constexpr int DTL = DPAD / 32;
  static constexpr int CPR = DPAD / 8;
  static constexpr int ROW_B = DPAD * T_SIZE;
  // Row-major operand reads (ds_read_b128): row l32 (+32 half as an
  // immediate), chunk hh * CPR/2 + s, i.e. d = hh * DPAD/2 + 8 s .. + 8.
  int row[KS];
  // Transposed reads: rows 4hh + te (+8jj, +16jp, +32 half), columns
  // dt*32 + (gq & 1)*16 + 4tc .. + 4 of each 16-lane group gq.
  int tr[2][DTL];
  __device__ __forceinline__ TileAddr(int lane) {
    const int l32 = lane & 31, hh = lane >> 5;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      row[s] = l32 * ROW_B + (((hh * (CPR / 2) + s) ^ pf_swz<CPR>(l32)) << 4);
    const int gq = lane >> 4, te = (lane & 15) >> 2, tc = lane & 3;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int dt = 0; dt < DTL; ++dt) {
        const int kr = jj * 8 + hh * 4 + te;
        const int d = dt * 32 + (gq & 1) * 16 + 4 * tc;
        tr[jj][dt] = kr * ROW_B + ((((d >> 3) ^ pf_swz<CPR>(kr)) << 4) | ((d & 7) * T_SIZE));
      }
  }
};

// Per-lane DMA offsets of a 64-row tile whose rows are `rs` elements apart:
// instruction u of wave w fills rows (w * NIW + u) * RPI + lane / CPR, chunk
// position lane % CPR = global chunk ^ pf_swz(row); chunks past head_dim
// re-read chunk 0 (they meet zero operand elements or land in discarded rows).
template <int NIW, int DPAD, typename T>
__device__ __forceinline__ PfLoadOffsets<NIW> tile_dma_offsets(int wave, int lane, int64_t rs,
                                                               int D) {
  constexpr int CPR = DPAD / 8, RPI = 64 / CPR;
  PfLoadOffsets<NIW> off;
#pragma unroll
  for (int u = 0; u < NIW; ++u) {
    const int row = (wave * NIW + u) * RPI + lane / CPR;
    int ch = (lane % CPR) ^ pf_swz<CPR>(row);
    ch = ch * 8 < D ? ch : 0;
    off.o[u] = static_cast<int>(((int64_t)row * rs + ch * 8) * sizeof(T));
  }
  return off;
}

// Row-operand registers: lane holds row `row` (when ok), d = hh*DPAD/2 + 8s.
template <typename T, int DPAD, typename v8>
__device__ __forceinline__ void load_row_operand(v8 (&op)[DPAD / 16], const T* rowp, bool ok,
                                                 int hh, int D) {
#pragma unroll
  for (int s = 0; s < DPAD / 16; ++s) {
    const int d = hh * (DPAD / 2) + s * 8;
    op[s] = (ok && d < D) ? *reinterpret_cast<const v8*>(rowp + d) : v8{};
  }
}

// Store a transposed accumulator (rows d, column = this lane's row of `out`).
template <typename T, int DTL>
__device__ __forceinline__ void store_transposed(T* out, const f32x16_t (&acc)[DTL], float mul,
                                                 int hh, int D) {
  typedef T t4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int dt = 0; dt < DTL; ++dt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = dt * 32 + j * 8 + hh * 4;
      if (d < D) {
        t4 w;
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = lc_from_f32<T>(acc[dt][j * 4 + i] * mul);
        *reinterpret_cast<t4*>(out + d) = w;
      }
    }
}

// ---------------------------------------------------------------------------
// dQ kernel. Workgroup = 4 waves of 32 query rows sharing one kv head (the
// forward's grouping: HW = gcd(G, 4) heads x 4 / HW row blocks). Per 64-key
// tile and wave (keys on accumulator rows, queries on lanes):
//   S^T  = K  Q^T   (A: K rows from LDS, B: Q^T registers)
//   dP^T = V  dO^T  (A: V rows from LDS, B: dO^T registers)
//   dS^T = 2^(S^T scale log2e - lse2) (dP^T - delta)   (per-lane lse2, delta)
//   dQ^T += K^T dS^T (A: transposed reads of the same K tile, B: dS^T)
// K and V tiles are double-buffered in LDS and fetched by buffer-to-LDS DMA
// one tile ahead.
// ---------------------------------------------------------------------------
// With an additive bias (BIAS != 0: 1 = dtype T, 2 = fp32) the kernel runs one
// wave per SIMD (the bias tile does not fit the two-wave register budget).
template <typename T, int DPAD, int BIAS>
__global__ __launch_bounds__(64 * kBwWaves) __attribute__((
    amdgpu_waves_per_eu(BIAS == 0 ? 2 : 1, BIAS == 0 ? 2 : 1))) void
attn_bwd_dq_mfma_kernel(BwdArgs a, int hw, int n_rbg) {
  typedef Mfma32<T> Ops;
  typedef typename Ops::v8 v8;
  typedef TileAddr<DPAD, (int)sizeof(T)> TA;
  constexpr int KS = TA::KS, DTL = TA::DTL, CPR = TA::CPR, ROW_B = TA::ROW_B;
  constexpr int RPI = 64 / CPR;
  constexpr int NIW = kBwTile / (RPI * kBwWaves);
  constexpr int TILE_B = kBwTile * ROW_B;
  __shared__ __align__(16) char lds_k0[TILE_B];
  __shared__ __align__(16) char lds_k1[TILE_B];
  __shared__ __align__(16) char lds_v0[TILE_B];
  __shared__ __align__(16) char lds_v1[TILE_B];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  const int rbw = kBwWaves / hw;
  const int n_hg = a.G / hw;
  const int nwg = gridDim.x;
  const int lin = blockIdx.x;
  int work = lin;
  if ((nwg & 7) == 0) work = (lin & 7) * (nwg >> 3) + (lin >> 3);
  const int unit = work / n_rbg;
  const int rbg = n_rbg - 1 - pf_snake(work - unit * n_rbg, n_rbg);
  const int kvh_hg = unit % (a.Hkv * n_hg);
  const int b = unit / (a.Hkv * n_hg);
  const int kvh = kvh_hg / n_hg;
  const int hgi = kvh_hg - kvh * n_hg;
  const int head = kvh * a.G + hgi * hw + (wave % hw);
  const int r0 = (rbg * rbw + wave / hw) * kBwRows;
  const int wg_last_row = min(a.Sq - 1, (rbg * rbw + rbw) * kBwRows - 1);
  const int kv_end = min(a.Skv, wg_last_row + a.q_offset + 1);
  const int my_kv_end = min(a.Skv, min(a.Sq - 1, r0 + kBwRows - 1) + a.q_offset + 1);
  const int nomask_end = min(a.Skv, r0 + a.q_offset + 1);
  const bool wave_active = r0 < a.Sq;

  const T* kbase = static_cast<const T*>(a.k) + b * a.ks[0] + (int64_t)kvh * a.ks[1];
  const T* vbase = static_cast<const T*>(a.v) + b * a.vs[0] + (int64_t)kvh * a.vs[1];
  const int kbytes = a.Skv > 0 ? static_cast<int>(((int64_t)(a.Skv - 1) * a.ks[2] + a.D) * sizeof(T)) : 0;
  const int vbytes = a.Skv > 0 ? static_cast<int>(((int64_t)(a.Skv - 1) * a.vs[2] + a.D) * sizeof(T)) : 0;

  const int qi = r0 + l32;
  const bool row_ok = wave_active && qi < a.Sq;
  v8 qop[KS], doop[KS];
  load_row_operand<T, DPAD>(qop, static_cast<const T*>(a.q) + b * a.qs[0] + (int64_t)head * a.qs[1] + (int64_t)qi * a.qs[2], row_ok, hh, a.D);
  load_row_operand<T, DPAD>(doop, static_cast<const T*>(a.dout) + b * a.dos[0] + (int64_t)head * a.dos[1] + (int64_t)qi * a.dos[2], row_ok, hh, a.D);
  const int64_t ridx = ((int64_t)b * a.Hq + head) * a.Sq + qi;
  // delta = rowsum(dO * O) of this lane's row: the O row in dO's operand
  // layout (lane half hh holds dims hh*DPAD/2 ..), fp32 products in dim
  // order within each half, then the two halves added; lse2 = lse * log2(e)
  // (+inf for a row that saw no key, so its probabilities are exactly 0).
  // Both go to the workspace for the dK/dV kernel.
  float dl, lse2;
  {
    v8 oop[KS];
    load_row_operand<T, DPAD>(oop, static_cast<const T*>(a.o) + b * a.os[0] + (int64_t)head * a.os[1] + (int64_t)qi * a.os[2], row_ok, hh, a.D);
    float part = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        part = fmaf(static_cast<float>(oop[s][e]), static_cast<float>(doop[s][e]), part);
    dl = part + __shfl_xor(part, 32, 64);
    const float l = row_ok ? a.lse[ridx] : -INFINITY;
    lse2 = l == -INFINITY ? INFINITY : l * kLog2e;
    if (row_ok && hh == 0) {
      const_cast<float*>(a.delta)[ridx] = dl;
      const_cast<float*>(a.lse2)[ridx] = lse2;
    }
  }

  // Additive bias of the tile, loaded before its products (see BiasTile).
  constexpr int besz = BIAS == 2 ? 4 : 2;
  BiasTile<T, BIAS == 0 ? 1 : BIAS> btile;
  const __amdgpu_buffer_rsrc_t brs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(static_cast<const char*>(BIAS != 0 ? a.bias : a.q) +
                        (BIAS != 0 ? (b * a.bs[0] + (int64_t)head * a.bs[1]) * besz : 0)),
      0,
      BIAS != 0 ? static_cast<int>(((int64_t)(a.Sq - 1) * a.bs[2] +
                                     (int64_t)(a.Skv - 1) * a.bs[3] + 1) * besz)
                : 0,
      0x00020000);
  const int brow_b = static_cast<int>((int64_t)qi * a.bs[2] * besz);
  const int bs3_b = static_cast<int>(a.bs[3] * besz);

  const PfLoadOffsets<NIW> koff = tile_dma_offsets<NIW, DPAD, T>(wave, lane, a.ks[2], a.D);
  const PfLoadOffsets<NIW> voff = tile_dma_offsets<NIW, DPAD, T>(wave, lane, a.vs[2], a.D);
  const int kstep_b = static_cast<int>(kBwTile * a.ks[2] * sizeof(T));
  const int vstep_b = static_cast<int>(kBwTile * a.vs[2] * sizeof(T));
  const TA ad(lane);

  f32x16_t dq[DTL];
#pragma unroll
  for (int i = 0; i < DTL; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[i][r] = 0.f;
  const int n_tiles = (kv_end + kBwTile - 1) / kBwTile;

  auto kbuf = [&](auto p_c) __attribute__((always_inline)) -> LC_LDS char* {
    if constexpr (decltype(p_c)::value == 0) return (LC_LDS char*)lds_k0;
    else return (LC_LDS char*)lds_k1;
  };
  auto vbuf = [&](auto p_c) __attribute__((always_inline)) -> LC_LDS char* {
    if constexpr (decltype(p_c)::value == 0) return (LC_LDS char*)lds_v0;
    else return (LC_LDS char*)lds_v1;
  };

  auto tile = [&](int t, LC_LDS const char* kl, LC_LDS const char* vl, auto mask_c)
                  __attribute__((always_inline)) {
    f32x16_t sa[2], dpa[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        sa[kt][r] = 0.f;
        dpa[kt][r] = 0.f;
      }
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        sa[kt] = Ops::mma(*reinterpret_cast<LC_LDS const v8*>(kl + ad.row[s] + kt * 32 * ROW_B),
                          qop[s], sa[kt]);
        dpa[kt] = Ops::mma(*reinterpret_cast<LC_LDS const v8*>(vl + ad.row[s] + kt * 32 * ROW_B),
                           doop[s], dpa[kt]);
      }
    v8 dsop[2][2];
    const int k0 = t * kBwTile;
    // Key k0 + c + 4hh (c the element's compile-time offset) is visible while
    // it is <= qi + q_offset and < Skv, i.e. c < key_lim.
    const int key_lim = min(qi + a.q_offset + 1, a.Skv) - k0 - hh * 4;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = fmaf(sa[kt][r], a.scale_log2, -lse2);
        if constexpr (BIAS != 0) x += btile.log2_at(kt, r);
        if constexpr (decltype(mask_c)::value) {
          if (kt * 32 + (r >> 2) * 8 + (r & 3) >= key_lim) x = -INFINITY;
        }
        const float p = lc_exp2(x);
        dsop[kt][r >> 3][r & 7] = static_cast<T>(p * (dpa[kt][r] - dl));
      }
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int jp = 0; jp < 2; ++jp)
#pragma unroll
        for (int dt = 0; dt < DTL; ++dt) {
          const int rowoff = (kt * 32 + jp * 16) * ROW_B;
          const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (LC_LDS i16x4_t*)(kl + ad.tr[0][dt] + rowoff));
          const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (LC_LDS i16x4_t*)(kl + ad.tr[1][dt] + rowoff));
          const i16x8_t both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
          dq[dt] = Ops::mma(__builtin_bit_cast(v8, both), dsop[kt][jp], dq[dt]);
        }
  };

  // Iteration t reads tile t from buffers PAR and fetches tile t+1 into the
  // other pair; the closing barrier publishes it and frees buffers PAR.
  auto iteration = [&](int t, auto par_c, auto mask_c) __attribute__((always_inline)) {
    constexpr auto other = std::integral_constant<int, decltype(par_c)::value ^ 1>{};
    const bool work = wave_active && t * kBwTile < my_kv_end;
    // Bias before the DMA: waiting for it does not wait for the DMA.
    if constexpr (BIAS != 0)
      if (work) btile.load(brs, brow_b, t * kBwTile, hh, bs3_b, a.bias_vec != 0);
    if (t + 1 < n_tiles) {
      pf_dma_tile<NIW, RPI, ROW_B>(kbase, kbytes, kbuf(other), wave_s, koff, (t + 1) * kstep_b);
      pf_dma_tile<NIW, RPI, ROW_B>(vbase, vbytes, vbuf(other), wave_s, voff, (t + 1) * vstep_b);
    }
    if (work) tile(t, kbuf(par_c), vbuf(par_c), mask_c);
    pf_barrier<true>();
  };

  if (n_tiles > 0) {
    pf_dma_tile<NIW, RPI, ROW_B>(kbase, kbytes, kbuf(std::integral_constant<int, 0>{}), wave_s,
                                 koff, 0);
    pf_dma_tile<NIW, RPI, ROW_B>(vbase, vbytes, vbuf(std::integral_constant<int, 0>{}), wave_s,
                                 voff, 0);
  }
  pf_barrier<true>();
  // Leading tiles below every row's diagonal need no mask.
  const int t_mask = min(n_tiles, nomask_end / kBwTile);
  const std::integral_constant<int, 0> p0{};
  const std::integral_constant<int, 1> p1{};
  int t = 0;
  for (; t + 1 < t_mask; t += 2) {
    iteration(t, p0, std::false_type{});
    iteration(t + 1, p1, std::false_type{});
  }
  if (t < t_mask) {
    iteration(t, p0, std::false_type{});
    ++t;
    if (t < n_tiles) {
      iteration(t, p1, std::true_type{});
      ++t;
    }
  }
  for (; t < n_tiles; t += 2) {
    iteration(t, p0, std::true_type{});
    if (t + 1 >= n_tiles) break;
    iteration(t + 1, p1, std::true_type{});
  }

  if (!row_ok) return;
  store_transposed<T, DTL>(static_cast<T*>(a.dq) + b * a.dqs[0] + (int64_t)head * a.dqs[1] +
                               (int64_t)qi * a.dqs[2],
                           dq, a.scale, hh, a.D);
}

// ---------------------------------------------------------------------------
// dK/dV kernel. Workgroup = 4 waves of 32 keys (one 128-key block of one kv
// head); it walks the G query heads of the group and, per head, the 64-row
// query tiles that see the block. Per tile and wave (queries on accumulator
// rows, keys on lanes):
//   S  = Q  K^T   (A: Q rows from LDS, B: K^T registers)
//   dP = dO V^T   (A: dO rows from LDS, B: V^T registers)
//   P  = 2^(S scale log2e - lse2),  dS = P (dP - delta)  (lse2, delta per
//        accumulator row, read from LDS)
//   dV^T += dO^T P   (A: transposed reads of the dO tile, B: P)
//   dK^T += Q^T dS   (A: transposed reads of the Q tile, B: dS)
// Q, dO, lse2 and delta tiles are double-buffered in LDS, fetched by DMA one
// tile ahead. Blocks are dispatched heaviest (earliest keys) first.
//
// Without a bias the tile runs as one software pipeline of four phases of
// 2 DPAD/16 MFMA slots each (16 at D 128; one wave per SIMD, so the schedule
// itself has to hide every latency):
//   phase 0  S, dP of query rows 0-31
//   phase 1  S, dP of rows 32-63, with the softmax of rows 0-31
//   phase 2  dV, dK of rows 0-31, with the softmax of rows 32-63
//   phase 3  dV, dK of rows 32-63
// and the LDS operand of slot i read at slot i - kBkRing into a register
// ring; scheduling fences pin the order so the compiler cannot pull the
// reads back next to their MFMAs. Unmasked and diagonal tiles run in two
// separate loops so that no tile body holds a branch.
// ---------------------------------------------------------------------------
// BIAS: 0 none, 1 = dtype T, 2 = fp32. Queries sit on accumulator rows here,
// so a lane's bias values (one key, 32 query rows) are read one element each;
// bias tiles keep the plain phase order (the 32 bias registers do not fit the
// pipeline's budget).
template <typename T, int DPAD, int BIAS>
__global__ __launch_bounds__(64 * kBkWaves) __attribute__((amdgpu_waves_per_eu(1, 1))) void
attn_bwd_dkv_mfma_kernel(BwdArgs a) {
  typedef Mfma32<T> Ops;
  typedef typename Ops::v8 v8;
  typedef TileAddr<DPAD, (int)sizeof(T)> TA;
  constexpr int KS = TA::KS, DTL = TA::DTL, CPR = TA::CPR, ROW_B = TA::ROW_B;
  constexpr int RPI = 64 / CPR;
  constexpr int NIW = kBwTile / (RPI * kBkWaves);
  constexpr int TILE_B = kBwTile * ROW_B;
  __shared__ __align__(16) char lds_q0[TILE_B];
  __shared__ __align__(16) char lds_q1[TILE_B];
  __shared__ __align__(16) char lds_o0[TILE_B];
  __shared__ __align__(16) char lds_o1[TILE_B];
  __shared__ __align__(16) float lds_l0[kBwTile];
  __shared__ __align__(16) float lds_l1[kBwTile];
  __shared__ __align__(16) float lds_d0[kBwTile];
  __shared__ __align__(16) float lds_d1[kBwTile];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  const int n_units = a.B * a.Hkv;
  const int kb = blockIdx.x / n_units;
  const int unit = blockIdx.x - kb * n_units;
  const int kvh = unit % a.Hkv;
  const int b = unit / a.Hkv;
  // This wave's first key. The pipelined path needs it wave-uniform (scalar
  // branches around branch-free tiles); the bias path keeps the per-lane copy,
  // with which its tiles allocate without spilling.
  const int key0 = kb * kBkKeys + (BIAS == 0 ? wave_s : wave) * 32;
  const int kj = key0 + l32;
  const bool key_ok = kj < a.Skv;

  v8 kop[KS], vop[KS];
  load_row_operand<T, DPAD>(kop, static_cast<const T*>(a.k) + b * a.ks[0] + (int64_t)kvh * a.ks[1] + (int64_t)kj * a.ks[2], key_ok, hh, a.D);
  load_row_operand<T, DPAD>(vop, static_cast<const T*>(a.v) + b * a.vs[0] + (int64_t)kvh * a.vs[1] + (int64_t)kj * a.vs[2], key_ok, hh, a.D);

  // Query tiles that see any key of the block: rows i >= first key - q_offset.
  const int qt0 = max(0, kb * kBkKeys - a.q_offset) / kBwTile;
  const int n_qt = (a.Sq + kBwTile - 1) / kBwTile;
  const int nq = max(0, n_qt - qt0);
  const int n_iter = nq * a.G;
  // Tiles from qt_nomask on see every key of this wave (i + q_offset >= key0 + 31).
  const int qt_nomask = max(0, key0 + 31 - a.q_offset + kBwTile - 1) / kBwTile;

  const PfLoadOffsets<NIW> qoff = tile_dma_offsets<NIW, DPAD, T>(wave, lane, a.qs[2], a.D);
  const PfLoadOffsets<NIW> ooff = tile_dma_offsets<NIW, DPAD, T>(wave, lane, a.dos[2], a.D);
  const int qbytes = a.Sq > 0 ? static_cast<int>(((int64_t)(a.Sq - 1) * a.qs[2] + a.D) * sizeof(T)) : 0;
  const int obytes = a.Sq > 0 ? static_cast<int>(((int64_t)(a.Sq - 1) * a.dos[2] + a.D) * sizeof(T)) : 0;
  const int qstep_b = static_cast<int>(kBwTile * a.qs[2] * sizeof(T));
  const int ostep_b = static_cast<int>(kBwTile * a.dos[2] * sizeof(T));
  const TA ad(lane);

  f32x16_t dk[DTL], dv[DTL];
#pragma unroll
  for (int i = 0; i < DTL; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      dk[i][r] = 0.f;
      dv[i][r] = 0.f;
    }

  auto qbuf = [&](auto p_c) __attribute__((always_inline)) -> LC_LDS char* {
    if constexpr (decltype(p_c)::value == 0) return (LC_LDS char*)lds_q0;
    else return (LC_LDS char*)lds_q1;
  };
  auto obuf = [&](auto p_c) __attribute__((always_inline)) -> LC_LDS char* {
    if constexpr (decltype(p_c)::value == 0) return (LC_LDS char*)lds_o0;
    else return (LC_LDS char*)lds_o1;
  };
  auto lbuf = [&](auto p_c) __attribute__((always_inline)) -> LC_LDS float* {
    if constexpr (decltype(p_c)::value == 0) return (LC_LDS float*)lds_l0;
    else return (LC_LDS float*)lds_l1;
  };
  auto dbuf = [&](auto p_c) __attribute__((always_inline)) -> LC_LDS float* {
    if constexpr (decltype(p_c)::value == 0) return (LC_LDS float*)lds_d0;
    else return (LC_LDS float*)lds_d1;
  };

  // Iteration it covers query tile n_qt - 1 - it / G of head g = it % G: the
  // walk runs from the last tile down, so the workgroups of one kv head that
  // run together read the same Q/dO tiles at about the same time (L2 hits),
  // and the diagonal tiles that need a mask come last.
  auto fetch = [&](int it, auto p_c) __attribute__((always_inline)) {
    const int step = it / a.G;
    const int g = it - step * a.G;
    const int qt = n_qt - 1 - step;
    const int h = kvh * a.G + g;
    const T* qb = static_cast<const T*>(a.q) + b * a.qs[0] + (int64_t)h * a.qs[1];
    const T* ob = static_cast<const T*>(a.dout) + b * a.dos[0] + (int64_t)h * a.dos[1];
    pf_dma_tile<NIW, RPI, ROW_B>(qb, qbytes, qbuf(p_c), wave_s, qoff, qt * qstep_b);
    pf_dma_tile<NIW, RPI, ROW_B>(ob, obytes, obuf(p_c), wave_s, ooff, qt * ostep_b);
    // lse2 (wave 0) and delta (wave 1) of the tile's 64 rows: one dword each.
    if (wave_s >= 2) return;
    const float* src = (wave_s == 0 ? a.lse2 : a.delta) + ((int64_t)b * a.Hq + h) * a.Sq;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(src), 0, a.Sq * 4, 0x00020000);
    LC_LDS float* dst = wave_s == 0 ? lbuf(p_c) : dbuf(p_c);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (LC_LDS void*)dst, 4, lane * 4,
                                             qt * kBwTile * 4, 0, 0);
  };

  // Bias of the tile of iteration `it`: query rows qt*64 + h2*32 + 8j + 4hh + i
  // of head g, this lane's key kj (register h2, 4j + i), loaded before the
  // next tile's DMA and consumed after the tile's S and dP products.
  float bv[2][16];
  auto load_bias = [&](int it) __attribute__((always_inline)) {
    if constexpr (BIAS != 0) {
      constexpr int besz = BIAS == 2 ? 4 : 2;
      const int step = it / a.G;
      const int g = it - step * a.G;
      const int qt = n_qt - 1 - step;
      const int h = kvh * a.G + g;
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<char*>(static_cast<const char*>(a.bias) +
                            (b * a.bs[0] + (int64_t)h * a.bs[1]) * besz),
          0,
          static_cast<int>(((int64_t)(a.Sq - 1) * a.bs[2] + (int64_t)(a.Skv - 1) * a.bs[3] + 1) *
                           besz),
          0x00020000);
      const int col_b = static_cast<int>((int64_t)kj * a.bs[3] * besz);
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = qt * kBwTile + h2 * 32 + (r >> 2) * 8 + hh * 4 + (r & 3);
          const int off = static_cast<int>((int64_t)row * a.bs[2] * besz) + col_b;
          if constexpr (BIAS == 2) {
            bv[h2][r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0));
          } else {
            const uint16_t hb = __builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0);
            bv[h2][r] = static_cast<float>(__builtin_bit_cast(T, hb));
          }
        }
    }
  };

  auto tile = [&](int qt, auto p_c, auto mask_c) __attribute__((always_inline)) {
    LC_LDS const char* ql = qbuf(p_c);
    LC_LDS const char* ol = obuf(p_c);
    LC_LDS const float* ll = lbuf(p_c);
    LC_LDS const float* dl = dbuf(p_c);
    if constexpr (BIAS != 0) {
      f32x16_t sa[2], dpa[2];
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          sa[h2][r] = 0.f;
          dpa[h2][r] = 0.f;
        }
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          sa[h2] = Ops::mma(*reinterpret_cast<LC_LDS const v8*>(ql + ad.row[s] + h2 * 32 * ROW_B),
                            kop[s], sa[h2]);
          dpa[h2] = Ops::mma(*reinterpret_cast<LC_LDS const v8*>(ol + ad.row[s] + h2 * 32 * ROW_B),
                             vop[s], dpa[h2]);
        }
      v8 pop[2][2], dsop[2][2];
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int row = h2 * 32 + j * 8 + hh * 4;
          const f32x4_t l4 = *reinterpret_cast<LC_LDS const f32x4_t*>(ll + row);
          const f32x4_t d4 = *reinterpret_cast<LC_LDS const f32x4_t*>(dl + row);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = j * 4 + i;
            float x = fmaf(sa[h2][r], a.scale_log2, -l4[i]);
            x += lc_bias_log2(bv[h2][r]);
            if constexpr (decltype(mask_c)::value) {
              // kj > qt * kBwTile + row + i + q_offset, with the lane's part
              // of the row moved to the left: one compare with a constant.
              if (h2 * 32 + j * 8 + i < kj - qt * kBwTile - hh * 4 - a.q_offset) x = -INFINITY;
            }
            const float p = lc_exp2(x);
            pop[h2][r >> 3][r & 7] = static_cast<T>(p);
            dsop[h2][r >> 3][r & 7] = static_cast<T>(p * (dpa[h2][r] - d4[i]));
          }
        }
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
        for (int jp = 0; jp < 2; ++jp)
#pragma unroll
          for (int dt = 0; dt < DTL; ++dt) {
            const int rowoff = (h2 * 32 + jp * 16) * ROW_B;
            const i16x4_t olo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (LC_LDS i16x4_t*)(ol + ad.tr[0][dt] + rowoff));
            const i16x4_t ohi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (LC_LDS i16x4_t*)(ol + ad.tr[1][dt] + rowoff));
            dv[dt] = Ops::mma(__builtin_bit_cast(v8, __builtin_shufflevector(olo, ohi, 0, 1, 2, 3, 4, 5, 6, 7)),
                              pop[h2][jp], dv[dt]);
            const i16x4_t qlo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (LC_LDS i16x4_t*)(ql + ad.tr[0][dt] + rowoff));
            const i16x4_t qhi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (LC_LDS i16x4_t*)(ql + ad.tr[1][dt] + rowoff));
            dk[dt] = Ops::mma(__builtin_bit_cast(v8, __builtin_shufflevector(qlo, qhi, 0, 1, 2, 3, 4, 5, 6, 7)),
                              dsop[h2][jp], dk[dt]);
          }
    } else {
      // S/dP accumulators of both 32-row halves, P and dS operands.
      f32x16_t acc_s[2], acc_p[2];
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          acc_s[x][r] = 0.f;
          acc_p[x][r] = 0.f;
        }
      v8 pop[2][2], dsop[2][2];
      f32x4_t l4[2][4], d4[2][4];
      auto read_rows = [&](int h2) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int row = h2 * 32 + j * 8 + hh * 4;
          l4[h2][j] = *reinterpret_cast<LC_LDS const f32x4_t*>(ll + row);
          d4[h2][j] = *reinterpret_cast<LC_LDS const f32x4_t*>(dl + row);
        }
      };
      // NPH MFMA slots per phase (2 KS for S/dP of a half = 4 DTL for its
      // dV/dK); EPS softmax elements per slot.
      constexpr int NPH = 2 * KS, EPS = 16 / NPH;
      static_assert(4 * DTL == NPH && NPH * EPS == 16, "slot table");
      // LDS operand of slot i: Q/dO rows for S/dP (even slot Q, odd dO),
      // transposed dO/Q for dV/dK (even slot dO, odd Q).
      auto operand = [&](int i) __attribute__((always_inline)) -> v8 {
        if (i < 2 * NPH) {
          const int h2 = i / NPH, s = (i % NPH) >> 1;
          LC_LDS const char* base = (i & 1) ? ol : ql;
          return *reinterpret_cast<LC_LDS const v8*>(base + ad.row[s] + h2 * 32 * ROW_B);
        }
        const int k = i - 2 * NPH;
        const int h2 = k / NPH, jp = (k % NPH) / (2 * DTL), dt = (k % (2 * DTL)) >> 1;
        LC_LDS const char* base = (k & 1) ? ql : ol;
        const int rowoff = (h2 * 32 + jp * 16) * ROW_B;
        const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LC_LDS i16x4_t*)(base + ad.tr[0][dt] + rowoff));
        const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LC_LDS i16x4_t*)(base + ad.tr[1][dt] + rowoff));
        return __builtin_bit_cast(v8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      };
      auto mfma = [&](int i, const v8& A) __attribute__((always_inline)) {
        if (i < 2 * NPH) {
          const int h2 = i / NPH, s = (i % NPH) >> 1;
          if (i & 1) acc_p[h2] = Ops::mma(A, vop[s], acc_p[h2]);
          else acc_s[h2] = Ops::mma(A, kop[s], acc_s[h2]);
          return;
        }
        const int k = i - 2 * NPH;
        const int h2 = k / NPH, jp = (k % NPH) / (2 * DTL), dt = (k % (2 * DTL)) >> 1;
        if (k & 1) dk[dt] = Ops::mma(A, dsop[h2][jp], dk[dt]);
        else dv[dt] = Ops::mma(A, pop[h2][jp], dv[dt]);
      };
      // P and dS of element r of half h2 (query row h2*32 + 8j + 4hh + i).
      auto softmax_elem = [&](int h2, int r) __attribute__((always_inline)) {
        const int j = r >> 2, i = r & 3;
        const int row = h2 * 32 + j * 8 + hh * 4;
        float x = fmaf(acc_s[h2][r], a.scale_log2, -l4[h2][j][i]);
        if constexpr (decltype(mask_c)::value) {
          // kj > qt * kBwTile + row + i + q_offset, with the lane's part of
          // the row moved to the left: one compare with a constant.
          if (h2 * 32 + j * 8 + i < kj - qt * kBwTile - hh * 4 - a.q_offset) x = -INFINITY;
        }
        const float p = lc_exp2(x);
        pop[h2][r >> 3][r & 7] = static_cast<T>(p);
        dsop[h2][r >> 3][r & 7] = static_cast<T>(p * (acc_p[h2][r] - d4[h2][j][i]));
      };
      v8 ring[kBkRing];
      read_rows(0);
#pragma unroll
      for (int i = 0; i < kBkRing; ++i) ring[i] = operand(i);
#pragma unroll
      for (int i = 0; i < 4 * NPH; ++i) {
        __builtin_amdgcn_sched_barrier(0);
        const v8 A = ring[i % kBkRing];
        mfma(i, A);
        if (i + kBkRing < 4 * NPH) ring[i % kBkRing] = operand(i + kBkRing);
        if (i == NPH) read_rows(1);
        const int ph = i / NPH, e0 = (i % NPH) * EPS;
        if (ph == 1 || ph == 2) {
#pragma unroll
          for (int e = 0; e < EPS; ++e) softmax_elem(ph - 1, e0 + e);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // MASK: false / true for tiles known to be unmasked / on the diagonal,
  // kRuntimeMask to pick per tile (the bias path).
  auto iteration = [&](int it, auto par_c, auto mask_c) __attribute__((always_inline)) {
    constexpr auto other = std::integral_constant<int, decltype(par_c)::value ^ 1>{};
    const int qt = n_qt - 1 - it / a.G;
    if constexpr (decltype(mask_c)::value == kRuntimeMask) {
      if (key0 < a.Skv) load_bias(it);
      if (it + 1 < n_iter) fetch(it + 1, other);
      if (key0 < a.Skv) {
        if (qt >= qt_nomask)
          tile(qt, par_c, std::false_type{});
        else
          tile(qt, par_c, std::true_type{});
      }
    } else {
      if (it + 1 < n_iter) fetch(it + 1, other);
      tile(qt, par_c, mask_c);
    }
    pf_barrier<true>();
  };
  // Iterations [begin, end) with buffer parity it & 1.
  auto run = [&](int begin, int end, auto mask_c) __attribute__((always_inline)) {
    int it = begin;
    if (it < end && (it & 1)) {
      iteration(it, std::integral_constant<int, 1>{}, mask_c);
      ++it;
    }
    for (; it + 1 < end; it += 2) {
      iteration(it, std::integral_constant<int, 0>{}, mask_c);
      iteration(it + 1, std::integral_constant<int, 1>{}, mask_c);
    }
    if (it < end) iteration(it, std::integral_constant<int, 0>{}, mask_c);
  };

  if (n_iter > 0) fetch(0, std::integral_constant<int, 0>{});
  pf_barrier<true>();
  if constexpr (BIAS != 0) {
    run(0, n_iter, std::integral_constant<int, kRuntimeMask>{});
  } else {
    // Waves whose keys all lie past Skv run the tiles on zero K/V operands and
    // store nothing; every wave passes the same barriers.
    const int n_nomask = min(n_iter, max(0, n_qt - qt_nomask) * a.G);
    run(0, n_nomask, std::false_type{});
    run(n_nomask, n_iter, std::true_type{});
  }

  if (!key_ok) return;
  store_transposed<T, DTL>(static_cast<T*>(a.dk) + b * a.dks[0] + (int64_t)kvh * a.dks[1] +
                               (int64_t)kj * a.dks[2],
                           dk, a.scale, hh, a.D);
  store_transposed<T, DTL>(static_cast<T*>(a.dv) + b * a.dvs[0] + (int64_t)kvh * a.dvs[1] +
                               (int64_t)kj * a.dvs[2],
                           dv, 1.0f, hh, a.D);
}

static int gcd_int(int x, int y) {
  while (y) {
    const int t = x % y;
    x = y;
    y = t;
  }
  return x;
}

template <typename T, int BIAS>
void launch_dq_mfma(const BwdArgs& a, unsigned nwg, int hw, int n_rbg, hipStream_t st) {
  if (a.D <= 64)
    attn_bwd_dq_mfma_kernel<T, 64, BIAS><<<nwg, 64 * kBwWaves, 0, st>>>(a, hw, n_rbg);
  else
    attn_bwd_dq_mfma_kernel<T, 128, BIAS><<<nwg, 64 * kBwWaves, 0, st>>>(a, hw, n_rbg);
}

template <typename T, int BIAS>
void launch_dkv_mfma(const BwdArgs& a, unsigned nwg, hipStream_t st) {
  if (a.D <= 64)
    attn_bwd_dkv_mfma_kernel<T, 64, BIAS><<<nwg, 64 * kBkWaves, 0, st>>>(a);
  else
    attn_bwd_dkv_mfma_kernel<T, 128, BIAS><<<nwg, 64 * kBkWaves, 0, st>>>(a);
}

template <typename T>
int launch_bwd_mfma(const BwdArgs& a, hipStream_t st) {
  const int hw = gcd_int(a.G, kBwWaves);
  const int rbw = kBwWaves / hw;
  const int n_rb = (a.Sq + kBwRows - 1) / kBwRows;
  const int n_rbg = (n_rb + rbw - 1) / rbw;
  const int64_t nwg_q = (int64_t)n_rbg * a.Hkv * (a.G / hw) * a.B;
  const int n_kb = (a.Skv + kBkKeys - 1) / kBkKeys;
  const int64_t nwg_k = (int64_t)n_kb * a.Hkv * a.B;
  LC_REQUIRE(nwg_q < (1LL << 31) && nwg_k < (1LL << 31), "lc_prefill_attn_bwd: grid too large");
  const int bias = a.bias == nullptr ? 0 : (a.bias_dtype == LC_DTYPE_F32 ? 2 : 1);
  if (nwg_q > 0) {
    if (bias == 0)
      launch_dq_mfma<T, 0>(a, (unsigned)nwg_q, hw, n_rbg, st);
    else if (bias == 1)
      launch_dq_mfma<T, 1>(a, (unsigned)nwg_q, hw, n_rbg, st);
    else
      launch_dq_mfma<T, 2>(a, (unsigned)nwg_q, hw, n_rbg, st);
  }
  if (nwg_k > 0) {
    if (bias == 0)
      launch_dkv_mfma<T, 0>(a, (unsigned)nwg_k, st);
    else if (bias == 1)
      launch_dkv_mfma<T, 1>(a, (unsigned)nwg_k, st);
    else
      launch_dkv_mfma<T, 2>(a, (unsigned)nwg_k, st);
  }
  return lc_check_launch("lc_prefill_attn_bwd (mfma)");
}

template <typename T>
int launch_delta(const void* o, const int64_t* o_strides, const BwdArgs& a, float* delta,
                 float* lse2, hipStream_t st) {
  const int64_t rows = (int64_t)a.B * a.Hq * a.Sq;
  const int64_t blocks = lc_cdiv(rows * 16, 256);
  LC_REQUIRE(blocks < (1LL << 31), "lc_prefill_attn_bwd: problem too large");
  if (blocks == 0) return LC_OK;
  bool vec = !std::is_same<T, float>::value && a.D % 8 == 0 && a.D <= 128 &&
             lc_aligned(o, 16) && lc_aligned(a.dout, 16);
  for (int i = 0; i < 3; ++i) vec = vec && o_strides[i] % 8 == 0 && a.dos[i] % 8 == 0;
  auto kern = vec ? attn_bwd_delta_kernel<T, true> : attn_bwd_delta_kernel<T, false>;
  kern<<<(unsigned)blocks, 256, 0, st>>>(
      static_cast<const T*>(o), static_cast<const T*>(a.dout), a.lse, delta, lse2, o_strides[0],
      o_strides[1], o_strides[2], a.dos[0], a.dos[1], a.dos[2], a.Hq, a.Sq, a.D, rows);
  return lc_check_launch("lc_prefill_attn_bwd (delta)");
}

template <typename T>
int run_bwd(const void* o, const int64_t* o_strides, BwdArgs a, float* delta, float* lse2,
            bool mfma, hipStream_t st) {
  a.delta = delta;
  a.lse2 = lse2;
  a.o = o;
  for (int i = 0; i < 4; ++i) a.os[i] = o_strides[i];
  if constexpr (!std::is_same<T, float>::value) {
    // The dQ kernel forms delta and lse2 for every query row (an empty query
    // side needs neither).
    if (mfma) return launch_bwd_mfma<T>(a, st);
  }
  int rc = launch_delta<T>(o, o_strides, a, delta, lse2, st);
  if (rc != LC_OK) return rc;
  return launch_bwd_generic<T>(a, st);
}

}  // namespace

extern "C" {

int64_t lc_prefill_attn_bwd_workspace_bytes(int64_t B, int64_t Hq, int64_t Sq) {
  if (B < 0 || Hq < 0 || Sq < 0) return -1;
  return 2 * (((B * Hq * Sq * 4) + 255) / 256 * 256);
}

int lc_prefill_attn_bwd(const void* q, const void* k, const void* v, const void* o,
                        const float* lse, const void* dout, void* dq, void* dk, void* dv,
                        int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Skv, int64_t D,
                        const int64_t* q_strides, const int64_t* k_strides,
                        const int64_t* v_strides, const int64_t* o_strides,
                        const int64_t* do_strides, const int64_t* dq_strides,
                        const int64_t* dk_strides, const int64_t* dv_strides, int64_t q_offset,
                        const void* bias, const int64_t* bias_strides, int bias_dtype,
                        float scale, void* workspace, int64_t workspace_bytes, int dtype,
                        void* stream) {
  LC_REQUIRE(q_strides && k_strides && v_strides && o_strides && do_strides && dq_strides &&
                 dk_strides && dv_strides,
             "lc_prefill_attn_bwd: null stride array");
  LC_REQUIRE(B >= 0 && B < 65536 && Sq >= 0 && Skv >= 0, "lc_prefill_attn_bwd: bad shape");
  // Pointers of empty tensors may be null (with Sq == 0, dk and dv are zeroed).
  LC_REQUIRE((q && o && lse && dout && dq) || B * Sq == 0,
             "lc_prefill_attn_bwd: null query-side pointer");
  LC_REQUIRE((k && v && dk && dv) || B * Skv == 0, "lc_prefill_attn_bwd: null key-side pointer");
  LC_REQUIRE(Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq < 65536,
             "lc_prefill_attn_bwd: n_heads (%lld) must be a multiple of n_kv_heads (%lld)",
             (long long)Hq, (long long)Hkv);
  LC_REQUIRE(D > 0 && D <= 256, "lc_prefill_attn_bwd: head_dim %lld not in [1, 256]",
             (long long)D);
  LC_REQUIRE(q_offset >= 0 && Sq < (1LL << 31) && Skv < (1LL << 31) && q_offset < (1LL << 30),
             "lc_prefill_attn_bwd: bad q_offset or sequence too long");
  LC_REQUIRE(q_strides[3] == 1 && k_strides[3] == 1 && v_strides[3] == 1 && o_strides[3] == 1 &&
                 do_strides[3] == 1 && dq_strides[3] == 1 && dk_strides[3] == 1 &&
                 dv_strides[3] == 1,
             "lc_prefill_attn_bwd: head_dim stride must be 1");
  LC_REQUIRE(bias == nullptr || bias_strides != nullptr,
             "lc_prefill_attn_bwd: bias without bias_strides");
  LC_REQUIRE(bias == nullptr || bias_dtype == LC_DTYPE_F32 || bias_dtype == dtype,
             "lc_prefill_attn_bwd: bias dtype must be fp32 or the dtype of q");
  if (bias != nullptr)
    for (int i = 0; i < 4; ++i)
      LC_REQUIRE(bias_strides[i] >= 0, "lc_prefill_attn_bwd: negative bias stride");
  const int64_t need = lc_prefill_attn_bwd_workspace_bytes(B, Hq, Sq);
  LC_REQUIRE(workspace_bytes >= need, "lc_prefill_attn_bwd: workspace %lld < %lld bytes",
             (long long)workspace_bytes, (long long)need);
  LC_REQUIRE(workspace || need == 0, "lc_prefill_attn_bwd: null workspace");
  LC_REQUIRE(lc_aligned(workspace, 16), "lc_prefill_attn_bwd: workspace not 16-byte aligned");
  if (B == 0 || (Sq == 0 && Skv == 0)) return LC_OK;

  BwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.dout = dout;
  a.lse = lse;
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  for (int i = 0; i < 4; ++i) {
    a.qs[i] = q_strides[i];
    a.ks[i] = k_strides[i];
    a.vs[i] = v_strides[i];
    a.dos[i] = do_strides[i];
    a.dqs[i] = dq_strides[i];
    a.dks[i] = dk_strides[i];
    a.dvs[i] = dv_strides[i];
  }
  a.B = (int)B;
  a.Hq = (int)Hq;
  a.Hkv = (int)Hkv;
  a.G = (int)(Hq / Hkv);
  a.Sq = (int)Sq;
  a.Skv = (int)Skv;
  a.D = (int)D;
  a.q_offset = (int)q_offset;
  a.scale = scale;
  a.scale_log2 = scale * kLog2e;
  a.bias = Skv > 0 ? bias : nullptr;
  a.bias_dtype = bias_dtype;
  if (bias != nullptr)
    for (int i = 0; i < 4; ++i) a.bs[i] = bias_strides[i];
  float* delta = static_cast<float*>(workspace);
  float* lse2 = delta + need / 8;
  const int64_t esz = lc_dtype_size(dtype);
  bool mfma = (dtype == LC_DTYPE_BF16 || dtype == LC_DTYPE_F16) && D % 8 == 0 && D <= 128;
  for (const void* p : {q, k, v, o, dout, (const void*)dq, (const void*)dk, (const void*)dv}) mfma = mfma && lc_aligned(p, 16);
  for (int i = 0; i < 3; ++i)
    mfma = mfma && q_strides[i] % 8 == 0 && k_strides[i] % 8 == 0 && v_strides[i] % 8 == 0 &&
           o_strides[i] % 8 == 0 && do_strides[i] % 8 == 0 && dq_strides[i] % 8 == 0 &&
           dk_strides[i] % 8 == 0 && dv_strides[i] % 8 == 0;
  // Buffer descriptors cover one head's rows with 32-bit byte offsets.
  mfma = mfma && (Skv * k_strides[2] + D) * esz < (1LL << 31) &&
         (Skv * v_strides[2] + D) * esz < (1LL << 31) &&
         (Sq * q_strides[2] + D) * esz < (1LL << 31) &&
         (Sq * do_strides[2] + D) * esz < (1LL << 31) && Sq * 4 < (1LL << 31);
  if (a.bias != nullptr) {
    // One (b, head) bias slice per buffer descriptor (32-bit byte offsets over
    // rows up to Sq + 63 and keys up to Skv + 127); 4-key vector loads as in
    // the forward.
    const int64_t besz = lc_dtype_size(bias_dtype);
    const int64_t s2 = a.bs[2], s3 = a.bs[3];
    mfma = mfma && ((int64_t)(Sq + kBwTile) * s2 + (Skv + kBkKeys) * s3 + 4) * besz < (1LL << 31);
    a.bias_vec = s3 == 1 && Skv % 4 == 0 && s2 % 4 == 0 && a.bs[0] % 4 == 0 &&
                 a.bs[1] % 4 == 0 && lc_aligned(bias, 4 * besz);
  }
  hipStream_t st = lc_stream(stream);
  switch (dtype) {
    case LC_DTYPE_F32:
      return run_bwd<float>(o, o_strides, a, delta, lse2, false, st);
    case LC_DTYPE_BF16:
      return run_bwd<bf16_t>(o, o_strides, a, delta, lse2, mfma, st);
    case LC_DTYPE_F16:
      return run_bwd<f16_t>(o, o_strides, a, delta, lse2, mfma, st);
    default:
      return lc_fail(LC_EINVAL, "lc_prefill_attn_bwd: unknown dtype %d", dtype);
  }
}

}  // extern "C"
