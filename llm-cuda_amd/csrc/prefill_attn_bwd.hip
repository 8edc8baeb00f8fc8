// Causal attention backward (dQ, dK, dV) with native GQA, no atomics.
//
// Given the forward's output O and natural-log logsumexp L, and dO:
//   delta_i = sum_d dO_id O_id                      (attn_bwd_delta_kernel)
//   P_ij    = exp(s_ij - L_i),  s_ij = q_i.k_j * scale (keys j <= i + q_offset)
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
  void* dq;
  void* dk;
  void* dv;
  int64_t qs[4], ks[4], vs[4], dos[4], dqs[4], dks[4], dvs[4];
  int B, Hq, Hkv, G, Sq, Skv, D, q_offset;
  float scale, scale_log2;
};

// ---------------------------------------------------------------------------
// delta = rowsum(dO * O) in fp32: 16 lanes per row.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void attn_bwd_delta_kernel(const T* __restrict__ o,
                                                             const T* __restrict__ dout,
                                                             float* __restrict__ delta,
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
    for (int d = sub; d < D; d += 16) acc = fmaf(lc_to_f32(orow[d]), lc_to_f32(drow[d]), acc);
  }
#pragma unroll
  for (int w = 8; w >= 1; w >>= 1) acc += __shfl_xor(acc, w, 64);
  if (row < rows && sub == 0) delta[row] = acc;
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
      const float p = lc_exp2(s * a.scale_log2 - lse2);
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
        const float p = lc_exp2(s * a.scale_log2 - lse_t[r]);
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

template <typename T>
int launch_delta(const void* o, const int64_t* o_strides, const BwdArgs& a, float* delta,
                 hipStream_t st) {
  const int64_t rows = (int64_t)a.B * a.Hq * a.Sq;
  const int64_t blocks = lc_cdiv(rows * 16, 256);
  LC_REQUIRE(blocks < (1LL << 31), "lc_prefill_attn_bwd: problem too large");
  if (blocks == 0) return LC_OK;
  attn_bwd_delta_kernel<T><<<(unsigned)blocks, 256, 0, st>>>(
      static_cast<const T*>(o), static_cast<const T*>(a.dout), delta, o_strides[0],
      o_strides[1], o_strides[2], a.dos[0], a.dos[1], a.dos[2], a.Hq, a.Sq, a.D, rows);
  return lc_check_launch("lc_prefill_attn_bwd (delta)");
}

template <typename T>
int run_bwd(const void* o, const int64_t* o_strides, BwdArgs a, float* delta, hipStream_t st) {
  int rc = launch_delta<T>(o, o_strides, a, delta, st);
  if (rc != LC_OK) return rc;
  a.delta = delta;
  return launch_bwd_generic<T>(a, st);
}

}  // namespace

extern "C" {

int64_t lc_prefill_attn_bwd_workspace_bytes(int64_t B, int64_t Hq, int64_t Sq) {
  if (B < 0 || Hq < 0 || Sq < 0) return -1;
  return ((B * Hq * Sq * 4) + 255) / 256 * 256;
}

int lc_prefill_attn_bwd(const void* q, const void* k, const void* v, const void* o,
                        const float* lse, const void* dout, void* dq, void* dk, void* dv,
                        int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Skv, int64_t D,
                        const int64_t* q_strides, const int64_t* k_strides,
                        const int64_t* v_strides, const int64_t* o_strides,
                        const int64_t* do_strides, const int64_t* dq_strides,
                        const int64_t* dk_strides, const int64_t* dv_strides, int64_t q_offset,
                        float scale, void* workspace, int64_t workspace_bytes, int dtype,
                        void* stream) {
  LC_REQUIRE(q && k && v && o && lse && dout && dq && dk && dv && workspace,
             "lc_prefill_attn_bwd: null pointer");
  LC_REQUIRE(q_strides && k_strides && v_strides && o_strides && do_strides && dq_strides &&
                 dk_strides && dv_strides,
             "lc_prefill_attn_bwd: null stride array");
  LC_REQUIRE(B >= 0 && B < 65536 && Sq >= 0 && Skv >= 0, "lc_prefill_attn_bwd: bad shape");
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
  const int64_t need = lc_prefill_attn_bwd_workspace_bytes(B, Hq, Sq);
  LC_REQUIRE(workspace_bytes >= need, "lc_prefill_attn_bwd: workspace %lld < %lld bytes",
             (long long)workspace_bytes, (long long)need);
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
  float* delta = static_cast<float*>(workspace);
  hipStream_t st = lc_stream(stream);
  switch (dtype) {
    case LC_DTYPE_F32:
      return run_bwd<float>(o, o_strides, a, delta, st);
    case LC_DTYPE_BF16:
      return run_bwd<bf16_t>(o, o_strides, a, delta, st);
    case LC_DTYPE_F16:
      return run_bwd<f16_t>(o, o_strides, a, delta, st);
    default:
      return lc_fail(LC_EINVAL, "lc_prefill_attn_bwd: unknown dtype %d", dtype);
  }
}

}  // extern "C"
