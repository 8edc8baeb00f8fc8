// Causal attention forward (prefill) with native GQA and logsumexp output.
//
// Two kernels, chosen by dtype and head_dim:
//   * prefill_mfma_kernel (bf16/f16, D in {64, 128}): flash attention on
//     v_mfma_f32_16x16x32_{bf16,f16} with K/V tiles double-buffered in LDS
//     (prefill_mfma.inc).
//   * prefill_generic_kernel (everything else, incl. fp32): one lane per query
//     row, fp32 FMA, K/V tiles staged through LDS.
// Both compute, for query row i of (b, h) and keys j < Skv with
// j <= i + q_offset: o = softmax(q.k_j * scale) v, lse = ln-sum-exp.
#include <math.h>

#include "lc_common.h"

namespace {

struct PrefillArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  int64_t qs[4], ks[4], vs[4], os[4];
  int B, Hq, Hkv, G, Sq, Skv, D, q_offset;
  float scale_log2;
};

// ---------------------------------------------------------------------------
// Generic kernel: block = one wave = 64 consecutive query rows of one (b, h).
// q row and o accumulator live in registers (DMAX floats each); K/V tiles of
// 16 keys are staged in LDS as fp32 and read as wave-uniform broadcasts.
// ---------------------------------------------------------------------------
template <typename T, int DMAX>
__global__ __launch_bounds__(64) void prefill_generic_kernel(PrefillArgs a) {
  constexpr int KT = 16;
  __shared__ float ks[KT][DMAX];
  __shared__ float vs[KT][DMAX];
  const int lane = threadIdx.x;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int i = blockIdx.x * 64 + lane;
  const int kvh = h / a.G;
  const bool row_ok = i < a.Sq;
  const T* qp = static_cast<const T*>(a.q) + b * a.qs[0] + h * a.qs[1] + (int64_t)i * a.qs[2];
  const T* kp = static_cast<const T*>(a.k) + b * a.ks[0] + kvh * a.ks[1];
  const T* vp = static_cast<const T*>(a.v) + b * a.vs[0] + kvh * a.vs[1];

  float qr[DMAX], acc[DMAX];
#pragma unroll
  for (int d = 0; d < DMAX; ++d) {
    qr[d] = (row_ok && d < a.D) ? lc_to_f32(qp[d]) : 0.f;
    acc[d] = 0.f;
  }
  // Keys visible to the last row of this tile.
  const int last_row = min(a.Sq - 1, (int)blockIdx.x * 64 + 63);
  const int kv_hi = min(a.Skv, last_row + a.q_offset + 1);
  const int my_hi = row_ok ? min(a.Skv, i + a.q_offset + 1) : 0;
  float m = -INFINITY, l = 0.f;

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
    const int jn = min(KT, my_hi - j0);
    for (int r = 0; r < jn; ++r) {
      float s = 0.f;
#pragma unroll
      for (int d = 0; d < DMAX; ++d) s = fmaf(qr[d], ks[r][d], s);
      s *= a.scale_log2;
      const float m_new = fmaxf(m, s);
      const float alpha = lc_exp2(m - m_new);
      const float p = lc_exp2(s - m_new);
      l = l * alpha + p;
#pragma unroll
      for (int d = 0; d < DMAX; ++d) acc[d] = fmaf(p, vs[r][d], acc[d] * alpha);
      m = m_new;
    }
  }
  if (!row_ok) return;
  T* op = static_cast<T*>(a.o) + b * a.os[0] + h * a.os[1] + (int64_t)i * a.os[2];
  const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
  for (int d = 0; d < DMAX; ++d)
    if (d < a.D) op[d] = lc_from_f32<T>(acc[d] * inv);
  if (a.lse != nullptr)
    a.lse[((int64_t)b * a.Hq + h) * a.Sq + i] = l > 0.f ? (m + lc_log2(l)) * kLn2 : -INFINITY;
}

template <typename T>
int launch_generic(const PrefillArgs& a, hipStream_t st) {
  dim3 grid((a.Sq + 63) / 64, a.Hq, a.B);
  if (a.D <= 32)
    prefill_generic_kernel<T, 32><<<grid, 64, 0, st>>>(a);
  else if (a.D <= 64)
    prefill_generic_kernel<T, 64><<<grid, 64, 0, st>>>(a);
  else if (a.D <= 128)
    prefill_generic_kernel<T, 128><<<grid, 64, 0, st>>>(a);
  else
    prefill_generic_kernel<T, 256><<<grid, 64, 0, st>>>(a);
  return lc_check_launch("lc_prefill_attn_fwd (generic)");
}

}  // namespace

extern "C" {

int lc_prefill_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                        int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Skv, int64_t D,
                        const int64_t* q_strides, const int64_t* k_strides,
                        const int64_t* v_strides, const int64_t* o_strides, int64_t q_offset,
                        float scale, int dtype, void* stream) {
  LC_REQUIRE(q && k && v && o && q_strides && k_strides && v_strides && o_strides,
             "lc_prefill_attn_fwd: null pointer");
  LC_REQUIRE(B >= 0 && B < 65536 && Sq >= 0 && Skv >= 0, "lc_prefill_attn_fwd: bad shape");
  LC_REQUIRE(Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Hq < 65536,
             "lc_prefill_attn_fwd: n_heads (%lld) must be a multiple of n_kv_heads (%lld)",
             (long long)Hq, (long long)Hkv);
  LC_REQUIRE(D > 0 && D <= 256, "lc_prefill_attn_fwd: head_dim %lld not in [1, 256]",
             (long long)D);
  LC_REQUIRE(q_offset >= 0, "lc_prefill_attn_fwd: q_offset must be >= 0");
  LC_REQUIRE(Sq < (1LL << 31) && Skv < (1LL << 31) && q_offset < (1LL << 30),
             "lc_prefill_attn_fwd: sequence too long");
  LC_REQUIRE(q_strides[3] == 1 && k_strides[3] == 1 && v_strides[3] == 1 && o_strides[3] == 1,
             "lc_prefill_attn_fwd: head_dim stride must be 1");
  if (B == 0 || Sq == 0) return LC_OK;

  PrefillArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.lse = lse;
  for (int i = 0; i < 4; ++i) {
    a.qs[i] = q_strides[i];
    a.ks[i] = k_strides[i];
    a.vs[i] = v_strides[i];
    a.os[i] = o_strides[i];
  }
  a.B = (int)B;
  a.Hq = (int)Hq;
  a.Hkv = (int)Hkv;
  a.G = (int)(Hq / Hkv);
  a.Sq = (int)Sq;
  a.Skv = (int)Skv;
  a.D = (int)D;
  a.q_offset = (int)q_offset;
  a.scale_log2 = scale * kLog2e;
  hipStream_t st = lc_stream(stream);
  switch (dtype) {
    case LC_DTYPE_F32:
      return launch_generic<float>(a, st);
    case LC_DTYPE_BF16:
      return launch_generic<bf16_t>(a, st);
    case LC_DTYPE_F16:
      return launch_generic<f16_t>(a, st);
    default:
      return lc_fail(LC_EINVAL, "lc_prefill_attn_fwd: unknown dtype %d", dtype);
  }
}

}  // extern "C"
