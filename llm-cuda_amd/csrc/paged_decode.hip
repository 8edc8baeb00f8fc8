// Split-K paged GQA flash-decode for gfx950, plus the cross-split merge.
//
// Work decomposition: one wavefront = one split = `split_tokens` consecutive
// tokens of one (sequence b, kv head, group of <= 16 query heads). All G query
// heads sharing a kv head are served by the same wave, so every K/V byte is
// read from HBM exactly once (the reference's decode kernel re-read K/V once
// per query head: kernels/triton/decode_attention.py:86-93,110-151).
//
// Per 32-token step a wave:
//   1. computes each lane's token -> (page, slot) through the block table and
//      issues 16-byte loads of its K and V row chunks straight from the page
//      pool (the next step's loads are in flight while this step computes);
//   2. S^T[16 tok x 16 heads] = K[16 tok x 32 d] * Q^T[32 d x 16 heads] on
//      v_mfma_f32_16x16x32_{bf16,f16}, D/32 MFMAs per 16 tokens;
//   3. online softmax in the exp2 domain (scale * log2 e folded into one
//      multiply), max exchanged across the 4 lanes of a head by xor-shuffles;
//   4. O^T[16 d x 16 heads] += V^T[16 d x 32 tok] * P^T[32 tok x 16 heads];
//      V^T comes from a wave-private LDS tile (row-major write, transposed
//      2-byte reads). P^T needs no data movement: the MFMA k index is mapped
//      to tokens so that the S^T accumulator registers ARE the P^T operand.
// Each split writes o/l (fp32) and its log2-domain logsumexp; the merge kernel
// combines splits with weights 2^(lse_s - lse).
#include <math.h>

#include "lc_common.h"

namespace {

struct DecodeArgs {
  const void* q;
  int64_t q_sb, q_sh;
  const void* kp;
  const void* vp;
  int64_t s_page, s_head, s_tok;
  const int32_t* bt;
  int64_t bt_stride;
  int max_pages;
  int num_pages;
  const int32_t* seq_lens;
  float* part_o;    // [B*Hq, max_splits, D]
  float* part_lse;  // [B*Hq, max_splits], log2 domain
  int B, Hq, Hkv, G, D, P, p_shift, split_tokens, max_splits, n_hgroups;
  float scale_log2;
};

__device__ __forceinline__ int seq_len_of(const DecodeArgs& a, int b) {
  int len = a.seq_lens[b];
  const int cap = a.max_pages * a.P;
  len = len < 0 ? 0 : len;
  return len > cap ? cap : len;
}

// Element offset of token `tok` of sequence b, kv head kvh; -1 if its page
// entry is invalid. Caller guarantees tok < max_pages * P.
__device__ __forceinline__ int64_t token_offset(const DecodeArgs& a, int b, int kvh, int tok) {
  int page_idx, slot;
  if (a.p_shift >= 0) {
    page_idx = tok >> a.p_shift;
    slot = tok & (a.P - 1);
  } else {
    page_idx = tok / a.P;
    slot = tok - page_idx * a.P;
  }
  const int phys = a.bt[(int64_t)b * a.bt_stride + page_idx];
  if (static_cast<unsigned>(phys) >= static_cast<unsigned>(a.num_pages)) return -1;
  return (int64_t)phys * a.s_page + (int64_t)kvh * a.s_head + (int64_t)slot * a.s_tok;
}

template <typename T>
struct MfmaOps;
template <>
struct MfmaOps<bf16_t> {
  typedef bf16x8_t v8;
  static __device__ __forceinline__ f32x4_t mma(v8 a, v8 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct MfmaOps<f16_t> {
  typedef f16x8_t v8;
  static __device__ __forceinline__ f32x4_t mma(v8 a, v8 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

constexpr int kWaves = 4;
constexpr int kStep = 32;  // tokens per MFMA step

template <typename T, int DPAD>
struct StepRegs {
  typename MfmaOps<T>::v8 k[2][DPAD / 32];
  typename MfmaOps<T>::v8 v[2][DPAD / 32];
  // Bit r of valid[gi]: token gi*16 + r of the step is live and has a valid
  // page (lanes r, r+16, r+32, r+48 load the same token, so bits 0..15 suffice).
  uint64_t valid[2];
};

template <typename T, int DPAD>
__device__ __forceinline__ void load_step(const DecodeArgs& a, const T* __restrict__ kp,
                                          const T* __restrict__ vp, int b, int kvh, int t,
                                          int t_end, int row, int q4, StepRegs<T, DPAD>& r) {
  typedef typename MfmaOps<T>::v8 v8;
#pragma unroll
  for (int gi = 0; gi < 2; ++gi) {
    const int tok = t + gi * 16 + row;
    const int64_t off = tok < t_end ? token_offset(a, b, kvh, tok) : -1;
    r.valid[gi] = __ballot(off >= 0);
#pragma unroll
    for (int s = 0; s < DPAD / 32; ++s) {
      const int d0 = s * 32 + q4 * 8;
      if (off >= 0 && d0 < a.D) {
        r.k[gi][s] = *reinterpret_cast<const v8*>(kp + off + d0);
        r.v[gi][s] = *reinterpret_cast<const v8*>(vp + off + d0);
      } else {
        r.k[gi][s] = v8{};
        r.v[gi][s] = v8{};
      }
    }
  }
}

template <typename T, int DPAD>
__global__ __launch_bounds__(64 * kWaves) void paged_decode_mfma_kernel(DecodeArgs a) {
  typedef MfmaOps<T> Ops;
  typedef typename Ops::v8 v8;
  constexpr int KS = DPAD / 32;      // MFMA k-steps over head_dim
  constexpr int DT = DPAD / 16;      // 16-row d tiles of the output
  constexpr int LROW = DPAD + 8;     // LDS row pitch (elements), 16 B pad
  extern __shared__ __align__(16) unsigned char smem_raw[];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int split = blockIdx.x * kWaves + wave;
  const int kvh = blockIdx.y / a.n_hgroups;
  const int hg = blockIdx.y - kvh * a.n_hgroups;
  const int b = blockIdx.z;
  if (split >= a.max_splits) return;
  const int len = seq_len_of(a, b);
  const int t_begin = split * a.split_tokens;
  if (t_begin >= len) return;
  const int t_end = min(len, t_begin + a.split_tokens);

  const int col = lane & 15;  // query head within the 16-wide tile
  const int q4 = lane >> 4;   // 0..3
  const int g = hg * 16 + col;
  const bool head_ok = g < a.G;
  const int h = kvh * a.G + g;

  T* lds = reinterpret_cast<T*>(smem_raw) + wave * (kStep * LROW);
  const T* kp = static_cast<const T*>(a.kp);
  const T* vp = static_cast<const T*>(a.vp);

  // Q^T operand: lane holds q[h, s*32 + q4*8 .. +8] for every k-step s.
  v8 qop[KS];
  {
    const T* qh = static_cast<const T*>(a.q) + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int d0 = s * 32 + q4 * 8;
      qop[s] = (head_ok && d0 < a.D) ? *reinterpret_cast<const v8*>(qh + d0) : v8{};
    }
  }

  f32x4_t o[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) o[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;
  float l_lane = 0.f;

  auto compute_step = [&](const StepRegs<T, DPAD>& r) {
    // Scores S^T: rows = tokens (q4*4 + i within each 16-token group), cols = heads.
    f32x4_t sacc[2];
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      sacc[gi] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) sacc[gi] = Ops::mma(r.k[gi][s], qop[s], sacc[gi]);
    }
    // V tile -> LDS (row-major [32 tok][LROW]) while the MFMAs drain.
#pragma unroll
    for (int gi = 0; gi < 2; ++gi)
#pragma unroll
      for (int s = 0; s < KS; ++s)
        *reinterpret_cast<v8*>(lds + (gi * 16 + col) * LROW + s * 32 + q4 * 8) = r.v[gi][s];

    float sc[2][4];
    float mx = -INFINITY;
#pragma unroll
    for (int gi = 0; gi < 2; ++gi)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool live = (r.valid[gi] >> (q4 * 4 + i)) & 1;
        const float v = sacc[gi][i] * a.scale_log2;
        sc[gi][i] = live ? v : -INFINITY;
        mx = fmaxf(mx, sc[gi][i]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = lc_exp2(m_run - m_use);
    m_run = m_new;

    float psum = 0.f;
    v8 pop;
#pragma unroll
    for (int gi = 0; gi < 2; ++gi)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = lc_exp2(sc[gi][i] - m_use);
        psum += p;
        pop[gi * 4 + i] = static_cast<T>(p);
      }
    l_lane = l_lane * alpha + psum;

    lc_wave_lds_fence();
    // V^T operand for d tile dt: lane holds V[tok(q4, j)][dt*16 + col], with
    // tok(q4, j) = q4*4 + j (j < 4) or 16 + q4*4 + (j - 4) (j >= 4).
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      v8 vop;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int tr = (j < 4) ? (q4 * 4 + j) : (16 + q4 * 4 + (j - 4));
        vop[j] = lds[tr * LROW + dt * 16 + col];
      }
      f32x4_t acc = o[dt];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] *= alpha;
      o[dt] = Ops::mma(vop, pop, acc);
    }
    lc_wave_lds_fence();
  };

  StepRegs<T, DPAD> ra, rb;
  load_step<T, DPAD>(a, kp, vp, b, kvh, t_begin, t_end, col, q4, ra);
  int t = t_begin;
  while (true) {
    const bool more_a = t + kStep < t_end;
    if (more_a) load_step<T, DPAD>(a, kp, vp, b, kvh, t + kStep, t_end, col, q4, rb);
    compute_step(ra);
    if (!more_a) break;
    t += kStep;
    const bool more_b = t + kStep < t_end;
    if (more_b) load_step<T, DPAD>(a, kp, vp, b, kvh, t + kStep, t_end, col, q4, ra);
    compute_step(rb);
    if (!more_b) break;
    t += kStep;
  }

  // Finalise this split: l summed over the 4 lanes of each head.
  float l_tot = l_lane + __shfl_xor(l_lane, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  if (!head_ok) return;
  const int64_t pidx = ((int64_t)b * a.Hq + h) * a.max_splits + split;
  const float inv_l = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  float* po = a.part_o + pidx * a.D;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    const int d0 = dt * 16 + q4 * 4;
    if (d0 < a.D) {
      f32x4_t w = o[dt];
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] *= inv_l;
      if (d0 + 4 <= a.D) {
        *reinterpret_cast<f32x4_t*>(po + d0) = w;
      } else {
        for (int i = 0; i < 4 && d0 + i < a.D; ++i) po[d0 + i] = w[i];
      }
    }
  }
  if (q4 == 0) a.part_lse[pidx] = l_tot > 0.f ? m_run + lc_log2(l_tot) : -INFINITY;
}

// Generic decode: one wave per (b, query head, split), lanes across head_dim,
// one token at a time (wave-reduced dot product). Any dtype, any D <= 256,
// any element strides. Same partial-output contract as the MFMA kernel.
template <typename T>
__global__ __launch_bounds__(64) void paged_decode_generic_kernel(DecodeArgs a) {
  const int lane = threadIdx.x;
  const int split = blockIdx.x;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int len = seq_len_of(a, b);
  const int t_begin = split * a.split_tokens;
  if (t_begin >= len) return;
  const int t_end = min(len, t_begin + a.split_tokens);
  const int kvh = h / a.G;
  const T* kp = static_cast<const T*>(a.kp);
  const T* vp = static_cast<const T*>(a.vp);
  const T* qh = static_cast<const T*>(a.q) + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh;

  float qv[4], acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + 64 * i;
    qv[i] = d < a.D ? lc_to_f32(qh[d]) : 0.f;
    acc[i] = 0.f;
  }
  float m_run = -INFINITY, l_run = 0.f;
  for (int t = t_begin; t < t_end; ++t) {
    const int64_t off = token_offset(a, b, kvh, t);
    if (off < 0) continue;  // uniform across the wave
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = lane + 64 * i;
      if (d < a.D) dot = fmaf(qv[i], lc_to_f32(kp[off + d]), dot);
    }
    const float s = lc_wave_sum(dot) * a.scale_log2;
    const float m_new = fmaxf(m_run, s);
    const float alpha = lc_exp2(m_run - m_new);
    const float p = lc_exp2(s - m_new);
    l_run = l_run * alpha + p;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = lane + 64 * i;
      const float vv = d < a.D ? lc_to_f32(vp[off + d]) : 0.f;
      acc[i] = fmaf(p, vv, acc[i] * alpha);
    }
    m_run = m_new;
  }
  const int64_t pidx = ((int64_t)b * a.Hq + h) * a.max_splits + split;
  const float inv_l = l_run > 0.f ? 1.0f / l_run : 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + 64 * i;
    if (d < a.D) a.part_o[pidx * a.D + d] = acc[i] * inv_l;
  }
  if (lane == 0) a.part_lse[pidx] = l_run > 0.f ? m_run + lc_log2(l_run) : -INFINITY;
}

// Cross-split merge: one wave per (b, h). lse = log2-sum-exp2 of split lses,
// out = sum_s 2^(lse_s - lse) * o_s. Writes the natural-log lse.
template <typename T>
__global__ __launch_bounds__(64) void decode_merge_kernel(DecodeArgs a, T* __restrict__ out,
                                                          int64_t o_sb, int64_t o_sh,
                                                          float* __restrict__ lse_out) {
  const int lane = threadIdx.x;
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int len = seq_len_of(a, b);
  const int nsplit = (len + a.split_tokens - 1) / a.split_tokens;
  const int64_t pbase = ((int64_t)b * a.Hq + h) * a.max_splits;
  T* oh = out + (int64_t)b * o_sb + (int64_t)h * o_sh;

  float mx = -INFINITY;
  for (int s = lane; s < nsplit; s += 64) mx = fmaxf(mx, a.part_lse[pbase + s]);
  mx = lc_wave_max(mx);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  float wsum = 0.f;
  if (mx != -INFINITY) {
    for (int s = 0; s < nsplit; ++s) {
      const float ls = a.part_lse[pbase + s];
      const float w = lc_exp2(ls - mx);
      wsum += w;
      const float* po = a.part_o + (pbase + s) * a.D;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = lane + 64 * i;
        if (d < a.D) acc[i] = fmaf(w, po[d], acc[i]);
      }
    }
  }
  const float inv = wsum > 0.f ? 1.0f / wsum : 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + 64 * i;
    if (d < a.D) oh[d] = lc_from_f32<T>(acc[i] * inv);
  }
  if (lse_out != nullptr && lane == 0)
    lse_out[(int64_t)b * a.Hq + h] = wsum > 0.f ? (mx + lc_log2(wsum)) * kLn2 : -INFINITY;
}

template <typename T, int DPAD>
int launch_mfma(const DecodeArgs& a, hipStream_t st) {
  const size_t lds = (size_t)kWaves * kStep * (DPAD + 8) * sizeof(T);
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&paged_decode_mfma_kernel<T, DPAD>),
        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess)
      return lc_fail(static_cast<int>(e), "lc_paged_decode_fwd: LDS attribute: %s",
                     hipGetErrorString(e));
    attr_set = true;
  }
  dim3 grid((a.max_splits + kWaves - 1) / kWaves, a.Hkv * a.n_hgroups, a.B);
  paged_decode_mfma_kernel<T, DPAD><<<grid, 64 * kWaves, lds, st>>>(a);
  return lc_check_launch("lc_paged_decode_fwd (mfma)");
}

template <typename T>
int launch_decode(DecodeArgs a, void* out, int64_t o_sb, int64_t o_sh, float* lse, bool mfma,
                  hipStream_t st) {
  int rc = LC_OK;
  if (mfma) {
    if constexpr (sizeof(T) == 2) {
      a.n_hgroups = (a.G + 15) / 16;
      if (a.D <= 64)
        rc = launch_mfma<T, 64>(a, st);
      else if (a.D <= 128)
        rc = launch_mfma<T, 128>(a, st);
      else
        rc = launch_mfma<T, 256>(a, st);
    }
  } else {
    dim3 grid(a.max_splits, a.Hq, a.B);
    paged_decode_generic_kernel<T><<<grid, 64, 0, st>>>(a);
    rc = lc_check_launch("lc_paged_decode_fwd (generic)");
  }
  if (rc != LC_OK) return rc;
  dim3 mgrid(a.Hq, a.B);
  decode_merge_kernel<T><<<mgrid, 64, 0, st>>>(a, static_cast<T*>(out), o_sb, o_sh, lse);
  return lc_check_launch("lc_paged_decode_fwd (merge)");
}

}  // namespace

extern "C" {

int64_t lc_paged_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t D, int64_t max_splits) {
  if (B < 0 || Hq < 0 || D < 0 || max_splits < 0) return -1;
  const int64_t n = B * Hq * max_splits;
  // partial o (fp32, D per split), then partial lse (fp32), 256-byte aligned.
  const int64_t o_bytes = ((n * D * 4) + 255) / 256 * 256;
  return o_bytes + n * 4;
}

int lc_paged_decode_fwd(const void* q, int64_t q_sb, int64_t q_sh, const void* key_pages,
                        const void* value_pages, int64_t kv_s_page, int64_t kv_s_head,
                        int64_t kv_s_tok, const int32_t* block_table, int64_t bt_stride,
                        int64_t max_pages_per_seq, int64_t num_pages, const int32_t* seq_lens,
                        void* out, int64_t o_sb, int64_t o_sh, float* lse, void* workspace,
                        int64_t workspace_bytes, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                        int64_t page_size, int64_t split_tokens, int64_t max_splits, float scale,
                        int dtype, void* stream) {
  LC_REQUIRE(q && key_pages && value_pages && block_table && seq_lens && out && workspace,
             "lc_paged_decode_fwd: null pointer");
  LC_REQUIRE(B >= 0 && B < 65536, "lc_paged_decode_fwd: batch %lld out of range", (long long)B);
  LC_REQUIRE(Hq > 0 && Hkv > 0 && Hq % Hkv == 0,
             "lc_paged_decode_fwd: n_heads (%lld) must be a multiple of n_kv_heads (%lld)",
             (long long)Hq, (long long)Hkv);
  LC_REQUIRE(D > 0 && D <= 256, "lc_paged_decode_fwd: head_dim %lld not in [1, 256]",
             (long long)D);
  LC_REQUIRE(page_size > 0 && max_pages_per_seq > 0 && num_pages > 0,
             "lc_paged_decode_fwd: page_size, max_pages_per_seq and num_pages must be > 0");
  LC_REQUIRE(max_pages_per_seq * page_size < (1LL << 31) && num_pages < (1LL << 31),
             "lc_paged_decode_fwd: cache too large for 32-bit token indices");
  LC_REQUIRE(bt_stride >= max_pages_per_seq, "lc_paged_decode_fwd: bt_stride < row length");
  LC_REQUIRE(split_tokens > 0 && split_tokens % 64 == 0,
             "lc_paged_decode_fwd: split_tokens must be a positive multiple of 64");
  LC_REQUIRE(max_splits > 0 && max_splits * split_tokens >= max_pages_per_seq * page_size,
             "lc_paged_decode_fwd: max_splits * split_tokens must cover the block-table "
             "capacity (%lld tokens)",
             (long long)(max_pages_per_seq * page_size));
  const int64_t need = lc_paged_decode_workspace_bytes(B, Hq, D, max_splits);
  LC_REQUIRE(workspace_bytes >= need, "lc_paged_decode_fwd: workspace %lld < %lld bytes",
             (long long)workspace_bytes, (long long)need);
  LC_REQUIRE(lc_aligned(workspace, 256), "lc_paged_decode_fwd: workspace not 256-byte aligned");
  if (B == 0) return LC_OK;

  DecodeArgs a{};
  a.q = q;
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.kp = key_pages;
  a.vp = value_pages;
  a.s_page = kv_s_page;
  a.s_head = kv_s_head;
  a.s_tok = kv_s_tok;
  a.bt = block_table;
  a.bt_stride = bt_stride;
  a.max_pages = static_cast<int>(max_pages_per_seq);
  a.num_pages = static_cast<int>(num_pages);
  a.seq_lens = seq_lens;
  const int64_t n = B * Hq * max_splits;
  a.part_o = static_cast<float*>(workspace);
  a.part_lse = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                        ((n * D * 4) + 255) / 256 * 256);
  a.B = static_cast<int>(B);
  a.Hq = static_cast<int>(Hq);
  a.Hkv = static_cast<int>(Hkv);
  a.G = static_cast<int>(Hq / Hkv);
  a.D = static_cast<int>(D);
  a.P = static_cast<int>(page_size);
  a.p_shift = (page_size & (page_size - 1)) == 0 ? __builtin_ctzll(page_size) : -1;
  a.split_tokens = static_cast<int>(split_tokens);
  a.max_splits = static_cast<int>(max_splits);
  a.n_hgroups = 1;
  a.scale_log2 = scale * kLog2e;

  const int esz = lc_dtype_size(dtype);
  const bool half = dtype == LC_DTYPE_BF16 || dtype == LC_DTYPE_F16;
  const bool mfma = half && D % 8 == 0 && q_sb % 8 == 0 && q_sh % 8 == 0 &&
                    kv_s_page % 8 == 0 && kv_s_head % 8 == 0 && kv_s_tok % 8 == 0 &&
                    lc_aligned(q, 16) && lc_aligned(key_pages, 16) &&
                    lc_aligned(value_pages, 16);
  (void)esz;
  hipStream_t st = lc_stream(stream);
  switch (dtype) {
    case LC_DTYPE_F32:
      return launch_decode<float>(a, out, o_sb, o_sh, lse, false, st);
    case LC_DTYPE_BF16:
      return launch_decode<bf16_t>(a, out, o_sb, o_sh, lse, mfma, st);
    case LC_DTYPE_F16:
      return launch_decode<f16_t>(a, out, o_sb, o_sh, lse, mfma, st);
    default:
      return lc_fail(LC_EINVAL, "lc_paged_decode_fwd: unknown dtype %d", dtype);
  }
}

}  // extern "C"
