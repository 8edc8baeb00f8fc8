// Split-K paged GQA flash-decode for gfx950, plus the cross-split merge.
//
// Work decomposition: one wavefront (= one workgroup) = one split =
// `split_tokens` consecutive tokens of one (sequence b, kv head, group of
// <= 16 query heads). All G query heads sharing a kv head are served by the
// same wave, so every K/V byte is read from HBM exactly once (the reference's
// decode kernel re-read K/V once per query head:
// kernels/triton/decode_attention.py:86-93,110-151).
//
// Main kernel (page_size a multiple of 32), per 32-token step:
//   1. the step's K and V rows (one page, so the page id is wave-uniform) are
//      read with fully coalesced 16-byte buffer loads (16 lanes per 256-byte
//      row) carrying the non-temporal hint, into one register staging buffer;
//   2. the staging buffer is copied to wave-private LDS tiles and the NEXT
//      step's loads are issued into it at once, so they fly while this step
//      computes from LDS;
//   3. S^T[16 tok x 16 heads] = K[16 tok x 32 d] * Q^T[32 d x 16 heads] on
//      v_mfma_f32_16x16x32_{bf16,f16} (K operands via ds_read_b128);
//   4. online softmax in the exp2 domain with lazy rescaling;
//   5. O^T[16 d x 16 heads] += V^T[16 d x 32 tok] * P^T[32 tok x 16 heads];
//      V^T operands come from ds_read_b64_tr_b16 transposed LDS reads, and
//      the MFMA k index is mapped to tokens so that the S^T accumulator
//      registers ARE the P^T operand.
// Each split writes o/l (fp32) and its log2-domain logsumexp; the merge
// kernel combines splits with weights 2^(lse_s - lse). An optional additive
// bias per (sequence, query head, token) (an attention mask) is added to the
// scaled scores.
#include <math.h>

#include <mutex>

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
  // Additive bias: element (b, h, t) at bias[b*bias_sb + h*bias_sh + t] for
  // t < bias_len (tokens past bias_len get none); dtype bias_dtype; null: none.
  const void* bias;
  int64_t bias_sb, bias_sh;
  int bias_len, bias_dtype;
  // Longest-first order (ORD): a ticket that is zero at entry and left zero,
  // or null (every workgroup keeps rank = its block id); ord_static: the
  // workgroups below this block id always keep their id as rank.
  int* ord_ticket;
  int ord_static;
};

// Bias of token tok for (b, h), in the exp2 domain; 0 past bias_len.
__device__ __forceinline__ float decode_bias(const DecodeArgs& a, int b, int h, int tok) {
  return tok < a.bias_len
             ? lc_bias_log2(lc_load_bias(a.bias, b * a.bias_sb + h * a.bias_sh + tok, a.bias_dtype))
             : 0.f;
}

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

constexpr int kStep = 32;  // tokens per MFMA step
// Lazy rescaling: the running reference max m_ref only moves when a new score
// exceeds it by more than this (log2 units). Every p = 2^(s - m_ref) is then
// <= 2^8, safe in bf16/f16 and fp32; o and l share m_ref, so o / l is exact.
constexpr float kRescaleLog2 = 8.0f;
// Buffer-resource word 3 for untyped (raw) buffer loads on gfx9-family parts.
constexpr int kBufferWord3 = 0x00020000;
// Cache-policy operand of the K/V buffer loads: the non-temporal bit. Every
// K/V byte is used exactly once, and streaming it past the caches measured
// ~10% faster than default-policy loads for this access pattern.
constexpr int kLoadNT = 2;

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x8_t __attribute__((ext_vector_type(8)));
#define LC_LDS __attribute__((address_space(3)))

template <typename T, int DPAD>
struct StepRegs {
  typename MfmaOps<T>::v8 k[2][DPAD / 32];
  typename MfmaOps<T>::v8 v[2][DPAD / 32];
  // Bit r of valid[gi]: token gi*16 + r of the step is live and its page is
  // valid (lanes r, r+16, r+32, r+48 load the same token).
  uint64_t valid[2];
};

// Any page size: each lane resolves its own token's page and loads its K/V
// chunks straight into MFMA operand layout (16 tokens x 64 contiguous bytes
// per instruction).
template <typename T, int DPAD>
__device__ __forceinline__ void load_step_lane(const DecodeArgs& a, const T* __restrict__ kp,
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

// Shared tail of both MFMA kernels: QK^T of one 32-token step is done by the
// caller; this folds the scores into the running softmax state and returns
// the P^T operand. sc[gi][i] are scaled, masked scores of tokens
// gi*16 + q4*4 + i for this lane's head.
template <typename T, int DT>
__device__ __forceinline__ typename MfmaOps<T>::v8 softmax_step(float (&sc)[2][4], float& m_ref,
                                                                float& l_lane, f32x4_t (&o)[DT]) {
  typedef typename MfmaOps<T>::v8 v8;
  float mx = fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])),
                   fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  if (__ballot(mx > m_ref + kRescaleLog2)) {  // wave-uniform, rare after the first step
    const float m_new = fmaxf(m_ref, mx);
    const float alpha = m_new == -INFINITY ? 1.f : lc_exp2(m_ref - m_new);
    l_lane *= alpha;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[dt][i] *= alpha;
    m_ref = m_new;
  }
  const float m_use = m_ref == -INFINITY ? 0.f : m_ref;
  v8 pop;
#pragma unroll
  for (int gi = 0; gi < 2; ++gi)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = lc_exp2(sc[gi][i] - m_use);
      l_lane += p;
      pop[gi * 4 + i] = static_cast<T>(p);
    }
  return pop;
}

// O^T += V^T * P^T for one 32-token step from a row-major LDS V tile.
// ds_read_b64_tr_b16 semantics (per 16-lane group): lane i receives element
// i % 4 of the 8-byte chunks addressed by lanes 4e + i / 4, e = 0..3. So lane
// 4e + c points at V[token(q4, e)][dt*16 + 4c] and lane i gets the column
// {V[token(q4, e)][dt*16 + i] : e = 0..3}.
template <typename T, int DT, int LROW>
__device__ __forceinline__ void pv_step(const T* lds_v, int q4, int col,
                                        typename MfmaOps<T>::v8 pop, f32x4_t (&o)[DT]) {
  typedef typename MfmaOps<T>::v8 v8;
  const int tr_e = col >> 2, tr_c = col & 3;
  LC_LDS const short* base = (LC_LDS const short*)(lds_v);
  const int r1 = (q4 * 4 + tr_e) * LROW + 4 * tr_c;       // tokens 4*q4 .. 4*q4+3
  const int r2 = (16 + q4 * 4 + tr_e) * LROW + 4 * tr_c;  // tokens 16+4*q4 .. +3
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LC_LDS i16x4_t*)(base + r1 + dt * 16));
    const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LC_LDS i16x4_t*)(base + r2 + dt * 16));
    const i16x8_t both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    o[dt] = MfmaOps<T>::mma(__builtin_bit_cast(v8, both), pop, o[dt]);
  }
}

// Writes this split's normalised partial output and log2-domain lse.
template <int DT>
__device__ __forceinline__ void store_partial(const DecodeArgs& a, int b, int h, int split,
                                              bool head_ok, int q4, float m_ref, float l_lane,
                                              const f32x4_t (&o)[DT]) {
  float l_tot = l_lane + __shfl_xor(l_lane, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  if (!head_ok) return;
  const int64_t pidx = ((int64_t)b * a.Hq + h) * a.max_splits + split;
  const float inv_l = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  float* po = a.part_o + pidx * a.D;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    const int d0 = dt * 16 + q4 * 4;
    if (d0 < a.D) {  // D % 8 == 0 on the MFMA path: 4-float groups are whole
      f32x4_t w = o[dt];
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] *= inv_l;
      *reinterpret_cast<f32x4_t*>(po + d0) = w;
    }
  }
  if (q4 == 0) a.part_lse[pidx] = l_tot > 0.f ? m_ref + lc_log2(l_tot) : -INFINITY;
}

// Query operands of head h (all zero for a padding head or past head_dim).
// The loads are unconditional (a padding head or chunk reads head h_safe's
// chunk 0 instead) and zeroed afterwards, so no branch separates them.
template <typename T, int DPAD>
__device__ __forceinline__ void load_q(const DecodeArgs& a, int b, int h, int h_safe,
                                       bool head_ok, int q4,
                                       typename MfmaOps<T>::v8 (&qop)[DPAD / 32]) {
  typedef typename MfmaOps<T>::v8 v8;
  const T* qh = static_cast<const T*>(a.q) + (int64_t)b * a.q_sb +
                (int64_t)(head_ok ? h : h_safe) * a.q_sh;
#pragma unroll
  for (int s = 0; s < DPAD / 32; ++s) {
    const int d0 = s * 32 + q4 * 8;
    const bool ok = head_ok && d0 < a.D;
    const v8 x = *reinterpret_cast<const v8*>(qh + (ok ? d0 : 0));
    qop[s] = ok ? x : v8{};
  }
}

// One wave's pass over tokens [t_begin, t_end) of (b, kvh) for its 16 query
// heads, with page_size % 32 == 0 (every step inside one page), t_begin a
// multiple of 32 and at most 64 pages touched (one block-table entry per
// lane). Folds the range into the running state (o, m_ref, l_lane). lds_k and
// lds_v are this wave's [32][DPAD + 16] tiles. load_q(qop) issues the query
// operand loads after the block-table load; finish_q(qop) runs after the
// first step's K/V loads are issued (a place for arithmetic on the loaded
// operands that should not hold up that issue). HB: the call carries an
// additive bias (loaded with the step's K/V, one step ahead).
// PRE: the caller has loaded a 64-page window of the sequence's block-table
// row that covers the range (entry window_base + lane per lane, -1 past the
// row) and passes it as row_entry, so no table load is issued here.
template <typename T, int DPAD, bool HB, bool PRE = false, typename QLoad, typename QFinish>
__device__ __forceinline__ void rows_range(const DecodeArgs& a, int b, int kvh, int h,
                                           bool head_ok, int t_begin, int t_end, QLoad load_q,
                                           QFinish finish_q, T* lds_k, T* lds_v,
                                           f32x4_t (&o)[DPAD / 16], float& m_ref,
                                           float& l_lane, int row_entry = -2,
                                           int window_base = 0) {
  typedef MfmaOps<T> Ops;
  typedef typename Ops::v8 v8;
  constexpr int KS = DPAD / 32;      // MFMA k-steps over head_dim
  constexpr int DT = DPAD / 16;      // 16-row d tiles of the output
  constexpr int CPR = DPAD / 8;      // 16-byte chunks per token row
  constexpr int RPI = 64 / CPR;      // token rows per load instruction
  constexpr int NI = kStep / RPI;    // load instructions per tensor per step
  constexpr int LROW = DPAD + 16;    // LDS row pitch (elements): rows 8 banks apart

  const int lane = threadIdx.x & 63;
  const int col = lane & 15;  // query head within the 16-wide tile / token row of operands
  const int q4 = lane >> 4;   // 0..3
  const int srow = lane / CPR;    // staging: token row within a load instruction
  const int schunk = lane % CPR;  // staging: 16-byte chunk within the row
  const bool chunk_in_d = schunk * 8 < a.D;

  // Block-table entries of this range, one per lane (or the preloaded row).
  const int first_page =
      PRE ? window_base : (a.p_shift >= 0 ? (t_begin >> a.p_shift) : (t_begin / a.P));
  const int last_page = a.p_shift >= 0 ? ((t_end - 1) >> a.p_shift) : ((t_end - 1) / a.P);
  int my_page = row_entry;
  if constexpr (!PRE)
    my_page =
        first_page + lane <= last_page ? a.bt[(int64_t)b * a.bt_stride + first_page + lane] : -1;
  v8 qop[KS];
  load_q(qop);

  u32x4_t sk[NI], sv[NI];
  // Bias of this lane's scores of the step at t: tokens t + gi*16 + q4*4 + i.
  float bnx[2][4];
  auto issue_bias = [&](int t) __attribute__((always_inline)) {
    if constexpr (HB) {
#pragma unroll
      for (int gi = 0; gi < 2; ++gi)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int tok = t + gi * 16 + q4 * 4 + i;
          bnx[gi][i] = head_ok && tok < t_end ? decode_bias(a, b, h, tok) : 0.f;
        }
    }
  };
  // Issue the loads of the step starting at t. Past the range end (the
  // prefetch after the last step) every offset is out of range: zeros, no
  // memory traffic, and no branch for the wait-count bookkeeping to merge.
  auto issue = [&](int t) -> bool {
    const int page_idx = a.p_shift >= 0 ? (t >> a.p_shift) : (t / a.P);
    const int slot0 = t - page_idx * a.P;
    const bool in_split = t < t_end;
    const int phys = __builtin_amdgcn_readlane(my_page, in_split ? page_idx - first_page : 0);
    const bool pvalid =
        in_split && static_cast<unsigned>(phys) < static_cast<unsigned>(a.num_pages);
    const int64_t base = pvalid ? (int64_t)phys * a.s_page + (int64_t)kvh * a.s_head : 0;
    const int nbytes =
        pvalid ? static_cast<int>(((int64_t)(a.P - 1) * a.s_tok + a.D) * sizeof(T)) : 0;
    const __amdgpu_buffer_rsrc_t rK = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<T*>(static_cast<const T*>(a.kp) + base), 0, nbytes, kBufferWord3);
    const __amdgpu_buffer_rsrc_t rV = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<T*>(static_cast<const T*>(a.vp) + base), 0, nbytes, kBufferWord3);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int row = i * RPI + srow;
      const bool live = pvalid && t + row < t_end && chunk_in_d;
      const int off =
          live ? static_cast<int>(((int64_t)(slot0 + row) * a.s_tok + schunk * 8) * sizeof(T))
               : -16;
      sk[i] = __builtin_amdgcn_raw_buffer_load_b128(rK, off, 0, kLoadNT);
      sv[i] = __builtin_amdgcn_raw_buffer_load_b128(rV, off, 0, kLoadNT);
    }
    return pvalid;
  };

  bool pvalid = issue(t_begin);
  issue_bias(t_begin);
  finish_q(qop);
  for (int t = t_begin; t < t_end; t += kStep) {
    // staging -> LDS (row-major [32 tok][LROW])
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int row = i * RPI + srow;
      *reinterpret_cast<u32x4_t*>(lds_k + row * LROW + schunk * 8) = sk[i];
      *reinterpret_cast<u32x4_t*>(lds_v + row * LROW + schunk * 8) = sv[i];
    }
    float bcu[2][4];
    if constexpr (HB) {
#pragma unroll
      for (int gi = 0; gi < 2; ++gi)
#pragma unroll
        for (int i = 0; i < 4; ++i) bcu[gi][i] = bnx[gi][i];
    }
    const bool cur_valid = pvalid;
    pvalid = issue(t + kStep);
    if (t + kStep < t_end) issue_bias(t + kStep);
    lc_compiler_fence();

    f32x4_t sacc[2];
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      sacc[gi] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const v8 kop = *reinterpret_cast<const v8*>(lds_k + (gi * 16 + col) * LROW + s * 32 + q4 * 8);
        sacc[gi] = Ops::mma(kop, qop[s], sacc[gi]);
      }
    }
    float sc[2][4];
#pragma unroll
    for (int gi = 0; gi < 2; ++gi)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool live = cur_valid && t + gi * 16 + q4 * 4 + i < t_end;
        const float x = HB ? fmaf(sacc[gi][i], a.scale_log2, bcu[gi][i])
                           : sacc[gi][i] * a.scale_log2;
        sc[gi][i] = live ? x : -INFINITY;
      }
    const v8 pop = softmax_step<T, DT>(sc, m_ref, l_lane, o);
    pv_step<T, DT, LROW>(lds_v, q4, col, pop, o);
    lc_compiler_fence();
  }
}

// Main kernel: page_size % 32 == 0; one wave per split, partials to the
// workspace for the merge kernel.
template <typename T, int DPAD, bool HB>
__global__ __launch_bounds__(64) void paged_decode_rows_kernel(DecodeArgs a) {
  typedef typename MfmaOps<T>::v8 v8;
  constexpr int DT = DPAD / 16;
  constexpr int LROW = DPAD + 16;
  __shared__ __align__(16) T lds_k[kStep * LROW];
  __shared__ __align__(16) T lds_v[kStep * LROW];

  const int lane = threadIdx.x;
  const int split = blockIdx.z;
  const int kvh = blockIdx.x / a.n_hgroups;
  const int hg = blockIdx.x - kvh * a.n_hgroups;
  // Sequence b's split z sits at grid row (b - z) mod B: the hardware deals
  // workgroups to each XCD's shader engines round-robin by id, so with b on
  // the row every split of a sequence went to one engine; rotated, a
  // sequence's splits spread over all four.
  const int b = (blockIdx.y + blockIdx.z) % a.B;
  const int len = seq_len_of(a, b);
  const int t_begin = split * a.split_tokens;
  if (t_begin >= len) return;
  const int t_end = min(len, t_begin + a.split_tokens);

  const int col = lane & 15;
  const int q4 = lane >> 4;
  const int g = hg * 16 + col;
  const bool head_ok = g < a.G;
  const int h = kvh * a.G + g;

  f32x4_t o[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) o[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_ref = -INFINITY;
  float l_lane = 0.f;
  rows_range<T, DPAD, HB>(
      a, b, kvh, h, head_ok, t_begin, t_end,
      [&](v8 (&qop)[DPAD / 32]) { load_q<T, DPAD>(a, b, h, kvh * a.G, head_ok, q4, qop); },
      [](v8 (&)[DPAD / 32]) {}, lds_k, lds_v, o, m_ref, l_lane);
  store_partial<DT>(a, b, h, split, head_ok, q4, m_ref, l_lane, o);
}

// Waves per workgroup of the single-split (cluster) kernel: its LDS is W
// per-wave K/V tiles, kept within one CU's 160 KiB.
template <int DPAD>
constexpr int cluster_waves() {
  return DPAD <= 128 ? 8 : 4;
}

// Inputs of the decode-step fusion (RoPE of the new token, its append to the
// pools and attention over the cache including it) run by the single-split
// kernel.
struct StepArgs {
  const void* k;  // new key of (b, kv head h): k + b*k_sb + h*k_sh, head_dim contiguous
  const void* v;
  int64_t k_sb, k_sh, v_sb, v_sh;
  const void* cos;  // RoPE tables: row p at cos + p*cs, full head_dim width
  const void* sin;
  int64_t cs, ss;
  int table_rows;
  void* kp;  // the pools, written at the new token's slot
  void* vp;
  int32_t* seq_lens;  // advanced by one per sequence
  int32_t* counters;  // [B]: zero on entry, zero again on return
};

// Longest-first order of the (sequence, split) pairs for a ragged batch of
// B <= 64 * kOrdChunks sequences (lane i of chunk c holds sequence 64c + i)
// and split_tokens <= 2^23 (the select's keys are 31 bits): every whole split
// (split_tokens tokens) first, sequence by sequence, then each sequence's
// final partial split, longest first (ties: lower sequence first). The
// hardware deals workgroups to the XCDs and, inside each, to its shader
// engines round-robin by id, whatever each one's work; in this order
// consecutive ids carry equal or similar work, so every engine gets an even
// share and its queue ends with its shortest splits. Returns (b << 16) |
// split of pair r and the sequence's length in len_out, or -1 when r is past
// the last pair.
// Inclusive prefix sum over the wave's 64 lanes on DPP moves (no LDS round
// trips): shifts of 1, 2, 4 and 8 lanes inside each 16-lane row, then the
// row totals broadcast from lane 15 into rows 1 and 3 and from lane 31 into
// rows 2 and 3. Lanes whose source lies outside the row read 0.
__device__ __forceinline__ int wave_incl_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return x;
}

constexpr int kOrdChunks = 4;
// int32 counters lc_paged_decode_fwd takes: the ticket, padded to 256 bytes.
constexpr int kDecodeCounterInts = 64;

// The batch's lengths for the order, sequence 64c + lane in li[c] (0 past B).
__device__ __forceinline__ void ord_lengths(const DecodeArgs& a, int lane,
                                            int (&li)[kOrdChunks]) {
  const int nc = (a.B + 63) >> 6;
#pragma unroll
  for (int c = 0; c < kOrdChunks; ++c) {
    const int bi = c * 64 + lane;
    li[c] = c < nc && bi < a.B ? seq_len_of(a, bi) : 0;
  }
}

// Number of (sequence, split) pairs with tokens: every whole split and every
// final partial split (wave-uniform).
__device__ __forceinline__ int ord_pair_count(const DecodeArgs& a, const int (&li)[kOrdChunks]) {
  const int nc = (a.B + 63) >> 6;
  int n = 0;
#pragma unroll
  for (int c = 0; c < kOrdChunks; ++c) {
    if (c >= nc) break;
    const int whole = li[c] / a.split_tokens;
    n += __builtin_amdgcn_readlane(wave_incl_scan(whole), 63) +
         __popcll(__ballot(li[c] - whole * a.split_tokens > 0));
  }
  return n;
}

__device__ __forceinline__ int ordered_pair_chunked(const DecodeArgs& a,
                                                    const int (&li)[kOrdChunks], int r, int lane,
                                                    int& len_out) {
  const int nc = (a.B + 63) >> 6;  // chunks in use (uniform)
  // Chunks past nc hold no sequence; every loop below skips them (uniform
  // branches), so a batch of <= 64 pays for one chunk only.
  int whole[kOrdChunks] = {}, rem[kOrdChunks] = {}, incl[kOrdChunks] = {};
  int carry = 0;  // whole splits of the earlier chunks
#pragma unroll
  for (int c = 0; c < kOrdChunks; ++c) {
    if (c >= nc) break;
    whole[c] = li[c] / a.split_tokens;
    rem[c] = li[c] - whole[c] * a.split_tokens;
    incl[c] = wave_incl_scan(whole[c]) + carry;  // prefix sum of the whole splits
    carry = __builtin_amdgcn_readlane(incl[c], 63);
  }
  const int n_whole = carry;
  int bb = -1, sp = 0, lb = 0;
  if (r < n_whole) {
#pragma unroll
    for (int c = 0; c < kOrdChunks; ++c) {
      if (c >= nc) break;
      const unsigned long long m = __ballot(incl[c] > r);
      if (bb < 0 && m != 0) {
        const int l = __builtin_ctzll(m);
        bb = c * 64 + l;
        sp = r - (__builtin_amdgcn_readlane(incl[c], l) - __builtin_amdgcn_readlane(whole[c], l));
        lb = __builtin_amdgcn_readlane(li[c], l);
      }
    }
  } else {
    // The k-th largest key (remainder, then lower sequence first) by a radix
    // select over the key bits, on ballots: the candidates shrink to one lane.
    unsigned long long cand[kOrdChunks] = {};
    unsigned key[kOrdChunks] = {};
    int k = r - n_whole, n_part = 0;
#pragma unroll
    for (int c = 0; c < kOrdChunks; ++c) {
      if (c >= nc) break;
      cand[c] = __ballot(rem[c] > 0);
      n_part += __popcll(cand[c]);
      key[c] = (static_cast<unsigned>(rem[c]) << 8) | static_cast<unsigned>(255 - (c * 64 + lane));
    }
    if (k >= n_part) return -1;
    const int top = 31 - __builtin_clz((static_cast<unsigned>(a.split_tokens) << 8) | 255u);
    for (int bit = top; bit >= 0; --bit) {
      unsigned long long ones[kOrdChunks];
      int cnt = 0;
#pragma unroll
      for (int c = 0; c < kOrdChunks; ++c) {
        if (c >= nc) break;
        ones[c] = __ballot((key[c] >> bit) & 1u) & cand[c];
        cnt += __popcll(ones[c]);
      }
      const bool take = k < cnt;
      if (!take) k -= cnt;
#pragma unroll
      for (int c = 0; c < kOrdChunks; ++c) {
        if (c >= nc) break;
        cand[c] = take ? ones[c] : (cand[c] & ~ones[c]);
      }
    }
#pragma unroll
    for (int c = 0; c < kOrdChunks; ++c) {
      if (c >= nc) break;
      if (bb < 0 && cand[c] != 0) {
        const int l = __builtin_ctzll(cand[c]);
        bb = c * 64 + l;
        sp = __builtin_amdgcn_readlane(whole[c], l);
        lb = __builtin_amdgcn_readlane(li[c], l);
      }
    }
  }
  len_out = lb;
  return (bb << 16) | sp;
}

// The same order for B <= 64 (one sequence per lane): the batches this path
// was first measured on take the shorter code (the chunked form measured ~1%
// slower at 64 sequences).
__device__ __forceinline__ int ordered_pair_64(const DecodeArgs& a, int li, int r, int lane,
                                               int& len_out) {
  const int whole = li / a.split_tokens;
  const int rem = li - whole * a.split_tokens;
  const int incl = wave_incl_scan(whole);  // inclusive prefix sum of the whole splits
  const int n_whole = __builtin_amdgcn_readlane(incl, 63);
  int bb, sp;
  if (r < n_whole) {
    bb = __builtin_ctzll(__ballot(incl > r));
    sp = r - (__builtin_amdgcn_readlane(incl, bb) - __builtin_amdgcn_readlane(whole, bb));
  } else {
    unsigned long long cand = __ballot(rem > 0);
    int k = r - n_whole;
    if (k >= __popcll(cand)) return -1;
    const unsigned key = (static_cast<unsigned>(rem) << 6) | static_cast<unsigned>(63 - lane);
    const int top = 31 - __builtin_clz((static_cast<unsigned>(a.split_tokens) << 6) | 63u);
    for (int bit = top; bit >= 0; --bit) {
      const unsigned long long ones = __ballot((key >> bit) & 1u) & cand;
      const int c = __popcll(ones);
      if (k < c) {
        cand = ones;
      } else {
        k -= c;
        cand &= ~ones;
      }
    }
    bb = __builtin_ctzll(cand);
    sp = __builtin_amdgcn_readlane(whole, bb);
  }
  len_out = __builtin_amdgcn_readlane(li, bb);
  return (bb << 16) | sp;
}

__device__ __forceinline__ int ordered_pair(const DecodeArgs& a, const int (&li)[kOrdChunks],
                                            int r, int lane, int& len_out) {
  return a.B <= 64 ? ordered_pair_64(a, li[0], r, lane, len_out)
                   : ordered_pair_chunked(a, li, r, lane, len_out);
}

// Single-split decode (max_splits == 1) for page_size % 32 == 0: one
// workgroup of W waves per (b, kv head, group of <= 16 query heads). The
// sequence's 32-token steps are dealt out evenly to the W waves by its
// device-side length, each wave runs the main kernel's pass over its range,
// and the W softmax states are merged through LDS into the final output and
// lse, so no partials and no merge kernel:
//   M = max_w m_w, out = sum_w 2^(m_w - M) o_w / sum_w 2^(m_w - M) l_w,
//   lse = (M + log2 sum_w 2^(m_w - M) l_w) * ln 2.
// The host takes this path only when every wave's range touches <= 64 pages.
//
// STEP (decode-step fusion; D % 16 == 0): q, k and v are the new token's
// unrotated projections and p = seq_lens[b] its position. q and k are rotated
// at p (tables at row min(p, table_rows - 1)) and rounded to T; the cache
// tokens [0, min(max(p, 0), capacity)) are attended as above, and the new
// token joins the merge as one more partial (m = its score, l = 1, o = v)
// when 0 <= p < capacity and its page entry is valid, in which case the
// head-group-0 workgroup also writes the rotated k and v at slot p. The last
// workgroup of sequence b to finish (a ticket on counters[b]) sets
// seq_lens[b] = p + 1 and returns counters[b] to zero; every workgroup takes
// its ticket after its last read of seq_lens[b]. Results equal the RoPE,
// append and decode launches in sequence, up to fp32 summation order.
//
// ORD (several splits, B <= 256, not STEP): a one-dimensional grid whose
// workgroup of rank i takes unit i % (Hkv * n_hgroups) of pair
// i / (Hkv * n_hgroups) in the order of ordered_pair; the splits and their
// partials are the same as in the (units, B, splits) grid. The rank is the
// block id, except that with a ticket (ord_ticket) the last quarter of the
// live ranks is handed out in the order the workgroups start, so the faster
// XCDs take more of the short final splits (which workgroup computes a split
// changes nothing in its partials).
template <typename T, int DPAD, bool HB, bool STEP, bool PRE, bool ORD = false>
__global__ __launch_bounds__(64 * cluster_waves<DPAD>()) void paged_decode_cluster_kernel(
    DecodeArgs a, T* __restrict__ out, int64_t o_sb, int64_t o_sh, float* __restrict__ lse_out,
    StepArgs sa) {
  typedef typename MfmaOps<T>::v8 v8;
  constexpr int W = cluster_waves<DPAD>();
  constexpr int KS = DPAD / 32;
  constexpr int DT = DPAD / 16;
  constexpr int LROW = DPAD + 16;
  constexpr int TILE = kStep * LROW;  // elements of one K or V tile
  constexpr int OP = DPAD + 4;        // fp32 pitch of a head's row in the merge buffer
  constexpr int PER_HEAD = DPAD / 4;  // merge items (4 elements each) per head
  constexpr int IPT = (16 * PER_HEAD + 64 * W - 1) / (64 * W);  // merge items per thread
  static_assert(16 * OP * 4 + 32 * 4 <= 2 * TILE * (int)sizeof(T),
                "a wave's merge record must fit in its K/V tiles");
  static_assert(PER_HEAD <= 64 && (PER_HEAD & (PER_HEAD - 1)) == 0,
                "a head's merge items are one power-of-two group of lanes");
  __shared__ __align__(16) T lds[W * 2 * TILE];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  int kvh, hg, b, split, ord_len = 0;
  if constexpr (ORD) {
    const int units = a.Hkv * a.n_hgroups;
    int li[kOrdChunks];
    ord_lengths(a, lane, li);
    int rank = blockIdx.x;
    if (a.ord_ticket != nullptr) {
      // Dynamic tail: the XCDs read at different rates, so the last quarter
      // of the live workgroups' ranks (the shortest splits) go to whichever
      // workgroups start first, through the ticket. A spare pool of an eighth
      // more workgroups lets the faster XCDs take more of them; workgroups
      // past it leave at once. Every workgroup in [s0, n_draw) draws exactly
      // once, so the one that draws the last value returns the ticket to zero.
      const int n_live = ord_pair_count(a, li) * units;
      const int s0 = max(min((int)gridDim.x, a.ord_static), n_live - (n_live >> 2));
      const int n_draw = max(s0, min((int)gridDim.x, n_live + (n_live >> 3)));
      if (rank >= n_draw) return;
      if (rank >= s0) {
        __shared__ int s_rank;
        if (threadIdx.x == 0) {
          const int t = __hip_atomic_fetch_add(a.ord_ticket, 1, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
          if (t == n_draw - s0 - 1)
            __hip_atomic_store(a.ord_ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          s_rank = s0 + t;
        }
        __syncthreads();
        rank = s_rank;
      }
    }
    const int r = rank / units;
    const int u = rank - r * units;
    const int pair = ordered_pair(a, li, r, lane, ord_len);
    if (pair < 0) return;
    kvh = u / a.n_hgroups;
    hg = u - kvh * a.n_hgroups;
    b = pair >> 16;
    split = pair & 0xffff;
  } else {
    kvh = blockIdx.x / a.n_hgroups;
    hg = blockIdx.x - kvh * a.n_hgroups;
    b = blockIdx.y;
    split = blockIdx.z;
  }
  const int cap = a.max_pages * a.P;
  // This workgroup's split: tokens [s_begin, s_begin + split_tokens).
  const int s_begin = split * a.split_tokens;
  // PRE (the split's pages fit 64 block-table entries): the window of the row
  // from the split's first page is loaded whole (one entry per lane) together
  // with the length, so the first K/V loads wait on one round trip, not on
  // the length and then the table.
  const int window_base = a.p_shift >= 0 ? (s_begin >> a.p_shift) : (s_begin / a.P);
  int row_entry = -1;
  if constexpr (PRE)
    row_entry = a.bt[(int64_t)b * a.bt_stride + min(window_base + lane, a.max_pages - 1)];
  const int p_new = STEP ? a.seq_lens[b] : 0;  // the new token's position
  const int len = STEP ? min(max(p_new, 0), cap) : ORD ? ord_len : seq_len_of(a, b);
  if constexpr (PRE) {
    row_entry = window_base + lane < a.max_pages ? row_entry : -1;
    // Keep the row load here, beside the length's, rather than sunk to its use.
    asm volatile("" : "+v"(row_entry));
  }
  // With several splits, a split past the length writes nothing (the merge
  // reads only the splits that hold tokens); a single split always writes the
  // output (zeros for an empty sequence).
  if (a.max_splits > 1 && s_begin >= len) return;
  const int prow = p_new < 0 ? 0 : min(p_new, sa.table_rows - 1);
  const int half = a.D / 2;
  const int s_len = min(len - s_begin, a.split_tokens);
  const int nsteps = s_len > 0 ? (s_len + kStep - 1) / kStep : 0;
  const int t_begin = s_begin + (wave * nsteps / W) * kStep;
  const int t_end = min(len, s_begin + ((wave + 1) * nsteps / W) * kStep);

  const int col = lane & 15;
  const int q4 = lane >> 4;
  const int g = hg * 16 + col;
  const bool head_ok = g < a.G;
  const int h = kvh * a.G + g;

  // STEP: the new token's slot, and this thread's merge items' operands
  // (4 elements each of q, k, their RoPE partners, cos, sin and v), loaded
  // before the main pass.
  // Every load below is unconditional, from a clamped address, and masked
  // where it is used, so no branch separates the loads from one another.
  int nt_phys = -1;
  u32x2_t nq[IPT], nqp[IPT], nk[IPT], nkp[IPT], nc[IPT], ns[IPT], nv[IPT];
  if constexpr (STEP) {
    const int pc = p_new >= 0 && p_new < cap ? p_new : 0;
    const int pi = a.p_shift >= 0 ? (pc >> a.p_shift) : (pc / a.P);
    if constexpr (PRE)  // single split: the window starts at page 0
      nt_phys = __builtin_amdgcn_readlane(row_entry, pi);
    else
      nt_phys = a.bt[(int64_t)b * a.bt_stride + pi];
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
      const int item = threadIdx.x + j * 64 * W;
      const int hc = item / PER_HEAD;
      const int d0 = (item - hc * PER_HEAD) * 4;
      const bool dok = hc < 16 && d0 < a.D;
      const bool qok = dok && hg * 16 + hc < a.G;
      const int dc = dok ? d0 : 0;
      const int pd = dc < half ? dc + half : dc - half;
      const T* qh = static_cast<const T*>(a.q) + (int64_t)b * a.q_sb +
                    (int64_t)(kvh * a.G + (qok ? hg * 16 + hc : 0)) * a.q_sh;
      const T* kh = static_cast<const T*>(sa.k) + (int64_t)b * sa.k_sb + (int64_t)kvh * sa.k_sh;
      const T* vh = static_cast<const T*>(sa.v) + (int64_t)b * sa.v_sb + (int64_t)kvh * sa.v_sh;
      const T* cr = static_cast<const T*>(sa.cos) + (int64_t)prow * sa.cs;
      const T* sr = static_cast<const T*>(sa.sin) + (int64_t)prow * sa.ss;
      nq[j] = *reinterpret_cast<const u32x2_t*>(qh + dc);
      nqp[j] = *reinterpret_cast<const u32x2_t*>(qh + pd);
      nk[j] = *reinterpret_cast<const u32x2_t*>(kh + dc);
      nkp[j] = *reinterpret_cast<const u32x2_t*>(kh + pd);
      nc[j] = *reinterpret_cast<const u32x2_t*>(cr + dc);
      ns[j] = *reinterpret_cast<const u32x2_t*>(sr + dc);
      nv[j] = *reinterpret_cast<const u32x2_t*>(vh + dc);
    }
  }

  f32x4_t o[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) o[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_ref = -INFINITY;
  float l_lane = 0.f;
  T* my_k = lds + wave * 2 * TILE;
  T* my_v = my_k + TILE;
  if (t_begin < t_end) {
    if constexpr (STEP) {
      // Query operands rotated at p: the lane's 8-element chunks, their
      // partners half a row away, and the table rows.
      v8 qpart[KS], cq[KS], sq[KS];
      const T* qh = static_cast<const T*>(a.q) + (int64_t)b * a.q_sb +
                    (int64_t)(head_ok ? h : kvh * a.G) * a.q_sh;
      const T* cr = static_cast<const T*>(sa.cos) + (int64_t)prow * sa.cs;
      const T* sr = static_cast<const T*>(sa.sin) + (int64_t)prow * sa.ss;
      rows_range<T, DPAD, HB, PRE>(
          a, b, kvh, h, head_ok, t_begin, t_end,
          [&](v8 (&qop)[KS]) {
#pragma unroll
            for (int s = 0; s < KS; ++s) {
              const int d0 = s * 32 + q4 * 8;
              const int dc = head_ok && d0 < a.D ? d0 : 0;
              const int pd = dc < half ? dc + half : dc - half;
              qop[s] = *reinterpret_cast<const v8*>(qh + dc);
              qpart[s] = *reinterpret_cast<const v8*>(qh + pd);
              cq[s] = *reinterpret_cast<const v8*>(cr + dc);
              sq[s] = *reinterpret_cast<const v8*>(sr + dc);
            }
          },
          [&](v8 (&qop)[KS]) {
#pragma unroll
            for (int s = 0; s < KS; ++s) {
              const int d0 = s * 32 + q4 * 8;
              const bool ok = head_ok && d0 < a.D;
              const bool lo = d0 < half;
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                const float x = static_cast<float>(qop[s][e]);
                const float xp = static_cast<float>(qpart[s][e]);
                const float c = static_cast<float>(cq[s][e]);
                const float sn = static_cast<float>(sq[s][e]);
                const T r = static_cast<T>(lo ? lc_rope_lo(x, xp, c, sn) : lc_rope_hi(xp, x, c, sn));
                qop[s][e] = ok ? r : static_cast<T>(0.f);
              }
            }
          },
          my_k, my_v, o, m_ref, l_lane, row_entry, window_base);
    } else {
      rows_range<T, DPAD, HB, PRE>(
          a, b, kvh, h, head_ok, t_begin, t_end,
          [&](v8 (&qop)[KS]) { load_q<T, DPAD>(a, b, h, kvh * a.G, head_ok, q4, qop); },
          [](v8 (&)[KS]) {}, my_k, my_v, o, m_ref, l_lane, row_entry, window_base);
    }
  }

  // This wave's record, over its own (now idle) tiles: o [16 heads][OP] fp32,
  // then m [16] and l [16].
  float l_tot = l_lane + __shfl_xor(l_lane, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  float* rec = reinterpret_cast<float*>(my_k);
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
    *reinterpret_cast<f32x4_t*>(rec + col * OP + dt * 16 + q4 * 4) = o[dt];
  if (q4 == 0) {
    rec[16 * OP + col] = m_ref;
    rec[16 * OP + 16 + col] = l_tot;
  }

  // STEP: rotate this thread's new-token items, write the new k and v (head
  // group 0, head 0's items cover the row), and form the new token's score of
  // each item's head (a dot product over the head's PER_HEAD lanes).
  float s_new[IPT], v_new[IPT][4];
  bool nt_ok = false;
  int64_t nt_off = 0;
  if constexpr (STEP) {
    // The new token is attended and stored iff it is inside the capacity and
    // its page entry is valid.
    nt_ok = p_new >= 0 && p_new < cap &&
            static_cast<unsigned>(nt_phys) < static_cast<unsigned>(a.num_pages);
    const int pi = a.p_shift >= 0 ? (p_new >> a.p_shift) : (p_new / a.P);
    nt_off = (int64_t)nt_phys * a.s_page + (int64_t)kvh * a.s_head +
             (int64_t)(p_new - pi * a.P) * a.s_tok;
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
      const int item = threadIdx.x + j * 64 * W;
      const int hc = item / PER_HEAD;
      const int d0 = (item - hc * PER_HEAD) * 4;
      const bool dok = hc < 16 && d0 < a.D;
      const bool qok = dok && hg * 16 + hc < a.G;
      const bool lo = d0 < half;
      typedef __attribute__((__vector_size__(4 * sizeof(T)))) T t4;
      const t4 xq = __builtin_bit_cast(t4, nq[j]), xqp = __builtin_bit_cast(t4, nqp[j]);
      const t4 xk = __builtin_bit_cast(t4, nk[j]), xkp = __builtin_bit_cast(t4, nkp[j]);
      const t4 xc = __builtin_bit_cast(t4, nc[j]), xs = __builtin_bit_cast(t4, ns[j]);
      const t4 xv = __builtin_bit_cast(t4, nv[j]);
      t4 kr;
      float dot = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float c = static_cast<float>(xc[e]), sn = static_cast<float>(xs[e]);
        const float q0 = static_cast<float>(xq[e]), q1 = static_cast<float>(xqp[e]);
        const float k0 = static_cast<float>(xk[e]), k1 = static_cast<float>(xkp[e]);
        const T qr = static_cast<T>(lo ? lc_rope_lo(q0, q1, c, sn) : lc_rope_hi(q1, q0, c, sn));
        kr[e] = static_cast<T>(lo ? lc_rope_lo(k0, k1, c, sn) : lc_rope_hi(k1, k0, c, sn));
        dot = fmaf(qok ? static_cast<float>(qr) : 0.f, static_cast<float>(kr[e]), dot);
        v_new[j][e] = static_cast<float>(xv[e]);
      }
#pragma unroll
      for (int off = 1; off < PER_HEAD; off <<= 1) dot += __shfl_xor(dot, off, 64);
      const int gg = hg * 16 + hc;
      float sc = dot * a.scale_log2;
      if constexpr (HB) {
        if (nt_ok && hc < 16 && gg < a.G) sc += decode_bias(a, b, kvh * a.G + gg, p_new);
      }
      s_new[j] = nt_ok ? sc : -INFINITY;
      if (nt_ok && hg == 0 && hc == 0 && d0 < a.D) {
        *reinterpret_cast<u32x2_t*>(static_cast<T*>(sa.kp) + nt_off + d0) =
            __builtin_bit_cast(u32x2_t, kr);
        *reinterpret_cast<u32x2_t*>(static_cast<T*>(sa.vp) + nt_off + d0) = nv[j];
      }
    }
  }
  __syncthreads();

  // Combine: each thread owns 4 consecutive elements of one head's row.
#pragma unroll
  for (int j = 0; j < IPT; ++j) {
    const int item = threadIdx.x + j * 64 * W;
    const int hc = item / PER_HEAD;
    const int d0 = (item - hc * PER_HEAD) * 4;
    const int gg = hg * 16 + hc;
    if (hc >= 16 || gg >= a.G || d0 >= a.D) continue;
    float mw[W], mx = STEP ? s_new[j] : -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      mw[w] = reinterpret_cast<const float*>(lds + w * 2 * TILE)[16 * OP + hc];
      mx = fmaxf(mx, mw[w]);
    }
    float acc[4] = {0.f, 0.f, 0.f, 0.f}, lsum = 0.f;
    if (mx != -INFINITY) {
#pragma unroll
      for (int w = 0; w < W; ++w) {
        const float* r = reinterpret_cast<const float*>(lds + w * 2 * TILE);
        const float e = mw[w] == -INFINITY ? 0.f : lc_exp2(mw[w] - mx);
        lsum = fmaf(e, r[16 * OP + 16 + hc], lsum);
        const f32x4_t ow = *reinterpret_cast<const f32x4_t*>(r + hc * OP + d0);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = fmaf(e, ow[i], acc[i]);
      }
      if constexpr (STEP) {
        const float e = s_new[j] == -INFINITY ? 0.f : lc_exp2(s_new[j] - mx);
        lsum += e;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = fmaf(e, v_new[j][i], acc[i]);
      }
    }
    const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
    const int hh = kvh * a.G + gg;
    if (a.max_splits > 1) {
      // The split's normalised partial and log2-domain lse, for the merge.
      const int64_t pidx = ((int64_t)b * a.Hq + hh) * a.max_splits + split;
      f32x4_t w;
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = acc[i] * inv;
      *reinterpret_cast<f32x4_t*>(a.part_o + pidx * a.D + d0) = w;
      if (d0 == 0) a.part_lse[pidx] = lsum > 0.f ? mx + lc_log2(lsum) : -INFINITY;
      continue;
    }
    T* oh = out + (int64_t)b * o_sb + (int64_t)hh * o_sh + d0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (d0 + i < a.D) oh[i] = lc_from_f32<T>(acc[i] * inv);
    if (lse_out != nullptr && d0 == 0)
      lse_out[(int64_t)b * a.Hq + hh] = lsum > 0.f ? (mx + lc_log2(lsum)) * kLn2 : -INFINITY;
  }

  if constexpr (STEP) {
    // Every wave of this workgroup read seq_lens[b] before the barrier above.
    if (threadIdx.x == 0) {
      const int n_wg = a.Hkv * a.n_hgroups;
      const int ticket = __hip_atomic_fetch_add(sa.counters + b, 1, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
      if (ticket == n_wg - 1) {
        __hip_atomic_store(sa.counters + b, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(sa.seq_lens + b, p_new + 1, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// Page sizes that are not multiples of 32: per-lane page resolution.
// Three waves per SIMD up to head_dim 128: at 144 VGPRs and 9 KiB of LDS the
// kernel fits them without spills, and the extra loads in flight measured 6%
// faster than two. (head_dim 256 would spill at three.)
template <typename T, int DPAD, bool HB>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(DPAD <= 128 ? 3 : 1))) void
paged_decode_lanes_kernel(DecodeArgs a) {
  typedef MfmaOps<T> Ops;
  typedef typename Ops::v8 v8;
  constexpr int KS = DPAD / 32;
  constexpr int DT = DPAD / 16;
  constexpr int LROW = DPAD + 16;
  __shared__ __align__(16) T lds_v[kStep * LROW];

  const int lane = threadIdx.x;
  const int split = blockIdx.z;
  const int kvh = blockIdx.x / a.n_hgroups;
  const int hg = blockIdx.x - kvh * a.n_hgroups;
  // Sequence b's split z sits at grid row (b - z) mod B: the hardware deals
  // workgroups to each XCD's shader engines round-robin by id, so with b on
  // the row every split of a sequence went to one engine; rotated, a
  // sequence's splits spread over all four.
  const int b = (blockIdx.y + blockIdx.z) % a.B;
  const int len = seq_len_of(a, b);
  const int t_begin = split * a.split_tokens;
  if (t_begin >= len) return;
  const int t_end = min(len, t_begin + a.split_tokens);
  const int col = lane & 15;
  const int q4 = lane >> 4;
  const int g = hg * 16 + col;
  const bool head_ok = g < a.G;
  const int h = kvh * a.G + g;
  const T* kp = static_cast<const T*>(a.kp);
  const T* vp = static_cast<const T*>(a.vp);

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
  float m_ref = -INFINITY;
  float l_lane = 0.f;

  for (int t = t_begin; t < t_end; t += kStep) {
    StepRegs<T, DPAD> r;
    load_step_lane<T, DPAD>(a, kp, vp, b, kvh, t, t_end, col, q4, r);
    f32x4_t sacc[2];
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
      sacc[gi] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) sacc[gi] = Ops::mma(r.k[gi][s], qop[s], sacc[gi]);
    }
#pragma unroll
    for (int gi = 0; gi < 2; ++gi)
#pragma unroll
      for (int s = 0; s < KS; ++s)
        *reinterpret_cast<v8*>(lds_v + (gi * 16 + col) * LROW + s * 32 + q4 * 8) = r.v[gi][s];
    float sc[2][4];
#pragma unroll
    for (int gi = 0; gi < 2; ++gi)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool live = (r.valid[gi] >> (q4 * 4 + i)) & 1;
        float x = sacc[gi][i] * a.scale_log2;
        if constexpr (HB) {
          const int tok = t + gi * 16 + q4 * 4 + i;
          if (head_ok && live) x += decode_bias(a, b, h, tok);
        }
        sc[gi][i] = live ? x : -INFINITY;
      }
    const v8 pop = softmax_step<T, DT>(sc, m_ref, l_lane, o);
    lc_compiler_fence();
    pv_step<T, DT, LROW>(lds_v, q4, col, pop, o);
    lc_compiler_fence();
  }
  store_partial<DT>(a, b, h, split, head_ok, q4, m_ref, l_lane, o);
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
    float s = lc_wave_sum(dot) * a.scale_log2;
    if (a.bias != nullptr) {
      s += decode_bias(a, b, h, t);
      if (s == -INFINITY) continue;  // uniform: every lane reads the same element
    }
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

// Cross-split merge: one wave per (b, h). Lanes take one split each to form
// the weights 2^(lse_s - max) in parallel; the weighted sum walks the splits
// kBatch at a time with independent, unpredicated row loads (each lane owns
// VPL consecutive floats of head_dim). The first batch of rows does not depend
// on the max and is loaded together with the split lses, so a merge of up to
// kBatch splits costs one memory round trip.
// out = sum_s w_s o_s / sum_s w_s; lse = (max + log2 sum_s w_s) * ln 2.
template <typename T, int VPL>
__global__ __launch_bounds__(64) void decode_merge_kernel(DecodeArgs a, T* __restrict__ out,
                                                          int64_t o_sb, int64_t o_sh,
                                                          float* __restrict__ lse_out) {
  constexpr int kBatch = 16;  // divides 64: a batch never spans two lse chunks
  const int lane = threadIdx.x;
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int len = seq_len_of(a, b);
  const int nsplit = (len + a.split_tokens - 1) / a.split_tokens;
  const int64_t pbase = ((int64_t)b * a.Hq + h) * a.max_splits;
  T* oh = out + (int64_t)b * o_sb + (int64_t)h * o_sh;
  const int d0 = lane * VPL;
  const int dl = d0 < a.D ? d0 : 0;  // lanes past head_dim read (and drop) column 0
  const float* rows = a.part_o + pbase * a.D + dl;

  // Rows j0 .. j0 + kBatch - 1, clamped to the last split (nsplit >= 1).
  float v[kBatch][VPL];
  auto load_batch = [&](int j0) __attribute__((always_inline)) {
#pragma unroll
    for (int jj = 0; jj < kBatch; ++jj) {
      const int j = min(j0 + jj, nsplit - 1);
#pragma unroll
      for (int e = 0; e < VPL; ++e) v[jj][e] = rows[(int64_t)j * a.D + e];
    }
  };

  float lse0 = -INFINITY;  // split `lane` of the first 64
  if (nsplit > 0) {
    if (lane < nsplit) lse0 = a.part_lse[pbase + lane];
    load_batch(0);
  }
  float mx = lse0;
  for (int s = lane + 64; s < nsplit; s += 64) mx = fmaxf(mx, a.part_lse[pbase + s]);
  mx = lc_wave_max(mx);
  float acc[VPL];
#pragma unroll
  for (int e = 0; e < VPL; ++e) acc[e] = 0.f;
  float wlane = 0.f;
  if (mx != -INFINITY) {
    for (int s0 = 0; s0 < nsplit; s0 += 64) {
      const int n = min(64, nsplit - s0);
      float ls = lse0;
      if (s0 > 0) ls = lane < n ? a.part_lse[pbase + s0 + lane] : -INFINITY;
      const float w = lane < n ? lc_exp2(ls - mx) : 0.f;
      wlane += w;
      for (int j0 = 0; j0 < n; j0 += kBatch) {
        if (s0 + j0 > 0) load_batch(s0 + j0);
#pragma unroll
        for (int jj = 0; jj < kBatch; ++jj) {
          const float wj = __int_as_float(
              __builtin_amdgcn_readlane(__float_as_int(w), min(j0 + jj, 63)));
          const float wk = j0 + jj < n ? wj : 0.f;
#pragma unroll
          for (int e = 0; e < VPL; ++e) acc[e] = fmaf(wk, v[jj][e], acc[e]);
        }
      }
    }
  }
  const float wsum = lc_wave_sum(wlane);
  const float inv = wsum > 0.f ? 1.0f / wsum : 0.f;
#pragma unroll
  for (int e = 0; e < VPL; ++e)
    if (d0 + e < a.D) oh[d0 + e] = lc_from_f32<T>(acc[e] * inv);
  if (lse_out != nullptr && lane == 0)
    lse_out[(int64_t)b * a.Hq + h] = wsum > 0.f ? (mx + lc_log2(wsum)) * kLn2 : -INFINITY;
}

template <typename T, int DPAD>
int launch_mfma(const DecodeArgs& a, bool rows, hipStream_t st) {
  // Split-major dispatch order (blockIdx.z = split): workgroups are handed
  // out in block-id order as earlier ones finish, so the last to start are
  // the final, mostly partial splits of the longest sequences rather than
  // full splits of the last sequences, which shortens the ragged tail.
  dim3 grid(a.Hkv * a.n_hgroups, a.B, a.max_splits);
  const bool hb = a.bias != nullptr;
  if (rows && hb)
    paged_decode_rows_kernel<T, DPAD, true><<<grid, 64, 0, st>>>(a);
  else if (rows)
    paged_decode_rows_kernel<T, DPAD, false><<<grid, 64, 0, st>>>(a);
  else if (hb)
    paged_decode_lanes_kernel<T, DPAD, true><<<grid, 64, 0, st>>>(a);
  else
    paged_decode_lanes_kernel<T, DPAD, false><<<grid, 64, 0, st>>>(a);
  return lc_check_launch("lc_paged_decode_fwd (mfma)");
}

template <typename T>
int launch_merge(const DecodeArgs& a, void* out, int64_t o_sb, int64_t o_sh, float* lse,
                 hipStream_t st) {
  dim3 mgrid(a.Hq, a.B);
  T* o = static_cast<T*>(out);
  if (a.D <= 64)
    decode_merge_kernel<T, 1><<<mgrid, 64, 0, st>>>(a, o, o_sb, o_sh, lse);
  else if (a.D <= 128)
    decode_merge_kernel<T, 2><<<mgrid, 64, 0, st>>>(a, o, o_sb, o_sh, lse);
  else
    decode_merge_kernel<T, 4><<<mgrid, 64, 0, st>>>(a, o, o_sb, o_sh, lse);
  return lc_check_launch("lc_paged_decode_fwd (merge)");
}

template <typename T, int DPAD>
int launch_cluster(const DecodeArgs& a, void* out, int64_t o_sb, int64_t o_sh, float* lse,
                   hipStream_t st) {
  // Split-major order (blockIdx.z = split), as in the one-wave kernel.
  dim3 grid(a.Hkv * a.n_hgroups, a.B, a.max_splits);
  const unsigned threads = 64 * cluster_waves<DPAD>();
  T* o = static_cast<T*>(out);
  const StepArgs none{};
  // A split starting at any multiple of split_tokens touches at most
  // (split_tokens - 1) / P + 2 pages; one split reads pages 0 .. max_pages-1.
  const bool pre = a.max_splits == 1 ? a.max_pages <= 64
                                     : (a.split_tokens - 1) / a.P + 2 <= 64;
  // Longest-first order where the workgroups take more than one round of the
  // CUs (with one round every workgroup starts at once and the order cannot
  // matter, and computing it would only lengthen each one's start).
  const int64_t n_wg = (int64_t)a.Hkv * a.n_hgroups * a.B * a.max_splits;
  if (a.max_splits > 1 && a.B <= 64 * kOrdChunks && a.split_tokens <= (1 << 23) &&
      n_wg > lc_cu_count() &&
      n_wg * threads < (1LL << 32)) {  // a 1-D dispatch's work-items fit 32 bits
    const dim3 g1(static_cast<unsigned>(n_wg));
    if (a.bias != nullptr && pre)
      paged_decode_cluster_kernel<T, DPAD, true, false, true, true>
          <<<g1, threads, 0, st>>>(a, o, o_sb, o_sh, lse, none);
    else if (a.bias != nullptr)
      paged_decode_cluster_kernel<T, DPAD, true, false, false, true>
          <<<g1, threads, 0, st>>>(a, o, o_sb, o_sh, lse, none);
    else if (pre)
      paged_decode_cluster_kernel<T, DPAD, false, false, true, true>
          <<<g1, threads, 0, st>>>(a, o, o_sb, o_sh, lse, none);
    else
      paged_decode_cluster_kernel<T, DPAD, false, false, false, true>
          <<<g1, threads, 0, st>>>(a, o, o_sb, o_sh, lse, none);
  } else if (a.bias != nullptr && pre)
    paged_decode_cluster_kernel<T, DPAD, true, false, true>
        <<<grid, threads, 0, st>>>(a, o, o_sb, o_sh, lse, none);
  else if (a.bias != nullptr)
    paged_decode_cluster_kernel<T, DPAD, true, false, false>
        <<<grid, threads, 0, st>>>(a, o, o_sb, o_sh, lse, none);
  else if (pre)
    paged_decode_cluster_kernel<T, DPAD, false, false, true>
        <<<grid, threads, 0, st>>>(a, o, o_sb, o_sh, lse, none);
  else
    paged_decode_cluster_kernel<T, DPAD, false, false, false>
        <<<grid, threads, 0, st>>>(a, o, o_sb, o_sh, lse, none);
  const int rc = lc_check_launch("lc_paged_decode_fwd (workgroup splits)");
  if (rc != LC_OK || a.max_splits == 1) return rc;
  return launch_merge<T>(a, out, o_sb, o_sh, lse, st);
}

template <typename T, int DPAD>
int launch_step(const DecodeArgs& a, const StepArgs& sa, void* out, int64_t o_sb, int64_t o_sh,
                float* lse, hipStream_t st) {
  dim3 grid(a.Hkv * a.n_hgroups, a.B);
  const unsigned threads = 64 * cluster_waves<DPAD>();
  T* o = static_cast<T*>(out);
  const bool pre = a.max_pages <= 64;
  if (a.bias != nullptr && pre)
    paged_decode_cluster_kernel<T, DPAD, true, true, true>
        <<<grid, threads, 0, st>>>(a, o, o_sb, o_sh, lse, sa);
  else if (a.bias != nullptr)
    paged_decode_cluster_kernel<T, DPAD, true, true, false>
        <<<grid, threads, 0, st>>>(a, o, o_sb, o_sh, lse, sa);
  else if (pre)
    paged_decode_cluster_kernel<T, DPAD, false, true, true>
        <<<grid, threads, 0, st>>>(a, o, o_sb, o_sh, lse, sa);
  else
    paged_decode_cluster_kernel<T, DPAD, false, true, false>
        <<<grid, threads, 0, st>>>(a, o, o_sb, o_sh, lse, sa);
  return lc_check_launch("lc_paged_decode_step");
}

template <typename T>
int launch_step_d(const DecodeArgs& a, const StepArgs& sa, void* out, int64_t o_sb,
                  int64_t o_sh, float* lse, hipStream_t st) {
  if (a.D <= 64) return launch_step<T, 64>(a, sa, out, o_sb, o_sh, lse, st);
  if (a.D <= 128) return launch_step<T, 128>(a, sa, out, o_sb, o_sh, lse, st);
  return launch_step<T, 256>(a, sa, out, o_sb, o_sh, lse, st);
}

template <typename T>
int launch_decode(DecodeArgs a, void* out, int64_t o_sb, int64_t o_sh, float* lse, bool mfma,
                  bool rows, bool cluster, hipStream_t st) {
  int rc = LC_OK;
  if (mfma && cluster) {
    if constexpr (sizeof(T) == 2) {
      a.n_hgroups = (a.G + 15) / 16;
      if (a.D <= 64) return launch_cluster<T, 64>(a, out, o_sb, o_sh, lse, st);
      if (a.D <= 128) return launch_cluster<T, 128>(a, out, o_sb, o_sh, lse, st);
      return launch_cluster<T, 256>(a, out, o_sb, o_sh, lse, st);
    }
  }
  if (mfma) {
    if constexpr (sizeof(T) == 2) {
      a.n_hgroups = (a.G + 15) / 16;
      if (a.D <= 64)
        rc = launch_mfma<T, 64>(a, rows, st);
      else if (a.D <= 128)
        rc = launch_mfma<T, 128>(a, rows, st);
      else
        rc = launch_mfma<T, 256>(a, rows, st);
    }
  } else {
    dim3 grid(a.max_splits, a.Hq, a.B);
    paged_decode_generic_kernel<T><<<grid, 64, 0, st>>>(a);
    rc = lc_check_launch("lc_paged_decode_fwd (generic)");
  }
  if (rc != LC_OK) return rc;
  return launch_merge<T>(a, out, o_sb, o_sh, lse, st);
}

// Validates a decode call and launches it with the given workspace (the
// caller's, or the device scratch of the allocation-free entry point).
int paged_decode_impl(const char* who, const void* q, int64_t q_sb, int64_t q_sh,
                      const void* key_pages, const void* value_pages, int64_t kv_s_page,
                      int64_t kv_s_head, int64_t kv_s_tok, const int32_t* block_table,
                      int64_t bt_stride, int64_t max_pages_per_seq, int64_t num_pages,
                      const int32_t* seq_lens, void* out, int64_t o_sb, int64_t o_sh, float* lse,
                      const void* bias, int64_t bias_sb, int64_t bias_sh, int64_t bias_len,
                      int bias_dtype, void* workspace, int64_t workspace_bytes, int32_t* counters,
                      int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t page_size,
                      int64_t split_tokens, int64_t max_splits, float scale, int dtype,
                      void* stream) {
  LC_REQUIRE((q && key_pages && value_pages && block_table && seq_lens && out && workspace) ||
                 B == 0,
             "%s: null pointer", who);
  LC_REQUIRE(B >= 0 && B < 65536, "%s: batch %lld out of range", who, (long long)B);
  LC_REQUIRE(Hq > 0 && Hkv > 0 && Hq % Hkv == 0,
             "%s: n_heads (%lld) must be a multiple of n_kv_heads (%lld)", who, (long long)Hq,
             (long long)Hkv);
  LC_REQUIRE(D > 0 && D <= 256, "%s: head_dim %lld not in [1, 256]", who, (long long)D);
  LC_REQUIRE(page_size > 0 && max_pages_per_seq > 0 && num_pages > 0,
             "%s: page_size, max_pages_per_seq and num_pages must be > 0", who);
  LC_REQUIRE(max_pages_per_seq * page_size < (1LL << 31) && num_pages < (1LL << 31),
             "%s: cache too large for 32-bit token indices", who);
  LC_REQUIRE(bt_stride >= max_pages_per_seq, "%s: bt_stride < row length", who);
  LC_REQUIRE(split_tokens > 0 && split_tokens % 64 == 0,
             "%s: split_tokens must be a positive multiple of 64", who);
  LC_REQUIRE(max_splits <= 65535, "%s: max_splits %lld > 65535", who, (long long)max_splits);
  LC_REQUIRE(max_splits > 0 && max_splits * split_tokens >= max_pages_per_seq * page_size,
             "%s: max_splits * split_tokens must cover the block-table capacity (%lld tokens)",
             who, (long long)(max_pages_per_seq * page_size));
  const int64_t need = lc_paged_decode_workspace_bytes(B, Hq, D, max_splits);
  LC_REQUIRE(workspace_bytes >= need, "%s: workspace %lld < %lld bytes", who,
             (long long)workspace_bytes, (long long)need);
  LC_REQUIRE(lc_aligned(workspace, 256), "%s: workspace not 256-byte aligned", who);
  LC_REQUIRE(lc_aligned(counters, 4), "%s: counters not 4-byte aligned", who);
  LC_REQUIRE(bias == nullptr || (bias_sb >= 0 && bias_sh >= 0 && bias_len >= 0 &&
                                 bias_len < (1LL << 31)),
             "%s: bad bias strides or length", who);
  LC_REQUIRE(bias == nullptr || bias_dtype == LC_DTYPE_F32 || bias_dtype == LC_DTYPE_F16 ||
                 bias_dtype == LC_DTYPE_BF16,
             "%s: unknown bias dtype %d", who, bias_dtype);
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
  a.bias = bias_len > 0 ? bias : nullptr;
  a.bias_sb = bias_sb;
  a.bias_sh = bias_sh;
  a.bias_len = static_cast<int>(bias_len);
  a.bias_dtype = bias_dtype;
  a.ord_ticket = counters;
  a.ord_static = lc_cu_count();

  const int esz = lc_dtype_size(dtype);
  const bool half = dtype == LC_DTYPE_BF16 || dtype == LC_DTYPE_F16;
  const bool mfma = half && D % 8 == 0 && q_sb % 8 == 0 && q_sh % 8 == 0 &&
                    kv_s_page % 8 == 0 && kv_s_head % 8 == 0 && kv_s_tok % 8 == 0 &&
                    lc_aligned(q, 16) && lc_aligned(key_pages, 16) &&
                    lc_aligned(value_pages, 16);
  // Row kernel: every 32-token step stays inside one page, a split touches at
  // most 64 pages (one per lane), and a page's head slice is addressable with
  // 31-bit byte offsets. A split that does not start on a page boundary
  // touches up to (split_tokens - 1) / page_size + 2 pages.
  const bool row_pages = page_size % 32 == 0 &&
                         ((page_size - 1) * kv_s_tok + D) * esz < (1LL << 31);
  const bool rows = row_pages && (split_tokens - 1) / page_size + 2 <= 64;
  // Workgroup splits (one workgroup of W waves per split, the split's steps
  // shared among its waves and merged in LDS) are taken for a single split,
  // for splits of >= 2048 tokens, and when the grid has <= 512 splits (one-wave
  // splits would leave most of the CUs' wave slots empty). Measured against
  // one wave per split: config 2 192 us at 2048-token splits against 197 us
  // at 512; 1024-token splits were 2-5% slower in workgroups on the ragged
  // shapes tried. Every wave's share, whole 32-token steps starting on a step
  // boundary, must fit the row kernel's 64 table entries.
  const int64_t waves = D <= 128 ? cluster_waves<128>() : cluster_waves<256>();
  const int64_t span = max_splits == 1 ? max_pages_per_seq * page_size : split_tokens;
  const int64_t wave_tokens = ((span + kStep - 1) / kStep + waves - 1) / waves * kStep;
  const int64_t units = B * Hkv * ((Hq / Hkv + 15) / 16);
  const bool cluster = row_pages &&
                       (max_splits == 1 || split_tokens >= 2048 || units * max_splits <= 512) &&
                       (wave_tokens - 1) / page_size + 2 <= 64;
  hipStream_t st = lc_stream(stream);
  switch (dtype) {
    case LC_DTYPE_F32:
      return launch_decode<float>(a, out, o_sb, o_sh, lse, false, false, false, st);
    case LC_DTYPE_BF16:
      return launch_decode<bf16_t>(a, out, o_sb, o_sh, lse, mfma, rows, cluster, st);
    case LC_DTYPE_F16:
      return launch_decode<f16_t>(a, out, o_sb, o_sh, lse, mfma, rows, cluster, st);
    default:
      return lc_fail(LC_EINVAL, "%s: unknown dtype %d", who, dtype);
  }
}

// Validates and launches the decode-step fusion (the single-split kernel's
// STEP mode).
int paged_decode_step_impl(const void* q, int64_t q_sb, int64_t q_sh, const void* k,
                           int64_t k_sb, int64_t k_sh, const void* v, int64_t v_sb, int64_t v_sh,
                           const void* cos, const void* sin, int64_t cos_stride,
                           int64_t sin_stride, int64_t table_rows, void* key_pages,
                           void* value_pages, int64_t kv_s_page, int64_t kv_s_head,
                           int64_t kv_s_tok, const int32_t* block_table, int64_t bt_stride,
                           int64_t max_pages_per_seq, int64_t num_pages, int32_t* seq_lens,
                           int32_t* counters, void* out, int64_t o_sb, int64_t o_sh, float* lse,
                           const void* bias, int64_t bias_sb, int64_t bias_sh, int64_t bias_len,
                           int bias_dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                           int64_t page_size, float scale, int dtype, void* stream) {
  static const char* who = "lc_paged_decode_step";
  LC_REQUIRE(B >= 0 && B < 65536, "%s: batch %lld out of range", who, (long long)B);
  if (B == 0) return LC_OK;
  LC_REQUIRE(q && k && v && cos && sin && key_pages && value_pages && block_table && seq_lens &&
                 counters && out,
             "%s: null pointer", who);
  LC_REQUIRE(dtype == LC_DTYPE_BF16 || dtype == LC_DTYPE_F16,
             "%s: dtype must be bf16 or f16 (got %d)", who, dtype);
  LC_REQUIRE(Hq > 0 && Hkv > 0 && Hq % Hkv == 0,
             "%s: n_heads (%lld) must be a multiple of n_kv_heads (%lld)", who, (long long)Hq,
             (long long)Hkv);
  LC_REQUIRE(D >= 16 && D <= 256 && D % 16 == 0,
             "%s: head_dim %lld must be a multiple of 16 in [16, 256]", who, (long long)D);
  LC_REQUIRE(page_size > 0 && page_size % 32 == 0 && max_pages_per_seq > 0 && num_pages > 0,
             "%s: page_size must be a positive multiple of 32, max_pages_per_seq and num_pages "
             "> 0", who);
  const int64_t cap = max_pages_per_seq * page_size;
  LC_REQUIRE(cap < (1LL << 31) && num_pages < (1LL << 31),
             "%s: cache too large for 32-bit token indices", who);
  LC_REQUIRE(bt_stride >= max_pages_per_seq, "%s: bt_stride < row length", who);
  const int64_t waves = D <= 128 ? cluster_waves<128>() : cluster_waves<256>();
  const int64_t wave_tokens = ((cap + kStep - 1) / kStep + waves - 1) / waves * kStep;
  LC_REQUIRE((wave_tokens - 1) / page_size + 2 <= 64,
             "%s: a capacity of %lld tokens is too large for the one-workgroup-per-sequence "
             "kernel (each of its %lld waves covers at most 64 pages); use lc_rope_kv_append "
             "and lc_paged_decode_fwd",
             who, (long long)cap, (long long)waves);
  LC_REQUIRE(((page_size - 1) * kv_s_tok + D) * 2 < (1LL << 31),
             "%s: a page's head slice exceeds 2 GiB", who);
  LC_REQUIRE(table_rows >= cap && table_rows < (1LL << 31),
             "%s: the cos/sin tables (%lld rows) must cover the block-table capacity (%lld "
             "positions)",
             who, (long long)table_rows, (long long)cap);
  LC_REQUIRE(q_sb >= 0 && q_sh >= 0 && k_sb >= 0 && k_sh >= 0 && v_sb >= 0 && v_sh >= 0 &&
                 cos_stride >= 0 && sin_stride >= 0 && kv_s_page >= 0 && kv_s_head >= 0 &&
                 kv_s_tok >= 0,
             "%s: negative stride", who);
  LC_REQUIRE(lc_aligned(q, 16) && q_sb % 8 == 0 && q_sh % 8 == 0 && lc_aligned(cos, 16) &&
                 lc_aligned(sin, 16) && cos_stride % 8 == 0 && sin_stride % 8 == 0 &&
                 lc_aligned(key_pages, 16) && lc_aligned(value_pages, 16) &&
                 kv_s_page % 8 == 0 && kv_s_head % 8 == 0 && kv_s_tok % 8 == 0,
             "%s: q, the cos/sin tables and the pools need 16-byte alignment and strides in "
             "multiples of 8 elements", who);
  LC_REQUIRE(lc_aligned(k, 8) && lc_aligned(v, 8) && k_sb % 4 == 0 && k_sh % 4 == 0 &&
                 v_sb % 4 == 0 && v_sh % 4 == 0,
             "%s: k and v need 8-byte alignment and strides in multiples of 4 elements", who);
  LC_REQUIRE(bias == nullptr || (bias_sb >= 0 && bias_sh >= 0 && bias_len >= 0 &&
                                 bias_len < (1LL << 31)),
             "%s: bad bias strides or length", who);
  LC_REQUIRE(bias == nullptr || bias_dtype == LC_DTYPE_F32 || bias_dtype == LC_DTYPE_F16 ||
                 bias_dtype == LC_DTYPE_BF16,
             "%s: unknown bias dtype %d", who, bias_dtype);

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
  a.B = static_cast<int>(B);
  a.Hq = static_cast<int>(Hq);
  a.Hkv = static_cast<int>(Hkv);
  a.G = static_cast<int>(Hq / Hkv);
  a.D = static_cast<int>(D);
  a.P = static_cast<int>(page_size);
  a.p_shift = (page_size & (page_size - 1)) == 0 ? __builtin_ctzll(page_size) : -1;
  a.split_tokens = static_cast<int>((cap + 63) / 64 * 64);
  a.max_splits = 1;
  a.n_hgroups = (a.G + 15) / 16;
  a.scale_log2 = scale * kLog2e;
  a.bias = bias_len > 0 ? bias : nullptr;
  a.bias_sb = bias_sb;
  a.bias_sh = bias_sh;
  a.bias_len = static_cast<int>(bias_len);
  a.bias_dtype = bias_dtype;

  StepArgs sa{};
  sa.k = k;
  sa.v = v;
  sa.k_sb = k_sb;
  sa.k_sh = k_sh;
  sa.v_sb = v_sb;
  sa.v_sh = v_sh;
  sa.cos = cos;
  sa.sin = sin;
  sa.cs = cos_stride;
  sa.ss = sin_stride;
  sa.table_rows = static_cast<int>(table_rows);
  sa.kp = key_pages;
  sa.vp = value_pages;
  sa.seq_lens = seq_lens;
  sa.counters = counters;
  hipStream_t st = lc_stream(stream);
  if (dtype == LC_DTYPE_BF16) return launch_step_d<bf16_t>(a, sa, out, o_sb, o_sh, lse, st);
  return launch_step_d<f16_t>(a, sa, out, o_sb, o_sh, lse, st);
}

// Device scratch of lc_paged_decode_fwd_noalloc, one per device (its address
// differs per device). Host code uses the address kept in g_scratch_ptr, never
// the symbol itself (on the host the name is only a handle).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's scratch address, looked up once per device; the
// stream must belong to the current device.
int scratch_for_stream(const char* who, void* stream, void** out);

}  // namespace

static __device__ __align__(256) unsigned char scratch[LC_DECODE_NOALLOC_SCRATCH_BYTES];

namespace {

int scratch_for_stream(const char* who, void* stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return lc_fail(static_cast<int>(e), "%s: hipGetDevice failed: %s", who,
                                      hipGetErrorString(e));
  if (stream != nullptr) {
    int sdev = -1;
    e = hipStreamGetDevice(lc_stream(stream), &sdev);
    if (e != hipSuccess)
      return lc_fail(static_cast<int>(e), "%s: hipStreamGetDevice failed: %s", who,
                     hipGetErrorString(e));
    if (sdev != dev)
      return lc_fail(LC_EINVAL, "%s: the stream belongs to device %d, the current device is %d",
                     who, sdev, dev);
  }
  if (dev < 0 || dev >= kMaxDevices)
    return lc_fail(LC_EUNSUPPORTED, "%s: device %d beyond the %d this library tracks", who, dev,
                   kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return lc_fail(e != hipSuccess ? static_cast<int>(e) : LC_EUNSUPPORTED,
                     "%s: no address for the device scratch on device %d: %s", who, dev,
                     hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return LC_OK;
}

}  // namespace

extern "C" {

int64_t lc_paged_decode_counter_count(void) { return kDecodeCounterInts; }

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
                        void* out, int64_t o_sb, int64_t o_sh, float* lse, const void* bias,
                        int64_t bias_sb, int64_t bias_sh, int64_t bias_len, int bias_dtype,
                        void* workspace, int64_t workspace_bytes, int32_t* counters,
                        int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t page_size,
                        int64_t split_tokens, int64_t max_splits, float scale, int dtype,
                        void* stream) {
  return paged_decode_impl("lc_paged_decode_fwd", q, q_sb, q_sh, key_pages, value_pages,
                           kv_s_page, kv_s_head, kv_s_tok, block_table, bt_stride,
                           max_pages_per_seq, num_pages, seq_lens, out, o_sb, o_sh, lse, bias,
                           bias_sb, bias_sh, bias_len, bias_dtype, workspace, workspace_bytes,
                           counters, B, Hq, Hkv, D, page_size, split_tokens, max_splits, scale,
                           dtype, stream);
}

int lc_paged_decode_fwd_noalloc(const void* q, int64_t q_sb, int64_t q_sh,
                                const void* key_pages, const void* value_pages,
                                int64_t kv_s_page, int64_t kv_s_head, int64_t kv_s_tok,
                                const int32_t* block_table, int64_t bt_stride,
                                int64_t max_pages_per_seq, int64_t num_pages,
                                const int32_t* seq_lens, void* out, int64_t o_sb, int64_t o_sh,
                                float* lse, const void* bias, int64_t bias_sb, int64_t bias_sh,
                                int64_t bias_len, int bias_dtype, int64_t B, int64_t Hq,
                                int64_t Hkv, int64_t D, int64_t page_size, int64_t split_tokens,
                                int64_t max_splits, float scale, int dtype, void* stream) {
  static const char* who = "lc_paged_decode_fwd_noalloc";
  if (B == 0) return LC_OK;
  const int64_t need = lc_paged_decode_workspace_bytes(B, Hq, D, max_splits);
  if (need > LC_DECODE_NOALLOC_SCRATCH_BYTES)
    return lc_fail(LC_EWORKSPACE,
                   "%s: %lld bytes of split partials (batch %lld x %lld heads x %lld splits x "
                   "head_dim %lld) exceed the %lld-byte device scratch; use fewer or larger "
                   "splits, or lc_paged_decode_fwd with a workspace",
                   who, (long long)need, (long long)B, (long long)Hq, (long long)max_splits,
                   (long long)D, (long long)LC_DECODE_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = scratch_for_stream(who, stream, &ws);
  if (rc != LC_OK) return rc;
  // No part of the scratch needs clearing: every split with tokens writes its
  // partials, and the merge reads only those splits. No ticket either (the
  // static longest-first order), so nothing here has to start at zero.
  return paged_decode_impl(who, q, q_sb, q_sh, key_pages, value_pages, kv_s_page, kv_s_head,
                           kv_s_tok, block_table, bt_stride, max_pages_per_seq, num_pages,
                           seq_lens, out, o_sb, o_sh, lse, bias, bias_sb, bias_sh, bias_len,
                           bias_dtype, ws, LC_DECODE_NOALLOC_SCRATCH_BYTES, nullptr, B, Hq,
                           Hkv, D, page_size, split_tokens, max_splits, scale, dtype, stream);
}

int lc_paged_decode_step(const void* q, int64_t q_sb, int64_t q_sh, const void* k,
                         int64_t k_sb, int64_t k_sh, const void* v, int64_t v_sb, int64_t v_sh,
                         const void* cos, const void* sin, int64_t cos_stride, int64_t sin_stride,
                         int64_t table_rows, void* key_pages, void* value_pages,
                         int64_t kv_s_page, int64_t kv_s_head, int64_t kv_s_tok,
                         const int32_t* block_table, int64_t bt_stride,
                         int64_t max_pages_per_seq, int64_t num_pages, int32_t* seq_lens,
                         int32_t* counters, void* out, int64_t o_sb, int64_t o_sh, float* lse,
                         const void* bias, int64_t bias_sb, int64_t bias_sh, int64_t bias_len,
                         int bias_dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                         int64_t page_size, float scale, int dtype, void* stream) {
  return paged_decode_step_impl(q, q_sb, q_sh, k, k_sb, k_sh, v, v_sb, v_sh, cos, sin,
                                cos_stride, sin_stride, table_rows, key_pages, value_pages,
                                kv_s_page, kv_s_head, kv_s_tok, block_table, bt_stride,
                                max_pages_per_seq, num_pages, seq_lens, counters, out, o_sb, o_sh,
                                lse, bias, bias_sb, bias_sh, bias_len, bias_dtype, B, Hq, Hkv, D,
                                page_size, scale, dtype, stream);
}

}  // extern "C"
