// Causal attention forward (prefill) with native GQA and logsumexp output.
//
// Two kernels, chosen by dtype and head_dim:
//   * prefill_mfma_kernel (bf16/f16, D a multiple of 8 up to 128): flash
//     attention on v_mfma_f32_32x32x16_{bf16,f16} with K/V tiles
//     double-buffered through LDS.
//   * prefill_generic_kernel (everything else, incl. fp32): one lane per query
//     row, fp32 FMA, K/V tiles staged through LDS.
// Both compute, for query row i of (b, h) and keys j < Skv with
// j <= i + q_offset: o = softmax(q.k_j * scale + bias_ij) v, lse = ln-sum-exp,
// where the optional additive bias (an attention mask) is read through
// broadcast strides.
#include <math.h>

#include <type_traits>

#include "attn_tiles.h"
#include "lc_common.h"

namespace {

using namespace lc_attn;

struct PrefillArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  int64_t qs[4], ks[4], vs[4], os[4];
  int B, Hq, Hkv, G, Sq, Skv, D, q_offset;
  float scale_log2;
  // Additive bias [B, Hq, Sq, Skv] with element strides bs (0 = broadcast);
  // null: none. bias_dtype is LC_DTYPE_*; bias_vec: the MFMA kernel may read
  // 4 consecutive keys with one load (see BiasTile).
  const void* bias;
  int64_t bs[4];
  int bias_dtype;
  int bias_vec;
  // Dynamic tail (no bias): a ticket that is zero at entry and left zero, and
  // the lightest dyn_light row groups of each of the dyn_units units handed
  // out through it; dyn_light == 0: every workgroup's item from its block id.
  int* ticket;
  int dyn_units, dyn_light;
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
  const int64_t brow = b * a.bs[0] + h * a.bs[1] + (int64_t)i * a.bs[2];
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
      if (a.bias != nullptr) {
        s += lc_bias_log2(lc_load_bias(a.bias, brow + (int64_t)(j0 + r) * a.bs[3], a.bias_dtype));
        if (s == -INFINITY) continue;  // key excluded by the mask
      }
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

// ---------------------------------------------------------------------------
// MFMA kernel (bf16/f16, D in {64, 128}).
//
// Workgroup = 4 waves that share one kv head: wave w computes 32 query rows of
// one q head. The workgroup covers HW = gcd(G, 4) heads of the kv group times
// 4 / HW blocks of 32 rows (G = 4: the group's 4 heads on the same rows), so
// every K/V tile staged in LDS feeds 4 waves. Two workgroups share a CU.
//
// Per 64-key tile and wave:
//   S^T[32 keys x 32 q] = K[32 keys x 16 d] * Q^T[16 d x 32 q], D/16 k-steps
//   per 32-key half, on v_mfma_f32_32x32x16_{bf16,f16}. Q^T stays in
//   registers (lane: query row l % 32, d = (l / 32) * D/2 + 8s .. +8); K
//   operands are ds_read_b128 of K rows in the same d order.
//   Keys land on accumulator rows (8j + 4h + i, h = l / 32) and queries on
//   lanes, so a query's max/sum over keys is 16 in-lane values + 1 swap.
//   O^T[32 d x 32 q] += V^T[32 d x 16 keys] * P^T[16 keys x 32 q]: the MFMA k
//   index h*8 + jj*4 + i is mapped to key 16jp + 8jj + 4h + i, so each lane's
//   P^T operand is its own S^T registers (rounded to bf16/f16); V^T operands
//   come from ds_read_b64_tr_b16 (4 keys x 16 d per 16-lane group).
//
// Software pipeline. The softmax of a tile is split in two halves:
//   SM1(t): mask, row max, running-max update, x = s * scale_log2 - m;
//   SM2(t): p = 2^x, row sum, P rounded to the MFMA type.
// Iteration t interleaves, in one instruction stream,
//   part A: QK^T of tile t+1 (MFMA) with SM2(t) (VALU);
//   part B: P(t) V(t) (MFMA) with SM1(t+1) (VALU),
// so the matrix cores and the VALU of one wave work side by side. A rescale
// of O (rare: the running max grew by more than 2^8) is applied after part B.
// Without a bias, only the first tile takes a row max: later tiles shift by
// the reference max as it stands, and a check between part A and part B
// (every lane's tile sum <= 2^8, which holds whenever every p <= 2^8) sends
// the rare tiles that fail it through a fix-up that takes their row max from
// the exponents and rescales every row that grew before their PV. The max tree and its ballot
// leave the loop (about a fifth of its non-exp VALU work).
// LDS holds two K and two V tile buffers as separate arrays. Iteration t reads
// K(t+1), V(t) and fetches K(t+2), V(t+1) by buffer-to-LDS DMA into the other
// two; one barrier per iteration publishes them. Reads and DMA targets are
// distinct LDS objects, so the compiler does not make the reads wait for the
// DMA in flight.
// ---------------------------------------------------------------------------
constexpr int kPfWaves = 4;
constexpr int kPfRows = 32;     // query rows per wave
constexpr int kPfKeys = 64;     // keys per tile
constexpr float kPfRescaleLog2 = 8.0f;
// int32 counters lc_prefill_attn_fwd takes: the dynamic tail's ticket, padded to 256 bytes.
constexpr int kPrefillCounterInts = 64;

// With an additive bias (BIAS != 0) the kernel runs one wave per SIMD: the
// bias tile held one iteration ahead does not fit the two-wave register
// budget without spills.
template <typename T, int DPAD, int BIAS>
__global__ __launch_bounds__(64 * kPfWaves) __attribute__((
    amdgpu_waves_per_eu(BIAS == 0 ? 2 : 1, BIAS == 0 ? 2 : 1))) void
prefill_mfma_kernel(PrefillArgs a, int hw, int n_rbg) {
  typedef Mfma32<T> Ops;
  typedef typename Ops::v8 v8;
  constexpr int KS = DPAD / 16;          // QK^T k-steps (16 d each)
  constexpr int DTL = DPAD / 32;         // 32-row d tiles of O^T
  constexpr int CPR = DPAD / 8;          // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;          // rows per 1 KB LDS-DMA instruction
  constexpr int NIW = kPfKeys / (RPI * kPfWaves);  // DMA instructions per wave per tile
  constexpr int TILE_B = kPfKeys * DPAD * (int)sizeof(T);  // bytes per K or V tile
  constexpr int ROW_B = DPAD * (int)sizeof(T);
  // K and V tile buffers (unpadded, chunks swizzled by pf_swz).
  __shared__ __align__(16) char lds_k0[TILE_B];
  __shared__ __align__(16) char lds_k1[TILE_B];
  __shared__ __align__(16) char lds_v0[TILE_B];
  __shared__ __align__(16) char lds_v1[TILE_B];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // Scalar copy for the DMA destinations (M0). Control flow keeps using the
  // vector copy: with every bound provably uniform the optimizer unswitches
  // the tile loop into many copies and the register allocation breaks down.
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  const int rbw = kPfWaves / hw;
  const int n_hg = a.G / hw;
  // XCD-aware order: the dispatcher deals consecutive workgroups round-robin
  // to the 8 XCDs (each with its own L2). Work item W = xcd * per_xcd + k is
  // given to the k-th workgroup landing on XCD xcd, so each XCD walks whole
  // (b, kv head, head group) units in turn and their K/V stays in its L2.
  // Within a unit the heaviest (latest) row groups come first, reversed in
  // every other run of four (pf_snake) so the XCD's shader engines get equal
  // shares.
  const int nwg = gridDim.x;
  //
  // Dynamic tail (dyn_light > 0): the XCDs run at different clocks, so the
  // lightest dyn_light row groups of every unit are not tied to an XCD. Block
  // ids below S = units x (n_rbg - dyn_light) walk the heavier row groups in
  // the order above (whole units per XCD); the others draw a rank t from the
  // ticket as they start, t-th of the light row groups heaviest first across
  // all units, and the extra workgroups past them (a spare pool, so that the
  // XCDs that finish first can take more) leave at once. Every workgroup from
  // S on draws exactly once, so the one that draws the last value returns the
  // ticket to zero.
  const int lin = blockIdx.x;
  int unit, rbg;
  if (BIAS == 0 && a.dyn_light > 0) {
    const int heavy = n_rbg - a.dyn_light;
    const int S = a.dyn_units * heavy;
    if (lin < S) {
      const int w = (lin & 7) * (S >> 3) + (lin >> 3);
      unit = w / heavy;
      rbg = n_rbg - 1 - pf_snake(w - unit * heavy, heavy);
    } else {
      __shared__ int s_rank;
      if (tid == 0) {
        const int t = __hip_atomic_fetch_add(a.ticket, 1, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        if (t == nwg - S - 1)
          __hip_atomic_store(a.ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_rank = t;
      }
      __syncthreads();
      // (wave-uniform: kept in SGPRs, as the block-id path's values are, so
      // the tile loop's addressing compiles as it does without the ticket)
      const int t = __builtin_amdgcn_readfirstlane(s_rank);
      if (t >= a.dyn_units * a.dyn_light) return;
      unit = t % a.dyn_units;
      rbg = a.dyn_light - 1 - t / a.dyn_units;
    }
  } else {
    int work = lin;
    if ((nwg & 7) == 0) work = (lin & 7) * (nwg >> 3) + (lin >> 3);
    unit = work / n_rbg;
    rbg = n_rbg - 1 - pf_snake(work - unit * n_rbg, n_rbg);
  }
  // Opaque from here on: the tile loop must not see which path chose them
  // (with both paths visible its register allocation grew past the budget).
  unit = __builtin_amdgcn_readfirstlane(unit);
  rbg = __builtin_amdgcn_readfirstlane(rbg);
  asm volatile("" : "+s"(unit), "+s"(rbg));
  const int kvh_hg = unit % (a.Hkv * n_hg);
  const int b = unit / (a.Hkv * n_hg);
  const int kvh = kvh_hg / n_hg;
  const int hgi = kvh_hg - kvh * n_hg;
  const int head = kvh * a.G + hgi * hw + (wave % hw);
  const int r0 = (rbg * rbw + wave / hw) * kPfRows;
  const int wg_last_row = min(a.Sq - 1, (rbg * rbw + rbw) * kPfRows - 1);
  const int kv_end = min(a.Skv, wg_last_row + a.q_offset + 1);  // keys any wave needs
  const int my_kv_end = min(a.Skv, min(a.Sq - 1, r0 + kPfRows - 1) + a.q_offset + 1);
  // Tiles entirely below this key bound are visible to every row of the wave.
  const int nomask_end = min(a.Skv, r0 + a.q_offset + 1);
  const bool wave_active = r0 < a.Sq;

  const T* qbase = static_cast<const T*>(a.q) + b * a.qs[0] + (int64_t)head * a.qs[1];
  const T* kbase = static_cast<const T*>(a.k) + b * a.ks[0] + (int64_t)kvh * a.ks[1];
  const T* vbase = static_cast<const T*>(a.v) + b * a.vs[0] + (int64_t)kvh * a.vs[1];
  // Buffer descriptors over this (b, kv head)'s K and V rows: rows past the
  // last key are out of range and land in LDS as zeros.
  const int kbytes = a.Skv > 0 ? static_cast<int>(((int64_t)(a.Skv - 1) * a.ks[2] + a.D) * sizeof(T)) : 0;
  const int vbytes = a.Skv > 0 ? static_cast<int>(((int64_t)(a.Skv - 1) * a.vs[2] + a.D) * sizeof(T)) : 0;

  // Additive bias (BIAS != 0): this (b, head)'s slice through one buffer
  // descriptor; the tile's values are loaded one iteration ahead of the SM1
  // that adds them (see BiasTile).
  const int qi = r0 + l32;
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
  auto load_bias = [&](int t) __attribute__((always_inline)) {
    if constexpr (BIAS != 0) btile.load(brs, brow_b, t * kPfKeys, hh, bs3_b, a.bias_vec != 0);
  };

  // Q^T operand registers.
  v8 qop[KS];
  {
    const bool ok = wave_active && qi < a.Sq;
    const T* qrow = qbase + (int64_t)qi * a.qs[2] + hh * (DPAD / 2);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int d = hh * (DPAD / 2) + s * 8;
      qop[s] = (ok && d < a.D) ? *reinterpret_cast<const v8*>(qrow + s * 8) : v8{};
    }
  }

  // Loop-invariant per-lane byte offsets.
  // LDS-DMA loads: instruction u of this wave fills rows (wave*NIW + u)*RPI ..;
  // lane l writes row + l / CPR at position l % CPR, i.e. global chunk
  // (l % CPR) ^ pf_swz(row) (chunks past head_dim re-read chunk 0: their K
  // meets zero Q elements and their V lands in discarded output rows).
  PfLoadOffsets<NIW> koff, voff;
#pragma unroll
  for (int u = 0; u < NIW; ++u) {
    const int row = (wave * NIW + u) * RPI + lane / CPR;
    int ch = (lane % CPR) ^ pf_swz<CPR>(row);
    ch = ch * 8 < a.D ? ch : 0;
    koff.o[u] = static_cast<int>(((int64_t)row * a.ks[2] + ch * 8) * sizeof(T));
    voff.o[u] = static_cast<int>(((int64_t)row * a.vs[2] + ch * 8) * sizeof(T));
  }
  const int kstep_b = static_cast<int>(kPfKeys * a.ks[2] * sizeof(T));
  const int vstep_b = static_cast<int>(kPfKeys * a.vs[2] * sizeof(T));
  // K operand reads: row kt*32 + l32, chunk hh*CPR/2 + s (kt is an immediate).
  int kaddr[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s)
    kaddr[s] = l32 * ROW_B + (((hh * (CPR / 2) + s) ^ pf_swz<CPR>(l32)) << 4);
  // V^T transposed reads: 16-lane group gq covers keys 4hh .. 4hh+3 (+8jj,
  // +16jp, +32kt as immediates) and d = dt*32 + (gq & 1)*16 .. +15; lane
  // 4e + c addresses key +e, d + 4c.
  int vaddr[2][DTL];
  {
    const int gq = lane >> 4, te = (lane & 15) >> 2, tc = lane & 3;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int dt = 0; dt < DTL; ++dt) {
        const int kr = jj * 8 + hh * 4 + te;
        const int d = dt * 32 + (gq & 1) * 16 + 4 * tc;
        vaddr[jj][dt] = kr * ROW_B + ((((d >> 3) ^ pf_swz<CPR>(kr)) << 4) | ((d & 7) * (int)sizeof(T)));
      }
  }

  f32x16_t o[DTL];
#pragma unroll
  for (int i = 0; i < DTL; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[i][r] = 0.f;
  float m_ref = -INFINITY, l_lane = 0.f;
  f32x16_t snx[2];  // raw S^T of the next tile (QK^T output)
  f32x16_t xcu[2];  // exponents of the current tile (SM1 output)
  v8 pop[2][2];     // P^T operands of the current tile (SM2 output)
  float alpha = 1.f;
  bool rescale = false;
  float l_tile = 0.f;  // this lane's share of the current tile's row sum
  const int n_tiles = (kv_end + kPfKeys - 1) / kPfKeys;

  auto kbuf = [&](auto p_c) __attribute__((always_inline)) -> LC_LDS char* {
    if constexpr (decltype(p_c)::value == 0) return (LC_LDS char*)lds_k0;
    else return (LC_LDS char*)lds_k1;
  };
  auto vbuf = [&](auto p_c) __attribute__((always_inline)) -> LC_LDS char* {
    if constexpr (decltype(p_c)::value == 0) return (LC_LDS char*)lds_v0;
    else return (LC_LDS char*)lds_v1;
  };
  auto live = [&](int t) __attribute__((always_inline)) {
    return wave_active && t < n_tiles && t * kPfKeys < my_kv_end;
  };

  auto qk = [&](LC_LDS const char* kt_lds) __attribute__((always_inline)) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) snx[kt][r] = 0.f;
    // The two 32-key halves alternate, so consecutive MFMAs are independent.
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
        snx[kt] = Ops::mma(*reinterpret_cast<LC_LDS const v8*>(kt_lds + kaddr[s] + kt * 32 * ROW_B),
                           qop[s], snx[kt]);
  };
  auto pv = [&](LC_LDS const char* vt_lds) __attribute__((always_inline)) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int jp = 0; jp < 2; ++jp)
#pragma unroll
        for (int dt = 0; dt < DTL; ++dt) {
          const int rowoff = (kt * 32 + jp * 16) * ROW_B;
          const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (LC_LDS i16x4_t*)(vt_lds + vaddr[0][dt] + rowoff));
          const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (LC_LDS i16x4_t*)(vt_lds + vaddr[1][dt] + rowoff));
          const i16x8_t both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
          o[dt] = Ops::mma(__builtin_bit_cast(v8, both), pop[kt][jp], o[dt]);
        }
  };
  // SM1 of the tile whose raw scores are in snx (keys k0 ..): sets xcu, the
  // running max and row sum; a required rescale of O is left to apply_rescale.
  auto sm1 = [&](int k0, auto mask_c) __attribute__((always_inline)) {
    if constexpr (BIAS != 0) {
      // Scores with the bias, in the exp2 domain.
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) snx[kt][r] = fmaf(snx[kt][r], a.scale_log2, btile.log2_at(kt, r));
    }
    if constexpr (decltype(mask_c)::value) {
      // Key k0 + c + 4hh (c the element's compile-time offset) is visible
      // while k0 + c + 4hh <= qi + q_offset and < Skv, i.e. c < key_lim.
      const int key_lim = min(qi + a.q_offset + 1, a.Skv) - k0 - hh * 4;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kt * 32 + (r >> 2) * 8 + (r & 3) >= key_lim) snx[kt][r] = -INFINITY;
    }
    // Without a bias raw scores are maxed and the scale (> 0) is applied with
    // the shift; with one they are already in the exp2 domain.
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, snx[kt][r]);
    mx = pf_half_max(mx);
    if constexpr (BIAS == 0) mx *= a.scale_log2;
    // The reference max only moves when some row's max grew by more than 2^8
    // (exact: O and l always share it).
    rescale = __ballot(mx > m_ref + kPfRescaleLog2) != 0;
    const float m_new = rescale ? fmaxf(m_ref, mx) : m_ref;
    alpha = m_new == -INFINITY ? 1.f : lc_exp2(m_ref - m_new);
    l_lane *= alpha;
    m_ref = m_new;
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        xcu[kt][r] = BIAS == 0 ? fmaf(snx[kt][r], a.scale_log2, -m_use) : snx[kt][r] - m_use;
  };
  auto sm2 = [&]() __attribute__((always_inline)) {
    // P^T operands: step (kt, jp) takes accumulator rows j = 2jp, 2jp + 1.
    // The row sum stays in fp32 (a sum of rounded P would cost the lse up to
    // 2^-9 relative when one key dominates).
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = lc_exp2(xcu[kt][r]);
        l_lane += p;
        pop[kt][r >> 3][r & 7] = static_cast<T>(p);
      }
  };
  auto apply_rescale = [&]() __attribute__((always_inline)) {
    if (__builtin_expect(rescale, 0)) {
#pragma unroll
      for (int dt = 0; dt < DTL; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
      rescale = false;
    }
  };

  // Without a bias, tiles after the first skip the row max: SM1L shifts by
  // the current reference max, SM2L exponentiates and sums, and check_fix
  // catches every tile where some p exceeds 2^8 (its lane's tile sum then
  // does too): that tile's row max is taken from its exponents, and rows
  // whose max grew move their reference max there (O and l rescaled, the
  // tile's p recomputed) before the tile's PV.
  auto sm1l = [&](int k0, auto mask_c) __attribute__((always_inline)) {
    if constexpr (decltype(mask_c)::value) {
      // Key k0 + c + 4hh (c the element's compile-time offset) is visible
      // while k0 + c + 4hh <= qi + q_offset and < Skv, i.e. c < key_lim.
      const int key_lim = min(qi + a.q_offset + 1, a.Skv) - k0 - hh * 4;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kt * 32 + (r >> 2) * 8 + (r & 3) >= key_lim) snx[kt][r] = -INFINITY;
    }
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) xcu[kt][r] = fmaf(snx[kt][r], a.scale_log2, -m_ref);
  };
  auto sm2l = [&]() __attribute__((always_inline)) {
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = lc_exp2(xcu[kt][r]);
        if (kt == 0) s0 += p; else s1 += p;
        pop[kt][r >> 3][r & 7] = static_cast<T>(p);
      }
    l_tile = s0 + s1;
  };
  auto check_fix = [&]() __attribute__((always_inline)) {
    if (__builtin_expect(__ballot(l_tile > 256.f) != 0, 0)) {
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, xcu[kt][r]);
      mx = pf_half_max(mx);
      // Every row whose max grew moves its reference max there (as the
      // max-tree path does once any row passes the threshold), so after a
      // fix every row's largest p is 1: leaving rows below the threshold
      // where they were measured less accurate on scores that climb steadily
      // (a larger O error, and one that the backward's dq then amplifies).
      const float d = mx > 0.f ? mx : 0.f;
      const float al = lc_exp2(-d);
      m_ref += d;
      l_lane *= al;
#pragma unroll
      for (int dt = 0; dt < DTL; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] *= al;
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = lc_exp2(xcu[kt][r] - d);
          if (kt == 0) s0 += p; else s1 += p;
          pop[kt][r >> 3][r & 7] = static_cast<T>(p);
        }
      l_tile = s0 + s1;
    }
    l_lane += l_tile;
  };

  // Iteration t (PAR = t & 1): reads K(t+1) from K buffer PAR ^ 1 and V(t)
  // from V buffer PAR; fetches K(t+2) -> K buffer PAR, V(t+1) -> V buffer
  // PAR ^ 1. MASK: tile t+1 needs the causal / key-range mask.
  auto iteration = [&](int t, auto par_c, auto mask_c) __attribute__((always_inline)) {
    constexpr int PAR = decltype(par_c)::value;
    constexpr auto other = std::integral_constant<int, PAR ^ 1>{};
    // The bias of tile t+1 (added in this iteration's SM1) is loaded before
    // the DMA, so that waiting for it does not wait for the DMA too.
    if (live(t + 1)) load_bias(t + 1);
    if (t + 2 < n_tiles)
      pf_dma_tile<NIW, RPI, ROW_B>(kbase, kbytes, kbuf(par_c), wave_s, koff, (t + 2) * kstep_b);
    if (t + 1 < n_tiles)
      pf_dma_tile<NIW, RPI, ROW_B>(vbase, vbytes, vbuf(other), wave_s, voff, (t + 1) * vstep_b);
    const int k1 = (t + 1) * kPfKeys;
    const bool cur = live(t), nxt = live(t + 1);
    if constexpr (BIAS == 0) {
      if (cur && nxt) {
        constexpr int NQ = 2 * KS, NP = 4 * DTL, LA = 4;
        qk(kbuf(other));
        sm2l();
        __builtin_amdgcn_sched_group_barrier(0x100, LA, 0);
#pragma unroll
        for (int j = 0; j < NQ; ++j) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if (j + LA < NQ) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
        }
        check_fix();
        pv(vbuf(par_c));
        sm1l(k1, mask_c);
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * LA, 0);
#pragma unroll
        for (int j = 0; j < NP; ++j) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if (j + LA < NP) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
        }
      } else {
        if (nxt) qk(kbuf(other));
        if (cur) {
          sm2l();
          check_fix();
          pv(vbuf(par_c));
        }
        if (nxt) sm1l(k1, mask_c);
      }
      pf_barrier<true>();
      return;
    }
    if (cur && nxt) {
      qk(kbuf(other));
      sm2();
      pv(vbuf(par_c));
      sm1(k1, mask_c);
      // Part A: 16 QK^T MFMAs, each followed by one K read 4 MFMAs ahead and
      // SM2 VALU work; part B: 16 PV MFMAs, each with two V^T reads ahead
      // and SM1 VALU work.
      constexpr int NQ = 2 * KS, NP = 4 * DTL, LA = 4;
      __builtin_amdgcn_sched_group_barrier(0x100, LA, 0);
#pragma unroll
      for (int j = 0; j < NQ + NP; ++j) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        const int nx = j + LA;
        if (nx < NQ)
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        else if (nx < NQ + NP)
          __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
      }
    } else {
      if (nxt) qk(kbuf(other));
      if (cur) {
        sm2();
        pv(vbuf(par_c));
      }
      if (nxt) sm1(k1, mask_c);
    }
    apply_rescale();
    pf_barrier<true>();  // this wave's DMA landed, every wave done with K(t+1), V(t)
  };

  // Prologue: K(0), V(0), K(1) in LDS; S(0) through SM1.
  if (n_tiles > 0) {
    pf_dma_tile<NIW, RPI, ROW_B>(kbase, kbytes, kbuf(std::integral_constant<int, 0>{}), wave_s,
                                 koff, 0);
    pf_dma_tile<NIW, RPI, ROW_B>(vbase, vbytes, vbuf(std::integral_constant<int, 0>{}), wave_s,
                                 voff, 0);
    if (n_tiles > 1)
      pf_dma_tile<NIW, RPI, ROW_B>(kbase, kbytes, kbuf(std::integral_constant<int, 1>{}), wave_s,
                                   koff, kstep_b);
  }
  if (live(0)) load_bias(0);
  pf_barrier<true>();
  if (live(0)) {
    qk(kbuf(std::integral_constant<int, 0>{}));
    sm1(0, std::true_type{});
    rescale = false;  // O is still zero
  }
  pf_barrier<false>();  // K buffer 0 is refilled in iteration 0
  // Iterations whose next tile needs no mask, then the rest (the diagonal
  // band); two loops rather than a branch per iteration, so each loop body
  // is a single straight-line interleaved block.
  const int t_mask = min(n_tiles, max(0, nomask_end / kPfKeys - 1));
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

  if (!wave_active) return;
  float l_tot = l_lane + __shfl_xor(l_lane, 32, 64);
  if (qi >= a.Sq) return;
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  T* orow = static_cast<T*>(a.o) + b * a.os[0] + (int64_t)head * a.os[1] + (int64_t)qi * a.os[2];
#pragma unroll
  for (int dt = 0; dt < DTL; ++dt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d = dt * 32 + j * 8 + hh * 4;
      if (d < a.D) {
        typedef T t4 __attribute__((ext_vector_type(4)));
        t4 w;
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = lc_from_f32<T>(o[dt][j * 4 + i] * inv);
        *reinterpret_cast<t4*>(orow + d) = w;
      }
    }
  if (a.lse != nullptr && hh == 0)
    a.lse[((int64_t)b * a.Hq + head) * a.Sq + qi] =
        l_tot > 0.f ? (m_ref + lc_log2(l_tot)) * kLn2 : -INFINITY;
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
void launch_mfma_bias(const PrefillArgs& a, dim3 grid, int hw, int n_rbg, hipStream_t st) {
  if (a.D <= 64)
    prefill_mfma_kernel<T, 64, BIAS><<<grid, 64 * kPfWaves, 0, st>>>(a, hw, n_rbg);
  else
    prefill_mfma_kernel<T, 128, BIAS><<<grid, 64 * kPfWaves, 0, st>>>(a, hw, n_rbg);
}

template <typename T>
int launch_mfma(const PrefillArgs& a, hipStream_t st) {
  const int hw = gcd_int(a.G, kPfWaves);
  const int rbw = kPfWaves / hw;
  const int n_rb = (a.Sq + kPfRows - 1) / kPfRows;
  const int n_rbg = (n_rb + rbw - 1) / rbw;
  const int64_t nwg = (int64_t)n_rbg * a.Hkv * (a.G / hw) * a.B;
  LC_REQUIRE(nwg < (1LL << 31), "lc_prefill_attn_fwd: grid too large");
  dim3 grid(static_cast<unsigned>(nwg));
  // Dynamic tail: with a ticket, no bias, whole units per XCD (units a
  // multiple of 8), >= 8 row groups per unit and more than two rounds of
  // workgroups (two per CU). Measured at config 3 against the static order in
  // one process (two boxes): 0.5165 vs 0.5213 ms and 0.5073 vs 0.5114 ms with
  // a light quarter and a spare pool of nwg / 16; a third, a fifth, or spare
  // pools of nwg / 8 and nwg / 32 were no better.
  const int units = static_cast<int>(nwg / n_rbg);
  if (a.ticket != nullptr && a.bias == nullptr && units % 8 == 0 && n_rbg >= 8 &&
      nwg > 2LL * lc_cu_count()) {
    PrefillArgs d = a;
    d.dyn_units = units;
    d.dyn_light = n_rbg / 4;
    const int64_t spare = nwg / 16;
    LC_REQUIRE(nwg + spare < (1LL << 31), "lc_prefill_attn_fwd: grid too large");
    launch_mfma_bias<T, 0>(d, dim3(static_cast<unsigned>(nwg + spare)), hw, n_rbg, st);
  } else if (a.bias == nullptr)
    launch_mfma_bias<T, 0>(a, grid, hw, n_rbg, st);
  else if (a.bias_dtype == LC_DTYPE_F32)
    launch_mfma_bias<T, 2>(a, grid, hw, n_rbg, st);
  else
    launch_mfma_bias<T, 1>(a, grid, hw, n_rbg, st);
  return lc_check_launch("lc_prefill_attn_fwd (mfma)");
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

int64_t lc_prefill_attn_counter_count(void) { return kPrefillCounterInts; }

int lc_prefill_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                        int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Skv, int64_t D,
                        const int64_t* q_strides, const int64_t* k_strides,
                        const int64_t* v_strides, const int64_t* o_strides, int64_t q_offset,
                        const void* bias, const int64_t* bias_strides, int bias_dtype,
                        int32_t* counters, float scale, int dtype, void* stream) {
  LC_REQUIRE(q_strides && k_strides && v_strides && o_strides,
             "lc_prefill_attn_fwd: null stride array");
  LC_REQUIRE(lc_aligned(counters, 4), "lc_prefill_attn_fwd: counters not 4-byte aligned");
  LC_REQUIRE(B >= 0 && B < 65536 && Sq >= 0 && Skv >= 0, "lc_prefill_attn_fwd: bad shape");
  // Pointers of empty tensors may be null.
  LC_REQUIRE((q && o) || B * Sq == 0, "lc_prefill_attn_fwd: null q or o");
  LC_REQUIRE((k && v) || B * Skv == 0, "lc_prefill_attn_fwd: null k or v");
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
  LC_REQUIRE(bias == nullptr || bias_strides != nullptr,
             "lc_prefill_attn_fwd: bias without bias_strides");
  LC_REQUIRE(bias == nullptr || bias_dtype == LC_DTYPE_F32 || bias_dtype == dtype,
             "lc_prefill_attn_fwd: bias dtype must be fp32 or the dtype of q");
  if (bias != nullptr)
    for (int i = 0; i < 4; ++i)
      LC_REQUIRE(bias_strides[i] >= 0, "lc_prefill_attn_fwd: negative bias stride");
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
  a.bias = Skv > 0 ? bias : nullptr;
  a.bias_dtype = bias_dtype;
  a.ticket = counters;
  if (bias != nullptr)
    for (int i = 0; i < 4; ++i) a.bs[i] = bias_strides[i];
  hipStream_t st = lc_stream(stream);
  // MFMA path: 16-bit types, D a multiple of 8 up to 128 (padded to 64 or
  // 128), 16-byte aligned rows.
  const int64_t esz = lc_dtype_size(dtype);
  bool mfma = (dtype == LC_DTYPE_BF16 || dtype == LC_DTYPE_F16) && D % 8 == 0 && D <= 128 &&
              lc_aligned(q, 16) && lc_aligned(k, 16) && lc_aligned(v, 16) && lc_aligned(o, 16) &&
              (Skv * k_strides[2] + D) * esz < (1LL << 31) &&
              (Skv * v_strides[2] + D) * esz < (1LL << 31);
  for (int i = 0; i < 3; ++i)
    mfma = mfma && q_strides[i] % 8 == 0 && k_strides[i] % 8 == 0 && v_strides[i] % 8 == 0 &&
           o_strides[i] % 8 == 0;
  if (a.bias != nullptr) {
    // The MFMA kernel reads one (b, head) bias slice through a buffer
    // descriptor with 32-bit byte offsets, rows up to Sq + 31 and keys up to
    // Skv + 63 included.
    const int64_t besz = lc_dtype_size(bias_dtype);
    const int64_t s2 = a.bs[2], s3 = a.bs[3];
    mfma = mfma && ((int64_t)(Sq + kPfRows) * s2 + (Skv + kPfKeys) * s3 + 4) * besz < (1LL << 31);
    // 4-key vector loads: unit key stride, 4-element aligned rows and base, and
    // Skv a multiple of 4 so no group straddles the end of a row.
    a.bias_vec = s3 == 1 && Skv % 4 == 0 && s2 % 4 == 0 && a.bs[0] % 4 == 0 &&
                 a.bs[1] % 4 == 0 && lc_aligned(bias, 4 * besz);
  }
  switch (dtype) {
    case LC_DTYPE_F32:
      return launch_generic<float>(a, st);
    case LC_DTYPE_BF16:
      return mfma ? launch_mfma<bf16_t>(a, st) : launch_generic<bf16_t>(a, st);
    case LC_DTYPE_F16:
      return mfma ? launch_mfma<f16_t>(a, st) : launch_generic<f16_t>(a, st);
    default:
      return lc_fail(LC_EINVAL, "lc_prefill_attn_fwd: unknown dtype %d", dtype);
  }
}

}  // extern "C"
