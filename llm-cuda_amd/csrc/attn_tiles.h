// Building blocks shared by the MFMA attention kernels (prefill forward and
// backward): 32x32x16 MFMA wrappers, the swizzled LDS tile layout, the
// buffer-to-LDS DMA of a 64-row tile, and the workgroup barrier used between
// pipeline stages.
#pragma once

#include <type_traits>

#include "lc_common.h"

namespace lc_attn {

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x8_t __attribute__((ext_vector_type(8)));
#define LC_LDS __attribute__((address_space(3)))

template <typename T>
struct Mfma32;
template <>
struct Mfma32<bf16_t> {
  typedef bf16x8_t v8;
  static __device__ __forceinline__ f32x16_t mma(v8 a, v8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma32<f16_t> {
  typedef f16x8_t v8;
  static __device__ __forceinline__ f32x16_t mma(v8 a, v8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};


// s_waitcnt immediates (gfx9 encoding: vmcnt [3:0] + [15:14], expcnt [6:4],
// lgkmcnt [11:8]).
constexpr int kWaitVm0Lgkm0 = 0x0070;  // vmcnt(0) lgkmcnt(0)
constexpr int kWaitLgkm0 = 0xC07F;     // lgkmcnt(0)

// Workgroup barrier: this wave's LDS reads (and, with WAIT_VM, its DMA) have
// completed before it arrives.
template <bool WAIT_VM>
__device__ __forceinline__ void pf_barrier() {
  __builtin_amdgcn_s_waitcnt(WAIT_VM ? kWaitVm0Lgkm0 : kWaitLgkm0);
  lc_compiler_fence();
  __builtin_amdgcn_s_barrier();
  lc_compiler_fence();
}

// LDS swizzle of the prefill K/V tiles: 16-byte chunk c of row r is stored at
// position c ^ pf_swz(r). Two read patterns must both be bank-conflict free:
//  * QK^T operands: 16 lanes read one chunk of 16 consecutive rows, so
//    pf_swz must be a bijection on r mod (rows per bank cycle);
//  * transposed V^T reads: a 16-lane group reads 4 consecutive rows x 4
//    consecutive chunks, so 4 consecutive rows must differ in the high
//    position bits.
// A plain XOR with r mod 16 fails the second (4 rows map onto the same 4
// positions); swapping the two 2-bit halves of r mod 16 satisfies both.
// Position of the q-th workgroup of a (batch, kv head, head group) unit in
// the causal kernels' heaviest-first row-group order, q < n: the order is
// reversed inside every other run of four. Each XCD deals its workgroups to
// its four shader engines round-robin, so with the plain order the first
// engine took the heaviest row group of every four (at 128 row groups per
// unit about 5% more work than the fourth); alternating the direction gives
// the four engines equal sums. A final partial run stays a permutation of
// itself.
__device__ __forceinline__ int pf_snake(int q, int n) {
  const int s = (q & ~3) | ((q & 4) ? 3 - (q & 3) : (q & 3));
  return s < n ? s : q;
}

template <int CPR>
__device__ __forceinline__ int pf_swz(int r) {
  if constexpr (CPR == 16) {
    return ((r & 3) << 2) | ((r >> 2) & 3);  // 256-byte rows: one row per bank cycle
  } else {
    return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);  // 128-byte rows: 2 rows per cycle
  }
}

template <int NIW>
struct PfLoadOffsets {
  int o[NIW];
};

// Buffer-to-LDS DMA of one tile: instruction u of wave w fills LDS rows
// (w * NIW + u) * RPI .. + RPI - 1 of dst. AUX is the loads' cache-policy
// operand (2 = non-temporal, for data read exactly once).
template <int NIW, int RPI, int ROW_B, int AUX = 0>
__device__ __forceinline__ void pf_dma_tile(const void* base, int nbytes, LC_LDS char* dst,
                                            int wave, PfLoadOffsets<NIW> off, int add) {
  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, nbytes, 0x00020000);
#pragma unroll
  for (int u = 0; u < NIW; ++u) {
    const int row0 = (wave * NIW + u) * RPI;
    // (a plain local int: the host pass of hipcc rejects this builtin when its
    // offset operand is a member of a dependent-type parameter)
    const int vo = off.o[u];
    // per-lane offset in voffset, the wave-uniform tile offset in soffset
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (LC_LDS void*)(dst + row0 * ROW_B), 16, vo, add,
                                             0, AUX);
  }
}

// pf_dma_tile issued as inline assembly, for streaming rings that keep more
// than one tile in flight: the same rows, offsets and zero fill; NT selects
// non-temporal loads (data read once). The compiler does not see these LDS
// writes. Issued through the builtin, it tracks them and, unable to tell a
// ring's stages apart, waits for every DMA in flight (the next tiles'
// included) before each LDS read, which leaves one tile in flight. The
// kernel's own s_waitcnt vmcnt + barrier must order its LDS reads after the
// data; the "memory" clobber keeps the compiler from moving LDS accesses
// across the DMA.
template <int NIW, int RPI, int ROW_B, bool NT>
__device__ __forceinline__ void pf_dma_tile_untracked(const void* base, int nbytes,
                                                      LC_LDS char* dst, int wave,
                                                      const PfLoadOffsets<NIW>& off, int soff) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const u32x4_t rsrc = {
      static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b))),
      static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b >> 32))) & 0xFFFFu,
      static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(nbytes)), 0x00020000u};
  const int so = __builtin_amdgcn_readfirstlane(soff);
#pragma unroll
  for (int u = 0; u < NIW; ++u) {
    const int row0 = (wave * NIW + u) * RPI;
    const int m0v = __builtin_amdgcn_readfirstlane(
        static_cast<int>(reinterpret_cast<uintptr_t>(dst + row0 * ROW_B)));
    // M0 (the LDS destination) is saved and restored around the load.
    int m0_saved;
    if constexpr (NT)
      __asm__ __volatile__(
          "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
          "buffer_load_dwordx4 %1, %2, %4 offen nt lds\n\ts_mov_b32 m0, %0"
          : "=&s"(m0_saved)
          : "v"(off.o[u]), "s"(rsrc), "s"(m0v), "s"(so)
          : "memory");
    else
      __asm__ __volatile__(
          "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
          "buffer_load_dwordx4 %1, %2, %4 offen lds\n\ts_mov_b32 m0, %0"
          : "=&s"(m0_saved)
          : "v"(off.o[u]), "s"(rsrc), "s"(m0v), "s"(so)
          : "memory");
  }
}

// Additive bias of one 64-key tile for the query row of each lane, in the
// layout of the 32x32 S^T accumulators: lane (l32 = query row, hh = lane / 32)
// holds keys k0 + kt*32 + j*8 + hh*4 + e (kt < 2, j < 4, e < 4), i.e. register
// kt, 4j + e. Storage: BIAS 1 = the data type T (bf16/f16), 2 = fp32. Loads go
// through a buffer descriptor over the row's (b, head) slice, so keys and rows
// past its end read 0 (those scores are masked or discarded anyway).
template <typename T, int BIAS>
struct BiasTile {
  static constexpr int ESZ = BIAS == 2 ? 4 : 2;
  typedef u32x4_t r4_t;
  typedef u32x2_t r2_t;
  typedef typename std::conditional<BIAS == 2, r4_t, r2_t>::type raw_t;
  raw_t r[2][4];

  // row_b: byte offset of the lane's query row in the slice; s3_b: key stride
  // in bytes; vec: keys contiguous and every 4-key group 4*ESZ-aligned and
  // wholly inside or outside the slice (one 8- or 16-byte load per group).
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, int row_b, int k0, int hh,
                                       int s3_b, bool vec) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = k0 + kt * 32 + j * 8 + hh * 4;
        if (vec) {
          const int off = row_b + key * ESZ;
          if constexpr (BIAS == 2)
            r[kt][j] = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
          else
            r[kt][j] = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int off = row_b + (key + e) * s3_b;
            if constexpr (BIAS == 2) {
              r[kt][j][e] = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0);
            } else {
              const uint32_t h = __builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0);
              if (e & 1)
                r[kt][j][e >> 1] |= h << 16;
              else
                r[kt][j][e >> 1] = h;
            }
          }
        }
      }
  }
  // Element (kt, 4j + e) in the exp2 domain (lc_bias_log2).
  __device__ __forceinline__ float log2_at(int kt, int r4) const {
    const int j = r4 >> 2, e = r4 & 3;
    float x;
    if constexpr (BIAS == 2) {
      x = __uint_as_float(r[kt][j][e]);
    } else {
      const uint32_t w = r[kt][j][e >> 1];
      const uint16_t h = static_cast<uint16_t>((e & 1) ? (w >> 16) : (w & 0xffffu));
      x = static_cast<float>(__builtin_bit_cast(T, h));
    }
    return lc_bias_log2(x);
  }
};

// Maximum of x over the two 32-lane halves of the wave (v_permlane32_swap).
__device__ __forceinline__ float pf_half_max(float x) {
  const unsigned u = __float_as_uint(x);
  const auto sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}

}  // namespace lc_attn
