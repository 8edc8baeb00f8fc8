// Shared device/host helpers for the gfx950 kernels of liblcuda_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lcuda.h"

// ---------------------------------------------------------------------------
// Host-side error reporting (defined in lc_api.hip).
// ---------------------------------------------------------------------------
int lc_fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Checks hipGetLastError() after a launch; returns LC_OK or the hipError_t.
int lc_check_launch(const char* what);
// Compute units of the current device (queried once; 256 if the query fails).
int lc_cu_count();

#define LC_REQUIRE(cond, ...)                  \
  do {                                         \
    if (!(cond)) return lc_fail(LC_EINVAL, __VA_ARGS__); \
  } while (0)

static inline hipStream_t lc_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

static inline bool lc_aligned(const void* p, int64_t bytes) {
  return (reinterpret_cast<uintptr_t>(p) % static_cast<uintptr_t>(bytes)) == 0;
}

static inline int lc_dtype_size(int dtype) { return dtype == LC_DTYPE_F32 ? 4 : 2; }

// ---------------------------------------------------------------------------
// Element types. Storage types are the native clang types; arithmetic is fp32.
// ---------------------------------------------------------------------------
typedef __bf16 bf16_t;
typedef _Float16 f16_t;

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float lc_to_f32(float x) { return x; }
__device__ __forceinline__ float lc_to_f32(bf16_t x) { return static_cast<float>(x); }
__device__ __forceinline__ float lc_to_f32(f16_t x) { return static_cast<float>(x); }

template <typename T>
__device__ __forceinline__ T lc_from_f32(float x);
template <>
__device__ __forceinline__ float lc_from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ bf16_t lc_from_f32<bf16_t>(float x) { return static_cast<bf16_t>(x); }
template <>
__device__ __forceinline__ f16_t lc_from_f32<f16_t>(float x) { return static_cast<f16_t>(x); }

// 16-byte vector of T: 8 x bf16/f16 or 4 x f32.
template <typename T>
struct Vec16 {
  static constexpr int N = 16 / sizeof(T);
  T v[N];
};

template <typename T>
__device__ __forceinline__ Vec16<T> lc_load16(const T* p) {
  u32x4_t raw = *reinterpret_cast<const u32x4_t*>(p);
  return __builtin_bit_cast(Vec16<T>, raw);
}
template <typename T>
__device__ __forceinline__ void lc_store16(T* p, const Vec16<T>& x) {
  *reinterpret_cast<u32x4_t*>(p) = __builtin_bit_cast(u32x4_t, x);
}

// Streaming variants with the non-temporal cache-policy bit, for data that is
// read or written exactly once.
template <typename T>
__device__ __forceinline__ Vec16<T> lc_load16_nt(const T* p) {
  u32x4_t raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return __builtin_bit_cast(Vec16<T>, raw);
}
template <typename T>
__device__ __forceinline__ void lc_store16_nt(T* p, const Vec16<T>& x) {
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, x), reinterpret_cast<u32x4_t*>(p));
}

// exp2 on the hardware transcendental unit (v_exp_f32). Input is clamped by the
// callers' max-subtraction to <= 0, where v_exp_f32 is accurate to ~1 ulp;
// -inf gives +0.
__device__ __forceinline__ float lc_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float lc_log2(float x) { return __builtin_amdgcn_logf(x); }

// RoPE of one element pair (x1 at d, x2 at d + D/2) with full-width tables,
// in fp32 with one fixed rounding order shared by every kernel that rotates:
//   lo = x1 c1 - x2 s1 (tables at d),  hi = x2 c2 + x1 s2 (tables at d + D/2).
__device__ __forceinline__ float lc_rope_lo(float x1, float x2, float c1, float s1) {
  return fmaf(x1, c1, -(x2 * s1));
}
__device__ __forceinline__ float lc_rope_hi(float x1, float x2, float c2, float s2) {
  return fmaf(x2, c2, x1 * s2);
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------------------
// Additive attention bias (an additive attention mask added to the scaled
// scores), taken into the exp2 domain. Entries below kBiasFloor (and NaN) act
// as kBiasFloor: such a key keeps zero weight next to any real score, and a
// row whose visible keys all carry such values averages them uniformly, as
// the softmax of equal scores does (the usual finfo.min padding masks);
// -inf excludes the key exactly.
// ---------------------------------------------------------------------------
constexpr float kBiasFloor = -1.0e30f;

__device__ __forceinline__ float lc_bias_log2(float b) {
  return b == -INFINITY ? -INFINITY : fmaxf(b, kBiasFloor) * 1.4426950408889634f;
}

// One bias element of run-time dtype (LC_DTYPE_*) at element offset off.
__device__ __forceinline__ float lc_load_bias(const void* p, int64_t off, int dtype) {
  if (dtype == LC_DTYPE_F32) return static_cast<const float*>(p)[off];
  const uint16_t bits = static_cast<const uint16_t*>(p)[off];
  if (dtype == LC_DTYPE_BF16) return __uint_as_float(static_cast<uint32_t>(bits) << 16);
  return static_cast<float>(__builtin_bit_cast(_Float16, bits));
}

// Wave64 reductions (ds_swizzle / DPP via __shfl_xor).
__device__ __forceinline__ float lc_wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float lc_wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Compiler-only barrier for LDS traffic that stays inside one wavefront. The
// hardware executes a wave's LDS instructions in issue order, so a read issued
// after a write sees it; only compiler reordering (e.g. of accesses through
// differently typed pointers) must be prevented. Emits no instruction and,
// unlike a memory-model fence, no wait on outstanding global loads.
__device__ __forceinline__ void lc_compiler_fence() { __asm__ __volatile__("" ::: "memory"); }

static inline int64_t lc_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
