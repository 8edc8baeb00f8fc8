// Single-pass, HBM-bound kernels of the Llama-3 block: RMSNorm, SwiGLU, RoPE.
//
// All three read each input byte once and write each output byte once with
// 16-byte (dwordx4) lane accesses when the layout allows it, and fall back to
// element-wise access (VEC = 1) for unaligned or oddly strided views.
// Arithmetic is fp32; results are rounded once to the storage type.
#include "lc_common.h"

// Activations are streamed: each input element is read once and each output
// written once, so their 16-byte accesses carry the non-temporal bit (measured
// 3-5% faster at the bandwidth shapes). RoPE's cos/sin tables, re-read by
// every head, keep the default policy.
#define EW_LD lc_load16_nt
#define EW_ST lc_store16_nt

namespace {

// ---------------------------------------------------------------------------
// RMSNorm: one workgroup per row. The row is held in registers (ITEMS vectors
// per lane) so it is read from HBM once; ITEMS == 0 selects a two-pass loop
// for rows too wide to cache (re-read hits L2).
// Follows kernels/cuda/csrc/rmsnorm_kernel.cu:26-49: y = (x * inv_rms) * w.
// ADD 1: the input row is s = x + r rounded to T (the decoder layer's
// residual add, models/llama3/model.py:29-42), written to s_out and then
// normalised. ADD 2: the same with r = round(sum of np fp32 partials), the
// partials of a projection whose sum was left to this kernel
// (lc_decode_linear_partials): partial p of the row at pp + p * pss + row *
// prs, added to 0.0f in order p = 0, 1, ... and rounded to T, as the
// projection's own epilogue would have.
// ---------------------------------------------------------------------------
template <typename T, typename W, int VEC, int ITEMS, int ADD>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const T* x, const W* __restrict__ w,
                                                      T* __restrict__ y, int hidden,
                                                      int64_t xs, int64_t ys, float eps,
                                                      const T* r, int64_t rs, T* s_out,
                                                      int64_t ss, const float* pp, int64_t prs,
                                                      int64_t pss, int np) {
  const int64_t row = blockIdx.x;
  // (x may alias s_out: every element is read by the thread that writes it)
  const T* xr = x + row * xs;
  T* yr = y + row * ys;
  const T* rr = ADD == 1 ? r + row * rs : nullptr;
  const float* pr = ADD == 2 ? pp + row * prs : nullptr;
  T* sr = ADD ? s_out + row * ss : nullptr;
  const int nvec = hidden / VEC;
  const int tid = threadIdx.x;
  const int nthreads = blockDim.x;

  // Addend vector vi (ADD 2): the partials summed in order, rounded to T.
  // The first four partials are loaded by issue_parts (so a caller can issue
  // several vectors' loads before the first sum); finish_parts adds them and
  // any further partials, four loads at a time.
  auto load_part = [&](int p, int vi, float (&t)[VEC]) __attribute__((always_inline)) {
    const float* src = pr + (int64_t)p * pss + (int64_t)vi * VEC;
    if constexpr (VEC % 4 == 0) {
#pragma unroll
      for (int q = 0; q < VEC / 4; ++q) {
        const f32x4_t v4 = *reinterpret_cast<const f32x4_t*>(src + 4 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e) t[4 * q + e] = v4[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) t[e] = src[e];
    }
  };
  auto issue_parts = [&](int vi, float (&t)[4][VEC]) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (k < np) load_part(k, vi, t[k]);
  };
  auto finish_parts = [&](int vi, float (&t)[4][VEC], T (&out)[VEC]) __attribute__((always_inline)) {
    float a[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) a[e] = 0.f;
    for (int p0 = 0; p0 < np; p0 += 4) {
      if (p0 > 0) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (p0 + k < np) load_part(p0 + k, vi, t[k]);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (p0 + k < np) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) a[e] += t[k][e];
        }
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) out[e] = lc_from_f32<T>(a[e]);
  };
  // Addend vector vi (ADD 1 or 2) in T.
  auto load_addend = [&](int vi, T (&out)[VEC]) __attribute__((always_inline)) {
    if constexpr (ADD == 2) {
      float t[4][VEC];
      issue_parts(vi, t);
      finish_parts(vi, t, out);
    } else if constexpr (VEC * sizeof(T) == 16) {
      const Vec16<T> b = EW_LD(rr + (int64_t)vi * VEC);
#pragma unroll
      for (int e = 0; e < VEC; ++e) out[e] = b.v[e];
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) out[e] = rr[(int64_t)vi * VEC + e];
    }
  };

  // Loads vector vi of the input row (x, or round(x + addend)) as fp32.
  auto load_row = [&](int vi, float (&v)[VEC]) {
    T add[VEC];
    if constexpr (ADD != 0) load_addend(vi, add);
    if constexpr (VEC * sizeof(T) == 16) {
      Vec16<T> a = EW_LD(xr + (int64_t)vi * VEC);
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[e] = lc_to_f32(a.v[e]);
      if constexpr (ADD != 0) {
        Vec16<T> sum;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          sum.v[e] = lc_from_f32<T>(v[e] + lc_to_f32(add[e]));
          v[e] = lc_to_f32(sum.v[e]);
        }
        EW_ST(sr + (int64_t)vi * VEC, sum);
      }
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const int64_t c = (int64_t)vi * VEC + e;
        v[e] = lc_to_f32(xr[c]);
        if constexpr (ADD != 0) {
          const T sum = lc_from_f32<T>(v[e] + lc_to_f32(add[e]));
          sr[c] = sum;
          v[e] = lc_to_f32(sum);
        }
      }
    }
  };

  float acc = 0.f;
  float cache[ITEMS > 0 ? ITEMS : 1][VEC];
  // The weights of the cached vectors are loaded up front, with the row, so
  // the scaling after the reduction waits on no second memory round trip.
  W wcache[ITEMS > 0 ? ITEMS : 1][VEC];
  if constexpr (ITEMS > 0) {
    // Every load of every item is issued before the first store of s_out
    // (which x may alias), with no branch between them (items past the row
    // re-read its last vector), so the items cost one memory round trip.
    T xraw[ITEMS][VEC], rraw[ITEMS][VEC];
    float praw[ADD == 2 ? ITEMS : 1][4][VEC];
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
      const int vi = min(tid + it * nthreads, nvec - 1);
#pragma unroll
      for (int e = 0; e < VEC; ++e) wcache[it][e] = w[(int64_t)vi * VEC + e];
      if constexpr (VEC * sizeof(T) == 16) {
        const Vec16<T> a = EW_LD(xr + (int64_t)vi * VEC);
#pragma unroll
        for (int e = 0; e < VEC; ++e) xraw[it][e] = a.v[e];
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) xraw[it][e] = xr[(int64_t)vi * VEC + e];
      }
      if constexpr (ADD == 1) load_addend(vi, rraw[it]);
      if constexpr (ADD == 2) issue_parts(vi, praw[it]);
    }
    if constexpr (ADD == 2) {
#pragma unroll
      for (int it = 0; it < ITEMS; ++it)
        finish_parts(min(tid + it * nthreads, nvec - 1), praw[it], rraw[it]);
    }
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
      const int vi = tid + it * nthreads;
      const bool live = vi < nvec;
      Vec16<T> sum;
      float sq = 0.f;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float v = lc_to_f32(xraw[it][e]);
        if constexpr (ADD != 0) {
          const T sv = lc_from_f32<T>(v + lc_to_f32(rraw[it][e]));
          sum.v[e % Vec16<T>::N] = sv;
          v = lc_to_f32(sv);
        }
        cache[it][e] = v;
        sq = fmaf(v, v, sq);
      }
      acc += live ? sq : 0.f;
      if constexpr (ADD != 0) {
        if (live) {
          if constexpr (VEC * sizeof(T) == 16) {
            EW_ST(sr + (int64_t)vi * VEC, sum);
          } else {
#pragma unroll
            for (int e = 0; e < VEC; ++e)
              sr[(int64_t)vi * VEC + e] = lc_from_f32<T>(cache[it][e]);
          }
        }
      }
    }
  } else {
    for (int vi = tid; vi < nvec; vi += nthreads) {
      float v[VEC];
      load_row(vi, v);
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc = fmaf(v[e], v[e], acc);
    }
  }

  __shared__ float red[4];
  acc = lc_wave_sum(acc);
  const int wave = tid >> 6;
  if ((tid & 63) == 0) red[wave] = acc;
  __syncthreads();
  float total = 0.f;
  const int nwaves = nthreads >> 6;  // <= 4 (launch bound 256)
#pragma unroll
  for (int i = 0; i < 4; ++i) total += i < nwaves ? red[i] : 0.f;
  const float inv_rms = rsqrtf(total / static_cast<float>(hidden) + eps);

  if constexpr (ITEMS > 0) {
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
      const int vi = tid + it * nthreads;
      if (vi < nvec) {
        Vec16<T> out;
        T* dst = yr + (int64_t)vi * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float wv = lc_to_f32(wcache[it][e]);
          const T rv = lc_from_f32<T>(cache[it][e] * inv_rms * wv);
          if constexpr (VEC * sizeof(T) == 16) {
            out.v[e] = rv;
          } else {
            dst[e] = rv;
          }
        }
        if constexpr (VEC * sizeof(T) == 16) EW_ST(dst, out);
      }
    }
  } else {
    // Second pass re-reads the input row (the stored sum when ADD; the same
    // thread wrote it).
    const T* src = ADD ? sr : xr;
    for (int vi = tid; vi < nvec; vi += nthreads) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const int64_t c = (int64_t)vi * VEC + e;
        yr[c] = lc_from_f32<T>(lc_to_f32(src[c]) * inv_rms * lc_to_f32(w[c]));
      }
    }
  }
}

// Addend of ADD 2: np fp32 partials, partial p of row r at pp + p * pss + r * prs.
struct RmsParts {
  const float* pp = nullptr;
  int64_t prs = 0, pss = 0;
  int np = 0;
};

template <typename T, typename W, int VEC, int ADD>
int launch_rmsnorm_vec(const T* x, const W* w, T* y, int64_t rows, int64_t hidden, int64_t xs,
                       int64_t ys, float eps, const T* r, int64_t rs, T* s_out, int64_t ss,
                       RmsParts pt, hipStream_t st) {
  const int64_t nvec = hidden / VEC;
  int threads = static_cast<int>(lc_cdiv(nvec, 64) * 64);
  if (threads > 256) threads = 256;
  if (threads < 64) threads = 64;
  const int64_t items = lc_cdiv(nvec, threads);
  dim3 grid(static_cast<unsigned>(rows));
#define LC_RMS(ITEMS)                                                                       \
  rmsnorm_kernel<T, W, VEC, ITEMS, ADD><<<grid, threads, 0, st>>>(x, w, y, (int)hidden, xs, \
                                                                  ys, eps, r, rs, s_out, ss, \
                                                                  pt.pp, pt.prs, pt.pss, pt.np)
  if (items <= 1)
    LC_RMS(1);
  else if (items <= 2)
    LC_RMS(2);
  else if (items <= 4)
    LC_RMS(4);
  else if (items <= 8)
    LC_RMS(8);
  else
    LC_RMS(0);
#undef LC_RMS
  return lc_check_launch(ADD == 2 ? "lc_add_rmsnorm_partials_fwd"
                                  : ADD ? "lc_add_rmsnorm_fwd" : "lc_rmsnorm_fwd");
}

template <typename T, typename W, int ADD>
int launch_rmsnorm(const void* x, const void* w, void* y, int64_t rows, int64_t hidden,
                   int64_t xs, int64_t ys, float eps, const void* r, int64_t rs, void* s_out,
                   int64_t ss, RmsParts pt, hipStream_t st) {
  constexpr int V = 16 / sizeof(T);
  bool vec_ok = (hidden % V == 0) && (xs % V == 0) && (ys % V == 0) && lc_aligned(x, 16) &&
                lc_aligned(y, 16);
  if (ADD) vec_ok = vec_ok && ss % V == 0 && lc_aligned(s_out, 16);
  if (ADD == 1) vec_ok = vec_ok && rs % V == 0 && lc_aligned(r, 16);
  if (ADD == 2) vec_ok = vec_ok && pt.prs % 4 == 0 && pt.pss % 4 == 0 && lc_aligned(pt.pp, 16);
  if (vec_ok)
    return launch_rmsnorm_vec<T, W, V, ADD>(
        static_cast<const T*>(x), static_cast<const W*>(w), static_cast<T*>(y), rows, hidden, xs,
        ys, eps, static_cast<const T*>(r), rs, static_cast<T*>(s_out), ss, pt, st);
  return launch_rmsnorm_vec<T, W, 1, ADD>(
      static_cast<const T*>(x), static_cast<const W*>(w), static_cast<T*>(y), rows, hidden, xs,
      ys, eps, static_cast<const T*>(r), rs, static_cast<T*>(s_out), ss, pt, st);
}

template <int ADD>
int dispatch_rmsnorm(const void* x, const void* w, void* y, int64_t rows, int64_t hidden,
                     int64_t xs, int64_t ys, float eps, const void* r, int64_t rs, void* s_out,
                     int64_t ss, RmsParts pt, int dtype, int w_dtype, hipStream_t st) {
  const bool wf = w_dtype == LC_DTYPE_F32;
  switch (dtype) {
    case LC_DTYPE_F32:
      return launch_rmsnorm<float, float, ADD>(x, w, y, rows, hidden, xs, ys, eps, r, rs, s_out,
                                               ss, pt, st);
    case LC_DTYPE_BF16:
      return wf ? launch_rmsnorm<bf16_t, float, ADD>(x, w, y, rows, hidden, xs, ys, eps, r, rs,
                                                     s_out, ss, pt, st)
                : launch_rmsnorm<bf16_t, bf16_t, ADD>(x, w, y, rows, hidden, xs, ys, eps, r, rs,
                                                      s_out, ss, pt, st);
    case LC_DTYPE_F16:
      return wf ? launch_rmsnorm<f16_t, float, ADD>(x, w, y, rows, hidden, xs, ys, eps, r, rs,
                                                    s_out, ss, pt, st)
                : launch_rmsnorm<f16_t, f16_t, ADD>(x, w, y, rows, hidden, xs, ys, eps, r, rs,
                                                    s_out, ss, pt, st);
    default:
      return lc_fail(LC_EINVAL, "%s: unknown dtype %d",
                     ADD == 2 ? "lc_add_rmsnorm_partials_fwd"
                              : ADD ? "lc_add_rmsnorm_fwd" : "lc_rmsnorm_fwd", dtype);
  }
}

// ---------------------------------------------------------------------------
// SwiGLU: out = g * sigmoid(g) * u, fp32 math
// (kernels/triton/swiglu.py:37-42: sig = 1 / (1 + exp(-g)); y = (g * sig) * u).
// 2-D grid: x over column vectors, y over rows (row loop beyond 65535).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float silu_mul(float g, float u) {
  const float e = lc_exp2(-g * kLog2e);
  const float sig = 1.0f / (1.0f + e);
  return (g * sig) * u;
}

template <typename T, int VEC>
__global__ __launch_bounds__(256) void swiglu_kernel(const T* __restrict__ g,
                                                     const T* __restrict__ u, T* __restrict__ o,
                                                     int64_t rows, int64_t cols, int64_t gs,
                                                     int64_t us, int64_t os) {
  const int64_t vi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t c0 = vi * VEC;
  if (c0 >= cols) return;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const T* gr = g + r * gs + c0;
    const T* ur = u + r * us + c0;
    T* orow = o + r * os + c0;
    if constexpr (VEC * sizeof(T) == 16) {
      Vec16<T> gv = EW_LD(gr);
      Vec16<T> uv = EW_LD(ur);
      Vec16<T> ov;
#pragma unroll
      for (int e = 0; e < VEC; ++e)
        ov.v[e] = lc_from_f32<T>(silu_mul(lc_to_f32(gv.v[e]), lc_to_f32(uv.v[e])));
      EW_ST(orow, ov);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        if (c0 + e < cols) orow[e] = lc_from_f32<T>(silu_mul(lc_to_f32(gr[e]), lc_to_f32(ur[e])));
      }
    }
  }
}

template <typename T>
int launch_swiglu(const void* g, const void* u, void* o, int64_t rows, int64_t cols, int64_t gs,
                  int64_t us, int64_t os, hipStream_t st) {
  constexpr int V = 16 / sizeof(T);
  const bool vec_ok = (cols % V == 0) && (gs % V == 0) && (us % V == 0) && (os % V == 0) &&
                      lc_aligned(g, 16) && lc_aligned(u, 16) && lc_aligned(o, 16);
  // Fully contiguous tensors are processed as one long row.
  if (gs == cols && us == cols && os == cols && rows > 1) {
    cols = rows * cols;
    rows = 1;
    gs = us = os = cols;
  }
  const int threads = 256;
  const int vec = vec_ok ? V : 1;
  const int64_t nvec = lc_cdiv(cols, vec);
  const int64_t gx = lc_cdiv(nvec, threads);
  LC_REQUIRE(gx < (1LL << 31), "lc_swiglu_fwd: too many columns (%lld)", (long long)cols);
  dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(rows < 65535 ? rows : 65535));
  if (vec_ok)
    swiglu_kernel<T, V><<<grid, threads, 0, st>>>(static_cast<const T*>(g),
                                                  static_cast<const T*>(u), static_cast<T*>(o),
                                                  rows, cols, gs, us, os);
  else
    swiglu_kernel<T, 1><<<grid, threads, 0, st>>>(static_cast<const T*>(g),
                                                  static_cast<const T*>(u), static_cast<T*>(o),
                                                  rows, cols, gs, us, os);
  return lc_check_launch("lc_swiglu_fwd");
}

// ---------------------------------------------------------------------------
// RoPE: one lane per VEC consecutive rotation pairs (d, d + D/2) of one
// (tensor, b, h, s) row; Q and K rows share one grid. Full-width cos/sin rows
// are read (cos[s, d] and cos[s, d + D/2] separately), so tables that are not
// built as cat(freqs, freqs) are honoured (models/llama3/rotary.py:81-109
// semantics, not the half-table shortcut of kernels/triton/rope.py:106-108).
// ---------------------------------------------------------------------------
// 16-byte chunks per lane of the vectorised RoPE kernel. At the bandwidth
// shape (Q [4,32,4096,128] + K [4,8,4096,128] views) one chunk per lane ran at
// 57.7 us, two at 60.8 us and four at 66.7 us: the activation stream is half
// writes, and more bytes in flight per lane do not raise it.
constexpr int kRopeItems = 1;

struct RopeTensor {
  const void* x;
  void* out;
  int64_t h;
  int64_t xs[4];
  int64_t os[4];
};

// I: index type of the row decomposition. 32-bit unsigned division is a short
// reciprocal sequence; 64-bit division is a long expansion that measurably
// slows this HBM-bound kernel, so it is used only for grids of 2^32 lanes or
// more.
// ITEMS: chunks per lane, grid-strided (item it of lane g is chunk
// g + it * lanes). Every item's loads are issued, from clamped indices and
// with no branch between them, before the first item is computed, so a lane
// keeps ITEMS x 32 bytes of activations in flight.
template <typename T, int VEC, typename I, int ITEMS>
__global__ __launch_bounds__(256) void rope_kernel(RopeTensor t1, RopeTensor t2,
                                                   const T* __restrict__ cos,
                                                   const T* __restrict__ sin, int64_t cs_s,
                                                   int64_t sn_s, int S, int half,
                                                   int64_t rows1, int64_t rows_total) {
  const I chunks = static_cast<I>(half / VEC);
  const I lanes = static_cast<I>(gridDim.x) * static_cast<I>(blockDim.x);
  const I gid0 = static_cast<I>(blockIdx.x) * static_cast<I>(blockDim.x) + threadIdx.x;
  const I total = static_cast<I>(rows_total) * chunks;

  struct Item {
    const T* xp;
    T* op;
    const T* cp;
    const T* sp;
    int d0;
  };
  // Addresses of chunk g (rows ordered (b, s, h), heads fastest: neighbouring
  // rows share one cos/sin row, served from L1 after the first, and for
  // activations laid out as [B, S, H, D] projection views they are also
  // adjacent in memory).
  auto locate = [&](I g) -> Item {
    const I row = g / chunks;
    const int d0 = static_cast<int>(g - row * chunks) * VEC;
    const bool second = row >= static_cast<I>(rows1);
    const RopeTensor& t = second ? t2 : t1;
    const I r = second ? row - static_cast<I>(rows1) : row;
    const I nh = static_cast<I>(t.h);
    const I bs = r / nh;
    const int64_t h = static_cast<int64_t>(r - bs * nh);
    const I bi = bs / static_cast<I>(S);
    const int s = static_cast<int>(bs - bi * static_cast<I>(S));
    const int64_t b = static_cast<int64_t>(bi);
    Item it;
    it.xp = static_cast<const T*>(t.x) + b * t.xs[0] + h * t.xs[1] + (int64_t)s * t.xs[2];
    it.op = static_cast<T*>(t.out) + b * t.os[0] + h * t.os[1] + (int64_t)s * t.os[2];
    it.cp = cos + (int64_t)s * cs_s;
    it.sp = sin + (int64_t)s * sn_s;
    it.d0 = d0;
    return it;
  };

  if constexpr (VEC * sizeof(T) == 16) {
    if (gid0 >= total) return;
    Item itm[ITEMS];
    Vec16<T> xa[ITEMS], xb[ITEMS], ca[ITEMS], cb[ITEMS], sa[ITEMS], sb[ITEMS];
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      const I g = min(gid0 + static_cast<I>(k) * lanes, total - 1);
      itm[k] = locate(g);
      xa[k] = EW_LD(itm[k].xp + itm[k].d0);
      xb[k] = EW_LD(itm[k].xp + itm[k].d0 + half);
      ca[k] = lc_load16(itm[k].cp + itm[k].d0);
      cb[k] = lc_load16(itm[k].cp + itm[k].d0 + half);
      sa[k] = lc_load16(itm[k].sp + itm[k].d0);
      sb[k] = lc_load16(itm[k].sp + itm[k].d0 + half);
    }
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) {
      Vec16<T> o1, o2;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float x1 = lc_to_f32(xa[k].v[e]), x2 = lc_to_f32(xb[k].v[e]);
        o1.v[e] = lc_from_f32<T>(lc_rope_lo(x1, x2, lc_to_f32(ca[k].v[e]), lc_to_f32(sa[k].v[e])));
        o2.v[e] = lc_from_f32<T>(lc_rope_hi(x1, x2, lc_to_f32(cb[k].v[e]), lc_to_f32(sb[k].v[e])));
      }
      if (gid0 + static_cast<I>(k) * lanes < total) {
        EW_ST(itm[k].op + itm[k].d0, o1);
        EW_ST(itm[k].op + itm[k].d0 + half, o2);
      }
    }
  } else {
    if (gid0 >= total) return;
    const Item it = locate(gid0);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float x1 = lc_to_f32(it.xp[it.d0 + e]);
      const float x2 = lc_to_f32(it.xp[it.d0 + e + half]);
      it.op[it.d0 + e] = lc_from_f32<T>(
          lc_rope_lo(x1, x2, lc_to_f32(it.cp[it.d0 + e]), lc_to_f32(it.sp[it.d0 + e])));
      it.op[it.d0 + e + half] = lc_from_f32<T>(lc_rope_hi(
          x1, x2, lc_to_f32(it.cp[it.d0 + e + half]), lc_to_f32(it.sp[it.d0 + e + half])));
    }
  }
}

template <typename T>
int launch_rope(const RopeTensor& t1, const RopeTensor& t2, const void* cos, const void* sin,
                int64_t cs_s, int64_t sn_s, int64_t B, int64_t S, int64_t D, hipStream_t st) {
  constexpr int V = 16 / sizeof(T);
  const int64_t half = D / 2;
  auto tensor_vec_ok = [&](const RopeTensor& t) {
    if (t.h == 0) return true;
    for (int i = 0; i < 3; ++i)
      if (t.xs[i] % V != 0 || t.os[i] % V != 0) return false;
    return lc_aligned(t.x, 16) && lc_aligned(t.out, 16);
  };
  const bool vec_ok = (half % V == 0) && (cs_s % V == 0) && (sn_s % V == 0) &&
                      lc_aligned(cos, 16) && lc_aligned(sin, 16) && tensor_vec_ok(t1) &&
                      tensor_vec_ok(t2);
  const int64_t rows1 = B * t1.h * S;
  const int64_t rows_total = rows1 + B * t2.h * S;
  const int vec = vec_ok ? V : 1;
  const int64_t chunks_total = rows_total * (half / vec);
  const int threads = 256;
  const int items = vec_ok ? kRopeItems : 1;
  const int64_t blocks = lc_cdiv(lc_cdiv(chunks_total, items), threads);
  LC_REQUIRE(blocks < (1LL << 31), "lc_rope_fwd: problem too large");
  if (blocks == 0) return LC_OK;
  // 32-bit indices while every chunk index (and a clamped item's) fits
  const bool idx32 = chunks_total + (int64_t)blocks * threads * items < (1LL << 32);
#define LC_ROPE(VEC_, I_, IT_)                                                            \
  rope_kernel<T, VEC_, I_, IT_><<<(unsigned)blocks, threads, 0, st>>>(                    \
      t1, t2, static_cast<const T*>(cos), static_cast<const T*>(sin), cs_s, sn_s, (int)S, \
      (int)half, rows1, rows_total)
  if (vec_ok) {
    if (idx32)
      LC_ROPE(V, uint32_t, kRopeItems);
    else
      LC_ROPE(V, int64_t, kRopeItems);
  } else {
    if (idx32)
      LC_ROPE(1, uint32_t, 1);
    else
      LC_ROPE(1, int64_t, 1);
  }
#undef LC_ROPE
  return lc_check_launch("lc_rope_fwd");
}

}  // namespace

extern "C" {

int lc_rmsnorm_fwd(const void* x, const void* w, void* y, int64_t rows, int64_t hidden,
                   int64_t x_row_stride, int64_t y_row_stride, float eps, int dtype, int w_dtype,
                   void* stream) {
  LC_REQUIRE(rows >= 0 && hidden > 0, "lc_rmsnorm_fwd: bad shape rows=%lld hidden=%lld",
             (long long)rows, (long long)hidden);
  LC_REQUIRE(hidden < (1LL << 31) && rows < (1LL << 31), "lc_rmsnorm_fwd: shape too large");
  LC_REQUIRE((x && w && y) || rows == 0, "lc_rmsnorm_fwd: null pointer");
  LC_REQUIRE(w_dtype == dtype || w_dtype == LC_DTYPE_F32,
             "lc_rmsnorm_fwd: weight dtype must equal x dtype or be fp32");
  if (rows == 0) return LC_OK;
  return dispatch_rmsnorm<0>(x, w, y, rows, hidden, x_row_stride, y_row_stride, eps, nullptr, 0,
                             nullptr, 0, RmsParts{}, dtype, w_dtype, lc_stream(stream));
}

int lc_add_rmsnorm_fwd(const void* x, const void* residual, const void* w, void* y,
                       void* sum_out, int64_t rows, int64_t hidden, int64_t x_row_stride,
                       int64_t r_row_stride, int64_t y_row_stride, int64_t s_row_stride,
                       float eps, int dtype, int w_dtype, void* stream) {
  LC_REQUIRE(rows >= 0 && hidden > 0, "lc_add_rmsnorm_fwd: bad shape rows=%lld hidden=%lld",
             (long long)rows, (long long)hidden);
  LC_REQUIRE(hidden < (1LL << 31) && rows < (1LL << 31), "lc_add_rmsnorm_fwd: shape too large");
  LC_REQUIRE((x && residual && w && y && sum_out) || rows == 0,
             "lc_add_rmsnorm_fwd: null pointer");
  LC_REQUIRE(w_dtype == dtype || w_dtype == LC_DTYPE_F32,
             "lc_add_rmsnorm_fwd: weight dtype must equal x dtype or be fp32");
  LC_REQUIRE(rows == 0 || (y != sum_out && y != x && y != residual),
             "lc_add_rmsnorm_fwd: y must not alias x, residual or sum_out");
  if (rows == 0) return LC_OK;
  return dispatch_rmsnorm<1>(x, w, y, rows, hidden, x_row_stride, y_row_stride, eps, residual,
                             r_row_stride, sum_out, s_row_stride, RmsParts{}, dtype, w_dtype,
                             lc_stream(stream));
}

int lc_add_rmsnorm_partials_fwd(const void* x, const float* partials, int64_t n_partials,
                                int64_t partial_stride, const void* w, void* y, void* sum_out,
                                int64_t rows, int64_t hidden, int64_t x_row_stride,
                                int64_t p_row_stride, int64_t y_row_stride, int64_t s_row_stride,
                                float eps, int dtype, int w_dtype, void* stream) {
  LC_REQUIRE(rows >= 0 && hidden > 0,
             "lc_add_rmsnorm_partials_fwd: bad shape rows=%lld hidden=%lld", (long long)rows,
             (long long)hidden);
  LC_REQUIRE(hidden < (1LL << 31) && rows < (1LL << 31),
             "lc_add_rmsnorm_partials_fwd: shape too large");
  LC_REQUIRE(n_partials >= 1 && n_partials <= 1024,
             "lc_add_rmsnorm_partials_fwd: %lld partials (1..1024)", (long long)n_partials);
  LC_REQUIRE((x && partials && w && y && sum_out) || rows == 0,
             "lc_add_rmsnorm_partials_fwd: null pointer");
  LC_REQUIRE(p_row_stride >= hidden && partial_stride >= 0,
             "lc_add_rmsnorm_partials_fwd: partial strides too small");
  LC_REQUIRE(w_dtype == dtype || w_dtype == LC_DTYPE_F32,
             "lc_add_rmsnorm_partials_fwd: weight dtype must equal x dtype or be fp32");
  LC_REQUIRE(rows == 0 || (y != sum_out && y != x),
             "lc_add_rmsnorm_partials_fwd: y must not alias x or sum_out");
  if (rows == 0) return LC_OK;
  RmsParts pt;
  pt.pp = partials;
  pt.prs = p_row_stride;
  pt.pss = partial_stride;
  pt.np = (int)n_partials;
  return dispatch_rmsnorm<2>(x, w, y, rows, hidden, x_row_stride, y_row_stride, eps, nullptr, 0,
                             sum_out, s_row_stride, pt, dtype, w_dtype, lc_stream(stream));
}

int lc_swiglu_fwd(const void* gate, const void* up, void* out, int64_t rows, int64_t cols,
                  int64_t gate_row_stride, int64_t up_row_stride, int64_t out_row_stride,
                  int dtype, void* stream) {
  LC_REQUIRE(rows >= 0 && cols >= 0, "lc_swiglu_fwd: bad shape");
  LC_REQUIRE((gate && up && out) || rows * cols == 0, "lc_swiglu_fwd: null pointer");
  if (rows == 0 || cols == 0) return LC_OK;
  hipStream_t st = lc_stream(stream);
  switch (dtype) {
    case LC_DTYPE_F32:
      return launch_swiglu<float>(gate, up, out, rows, cols, gate_row_stride, up_row_stride,
                                  out_row_stride, st);
    case LC_DTYPE_BF16:
      return launch_swiglu<bf16_t>(gate, up, out, rows, cols, gate_row_stride, up_row_stride,
                                   out_row_stride, st);
    case LC_DTYPE_F16:
      return launch_swiglu<f16_t>(gate, up, out, rows, cols, gate_row_stride, up_row_stride,
                                  out_row_stride, st);
    default:
      return lc_fail(LC_EINVAL, "lc_swiglu_fwd: unknown dtype %d", dtype);
  }
}

int lc_rope_fwd(const void* x1, void* out1, int64_t h1, const int64_t* x1_strides,
                const int64_t* out1_strides, const void* x2, void* out2, int64_t h2,
                const int64_t* x2_strides, const int64_t* out2_strides, const void* cos,
                const void* sin, int64_t cos_stride_s, int64_t sin_stride_s, int64_t B,
                int64_t S, int64_t D, int dtype, void* stream) {
  LC_REQUIRE(D > 0 && D % 2 == 0, "lc_rope_fwd: head_dim must be even and > 0 (got %lld)",
             (long long)D);
  LC_REQUIRE(B >= 0 && S >= 0 && h1 >= 0 && h2 >= 0, "lc_rope_fwd: bad shape");
  if (B * S * (h1 + h2) == 0) return LC_OK;  // nothing to rotate (pointers may be null)
  LC_REQUIRE(h1 == 0 || (x1 && out1 && x1_strides && out1_strides), "lc_rope_fwd: null pointer");
  LC_REQUIRE(cos && sin, "lc_rope_fwd: null cos/sin");
  LC_REQUIRE(h2 == 0 || (x2 && out2 && x2_strides && out2_strides),
             "lc_rope_fwd: second tensor incomplete");
  LC_REQUIRE((h1 == 0 || (x1_strides[3] == 1 && out1_strides[3] == 1)) &&
                 (h2 == 0 || (x2_strides[3] == 1 && out2_strides[3] == 1)),
             "lc_rope_fwd: head_dim stride must be 1");
  // The grid covers h1 rows of tensor 1 and h2 of tensor 2, so a tensor with
  // no heads is never addressed.
  RopeTensor t1{x1, out1, h1, {}, {}};
  RopeTensor t2{x2, out2, h2, {}, {}};
  for (int i = 0; i < 4; ++i) {
    t1.xs[i] = h1 ? x1_strides[i] : 0;
    t1.os[i] = h1 ? out1_strides[i] : 0;
    t2.xs[i] = h2 ? x2_strides[i] : 0;
    t2.os[i] = h2 ? out2_strides[i] : 0;
  }
  LC_REQUIRE(B * (h1 + h2) * S < (1LL << 40), "lc_rope_fwd: problem too large");
  hipStream_t st = lc_stream(stream);
  switch (dtype) {
    case LC_DTYPE_F32:
      return launch_rope<float>(t1, t2, cos, sin, cos_stride_s, sin_stride_s, B, S, D, st);
    case LC_DTYPE_BF16:
      return launch_rope<bf16_t>(t1, t2, cos, sin, cos_stride_s, sin_stride_s, B, S, D, st);
    case LC_DTYPE_F16:
      return launch_rope<f16_t>(t1, t2, cos, sin, cos_stride_s, sin_stride_s, B, S, D, st);
    default:
      return lc_fail(LC_EINVAL, "lc_rope_fwd: unknown dtype %d", dtype);
  }
}

}  // extern "C"
