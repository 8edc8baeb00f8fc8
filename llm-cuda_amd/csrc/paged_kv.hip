// Page-pool data movement for the paged KV cache: append (scatter new tokens
// through the block table) and gather (contiguous copy of the live tokens).
// Both are pure copies: the bytes written equal the bytes read (bit-exact).
//
// Address of token t of sequence b, kv head h, element d:
//   pool + block_table[b, t / P] * s_page + h * s_head + (t % P) * s_tok + d
// (models/llama3/kv_cache.py:55-61 with the identity table replaced by a
// real block table).
#include "lc_common.h"

namespace {

struct KvPool {
  void* kp;
  void* vp;
  int64_t s_page, s_head, s_tok;
  const int32_t* bt;
  int64_t bt_stride;
  int max_pages, num_pages, P;
};

// -1 when the token has no valid page.
__device__ __forceinline__ int64_t pool_offset(const KvPool& p, int b, int h, int64_t t) {
  if (t < 0 || t >= (int64_t)p.max_pages * p.P) return -1;
  const int page_idx = static_cast<int>(t / p.P);
  const int slot = static_cast<int>(t - (int64_t)page_idx * p.P);
  const int phys = p.bt[(int64_t)b * p.bt_stride + page_idx];
  if (static_cast<unsigned>(phys) >= static_cast<unsigned>(p.num_pages)) return -1;
  return (int64_t)phys * p.s_page + (int64_t)h * p.s_head + (int64_t)slot * p.s_tok;
}

// One lane per VEC elements of one (b, h, s) row; K and V rows in one pass.
template <typename T, int VEC>
__global__ __launch_bounds__(256) void kv_append_kernel(KvPool pool, const T* __restrict__ kn,
                                                        const T* __restrict__ vn, int64_t ks0,
                                                        int64_t ks1, int64_t ks2, int64_t vs0,
                                                        int64_t vs1, int64_t vs2,
                                                        const int32_t* __restrict__ start_pos,
                                                        int Hkv, int S, int D, int64_t rows) {
  const int chunks = D / VEC;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = gid / chunks;
  if (row >= rows) return;
  const int d0 = static_cast<int>(gid - row * chunks) * VEC;
  const int s = static_cast<int>(row % S);
  const int64_t bh = row / S;
  const int h = static_cast<int>(bh % Hkv);
  const int b = static_cast<int>(bh / Hkv);
  const int64_t off = pool_offset(pool, b, h, (int64_t)start_pos[b] + s);
  if (off < 0) return;
  const T* ksrc = kn + b * ks0 + h * ks1 + (int64_t)s * ks2 + d0;
  const T* vsrc = vn + b * vs0 + h * vs1 + (int64_t)s * vs2 + d0;
  T* kdst = static_cast<T*>(pool.kp) + off + d0;
  T* vdst = static_cast<T*>(pool.vp) + off + d0;
  if constexpr (VEC * sizeof(T) == 16) {
    lc_store16(kdst, lc_load16(ksrc));
    lc_store16(vdst, lc_load16(vsrc));
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      kdst[e] = ksrc[e];
      vdst[e] = vsrc[e];
    }
  }
}

template <typename T, int VEC>
__global__ __launch_bounds__(256) void kv_gather_kernel(KvPool pool, T* __restrict__ ko,
                                                        T* __restrict__ vo, int Hkv, int64_t L,
                                                        int D, int64_t rows) {
  const int chunks = D / VEC;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = gid / chunks;  // row = (b * Hkv + h) * L + t
  if (row >= rows) return;
  const int d0 = static_cast<int>(gid - row * chunks) * VEC;
  const int64_t t = row % L;
  const int64_t bh = row / L;
  const int h = static_cast<int>(bh % Hkv);
  const int b = static_cast<int>(bh / Hkv);
  const int64_t off = pool_offset(pool, b, h, t);
  T* kd = ko + row * D + d0;
  T* vd = vo + row * D + d0;
  if constexpr (VEC * sizeof(T) == 16) {
    Vec16<T> kz{}, vz{};
    if (off >= 0) {
      kz = lc_load16(static_cast<const T*>(pool.kp) + off + d0);
      vz = lc_load16(static_cast<const T*>(pool.vp) + off + d0);
    }
    lc_store16(kd, kz);
    lc_store16(vd, vz);
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      kd[e] = off >= 0 ? static_cast<const T*>(pool.kp)[off + d0 + e] : T(0);
      vd[e] = off >= 0 ? static_cast<const T*>(pool.vp)[off + d0 + e] : T(0);
    }
  }
}

template <typename T>
int launch_append(const KvPool& pool, const void* kn, const void* vn, const int64_t* ks,
                  const int64_t* vs, const int32_t* start_pos, int64_t B, int64_t Hkv, int64_t S,
                  int64_t D, hipStream_t st) {
  constexpr int V = 16 / sizeof(T);
  bool vec_ok = D % V == 0 && lc_aligned(kn, 16) && lc_aligned(vn, 16) &&
                lc_aligned(pool.kp, 16) && lc_aligned(pool.vp, 16) && pool.s_page % V == 0 &&
                pool.s_head % V == 0 && pool.s_tok % V == 0;
  for (int i = 0; i < 3; ++i) vec_ok = vec_ok && ks[i] % V == 0 && vs[i] % V == 0;
  const int vec = vec_ok ? V : 1;
  const int64_t rows = B * Hkv * S;
  const int64_t blocks = lc_cdiv(rows * (D / vec), 256);
  LC_REQUIRE(blocks < (1LL << 31), "lc_paged_kv_append: problem too large");
  if (blocks == 0) return LC_OK;
  if (vec_ok)
    kv_append_kernel<T, V><<<(unsigned)blocks, 256, 0, st>>>(
        pool, static_cast<const T*>(kn), static_cast<const T*>(vn), ks[0], ks[1], ks[2], vs[0],
        vs[1], vs[2], start_pos, (int)Hkv, (int)S, (int)D, rows);
  else
    kv_append_kernel<T, 1><<<(unsigned)blocks, 256, 0, st>>>(
        pool, static_cast<const T*>(kn), static_cast<const T*>(vn), ks[0], ks[1], ks[2], vs[0],
        vs[1], vs[2], start_pos, (int)Hkv, (int)S, (int)D, rows);
  return lc_check_launch("lc_paged_kv_append");
}

template <typename T>
int launch_gather(const KvPool& pool, void* ko, void* vo, int64_t B, int64_t Hkv, int64_t L,
                  int64_t D, hipStream_t st) {
  constexpr int V = 16 / sizeof(T);
  const bool vec_ok = D % V == 0 && lc_aligned(ko, 16) && lc_aligned(vo, 16) &&
                      lc_aligned(pool.kp, 16) && lc_aligned(pool.vp, 16) &&
                      pool.s_page % V == 0 && pool.s_head % V == 0 && pool.s_tok % V == 0;
  const int vec = vec_ok ? V : 1;
  const int64_t rows = B * Hkv * L;
  const int64_t blocks = lc_cdiv(rows * (D / vec), 256);
  LC_REQUIRE(blocks < (1LL << 31), "lc_paged_kv_gather: problem too large");
  if (blocks == 0) return LC_OK;
  if (vec_ok)
    kv_gather_kernel<T, V><<<(unsigned)blocks, 256, 0, st>>>(
        pool, static_cast<T*>(ko), static_cast<T*>(vo), (int)Hkv, L, (int)D, rows);
  else
    kv_gather_kernel<T, 1><<<(unsigned)blocks, 256, 0, st>>>(
        pool, static_cast<T*>(ko), static_cast<T*>(vo), (int)Hkv, L, (int)D, rows);
  return lc_check_launch("lc_paged_kv_gather");
}

int check_pool(const char* fn, int64_t s_page, int64_t s_head, int64_t s_tok,
               int64_t max_pages_per_seq, int64_t num_pages, int64_t bt_stride,
               int64_t page_size, int64_t Hkv, int64_t D) {
  LC_REQUIRE(page_size > 0 && max_pages_per_seq > 0 && num_pages > 0 && Hkv > 0 && D > 0,
             "%s: page_size, max_pages_per_seq, num_pages, n_kv_heads, head_dim must be > 0",
             fn);
  LC_REQUIRE(bt_stride >= max_pages_per_seq, "%s: bt_stride < max_pages_per_seq", fn);
  LC_REQUIRE(num_pages < (1LL << 31) && max_pages_per_seq < (1LL << 31), "%s: too many pages",
             fn);
  LC_REQUIRE(s_page >= 0 && s_head >= 0 && s_tok >= 0, "%s: negative pool stride", fn);
  return LC_OK;
}

}  // namespace

extern "C" {

int lc_paged_kv_append(const void* k_new, const void* v_new, const int64_t* k_strides,
                       const int64_t* v_strides, void* key_pages, void* value_pages,
                       int64_t kv_s_page, int64_t kv_s_head, int64_t kv_s_tok,
                       const int32_t* block_table, int64_t bt_stride, int64_t max_pages_per_seq,
                       int64_t num_pages, const int32_t* start_pos, int64_t B, int64_t Hkv,
                       int64_t S, int64_t D, int64_t page_size, int dtype, void* stream) {
  LC_REQUIRE(k_new && v_new && k_strides && v_strides && key_pages && value_pages &&
                 block_table && start_pos,
             "lc_paged_kv_append: null pointer");
  LC_REQUIRE(B >= 0 && S >= 0, "lc_paged_kv_append: bad shape");
  LC_REQUIRE(k_strides[3] == 1 && v_strides[3] == 1, "lc_paged_kv_append: head_dim stride != 1");
  int rc = check_pool("lc_paged_kv_append", kv_s_page, kv_s_head, kv_s_tok, max_pages_per_seq,
                      num_pages, bt_stride, page_size, Hkv, D);
  if (rc != LC_OK) return rc;
  KvPool pool{key_pages, value_pages, kv_s_page, kv_s_head, kv_s_tok, block_table, bt_stride,
              (int)max_pages_per_seq, (int)num_pages, (int)page_size};
  hipStream_t st = lc_stream(stream);
  switch (dtype) {
    case LC_DTYPE_F32:
      return launch_append<float>(pool, k_new, v_new, k_strides, v_strides, start_pos, B, Hkv, S,
                                  D, st);
    case LC_DTYPE_BF16:
      return launch_append<bf16_t>(pool, k_new, v_new, k_strides, v_strides, start_pos, B, Hkv,
                                   S, D, st);
    case LC_DTYPE_F16:
      return launch_append<f16_t>(pool, k_new, v_new, k_strides, v_strides, start_pos, B, Hkv,
                                  S, D, st);
    default:
      return lc_fail(LC_EINVAL, "lc_paged_kv_append: unknown dtype %d", dtype);
  }
}

int lc_paged_kv_gather(const void* key_pages, const void* value_pages, int64_t kv_s_page,
                       int64_t kv_s_head, int64_t kv_s_tok, const int32_t* block_table,
                       int64_t bt_stride, int64_t max_pages_per_seq, int64_t num_pages,
                       void* k_out, void* v_out, int64_t B, int64_t Hkv, int64_t L, int64_t D,
                       int64_t page_size, int dtype, void* stream) {
  LC_REQUIRE(key_pages && value_pages && block_table && k_out && v_out,
             "lc_paged_kv_gather: null pointer");
  LC_REQUIRE(B >= 0 && L >= 0, "lc_paged_kv_gather: bad shape");
  int rc = check_pool("lc_paged_kv_gather", kv_s_page, kv_s_head, kv_s_tok, max_pages_per_seq,
                      num_pages, bt_stride, page_size, Hkv, D);
  if (rc != LC_OK) return rc;
  LC_REQUIRE(L <= max_pages_per_seq * page_size,
             "lc_paged_kv_gather: L=%lld exceeds the block-table capacity %lld", (long long)L,
             (long long)(max_pages_per_seq * page_size));
  KvPool pool{const_cast<void*>(key_pages), const_cast<void*>(value_pages), kv_s_page,
              kv_s_head, kv_s_tok, block_table, bt_stride, (int)max_pages_per_seq,
              (int)num_pages, (int)page_size};
  hipStream_t st = lc_stream(stream);
  switch (dtype) {
    case LC_DTYPE_F32:
      return launch_gather<float>(pool, k_out, v_out, B, Hkv, L, D, st);
    case LC_DTYPE_BF16:
      return launch_gather<bf16_t>(pool, k_out, v_out, B, Hkv, L, D, st);
    case LC_DTYPE_F16:
      return launch_gather<f16_t>(pool, k_out, v_out, B, Hkv, L, D, st);
    default:
      return lc_fail(LC_EINVAL, "lc_paged_kv_gather: unknown dtype %d", dtype);
  }
}

}  // extern "C"
