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

// Decode-time fusion of RoPE with the cache append (one workgroup per
// sequence b, positions p = seq_lens[b] + s):
//   q_out[b, h, s]                      = rope(q[b, h, s], p)
//   key_pages[page(b, p), h, p % P]     = rope(k[b, h, s], p)
//   value_pages[page(b, p), h, p % P]   = v[b, h, s]
// then seq_lens[b] += S. The rotation is the RoPE kernel's (full-width
// tables, fp32, one rounding): lo = x1 c1 - x2 s1, hi = x2 c2 + x1 s2 over the
// two halves of the row; cos/sin rows are indexed by p, so a captured graph
// stays valid at any position.
struct RopeAppendArgs {
  const void* q;
  const void* k;
  const void* v;
  void* qo;
  int64_t qs[3], ks[3], vs[3], qos[3];  // (b, h, s) element strides; d stride 1
  const void* cos;
  const void* sin;
  int64_t cs, ss;  // table row strides
  int table_rows;
  int32_t* seq_lens;
  int Hq, Hkv, S, D;
};

// VEC consecutive elements of a row, held in registers.
template <typename T, int VEC>
struct Chunk {
  T v[VEC];
};
template <typename T, int VEC>
__device__ __forceinline__ Chunk<T, VEC> chunk_load(const T* p) {
  if constexpr (VEC * sizeof(T) == 16) {
    return __builtin_bit_cast(Chunk<T, VEC>, lc_load16(p));
  } else {
    Chunk<T, VEC> c;
#pragma unroll
    for (int e = 0; e < VEC; ++e) c.v[e] = p[e];
    return c;
  }
}
template <typename T, int VEC>
__device__ __forceinline__ void chunk_store(T* p, const Chunk<T, VEC>& c) {
  if constexpr (VEC * sizeof(T) == 16) {
    lc_store16(p, __builtin_bit_cast(Vec16<T>, c));
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e) p[e] = c.v[e];
  }
}

// One item per thread: a rotated chunk pair of a q or k row, or a copied chunk
// of a v row. Every thread issues the same loads with no branch between them
// (threads past the end repeat the last item, v items re-read their own chunk
// and the first cos/sin chunk), so a pass costs two round trips before its
// stores: the sources with seq_lens[b], then the cos/sin rows and the
// block-table entry at position p.
template <typename T, int VEC>
__global__ __launch_bounds__(1024) void rope_kv_append_kernel(KvPool pool, RopeAppendArgs a) {
  const int b = blockIdx.x;
  const int half = a.D / 2;
  const int hc = half / VEC;  // rotated chunk pairs per row
  const int vc = a.D / VEC;   // copied chunks per V row
  const int nq = a.S * a.Hq * hc;
  const int nk = a.S * a.Hkv * hc;
  const int nv = a.S * a.Hkv * vc;
  const int total = nq + nk + nv;
  const int capacity = pool.max_pages * pool.P;
  const T* cos = static_cast<const T*>(a.cos);
  const T* sin = static_cast<const T*>(a.sin);
  const int start = a.seq_lens[b];  // every thread reads it before the update below
  for (int i0 = 0; i0 < total; i0 += blockDim.x) {
    const int i = i0 + threadIdx.x;
    const int ic = i < total ? i : total - 1;
    const int kind = ic < nq ? 0 : (ic < nq + nk ? 1 : 2);  // q, k, v
    const int j = kind == 0 ? ic : (kind == 1 ? ic - nq : ic - nq - nk);
    const int per_row = kind == 2 ? vc : hc;
    const int heads = kind == 0 ? a.Hq : a.Hkv;
    const int c = j % per_row;
    const int hs = j / per_row;
    const int h = hs % heads;
    const int s = hs / heads;
    const int d0 = c * VEC;
    const T* src = kind == 0 ? static_cast<const T*>(a.q) + b * a.qs[0] + h * a.qs[1] + s * a.qs[2]
                 : kind == 1 ? static_cast<const T*>(a.k) + b * a.ks[0] + h * a.ks[1] + s * a.ks[2]
                             : static_cast<const T*>(a.v) + b * a.vs[0] + h * a.vs[1] + s * a.vs[2];
    const Chunk<T, VEC> xa = chunk_load<T, VEC>(src + d0);
    const Chunk<T, VEC> xb = chunk_load<T, VEC>(src + (kind == 2 ? d0 : d0 + half));
    const int pos = start + s;
    const int prow = pos < 0 ? 0 : (pos >= a.table_rows ? a.table_rows - 1 : pos);
    const int dc = kind == 2 ? 0 : d0;
    const T* cp = cos + (int64_t)prow * a.cs + dc;
    const T* sp = sin + (int64_t)prow * a.ss + dc;
    const Chunk<T, VEC> ca = chunk_load<T, VEC>(cp), cb = chunk_load<T, VEC>(cp + half);
    const Chunk<T, VEC> sa = chunk_load<T, VEC>(sp), sb = chunk_load<T, VEC>(sp + half);
    const bool in_cap = pos >= 0 && pos < capacity;
    const int page_idx = in_cap ? pos / pool.P : 0;
    const int phys = pool.bt[(int64_t)b * pool.bt_stride + page_idx];
    // A k/v item whose position has no valid page is dropped.
    const bool paged_ok = in_cap && static_cast<unsigned>(phys) < static_cast<unsigned>(pool.num_pages);
    if (!((i < total) & ((kind == 0) | paged_ok))) continue;
    const int64_t off = (int64_t)phys * pool.s_page + (int64_t)h * pool.s_head +
                        (int64_t)(pos - page_idx * pool.P) * pool.s_tok;
    if (kind == 2) {
      chunk_store<T, VEC>(static_cast<T*>(pool.vp) + off + d0, xa);
      continue;
    }
    Chunk<T, VEC> o1, o2;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float x1 = lc_to_f32(xa.v[e]), x2 = lc_to_f32(xb.v[e]);
      o1.v[e] = lc_from_f32<T>(lc_rope_lo(x1, x2, lc_to_f32(ca.v[e]), lc_to_f32(sa.v[e])));
      o2.v[e] = lc_from_f32<T>(lc_rope_hi(x1, x2, lc_to_f32(cb.v[e]), lc_to_f32(sb.v[e])));
    }
    T* dst = kind == 1 ? static_cast<T*>(pool.kp) + off
                       : static_cast<T*>(a.qo) + b * a.qos[0] + h * a.qos[1] + s * a.qos[2];
    chunk_store<T, VEC>(dst + d0, o1);
    chunk_store<T, VEC>(dst + d0 + half, o2);
  }
  __syncthreads();
  if (threadIdx.x == 0) a.seq_lens[b] = start + a.S;
}

template <typename T>
int launch_rope_append(const KvPool& pool, const RopeAppendArgs& a, int64_t B, hipStream_t st) {
  constexpr int V = 16 / sizeof(T);
  bool vec_ok = (a.D / 2) % V == 0 && lc_aligned(a.q, 16) && lc_aligned(a.k, 16) &&
                lc_aligned(a.v, 16) && lc_aligned(a.qo, 16) && lc_aligned(a.cos, 16) &&
                lc_aligned(a.sin, 16) && lc_aligned(pool.kp, 16) && lc_aligned(pool.vp, 16) &&
                a.cs % V == 0 && a.ss % V == 0 && pool.s_page % V == 0 && pool.s_head % V == 0 &&
                pool.s_tok % V == 0;
  for (int i = 0; i < 3; ++i)
    vec_ok = vec_ok && a.qs[i] % V == 0 && a.ks[i] % V == 0 && a.vs[i] % V == 0 &&
             a.qos[i] % V == 0;
  // Items per sequence: (Hq + Hkv) rotated rows of D/2/vec chunk pairs and
  // Hkv copied rows of D/vec chunks per new token; one thread each, up to 1024.
  const int64_t hc = a.D / 2 / (vec_ok ? V : 1);
  const int64_t items = (int64_t)a.S * (a.Hq + 3 * a.Hkv) * hc;
  const unsigned threads = (unsigned)(items >= 1024 ? 1024 : lc_cdiv(items, 64) * 64);
  if (threads == 0) return LC_OK;
  if (vec_ok)
    rope_kv_append_kernel<T, V><<<(unsigned)B, threads, 0, st>>>(pool, a);
  else
    rope_kv_append_kernel<T, 1><<<(unsigned)B, threads, 0, st>>>(pool, a);
  return lc_check_launch("lc_rope_kv_append");
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
  LC_REQUIRE(B >= 0 && S >= 0, "lc_paged_kv_append: bad shape");
  if (B * S == 0) return LC_OK;  // nothing to append (pointers may be null)
  LC_REQUIRE(k_new && v_new && k_strides && v_strides && key_pages && value_pages &&
                 block_table && start_pos,
             "lc_paged_kv_append: null pointer");
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
  LC_REQUIRE(B >= 0 && L >= 0, "lc_paged_kv_gather: bad shape");
  if (B * L == 0) return LC_OK;  // nothing to gather (pointers may be null)
  LC_REQUIRE(key_pages && value_pages && block_table && k_out && v_out,
             "lc_paged_kv_gather: null pointer");
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

int lc_rope_kv_append(const void* q, const int64_t* q_strides, const void* k,
                      const int64_t* k_strides, const void* v, const int64_t* v_strides,
                      void* q_out, const int64_t* q_out_strides, const void* cos,
                      const void* sin, int64_t cos_stride, int64_t sin_stride,
                      int64_t table_rows, void* key_pages, void* value_pages, int64_t kv_s_page,
                      int64_t kv_s_head, int64_t kv_s_tok, const int32_t* block_table,
                      int64_t bt_stride, int64_t max_pages_per_seq, int64_t num_pages,
                      int32_t* seq_lens, int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D,
                      int64_t page_size, int dtype, void* stream) {
  LC_REQUIRE(B >= 0 && B < (1LL << 31) && Hq > 0 && S >= 0 && D > 0 && D % 2 == 0,
             "lc_rope_kv_append: bad shape");
  if (B * S == 0) return LC_OK;  // no new tokens (pointers may be null)
  LC_REQUIRE(q && q_strides && k && k_strides && v && v_strides && q_out && q_out_strides &&
                 cos && sin && key_pages && value_pages && block_table && seq_lens,
             "lc_rope_kv_append: null pointer");
  LC_REQUIRE(S * (Hq + 2 * Hkv) * D < (1LL << 30), "lc_rope_kv_append: too many new tokens");
  LC_REQUIRE(q_strides[3] == 1 && k_strides[3] == 1 && v_strides[3] == 1 && q_out_strides[3] == 1,
             "lc_rope_kv_append: head_dim stride must be 1");
  int rc = check_pool("lc_rope_kv_append", kv_s_page, kv_s_head, kv_s_tok, max_pages_per_seq,
                      num_pages, bt_stride, page_size, Hkv, D);
  if (rc != LC_OK) return rc;
  LC_REQUIRE(table_rows >= max_pages_per_seq * page_size && table_rows < (1LL << 31),
             "lc_rope_kv_append: the cos/sin tables (%lld rows) must cover the block-table "
             "capacity (%lld positions)",
             (long long)table_rows, (long long)(max_pages_per_seq * page_size));
  if (B == 0 || S == 0) return LC_OK;
  KvPool pool{key_pages, value_pages, kv_s_page, kv_s_head, kv_s_tok, block_table, bt_stride,
              (int)max_pages_per_seq, (int)num_pages, (int)page_size};
  RopeAppendArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.qo = q_out;
  for (int i = 0; i < 3; ++i) {
    a.qs[i] = q_strides[i];
    a.ks[i] = k_strides[i];
    a.vs[i] = v_strides[i];
    a.qos[i] = q_out_strides[i];
  }
  a.cos = cos;
  a.sin = sin;
  a.cs = cos_stride;
  a.ss = sin_stride;
  a.table_rows = (int)table_rows;
  a.seq_lens = seq_lens;
  a.Hq = (int)Hq;
  a.Hkv = (int)Hkv;
  a.S = (int)S;
  a.D = (int)D;
  hipStream_t st = lc_stream(stream);
  switch (dtype) {
    case LC_DTYPE_F32:
      return launch_rope_append<float>(pool, a, B, st);
    case LC_DTYPE_BF16:
      return launch_rope_append<bf16_t>(pool, a, B, st);
    case LC_DTYPE_F16:
      return launch_rope_append<f16_t>(pool, a, B, st);
    default:
      return lc_fail(LC_EINVAL, "lc_rope_kv_append: unknown dtype %d", dtype);
  }
}

}  // extern "C"
