/*
 * lcuda.h — C ABI of liblcuda_hip.so, the gfx950 (MI355X) kernels behind the
 * Llama-3 inference attention path of llm_cuda.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers owned by the caller. The library never
 *     allocates or frees device memory and keeps no device state, except the
 *     fixed scratch array behind lc_paged_decode_fwd_noalloc.
 *   - Sizes and strides are int64 counts of ELEMENTS (not bytes). The last
 *     (head_dim / hidden) dimension must have stride 1.
 *   - `dtype` is one of LC_DTYPE_*; all inputs and outputs of one call share it
 *     unless a parameter says otherwise. Arithmetic is fp32 throughout.
 *   - `stream` is a hipStream_t (the caller's current stream); 0 = null stream.
 *     Launches are asynchronous; no entry point synchronises.
 *   - Return value: LC_OK (0) on success, a negative LC_E* code when the
 *     arguments are rejected before any launch, or a positive hipError_t when
 *     the launch itself failed. lc_last_error() then holds a message
 *     (thread-local, valid until the next call on the same thread).
 *
 * Each declaration names the reference interface it replaces
 * (paths relative to calvin-fei/llm-cuda, src/llm_cuda/...).
 */
#ifndef LCUDA_H_
#define LCUDA_H_

#include <stdint.h>

#if defined(__GNUC__)
#define LC_API __attribute__((visibility("default")))
#else
#define LC_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

enum {
  LC_DTYPE_F32 = 0,
  LC_DTYPE_F16 = 1,
  LC_DTYPE_BF16 = 2,
};

enum {
  LC_OK = 0,
  LC_EINVAL = -1,       /* bad argument (shape, stride, dtype, null pointer) */
  LC_EUNSUPPORTED = -2, /* valid request this build does not implement       */
  LC_EWORKSPACE = -3,   /* workspace (or the fixed scratch) too small        */
};

/* Library identity. Replaces the extension self-check of
 * runners/build_cuda_extension.py:1-34 (which printed exported symbols). */
LC_API int lc_version(void);
LC_API const char* lc_last_error(void);

/* RMSNorm forward: y[r, :] = x[r, :] * rsqrt(mean(x[r, :]^2) + eps) * w.
 * Replaces kernels/cuda/csrc/rmsnorm_extension.cpp:9-23 (rms_norm_forward),
 * kernels/cuda/csrc/rmsnorm_kernel.cu:7-78 and kernels/triton/rmsnorm.py:13-75.
 * x, y: [rows, hidden] with row strides; w: [hidden] contiguous, of dtype
 * w_dtype (the reference requires w_dtype == dtype; fp32 weights are also
 * accepted here). Any hidden size (the Triton path stopped at 4096). */
LC_API int lc_rmsnorm_fwd(const void* x, const void* w, void* y, int64_t rows, int64_t hidden,
                   int64_t x_row_stride, int64_t y_row_stride, float eps, int dtype,
                   int w_dtype, void* stream);

/* Residual add fused with RMSNorm: s = x + residual (rounded to dtype, as a
 * torch add in that dtype), sum_out = s, y = rmsnorm(s) * w.
 * Replaces the pair `x = x + attn_out; post_attention_layernorm(x)` of
 * models/llama3/model.py:29-42 (one HBM pass instead of three).
 * x, residual, y, sum_out: [rows, hidden] with row strides; sum_out may be x
 * or residual (in place) but y must not alias any input. */
LC_API int lc_add_rmsnorm_fwd(const void* x, const void* residual, const void* w, void* y,
                       void* sum_out, int64_t rows, int64_t hidden, int64_t x_row_stride,
                       int64_t r_row_stride, int64_t y_row_stride, int64_t s_row_stride,
                       float eps, int dtype, int w_dtype, void* stream);

/* lc_add_rmsnorm_fwd with the residual addend given as n_partials fp32
 * partial sums left by lc_decode_linear_partials: residual = round(0.0f +
 * p_0 + p_1 + ... + p_{n-1}) elementwise, summed in that order and rounded to
 * dtype (the value lc_decode_linear would have written), then s = x +
 * residual, sum_out = s, y = rmsnorm(s) * w. It replaces the same reference
 * pair as lc_add_rmsnorm_fwd (models/llama3/model.py:29-42) when the
 * projection before it (o_proj, down_proj) leaves its split-K sum to it.
 * Partial p of row r: partials + p * partial_stride + r * p_row_stride (fp32
 * elements). sum_out may be x; y must not alias x or sum_out. 1 <= n_partials
 * <= 1024. */
LC_API int lc_add_rmsnorm_partials_fwd(const void* x, const float* partials, int64_t n_partials,
                                       int64_t partial_stride, const void* w, void* y,
                                       void* sum_out, int64_t rows, int64_t hidden,
                                       int64_t x_row_stride, int64_t p_row_stride,
                                       int64_t y_row_stride, int64_t s_row_stride, float eps,
                                       int dtype, int w_dtype, void* stream);

/* SwiGLU forward: out = silu(gate) * up = gate * sigmoid(gate) * up (fp32 math).
 * Replaces csrc/rmsnorm_extension.cpp:25-40 (swiglu_forward),
 * csrc/swiglu_kernel.cu:7-57 and kernels/triton/swiglu.py:15-42,91-145.
 * gate, up, out: [rows, cols] with row strides; any cols. */
LC_API int lc_swiglu_fwd(const void* gate, const void* up, void* out, int64_t rows, int64_t cols,
                  int64_t gate_row_stride, int64_t up_row_stride, int64_t out_row_stride,
                  int dtype, void* stream);

/* RoPE forward on one or two tensors in one launch (Q and K of a layer).
 * out[.., d]      = x[.., d]      * cos[s, d]      - x[.., d+D/2] * sin[s, d]
 * out[.., d+D/2]  = x[.., d+D/2]  * cos[s, d+D/2]  + x[.., d]     * sin[s, d+D/2]
 * for d < D/2, i.e. x*cos + rotate_half(x)*sin with the FULL-width tables.
 * Replaces kernels/triton/rope.py:37-125,156-222 and the fallback of
 * models/llama3/rotary.py:81-109.
 * x{1,2}: [B, H{1,2}, S, D] with strides x*_strides[4] (any layout, e.g. the
 * transposed projection views); out{1,2}: [B, H, S, D] with out*_strides[4]
 * (may alias x in place). cos, sin: [S, D] with row strides cs_stride_s /
 * sin_stride_s. Pass x2 = out2 = NULL, h2 = 0 for a single tensor. D even. */
LC_API int lc_rope_fwd(const void* x1, void* out1, int64_t h1, const int64_t* x1_strides,
                const int64_t* out1_strides, const void* x2, void* out2, int64_t h2,
                const int64_t* x2_strides, const int64_t* out2_strides, const void* cos,
                const void* sin, int64_t cos_stride_s, int64_t sin_stride_s, int64_t B,
                int64_t S, int64_t D, int dtype, void* stream);

/* Causal attention forward with native GQA, an optional additive mask and
 * logsumexp.
 * o[b,h,i,:] = sum_j softmax_j(q[b,h,i,:].k[b,h/G,j,:] * scale + bias[b,h,i,j])
 *              v[b,h/G,j,:]
 * over keys j <= i + q_offset (j < Skv); lse[b,h,i] = natural-log logsumexp of
 * the scaled, masked scores (fp32, contiguous [B, Hq, Sq]; may be NULL).
 * Replaces kernels/triton/attention.py:74-178,323-378,501-535 (forward, with
 * the attention_mask of _torch_sdpa_fallback :457-477),
 * csrc/attention_kernel.cu:12-153 and, for q_offset > 0,
 * models/llama3/attention.py:63-89 (_torch_attention with past_len and
 * attention_mask).
 * q, o: [B, Hq, Sq, D]; k, v: [B, Hkv, Skv, D]; strides in *_strides[4].
 * bias (may be NULL): the additive mask [B, Hq, Sq, Skv] read with element
 * strides bias_strides[4] (0 broadcasts a dimension), of dtype bias_dtype
 * (fp32 or the dtype of q). Entries below -1e30 (and NaN) act as -1e30, so a
 * row whose visible keys are all so masked averages them, as the reference's
 * softmax of equal scores does; -inf excludes a key, and a row without any
 * visible key gives o = 0, lse = -inf (the reference gives NaN there).
 * Hq % Hkv == 0. bf16/f16 run on MFMA (D in {64, 128}); other cases run a
 * generic fp32-FMA kernel (D <= 256).
 * counters: lc_prefill_attn_counter_count() int32 values that are zero at
 *   entry and are left zero, or NULL. With counters, the MFMA kernel hands the
 *   lightest quarter of its row groups out to the workgroups in the order they
 *   start (the XCDs run at different clocks); with NULL every workgroup's row
 *   group follows from its block id. The outputs are the same either way.
 *   Calls that may overlap (other streams) need their own counters. */
LC_API int64_t lc_prefill_attn_counter_count(void);
LC_API int lc_prefill_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                        int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Skv, int64_t D,
                        const int64_t* q_strides, const int64_t* k_strides,
                        const int64_t* v_strides, const int64_t* o_strides, int64_t q_offset,
                        const void* bias, const int64_t* bias_strides, int bias_dtype,
                        int32_t* counters, float scale, int dtype, void* stream);

/* Bytes of workspace lc_prefill_attn_bwd needs: two fp32 values per query row
 * (delta = rowsum(dO*O), and lse * log2(e)). */
LC_API int64_t lc_prefill_attn_bwd_workspace_bytes(int64_t B, int64_t Hq, int64_t Sq);

/* Causal attention backward with native GQA: given the forward's o and lse
 * (lc_prefill_attn_fwd) and the output gradient dout, writes
 *   dq[b,h,i]   = scale * sum_j dS_ij k[b,h/G,j]
 *   dk[b,g,j]   = scale * sum_{h in group g, i} dS_ij q[b,h,i]
 *   dv[b,g,j]   =         sum_{h in group g, i} P_ij dout[b,h,i]
 * with P_ij = exp(q_i.k_j * scale + bias_ij - lse_i) on keys j <= i + q_offset
 * and dS_ij = P_ij (dout_i.v_j - rowsum(dout_i * o_i)). dq, dk, dv are
 * written, not accumulated (no atomics; no zero-fill needed). bias,
 * bias_strides, bias_dtype: the forward's additive mask (may be NULL); it
 * gets no gradient.
 * Replaces kernels/triton/attention.py:181-320 (_fused_causal_attn_bwd) and
 * :380-454 (_FusedCausalAttentionFunction.backward), which was MHA-only.
 * q, o, dout, dq: [B, Hq, Sq, D]; k, v, dk, dv: [B, Hkv, Skv, D]; lse fp32
 * contiguous [B, Hq, Sq]; strides in *_strides[4] (head_dim stride 1).
 * workspace: >= lc_prefill_attn_bwd_workspace_bytes, 16-byte aligned.
 * bf16/f16 with D % 8 == 0, D <= 128 run on MFMA; other cases on a generic
 * fp32-FMA kernel (D <= 256). */
LC_API int lc_prefill_attn_bwd(const void* q, const void* k, const void* v, const void* o,
                        const float* lse, const void* dout, void* dq, void* dk, void* dv,
                        int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Skv, int64_t D,
                        const int64_t* q_strides, const int64_t* k_strides,
                        const int64_t* v_strides, const int64_t* o_strides,
                        const int64_t* do_strides, const int64_t* dq_strides,
                        const int64_t* dk_strides, const int64_t* dv_strides, int64_t q_offset,
                        const void* bias, const int64_t* bias_strides, int bias_dtype,
                        float scale, void* workspace, int64_t workspace_bytes, int dtype,
                        void* stream);

/* Bytes of workspace lc_lm_head_argmax needs (per-block partial maxima). */
LC_API int64_t lc_lm_head_argmax_workspace_bytes(int64_t B, int64_t V);

/* int32 elements of the counters buffer lc_lm_head_argmax takes (packed
 * per-row best keys and a ticket; 272 bytes). */
LC_API int64_t lc_lm_head_argmax_counter_count(void);

/* Greedy next token fused with the lm_head projection:
 *   ids[b] = argmax_v round(hidden[b, :] . weight[v, :])
 * round() = the fp32 dot product rounded to `dtype` (the dtype of the logits
 * the reference compares); NaN ranks highest; ties go to the smallest index
 * (torch.argmax). max_logit (fp32 [B], may be NULL) receives the winning
 * rounded logit. The [B, V] logits are never written.
 * Replaces models/llama3/model.py:156 (self.lm_head(hidden_states)) followed
 * by model.py:214 (torch.argmax(logits[:, -1, :], dim=-1)) at the last position.
 * hidden: [B, K] with row stride hidden_row_stride; weight: [V, K] (nn.Linear
 * layout) with row stride weight_row_stride; ids: int64 [B].
 * bf16/f16 with K % 128 == 0 run on MFMA; other cases on a generic kernel.
 * counters (may be NULL): an 8-byte aligned int32 buffer of
 * lc_lm_head_argmax_counter_count() elements that is zero at entry and is
 * left zero; with it the MFMA path selects the ids in its own launch
 * (64-bit atomic max on packed (value, index) keys, the last workgroup
 * writing the ids), without it a second launch reduces per-workgroup
 * partials held in the workspace. Calls sharing one counters buffer must not
 * overlap. */
LC_API int lc_lm_head_argmax(const void* hidden, int64_t hidden_row_stride, const void* weight,
                      int64_t weight_row_stride, int64_t B, int64_t K, int64_t V, int64_t* ids,
                      float* max_logit, void* workspace, int64_t workspace_bytes,
                      int32_t* counters, int dtype, void* stream);

/* Bytes of fp32 workspace lc_decode_linear needs for a given shape, mode and
 * split request (two partials per workgroup; 256 when every workgroup's share
 * is whole row blocks), or -1 for invalid sizes. */
LC_API int64_t lc_decode_linear_workspace_bytes(int64_t M, int64_t N, int64_t K, int mode,
                                                int splits);

/* Number of int32 ticket counters lc_decode_linear needs for N output columns
 * (one per block of 64 columns, 32 in mode 1), or -1. */
LC_API int64_t lc_decode_linear_counter_count(int64_t N, int mode);

/* Projection of up to 32 rows (a decode step's batch), the weight streamed once:
 *   mode 0: y[m, n] = round(x[m, :] . weight[n, :])                   n < N
 *   mode 1: y[m, n] = round(silu(g) * u), g = round(x[m] . weight[n]),
 *           u = round(x[m] . weight[N + n])                             n < N
 * fp32 accumulation, round() to `dtype`, silu in fp32. Mode 0 replaces the
 * nn.Linear projections of a decode step (models/llama3/attention.py:100-102
 * q/k/v and :154 o_proj; mlp.py:35-37); mode 1 replaces
 * swiglu(gate_proj(x), up_proj(x)) (mlp.py:39-43, kernels/triton/swiglu.py:15-42)
 * over the concatenated [gate; up] weight [2N, K], with the reference's
 * roundings (g and u rounded as the projections' outputs).
 * x: [M, K] row stride x_row_stride; weight: [N or 2N, K] (nn.Linear layout);
 * y: [M, N] row stride y_row_stride. bf16/f16; 1 <= M <= 32 (M == 0 is a
 * no-op); K % 128 == 0; x and weight rows 16-byte aligned, y rows 8-byte
 * aligned; weight and x each under 2 GiB.
 * The weight's (row block, K tile) units are dealt to the workgroups in equal
 * contiguous shares. splits: workgroups per row block (0 = as few workgroups
 * as give each no more units than an even spread over the CUs). A row block
 * shared by several workgroups is summed through `workspace`
 * (>= lc_decode_linear_workspace_bytes) in workgroup order by the last of
 * them to finish, so results do not depend on the schedule.
 * counters: lc_decode_linear_counter_count(N, mode) int32 values that are zero
 * on entry; the call returns them to zero. Calls that overlap in time must not
 * share workspace or counters. */
LC_API int lc_decode_linear(const void* x, int64_t x_row_stride, const void* weight,
                            int64_t weight_row_stride, void* y, int64_t y_row_stride, int64_t M,
                            int64_t N, int64_t K, int mode, int splits, void* workspace,
                            int64_t workspace_bytes, int* counters, int dtype, void* stream);

/* Shares per row block lc_decode_linear_partials uses by default for an
 * [N, K] weight (the number of partials it writes per output), or -1. */
LC_API int64_t lc_decode_linear_partial_count(int64_t N, int64_t K);

/* lc_decode_linear mode 0 with its split-K sum left to the consumer: each of
 * `shares` equal K-shares of every row block (0 = the library's choice,
 * lc_decode_linear_partial_count) writes its fp32 partial to
 * partials[(s * M + m) * N + n], with no hand-off between workgroups (no
 * workspace, no counters). round(0.0f + p_0 + ... + p_{shares-1}) equals
 * lc_decode_linear's output. For the decode step's o_proj and down_proj
 * (models/llama3/attention.py:154, mlp.py:35-37), whose sums
 * lc_add_rmsnorm_partials_fwd adds. shares must divide the tiles of a row
 * block; N % 4 == 0; partials 16-byte aligned, [shares, M, N] contiguous. */
LC_API int lc_decode_linear_partials(const void* x, int64_t x_row_stride, const void* weight,
                                     int64_t weight_row_stride, float* partials, int64_t M,
                                     int64_t N, int64_t K, int shares, int dtype, void* stream);

/* Bytes of fp32 workspace lc_paged_decode_fwd needs for these sizes
 * (partial outputs and logsumexps of every split). */
LC_API int64_t lc_paged_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t D, int64_t max_splits);

/* Number of int32 counters lc_paged_decode_fwd takes (its counters argument). */
LC_API int64_t lc_paged_decode_counter_count(void);

/* Split-K paged GQA flash-decode: one query token per sequence against the
 * K/V pages named by the block table, then a cross-split logsumexp merge.
 * out[b,h,:] = softmax(q[b,h,:].K_b^T * scale) V_b over the seq_lens[b] tokens
 * of sequence b, where token t lives in page block_table[b, t / page_size],
 * slot t % page_size. lse[b,h] (fp32, contiguous [B, Hq], may be NULL) is the
 * natural-log logsumexp of the scaled scores; empty sequences give out = 0,
 * lse = -inf.
 * bias (may be NULL): an additive mask added to the scaled score of token t
 * of sequence b for query head h, bias[b*bias_sb + h*bias_sh + t] (strides in
 * elements, 0 broadcasts) for t < bias_len; tokens at or past bias_len get
 * none. bias_dtype: LC_DTYPE_F32, _F16 or _BF16. Clamping of very negative
 * values and -inf as in lc_prefill_attn_fwd (the reference's decode step with
 * an attention_mask, models/llama3/attention.py:63-89,138-147).
 * Replaces kernels/triton/decode_attention.py:47-159,204-287 reading the
 * contiguous copy made by models/llama3/kv_cache.py:65-83 (get_kv): here the
 * pages are read in place.
 * q, out: [B, Hq, D] with (batch, head) strides q_sb/q_sh, o_sb/o_sh.
 * key_pages, value_pages: [num_pages, Hkv, page_size, D] pools with shared
 *   element strides kv_s_page, kv_s_head, kv_s_tok.
 * block_table: int32 [B, max_pages_per_seq] (row stride bt_stride);
 *   entries outside [0, num_pages) are never dereferenced (their tokens are
 *   skipped). seq_lens: int32 [B], clamped to max_pages_per_seq * page_size.
 * split_tokens: tokens per split (multiple of 64); max_splits *
 *   split_tokens must cover the block-table capacity max_pages_per_seq *
 *   page_size (so no clamped length can need more splits than the grid has).
 *   max_splits == 1 (bf16/f16, page_size a multiple of 32, a capacity within
 *   the limit of lc_paged_decode_step) runs one workgroup of 8 waves (4 above
 *   head_dim 128) per (sequence, head group) that shares the sequence's
 *   tokens evenly among its waves and merges them in LDS, with no merge
 *   launch; it suits batches of equal lengths whose units (sequences x kv
 *   heads x head groups) fill whole rounds of the CUs.
 * workspace: >= lc_paged_decode_workspace_bytes(B, Hq, D, max_splits).
 * counters: lc_paged_decode_counter_count() int32 values that are zero at
 *   entry and are left zero, or NULL. Ragged batches whose splits take more
 *   than one round of the CUs run in a longest-first order of (sequence,
 *   split) pairs; with counters, its last quarter is handed out to the
 *   workgroups in the order they start (the XCDs read at different rates),
 *   with NULL the order is static. The outputs are the same either way.
 *   Calls that may overlap (other streams) need their own counters. */
LC_API int lc_paged_decode_fwd(const void* q, int64_t q_sb, int64_t q_sh, const void* key_pages,
                        const void* value_pages, int64_t kv_s_page, int64_t kv_s_head,
                        int64_t kv_s_tok, const int32_t* block_table, int64_t bt_stride,
                        int64_t max_pages_per_seq, int64_t num_pages, const int32_t* seq_lens,
                        void* out, int64_t o_sb, int64_t o_sh, float* lse, const void* bias,
                        int64_t bias_sb, int64_t bias_sh, int64_t bias_len, int bias_dtype,
                        void* workspace, int64_t workspace_bytes, int32_t* counters, int64_t B,
                        int64_t Hq, int64_t Hkv, int64_t D, int64_t page_size,
                        int64_t split_tokens, int64_t max_splits, float scale, int dtype,
                        void* stream);

/* Size of the device scratch behind lc_paged_decode_fwd_noalloc: the largest
 * lc_paged_decode_workspace_bytes(B, Hq, D, max_splits) it accepts (32 MiB:
 * e.g. B 64 x 32 heads x 16 splits x head_dim 128 at the 8B shape, or
 * B 8 x 64 heads x 64 splits x 128 at the 70B long-context shape). */
#define LC_DECODE_NOALLOC_SCRATCH_BYTES (32LL << 20)

/* lc_paged_decode_fwd without a workspace argument: the split partials live in
 * a fixed device array of LC_DECODE_NOALLOC_SCRATCH_BYTES owned by the library
 * (one per GPU, held until the process ends). No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops and harnesses that forbid hipMalloc). It allocates
 * nothing and calls no allocating routine; the first call on a device looks
 * up that device's copy of the array once. Semantics and arguments are those
 * of lc_paged_decode_fwd with NULL counters (the static order); the stream
 * must belong to the current device.
 * Returns LC_EWORKSPACE (no launch) when the partials of (B, Hq, D,
 * max_splits) exceed the scratch. Every call on one GPU shares its scratch:
 * calls that overlap on that GPU (other streams or threads) race and must be
 * serialised by the caller. Nothing in the scratch needs to start at zero. */
LC_API int lc_paged_decode_fwd_noalloc(const void* q, int64_t q_sb, int64_t q_sh,
                                       const void* key_pages, const void* value_pages,
                                       int64_t kv_s_page, int64_t kv_s_head, int64_t kv_s_tok,
                                       const int32_t* block_table, int64_t bt_stride,
                                       int64_t max_pages_per_seq, int64_t num_pages,
                                       const int32_t* seq_lens, void* out, int64_t o_sb,
                                       int64_t o_sh, float* lse, const void* bias,
                                       int64_t bias_sb, int64_t bias_sh, int64_t bias_len,
                                       int bias_dtype, int64_t B, int64_t Hq, int64_t Hkv,
                                       int64_t D, int64_t page_size, int64_t split_tokens,
                                       int64_t max_splits, float scale, int dtype, void* stream);

/* Scatter S new tokens per sequence into the page pools through the block
 * table: pages[bt[b, (p0_b+s)/P], h, (p0_b+s)%P, :] = x[b, h, s, :] with
 * p0_b = start_pos[b] (int32 [B], device). K and V in one launch.
 * Replaces the per-token Python copy loop of models/llama3/kv_cache.py:38-63
 * (PagedKVLayerCache.append). k_new, v_new: [B, Hkv, S, D] with strides
 * k_strides[4] / v_strides[4]. Tokens whose page entry is outside
 * [0, num_pages) or whose position is >= max_pages_per_seq * P are dropped. */
LC_API int lc_paged_kv_append(const void* k_new, const void* v_new, const int64_t* k_strides,
                       const int64_t* v_strides, void* key_pages, void* value_pages,
                       int64_t kv_s_page, int64_t kv_s_head, int64_t kv_s_tok,
                       const int32_t* block_table, int64_t bt_stride, int64_t max_pages_per_seq,
                       int64_t num_pages, const int32_t* start_pos, int64_t B, int64_t Hkv,
                       int64_t S, int64_t D, int64_t page_size, int dtype, void* stream);

/* Decode-time RoPE + cache append in one launch (one workgroup per sequence).
 * With p = seq_lens[b] + s for s < S:
 *   q_out[b, h, s, :] = rope(q[b, h, s, :], p)                       h < Hq
 *   key_pages[bt[b, p/P], h, p%P, :] = rope(k[b, h, s, :], p)        h < Hkv
 *   value_pages[bt[b, p/P], h, p%P, :] = v[b, h, s, :]
 * then seq_lens[b] += S (int32 [B], device, read and advanced in place).
 * rope(x, p) = x * cos[p] + rotate_half(x) * sin[p] in fp32, rounded once,
 * with full-width tables cos/sin [table_rows, D] (row strides cos_stride /
 * sin_stride) that must cover the block-table capacity.
 * Replaces the decode-step sequence RoPE (kernels/triton/rope.py:156-222 via
 * models/llama3/rotary.py:81-109) then PagedKVLayerCache.append
 * (models/llama3/kv_cache.py:38-63) of models/llama3/attention.py:100-124.
 * q, k, v, q_out: [B, H, S, D] with strides (any, head_dim stride 1). Tokens
 * whose page entry is invalid are dropped from the cache, as in
 * lc_paged_kv_append. */
LC_API int lc_rope_kv_append(const void* q, const int64_t* q_strides, const void* k,
                      const int64_t* k_strides, const void* v, const int64_t* v_strides,
                      void* q_out, const int64_t* q_out_strides, const void* cos,
                      const void* sin, int64_t cos_stride, int64_t sin_stride,
                      int64_t table_rows, void* key_pages, void* value_pages, int64_t kv_s_page,
                      int64_t kv_s_head, int64_t kv_s_tok, const int32_t* block_table,
                      int64_t bt_stride, int64_t max_pages_per_seq, int64_t num_pages,
                      int32_t* seq_lens, int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t D,
                      int64_t page_size, int dtype, void* stream);

/* One decode step of attention in one launch: lc_rope_kv_append with S = 1
 * followed by lc_paged_decode_fwd over the advanced lengths, without the
 * rotated q ever leaving the kernel. With p = seq_lens[b] (read before the
 * update):
 *   key_pages/value_pages at slot p   <- rope(k[b, h], p), v[b, h]
 *   out[b, h, :] = softmax(rope(q[b, h], p) . K_b^T * scale [+ bias]) V_b
 *                  over tokens 0 .. min(p + 1, capacity) - 1 of sequence b
 *   seq_lens[b] = p + 1
 * with the conventions of those two entries (tokens with invalid page entries
 * are dropped, lengths clamp to the capacity max_pages_per_seq * page_size,
 * lse (may be NULL) natural-log, bias as in lc_paged_decode_fwd over token
 * indices including p). rope() is rounded to dtype before use, so results
 * equal the two-launch sequence up to fp32 summation order. Runs the
 * single-split kernel: one workgroup of 8 waves (4 above head_dim 128) per
 * (sequence, group of <= 16 query heads), the cached tokens dealt out evenly
 * to its waves. Replaces the decode branch of models/llama3/attention.py:
 * 100-150 (RoPE at past_len, kv_cache.py:38-63 append, then the decode
 * attention of kernels/triton/decode_attention.py:204-287 over the
 * kv_cache.py:65-83 copy).
 * q: [B, Hq, D], k, v: [B, Hkv, D] (strides q_sb/q_sh, k_sb/k_sh, v_sb/v_sh;
 *   head_dim contiguous); out: [B, Hq, D] with strides o_sb/o_sh.
 * counters: int32 [B] device scratch that must hold zeros; each launch leaves
 *   it at zero (the last workgroup of a sequence to finish advances its
 *   length). Launches that share counters or seq_lens must not overlap.
 * Requires dtype bf16 or f16, head_dim a multiple of 16 (<= 256), page_size a
 * multiple of 32, a capacity of at most 126 steps of 32 tokens per wave
 * (32256 tokens at head_dim <= 128, 16128 above, for page_size 64), cos/sin
 * tables covering the capacity, 16-byte-aligned q, cos, sin and pools with
 * strides in multiples of 8 elements, and 8-byte-aligned k, v with strides in
 * multiples of 4; otherwise LC_EINVAL without a launch. */
LC_API int lc_paged_decode_step(const void* q, int64_t q_sb, int64_t q_sh, const void* k,
                                int64_t k_sb, int64_t k_sh, const void* v, int64_t v_sb,
                                int64_t v_sh, const void* cos, const void* sin,
                                int64_t cos_stride, int64_t sin_stride, int64_t table_rows,
                                void* key_pages, void* value_pages, int64_t kv_s_page,
                                int64_t kv_s_head, int64_t kv_s_tok, const int32_t* block_table,
                                int64_t bt_stride, int64_t max_pages_per_seq, int64_t num_pages,
                                int32_t* seq_lens, int32_t* counters, void* out, int64_t o_sb,
                                int64_t o_sh, float* lse, const void* bias, int64_t bias_sb,
                                int64_t bias_sh, int64_t bias_len, int bias_dtype, int64_t B,
                                int64_t Hq, int64_t Hkv, int64_t D, int64_t page_size,
                                float scale, int dtype, void* stream);

/* Gather the first L tokens of every sequence into contiguous
 * k_out, v_out [B, Hkv, L, D] (bit-exact copy through the block table).
 * Replaces models/llama3/kv_cache.py:65-83 (PagedKVLayerCache.get_kv).
 * Tokens whose page entry is outside [0, num_pages) are written as zero. */
LC_API int lc_paged_kv_gather(const void* key_pages, const void* value_pages, int64_t kv_s_page,
                       int64_t kv_s_head, int64_t kv_s_tok, const int32_t* block_table,
                       int64_t bt_stride, int64_t max_pages_per_seq, int64_t num_pages,
                       void* k_out, void* v_out, int64_t B, int64_t Hkv, int64_t L, int64_t D,
                       int64_t page_size, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LCUDA_H_ */
