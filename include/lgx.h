/*
 * lgx.h -- C ABI of liblgx, the MI355X (gfx950) back-end for the Q8
 * LLM-decode hot path.
 *
 * Boundary.  The reference (Brahmastra-Labs/logicaffeine, LOGOS 0.10.1) has no
 * GPU back-end and therefore no kernel entry points to keep: nothing in it
 * calls a GEMV, an attention kernel or a decode step.  This ABI is the seam a
 * LOGOS-side back-end would bind, and it follows the reference's own native
 * boundary conventions:
 *   - status-code returns, never an exception or panic across the ABI
 *     (LogosStatus, crates/logicaffeine_compile/src/codegen/ffi.rs:196-209,
 *     with the same numeric values where the meaning is the same);
 *   - a thread-keyed last-error string valid until the next call on that
 *     thread (logos_last_error / logos_clear_error, codegen/ffi.rs:227-270);
 *   - an ABI version query (LOGOS_ABI_VERSION / logos_abi_version,
 *     codegen/ffi.rs:272-285);
 *   - opaque handles with explicit create/destroy (codegen/ffi.rs:62-75);
 *   - "load a built module, resolve symbols, keep the module alive for the
 *     handle's lifetime, count calls" (load_aot_native / AotNativeFn,
 *     crates/logicaffeine_compile/src/vm/aot_tier.rs:25-43, 86-111): here the
 *     module is lgx_kernels.hsaco, loaded with hipModuleLoad, kernels resolved
 *     with hipModuleGetFunction and launched with hipModuleLaunchKernel.
 *     Unlike the reference's AOT tier there is no fallback: a missing module
 *     is LGX_MODULE_LOAD_FAILED.
 *
 * Memory.  Every tensor argument is a device pointer owned by the caller; the
 * library never frees caller memory.  A ctx owns only its module and a
 * scratch workspace for range partials (grown on demand; with more than one
 * 32-block range a product is two launches, the second applying the tree).  Calls are
 * asynchronous on `stream` (a hipStream_t; NULL = the null stream); argument
 * errors are reported synchronously, kernel faults at the caller's next
 * synchronisation.  Calls that share one ctx must be ordered on one stream
 * (they share the workspace); use one ctx per concurrent stream.
 *
 * Q8_0 matrices.  W is [n][k] with k % 32 == 0: int8 quants and one binary16
 * scale per 32-block (raw IEEE half bits).  The device kernels read the quants
 * in the T16 tile order and the scales in the S16 tile order (see
 * lgx_q8_repack_t16); n % 16 == 0 and k % 64 == 0, k <= 32768.
 *
 * Canonical arithmetic.  y[m][n] of the Q8 x Q8 products is
 *   s_b = sum_{i<32} qw[n][32b+i] * qx[m][32b+i]                (int32)
 *   P_r = fmaf((float)s_b, f32(dw[n][b]) * f32(dx[m][b]), P_r)  b ascending in
 *         range r = blocks [32r, 32r+32), P_r from +0
 *   y   = pairwise tree over r (stride 1, 2, 4, ...: P_i += P_{i+s})
 * so lgx_q8q8_gemv and lgx_q8_gemm agree bit-for-bit with each other and with
 * the CPU oracle at any batch size.
 */
#ifndef LGX_H
#define LGX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LGX_ABI_VERSION 1u

/* Values 0-9 mirror LogosStatus (codegen/ffi.rs:196-209) where the meaning
 * carries over; 10+ are device-specific. */
typedef enum lgx_status {
    LGX_OK = 0,
    LGX_ERROR = 1,
    LGX_INVALID_ARGUMENT = 2,   /* LogosStatus::RefinementViolation: a contract on an argument */
    LGX_NULL_POINTER = 3,
    LGX_OUT_OF_BOUNDS = 4,
    LGX_MODULE_LOAD_FAILED = 5, /* LogosStatus::DeserializationFailed: the code object or a weight file */
    LGX_INVALID_HANDLE = 6,
    LGX_INTERNAL_PANIC = 8,     /* LogosStatus::ThreadPanic: a C++ exception caught at the ABI */
    LGX_OUT_OF_MEMORY = 9,      /* LogosStatus::MemoryExhausted */
    LGX_HIP_ERROR = 10,
    LGX_NO_DEVICE = 11,
    LGX_UNSUPPORTED = 12
} lgx_status;

typedef struct lgx_ctx lgx_ctx;

/* Device-side layouts of Q8_0 quants. */
#define LGX_Q8_ROWMAJOR 0  /* qs[n][k] */
#define LGX_Q8_T16 1       /* 16-row x 64-column tiles in MFMA B-operand order */

typedef struct lgx_q8_matrix {
    const int8_t* qs;     /* quants in `layout` order */
    const uint16_t* d;    /* binary16 scales: row-major [n][k/32], or S16 with LGX_Q8_T16 */
    int32_t n, k;
    int32_t layout;       /* the kernels require LGX_Q8_T16 */
} lgx_q8_matrix;

/* ---- runtime (conventions of codegen/ffi.rs) ---- */
uint32_t lgx_abi_version(void);
const char* lgx_version(void);
/* Last error message of this thread, or NULL.  Valid until the next lgx call
 * on the same thread. */
const char* lgx_last_error(void);
void lgx_clear_error(void);

/* Load `hsaco_path` (NULL: lgx_kernels.hsaco beside liblgx.so) on `device`. */
lgx_status lgx_ctx_create(int32_t device, const char* hsaco_path, lgx_ctx** out);
/* Fails with LGX_INVALID_ARGUMENT (and frees nothing) while an lgx_model
 * created on ctx has not been destroyed. */
lgx_status lgx_ctx_destroy(lgx_ctx* ctx);
/* Number of kernel launches made through `ctx` (AotNativeFn::call_count). */
uint64_t lgx_ctx_launch_count(const lgx_ctx* ctx);
/* Name of the loaded code object's target (e.g. "gfx950"). */
const char* lgx_ctx_arch(const lgx_ctx* ctx);
/* Per-kernel device timing.  While enabled, every launch through ctx carries
 * start/stop events on its own dispatch (hipExtModuleLaunchKernel), so the
 * times are kernel execution only.  Enabling starts a fresh window.
 * lgx_ctx_kernel_stats waits for the window's launches of `kernel_name` and
 * returns their number and summed milliseconds. */
lgx_status lgx_ctx_set_kernel_timing(lgx_ctx* ctx, int32_t enable);
lgx_status lgx_ctx_kernel_stats(lgx_ctx* ctx, const char* kernel_name, uint64_t* count,
                                double* total_ms);

/* ---- Q8_0 layout ---- */
/* Row-major quants [n][k] and scales [n][k/32] -> the device layouts.
 * Quants, T16: unit u = (row/16)*(k/64) + k/64-pair p holds 1 KiB; lane
 * l = (row%16) + 16*c owns bytes [l*16, l*16+16): k = 64p+8c+j (j < 8) then
 * k = 64p+32+8c+j.  Scales, S16: element
 * ((row/16 * nhalf + b/16) * 16 + row%16) * 16 + b%16 holds the scale of
 * block b (zero past k/32), nhalf = ceil(k/512); lgx_q8_scale_count()
 * elements.  The unpack calls invert both. */
size_t lgx_q8_scale_count(int32_t n, int32_t k);
lgx_status lgx_q8_repack_t16(lgx_ctx* ctx, const int8_t* qs_rowmajor, const uint16_t* d_rowmajor,
                             int32_t n, int32_t k, int8_t* qs_t16, uint16_t* d_s16, void* stream);
lgx_status lgx_q8_unpack_t16(lgx_ctx* ctx, const int8_t* qs_t16, const uint16_t* d_s16, int32_t n,
                             int32_t k, int8_t* qs_rowmajor, uint16_t* d_rowmajor, void* stream);

/* ---- Q8_0 activation quantisation (GGML reference rule) ----
 * x[m][k] binary32 -> qs[m][k] int8, d[m][k/32] binary16:
 * d = amax/127, q = clamp(roundf(x * (1/d)), -127, 127). */
lgx_status lgx_quantize_q8_0(lgx_ctx* ctx, const float* x, int32_t m, int32_t k, int8_t* qs,
                             uint16_t* d, void* stream);

/* ---- GEMV / GEMM ---- */
/* y[n] = W x with binary32 x[k] (dequantised product; tolerance 1e-3 rel /
 * 1e-4 abs against an exact reference). */
lgx_status lgx_q8_gemv_f32(lgx_ctx* ctx, const lgx_q8_matrix* W, const float* x, float* y,
                           void* stream);
/* y[n] = W xq with a Q8_0 activation (xq[k], xd[k/32]); canonical schedule.
 * dbg_blockdots (nullable): receives the int32 block dots s[n][k/32]. */
lgx_status lgx_q8q8_gemv(lgx_ctx* ctx, const lgx_q8_matrix* W, const int8_t* xq,
                         const uint16_t* xd, float* y, int32_t* dbg_blockdots, void* stream);
/* y[n] = W Q8_0(x) for a binary32 x[k]: the Q8_0 quantisation of x (bit-
 * identical to lgx_quantize_q8_0) is fused into the GEMV prologue, then the
 * canonical Q8 x Q8 schedule.  xq_out / xd_out (nullable) receive Q8_0(x). */
lgx_status lgx_q8q8_gemv_quantize(lgx_ctx* ctx, const lgx_q8_matrix* W, const float* x, float* y,
                                  int8_t* xq_out, uint16_t* xd_out, void* stream);
/* Grouped y[i] = W[i] Q8_0(x[i]) for `count` (1..8) independent matrices in
 * one launch (the lgx_q8q8_gemv_quantize schedule for each). */
lgx_status lgx_q8q8_gemv_quantize_group(lgx_ctx* ctx, int32_t count, const lgx_q8_matrix* W,
                                        const float* const* x, float* const* y, void* stream);
/* Y[m][n] = Xq W^T for m Q8_0 activation rows (Xq[m][k], Xd[m][k/32]), int8
 * MFMA; canonical schedule, so row i equals lgx_q8q8_gemv of row i. */
lgx_status lgx_q8_gemm(lgx_ctx* ctx, const lgx_q8_matrix* W, const int8_t* xq,
                       const uint16_t* xd, int32_t m, float* y, void* stream);
/* Grouped Y[i][m][n_i] = Q8_0(X[i]) W[i]^T for `count` (1..8) independent
 * matrices over m binary32 activation rows each (X[i] is [m][k_i]): for
 * m = 2..8 (every k_i <= 16384, where the device's LDS per workgroup holds
 * the rows' ranges) the quantisation, products and range trees of all
 * matrices in one launch; otherwise the Q8_0 of every X[i] in one launch,
 * the products of all matrices in one more, their range trees in a third
 * (none when no matrix has several).  Row r of Y[i] is bit-identical to
 * lgx_q8q8_gemv_quantize of row r of X[i]; m = 1 is the grouped GEMV
 * (lgx_q8q8_gemv_quantize_group).  The three-launch form's quantised
 * activations and range partials live in the ctx workspace.
 * Like lgx_q8_gemm, this is the batched form of the reference's per-row
 * Q8_0 matrix-vector product. */
lgx_status lgx_q8_gemm_quantize_group(lgx_ctx* ctx, int32_t count, const lgx_q8_matrix* W,
                                      const float* const* x, int32_t m, float* const* y,
                                      void* stream);

/* Allocation-free lgx_q8_gemm.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops and harnesses that forbid hipMalloc).  Same arguments, same
 * results bit for bit as lgx_q8_gemm, but the intermediate buffers (range
 * partials, the T16 activation copy of the large-m path) live in a fixed
 * device array of LGX_NOALLOC_SCRATCH_BYTES that the library holds on each
 * device until the process ends; the call allocates nothing and never uses
 * per-kernel timing events.  A product whose intermediates exceed the
 * array fails with LGX_OUT_OF_BOUNDS.  All calls on one device share the
 * array: calls that overlap on one device (two streams, two threads, two
 * ctxs) race. */
#define LGX_NOALLOC_SCRATCH_BYTES (32u << 20)
lgx_status lgx_q8_gemm_noalloc(lgx_ctx* ctx, const lgx_q8_matrix* W, const int8_t* xq,
                               const uint16_t* xd, int32_t m, float* y, void* stream);

/* ---- paged GQA decode attention ---- */
/* out[b][h][:] = softmax(q[b][h] . K_t / sqrt(d)) V_t over the first
 * seq_len[b] cached tokens of sequence b, for KV head h / (hq/hkv).
 * K/V pages are binary16 [num_pages][hkv][16][d]; token t of sequence b is
 * slot t%16 of page page_table[b][t/16] (page_table is [B][maxp] int32).
 * d is 64 or 128, hq/hkv in 1..8.  Canonical schedule: 256-token
 * chunks, per chunk the score chain over d, max, exp, halving-tree sum and
 * the PV chain over tokens; chunks merged by log-sum-exp in chunk order.
 * Device-side seq_len values are clamped to max_seq_len (<= maxp*16, host
 * argument sizing the grid) and page ids to [0, num_pages); seq_len 0 gives
 * zeros.  Replaces no reference interface: the reference has no attention. */
lgx_status lgx_gqa_decode_attn(lgx_ctx* ctx, const float* q, const uint16_t* kpages,
                               const uint16_t* vpages, const int32_t* page_table,
                               const int32_t* seq_len, int32_t B, int32_t hq, int32_t hkv,
                               int32_t d, int32_t maxp, int32_t num_pages, int32_t max_seq_len,
                               float* out, void* stream);

/* Causal attention of a prefill chunk: B sequences with P new query rows
 * each.  Row b*P + j of q ([B*P][hq][d]) is the query at position
 * seq_len[b] + j, whose K/V rows are already cached; it attends to the first
 * seq_len[b] + j + 1 tokens of sequence b (clamped to max_seq_len).  Each row
 * runs the decode schedule above, so its output equals lgx_gqa_decode_attn
 * of that row at length seq_len[b] + j + 1.  out: [B*P][hq][d].  Replaces no
 * reference interface: the reference has no attention. */
lgx_status lgx_gqa_prefill_attn(lgx_ctx* ctx, const float* q, const uint16_t* kpages,
                                const uint16_t* vpages, const int32_t* page_table,
                                const int32_t* seq_len, int32_t B, int32_t P, int32_t hq,
                                int32_t hkv, int32_t d, int32_t maxp, int32_t num_pages,
                                int32_t max_seq_len, float* out, void* stream);
/* lgx_gqa_prefill_attn's causal attention on binary16 MFMA (flash
 * attention: online softmax over 64-token tiles, q scaled by 1/sqrt(d) and
 * rounded to binary16, P in binary16, binary32 accumulation): not the
 * canonical schedule; within 2e-3 of it.  Same arguments; the fast prefill
 * mode's attention.  No counterpart in the reference. */
lgx_status lgx_gqa_prefill_attn_fast(lgx_ctx* ctx, const float* q, const uint16_t* kpages,
                                     const uint16_t* vpages, const int32_t* page_table,
                                     const int32_t* seq_len, int32_t B, int32_t P, int32_t hq,
                                     int32_t hkv, int32_t d, int32_t maxp, int32_t num_pages,
                                     int32_t max_seq_len, float* out, void* stream);

/* ---- range partials (for consumers that fuse the range tree) ---- */
/* Number of canonical 32-block ranges of K = the partial count of a product. */
int32_t lgx_q8_range_count(int32_t k);
/* part[r][n] = the canonical chain of range r of W Q8_0(x), r < range count
 * (with one range, part is y).  Same quantisation outputs as above. */
lgx_status lgx_q8q8_gemv_quantize_partials(lgx_ctx* ctx, const lgx_q8_matrix* W, const float* x,
                                           float* part, int8_t* xq_out, uint16_t* xd_out,
                                           void* stream);
/* part[r][m][n] for m activation rows (M = 1 uses the GEMV kernel). */
lgx_status lgx_q8_gemm_partials(lgx_ctx* ctx, const lgx_q8_matrix* W, const int8_t* xq,
                                const uint16_t* xd, int32_t m, float* part, void* stream);
/* y[i] = pairwise tree over part[0..nranges)[i], i < count. */
lgx_status lgx_q8_range_combine(lgx_ctx* ctx, const float* part, int32_t nranges, int64_t count,
                                float* y, void* stream);

/* ---- decode-step glue (each also fused into lgx_qwen_decode_step) ----
 * The reference has none of these; the bit-level rules are fixed here and
 * match the CPU oracle exactly. */
/* out[m][h] = binary32 of the binary16 rows emb[tokens[i]] (ids clamped to
 * [0, vocab)). */
lgx_status lgx_embed_f16(lgx_ctx* ctx, const uint16_t* emb, const int32_t* tokens, int32_t m,
                         int32_t h, int32_t vocab, float* out, void* stream);
/* y = x * (1/sqrtf(S/n + eps)) * w per row, S = halving tree of squares
 * over the next power of two >= n (zero padded); y (binary32) and/or its
 * Q8_0 (xq, xd: the lgx_quantize_q8_0 rule) are written.  n <= 8192. */
lgx_status lgx_rmsnorm_quant(lgx_ctx* ctx, const float* x, const float* w, int32_t m, int32_t n,
                             float eps, float* y, int8_t* xq, uint16_t* xd, void* stream);
/* The decode step's residual form: h[m][n] += pairwise tree over the nr
 * range partials part[nr][m][n] (the output of lgx_q8_gemm_partials), h is
 * written back, then lgx_rmsnorm_quant of the new h.  nr <= 32. */
lgx_status lgx_add_rmsnorm_quant(lgx_ctx* ctx, const float* part, int32_t nr, float* h,
                                 const float* w, int32_t m, int32_t n, float eps, float* y,
                                 int8_t* xq, uint16_t* xd, void* stream);
/* For each sequence b: r = qkv[b] (+ bias) with rows q heads | k heads |
 * v heads; rotate-half RoPE at position p = seq_len[b] on the q and k heads
 * (pairs (i, i + d/2), cos/sin from the tables [max_seq][d/2]); q -> q_out
 * [B][hq][d]; k, v -> binary16 (RNE) slot p % 16 of page
 * page_table[b][p / 16] (pages [num_pages][hkv][16][d]).  seq_len is not
 * advanced.  Positions clamp to max_seq - 1 and page ids to [0, num_pages). */
lgx_status lgx_rope_kv_append(lgx_ctx* ctx, const float* qkv, const float* bias,
                              const float* cos_t, const float* sin_t, const int32_t* seq_len,
                              const int32_t* page_table, uint16_t* kpages, uint16_t* vpages,
                              float* q_out, int32_t B, int32_t hq, int32_t hkv, int32_t d,
                              int32_t maxp, int32_t num_pages, int32_t max_seq, void* stream);
/* a[m][i] = silu(g) * u with g = gu[m][i], u = gu[m][inter + i],
 * silu(g) = g / (1 + exp(-g)); a (binary32) and/or Q8_0(a) written. */
lgx_status lgx_swiglu_quant(lgx_ctx* ctx, const float* gu, int32_t m, int32_t inter, float* y,
                            int8_t* xq, uint16_t* xd, void* stream);
/* logits[m][v] = canonical dot of x[m] with emb[v] (binary16 tied
 * embedding): a sequential fmaf chain over each 1024-column range of k, then
 * the pairwise tree over the ranges (one range, the chain itself, for
 * h <= 1024); h % 64 == 0, h <= 8192. */
lgx_status lgx_lm_head_f16(lgx_ctx* ctx, const float* x, const uint16_t* emb, int32_t m,
                           int32_t h, int32_t vocab, float* logits, void* stream);
/* Binary16 rows [rows][h] -> T64 order: 1 KiB units (g, j), lane l of a
 * unit holding columns [8j, 8j+8) of row 64g + l (zero rows pad the last
 * group); dst holds lgx_f16_t64_count(rows, h) binary16 values.  h % 8 == 0. */
int64_t lgx_f16_t64_count(int32_t rows, int32_t h);
lgx_status lgx_f16_repack_t64(lgx_ctx* ctx, const uint16_t* src, int32_t rows, int32_t h,
                              uint16_t* dst, void* stream);
/* lgx_lm_head_f16 over a T64 embedding (same logits, bit for bit): one
 * whole-1 KiB wave load per 64 rows x 8 columns, activations through the
 * scalar cache.  h % 64 == 0, h <= 8192, m <= 64. */
lgx_status lgx_lm_head_f16_t64(lgx_ctx* ctx, const float* x, const uint16_t* emb_t64, int32_t m,
                               int32_t h, int32_t vocab, float* logits, void* stream);
/* Per-row constants of a binary16 embedding [vocab][h] for
 * lgx_lm_head_argmax_f16: rowc[v] = upper bounds of (sum_k |emb[v][k]|, the
 * same sum over its subnormal entries, ||emb[v]||_2), then 0; +inf in the
 * first three for a row with a non-finite entry; rowc holds 4 * vocab
 * floats.  h <= 1024.
 * No counterpart in the reference: the precomputation of the certified
 * greedy lm_head below. */
lgx_status lgx_lm_head_rowconst(lgx_ctx* ctx, const uint16_t* emb, int32_t vocab, int32_t h,
                                float* rowc, void* stream);
/* out[i] = lgx_argmax of row i of lgx_lm_head_f16(x, emb) -- the same token,
 * bit for bit -- without the full logits: binary16 MFMA logits with a
 * rigorous error bound per (row, vocabulary row), then the exact chain only
 * for the vocabulary rows whose bound reaches the largest lower bound (all
 * rows of a slice with more than 8 of them, all rows of an x row that is not
 * finite or outside [2^-60, 2^60] in magnitude).  emb: row-major [vocab][h];
 * emb_t64 its lgx_f16_repack_t64 form; rowc from lgx_lm_head_rowconst.
 * bounds (nullable, [m][vocab][2]): the scaled approximation and its bound,
 * for verification.  m <= 32, h % 64 == 0, h <= 1024, vocab <= 655360.
 * No counterpart in the reference: the same pick as lgx_lm_head_f16 followed
 * by lgx_argmax, for greedy decode of a tied-embedding model. */
lgx_status lgx_lm_head_argmax_f16(lgx_ctx* ctx, const float* x, const uint16_t* emb,
                                  const uint16_t* emb_t64, const float* rowc, int32_t m,
                                  int32_t h, int32_t vocab, int32_t* out, float* bounds,
                                  void* stream);
/* out[i] = first index of the maximum of logits[i][:], NaN skipped (all NaN
 * gives 0); -0 and +0 compare equal. */
lgx_status lgx_argmax(lgx_ctx* ctx, const float* logits, int32_t m, int32_t vocab, int32_t* out,
                      void* stream);
/* Seeded top-k / top-p sampling: out[b] is drawn from row b of logits
 * ([m][vocab] binary32).  Canonical rule (the CPU oracle restates it):
 *   candidates  the top_k logits by value (ties: lower index first; NaN never
 *               a candidate; -0 == +0), in that order j = 0, 1, ...
 *   weights     e_j = expf((l_j - l_0) * (1/temperature)) (the library's
 *               expf), c_j = c_{j-1} + e_j in binary32, c_{-1} = 0
 *   nucleus     J = first j with c_j >= top_p * c_last
 *   draw        x = element positions[b] of SplitMix64 stream b of `seed`
 *               (the tensor generator's stream convention), u = (x >> 40) *
 *               2^-24, token = candidate of the first j <= J with
 *               c_j > u * c_J (J if none); no candidate at all gives 0.
 * 1 <= top_k <= 64, 0 < top_p <= 1, temperature finite and > 0,
 * vocab <= 262144.  The reference has no sampler; the seeded SplitMix64
 * stream follows crates/logicaffeine_runtime/src/seed.rs:15-38. */
lgx_status lgx_sample(lgx_ctx* ctx, const float* logits, int32_t m, int32_t vocab, int32_t top_k,
                      float top_p, float temperature, uint64_t seed, const int32_t* positions,
                      int32_t* out, void* stream);

/* ---- random-init Qwen2-shaped Q8_0 model (batched greedy decode) ---- */
/* Opaque model handle, created from a seed and freed explicitly, as the
 * reference's handle classes are (codegen/ffi.rs:62-75).  The reference has
 * no model runtime; these are the entry points its emitted host code would
 * bind for the decode step. */
typedef struct lgx_model lgx_model;

typedef struct {
    int32_t n_layers, hidden, intermediate, n_heads, n_kv_heads, head_dim, vocab;
    int32_t tied_embedding; /* 1: logits from the binary16 embedding (the
                               lgx_lm_head_f16 dot: 1024-column range chains
                               and their tree) */
    int32_t max_batch, max_seq;
    float rms_eps;          /* 1e-6 */
    double rope_theta;      /* 1e6 */
    double emb_sigma;       /* embedding N(0, emb_sigma) */
} lgx_qwen_config;

/* Tensor ids of lgx_model_tensor (device pointers owned by the model). */
enum {
    LGX_T_EMB = 0,        /* binary16 [vocab][hidden] */
    LGX_T_LM_Q = 1,       /* untied lm_head quants, T16 layout */
    LGX_T_LM_D = 2,       /* untied lm_head scales, S16 layout */
    LGX_T_QKV_Q = 3, LGX_T_QKV_D = 4,
    LGX_T_O_Q = 5, LGX_T_O_D = 6,
    LGX_T_GU_Q = 7, LGX_T_GU_D = 8,
    LGX_T_DOWN_Q = 9, LGX_T_DOWN_D = 10,
    LGX_T_QKV_BIAS = 11,  /* binary32 [(hq + 2 hkv) d] */
    LGX_T_K_PAGES = 12,   /* binary16 [num_pages][hkv][16][d] */
    LGX_T_V_PAGES = 13,
    LGX_T_PAGE_TABLE = 14,/* int32 [max_batch][maxp], a seeded permutation */
    LGX_T_SEQ_LEN = 15,   /* int32 [max_batch] */
    LGX_T_HIDDEN = 16,    /* binary32 [max_batch][hidden]: last final-norm output */
    LGX_T_ATTN_NORM = 17, /* binary32 [hidden] RMSNorm weight before attention */
    LGX_T_FFN_NORM = 18,  /* binary32 [hidden] RMSNorm weight before the MLP */
    LGX_T_OUT_NORM = 19,  /* binary32 [hidden] final RMSNorm weight */
    LGX_T_EMB_Q = 20,     /* Q8_0 embedding quants (a checkpoint's Q8_0 token_embd), T16 */
    LGX_T_EMB_D = 21      /* Q8_0 embedding scales, S16 */
};

/* Generates every tensor from SplitMix64 streams of `seed` (quants uniform on
 * [-127, 127], scales |N(0, 0.02)|/127, qkv bias N(0, 0.02), embedding
 * N(0, emb_sigma), norm weights 1) and allocates the paged KV cache for
 * max_batch sequences of max_seq tokens.  Synchronous.  A model holds its
 * RMSNorm weights per layer (1 here; a checkpoint's own values when loaded). */
lgx_status lgx_model_create(lgx_ctx* ctx, const lgx_qwen_config* cfg, uint64_t seed,
                            lgx_model** out);
lgx_status lgx_model_destroy(lgx_model* m);
/* ---- Q8_0 checkpoints (GGUF) ----
 * A Qwen2 model file in the GGUF container (versions 2 and 3, the llama.cpp
 * format): metadata general.architecture = "qwen2", qwen2.block_count,
 * .embedding_length, .feed_forward_length, .attention.head_count,
 * .attention.head_count_kv (optional: .attention.key_length,
 * .attention.layer_norm_rms_epsilon, .rope.freq_base); tensors
 * token_embd.weight (F16 or Q8_0), output_norm.weight (F32), output.weight
 * (Q8_0; absent = tied embedding), and per layer N blk.N.attn_norm / ffn_norm
 * (F32), attn_q / attn_k / attn_v / attn_output / ffn_gate / ffn_up /
 * ffn_down .weight (Q8_0: blocks of a binary16 scale + 32 int8) and
 * attn_q / attn_k / attn_v .bias (F32).  The query/key rows are taken in
 * the file's (Hugging Face rotate-half) order.  A Q8_0 token_embd
 * (vocab % 16 == 0) is gathered as f32(d) * q per element, and a tied model
 * with it takes its logits from the Q8 product of the Q8_0 final-norm rows
 * with that matrix, as an untied Q8_0 output.weight would (a binary16
 * token_embd keeps the binary16 lm_head).  No counterpart in the reference,
 * which has no model format.
 * lgx_gguf_config parses the file on the host (no device) and returns the
 * model shape with max_batch / max_seq filled in; lgx_model_load_gguf builds
 * the model from the file (synchronous; the file is read tensor by tensor).
 * A file that is not GGUF or is truncated gives LGX_MODULE_LOAD_FAILED, a
 * missing or misshapen tensor LGX_INVALID_ARGUMENT, another tensor type or
 * architecture LGX_UNSUPPORTED. */
lgx_status lgx_gguf_config(const char* path, int32_t max_batch, int32_t max_seq,
                           lgx_qwen_config* out);
lgx_status lgx_model_load_gguf(lgx_ctx* ctx, const char* path, int32_t max_batch,
                               int32_t max_seq, lgx_model** out);
/* The configuration a model was built with. */
lgx_status lgx_model_config(const lgx_model* m, lgx_qwen_config* out);
/* seq_len[:] = 0 (the KV cache is overwritten as sequences grow again). */
lgx_status lgx_model_reset(lgx_model* m, void* stream);
/* One greedy decode step for sequences 0..B-1: tokens[b] (device int32) is
 * the current token of sequence b, appended at position seq_len[b]; on return
 * (stream order) tokens[b] holds the argmax next token and seq_len[b] += 1.
 * Sequence lengths are tracked on the host as well (seq_len changes only
 * through these calls): a step that would take a sequence past max_seq fails
 * with LGX_OUT_OF_BOUNDS before anything is launched; the same holds for
 * lgx_qwen_generate (nsteps positions) and lgx_qwen_prefill (P positions). */
lgx_status lgx_qwen_decode_step(lgx_model* m, int32_t B, int32_t* tokens, void* stream);
/* Feeds prompt[b][0..P) (device int32 [B][P]) for sequences 0..B-1 at
 * positions seq_len[b]..+P, filling the KV cache; next[b] receives the
 * greedy token after the prompt and seq_len[b] += P.  Each position goes
 * through the decode schedule, so prefill and decode produce the same
 * cache bits.  The first P-1 positions run as batched chunks (large-M
 * products, causal multi-query attention); the call reads the current
 * lengths once (synchronising the stream) and fails with
 * LGX_OUT_OF_BOUNDS when seq_len[b] + P exceeds max_seq. */
lgx_status lgx_qwen_prefill(lgx_model* m, int32_t B, int32_t P, const int32_t* prompt,
                            int32_t* next, void* stream);
/* nsteps greedy decode steps, each identical in effect to
 * lgx_qwen_decode_step(m, B, tokens).  The first call for a (B, tokens)
 * pair records one step into a HIP graph (no memset nodes, no allocation)
 * and every step replays it, so a step costs one graph launch on the host.
 * history (NULL or device int32 [nsteps][B]) receives tokens after each
 * step.  With per-kernel timing on, the steps are launched eagerly. */
lgx_status lgx_qwen_generate(lgx_model* m, int32_t B, int32_t* tokens, int32_t nsteps,
                             int32_t* history, void* stream);
/* Device pointer and size in bytes of a model tensor (layer ignored for the
 * global ones), for reading.  The model keeps derived copies of some tensors
 * (a tied embedding's T64 copy and row constants, built once), so writes
 * through this pointer are not supported. */
lgx_status lgx_model_tensor(lgx_model* m, int32_t layer, int32_t which, const void** dev,
                            size_t* bytes);
/* Token choice of every later decode step, generate and prefill of m:
 * temperature 0 restores greedy argmax; otherwise the lgx_sample rule with
 * stream b = sequence b and draw index = the position the step consumes
 * (seq_len[b] before its += 1).  Drops the recorded HIP graphs (waits for
 * the device if any exist). */
lgx_status lgx_model_set_sampling(lgx_model* m, float temperature, int32_t top_k, float top_p,
                                  uint64_t seed);
/* Prefill modes of lgx_qwen_prefill.  LGX_PREFILL_EXACT (the default): every
 * prompt position runs the decode step's canonical schedule, so the cache,
 * tokens and logits equal the CPU oracle's bit for bit.  LGX_PREFILL_FAST:
 * the prompt positions before the last run in binary16: each layer's Q8_0
 * weights dequantised to binary16 (RNE of d * q), the norm, attention and
 * SwiGLU outputs rounded to binary16, every product a binary16 GEMM with
 * binary32 accumulation (hipBLASLt), the attention that of
 * lgx_gqa_prefill_attn_fast; the norms, RoPE, KV append and SwiGLU keep
 * their exact operations on those inputs.  The cache so left differs from
 * the exact one by rounding (the Q8_0 activation quantisation above all);
 * the last prompt position runs the exact decode step, so its token and
 * logits, and every decode step after, are exact given the cache.  Setting
 * LGX_PREFILL_FAST does the mode's one-time work before it returns
 * (synchronising the device): the prefill buffers, every layer's weights
 * in binary16 (2 bytes per weight, kept until lgx_model_destroy), the GEMM
 * library and its plans for chunks of max_batch sequences; if any of it
 * fails, the error is returned and the mode stays as it was.  Under
 * LGX_PREFILL=serial (every position through the decode step) the mode has
 * no effect.  No counterpart in the reference. */
enum { LGX_PREFILL_EXACT = 0, LGX_PREFILL_FAST = 1 };
lgx_status lgx_model_set_prefill_mode(lgx_model* m, int32_t mode);
/* out[B][vocab] = logits of the last decode/prefill step (binary32); B must
 * be that step's batch. */
lgx_status lgx_qwen_logits(lgx_model* m, int32_t B, float* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* LGX_H */
