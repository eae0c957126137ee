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
    LGX_MODULE_LOAD_FAILED = 5, /* LogosStatus::DeserializationFailed: the code object */
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
/* Y[m][n] = Xq W^T for m Q8_0 activation rows (Xq[m][k], Xd[m][k/32]), int8
 * MFMA; canonical schedule, so row i equals lgx_q8q8_gemv of row i. */
lgx_status lgx_q8_gemm(lgx_ctx* ctx, const lgx_q8_matrix* W, const int8_t* xq,
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

#ifdef __cplusplus
}
#endif
#endif /* LGX_H */
