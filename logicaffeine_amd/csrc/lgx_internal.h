// lgx_internal.h -- definitions shared by the liblgx translation units:
// error state, the kernel table resolved from lgx_kernels.hsaco, the context
// object, and the launch helpers.  Not part of the ABI.
#pragma once
#include <hip/hip_runtime_api.h>

#include <dlfcn.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/lgx.h"
#include "lgx_kargs.h"

// From hip/hip_ext.h (whose templates need the HIP compiler; this file is
// plain C++): module launch with start/stop events on the dispatch itself.
extern "C" hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t globalWorkSizeX,
                                               uint32_t globalWorkSizeY, uint32_t globalWorkSizeZ,
                                               uint32_t localWorkSizeX, uint32_t localWorkSizeY,
                                               uint32_t localWorkSizeZ, size_t sharedMemBytes,
                                               hipStream_t hStream, void** kernelParams,
                                               void** extra, hipEvent_t startEvent,
                                               hipEvent_t stopEvent, uint32_t flags);

namespace lgxi {

inline thread_local std::string g_last_error;
inline thread_local bool g_has_error = false;
// Set while an allocation-free entry point runs on this thread: its launches
// never take timing events (creating them may allocate).
inline thread_local bool g_untimed = false;

// LGX_TRACE (set, non-empty and not "0"): one line on stderr for every kernel
// launch, binary16 GEMM call and graph replay, written when the host issues
// it (the launches of a recorded graph once, at capture, marked "captured").
// The environment is read once per process.  After LOGOS_TIER_TRACE
// (crates/logicaffeine_compile/src/vm/tier_trace.rs:1-29).
inline bool trace_on() {
    static const bool on = [] {
        const char* v = std::getenv("LGX_TRACE");
        return v != nullptr && v[0] != '\0' && std::strcmp(v, "0") != 0;
    }();
    return on;
}

// One trace line: "[lgx] " + the formatted text + newline, in one write.
inline void trace_line(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    const int n = vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (n < 0) return;
    std::fprintf(stderr, "[lgx] %s\n", buf);
}

inline lgx_status fail(lgx_status st, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    g_has_error = true;
    return st;
}

template <class F>
lgx_status guarded(const char* name, F&& f) {
    try {
        return f();
    } catch (const std::bad_alloc&) {
        return fail(LGX_OUT_OF_MEMORY, "%s: host allocation failed", name);
    } catch (const std::exception& e) {
        return fail(LGX_INTERNAL_PANIC, "%s: internal error: %s", name, e.what());
    } catch (...) {
        return fail(LGX_INTERNAL_PANIC, "%s: unknown internal error", name);
    }
}

#define LGX_HIP(call)                                                                   \
    do {                                                                                \
        hipError_t e_ = (call);                                                         \
        if (e_ != hipSuccess)                                                           \
            return fail(LGX_HIP_ERROR, "%s: %s failed: %s", __func__, #call,            \
                        hipGetErrorString(e_));                                         \
    } while (0)

// Kernel table: name in the code object -> slot.
enum Kern {
    K_REPACK,
    K_QUANT,
    K_Q8Q8_GEMV,
    K_Q8_GEMV_F32,
    K_COMBINE,
    K_GEMV_MFMA,
    K_GEMV_MFMA_QX,
    K_GEMM_MFMA16,
    K_GEMM_MFMA32,
    K_GEMM_MFMA64,
    K_REPACK_S16,
    K_ATTN_D64_G1,   // + (gq - 1): gq = 1..8
    K_ATTN_D128_G1 = K_ATTN_D64_G1 + 8,
    K_ATTN_COMBINE_D64 = K_ATTN_D128_G1 + 8,
    K_ATTN_COMBINE_D128,
    K_EMBED,
    K_ADD_RMSNORM_QUANT,
    K_QKV_ROPE_APPEND,
    K_ATTN_COMBINE_QUANT_D64,
    K_ATTN_COMBINE_QUANT_D128,
    K_SWIGLU_QUANT,
    K_LM_HEAD_F16,
    K_ARGMAX_PARTIAL,
    K_ARGMAX_FINAL,
    K_ADVANCE,
    K_GEMV_WG4,
    K_GEMV_WG8,
    K_GEMV_WG16,
    K_GEMV_GRP4,
    K_GEMV_GRP8,
    K_GEMV_GRP16,
    K_REPACK_F16_T64,
    K_LM_HEAD_T64,
    K_ROWS_TO_T16,
    K_GEMV_GRPQ4,
    K_GEMV_GRPQ8,
    K_GEMV_GRPQ16,
    K_NORM4_R8,
    K_NORM4_R20,
    K_ACT_T16,
    K_GEMM_TILED,
    K_GEMM_TILED64,
    K_GEMM_TILED32,
    K_PFA_D64_G1,    // + (gq - 1)
    K_PFA_D128_G1 = K_PFA_D64_G1 + 8,
    K_SAMPLE_PARTIAL = K_PFA_D128_G1 + 8,
    K_SAMPLE_FINAL,
    K_GEMM_MFMA16_QKV,
    K_GEMM_MFMA16_SWIGLU,
    K_NORM_W,
    K_GEMM_MFMA16_GROUP,
    K_GEMM_TILED_GROUP,
    K_GEMM_TILED64_GROUP,
    K_GEMM_TILED32_GROUP,
    K_QUANT_GROUP,
    K_COMBINE_GROUP,
    K_LM_ROWCONST,
    K_LM_CERT,
    K_LM_PICK,
    K_NORM4S_R8,
    K_GEMM_TILED64_S4,
    K_GEMM_TILED32_S4,
    K_EMBED_Q8,
    K_DEQUANT_F16,
    K_SWIGLU_F16,
    K_FPA_D64_G1,    // + (gq - 1): fast (binary16 MFMA) prefill attention
    K_FPA_D128_G1 = K_FPA_D64_G1 + 8,
    K_MERGE_O_D64 = K_FPA_D128_G1 + 8,
    K_MERGE_O_D128,
    K_NORM_QKV_D64,
    K_NORM_QKV_D128,
    K_GEMM_GRPM16,
    K_COUNT
};
inline const char* const kKernelNames[] = {
    "lgx_k_repack_t16", "lgx_k_quantize_q8_0", "lgx_k_q8q8_gemv",
    "lgx_k_q8_gemv_f32", "lgx_k_q8_combine",
    "lgx_k_q8_gemv_mfma", "lgx_k_q8_gemv_mfma_qx", "lgx_k_q8_gemm_mfma16",
    "lgx_k_q8_gemm_mfma32", "lgx_k_q8_gemm_mfma64", "lgx_k_repack_s16",
    "lgx_k_attn_chunk_d64_g1", "lgx_k_attn_chunk_d64_g2", "lgx_k_attn_chunk_d64_g3",
    "lgx_k_attn_chunk_d64_g4", "lgx_k_attn_chunk_d64_g5", "lgx_k_attn_chunk_d64_g6",
    "lgx_k_attn_chunk_d64_g7", "lgx_k_attn_chunk_d64_g8",
    "lgx_k_attn_chunk_d128_g1", "lgx_k_attn_chunk_d128_g2", "lgx_k_attn_chunk_d128_g3",
    "lgx_k_attn_chunk_d128_g4", "lgx_k_attn_chunk_d128_g5", "lgx_k_attn_chunk_d128_g6",
    "lgx_k_attn_chunk_d128_g7", "lgx_k_attn_chunk_d128_g8",
    "lgx_k_attn_combine_d64", "lgx_k_attn_combine_d128",
    "lgx_k_embed", "lgx_k_add_rmsnorm_quant", "lgx_k_qkv_rope_append",
    "lgx_k_attn_combine_quant_d64", "lgx_k_attn_combine_quant_d128", "lgx_k_swiglu_quant",
    "lgx_k_lm_head_f16", "lgx_k_argmax_partial", "lgx_k_argmax_final", "lgx_k_advance",
    "lgx_k_q8_gemv_wg4", "lgx_k_q8_gemv_wg8", "lgx_k_q8_gemv_wg16",
    "lgx_k_q8_gemv_grp4", "lgx_k_q8_gemv_grp8", "lgx_k_q8_gemv_grp16",
    "lgx_k_repack_f16_t64", "lgx_k_lm_head_t64", "lgx_k_rows_to_t16",
    "lgx_k_q8_gemv_grpq4", "lgx_k_q8_gemv_grpq8", "lgx_k_q8_gemv_grpq16",
    "lgx_k_add_rmsnorm_quant4_r8", "lgx_k_add_rmsnorm_quant4_r20",
    "lgx_k_act_to_t16", "lgx_k_q8_gemm_tiled", "lgx_k_q8_gemm_tiled64", "lgx_k_q8_gemm_tiled32",
    "lgx_k_attn_prefill_d64_g1", "lgx_k_attn_prefill_d64_g2", "lgx_k_attn_prefill_d64_g3",
    "lgx_k_attn_prefill_d64_g4", "lgx_k_attn_prefill_d64_g5", "lgx_k_attn_prefill_d64_g6",
    "lgx_k_attn_prefill_d64_g7", "lgx_k_attn_prefill_d64_g8",
    "lgx_k_attn_prefill_d128_g1", "lgx_k_attn_prefill_d128_g2", "lgx_k_attn_prefill_d128_g3",
    "lgx_k_attn_prefill_d128_g4", "lgx_k_attn_prefill_d128_g5", "lgx_k_attn_prefill_d128_g6",
    "lgx_k_attn_prefill_d128_g7", "lgx_k_attn_prefill_d128_g8",
    "lgx_k_sample_partial", "lgx_k_sample_final",
    "lgx_k_q8_gemm_mfma16_qkv", "lgx_k_q8_gemm_mfma16_swiglu", "lgx_k_add_rmsnorm_quant_w",
    "lgx_k_q8_gemm_mfma16_group", "lgx_k_q8_gemm_tiled_group", "lgx_k_q8_gemm_tiled64_group",
    "lgx_k_q8_gemm_tiled32_group", "lgx_k_quantize_group", "lgx_k_q8_combine_group",
    "lgx_k_lm_rowconst", "lgx_k_lm_cert", "lgx_k_lm_pick", "lgx_k_add_rmsnorm_quant4s_r8",
    "lgx_k_q8_gemm_tiled64s4", "lgx_k_q8_gemm_tiled32s4", "lgx_k_embed_q8", "lgx_k_dequant_f16",
    "lgx_k_swiglu_f16",
    "lgx_k_attn_prefill_fast_d64_g1", "lgx_k_attn_prefill_fast_d64_g2", "lgx_k_attn_prefill_fast_d64_g3",
    "lgx_k_attn_prefill_fast_d64_g4", "lgx_k_attn_prefill_fast_d64_g5", "lgx_k_attn_prefill_fast_d64_g6",
    "lgx_k_attn_prefill_fast_d64_g7", "lgx_k_attn_prefill_fast_d64_g8",
    "lgx_k_attn_prefill_fast_d128_g1", "lgx_k_attn_prefill_fast_d128_g2", "lgx_k_attn_prefill_fast_d128_g3",
    "lgx_k_attn_prefill_fast_d128_g4", "lgx_k_attn_prefill_fast_d128_g5", "lgx_k_attn_prefill_fast_d128_g6",
    "lgx_k_attn_prefill_fast_d128_g7", "lgx_k_attn_prefill_fast_d128_g8",
    "lgx_k_attn_merge_o_d64", "lgx_k_attn_merge_o_d128", "lgx_k_norm_qkv_d64", "lgx_k_norm_qkv_d128",
    "lgx_k_q8_gemm_grpm16",
};

static_assert(sizeof(kKernelNames) / sizeof(kKernelNames[0]) == K_COUNT,
              "one code-object name per kernel slot");

// Attention chunk kernel for head_dim d and query heads per KV head gq.
inline int attn_kernel(int d, int gq) {
    if (gq < 1 || gq > 8) return -1;
    return (d == 64 ? K_ATTN_D64_G1 : K_ATTN_D128_G1) + gq - 1;
}

// Prefill (multi-query causal) attention kernel for head_dim d, gq heads per KV head.
inline int prefill_attn_kernel(int d, int gq) {
    if (gq < 1 || gq > 8) return -1;
    return (d == 64 ? K_PFA_D64_G1 : K_PFA_D128_G1) + gq - 1;
}
// Debug/tuning knobs read once per ctx from the environment:
//   LGX_GEMV=dot4   route lgx_q8q8_gemv to the v_dot4 GEMV instead of MFMA
//   LGX_WG_TARGET=n workgroups the streaming kernels aim for (default 512)
inline int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

}  // namespace lgxi

struct lgx_ctx {
    uint32_t magic = 0x4c47584bu;  // "LGXK"
    int device = 0;
    hipModule_t module = nullptr;
    hipFunction_t fn[lgxi::K_COUNT] = {};
    std::string arch;
    bool gemv_dot4 = false;       // LGX_GEMV=dot4: per-(tile, range) dot4 GEMV
    bool gemv_split = false;      // LGX_GEMV=split: per-(tile, range) MFMA GEMV
    int gemv_wgs = 0;             // LGX_GEMV_WGS: M = 1 GEMV waves per workgroup (0: auto)
    bool gemv_whole = false;      // LGX_GEMV=whole: block dots through LDS, chains after
    int gemm_mt = 0;              // LGX_GEMM_MT: force the M > 1 m-tile width (0: by m)
    int tiled_min = 33;           // LGX_GEMM_TILED_MIN: smallest m through the tiled product
    int tiled_rows = 0;           // LGX_GEMM_TILED_ROWS: force 128/64/32 activation rows per workgroup
    int tiled_grp = 0;            // LGX_GEMM_TILED_GRP: force 1/2/4 ranges per group
    int tiled_wpc = 4;            // LGX_GEMM_TILED_WPC: workgroups per CU the automatic group choice keeps
    bool decode_streaming = false; // LGX_DECODE_GEMM=streaming: decode products of m >= 17
                                   // rows through the streaming kernels
    bool decode_fuse = true;      // LGX_DECODE_FUSE=0: decode glue in kernels of its own
    int fuse_cols32 = 1;          // LGX_FUSE_SWIGLU_COLS: SwiGLU columns per fused workgroup / 32
    int merge_o_tiles = 8;        // LGX_MERGE_O_TILES: o_proj row tiles per merge+o workgroup (1..16)
    bool gemm_grpm = true;        // LGX_GEMM_GRPM=0: grouped products of 2..8 rows on the multi-launch path
    int max_lds = 65536;          // LDS bytes a workgroup may hold (the device's figure)
    bool tiled_swiglu = true;     // LGX_TILED_SWIGLU=0: tiled gate|up products leave their outputs to lgx_k_swiglu_quant
    int norm_waves = 1;           // LGX_NORM_WAVES: rows (waves) per workgroup of the wave norm (0: off)
    bool lm_cert = true;          // LGX_LM_CERT=0: greedy tied lm_head through the full logits
    bool tiled_s4 = true;         // LGX_TILED_S4=0: tiled products always in stages of 2 pairs
    bool prefill_serial = false;  // LGX_PREFILL=serial: prefill as P decode passes
    int prefill_chunk = 0;        // LGX_PREFILL_CHUNK: positions per prefill chunk (0: by batch)
    int ncu = 256;                // compute units of the device
    int wg_target = 512;
    std::atomic<uint64_t> launches{0};
    std::atomic<int> live_models{0};  // lgx_model handles built on this ctx and not destroyed
    void* ws = nullptr;       // range partials
    size_t ws_bytes = 0;
    void* scratch = nullptr;  // this device's LGX_NOALLOC_SCRATCH_BYTES array (lgx_scratch.hip)
    std::mutex ws_mu;
    // per-kernel device timing (lgx_ctx_set_kernel_timing): launches go
    // through hipExtModuleLaunchKernel with start/stop events attached to the
    // dispatch itself
    bool timing = false;
    struct Timed {
        int kern;
        hipEvent_t start, stop;
    };
    std::vector<Timed> timed;
    std::vector<hipEvent_t> event_pool;
};

// lgx_f16gemm.cpp: the fast prefill's plain binary16 GEMM (hipBLASLt),
// y[m][n] = x[m][k] . w[n][k]^T, both binary16 row-major, y binary32 or
// (y16) binary16.
namespace lgxi {
struct F16Gemm;
lgx_status f16gemm_create(F16Gemm** out);
void f16gemm_destroy(F16Gemm* g);
lgx_status f16gemm_run(F16Gemm* g, const uint16_t* w, const uint16_t* x, void* y, bool y16, int m,
                       int n, int k, void* stream);
// the plan of that shape made now (hipBLASLt's heuristic query), nothing run
lgx_status f16gemm_prepare(F16Gemm* g, const uint16_t* w, const uint16_t* x, void* y, bool y16, int m,
                           int n, int k, void* stream);
}  // namespace lgxi

// lgx_scratch.hip: device address of the fixed scratch array on `device`
// (current), resolved once per device with hipGetSymbolAddress.
extern "C" hipError_t lgxi_scratch_ptr(int device, void** out);

namespace lgxi {

inline bool valid_ctx(const lgx_ctx* c) { return c != nullptr && c->magic == 0x4c47584bu; }

inline std::string default_hsaco_path() {
    Dl_info info{};
    if (dladdr((void*)&lgx_abi_version, &info) && info.dli_fname) {
        std::string p(info.dli_fname);
        size_t slash = p.rfind('/');
        std::string dir = slash == std::string::npos ? std::string(".") : p.substr(0, slash);
        return dir + "/lgx_kernels.hsaco";
    }
    return "lgx_kernels.hsaco";
}

inline hipError_t pooled_event(lgx_ctx* c, hipEvent_t* ev) {
    if (!c->event_pool.empty()) {
        *ev = c->event_pool.back();
        c->event_pool.pop_back();
        return hipSuccess;
    }
    return hipEventCreate(ev);
}

template <class Args>
lgx_status launch(lgx_ctx* c, Kern k, dim3 grid, dim3 block, const Args& args, void* stream,
                  unsigned shmem = 0) {
    void* params[] = {(void*)&args};
    hipError_t e;
    if (c->timing && !g_untimed) {
        lgx_ctx::Timed t{k, nullptr, nullptr};
        if ((e = pooled_event(c, &t.start)) != hipSuccess || (e = pooled_event(c, &t.stop)) != hipSuccess)
            return fail(LGX_HIP_ERROR, "hipEventCreate: %s", hipGetErrorString(e));
        e = hipExtModuleLaunchKernel(c->fn[k], grid.x * block.x, grid.y * block.y,
                                     grid.z * block.z, block.x, block.y, block.z, shmem,
                                     (hipStream_t)stream, params, nullptr, t.start, t.stop, 0);
        if (e == hipSuccess) c->timed.push_back(t);
    } else {
        e = hipModuleLaunchKernel(c->fn[k], grid.x, grid.y, grid.z, block.x, block.y, block.z,
                                  shmem, (hipStream_t)stream, params, nullptr);
    }
    if (e != hipSuccess)
        return fail(LGX_HIP_ERROR, "hipModuleLaunchKernel(%s): %s", kKernelNames[k],
                    hipGetErrorString(e));
    const uint64_t n = c->launches.fetch_add(1, std::memory_order_relaxed);
    if (trace_on()) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        (void)hipStreamIsCapturing((hipStream_t)stream, &cs);
        trace_line("launch dev=%d n=%llu %s grid=%ux%ux%u block=%ux%ux%u lds=%u stream=%p%s", c->device,
                   (unsigned long long)n, kKernelNames[k], grid.x, grid.y, grid.z, block.x, block.y, block.z,
                   shmem, stream, cs == hipStreamCaptureStatusActive ? " captured" : "");
    }
    return LGX_OK;
}

inline lgx_status enter(lgx_ctx* c) {
    if (!valid_ctx(c)) return fail(LGX_INVALID_HANDLE, "invalid lgx_ctx handle");
    LGX_HIP(hipSetDevice(c->device));
    g_has_error = false;
    return LGX_OK;
}

// Scratch for range partials, grown on demand.  hipFree of the old buffer
// waits for the device, so work still using it has finished.
inline lgx_status ensure_ws(lgx_ctx* c, size_t bytes, float** out) {
    std::lock_guard<std::mutex> lk(c->ws_mu);
    if (bytes > c->ws_bytes) {
        size_t nb = bytes < (size_t)1 << 20 ? (size_t)1 << 20 : bytes + bytes / 2;
        if (c->ws) LGX_HIP(hipFree(c->ws));
        c->ws = nullptr;
        c->ws_bytes = 0;
        hipError_t e = hipMalloc(&c->ws, nb);
        if (e != hipSuccess)
            return fail(LGX_OUT_OF_MEMORY, "workspace of %zu bytes: %s", nb, hipGetErrorString(e));
        c->ws_bytes = nb;
    }
    *out = (float*)c->ws;
    return LGX_OK;
}

inline unsigned cdiv(int64_t a, int64_t b);

// Residual + RMSNorm (+ Q8_0) of a.m rows: the float4-slot kernels where the
// row fits them (n % 4 == 0, n <= 4096, nr <= 20), else the general one.
inline lgx_status launch_norm(lgx_ctx* c, const lgx_norm_args& a, void* stream) {
    const int nr = a.part ? a.nr : 1;
    // one wave per row for many short rows (prefill); a small batch (decode)
    // runs faster spread over the 512-thread kernel's waves
    if (c->norm_waves > 0 && a.m >= 64 && a.n % 4 == 0 && a.n <= 1024 && nr <= 8 &&
        (!a.xq || a.n % 32 == 0))
        return launch(c, K_NORM_W, dim3(cdiv(a.m, c->norm_waves)), dim3(64 * c->norm_waves), a,
                      stream, 0u);
    // float4 slots through buffer descriptors: the partials' byte span must
    // stay below 2^31
    const bool span_ok = !a.part || ((int64_t)(nr - 1) * a.m * a.n + a.n) * 4 < (1LL << 31);
    if (a.n % 4 == 0 && a.n <= 4096 && nr <= 20 && span_ok)
        return launch(c, nr > 8 ? K_NORM4_R20 : a.n <= 2048 ? K_NORM4S_R8 : K_NORM4_R8, dim3(a.m),
                      dim3(512), a, stream, 0u);
    return launch(c, K_ADD_RMSNORM_QUANT, dim3(a.m), dim3(LGX_GLUE_NT), a, stream, 0u);
}
inline int argmax_slices(int vocab) { return (vocab + LGX_ARGMAX_SLICE - 1) / LGX_ARGMAX_SLICE; }

// Certified greedy token of a tied binary16 lm_head (m <= LGX_LMC_MAXB rows
// of x [m][h], h % 64 == 0, h <= LGX_LMC_MAXH): summaries of the slices
// into summ (m * lm_cert_slices(vocab) records), then the per-row pick
// (+ seq_len advance).
inline int lm_cert_slices(int vocab) { return cdiv(cdiv(vocab, 64), LGX_LMC_GROUPS); }
inline lgx_status launch_lm_cert(lgx_ctx* c, const float* x, const uint16_t* emb,
                                 const uint16_t* emb_t64, const float* rowc, int m, int h,
                                 int vocab, lgx_lmc_summary* summ, float* dbg, int32_t* tokens,
                                 int32_t* seq_len, int advance, void* stream) {
    const int ns = lm_cert_slices(vocab);
    lgx_lmc_args a{x, emb_t64, rowc, summ, dbg, m, h, vocab, ns};
    lgx_status st = launch(c, K_LM_CERT, dim3(ns), dim3(64 * LGX_LMC_GROUPS), a, stream);
    if (st != LGX_OK) return st;
    lgx_lmp_args p{x, emb, summ, tokens, seq_len, m, h, vocab, ns, advance};
    return launch(c, K_LM_PICK, dim3(m), dim3(512), p, stream);
}
inline lgx_status launch_lm_rowconst(lgx_ctx* c, const uint16_t* emb, int vocab, int h,
                                     float* rowc, void* stream) {
    lgx_lmrc_args a{emb, rowc, vocab, h};
    return launch(c, K_LM_ROWCONST, dim3(cdiv(vocab, 4)), dim3(256), a, stream);
}

// Greedy token of m rows of (range-partial) logits: candidates per slice,
// then the per-row pick (+ seq_len advance).  cand holds m * slices floats
// followed by m * slices ints.
inline lgx_status launch_argmax(lgx_ctx* c, const float* part, int nr, int m, int vocab,
                                int32_t* tokens, int32_t* seq_len, int advance, void* cand,
                                void* stream);

// Seeded top-k / top-p draw of m rows of (range-partial) logits: slice
// candidates (m * slices * LGX_SAMPLE_MAX_K keys in cand), then the per-row
// draw; stream of row b is stream0 + b, draw index pos[b] (or seq_len[b]).
struct SampleParams {
    int32_t top_k = 0;      // 0: greedy (argmax)
    float top_p = 1.0f;
    float inv_temp = 1.0f;
    uint64_t seed = 0;
};
inline lgx_status sample_check(int32_t top_k, float top_p, float temperature, int vocab,
                               SampleParams* out) {
    if (top_k < 1 || top_k > LGX_SAMPLE_MAX_K)
        return fail(LGX_INVALID_ARGUMENT, "top_k = %d outside [1, %d]", top_k, LGX_SAMPLE_MAX_K);
    if (!(top_p > 0.0f && top_p <= 1.0f))
        return fail(LGX_INVALID_ARGUMENT, "top_p = %g outside (0, 1]", (double)top_p);
    if (!(temperature > 0.0f) || !std::isfinite(temperature))
        return fail(LGX_INVALID_ARGUMENT, "temperature = %g: need a finite value > 0",
                    (double)temperature);
    if (vocab <= 0 || vocab > 64 * LGX_ARGMAX_SLICE)
        return fail(LGX_UNSUPPORTED, "vocab = %d outside [1, %d] for sampling", vocab,
                    64 * LGX_ARGMAX_SLICE);
    out->top_k = top_k;
    out->top_p = top_p;
    out->inv_temp = 1.0f / temperature;
    return LGX_OK;
}
inline size_t sample_cand_bytes(int m, int vocab) {
    return (size_t)m * argmax_slices(vocab) * LGX_SAMPLE_MAX_K * sizeof(uint64_t);
}
inline lgx_status launch_sample(lgx_ctx* c, const SampleParams& sp, const float* part, int nr,
                                int m, int vocab, const int32_t* pos, int32_t* tokens,
                                int32_t* seq_len, int advance, void* cand, void* stream) {
    lgx_sample_args a{};
    a.part = part;
    a.nr = nr;
    a.tokens = tokens;
    a.seq_len = seq_len;
    a.pos = pos;
    a.cand = (uint64_t*)cand;
    a.seed = sp.seed;
    a.m = m;
    a.vocab = vocab;
    a.nslices = argmax_slices(vocab);
    a.top_k = sp.top_k;
    a.advance = advance;
    a.stream0 = 0;
    a.top_p = sp.top_p;
    a.inv_temp = sp.inv_temp;
    lgx_status st = launch(c, K_SAMPLE_PARTIAL, dim3(a.nslices, m), dim3(256), a, stream);
    if (st != LGX_OK) return st;
    return launch(c, K_SAMPLE_FINAL, dim3(m), dim3(64), a, stream);
}

inline lgx_status check_q8(const lgx_q8_matrix* W) {
    if (!W) return fail(LGX_NULL_POINTER, "W is NULL");
    if (!W->qs || !W->d) return fail(LGX_NULL_POINTER, "W->qs / W->d is NULL");
    if (W->layout != LGX_Q8_T16)
        return fail(LGX_INVALID_ARGUMENT, "W->layout must be LGX_Q8_T16 (got %d)", W->layout);
    if (W->n <= 0 || W->k <= 0 || W->n % 16 != 0 || W->k % 64 != 0)
        return fail(LGX_INVALID_ARGUMENT, "W shape [%d x %d]: need n %% 16 == 0, k %% 64 == 0",
                    W->n, W->k);
    if (W->k > 32 * LGX_Q8_RANGE_BLOCKS * LGX_MAX_RANGES)
        return fail(LGX_OUT_OF_BOUNDS, "W->k = %d exceeds %d", W->k,
                    32 * LGX_Q8_RANGE_BLOCKS * LGX_MAX_RANGES);
    return LGX_OK;
}

inline unsigned cdiv(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }
inline int nranges_of(int k) { return (k / 32 + LGX_Q8_RANGE_BLOCKS - 1) / LGX_Q8_RANGE_BLOCKS; }

// M > 1 product kernel: m-tile width 16 / 32 / 64 rows (LGX_GEMM_MT forces one).
inline Kern gemm_kernel(const lgx_ctx* c, int m) {
    const int mt = c->gemm_mt;
    if (mt == 16) return K_GEMM_MFMA16;
    if (mt == 32) return K_GEMM_MFMA32;
    if (mt == 64) return K_GEMM_MFMA64;
    return m <= 16 ? K_GEMM_MFMA16 : m <= 32 ? K_GEMM_MFMA32 : K_GEMM_MFMA64;
}

// Shared driver of the GEMV/GEMM kernels: one launch over (row tiles, ranges,
// m-groups); with more than one range the partials go to the workspace and
// the combine kernel applies the canonical tree.
inline lgx_status run_q8(lgx_ctx* c, Kern kern, const lgx_q8_matrix* W, const float* xf,
                  const int8_t* xq, const uint16_t* xd, int m, float* y, int32_t* dbg,
                  void* stream, int8_t* xq_out = nullptr, uint16_t* xd_out = nullptr,
                  float* part_out = nullptr, float* part_ws = nullptr) {
    lgx_gemv_args a{};
    a.wt = W->qs;
    a.wd = W->d;
    a.xf = xf;
    a.xq = xq;
    a.xd = xd;
    a.y = y;
    a.dbg = dbg;
    a.xq_out = xq_out;
    a.xd_out = xd_out;
    a.n = W->n;
    a.k = W->k;
    a.m = m;
    a.ntiles = W->n / 16;
    a.nranges = nranges_of(W->k);
    a.nmgroups = (m + 63) / 64;
    if (part_out) {
        // caller-owned partials [nranges][m][n]; no tree here
        a.part = part_out;
        a.y = part_out;
    } else if (a.nranges > 1 && part_ws) {
        a.part = part_ws;   // caller-provided room for nranges * m * n partials
    } else if (a.nranges > 1) {
        lgx_status st = ensure_ws(c, (size_t)a.nranges * m * W->n * sizeof(float), &a.part);
        if (st != LGX_OK) return st;
    }
    const bool streaming =
        kern == K_GEMM_MFMA16 || kern == K_GEMM_MFMA32 || kern == K_GEMM_MFMA64;
    const int mrows = kern == K_GEMM_MFMA16 ? 16 : kern == K_GEMM_MFMA32 ? 32 : 64;
    const int nw = kern == K_GEMM_MFMA64 ? 8 : 4;  // waves per workgroup
    a.nmgroups = streaming ? (m + mrows - 1) / mrows : 1;
    a.tpw = 1;
    if (streaming) {
        // tiles per wave: enough work per wave that the grid is about
        // wg_target workgroups of nw waves
        int64_t tasks = (int64_t)a.ntiles * a.nranges * a.nmgroups;
        int64_t tpw = (tasks + (int64_t)nw * c->wg_target - 1) / ((int64_t)nw * c->wg_target);
        a.tpw = (int)(tpw < 1 ? 1 : tpw > 64 ? 64 : tpw);
    }
    dim3 grid(cdiv(a.ntiles, (int64_t)(streaming ? nw : 4) * a.tpw) * (streaming ? a.nmgroups : 1),
              a.nranges, 1);
    lgx_status st = launch(c, kern, grid, dim3(streaming ? 64 * nw : 256), a, stream);
    if (st != LGX_OK || a.nranges == 1 || part_out) return st;
    lgx_combine_args ca{a.part, y, (int64_t)m * W->n, a.nranges};
    return launch(c, K_COMBINE, dim3(cdiv(ca.count, 256)), dim3(256), ca, stream);
}

// Tiled product: activations in T16 tiles (ceil(m/16) of them), group
// partials part[ceil(nr / grp)][m][n] (canonical subtrees of grp aligned
// ranges, grp in {1, 2, 4}).  Activation rows per workgroup: 128
// (K_GEMM_TILED), 64 or 32.  With swiglu = I (W the [gate; up] matrix of
// 2I rows, I % 32 == 0, one group) the SwiGLU + Q8_0 of the outputs goes to
// sq (T16) / sd instead of part.
inline int tiled_groups(int k, int grp = LGX_TG_RANGES) { return (nranges_of(k) + grp - 1) / grp; }
inline lgx_status run_q8_tiled(lgx_ctx* c, const lgx_q8_matrix* W, const int8_t* xt,
                               const uint16_t* xd, int m, float* part, void* stream,
                               Kern kern = K_GEMM_TILED, int grp = LGX_TG_RANGES,
                               int swiglu = 0, int8_t* sq = nullptr, uint16_t* sd = nullptr) {
    const int mrows = kern == K_GEMM_TILED ? 128 : kern == K_GEMM_TILED64 ? 64 : 32;
    lgx_gemm_tiled_args a{};
    a.wt = W->qs;
    a.wd = W->d;
    a.xt = xt;
    a.xd = xd;
    a.part = part;
    a.n = W->n;
    a.k = W->k;
    a.m = m;
    a.grp = grp;
    a.ngroups = tiled_groups(W->k, grp);
    if (swiglu) {
        if (swiglu % 32 || W->n != 2 * swiglu || a.ngroups != 1 || !sq || !sd)
            return fail(LGX_INVALID_ARGUMENT, "tiled SwiGLU product: n %d, I %d, %d groups", W->n,
                        swiglu, a.ngroups);
        a.swiglu = swiglu;
        a.sq = sq;
        a.sd = sd;
    }
    a.ntn = (int)cdiv(W->n, LGX_TG_N);
    a.ntm = (int)cdiv(m, mrows);
    const int64_t wgs = (int64_t)a.ntn * a.ntm * a.ngroups;
    if (wgs > INT32_MAX) return fail(LGX_OUT_OF_BOUNDS, "tiled product of %lld workgroups", (long long)wgs);
    // a grid of at most two workgroups per compute unit runs in stages of 4
    // pairs: half the dependent memory rounds per workgroup (config-4 o_proj,
    // 448 workgroups: 8.8 against 10.1 us; at 576 workgroups, three share some
    // compute units and the 2-pair stages are faster: 11.9 against 12.8 us)
    if (c->tiled_s4 && wgs <= 2 * (int64_t)c->ncu) {
        if (kern == K_GEMM_TILED32) kern = K_GEMM_TILED32_S4;
        else if (kern == K_GEMM_TILED64) kern = K_GEMM_TILED64_S4;
    }
    return launch(c, kern, dim3((unsigned)wgs), dim3(256), a, stream);
}
// Tiled kernel for m rows: 128 activation rows per workgroup from m >= 128,
// else 32, which also beats 64 at m = 64 (LGX_GEMM_TILED_ROWS forces one).
inline Kern tiled_kernel(const lgx_ctx* c, int m) {
    const int rows = c->tiled_rows ? c->tiled_rows : m >= 128 ? 128 : 32;
    return rows == 128 ? K_GEMM_TILED : rows == 64 ? K_GEMM_TILED64 : K_GEMM_TILED32;
}
// Ranges per group for a product of n outputs, reduction k, over m rows
// through `kern`: the largest of 4, 2, 1 that still gives four workgroups
// per compute unit (fewer partials when the grid is full anyway).
inline int tiled_grp(const lgx_ctx* c, Kern kern, int n, int k, int m) {
    if (c->tiled_grp) return c->tiled_grp;
    const int mrows = kern == K_GEMM_TILED ? 128 : kern == K_GEMM_TILED64 ? 64 : 32;
    const int64_t tiles = (int64_t)cdiv(n, LGX_TG_N) * cdiv(m, mrows);
    for (int grp = 4; grp > 1; grp >>= 1)
        if (tiles * tiled_groups(k, grp) >= (int64_t)c->tiled_wpc * c->ncu) return grp;
    return 1;
}

// Tree + bias + RoPE + K/V append over `rows` rows: 256 rotation pairs per
// workgroup along y.
inline lgx_status launch_qkv_rope(lgx_ctx* c, const lgx_qkv_args& a, int rows, void* stream) {
    const int64_t pairs = (int64_t)(a.hq + 2 * a.hkv) * (a.d / 2);
    return launch(c, K_QKV_ROPE_APPEND, dim3((unsigned)rows, (unsigned)cdiv(pairs, 256)), dim3(256), a,
                  stream);
}

// Row-major int8 activations [m][k] -> T16 tiles at dst (ceil(m/16)*16*k bytes).
inline lgx_status act_to_t16(lgx_ctx* c, const int8_t* xq, int m, int k, int8_t* dst, void* stream) {
    lgx_act_t16_args a{xq, dst, m, k};
    const int64_t slots = (int64_t)cdiv(m, 16) * (k / 64) * 64;
    return launch(c, K_ACT_T16, dim3(cdiv(slots, 256)), dim3(256), a, stream);
}

// Launch of the prefill attention over B sequences x a.qpr query rows:
// one workgroup per (sequence, KV head, chunk of the grid, block of 4 rows).
// Fast prefill attention (binary16 MFMA flash attention, not the canonical
// schedule): one workgroup of gq waves per (sequence, KV head, 16 query
// positions); writes out (binary32) and / or xq / xd (Q8_0).
inline lgx_status launch_prefill_attn_fast(lgx_ctx* c, const lgx_attn_args& a, int d, void* stream) {
    const int gq = a.hq / a.hkv;
    if (gq < 1 || gq > 8 || (d != 64 && d != 128)) return fail(LGX_UNSUPPORTED, "fast prefill attention shape");
    const int k = (d == 64 ? K_FPA_D64_G1 : K_FPA_D128_G1) + gq - 1;
    const int64_t wgs = (int64_t)a.B * a.hkv * ((std::max(a.qpr, 1) + 15) / 16);
    if (wgs > INT32_MAX) return fail(LGX_OUT_OF_BOUNDS, "fast prefill attention grid");
    if (wgs == 0) return LGX_OK;
    return launch(c, (Kern)k, dim3((unsigned)wgs), dim3(64 * gq), a, stream);
}
inline lgx_status launch_prefill_attn(lgx_ctx* c, const lgx_attn_args& a, int d, void* stream) {
    const int k = prefill_attn_kernel(d, a.hq / a.hkv);
    const int64_t wgs = (int64_t)a.B * a.hkv * a.ncg * ((std::max(a.qpr, 1) + 3) / 4);
    if (k < 0 || wgs > INT32_MAX) return fail(LGX_UNSUPPORTED, "prefill attention shape");
    if (wgs == 0) return LGX_OK;
    return launch(c, (Kern)k, dim3((unsigned)wgs), dim3(512), a, stream);
}

}  // namespace lgxi


namespace lgxi {
inline lgx_status launch_argmax(lgx_ctx* c, const float* part, int nr, int m, int vocab,
                                int32_t* tokens, int32_t* seq_len, int advance, void* cand,
                                void* stream) {
    const int ns = argmax_slices(vocab);
    lgx_argmax_args a{};
    a.part = part;
    a.nr = nr;
    a.tokens = tokens;
    a.seq_len = seq_len;
    a.cand_v = (float*)cand;
    a.cand_i = (int32_t*)((float*)cand + (int64_t)m * ns);
    a.m = m;
    a.vocab = vocab;
    a.advance = advance;
    a.nslices = ns;
    lgx_status st = launch(c, K_ARGMAX_PARTIAL, dim3(ns, m), dim3(256), a, stream);
    if (st != LGX_OK) return st;
    return launch(c, K_ARGMAX_FINAL, dim3(m), dim3(64), a, stream);
}
}  // namespace lgxi

namespace lgxi {
// Whole-K GEMV shape for reduction length k in a workgroup of W waves:
// log2 of the waves per tile (about 8 of the 64-column pairs per wave) and
// the LDS bytes (0 if they exceed 64 KiB).
inline int gemv_wg_lwt(int k, int W) {
    const int np = k / 64;
    int lwt = 0;
    while ((1 << lwt) < W && (1 << lwt) * 8 < np) ++lwt;
    return lwt;
}
inline size_t gemv_wg_lds(int k, int W = 4) {
    const size_t nb = k / 32, nr = (nb + LGX_Q8_RANGE_BLOCKS - 1) / LGX_Q8_RANGE_BLOCKS;
    const size_t tpw = (size_t)W >> gemv_wg_lwt(k, W);
    const size_t bytes = (size_t)k + 4 * nb + tpw * (64 * nb + 64 * nr);
    return bytes <= 65536 ? bytes : 0;
}

// Launch the M = 1 GEMV over `count` independent matrices: by default the
// grouped kernel with a tile's ranges inside one workgroup; LGX_GEMV=whole
// selects the whole-K kernel (block dots through LDS).
inline lgx_status run_gemv_group(lgx_ctx* c, const lgx_gemv_mat* mats, int count, void* stream) {
    if (count < 1 || count > LGX_GROUP_MAX)
        return fail(LGX_INVALID_ARGUMENT, "group of %d matrices (1..%d)", count, LGX_GROUP_MAX);
    lgx_gemv_group_args ga{};
    ga.count = count;
    int wgs = 0;
    size_t lds = 0;
    if (c->gemv_whole) {
        int npmax = 0;
        for (int i = 0; i < count; ++i) npmax = std::max(npmax, mats[i].k / 64);
        int W = npmax > 64 ? 16 : 4;
        if (c->gemv_wgs == 4 || c->gemv_wgs == 8 || c->gemv_wgs == 16) W = c->gemv_wgs;
        for (int i = 0; i < count; ++i) {
            ga.mat[i] = mats[i];
            const int lwt = gemv_wg_lwt(mats[i].k, W);
            ga.mat[i].pad = lwt;
            ga.tile0[i] = wgs;
            const int tpw = W >> lwt;
            wgs += (mats[i].n / 16 + tpw - 1) / tpw;
            const size_t l = gemv_wg_lds(mats[i].k, W);
            if (l == 0)
                return fail(LGX_UNSUPPORTED, "k = %d too long for the whole-K GEMV", mats[i].k);
            lds = std::max(lds, l);
        }
        ga.tile0[count] = wgs;
        const Kern k = W == 16 ? K_GEMV_WG16 : W == 8 ? K_GEMV_WG8 : K_GEMV_WG4;
        return launch(c, k, dim3(wgs), dim3(64 * W), ga, stream, (unsigned)lds);
    }
    int nrmax = 1;
    const bool xf = mats[0].xf != nullptr;
    for (int i = 0; i < count; ++i) {
        nrmax = std::max(nrmax, (mats[i].k / 32 + LGX_Q8_RANGE_BLOCKS - 1) / LGX_Q8_RANGE_BLOCKS);
        if ((mats[i].xf != nullptr) != xf)
            return fail(LGX_INVALID_ARGUMENT, "a group mixes binary32 and Q8_0 activations");
    }
    int W = nrmax <= 4 ? 4 : nrmax <= 8 ? 8 : 16;
    if (c->gemv_wgs == 4 || c->gemv_wgs == 8 || c->gemv_wgs == 16) W = c->gemv_wgs;
    // Tiles per workgroup: the smallest per-workgroup byte budget T for which
    // the grid fits the device (ncu * 16 / W workgroups, each CU holding 16
    // waves), tpw_i = clamp(T / tile bytes, 1, W / ranges): the bytes per
    // workgroup are as even as whole tiles allow.
    int tmax[LGX_GROUP_MAX], tpw[LGX_GROUP_MAX], nrg[LGX_GROUP_MAX];
    double tb[LGX_GROUP_MAX];
    std::vector<double> cand;
    for (int i = 0; i < count; ++i) {
        nrg[i] = (mats[i].k / 32 + LGX_Q8_RANGE_BLOCKS - 1) / LGX_Q8_RANGE_BLOCKS;
        tmax[i] = W / std::min(nrg[i], W);
        tb[i] = 17.0 * mats[i].k;                      // 16 rows x k x 1.0625 B
        for (int j = 1; j <= tmax[i]; ++j) cand.push_back(j * tb[i]);
    }
    std::sort(cand.begin(), cand.end());
    const int64_t cap = (int64_t)c->ncu * (16 / W);
    auto grid_for = [&](double T, int* tp) {
        int64_t n = 0;
        for (int i = 0; i < count; ++i) {
            tp[i] = std::max(1, std::min(tmax[i], (int)(T / tb[i] + 1e-9)));
            n += (mats[i].n / 16 + tp[i] - 1) / tp[i];
        }
        return n;
    };
    for (int i = 0; i < count; ++i) tpw[i] = tmax[i];
    for (double T : cand) {
        int tp[LGX_GROUP_MAX];
        if (grid_for(T, tp) <= cap) {
            std::copy(tp, tp + count, tpw);
            break;
        }
    }
    for (int i = 0; i < count; ++i) {
        ga.mat[i] = mats[i];
        ga.mat[i].pad = tpw[i];
        ga.tile0[i] = wgs;
        wgs += (mats[i].n / 16 + tpw[i] - 1) / tpw[i];
        lds = std::max(lds, (size_t)W * (1024 + 32 * 4) + 64 * (size_t)tpw[i] * nrg[i]);
    }
    ga.tile0[count] = wgs;
    const Kern k = xf ? (W == 16 ? K_GEMV_GRP16 : W == 8 ? K_GEMV_GRP8 : K_GEMV_GRP4)
                      : (W == 16 ? K_GEMV_GRPQ16 : W == 8 ? K_GEMV_GRPQ8 : K_GEMV_GRPQ4);
    return launch(c, k, dim3(wgs), dim3(64 * W), ga, stream, (unsigned)lds);
}

// Grouped products of 2..LGX_GRPM_ROWS binary32 rows in one launch
// (lgx_k_q8_gemm_grpm16): the grouped GEMV's tiles per workgroup, one wave
// per (tile slot, range), every matrix at most 16 ranges (k <= 16384).
inline bool gemm_grpm_ok(const lgx_ctx* c, const lgx_gemv_mat* mats, int count, int m) {
    if (!c->gemm_grpm || m < 2 || m > LGX_GRPM_ROWS) return false;
    for (int i = 0; i < count; ++i) {
        const int nr = (mats[i].k / 32 + LGX_Q8_RANGE_BLOCKS - 1) / LGX_Q8_RANGE_BLOCKS;
        // the staging of every range and the partials of 16 / nr tiles
        const size_t lds = (size_t)nr * LGX_GRPM_ROWS * (1024 + 32 * 4) + (size_t)16 * LGX_GRPM_ROWS * 16 * 4;
        if (nr > 16 || lds > (size_t)c->max_lds) return false;
    }
    return true;
}
inline lgx_status run_gemm_grpm(lgx_ctx* c, const lgx_gemv_mat* mats, int count, int m, void* stream) {
    constexpr int W = 16;
    lgx_gemv_group_args ga{};
    ga.count = count;
    ga.pad = m;
    int tmax[LGX_GROUP_MAX], tpw[LGX_GROUP_MAX], nrg[LGX_GROUP_MAX];
    double tb[LGX_GROUP_MAX];
    std::vector<double> cand;
    for (int i = 0; i < count; ++i) {
        nrg[i] = (mats[i].k / 32 + LGX_Q8_RANGE_BLOCKS - 1) / LGX_Q8_RANGE_BLOCKS;
        tmax[i] = W / nrg[i];
        tb[i] = 17.0 * mats[i].k;                      // 16 rows x k x 1.0625 B
        for (int j = 1; j <= tmax[i]; ++j) cand.push_back(j * tb[i]);
    }
    std::sort(cand.begin(), cand.end());
    // as run_gemv_group: the smallest per-workgroup byte budget whose grid
    // fits one workgroup per compute unit
    auto grid_for = [&](double T, int* tp) {
        int64_t n = 0;
        for (int i = 0; i < count; ++i) {
            tp[i] = std::max(1, std::min(tmax[i], (int)(T / tb[i] + 1e-9)));
            n += (mats[i].n / 16 + tp[i] - 1) / tp[i];
        }
        return n;
    };
    for (int i = 0; i < count; ++i) tpw[i] = tmax[i];
    for (double T : cand) {
        int tp[LGX_GROUP_MAX];
        if (grid_for(T, tp) <= (int64_t)c->ncu) {
            std::copy(tp, tp + count, tpw);
            break;
        }
    }
    int wgs = 0;
    size_t lds = 0;
    for (int i = 0; i < count; ++i) {
        ga.mat[i] = mats[i];
        ga.mat[i].pad = tpw[i];
        ga.tile0[i] = wgs;
        wgs += (mats[i].n / 16 + tpw[i] - 1) / tpw[i];
        lds = std::max(lds, (size_t)nrg[i] * LGX_GRPM_ROWS * (1024 + 32 * 4) +
                                (size_t)tpw[i] * nrg[i] * LGX_GRPM_ROWS * 16 * 4);
    }
    ga.tile0[count] = wgs;
    return launch(c, K_GEMM_GRPM16, dim3(wgs), dim3(64 * W), ga, stream, (unsigned)lds);
}

// Whether the M = 1 products of reduction length k go through run_gemv_group.
inline bool gemv_group_ok(const lgx_ctx* c, int k) {
    return !c->gemv_whole || gemv_wg_lds(k) != 0;
}

inline lgx_gemv_mat gemv_mat(const lgx_q8_matrix* W, const float* xf, const int8_t* xq,
                             const uint16_t* xd, float* y, int part_out) {
    lgx_gemv_mat m{};
    m.wt = W->qs;
    m.wd = W->d;
    m.xf = xf;
    m.xq = xq;
    m.xd = xd;
    m.y = y;
    m.n = W->n;
    m.k = W->k;
    m.part_out = part_out;
    return m;
}
}  // namespace lgxi
