// lgx_host.cpp -- liblgx: the extern "C" launcher over hipModuleLoad /
// hipModuleGetFunction / hipModuleLaunchKernel for the kernels in
// lgx_kernels.hsaco.  No CUDA-compat headers, no runtime-API kernel
// launches: kernels are resolved by name from the code object, exactly as
// the reference's AOT tier resolves `logos_native_<fn>` symbols from a built
// library (crates/logicaffeine_compile/src/vm/aot_tier.rs:86-111).
//
// Error discipline follows crates/logicaffeine_compile/src/codegen/ffi.rs:
// every entry point returns a status, stores a thread-local message, and
// catches every C++ exception at the boundary (ffi.rs:329-340 wraps every
// export in catch_unwind the same way).
#include <hip/hip_runtime_api.h>

#include <dlfcn.h>

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

namespace {

thread_local std::string g_last_error;
thread_local bool g_has_error = false;

lgx_status fail(lgx_status st, const char* fmt, ...) {
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
    K_COUNT
};
const char* const kKernelNames[] = {
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
};

static_assert(sizeof(kKernelNames) / sizeof(kKernelNames[0]) == K_COUNT,
              "one code-object name per kernel slot");

// Attention chunk kernel for head_dim d and query heads per KV head gq.
int attn_kernel(int d, int gq) {
    if (gq < 1 || gq > 8) return -1;
    return (d == 64 ? K_ATTN_D64_G1 : K_ATTN_D128_G1) + gq - 1;
}

// Debug/tuning knobs read once per ctx (documented in DESIGN.md):
//   LGX_GEMV=dot4   route lgx_q8q8_gemv to the v_dot4 GEMV instead of MFMA
//   LGX_WG_TARGET=n workgroups the streaming kernels aim for (default 512)
int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

}  // namespace

struct lgx_ctx {
    uint32_t magic = 0x4c47584bu;  // "LGXK"
    int device = 0;
    hipModule_t module = nullptr;
    hipFunction_t fn[K_COUNT] = {};
    std::string arch;
    bool gemv_dot4 = false;
    int wg_target = 512;
    std::atomic<uint64_t> launches{0};
    void* ws = nullptr;       // range partials
    size_t ws_bytes = 0;
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

namespace {

bool valid_ctx(const lgx_ctx* c) { return c != nullptr && c->magic == 0x4c47584bu; }

std::string default_hsaco_path() {
    Dl_info info{};
    if (dladdr((void*)&lgx_abi_version, &info) && info.dli_fname) {
        std::string p(info.dli_fname);
        size_t slash = p.rfind('/');
        std::string dir = slash == std::string::npos ? std::string(".") : p.substr(0, slash);
        return dir + "/lgx_kernels.hsaco";
    }
    return "lgx_kernels.hsaco";
}

hipError_t pooled_event(lgx_ctx* c, hipEvent_t* ev) {
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
    if (c->timing) {
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
    c->launches.fetch_add(1, std::memory_order_relaxed);
    return LGX_OK;
}

lgx_status enter(lgx_ctx* c) {
    if (!valid_ctx(c)) return fail(LGX_INVALID_HANDLE, "invalid lgx_ctx handle");
    LGX_HIP(hipSetDevice(c->device));
    g_has_error = false;
    return LGX_OK;
}

// Scratch for range partials, grown on demand.  hipFree of the old buffer
// waits for the device, so work still using it has finished.
lgx_status ensure_ws(lgx_ctx* c, size_t bytes, float** out) {
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

lgx_status check_q8(const lgx_q8_matrix* W) {
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

// Shared driver of the GEMV/GEMM kernels: one launch over (row tiles, ranges,
// m-groups); with more than one range the partials go to the workspace and
// the combine kernel applies the canonical tree.
lgx_status run_q8(lgx_ctx* c, Kern kern, const lgx_q8_matrix* W, const float* xf,
                  const int8_t* xq, const uint16_t* xd, int m, float* y, int32_t* dbg,
                  void* stream, int8_t* xq_out = nullptr, uint16_t* xd_out = nullptr,
                  float* part_out = nullptr) {
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
    } else if (a.nranges > 1) {
        lgx_status st = ensure_ws(c, (size_t)a.nranges * m * W->n * sizeof(float), &a.part);
        if (st != LGX_OK) return st;
    }
    const bool streaming =
        kern == K_GEMM_MFMA16 || kern == K_GEMM_MFMA32 || kern == K_GEMM_MFMA64;
    const int mrows = kern == K_GEMM_MFMA16 ? 16 : kern == K_GEMM_MFMA32 ? 32 : 64;
    a.nmgroups = streaming ? (m + mrows - 1) / mrows : 1;
    a.tpw = 1;
    if (streaming) {
        // tiles per wave: enough work per wave that the grid is about
        // wg_target workgroups of 4 waves
        int64_t tasks = (int64_t)a.ntiles * a.nranges * a.nmgroups;
        int64_t tpw = (tasks + 4LL * c->wg_target - 1) / (4LL * c->wg_target);
        a.tpw = (int)(tpw < 1 ? 1 : tpw > 64 ? 64 : tpw);
    }
    dim3 grid(cdiv(a.ntiles, 4LL * a.tpw), a.nranges,
              streaming ? a.nmgroups : 1);
    lgx_status st = launch(c, kern, grid, dim3(256), a, stream);
    if (st != LGX_OK || a.nranges == 1 || part_out) return st;
    lgx_combine_args ca{a.part, y, (int64_t)m * W->n, a.nranges};
    return launch(c, K_COMBINE, dim3(cdiv(ca.count, 256)), dim3(256), ca, stream);
}

}  // namespace

extern "C" {

uint32_t lgx_abi_version(void) { return LGX_ABI_VERSION; }

const char* lgx_version(void) { return "lgx 0.1.0 (gfx950)"; }

const char* lgx_last_error(void) { return g_has_error ? g_last_error.c_str() : nullptr; }

void lgx_clear_error(void) {
    g_has_error = false;
    g_last_error.clear();
}

lgx_status lgx_ctx_create(int32_t device, const char* hsaco_path, lgx_ctx** out) {
    return guarded(__func__, [&]() -> lgx_status {
        if (!out) return fail(LGX_NULL_POINTER, "out is NULL");
        *out = nullptr;
        int ndev = 0;
        hipError_t e = hipGetDeviceCount(&ndev);
        if (e != hipSuccess || ndev == 0)
            return fail(LGX_NO_DEVICE, "no HIP device available (%s)",
                        e == hipSuccess ? "count 0" : hipGetErrorString(e));
        if (device < 0 || device >= ndev)
            return fail(LGX_OUT_OF_BOUNDS, "device %d out of range [0, %d)", device, ndev);
        LGX_HIP(hipSetDevice(device));
        hipDeviceProp_t prop;
        LGX_HIP(hipGetDeviceProperties(&prop, device));
        std::string arch(prop.gcnArchName);
        arch = arch.substr(0, arch.find(':'));
        if (arch != "gfx950")
            return fail(LGX_UNSUPPORTED, "device %d is %s; lgx kernels are built for gfx950",
                        device, arch.c_str());
        std::string path = hsaco_path ? std::string(hsaco_path) : default_hsaco_path();
        hipModule_t mod = nullptr;
        e = hipModuleLoad(&mod, path.c_str());
        if (e != hipSuccess)
            return fail(LGX_MODULE_LOAD_FAILED, "hipModuleLoad(%s): %s", path.c_str(),
                        hipGetErrorString(e));
        lgx_ctx* c = new lgx_ctx();
        c->device = device;
        c->module = mod;
        c->arch = arch;
        const char* gv = getenv("LGX_GEMV");
        c->gemv_dot4 = gv && std::string(gv) == "dot4";
        c->wg_target = env_int("LGX_WG_TARGET", 512);
        if (c->wg_target < 1) c->wg_target = 1;
        for (int k = 0; k < K_COUNT; ++k) {
            e = hipModuleGetFunction(&c->fn[k], mod, kKernelNames[k]);
            if (e != hipSuccess) {
                (void)hipModuleUnload(mod);
                delete c;
                return fail(LGX_MODULE_LOAD_FAILED, "hipModuleGetFunction(%s) in %s: %s",
                            kKernelNames[k], path.c_str(), hipGetErrorString(e));
            }
        }
        *out = c;
        g_has_error = false;
        return LGX_OK;
    });
}

lgx_status lgx_ctx_destroy(lgx_ctx* c) {
    return guarded(__func__, [&]() -> lgx_status {
        if (!valid_ctx(c)) return fail(LGX_INVALID_HANDLE, "invalid lgx_ctx handle");
        (void)hipSetDevice(c->device);
        for (auto& t : c->timed) {
            (void)hipEventDestroy(t.start);
            (void)hipEventDestroy(t.stop);
        }
        for (auto ev : c->event_pool) (void)hipEventDestroy(ev);
        if (c->ws) (void)hipFree(c->ws);
        if (c->module) (void)hipModuleUnload(c->module);
        c->magic = 0;
        delete c;
        return LGX_OK;
    });
}

uint64_t lgx_ctx_launch_count(const lgx_ctx* c) {
    return valid_ctx(c) ? c->launches.load(std::memory_order_relaxed) : 0;
}

const char* lgx_ctx_arch(const lgx_ctx* c) { return valid_ctx(c) ? c->arch.c_str() : nullptr; }

lgx_status lgx_ctx_set_kernel_timing(lgx_ctx* c, int32_t enable) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (enable) {
            // a fresh window: previous records go back to the pool once done
            for (auto& t : c->timed) {
                LGX_HIP(hipEventSynchronize(t.stop));
                c->event_pool.push_back(t.start);
                c->event_pool.push_back(t.stop);
            }
            c->timed.clear();
        }
        c->timing = enable != 0;
        return LGX_OK;
    });
}

lgx_status lgx_ctx_kernel_stats(lgx_ctx* c, const char* kernel_name, uint64_t* count,
                                double* total_ms) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!kernel_name || !count || !total_ms) return fail(LGX_NULL_POINTER, "NULL argument");
        uint64_t n = 0;
        double ms = 0.0;
        for (auto& t : c->timed) {
            if (std::strcmp(kKernelNames[t.kern], kernel_name) != 0) continue;
            LGX_HIP(hipEventSynchronize(t.stop));
            float e = 0.0f;
            LGX_HIP(hipEventElapsedTime(&e, t.start, t.stop));
            ++n;
            ms += e;
        }
        *count = n;
        *total_ms = ms;
        return LGX_OK;
    });
}

size_t lgx_q8_scale_count(int32_t n, int32_t k) {
    if (n <= 0 || k <= 0 || n % 16 != 0 || k % 64 != 0) return 0;
    return (size_t)(n / 16) * (size_t)((k + 511) / 512) * 256;
}

static lgx_status repack_impl(lgx_ctx* c, const int8_t* qsrc, const uint16_t* dsrc, int32_t n,
                              int32_t k, int8_t* qdst, uint16_t* ddst, int to_t16, void* stream) {
    lgx_status st = enter(c);
    if (st != LGX_OK) return st;
    if (!qsrc || !qdst || !dsrc || !ddst) return fail(LGX_NULL_POINTER, "NULL quants/scales pointer");
    if (n <= 0 || k <= 0 || n % 16 != 0 || k % 64 != 0)
        return fail(LGX_INVALID_ARGUMENT, "shape [%d x %d]: need n %% 16 == 0, k %% 64 == 0", n, k);
    lgx_repack_args a{qsrc, qdst, n, k, to_t16};
    int64_t total = (int64_t)(n / 16) * (k / 64) * 64;
    st = launch(c, K_REPACK, dim3(cdiv(total, 256)), dim3(256), a, stream);
    if (st != LGX_OK) return st;
    lgx_srepack_args sa{dsrc, ddst, n, k, to_t16};
    return launch(c, K_REPACK_S16, dim3(cdiv((int64_t)lgx_q8_scale_count(n, k), 256)), dim3(256),
                  sa, stream);
}

lgx_status lgx_q8_repack_t16(lgx_ctx* c, const int8_t* qs, const uint16_t* d, int32_t n,
                             int32_t k, int8_t* qs_t16, uint16_t* d_s16, void* stream) {
    return guarded(__func__, [&] { return repack_impl(c, qs, d, n, k, qs_t16, d_s16, 1, stream); });
}

lgx_status lgx_q8_unpack_t16(lgx_ctx* c, const int8_t* qs_t16, const uint16_t* d_s16, int32_t n,
                             int32_t k, int8_t* qs, uint16_t* d, void* stream) {
    return guarded(__func__, [&] { return repack_impl(c, qs_t16, d_s16, n, k, qs, d, 0, stream); });
}

lgx_status lgx_quantize_q8_0(lgx_ctx* c, const float* x, int32_t m, int32_t k, int8_t* qs,
                             uint16_t* d, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!x || !qs || !d) return fail(LGX_NULL_POINTER, "NULL tensor pointer");
        if (m <= 0 || k <= 0 || k % 32 != 0)
            return fail(LGX_INVALID_ARGUMENT, "shape [%d x %d]: need m > 0, k %% 32 == 0", m, k);
        lgx_quant_args a{x, qs, d, m, k};
        return launch(c, K_QUANT, dim3(cdiv((int64_t)m * (k / 32), 256)), dim3(256), a, stream);
    });
}

lgx_status lgx_q8_gemv_f32(lgx_ctx* c, const lgx_q8_matrix* W, const float* x, float* y,
                           void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if ((st = check_q8(W)) != LGX_OK) return st;
        if (!x || !y) return fail(LGX_NULL_POINTER, "NULL x or y");
        return run_q8(c, K_Q8_GEMV_F32, W, x, nullptr, nullptr, 1, y, nullptr, stream);
    });
}

lgx_status lgx_q8q8_gemv(lgx_ctx* c, const lgx_q8_matrix* W, const int8_t* xq,
                         const uint16_t* xd, float* y, int32_t* dbg, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if ((st = check_q8(W)) != LGX_OK) return st;
        if (!xq || !xd || !y) return fail(LGX_NULL_POINTER, "NULL xq, xd or y");
        // the block-dot debug output exists only in the v_dot4 kernel
        if (dbg || c->gemv_dot4)
            return run_q8(c, K_Q8Q8_GEMV, W, nullptr, xq, xd, 1, y, dbg, stream);
        return run_q8(c, K_GEMV_MFMA, W, nullptr, xq, xd, 1, y, nullptr, stream);
    });
}

lgx_status lgx_q8q8_gemv_quantize(lgx_ctx* c, const lgx_q8_matrix* W, const float* x, float* y,
                                  int8_t* xq_out, uint16_t* xd_out, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if ((st = check_q8(W)) != LGX_OK) return st;
        if (!x || !y) return fail(LGX_NULL_POINTER, "NULL x or y");
        return run_q8(c, K_GEMV_MFMA_QX, W, x, nullptr, nullptr, 1, y, nullptr, stream, xq_out,
                      xd_out);
    });
}

int32_t lgx_q8_range_count(int32_t k) { return k > 0 ? nranges_of(k) : 0; }

lgx_status lgx_q8q8_gemv_quantize_partials(lgx_ctx* c, const lgx_q8_matrix* W, const float* x,
                                           float* part, int8_t* xq_out, uint16_t* xd_out,
                                           void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if ((st = check_q8(W)) != LGX_OK) return st;
        if (!x || !part) return fail(LGX_NULL_POINTER, "NULL x or part");
        return run_q8(c, K_GEMV_MFMA_QX, W, x, nullptr, nullptr, 1, part, nullptr, stream, xq_out,
                      xd_out, part);
    });
}

lgx_status lgx_q8_gemm_partials(lgx_ctx* c, const lgx_q8_matrix* W, const int8_t* xq,
                                const uint16_t* xd, int32_t m, float* part, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if ((st = check_q8(W)) != LGX_OK) return st;
        if (!xq || !xd || !part) return fail(LGX_NULL_POINTER, "NULL xq, xd or part");
        if (m <= 0 || m > 65535 * 64) return fail(LGX_OUT_OF_BOUNDS, "m = %d out of range", m);
        Kern k = m == 1 ? K_GEMV_MFMA : m <= 16 ? K_GEMM_MFMA16 : m <= 32 ? K_GEMM_MFMA32
                                                                          : K_GEMM_MFMA64;
        return run_q8(c, k, W, nullptr, xq, xd, m, part, nullptr, stream, nullptr, nullptr, part);
    });
}

lgx_status lgx_q8_range_combine(lgx_ctx* c, const float* part, int32_t nranges, int64_t count,
                                float* y, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!part || !y) return fail(LGX_NULL_POINTER, "NULL part or y");
        if (nranges < 1 || nranges > LGX_MAX_RANGES || count <= 0)
            return fail(LGX_INVALID_ARGUMENT, "nranges %d / count %lld", nranges, (long long)count);
        lgx_combine_args ca{part, y, count, nranges};
        return launch(c, K_COMBINE, dim3(cdiv(count, 256)), dim3(256), ca, stream);
    });
}

lgx_status lgx_gqa_decode_attn(lgx_ctx* c, const float* q, const uint16_t* kpages,
                               const uint16_t* vpages, const int32_t* page_table,
                               const int32_t* seq_len, int32_t B, int32_t hq, int32_t hkv,
                               int32_t d, int32_t maxp, int32_t num_pages, int32_t max_seq_len,
                               float* out, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!q || !kpages || !vpages || !page_table || !seq_len || !out)
            return fail(LGX_NULL_POINTER, "NULL tensor pointer");
        if (B <= 0 || hq <= 0 || hkv <= 0 || hq % hkv != 0 || maxp <= 0 || num_pages <= 0)
            return fail(LGX_INVALID_ARGUMENT, "B=%d hq=%d hkv=%d maxp=%d num_pages=%d", B, hq, hkv,
                        maxp, num_pages);
        const int k = attn_kernel(d, hq / hkv);
        if ((d != 64 && d != 128) || k < 0)
            return fail(LGX_UNSUPPORTED, "head_dim %d / %d query heads per KV head", d, hq / hkv);
        if (max_seq_len <= 0 || max_seq_len > maxp * LGX_PAGE)
            return fail(LGX_OUT_OF_BOUNDS, "max_seq_len %d outside (0, %d]", max_seq_len,
                        maxp * LGX_PAGE);
        lgx_attn_args a{};
        a.q = q;
        a.kpages = kpages;
        a.vpages = vpages;
        a.page_table = page_table;
        a.seq_len = seq_len;
        a.out = out;
        a.B = B;
        a.hq = hq;
        a.hkv = hkv;
        a.maxp = maxp;
        a.num_pages = num_pages;
        a.maxlen = max_seq_len;
        a.nchunk = (max_seq_len + LGX_ATTN_CHUNK - 1) / LGX_ATTN_CHUNK;
        a.scale = (float)(1.0 / std::sqrt((double)d));
        st = ensure_ws(c, (size_t)B * hq * a.nchunk * (d + 2) * sizeof(float), &a.part);
        if (st != LGX_OK) return st;
        st = launch(c, (Kern)k, dim3(a.nchunk, B * hkv), dim3(256), a, stream);
        if (st != LGX_OK) return st;
        return launch(c, d == 64 ? K_ATTN_COMBINE_D64 : K_ATTN_COMBINE_D128, dim3(B * hq), dim3(d),
                      a, stream);
    });
}

lgx_status lgx_q8_gemm(lgx_ctx* c, const lgx_q8_matrix* W, const int8_t* xq, const uint16_t* xd,
                       int32_t m, float* y, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if ((st = check_q8(W)) != LGX_OK) return st;
        if (!xq || !xd || !y) return fail(LGX_NULL_POINTER, "NULL xq, xd or y");
        if (m <= 0 || m > 65535 * 64) return fail(LGX_OUT_OF_BOUNDS, "m = %d out of range", m);
        Kern k = m <= 16 ? K_GEMM_MFMA16 : m <= 32 ? K_GEMM_MFMA32 : K_GEMM_MFMA64;
        return run_q8(c, k, W, nullptr, xq, xd, m, y, nullptr, stream);
    });
}

}  // extern "C"
