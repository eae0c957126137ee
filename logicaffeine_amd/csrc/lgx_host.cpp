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
#include <cstring>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>

#include "../../include/lgx.h"
#include "lgx_kargs.h"

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
    K_Q8_GEMM,
    K_COUNT
};
const char* const kKernelNames[K_COUNT] = {
    "lgx_k_repack_t16", "lgx_k_quantize_q8_0", "lgx_k_q8q8_gemv",
    "lgx_k_q8_gemv_f32", "lgx_k_q8_gemm_mfma",
};

}  // namespace

struct lgx_ctx {
    uint32_t magic = 0x4c47584bu;  // "LGXK"
    int device = 0;
    hipModule_t module = nullptr;
    hipFunction_t fn[K_COUNT] = {};
    std::string arch;
    std::atomic<uint64_t> launches{0};
    void* ws = nullptr;
    size_t ws_bytes = 0;
    std::mutex ws_mu;
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

template <class Args>
lgx_status launch(lgx_ctx* c, Kern k, dim3 grid, dim3 block, const Args& args, void* stream) {
    void* params[] = {(void*)&args};
    hipError_t e = hipModuleLaunchKernel(c->fn[k], grid.x, grid.y, grid.z, block.x, block.y,
                                         block.z, 0, (hipStream_t)stream, params, nullptr);
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

// Workspace for range partials and arrival counters; grown on demand.  A new
// buffer is zero-filled once (the kernels leave every counter at zero when
// they finish).  hipFree of the old buffer waits for the device, so work still
// using it has finished.
lgx_status ensure_ws(lgx_ctx* c, size_t bytes, void** out) {
    std::lock_guard<std::mutex> lk(c->ws_mu);
    if (bytes > c->ws_bytes) {
        size_t nb = bytes < (size_t)1 << 20 ? (size_t)1 << 20 : bytes + bytes / 2;
        if (c->ws) LGX_HIP(hipFree(c->ws));
        c->ws = nullptr;
        c->ws_bytes = 0;
        hipError_t e = hipMalloc(&c->ws, nb);
        if (e != hipSuccess)
            return fail(LGX_OUT_OF_MEMORY, "workspace of %zu bytes: %s", nb, hipGetErrorString(e));
        LGX_HIP(hipMemset(c->ws, 0, nb));
        LGX_HIP(hipDeviceSynchronize());
        c->ws_bytes = nb;
    }
    *out = c->ws;
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

// Shared driver of the three GEMV/GEMM kernels.
lgx_status run_q8(lgx_ctx* c, Kern kern, const lgx_q8_matrix* W, const float* xf,
                  const int8_t* xq, const uint16_t* xd, int m, float* y, int32_t* dbg,
                  void* stream) {
    lgx_gemv_args a{};
    a.wt = W->qs;
    a.wd = W->d;
    a.xf = xf;
    a.xq = xq;
    a.xd = xd;
    a.y = y;
    a.dbg = dbg;
    a.n = W->n;
    a.k = W->k;
    a.m = m;
    a.ntiles = W->n / 16;
    a.nranges = nranges_of(W->k);
    a.nmgroups = (m + 63) / 64;
    if (a.nranges > 1) {
        // [counters: ntiles * nmgroups int32, padded to 256 B][partials]
        size_t cnt_bytes = ((size_t)a.ntiles * a.nmgroups * sizeof(int32_t) + 255) & ~(size_t)255;
        void* ws = nullptr;
        lgx_status st =
            ensure_ws(c, cnt_bytes + (size_t)a.nranges * m * W->n * sizeof(float), &ws);
        if (st != LGX_OK) return st;
        a.counter = (int32_t*)ws;
        a.part = (float*)((char*)ws + cnt_bytes);
    }
    dim3 grid(cdiv(a.ntiles, 4), a.nranges, kern == K_Q8_GEMM ? a.nmgroups : 1);
    return launch(c, kern, grid, dim3(256), a, stream);
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

static lgx_status repack_impl(lgx_ctx* c, const int8_t* src, int32_t n, int32_t k, int8_t* dst,
                              int to_t16, void* stream) {
    lgx_status st = enter(c);
    if (st != LGX_OK) return st;
    if (!src || !dst) return fail(LGX_NULL_POINTER, "NULL quants pointer");
    if (n <= 0 || k <= 0 || n % 16 != 0 || k % 64 != 0)
        return fail(LGX_INVALID_ARGUMENT, "shape [%d x %d]: need n %% 16 == 0, k %% 64 == 0", n, k);
    lgx_repack_args a{src, dst, n, k, to_t16};
    int64_t total = (int64_t)(n / 16) * (k / 64) * 64;
    return launch(c, K_REPACK, dim3(cdiv(total, 256)), dim3(256), a, stream);
}

lgx_status lgx_q8_repack_t16(lgx_ctx* c, const int8_t* qs, int32_t n, int32_t k, int8_t* out,
                             void* stream) {
    return guarded(__func__, [&] { return repack_impl(c, qs, n, k, out, 1, stream); });
}

lgx_status lgx_q8_unpack_t16(lgx_ctx* c, const int8_t* t16, int32_t n, int32_t k, int8_t* out,
                             void* stream) {
    return guarded(__func__, [&] { return repack_impl(c, t16, n, k, out, 0, stream); });
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
        return run_q8(c, K_Q8Q8_GEMV, W, nullptr, xq, xd, 1, y, dbg, stream);
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
        return run_q8(c, K_Q8_GEMM, W, nullptr, xq, xd, m, y, nullptr, stream);
    });
}

}  // extern "C"
