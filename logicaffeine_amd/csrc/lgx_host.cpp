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
#include <algorithm>

#include "lgx_internal.h"

using namespace lgxi;

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
        const char* env_path = getenv("LGX_HSACO");
        std::string path = hsaco_path             ? std::string(hsaco_path)
                           : env_path && *env_path ? std::string(env_path)
                                                   : default_hsaco_path();
        hipModule_t mod = nullptr;
        e = hipModuleLoad(&mod, path.c_str());
        if (e != hipSuccess)
            return fail(LGX_MODULE_LOAD_FAILED, "hipModuleLoad(%s): %s", path.c_str(),
                        hipGetErrorString(e));
        // the allocation-free entry point's scratch on this device
        void* scratch = nullptr;
        e = lgxi_scratch_ptr(device, &scratch);
        if (e != hipSuccess) {
            (void)hipModuleUnload(mod);
            return fail(LGX_HIP_ERROR, "hipGetSymbolAddress(scratch) on device %d: %s", device,
                        hipGetErrorString(e));
        }
        lgx_ctx* c = new lgx_ctx();
        c->device = device;
        c->module = mod;
        c->scratch = scratch;
        c->arch = arch;
        const char* gv = getenv("LGX_GEMV");
        c->gemv_dot4 = gv && std::string(gv) == "dot4";
        c->gemv_split = gv && std::string(gv) == "split";
        c->gemv_whole = gv && std::string(gv) == "whole";
        c->gemv_wgs = env_int("LGX_GEMV_WGS", 0);
        c->gemm_mt = env_int("LGX_GEMM_MT", 0);
        c->tiled_min = env_int("LGX_GEMM_TILED_MIN", 33);
        c->tiled_rows = env_int("LGX_GEMM_TILED_ROWS", 0);
        c->tiled_grp = env_int("LGX_GEMM_TILED_GRP", 0);
        if (c->tiled_grp != 1 && c->tiled_grp != 2 && c->tiled_grp != 4) c->tiled_grp = 0;
        c->tiled_wpc = std::max(1, env_int("LGX_GEMM_TILED_WPC", 4));
        const char* dg = getenv("LGX_DECODE_GEMM");
        c->decode_streaming = dg && std::string(dg) == "streaming";
        const char* pfv = getenv("LGX_PREFILL");
        c->prefill_serial = pfv && std::string(pfv) == "serial";
        c->prefill_chunk = env_int("LGX_PREFILL_CHUNK", 0);
        c->decode_fuse = env_int("LGX_DECODE_FUSE", 1) != 0;
        c->fuse_cols32 = env_int("LGX_FUSE_SWIGLU_COLS", 32) == 64 ? 2 : 1;
        c->merge_o_tiles = std::min(std::max(env_int("LGX_MERGE_O_TILES", 8), 1), 16);
        c->gemm_grpm = env_int("LGX_GEMM_GRPM", 1) != 0;
        c->tiled_swiglu = env_int("LGX_TILED_SWIGLU", 1) != 0;
        c->norm_waves = std::min(std::max(env_int("LGX_NORM_WAVES", 1), 0), 4);
        c->lm_cert = env_int("LGX_LM_CERT", 1) != 0;
        c->tiled_s4 = env_int("LGX_TILED_S4", 1) != 0;
        int ncu = 0;
        if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, device) ==
                hipSuccess &&
            ncu > 0)
            c->ncu = ncu;
        int lds = 0;
        if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, device) == hipSuccess &&
            lds > 0)
            c->max_lds = lds;
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
        const int live = c->live_models.load();
        if (live > 0)
            return fail(LGX_INVALID_ARGUMENT,
                        "%d lgx_model handle(s) still use this ctx: destroy them first", live);
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

static bool use_wg(const lgx_ctx* c, const lgx_q8_matrix* W) {
    return !c->gemv_dot4 && !c->gemv_split && gemv_group_ok(c, W->k);
}

lgx_status lgx_q8q8_gemv(lgx_ctx* c, const lgx_q8_matrix* W, const int8_t* xq,
                         const uint16_t* xd, float* y, int32_t* dbg, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if ((st = check_q8(W)) != LGX_OK) return st;
        if (!xq || !xd || !y) return fail(LGX_NULL_POINTER, "NULL xq, xd or y");
        // the int32 block dots come from the v_dot4 GEMV (or the whole-K
        // kernel); the grouped kernel keeps stores out of its load loop
        if (use_wg(c, W) && (!dbg || c->gemv_whole)) {
            lgx_gemv_mat m = gemv_mat(W, nullptr, xq, xd, y, 0);
            m.dbg = dbg;
            return run_gemv_group(c, &m, 1, stream);
        }
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
        if ((xq_out == nullptr) != (xd_out == nullptr))
            return fail(LGX_NULL_POINTER, "xq_out and xd_out go together");
        if (use_wg(c, W)) {
            lgx_gemv_mat m = gemv_mat(W, x, nullptr, nullptr, y, 0);
            m.xq_out = xq_out;
            m.xd_out = xd_out;
            return run_gemv_group(c, &m, 1, stream);
        }
        return run_q8(c, K_GEMV_MFMA_QX, W, x, nullptr, nullptr, 1, y, nullptr, stream, xq_out,
                      xd_out);
    });
}

lgx_status lgx_q8q8_gemv_quantize_group(lgx_ctx* c, int32_t count, const lgx_q8_matrix* W,
                                        const float* const* x, float* const* y, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!W || !x || !y) return fail(LGX_NULL_POINTER, "NULL W, x or y array");
        if (count < 1 || count > LGX_GROUP_MAX)
            return fail(LGX_OUT_OF_BOUNDS, "count = %d (1..%d)", count, LGX_GROUP_MAX);
        lgx_gemv_mat mats[LGX_GROUP_MAX];
        for (int i = 0; i < count; ++i) {
            if ((st = check_q8(&W[i])) != LGX_OK) return st;
            if (!x[i] || !y[i]) return fail(LGX_NULL_POINTER, "NULL x[%d] or y[%d]", i, i);
            if (!gemv_group_ok(c, W[i].k))
                return fail(LGX_UNSUPPORTED, "W[%d].k = %d too long for a grouped GEMV", i, W[i].k);
            mats[i] = gemv_mat(&W[i], x[i], nullptr, nullptr, y[i], 0);
        }
        // longest reductions first: their workgroups start earliest
        std::stable_sort(mats, mats + count,
                         [](const lgx_gemv_mat& a, const lgx_gemv_mat& b) { return a.k > b.k; });
        return run_gemv_group(c, mats, count, stream);
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
        if ((xq_out == nullptr) != (xd_out == nullptr))
            return fail(LGX_NULL_POINTER, "xq_out and xd_out go together");
        if (use_wg(c, W)) {
            lgx_gemv_mat m = gemv_mat(W, x, nullptr, nullptr, part, 1);
            m.xq_out = xq_out;
            m.xd_out = xd_out;
            return run_gemv_group(c, &m, 1, stream);
        }
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
        if (m == 1 && use_wg(c, W)) {
            lgx_gemv_mat g = gemv_mat(W, nullptr, xq, xd, part, 1);
            return run_gemv_group(c, &g, 1, stream);
        }
        Kern k = m == 1 ? K_GEMV_MFMA : gemm_kernel(c, m);
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

lgx_status lgx_gqa_prefill_attn(lgx_ctx* c, const float* q, const uint16_t* kpages,
                                const uint16_t* vpages, const int32_t* page_table,
                                const int32_t* seq_len, int32_t B, int32_t P, int32_t hq,
                                int32_t hkv, int32_t d, int32_t maxp, int32_t num_pages,
                                int32_t max_seq_len, float* out, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!q || !kpages || !vpages || !page_table || !seq_len || !out)
            return fail(LGX_NULL_POINTER, "NULL tensor pointer");
        if (B <= 0 || P <= 0 || hq <= 0 || hkv <= 0 || hq % hkv != 0 || maxp <= 0 || num_pages <= 0)
            return fail(LGX_INVALID_ARGUMENT, "B=%d P=%d hq=%d hkv=%d maxp=%d num_pages=%d", B, P, hq,
                        hkv, maxp, num_pages);
        if ((d != 64 && d != 128) || prefill_attn_kernel(d, hq / hkv) < 0)
            return fail(LGX_UNSUPPORTED, "head_dim %d / %d query heads per KV head", d, hq / hkv);
        if (max_seq_len <= 0 || max_seq_len > maxp * LGX_PAGE)
            return fail(LGX_OUT_OF_BOUNDS, "max_seq_len %d outside (0, %d]", max_seq_len,
                        maxp * LGX_PAGE);
        if ((int64_t)B * P * hq > INT32_MAX) return fail(LGX_OUT_OF_BOUNDS, "B*P*hq too large");
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
        a.ncg = a.nchunk;
        a.len_add = 1;
        a.qpr = P;
        a.scale = (float)(1.0 / std::sqrt((double)d));
        st = ensure_ws(c, (size_t)B * P * hq * a.nchunk * (d + 2) * sizeof(float), &a.part);
        if (st != LGX_OK) return st;
        if ((st = launch_prefill_attn(c, a, d, stream)) != LGX_OK) return st;
        return launch(c, d == 64 ? K_ATTN_COMBINE_D64 : K_ATTN_COMBINE_D128, dim3(B * P * hq), dim3(d),
                      a, stream);
    });
}

lgx_status lgx_gqa_prefill_attn_fast(lgx_ctx* c, const float* q, const uint16_t* kpages,
                                     const uint16_t* vpages, const int32_t* page_table,
                                     const int32_t* seq_len, int32_t B, int32_t P, int32_t hq,
                                     int32_t hkv, int32_t d, int32_t maxp, int32_t num_pages,
                                     int32_t max_seq_len, float* out, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!q || !kpages || !vpages || !page_table || !seq_len || !out)
            return fail(LGX_NULL_POINTER, "NULL tensor pointer");
        if (B <= 0 || P <= 0 || hq <= 0 || hkv <= 0 || hq % hkv != 0 || maxp <= 0 || num_pages <= 0)
            return fail(LGX_INVALID_ARGUMENT, "B=%d P=%d hq=%d hkv=%d maxp=%d num_pages=%d", B, P, hq,
                        hkv, maxp, num_pages);
        if ((d != 64 && d != 128) || hq / hkv > 8)
            return fail(LGX_UNSUPPORTED, "head_dim %d / %d query heads per KV head", d, hq / hkv);
        if (max_seq_len <= 0 || max_seq_len > maxp * LGX_PAGE)
            return fail(LGX_OUT_OF_BOUNDS, "max_seq_len %d outside (0, %d]", max_seq_len,
                        maxp * LGX_PAGE);
        if ((int64_t)B * P * hq > INT32_MAX) return fail(LGX_OUT_OF_BOUNDS, "B*P*hq too large");
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
        a.len_add = 1;
        a.qpr = P;
        a.scale = (float)(1.0 / std::sqrt((double)d));
        return launch_prefill_attn_fast(c, a, d, stream);
    });
}

// lgx_q8_gemm over the workspace `scratch` of `cap` bytes (nullptr: the
// ctx's grow-on-demand workspace).
static lgx_status q8_gemm_impl(lgx_ctx* c, const lgx_q8_matrix* W, const int8_t* xq,
                               const uint16_t* xd, int32_t m, float* y, void* stream,
                               void* scratch, size_t cap) {
    lgx_status st = enter(c);
    if (st != LGX_OK) return st;
    if ((st = check_q8(W)) != LGX_OK) return st;
    if (!xq || !xd || !y) return fail(LGX_NULL_POINTER, "NULL xq, xd or y");
    if (m <= 0 || m > 65535 * 64) return fail(LGX_OUT_OF_BOUNDS, "m = %d out of range", m);
    if (m == 1 && use_wg(c, W)) {
        // the grouped GEMV applies the range tree in LDS: no workspace
        lgx_gemv_mat g = gemv_mat(W, nullptr, xq, xd, y, 0);
        return run_gemv_group(c, &g, 1, stream);
    }
    auto room = [&](size_t bytes, float** out) -> lgx_status {
        if (!scratch) return ensure_ws(c, bytes, out);
        if (bytes > cap)
            return fail(LGX_OUT_OF_BOUNDS,
                        "[%d x %d] product over m = %d needs %zu scratch bytes (limit %zu)", W->n,
                        W->k, m, bytes, cap);
        *out = (float*)scratch;
        return LGX_OK;
    };
    if (m >= c->tiled_min) {
        // T16 copy of the activations, then the group partials (straight
        // into y when K is one group) and the tree over the groups
        const Kern kern = tiled_kernel(c, m);
        const int grp = tiled_grp(c, kern, W->n, W->k, m);
        const int ng = tiled_groups(W->k, grp);
        const size_t xbytes = ((size_t)cdiv(m, 16) * 16 * W->k + 255) / 256 * 256;
        float* ws = nullptr;
        if ((st = room(xbytes + (ng > 1 ? (size_t)ng * m * W->n * 4 : 0), &ws)) != LGX_OK)
            return st;
        int8_t* xt = (int8_t*)ws;
        float* part = ng > 1 ? (float*)((char*)ws + xbytes) : y;
        if ((st = act_to_t16(c, xq, m, W->k, xt, stream)) != LGX_OK ||
            (st = run_q8_tiled(c, W, xt, xd, m, part, stream, kern, grp)) != LGX_OK || ng == 1)
            return st;
        lgx_combine_args ca{part, y, (int64_t)m * W->n, ng};
        return launch(c, K_COMBINE, dim3(cdiv(ca.count, 256)), dim3(256), ca, stream);
    }
    const int nr = nranges_of(W->k);
    float* part = nullptr;
    if (nr > 1 && (st = room((size_t)nr * m * W->n * sizeof(float), &part)) != LGX_OK) return st;
    return run_q8(c, gemm_kernel(c, m), W, nullptr, xq, xd, m, y, nullptr, stream, nullptr, nullptr,
                  nullptr, part);
}

lgx_status lgx_q8_gemm_quantize_group(lgx_ctx* c, int32_t count, const lgx_q8_matrix* W,
                                      const float* const* x, int32_t m, float* const* y,
                                      void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!W || !x || !y) return fail(LGX_NULL_POINTER, "NULL W, x or y array");
        if (count < 1 || count > LGX_MGROUP_MAX)
            return fail(LGX_OUT_OF_BOUNDS, "count = %d (1..%d)", count, LGX_MGROUP_MAX);
        if (m <= 0 || m > 65535 * 64) return fail(LGX_OUT_OF_BOUNDS, "m = %d out of range", m);
        for (int i = 0; i < count; ++i) {
            if ((st = check_q8(&W[i])) != LGX_OK) return st;
            if (!x[i] || !y[i]) return fail(LGX_NULL_POINTER, "NULL x[%d] or y[%d]", i, i);
        }
        if (m == 1) {
            lgx_gemv_mat mats[LGX_GROUP_MAX];
            for (int i = 0; i < count; ++i) {
                if (!gemv_group_ok(c, W[i].k))
                    return fail(LGX_UNSUPPORTED, "W[%d].k = %d too long for a grouped GEMV", i,
                                W[i].k);
                mats[i] = gemv_mat(&W[i], x[i], nullptr, nullptr, y[i], 0);
            }
            std::stable_sort(mats, mats + count, [](const lgx_gemv_mat& a, const lgx_gemv_mat& b) {
                return a.k > b.k;
            });
            return run_gemv_group(c, mats, count, stream);
        }
        {
            // 2..8 rows: one launch (quantisation, products, trees)
            lgx_gemv_mat mats[LGX_GROUP_MAX];
            for (int i = 0; i < count && count <= LGX_GROUP_MAX; ++i)
                mats[i] = gemv_mat(&W[i], x[i], nullptr, nullptr, y[i], 0);
            if (count <= LGX_GROUP_MAX && gemm_grpm_ok(c, mats, count, m)) {
                std::stable_sort(mats, mats + count,
                                 [](const lgx_gemv_mat& a, const lgx_gemv_mat& b) { return a.k > b.k; });
                return run_gemm_grpm(c, mats, count, m, stream);
            }
        }
        // the tiled product from 17 rows (config 1 at M = 32: 28.9 us against
        // 35.4 us per step on the 16-row streaming kernels)
        const bool tiled = m >= std::min(c->tiled_min, 17);
        const Kern tk = tiled_kernel(c, m);
        const int trows = tk == K_GEMM_TILED ? 128 : tk == K_GEMM_TILED64 ? 64 : 32;
        // ranges per group of the tiled products: 2, or 1 when that leaves
        // fewer than two workgroups per compute unit over all the matrices
        // together.  Groups of 4 make the long-K matrix's workgroups the
        // launch's tail (config 1 at M = 64: 41 us against 32 us per step)
        int grp = 1;
        if (tiled) {
            if (c->tiled_grp) {
                grp = c->tiled_grp;
            } else {
                for (grp = 2; grp > 1; grp >>= 1) {
                    int64_t wgs = 0;
                    for (int i = 0; i < count; ++i)
                        wgs += (int64_t)cdiv(W[i].n, LGX_TG_N) * cdiv(m, trows) * tiled_groups(W[i].k, grp);
                    if (wgs >= 2LL * c->ncu) break;
                }
            }
        }
        // workspace: per matrix the Q8_0 activations (T16 tiles padded to 16
        // rows on the tiled path), their scales, and partials when there are
        // several ranges / groups; 256-byte aligned pieces
        auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
        size_t xq_b[LGX_MGROUP_MAX], xd_b[LGX_MGROUP_MAX], pt_b[LGX_MGROUP_MAX];
        int nparts[LGX_MGROUP_MAX];
        size_t total = 0;
        for (int i = 0; i < count; ++i) {
            const int k = W[i].k, n = W[i].n;
            xq_b[i] = al((size_t)(tiled ? cdiv(m, 16) * 16 : m) * k);
            xd_b[i] = al((size_t)m * (k / 32) * 2);
            nparts[i] = tiled ? tiled_groups(k, grp) : nranges_of(k);
            pt_b[i] = nparts[i] > 1 ? al((size_t)nparts[i] * m * n * sizeof(float)) : 0;
            total += xq_b[i] + xd_b[i] + pt_b[i];
        }
        float* ws = nullptr;
        if ((st = ensure_ws(c, total, &ws)) != LGX_OK) return st;
        char* wp = (char*)ws;
        int8_t* xq[LGX_MGROUP_MAX];
        uint16_t* xd[LGX_MGROUP_MAX];
        float* part[LGX_MGROUP_MAX];
        for (int i = 0; i < count; ++i) {
            xq[i] = (int8_t*)wp;
            wp += xq_b[i];
            xd[i] = (uint16_t*)wp;
            wp += xd_b[i];
            part[i] = pt_b[i] ? (float*)wp : y[i];
            wp += pt_b[i];
        }
        // 1. Q8_0 of every activation matrix
        lgx_quant_group_args qa{};
        qa.m = m;
        qa.count = count;
        qa.t16 = tiled ? 1 : 0;
        qa.blk0[0] = 0;
        for (int i = 0; i < count; ++i) {
            qa.x[i] = x[i];
            qa.xq[i] = xq[i];
            qa.xd[i] = xd[i];
            qa.k[i] = W[i].k;
            qa.blk0[i + 1] = qa.blk0[i] + (int64_t)m * (W[i].k / 32);
        }
        if ((st = launch(c, K_QUANT_GROUP, dim3(cdiv(qa.blk0[count] * 8, 256)), dim3(256), qa,
                         stream)) != LGX_OK)
            return st;
        // 2. the products
        if (tiled) {
            lgx_tiled_group_args ta{};
            ta.count = count;
            ta.wg0[0] = 0;
            for (int i = 0; i < count; ++i) {
                lgx_gemm_tiled_args& a = ta.mat[i];
                a.wt = W[i].qs;
                a.wd = W[i].d;
                a.xt = xq[i];
                a.xd = xd[i];
                a.part = part[i];
                a.n = W[i].n;
                a.k = W[i].k;
                a.m = m;
                a.grp = grp;
                a.ngroups = tiled_groups(W[i].k, grp);
                a.ntn = (int)cdiv(W[i].n, LGX_TG_N);
                a.ntm = (int)cdiv(m, trows);
                const int64_t wgs = (int64_t)a.ntn * a.ntm * a.ngroups;
                const int64_t end = ta.wg0[i] + (wgs + 7) / 8 * 8;
                if (end > INT32_MAX) return fail(LGX_OUT_OF_BOUNDS, "grouped product too large");
                ta.wg0[i + 1] = (int32_t)end;
            }
            const Kern gk = tk == K_GEMM_TILED   ? K_GEMM_TILED_GROUP
                            : tk == K_GEMM_TILED64 ? K_GEMM_TILED64_GROUP
                                                   : K_GEMM_TILED32_GROUP;
            if ((st = launch(c, gk, dim3(ta.wg0[count]), dim3(256), ta, stream)) != LGX_OK) return st;
        } else {
            // 16-row m-groups (several workgroups per weight tile, the
            // later reads from L2); 17 rows and more take the tiled path
            const int mrows = 16;
            lgx_stream_group_args sa{};
            sa.count = count;
            sa.wg0[0] = 0;
            for (int i = 0; i < count; ++i) {
                lgx_gemv_args& a = sa.mat[i];
                a.wt = W[i].qs;
                a.wd = W[i].d;
                a.xq = xq[i];
                a.xd = xd[i];
                a.y = y[i];
                a.part = part[i];
                a.n = W[i].n;
                a.k = W[i].k;
                a.m = m;
                a.ntiles = W[i].n / 16;
                a.nranges = nranges_of(W[i].k);
                a.nmgroups = (int)cdiv(m, mrows);
                const int64_t tasks = (int64_t)a.ntiles * a.nranges * a.nmgroups;
                const int64_t tpw = (tasks + 4LL * c->wg_target - 1) / (4LL * c->wg_target);
                a.tpw = (int)(tpw < 1 ? 1 : tpw > 64 ? 64 : tpw);
                sa.gx[i] = (int)(cdiv(a.ntiles, 4LL * a.tpw) * a.nmgroups);
                const int64_t end = sa.wg0[i] + (int64_t)sa.gx[i] * a.nranges;
                if (end > INT32_MAX) return fail(LGX_OUT_OF_BOUNDS, "grouped product too large");
                sa.wg0[i + 1] = (int32_t)end;
            }
            if ((st = launch(c, K_GEMM_MFMA16_GROUP,
                             dim3(sa.wg0[count]), dim3(256), sa, stream)) != LGX_OK)
                return st;
        }
        // 3. the trees of the products with several ranges / groups
        lgx_combine_group_args ca{};
        int nc = 0;
        ca.el0[0] = 0;
        for (int i = 0; i < count; ++i) {
            if (nparts[i] <= 1) continue;
            ca.part[nc] = part[i];
            ca.y[nc] = y[i];
            ca.nr[nc] = nparts[i];
            ca.el0[nc + 1] = ca.el0[nc] + (int64_t)m * W[i].n;
            ++nc;
        }
        ca.count = nc;
        if (nc == 0) return LGX_OK;
        return launch(c, K_COMBINE_GROUP, dim3(cdiv(ca.el0[nc], 256)), dim3(256), ca, stream);
    });
}

lgx_status lgx_q8_gemm(lgx_ctx* c, const lgx_q8_matrix* W, const int8_t* xq, const uint16_t* xd,
                       int32_t m, float* y, void* stream) {
    return guarded(__func__, [&] { return q8_gemm_impl(c, W, xq, xd, m, y, stream, nullptr, 0); });
}

lgx_status lgx_q8_gemm_noalloc(lgx_ctx* c, const lgx_q8_matrix* W, const int8_t* xq,
                               const uint16_t* xd, int32_t m, float* y, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        if (!valid_ctx(c)) return fail(LGX_INVALID_HANDLE, "invalid lgx_ctx handle");
        if (!c->scratch) return fail(LGX_HIP_ERROR, "no device scratch on device %d", c->device);
        struct Untimed {
            Untimed() { g_untimed = true; }
            ~Untimed() { g_untimed = false; }
        } untimed;
        return q8_gemm_impl(c, W, xq, xd, m, y, stream, c->scratch, LGX_NOALLOC_SCRATCH_BYTES);
    });
}

}  // extern "C"
