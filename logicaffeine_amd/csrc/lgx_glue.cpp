// lgx_glue.cpp -- standalone entry points of the decode-step glue kernels
// (embedding gather, RMSNorm + Q8_0, RoPE + paged KV append, SwiGLU + Q8_0,
// binary16 lm_head, argmax).  The decode step in lgx_model.cpp launches the
// same kernels with range partials as inputs; here every input is a plain
// binary32 tensor (one range), which is how a caller outside the model uses
// them and how the tests compare each one with the CPU oracle.
#include <algorithm>
#include <cmath>

#include "lgx_internal.h"

using namespace lgxi;

namespace {
constexpr int kNormMax = 8192, kQkvMax = 8192, kLmMaxH = 8192, kLmMaxM = 64;
}

extern "C" {

lgx_status lgx_embed_f16(lgx_ctx* c, const uint16_t* emb, const int32_t* tokens, int32_t m,
                         int32_t h, int32_t vocab, float* out, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!emb || !tokens || !out) return fail(LGX_NULL_POINTER, "NULL tensor");
        if (m <= 0 || h <= 0 || vocab <= 0)
            return fail(LGX_INVALID_ARGUMENT, "m %d, h %d, vocab %d", m, h, vocab);
        lgx_embed_args a{emb, tokens, out, m, h, vocab, 1, 1};
        return launch(c, K_EMBED, dim3(m), dim3(256), a, stream);
    });
}

lgx_status lgx_rmsnorm_quant(lgx_ctx* c, const float* x, const float* w, int32_t m, int32_t n,
                             float eps, float* y, int8_t* xq, uint16_t* xd, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!x || !w) return fail(LGX_NULL_POINTER, "NULL x or w");
        if (!y && !xq) return fail(LGX_NULL_POINTER, "no output (y and xq are NULL)");
        if ((xq == nullptr) != (xd == nullptr)) return fail(LGX_NULL_POINTER, "xq and xd go together");
        if (m <= 0 || n <= 0 || n > kNormMax)
            return fail(LGX_INVALID_ARGUMENT, "m %d, n %d (n <= %d)", m, n, kNormMax);
        if (xq && n % 32) return fail(LGX_INVALID_ARGUMENT, "Q8_0 output needs n %% 32 == 0");
        lgx_norm_args a{};
        a.part = nullptr;
        a.nr = 1;
        a.h = const_cast<float*>(x);   // read only when part is NULL
        a.w = w;
        a.xn = y;
        a.xq = xq;
        a.xd = xd;
        a.m = m;
        a.n = n;
        a.eps = eps;
        return launch_norm(c, a, stream);
    });
}

lgx_status lgx_add_rmsnorm_quant(lgx_ctx* c, const float* part, int32_t nr, float* h,
                                 const float* w, int32_t m, int32_t n, float eps, float* y,
                                 int8_t* xq, uint16_t* xd, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!part || !h || !w) return fail(LGX_NULL_POINTER, "NULL part, h or w");
        if (!y && !xq) return fail(LGX_NULL_POINTER, "no output (y and xq are NULL)");
        if ((xq == nullptr) != (xd == nullptr)) return fail(LGX_NULL_POINTER, "xq and xd go together");
        if (m <= 0 || n <= 0 || n > kNormMax)
            return fail(LGX_INVALID_ARGUMENT, "m %d, n %d (n <= %d)", m, n, kNormMax);
        if (nr <= 0 || nr > LGX_MAX_RANGES)
            return fail(LGX_INVALID_ARGUMENT, "nr %d outside [1, %d]", nr, LGX_MAX_RANGES);
        if (xq && n % 32) return fail(LGX_INVALID_ARGUMENT, "Q8_0 output needs n %% 32 == 0");
        lgx_norm_args a{};
        a.part = part;
        a.nr = nr;
        a.h = h;
        a.w = w;
        a.xn = y;
        a.xq = xq;
        a.xd = xd;
        a.m = m;
        a.n = n;
        a.eps = eps;
        return launch_norm(c, a, stream);
    });
}

lgx_status lgx_rope_kv_append(lgx_ctx* c, const float* qkv, const float* bias, const float* cos_t,
                              const float* sin_t, const int32_t* seq_len,
                              const int32_t* page_table, uint16_t* kpages, uint16_t* vpages,
                              float* q_out, int32_t B, int32_t hq, int32_t hkv, int32_t d,
                              int32_t maxp, int32_t num_pages, int32_t max_seq, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!qkv || !cos_t || !sin_t || !seq_len || !page_table || !kpages || !vpages || !q_out)
            return fail(LGX_NULL_POINTER, "NULL tensor");
        if (B <= 0 || hq <= 0 || hkv <= 0 || d <= 0 || d % 2 || maxp <= 0 || num_pages <= 0 ||
            max_seq <= 0)
            return fail(LGX_INVALID_ARGUMENT, "B %d hq %d hkv %d d %d maxp %d pages %d max_seq %d",
                        B, hq, hkv, d, maxp, num_pages, max_seq);
        if ((int64_t)(hq + 2 * hkv) * d > kQkvMax)
            return fail(LGX_UNSUPPORTED, "(hq + 2 hkv) d = %d > %d", (hq + 2 * hkv) * d, kQkvMax);
        if ((int64_t)maxp * LGX_PAGE < max_seq)
            return fail(LGX_OUT_OF_BOUNDS, "max_seq %d exceeds maxp * 16 = %d", max_seq,
                        maxp * LGX_PAGE);
        lgx_qkv_args a{};
        a.part = qkv;
        a.nr = 1;
        a.bias = bias;
        a.cos_t = cos_t;
        a.sin_t = sin_t;
        a.seq_len = seq_len;
        a.page_table = page_table;
        a.kpages = kpages;
        a.vpages = vpages;
        a.q_out = q_out;
        a.m = B;
        a.hq = hq;
        a.hkv = hkv;
        a.d = d;
        a.maxp = maxp;
        a.num_pages = num_pages;
        a.max_seq = max_seq;
        return launch_qkv_rope(c, a, B, stream);
    });
}

lgx_status lgx_swiglu_quant(lgx_ctx* c, const float* gu, int32_t m, int32_t inter, float* y,
                            int8_t* xq, uint16_t* xd, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!gu) return fail(LGX_NULL_POINTER, "NULL gate|up");
        if (!y && !xq) return fail(LGX_NULL_POINTER, "no output (y and xq are NULL)");
        if ((xq == nullptr) != (xd == nullptr)) return fail(LGX_NULL_POINTER, "xq and xd go together");
        if (m <= 0 || inter <= 0 || inter % 32)
            return fail(LGX_INVALID_ARGUMENT, "m %d, inter %d (multiple of 32)", m, inter);
        lgx_swiglu_args a{gu, 1, xq, xd, y, m, inter, 0};
        return launch(c, K_SWIGLU_QUANT, dim3(m, cdiv(inter / 32, 32)), dim3(256), a, stream);
    });
}

lgx_status lgx_lm_head_f16(lgx_ctx* c, const float* x, const uint16_t* emb, int32_t m, int32_t h,
                           int32_t vocab, float* logits, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!x || !emb || !logits) return fail(LGX_NULL_POINTER, "NULL tensor");
        if (m <= 0 || vocab <= 0 || h <= 0 || h % 64 || h > kLmMaxH)
            return fail(LGX_UNSUPPORTED, "m %d, vocab %d, h %d (h %% 64 == 0, h <= %d)", m, vocab,
                        h, kLmMaxH);
        // one chain per 1024-column range; more than one range: the range
        // partials in the workspace, then the pairwise tree into logits
        const int nr = (h + 1023) / 1024;
        for (int r0 = 0; r0 < m; r0 += kLmMaxM) {
            const int mm = std::min(kLmMaxM, m - r0);
            float* out = logits + (int64_t)r0 * vocab;
            float* part = out;
            if (nr > 1 && (st = ensure_ws(c, (size_t)nr * mm * vocab * sizeof(float), &part)) != LGX_OK)
                return st;
            lgx_lmhead_args a{x + (int64_t)r0 * h, emb, part, mm, h, vocab};
            if ((st = launch(c, K_LM_HEAD_F16, dim3(cdiv(vocab, 256), nr), dim3(256), a, stream)) !=
                LGX_OK)
                return st;
            if (nr > 1) {
                lgx_combine_args ca{part, out, (int64_t)mm * vocab, nr};
                if ((st = launch(c, K_COMBINE, dim3(cdiv(ca.count, 256)), dim3(256), ca, stream)) != LGX_OK)
                    return st;
            }
        }
        return LGX_OK;
    });
}

int64_t lgx_f16_t64_count(int32_t rows, int32_t h) {
    if (rows <= 0 || h <= 0) return 0;
    return (int64_t)((rows + 63) / 64) * 64 * h;
}

lgx_status lgx_f16_repack_t64(lgx_ctx* c, const uint16_t* src, int32_t rows, int32_t h,
                              uint16_t* dst, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!src || !dst) return fail(LGX_NULL_POINTER, "NULL src or dst");
        if (rows <= 0 || h <= 0 || h % 8)
            return fail(LGX_INVALID_ARGUMENT, "rows %d, h %d (h %% 8 == 0)", rows, h);
        lgx_t64_args a{src, dst, rows, h};
        return launch(c, K_REPACK_F16_T64, dim3(cdiv(lgx_f16_t64_count(rows, h) / 8, 256)),
                      dim3(256), a, stream);
    });
}

lgx_status lgx_lm_head_f16_t64(lgx_ctx* c, const float* x, const uint16_t* emb_t64, int32_t m,
                               int32_t h, int32_t vocab, float* logits, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!x || !emb_t64 || !logits) return fail(LGX_NULL_POINTER, "NULL tensor");
        if (m <= 0 || m > kLmMaxM || vocab <= 0 || h <= 0 || h % 64 || h > kLmMaxH)
            return fail(LGX_UNSUPPORTED, "m %d (<= %d), vocab %d, h %d (h %% 64 == 0, h <= %d)",
                        m, kLmMaxM, vocab, h, kLmMaxH);
        // the activation in T16 column order in the workspace, followed there
        // by the range partials when h holds more than one 1024-column range
        const int mc = (m + 15) / 16, nr = (h + 1023) / 1024;
        const size_t nxt = (size_t)mc * 16 * h;
        float* xt = nullptr;
        if ((st = ensure_ws(c, (nxt + (nr > 1 ? (size_t)nr * m * vocab : 0)) * sizeof(float), &xt)) !=
            LGX_OK)
            return st;
        lgx_t64_args ta{x, xt, m, h};
        if ((st = launch(c, K_ROWS_TO_T16, dim3(cdiv((int64_t)m * h, 256)), dim3(256), ta,
                         stream)) != LGX_OK)
            return st;
        float* part = nr > 1 ? xt + nxt : logits;
        lgx_lmhead_args a{xt, emb_t64, part, m, h, vocab};
        if ((st = launch(c, K_LM_HEAD_T64, dim3(cdiv(vocab, 64), mc, nr), dim3(64), a, stream)) != LGX_OK)
            return st;
        if (nr == 1) return LGX_OK;
        lgx_combine_args ca{part, logits, (int64_t)m * vocab, nr};
        return launch(c, K_COMBINE, dim3(cdiv(ca.count, 256)), dim3(256), ca, stream);
    });
}

lgx_status lgx_argmax(lgx_ctx* c, const float* logits, int32_t m, int32_t vocab, int32_t* out,
                      void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!logits || !out) return fail(LGX_NULL_POINTER, "NULL tensor");
        if (m <= 0 || vocab <= 0) return fail(LGX_INVALID_ARGUMENT, "m %d, vocab %d", m, vocab);
        float* cand = nullptr;
        if ((st = ensure_ws(c, (size_t)m * argmax_slices(vocab) * 8, &cand)) != LGX_OK) return st;
        return launch_argmax(c, logits, 1, m, vocab, out, nullptr, 0, cand, stream);
    });
}

lgx_status lgx_lm_head_rowconst(lgx_ctx* c, const uint16_t* emb, int32_t vocab, int32_t h,
                                float* rowc, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!emb || !rowc) return fail(LGX_NULL_POINTER, "NULL tensor");
        if (vocab <= 0 || h <= 0 || h > LGX_LMC_MAXH)
            return fail(LGX_INVALID_ARGUMENT, "vocab %d, h %d (h <= %d)", vocab, h, LGX_LMC_MAXH);
        return launch_lm_rowconst(c, emb, vocab, h, rowc, stream);
    });
}

lgx_status lgx_lm_head_argmax_f16(lgx_ctx* c, const float* x, const uint16_t* emb,
                                  const uint16_t* emb_t64, const float* rowc, int32_t m,
                                  int32_t h, int32_t vocab, int32_t* out, float* bounds,
                                  void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!x || !emb || !emb_t64 || !rowc || !out) return fail(LGX_NULL_POINTER, "NULL tensor");
        if (m <= 0 || m > LGX_LMC_MAXB || vocab <= 0 || h <= 0 || h % 64 || h > LGX_LMC_MAXH ||
            lm_cert_slices(vocab) > 1024)
            return fail(LGX_UNSUPPORTED, "m %d (<= %d), vocab %d (<= 655360), h %d (h %% 64 == 0, h <= %d)",
                        m, LGX_LMC_MAXB, vocab, h, LGX_LMC_MAXH);
        float* ws = nullptr;
        if ((st = ensure_ws(c, (size_t)m * lm_cert_slices(vocab) * sizeof(lgx_lmc_summary), &ws)) !=
            LGX_OK)
            return st;
        return launch_lm_cert(c, x, emb, emb_t64, rowc, m, h, vocab, (lgx_lmc_summary*)ws, bounds,
                              out, nullptr, 0, stream);
    });
}

lgx_status lgx_sample(lgx_ctx* c, const float* logits, int32_t m, int32_t vocab, int32_t top_k,
                      float top_p, float temperature, uint64_t seed, const int32_t* positions,
                      int32_t* out, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!logits || !positions || !out) return fail(LGX_NULL_POINTER, "NULL tensor");
        if (m <= 0 || m > 65535) return fail(LGX_INVALID_ARGUMENT, "m = %d", m);
        SampleParams sp;
        if ((st = sample_check(top_k, top_p, temperature, vocab, &sp)) != LGX_OK) return st;
        sp.seed = seed;
        float* cand = nullptr;
        if ((st = ensure_ws(c, sample_cand_bytes(m, vocab), &cand)) != LGX_OK) return st;
        return launch_sample(c, sp, logits, 1, m, vocab, positions, out, nullptr, 0, cand, stream);
    });
}

}  // extern "C"
