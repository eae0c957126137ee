// lgx_model.cpp -- the random-init Qwen2-shaped Q8_0 model on one device:
// creation from a seed, the batched greedy decode step and the teacher-forced
// prefill.  One decode step is a chain of stream-ordered launches that never
// returns to the host:
//
//   embed(tokens) -> h
//   per layer:  norm+Q8(h [+= down partials of the previous layer])
//               -> QKV product (range partials) -> tree+bias+RoPE+KV append
//               -> attention chunks -> chunk merge+Q8
//               -> O product -> h += tree, norm+Q8
//               -> gate|up product -> tree+SwiGLU+Q8 -> down product
//   final norm (+Q8) -> lm_head (fp16 tied: exact chain; Q8 untied: product)
//   -> argmax over the vocabulary, tokens <- next, seq_len += 1
//
// Every product writes its canonical range partials and the consumer applies
// the tree, so the step has no combine launches and every value is the one
// the CPU oracle computes.  The reference has no model runtime; the seam it
// would bind is the extern "C" surface in include/lgx.h.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "lgx_gen.h"
#include "lgx_gguf.h"
#include "lgx_internal.h"

using namespace lgxi;

namespace {
constexpr uint32_t kModelMagic = 0x4c47584du;  // "LGXM"

struct DevQ8 {
    int8_t* qs = nullptr;
    uint16_t* d = nullptr;
    lgx_q8_matrix m{};
};
}  // namespace

struct lgx_model {
    uint32_t magic = kModelMagic;
    lgx_ctx* ctx = nullptr;
    lgx_qwen_config c{};
    uint64_t seed = 0;
    int32_t qkv_n = 0, maxp = 0, num_pages = 0, nchunk = 0;
    std::vector<DevQ8> qkv, o, gu, dn;
    DevQ8 lm;
    std::vector<float*> bias;
    std::vector<float*> attn_norm, ffn_norm;   // RMSNorm weights per layer
    float* out_norm = nullptr;                 // final RMSNorm weight
    std::vector<uint16_t*> kc, vc;
    uint16_t* emb = nullptr;
    // a checkpoint's Q8_0 token embedding (T16 / S16 tiles): the gather
    // dequantises it, and a tied model's lm_head is the Q8 product with it
    // (lm then describes the same tiles); emb stays null
    bool emb_q8 = false;
    DevQ8 embq;
    uint16_t* emb_t64 = nullptr;   // tied lm_head: the embedding in T64 order
    float* xt = nullptr;           // tied lm_head: final-norm rows in T16 column order
    // certified greedy lm_head (tied): per-row embedding constants, slice
    // summaries, and whether the embedding is finite (the path's condition)
    float* lm_rowc = nullptr;
    lgx_lmc_summary* lm_summ = nullptr;
    bool lm_cert_ok = false;
    float *cos_t = nullptr, *sin_t = nullptr;
    int32_t* page_table = nullptr;
    int32_t* seq_len = nullptr;
    // host shadow of seq_len: every call that advances the device lengths
    // updates it, so max_seq is checked before anything is launched
    std::vector<int32_t> len;
    // activations for max_batch rows
    float* h = nullptr;
    float* h2 = nullptr;       // second residual buffer (lgx_k_norm_qkv_d* writes its sum there)
    float* hcur = nullptr;     // the buffer holding the residual after layers()
    float* xn = nullptr;
    int8_t* xq = nullptr;
    uint16_t* xd = nullptr;
    int8_t* sq = nullptr;          // fused SwiGLU output (Q8_0 [max_batch][inter], T16 tiles
    uint16_t* sd = nullptr;        // for the tiled products): the gate|up product still reads xq
    float* q = nullptr;
    float* part = nullptr;
    float* attn_part = nullptr;
    float* logits = nullptr;
    float* cand = nullptr;     // argmax candidates [max_batch][slices] (value, index)
    uint64_t* scand = nullptr; // sampling candidates [max_batch][slices][LGX_SAMPLE_MAX_K]
    SampleParams samp;         // top_k 0: greedy
    int32_t last_nr = 1;       // partial count of the last lm_head
    int32_t last_B = 0;        // batch of the last lm_head
    bool last_cert = false;    // the last lm_head left no logits (certified greedy pick)
    bool fast_prefill = false; // lgx_model_set_prefill_mode: binary16 prefill
    F16Gemm* f16 = nullptr;    // fast prefill: binary16 GEMM plans and workspace
    std::vector<void*> allocs;
    bool counted = false;      // holds one of ctx->live_models
    // recorded decode steps (lgx_qwen_generate), one per (B, tokens) pair
    struct StepGraph {
        int32_t B;
        int32_t* tokens;
        int32_t last_nr;
        bool last_cert;
        hipGraphExec_t exec;
    };
    std::vector<StepGraph> graphs;
    hipStream_t capture = nullptr;   // recording only: capture needs a non-null stream
    // batched prefill: buffers for max_batch * chunk rows, allocated on first use
    struct Prefill {
        int32_t chunk = 0;           // positions per sequence per chunk
        float* h = nullptr;          // [rows][H] residual stream
        int8_t* xt = nullptr;        // [rows16][kmax] Q8_0 activations in T16 tiles
        uint16_t* xd = nullptr;      // [rows][kmax / 32]
        float* q = nullptr;          // [rows][hq][d]
        float* part = nullptr;       // group partials of the products
        float* attn_part = nullptr;  // [rows][hq][nchunk][d + 2]
        int8_t* sq = nullptr;        // [rows16][I] SwiGLU Q8_0 in T16 tiles (fused gate|up)
        uint16_t* sd = nullptr;      // [rows][I / 32]
        // fast prefill (allocated on its first use): every layer's weights
        // in binary16 (per layer qkv, o, gate|up, down, row-major), the GEMM
        // operand rows and the gate|up output rows
        uint16_t* w16 = nullptr;
        uint16_t* x16 = nullptr;     // [rows][kmax] binary16
        uint16_t* gu16 = nullptr;    // [rows][2 I] binary16
    } pf;

    ~lgx_model() {
        if (counted) ctx->live_models.fetch_sub(1);
        if (f16) f16gemm_destroy(f16);
        for (StepGraph& g : graphs) (void)hipGraphExecDestroy(g.exec);
        if (capture) (void)hipStreamDestroy(capture);
        for (void* p : allocs) (void)hipFree(p);
    }
};

namespace {

bool valid_model(const lgx_model* m) { return m && m->magic == kModelMagic && valid_ctx(m->ctx); }

template <class T>
lgx_status dev_alloc(lgx_model* m, T** p, size_t count) {
    void* v = nullptr;
    hipError_t e = hipMalloc(&v, std::max<size_t>(count * sizeof(T), 256));
    if (e != hipSuccess)
        return fail(LGX_OUT_OF_MEMORY, "model allocation of %zu bytes: %s", count * sizeof(T),
                    hipGetErrorString(e));
    m->allocs.push_back(v);
    *p = (T*)v;
    return LGX_OK;
}

// Where a model's tensors come from: the seeded generator or a checkpoint
// file.  Q8_0 matrices are row-major quants [n][k] + scales [n][k/32].
enum { W_QKV, W_O, W_GU, W_DN, W_LM, W_EMB };
enum { V_BIAS, V_ATTN_NORM, V_FFN_NORM, V_OUT_NORM };
struct Source {
    virtual ~Source() = default;
    virtual lgx_status q8(int which, int layer, int32_t n, int32_t k, int8_t* qs, uint16_t* d) = 0;
    virtual lgx_status vec(int which, int layer, int32_t n, float* out) = 0;
    virtual lgx_status emb(int32_t V, int32_t H, uint16_t* out) = 0;
    // the embedding comes as a Q8_0 matrix (q8(W_EMB, ...)) instead of binary16
    virtual bool emb_is_q8() const { return false; }
};

// The random-init model: SplitMix64 streams 1000 + 16 layer + {0,1: Wqkv;
// 2,3: Wo; 4,5: Wgate|up; 6,7: Wdown; 8: qkv bias}, 1 embedding, 2/3 the
// untied lm_head; norm weights 1.
struct GenSource : Source {
    uint64_t seed;
    double emb_sigma;
    GenSource(uint64_t s, double sig) : seed(s), emb_sigma(sig) {}
    lgx_status q8(int which, int layer, int32_t n, int32_t k, int8_t* qs, uint16_t* d) override {
        const uint64_t stream = which == W_LM ? 2 : 1000 + 16 * (uint64_t)layer + 2 * which;
        lgxg::gen_i8(seed, stream, qs, (int64_t)n * k);
        lgxg::gen_q8_scales(seed, stream + 1, d, (int64_t)n * (k / 32));
        return LGX_OK;
    }
    lgx_status vec(int which, int layer, int32_t n, float* out) override {
        if (which == V_BIAS)
            lgxg::gen_normal_f32(seed, 1000 + 16 * (uint64_t)layer + 8, 0.02, out, n);
        else
            std::fill(out, out + n, 1.0f);
        return LGX_OK;
    }
    lgx_status emb(int32_t V, int32_t H, uint16_t* out) override {
        lgxg::gen_normal_f16(seed, 1, emb_sigma, out, (int64_t)V * H);
        return LGX_OK;
    }
};

// A Qwen2 GGUF file: the fused QKV rows are attn_q | attn_k | attn_v, the
// fused gate|up rows ffn_gate | ffn_up.
struct GgufSource : Source {
    const lgxf::Gguf& g;
    lgx_qwen_config c;
    GgufSource(const lgxf::Gguf& gg, const lgx_qwen_config& cf) : g(gg), c(cf) {}
    static std::string blk(int l, const char* t) { return "blk." + std::to_string(l) + "." + t; }
    lgx_status q8(int which, int layer, int32_t n, int32_t k, int8_t* qs, uint16_t* d) override {
        const int qd = c.n_heads * c.head_dim, kd = c.n_kv_heads * c.head_dim;
        lgx_status st;
        switch (which) {
            case W_QKV:
                if ((st = g.read_q8(blk(layer, "attn_q.weight"), qd, k, qs, d)) ||
                    (st = g.read_q8(blk(layer, "attn_k.weight"), kd, k, qs + (int64_t)qd * k,
                                    d + (int64_t)qd * (k / 32))))
                    return st;
                return g.read_q8(blk(layer, "attn_v.weight"), kd, k, qs + (int64_t)(qd + kd) * k,
                                 d + (int64_t)(qd + kd) * (k / 32));
            case W_O: return g.read_q8(blk(layer, "attn_output.weight"), n, k, qs, d);
            case W_GU:
                if ((st = g.read_q8(blk(layer, "ffn_gate.weight"), n / 2, k, qs, d))) return st;
                return g.read_q8(blk(layer, "ffn_up.weight"), n / 2, k, qs + (int64_t)(n / 2) * k,
                                 d + (int64_t)(n / 2) * (k / 32));
            case W_DN: return g.read_q8(blk(layer, "ffn_down.weight"), n, k, qs, d);
            case W_EMB: return g.read_q8("token_embd.weight", n, k, qs, d);
            default: return g.read_q8("output.weight", n, k, qs, d);
        }
    }
    lgx_status vec(int which, int layer, int32_t n, float* out) override {
        using lgxf::GGML_F32;
        if (which == V_BIAS) {
            const int qd = c.n_heads * c.head_dim, kd = c.n_kv_heads * c.head_dim;
            lgx_status st;
            if ((st = g.read_raw(blk(layer, "attn_q.bias"), GGML_F32, 1, qd, out)) ||
                (st = g.read_raw(blk(layer, "attn_k.bias"), GGML_F32, 1, kd, out + qd)))
                return st;
            return g.read_raw(blk(layer, "attn_v.bias"), GGML_F32, 1, kd, out + qd + kd);
        }
        if (which == V_OUT_NORM) return g.read_raw("output_norm.weight", GGML_F32, 1, n, out);
        return g.read_raw(blk(layer, which == V_ATTN_NORM ? "attn_norm.weight" : "ffn_norm.weight"),
                          GGML_F32, 1, n, out);
    }
    lgx_status emb(int32_t V, int32_t H, uint16_t* out) override {
        return g.read_raw("token_embd.weight", lgxf::GGML_F16, V, H, out);
    }
    bool emb_is_q8() const override {
        const lgxf::TensorInfo* t = g.tensor("token_embd.weight");
        return t && t->type == lgxf::GGML_Q8_0;
    }
};

// Take a Q8_0 matrix from the source, upload it row-major into the staging
// buffers and repack into the device tile layouts.
lgx_status make_q8(lgx_model* m, Source& src, int which, int layer, int32_t n, int32_t k,
                   DevQ8* out, int8_t* stage_q, uint16_t* stage_d, std::vector<int8_t>& hq,
                   std::vector<uint16_t>& hd) {
    const int64_t nq = (int64_t)n * k, nd = (int64_t)n * (k / 32);
    hq.resize(nq);
    hd.resize(nd);
    lgx_status st = src.q8(which, layer, n, k, hq.data(), hd.data());
    if (st != LGX_OK) return st;
    if ((st = dev_alloc(m, &out->qs, (size_t)nq)) != LGX_OK) return st;
    if ((st = dev_alloc(m, &out->d, lgx_q8_scale_count(n, k))) != LGX_OK) return st;
    LGX_HIP(hipMemcpy(stage_q, hq.data(), nq, hipMemcpyHostToDevice));
    LGX_HIP(hipMemcpy(stage_d, hd.data(), nd * 2, hipMemcpyHostToDevice));
    lgx_repack_args ra{stage_q, out->qs, n, k, 1};
    if ((st = launch(m->ctx, K_REPACK, dim3(cdiv((int64_t)(n / 16) * (k / 64) * 64, 256)), dim3(256),
                     ra, nullptr)) != LGX_OK)
        return st;
    lgx_srepack_args sa{stage_d, out->d, n, k, 1};
    if ((st = launch(m->ctx, K_REPACK_S16, dim3(cdiv((int64_t)lgx_q8_scale_count(n, k), 256)),
                     dim3(256), sa, nullptr)) != LGX_OK)
        return st;
    LGX_HIP(hipDeviceSynchronize());     // staging reused by the next matrix
    out->m = lgx_q8_matrix{out->qs, out->d, n, k, LGX_Q8_T16};
    return LGX_OK;
}

// Embedding rows of m tokens (row r = b * qpr + j takes tokens[b * stride + j])
// into h [m][hidden]: binary16 rows widened, or Q8_0 rows dequantised.
lgx_status embed(lgx_model* md, const int32_t* tokens, int stride, int qpr, float* h, int m,
                 void* stream) {
    const lgx_qwen_config& cf = md->c;
    if (md->emb_q8) {
        lgx_embed_q8_args a{md->embq.qs, md->embq.d, tokens, h, m, cf.hidden, cf.vocab, stride, qpr};
        return launch(md->ctx, K_EMBED_Q8, dim3(m), dim3(256), a, stream);
    }
    lgx_embed_args a{md->emb, tokens, h, m, cf.hidden, cf.vocab, stride, qpr};
    return launch(md->ctx, K_EMBED, dim3(m), dim3(256), a, stream);
}

// The binary16 lm_head of a tied embedding (else the Q8 product with lm).
bool f16_head(const lgx_model* md) { return md->c.tied_embedding && !md->emb_q8; }

lgx_status check_config(const lgx_qwen_config* c) {
    const int hq = c->n_heads, hkv = c->n_kv_heads, d = c->head_dim, H = c->hidden,
              I = c->intermediate;
    if (c->n_layers <= 0 || H <= 0 || I <= 0 || hq <= 0 || hkv <= 0 || c->vocab <= 0 ||
        c->max_batch <= 0 || c->max_seq <= 0)
        return fail(LGX_INVALID_ARGUMENT, "non-positive model dimension");
    if ((d != 64 && d != 128) || hq % hkv != 0 || hq / hkv > 8)
        return fail(LGX_UNSUPPORTED, "head_dim %d, %d/%d heads", d, hq, hkv);
    if (H % 64 || I % 64 || (hq * d) % 64 || ((hq + 2 * hkv) * d) % 16)
        return fail(LGX_UNSUPPORTED, "hidden/intermediate/head sizes must be multiples of 64");
    if (H > 8192 || (hq + 2 * hkv) * d > 8192 || hq * d > 8192 || I > 32768)
        return fail(LGX_UNSUPPORTED, "hidden %d / qkv %d / intermediate %d too large", H,
                    (hq + 2 * hkv) * d, I);
    if (!c->tied_embedding && c->vocab % 16)
        return fail(LGX_UNSUPPORTED, "untied Q8_0 lm_head needs vocab %% 16 == 0");
    return LGX_OK;
}


// Decode products of m >= 33 rows go through the tiled product (32 activation
// rows per workgroup, ranges grouped for a full grid; at 32 rows and below
// the streaming kernels are as fast); their activations are written in T16
// tiles by the producers (norm, attention merge, SwiGLU).
bool dec_tiled(const lgx_model* md, int m) { return m >= 33 && !md->ctx->decode_streaming; }

// Decode tiled kernel for W over m rows: 64 activation rows per workgroup
// (each weight tile read by one workgroup, not two) for the products whose
// 32-row grid holds more than four workgroups per compute unit, 32 rows for
// the small ones (config 4, per launch: lm_head 160 against 174 us, gate|up
// 50.4 against 51.5, down 30.6 against 31.8; qkv 13.4 against 11.9, o 10.2
// against 8.8).  LGX_GEMM_TILED_ROWS forces one width.
Kern dec_kernel(const lgx_model* md, const DevQ8& W, int m) {
    const lgx_ctx* c = md->ctx;
    if (c->tiled_rows || m < 49) return tiled_kernel(c, m);
    const int64_t tiles32 = cdiv(W.m.n, LGX_TG_N) * cdiv(m, 32);
    const int grp = tiled_grp(c, K_GEMM_TILED32, W.m.n, W.m.k, m);
    return tiles32 * tiled_groups(W.m.k, grp) > 4 * (int64_t)c->ncu ? K_GEMM_TILED64 : K_GEMM_TILED32;
}
// Ranges per group of a decode tiled product; the SwiGLU-fused gate|up
// product keeps its whole reduction in one group.
int dec_grp(const lgx_model* md, const DevQ8& W, int m, bool swiglu = false) {
    const lgx_ctx* c = md->ctx;
    if (swiglu && !c->tiled_grp && nranges_of(W.m.k) <= LGX_TG_RANGES) return LGX_TG_RANGES;
    return tiled_grp(c, dec_kernel(md, W, m), W.m.n, W.m.k, m);
}

// Partials a product of W over m rows leaves for its consumer's tree.
int parts(const lgx_model* md, const DevQ8& W, int m) {
    if (!dec_tiled(md, m)) return nranges_of(W.m.k);
    return tiled_groups(W.m.k, dec_grp(md, W, m));
}

lgx_status product(lgx_model* md, const DevQ8& W, int m, void* stream,
                   const int8_t* xq = nullptr, const uint16_t* xd = nullptr) {
    if (!xq) {
        xq = md->xq;
        xd = md->xd;
    }
    if (dec_tiled(md, m))
        return run_q8_tiled(md->ctx, &W.m, xq, xd, m, md->part, stream, dec_kernel(md, W, m),
                            dec_grp(md, W, m));
    if (m == 1 && gemv_group_ok(md->ctx, W.m.k)) {
        const lgx_gemv_mat g = gemv_mat(&W.m, nullptr, xq, xd, md->part, 1);
        return run_gemv_group(md->ctx, &g, 1, stream);
    }
    // decode batches of 17..32 rows: two 16-row m-groups (twice the
    // workgroups of the 32-row kernel, half the activation staging each;
    // the weight tile's second read hits L2)
    const Kern k = m == 1 ? K_GEMV_MFMA
                   : (m > 16 && m <= 32 && !md->ctx->gemm_mt) ? K_GEMM_MFMA16
                                                              : gemm_kernel(md->ctx, m);
    return run_q8(md->ctx, k, &W.m, nullptr, xq, xd, m, md->part, nullptr, stream, nullptr,
                  nullptr, md->part);
}

// Tiled gate|up products that finish with SwiGLU + Q8_0 in their own
// workgroups (into sq / sd): the whole reduction in one range group.
bool tiled_swiglu(const lgx_model* md, int m) {
    const lgx_ctx* c = md->ctx;
    return c->tiled_swiglu && dec_tiled(md, m) && md->c.intermediate % 32 == 0 &&
           tiled_groups(md->gu[0].m.k, dec_grp(md, md->gu[0], m, true)) == 1;
}

// Decode products whose consumer runs in the product's own workgroups
// (lgx_k_q8_gemm_mfma16_qkv / _swiglu): 2+ rows on the streaming kernels
// and K in one range, so every output is final where it is computed.
bool fused(const lgx_model* md, int m) {
    const lgx_ctx* c = md->ctx;
    return c->decode_fuse && m > 1 && !dec_tiled(md, m) && nranges_of(md->c.hidden) == 1 &&
           (c->gemm_mt == 0 || c->gemm_mt == 16);
}

// Decode steps whose attention merge runs inside the o_proj product
// (lgx_k_attn_merge_o_d*): o_proj's K = hq * d in one range, the merge in
// one round of at most 16 chunks, products on the streaming kernels (the
// tiled ones read each weight tile once for many rows; this kernel reads
// o's weights once per sequence, from L2).
bool merge_o(const lgx_model* md, int m) {
    const lgx_qwen_config& cf = md->c;
    const int k = cf.n_heads * cf.head_dim;
    return md->ctx->decode_fuse && !dec_tiled(md, m) && k <= 1024 && k % 64 == 0 && md->nchunk <= 16 &&
           (cf.head_dim == 64 || cf.head_dim == 128);
}

// Decode steps whose attention-side norm runs inside the qkv product
// (lgx_k_norm_qkv_d*): hidden in one range, qkv columns in whole groups of
// 128 (whole heads), at most LGX_NQ_MAXR partials of the down product,
// products on the streaming kernels (each sequence's workgroups read the
// qkv weights from L2).
bool norm_qkv(const lgx_model* md, int m) {
    const lgx_qwen_config& cf = md->c;
    const int d = cf.head_dim;
    return md->ctx->decode_fuse && !dec_tiled(md, m) && cf.hidden <= 1024 && cf.hidden % 64 == 0 &&
           (d == 64 || d == 128) && md->qkv_n % (16 * LGX_NQ_TILES) == 0 &&
           parts(md, md->dn[0], m) <= LGX_NQ_MAXR;
}

lgx_status run_fused(lgx_model* md, Kern kern, const DevQ8& W, int m, int tpw, int ngroups,
                     lgx_gemm_fused_args& f, void* stream) {
    lgx_gemv_args& a = f.g;
    a.wt = W.m.qs;
    a.wd = W.m.d;
    a.xq = md->xq;
    a.xd = md->xd;
    a.n = W.m.n;
    a.k = W.m.k;
    a.m = m;
    a.ntiles = W.m.n / 16;
    a.nranges = 1;
    a.nmgroups = (int)cdiv(m, 16);
    a.tpw = tpw;
    return launch(md->ctx, kern, dim3(ngroups * a.nmgroups), dim3(256), f, stream);
}

lgx_status norm(lgx_model* md, float* h, const float* w, int m, int n, int nr_part, bool with_part,
                float* xn, bool q8, void* stream, float* xt = nullptr) {
    lgx_norm_args a{};
    a.xt = xt;
    a.part = with_part ? md->part : nullptr;
    a.nr = nr_part;
    a.h = h;
    a.w = w;
    a.xn = xn;
    a.xq = q8 ? md->xq : nullptr;
    a.xd = q8 ? md->xd : nullptr;
    a.xq_t16 = q8 && dec_tiled(md, m);
    a.m = m;
    a.n = n;
    a.eps = md->c.rms_eps;
    return launch_norm(md->ctx, a, stream);
}

// One token per sequence 0..B-1 through every layer; leaves the down
// partials of the last layer in md->part (for the final norm).
lgx_status layers(lgx_model* md, int B, const int32_t* tokens, int tokens_stride, void* stream) {
    lgx_ctx* c = md->ctx;
    const lgx_qwen_config& cf = md->c;
    const int H = cf.hidden, I = cf.intermediate, d = cf.head_dim, hq = cf.n_heads,
              hkv = cf.n_kv_heads;
    lgx_status st;
    if ((st = embed(md, tokens, tokens_stride, 1, md->h, B, stream)) != LGX_OK) return st;
    float* hcur = md->h;   // the residual; lgx_k_norm_qkv_d* moves it to the other buffer
    const bool nq = norm_qkv(md, B);
    for (int l = 0; l < cf.n_layers; ++l) {
        // norm (+ residual of the previous layer's down product) -> Q8
        if (!nq && (st = norm(md, hcur, md->attn_norm[l], B, H, parts(md, md->dn[0], B), l > 0, nullptr,
                              true, stream)) != LGX_OK)
            return st;
        lgx_qkv_args qa{};
        qa.part = md->part;
        qa.nr = parts(md, md->qkv[l], B);
        qa.bias = md->bias[l];
        qa.cos_t = md->cos_t;
        qa.sin_t = md->sin_t;
        qa.seq_len = md->seq_len;
        qa.page_table = md->page_table;
        qa.kpages = md->kc[l];
        qa.vpages = md->vc[l];
        qa.q_out = md->q;
        qa.m = B;
        qa.hq = hq;
        qa.hkv = hkv;
        qa.d = d;
        qa.maxp = md->maxp;
        qa.num_pages = md->num_pages;
        qa.max_seq = cf.max_seq;
        if (nq) {
            // residual, norm, Q8_0, qkv, RoPE and KV append in one launch:
            // workgroup = (sequence, LGX_NQ_TILES row tiles of qkv), each
            // normalising the sequence's row itself; the residual moves to
            // the other buffer (the sequence's other workgroups still read
            // this one)
            float* hnext = hcur == md->h ? md->h2 : md->h;
            lgx_norm_qkv_args a{};
            a.q = qa;
            a.h = hcur;
            a.part = l > 0 ? md->part : nullptr;
            a.nr = l > 0 ? parts(md, md->dn[0], B) : 0;
            a.h_out = hnext;
            a.w = md->attn_norm[l];
            a.wt = md->qkv[l].m.qs;
            a.wd = md->qkv[l].m.d;
            a.H = H;
            a.n = md->qkv_n;
            a.ngroups = md->qkv_n / (16 * LGX_NQ_TILES);
            a.eps = cf.rms_eps;
            if ((st = launch(c, d == 64 ? K_NORM_QKV_D64 : K_NORM_QKV_D128, dim3((unsigned)(B * a.ngroups)),
                             dim3(64 * LGX_NQ_TILES), a, stream)) != LGX_OK)
                return st;
            hcur = hnext;
        } else if (fused(md, B)) {
            // one workgroup per (head, 16-row m-group)
            lgx_gemm_fused_args f{};
            f.q = qa;
            if ((st = run_fused(md, K_GEMM_MFMA16_QKV, md->qkv[l], B, d / 64, hq + 2 * hkv, f,
                                stream)) != LGX_OK)
                return st;
        } else {
            if ((st = product(md, md->qkv[l], B, stream)) != LGX_OK) return st;
            if ((st = launch_qkv_rope(c, qa, B, stream)) !=
                LGX_OK)
                return st;
        }
        lgx_attn_args aa{};
        aa.q = md->q;
        aa.kpages = md->kc[l];
        aa.vpages = md->vc[l];
        aa.page_table = md->page_table;
        aa.seq_len = md->seq_len;
        aa.part = md->attn_part;
        aa.out = nullptr;
        aa.B = B;
        aa.hq = hq;
        aa.hkv = hkv;
        aa.maxp = md->maxp;
        aa.nchunk = md->nchunk;
        aa.num_pages = md->num_pages;
        aa.maxlen = cf.max_seq;
        aa.len_add = 1;
        aa.scale = (float)(1.0 / std::sqrt((double)d));
        aa.xq = md->xq;
        aa.xq_t16 = dec_tiled(md, B);
        aa.xd = md->xd;
        if ((st = launch(c, (Kern)attn_kernel(d, hq / hkv), dim3(md->nchunk, B * hkv), dim3(256), aa,
                         stream)) != LGX_OK)
            return st;
        if (merge_o(md, B)) {
            // merge and o_proj in one launch: workgroup = (sequence,
            // merge_o_tiles row tiles of o), each merging the sequence's
            // heads itself
            lgx_merge_o_args mo{};
            mo.at = aa;
            mo.wt = md->o[l].m.qs;
            mo.wd = md->o[l].m.d;
            mo.y = md->part;
            mo.n = H;
            mo.k = hq * d;
            mo.tiles = c->merge_o_tiles;
            mo.ngroups = (int)cdiv(H / 16, mo.tiles);
            if ((st = launch(c, d == 64 ? K_MERGE_O_D64 : K_MERGE_O_D128, dim3((unsigned)(B * mo.ngroups)),
                             dim3(1024), mo, stream)) != LGX_OK)
                return st;
        } else {
            if ((st = launch(c, d == 64 ? K_ATTN_COMBINE_QUANT_D64 : K_ATTN_COMBINE_QUANT_D128,
                             dim3(B * hq), dim3(d), aa, stream)) != LGX_OK)
                return st;
            if ((st = product(md, md->o[l], B, stream)) != LGX_OK) return st;
        }
        if ((st = norm(md, hcur, md->ffn_norm[l], B, H, parts(md, md->o[l], B), true, nullptr, true,
                       stream)) != LGX_OK)
            return st;
        if (fused(md, B) && I % (32 * c->fuse_cols32) == 0) {
            // one workgroup per (32 * cols32 SwiGLU columns, m-group); the Q8_0
            // output goes to sq / sd, which the down product reads
            lgx_gemm_fused_args f{};
            f.s = lgx_swiglu_args{nullptr, 1, md->sq, md->sd, nullptr, B, I, 0};
            if ((st = run_fused(md, K_GEMM_MFMA16_SWIGLU, md->gu[l], B, c->fuse_cols32,
                                I / (32 * c->fuse_cols32), f, stream)) != LGX_OK)
                return st;
            if ((st = product(md, md->dn[l], B, stream, md->sq, md->sd)) != LGX_OK) return st;
            continue;
        }
        if (tiled_swiglu(md, B)) {
            const DevQ8& W = md->gu[l];
            if ((st = run_q8_tiled(c, &W.m, md->xq, md->xd, B, md->part, stream, dec_kernel(md, W, B),
                                   dec_grp(md, W, B, true), I, md->sq, md->sd)) != LGX_OK)
                return st;
            if ((st = product(md, md->dn[l], B, stream, md->sq, md->sd)) != LGX_OK) return st;
            continue;
        }
        if ((st = product(md, md->gu[l], B, stream)) != LGX_OK) return st;
        lgx_swiglu_args sw{md->part, parts(md, md->gu[l], B), md->xq, md->xd, nullptr, B, I,
                           dec_tiled(md, B) ? 1 : 0};
        if ((st = launch(c, K_SWIGLU_QUANT, dim3(B, cdiv(I / 32, 32)), dim3(256), sw, stream)) !=
            LGX_OK)
            return st;
        if ((st = product(md, md->dn[l], B, stream)) != LGX_OK) return st;
    }
    md->hcur = hcur;
    return LGX_OK;
}

// Final norm, lm_head and greedy token into `next`; seq_len += 1.
lgx_status head(lgx_model* md, int B, int32_t* next, void* stream) {
    lgx_ctx* c = md->ctx;
    const lgx_qwen_config& cf = md->c;
    const int H = cf.hidden;
    lgx_status st;
    const bool tied = f16_head(md);
    if ((st = norm(md, md->hcur, md->out_norm, B, H, parts(md, md->dn[0], B), true, md->xn, !tied, stream,
                   tied ? md->xt : nullptr)) != LGX_OK)
        return st;
    if (tied && md->lm_cert_ok && md->ctx->lm_cert && md->samp.top_k == 0 && B <= LGX_LMC_MAXB) {
        // greedy: the certified pick from the final-norm rows (xn), no logits
        md->last_nr = 1;
        md->last_B = B;
        md->last_cert = true;
        return launch_lm_cert(c, md->xn, md->emb, md->emb_t64, md->lm_rowc, B, H, cf.vocab,
                              md->lm_summ, nullptr, next, md->seq_len, 1, stream);
    }
    md->last_cert = false;
    const float* lg;
    int nr;
    if (tied) {
        // one chain per 1024-column range of the hidden size: range partials
        // [nr][B][vocab], the argmax / draw applies the tree
        nr = nranges_of(H);
        lgx_lmhead_args la{md->xt, md->emb_t64, md->logits, B, H, cf.vocab};
        if ((st = launch(c, K_LM_HEAD_T64, dim3(cdiv(cf.vocab, 64), cdiv(B, 16), nr), dim3(64), la,
                         stream)) != LGX_OK)
            return st;
        lg = md->logits;
    } else {
        if ((st = product(md, md->lm, B, stream)) != LGX_OK) return st;
        lg = md->part;
        nr = parts(md, md->lm, B);
    }
    md->last_nr = nr;
    md->last_B = B;
    if (md->samp.top_k > 0)   // draw index: the position just consumed (seq_len before += 1)
        return launch_sample(c, md->samp, lg, nr, B, cf.vocab, nullptr, next, md->seq_len, 1,
                             md->scand, stream);
    return launch_argmax(c, lg, nr, B, cf.vocab, next, md->seq_len, 1, md->cand, stream);
}

// ---- batched prefill ----------------------------------------------------
// Rows b * n + j of a chunk are positions seq_len[b] + j of the B sequences;
// every kernel runs the decode step's schedule per row, so the cache holds
// the values a token-by-token prefill writes.

lgx_status prefill_alloc(lgx_model* md) {
    if (md->pf.chunk) return LGX_OK;
    const lgx_qwen_config& cf = md->c;
    const int H = cf.hidden, I = cf.intermediate, d = cf.head_dim, hq = cf.n_heads;
    // about 8192 rows per chunk: enough rows for the tiled products
    int chunk = std::max(16, (8192 / cf.max_batch + 15) / 16 * 16);
    if (md->ctx->prefill_chunk > 0) chunk = md->ctx->prefill_chunk;
    chunk = std::min(chunk, (cf.max_seq + 15) / 16 * 16);
    const int64_t rows = (int64_t)cf.max_batch * chunk, rows16 = (rows + 15) / 16 * 16;
    const int kmax = std::max({H, I, hq * d});
    int64_t part = 0;
    auto upd = [&](int n, int k) { part = std::max<int64_t>(part, (int64_t)tiled_groups(k) * rows * n); };
    upd(md->qkv_n, H);
    upd(H, hq * d);
    upd(2 * I, H);
    upd(H, I);
    lgx_model::Prefill& pf = md->pf;
    lgx_status st;
    if ((st = dev_alloc(md, &pf.h, (size_t)rows * H)) ||
        (st = dev_alloc(md, &pf.xt, (size_t)rows16 * kmax)) ||
        (st = dev_alloc(md, &pf.xd, (size_t)rows * kmax / 32)) ||
        (st = dev_alloc(md, &pf.q, (size_t)rows * hq * d)) || (st = dev_alloc(md, &pf.part, (size_t)part)) ||
        (st = dev_alloc(md, &pf.attn_part, (size_t)rows * hq * md->nchunk * (d + 2))) ||
        (st = dev_alloc(md, &pf.sq, (size_t)rows16 * I)) || (st = dev_alloc(md, &pf.sd, (size_t)rows * I / 32)))
        return st;
    pf.chunk = chunk;
    return LGX_OK;
}

// Product of W over the chunk's M rows (Q8_0 in T16 tiles pf.xt, scales
// pf.xd, written so by the producers): group partials of 4 ranges into pf.part.
lgx_status pf_product(lgx_model* md, const DevQ8& W, int M, void* stream) {
    return run_q8_tiled(md->ctx, &W.m, md->pf.xt, md->pf.xd, M, md->pf.part, stream);
}

lgx_status pf_norm(lgx_model* md, const float* w, int M, int n, int nr, bool with_part,
                   void* stream) {
    lgx_norm_args a{};
    a.part = with_part ? md->pf.part : nullptr;
    a.nr = nr;
    a.h = md->pf.h;
    a.w = w;
    a.xq = md->pf.xt;
    a.xd = md->pf.xd;
    a.xq_t16 = 1;
    a.m = M;
    a.n = n;
    a.eps = md->c.rms_eps;
    return launch_norm(md->ctx, a, stream);
}

// binary16 weights of one layer: qkv, o, gate|up, down, row-major
int64_t layer_w16(const lgx_model* md) {
    const lgx_qwen_config& cf = md->c;
    const int64_t H = cf.hidden, I = cf.intermediate, hd = (int64_t)cf.n_heads * cf.head_dim;
    return md->qkv_n * H + H * hd + 2 * I * H + H * I;
}

lgx_status dequant16(lgx_model* md, const DevQ8& W, uint16_t* out, void* stream) {
    lgx_dequant_args a{W.m.qs, W.m.d, out, W.m.n, W.m.k};
    const int64_t threads = (int64_t)W.m.n * (W.m.k / 8);
    return launch(md->ctx, K_DEQUANT_F16, dim3((unsigned)cdiv(threads, 256)), dim3(256), a, stream);
}

// The fast prefill's buffers, on its first use: every layer's weights in
// binary16 (dequantised here, once: the weights never change), the
// binary16 GEMM operand rows and the gate|up output rows.
lgx_status prefill_fast_alloc(lgx_model* md, void* stream) {
    lgx_model::Prefill& pf = md->pf;
    if (pf.w16) return LGX_OK;
    const lgx_qwen_config& cf = md->c;
    const int64_t H = cf.hidden, I = cf.intermediate, hd = (int64_t)cf.n_heads * cf.head_dim;
    const int64_t rows = (int64_t)cf.max_batch * pf.chunk;
    const int64_t kmax = std::max({H, I, hd}), lw = layer_w16(md);
    uint16_t *w16 = nullptr, *x16 = nullptr, *gu16 = nullptr;
    lgx_status st;
    if ((st = dev_alloc(md, &w16, (size_t)(lw * cf.n_layers))) ||
        (st = dev_alloc(md, &x16, (size_t)(rows * kmax))) ||
        (st = dev_alloc(md, &gu16, (size_t)(rows * 2 * I))))
        return st;
    for (int l = 0; l < cf.n_layers; ++l) {
        uint16_t* w = w16 + lw * l;
        if ((st = dequant16(md, md->qkv[l], w, stream)) != LGX_OK ||
            (st = dequant16(md, md->o[l], w + md->qkv_n * H, stream)) != LGX_OK ||
            (st = dequant16(md, md->gu[l], w + md->qkv_n * H + H * hd, stream)) != LGX_OK ||
            (st = dequant16(md, md->dn[l], w + md->qkv_n * H + H * hd + 2 * I * H, stream)) != LGX_OK)
            return st;
    }
    if (!md->f16 && (st = f16gemm_create(&md->f16)) != LGX_OK) return st;
    pf.w16 = w16;
    pf.x16 = x16;
    pf.gu16 = gu16;
    return LGX_OK;
}

// prefill_chunk in the fast mode: every product a binary16 GEMM (the
// dequantised weights, binary16 activations, binary32 accumulation; binary32
// outputs, binary16 for gate|up), the norms and RoPE / KV append as in the
// exact chunk on one-range outputs, SwiGLU on binary16, the attention
// lgx_gqa_prefill_attn_fast's kernel.
lgx_status prefill_chunk_fast(lgx_model* md, int B, int n, const int32_t* tokens, int stride,
                              void* stream) {
    lgx_ctx* c = md->ctx;
    const lgx_qwen_config& cf = md->c;
    const int H = cf.hidden, I = cf.intermediate, d = cf.head_dim, hq = cf.n_heads,
              hkv = cf.n_kv_heads;
    const int M = B * n;
    lgx_model::Prefill& pf = md->pf;
    lgx_status st;
    auto norm16 = [&](const float* w, bool with_part) {
        lgx_norm_args a{};
        a.part = with_part ? pf.part : nullptr;
        a.nr = 1;
        a.h = pf.h;
        a.w = w;
        a.x16 = pf.x16;
        a.m = M;
        a.n = H;
        a.eps = cf.rms_eps;
        return launch_norm(c, a, stream);
    };
    if ((st = embed(md, tokens, stride, n, pf.h, M, stream)) != LGX_OK) return st;
    for (int l = 0; l < cf.n_layers; ++l) {
        const uint16_t* wq = pf.w16 + layer_w16(md) * l;
        const uint16_t* wo = wq + (int64_t)md->qkv_n * H;
        const uint16_t* wg = wo + (int64_t)H * hq * d;
        const uint16_t* wd = wg + (int64_t)2 * I * H;
        if ((st = norm16(md->attn_norm[l], l > 0)) != LGX_OK ||
            (st = f16gemm_run(md->f16, wq, pf.x16, pf.part, false, M, md->qkv_n, H, stream)) != LGX_OK)
            return st;
        lgx_qkv_args qa{};
        qa.part = pf.part;
        qa.nr = 1;
        qa.bias = md->bias[l];
        qa.cos_t = md->cos_t;
        qa.sin_t = md->sin_t;
        qa.seq_len = md->seq_len;
        qa.page_table = md->page_table;
        qa.kpages = md->kc[l];
        qa.vpages = md->vc[l];
        qa.q_out = pf.q;
        qa.m = M;
        qa.hq = hq;
        qa.hkv = hkv;
        qa.d = d;
        qa.maxp = md->maxp;
        qa.num_pages = md->num_pages;
        qa.max_seq = cf.max_seq;
        qa.qpr = n;
        if ((st = launch_qkv_rope(c, qa, M, stream)) != LGX_OK) return st;
        if (l == cf.n_layers - 1) break;
        lgx_attn_args aa{};
        aa.q = pf.q;
        aa.kpages = md->kc[l];
        aa.vpages = md->vc[l];
        aa.page_table = md->page_table;
        aa.seq_len = md->seq_len;
        aa.B = B;
        aa.hq = hq;
        aa.hkv = hkv;
        aa.maxp = md->maxp;
        aa.num_pages = md->num_pages;
        aa.maxlen = cf.max_seq;
        aa.len_add = 1;
        aa.scale = (float)(1.0 / std::sqrt((double)d));
        aa.qpr = n;
        aa.out16 = pf.x16;
        lgx_swiglu16_args sw{pf.gu16, pf.x16, M, I};
        if ((st = launch_prefill_attn_fast(c, aa, d, stream)) != LGX_OK ||
            (st = f16gemm_run(md->f16, wo, pf.x16, pf.part, false, M, H, hq * d, stream)) != LGX_OK ||
            (st = norm16(md->ffn_norm[l], true)) != LGX_OK ||
            (st = f16gemm_run(md->f16, wg, pf.x16, pf.gu16, true, M, 2 * I, H, stream)) != LGX_OK ||
            (st = launch(c, K_SWIGLU_F16, dim3((unsigned)cdiv((int64_t)M * (I / 8), 256)), dim3(256), sw,
                         stream)) != LGX_OK ||
            (st = f16gemm_run(md->f16, wd, pf.x16, pf.part, false, M, H, I, stream)) != LGX_OK)
            return st;
    }
    lgx_advance_args av{md->seq_len, B, n, 1};
    return launch(c, K_ADVANCE, dim3(cdiv(B, 64)), dim3(64), av, stream);
}

// One chunk: positions seq_len[b] + j (j < n) of the B sequences, tokens
// tokens[b * stride + j]; ncg chunks of 256 cached tokens bound the
// attention grid.  Leaves seq_len[b] += n.  The last layer stops after its
// KV append: its attention and MLP only feed the hidden state of these
// positions, which no later step reads.
lgx_status prefill_chunk(lgx_model* md, int B, int n, const int32_t* tokens, int stride, int ncg,
                         void* stream) {
    lgx_ctx* c = md->ctx;
    const lgx_qwen_config& cf = md->c;
    const int H = cf.hidden, I = cf.intermediate, d = cf.head_dim, hq = cf.n_heads,
              hkv = cf.n_kv_heads;
    const int M = B * n;
    lgx_model::Prefill& pf = md->pf;
    lgx_status st;
    if ((st = embed(md, tokens, stride, n, pf.h, M, stream)) != LGX_OK) return st;
    for (int l = 0; l < cf.n_layers; ++l) {
        if ((st = pf_norm(md, md->attn_norm[l], M, H, tiled_groups(I), l > 0, stream)) != LGX_OK)
            return st;
        if ((st = pf_product(md, md->qkv[l], M, stream)) != LGX_OK) return st;
        lgx_qkv_args qa{};
        qa.part = pf.part;
        qa.nr = tiled_groups(H);
        qa.bias = md->bias[l];
        qa.cos_t = md->cos_t;
        qa.sin_t = md->sin_t;
        qa.seq_len = md->seq_len;
        qa.page_table = md->page_table;
        qa.kpages = md->kc[l];
        qa.vpages = md->vc[l];
        qa.q_out = pf.q;
        qa.m = M;
        qa.hq = hq;
        qa.hkv = hkv;
        qa.d = d;
        qa.maxp = md->maxp;
        qa.num_pages = md->num_pages;
        qa.max_seq = cf.max_seq;
        qa.qpr = n;
        if ((st = launch_qkv_rope(c, qa, M, stream)) != LGX_OK)
            return st;
        if (l == cf.n_layers - 1) break;
        lgx_attn_args aa{};
        aa.q = pf.q;
        aa.kpages = md->kc[l];
        aa.vpages = md->vc[l];
        aa.page_table = md->page_table;
        aa.seq_len = md->seq_len;
        aa.part = pf.attn_part;
        aa.B = B;
        aa.hq = hq;
        aa.hkv = hkv;
        aa.maxp = md->maxp;
        aa.nchunk = md->nchunk;
        aa.num_pages = md->num_pages;
        aa.maxlen = cf.max_seq;
        aa.len_add = 1;
        aa.scale = (float)(1.0 / std::sqrt((double)d));
        aa.xq = pf.xt;
        aa.xq_t16 = 1;
        aa.xd = pf.xd;
        aa.qpr = n;
        aa.ncg = ncg;
        if ((st = launch_prefill_attn(c, aa, d, stream)) != LGX_OK ||
            (st = launch(c, d == 64 ? K_ATTN_COMBINE_QUANT_D64 : K_ATTN_COMBINE_QUANT_D128,
                         dim3(M * hq), dim3(d), aa, stream)) != LGX_OK)
            return st;
        if ((st = pf_product(md, md->o[l], M, stream)) != LGX_OK) return st;
        if ((st = pf_norm(md, md->ffn_norm[l], M, H, tiled_groups(hq * d), true, stream)) != LGX_OK)
            return st;
        if (c->tiled_swiglu && I % 32 == 0 && tiled_groups(H) == 1) {
            // SwiGLU + Q8_0 in the gate|up product's workgroups, into pf.sq / pf.sd
            if ((st = run_q8_tiled(c, &md->gu[l].m, pf.xt, pf.xd, M, pf.part, stream, K_GEMM_TILED,
                                   LGX_TG_RANGES, I, pf.sq, pf.sd)) != LGX_OK ||
                (st = run_q8_tiled(c, &md->dn[l].m, pf.sq, pf.sd, M, pf.part, stream)) != LGX_OK)
                return st;
            continue;
        }
        if ((st = pf_product(md, md->gu[l], M, stream)) != LGX_OK) return st;
        lgx_swiglu_args sw{pf.part, tiled_groups(H), pf.xt, pf.xd, nullptr, M, I, 1};
        if ((st = launch(c, K_SWIGLU_QUANT, dim3(M, cdiv(I / 32, 32)), dim3(256), sw, stream)) != LGX_OK)
            return st;
        if ((st = pf_product(md, md->dn[l], M, stream)) != LGX_OK) return st;
    }
    lgx_advance_args av{md->seq_len, B, n, 1};
    return launch(c, K_ADVANCE, dim3(cdiv(B, 64)), dim3(64), av, stream);
}

// Sequences 0..B-1 about to grow by `add` positions: every new position
// must stay below max_seq (the kernels would clamp it and overwrite the last
// KV slot).  Checked on the host shadow, before any launch.
lgx_status check_growth(const lgx_model* md, int B, int64_t add) {
    for (int b = 0; b < B; ++b)
        if ((int64_t)md->len[b] + add > md->c.max_seq)
            return fail(LGX_OUT_OF_BOUNDS, "sequence %d: %d + %lld positions exceed max_seq %d", b,
                        md->len[b], (long long)add, md->c.max_seq);
    return LGX_OK;
}
void grow(lgx_model* md, int B, int64_t add) {
    for (int b = 0; b < B; ++b) md->len[b] += (int32_t)add;
}

constexpr size_t kGraphMax = 8;

// The recorded decode step for (B, tokens): captured on the model's private
// stream (nothing runs while recording) and instantiated once.  Every kernel
// argument is a model buffer, B or tokens, so a replay is the eager step.
lgx_status step_graph(lgx_model* md, int B, int32_t* tokens, hipGraphExec_t* out) {
    for (const lgx_model::StepGraph& g : md->graphs)
        if (g.B == B && g.tokens == tokens) {
            md->last_nr = g.last_nr;
            md->last_cert = g.last_cert;
            md->last_B = B;
            *out = g.exec;
            return LGX_OK;
        }
    if (!md->capture) LGX_HIP(hipStreamCreateWithFlags(&md->capture, hipStreamNonBlocking));
    if (md->graphs.size() >= kGraphMax) {
        LGX_HIP(hipDeviceSynchronize());   // the oldest recording may still be running
        (void)hipGraphExecDestroy(md->graphs.front().exec);
        md->graphs.erase(md->graphs.begin());
    }
    LGX_HIP(hipStreamBeginCapture(md->capture, hipStreamCaptureModeThreadLocal));
    lgx_status st = layers(md, B, tokens, 1, md->capture);
    if (st == LGX_OK) st = head(md, B, tokens, md->capture);
    hipGraph_t graph = nullptr;
    const hipError_t e = hipStreamEndCapture(md->capture, &graph);
    if (st != LGX_OK || e != hipSuccess) {
        if (graph) (void)hipGraphDestroy(graph);
        if (st != LGX_OK) return st;
        return fail(LGX_HIP_ERROR, "hipStreamEndCapture: %s", hipGetErrorString(e));
    }
    hipGraphExec_t exec = nullptr;
    const hipError_t ei = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (ei != hipSuccess)
        return fail(LGX_HIP_ERROR, "hipGraphInstantiate: %s", hipGetErrorString(ei));
    md->graphs.push_back({B, tokens, md->last_nr, md->last_cert, exec});
    *out = exec;
    return LGX_OK;
}

}  // namespace

namespace {

// Allocate the model for *cfg and fill its tensors from src (ctx entered,
// cfg checked).  `seed` also seeds the page-table permutation.
lgx_status model_build(lgx_ctx* c, const lgx_qwen_config* cfg, uint64_t seed, Source& src,
                       lgx_model** out) {
        lgx_status st;
        *out = nullptr;
        auto* m = new lgx_model();
        m->ctx = c;
        m->counted = true;
        c->live_models.fetch_add(1);
        m->c = *cfg;
        m->len.assign(cfg->max_batch, 0);
        m->seed = seed;
        const lgx_qwen_config& cf = *cfg;
        const int H = cf.hidden, I = cf.intermediate, d = cf.head_dim, hq = cf.n_heads,
                  hkv = cf.n_kv_heads, L = cf.n_layers, B = cf.max_batch;
        m->qkv_n = (hq + 2 * hkv) * d;
        m->maxp = (cf.max_seq + LGX_PAGE - 1) / LGX_PAGE;
        m->num_pages = B * m->maxp;
        m->nchunk = (cf.max_seq + LGX_ATTN_CHUNK - 1) / LGX_ATTN_CHUNK;
        auto done = [&](lgx_status s) {
            if (s != LGX_OK) delete m;
            else *out = m;
            return s;
        };
        // staging for the row-major upload of the largest Q8 matrix
        int64_t big = std::max<int64_t>({(int64_t)m->qkv_n * H, (int64_t)H * hq * d,
                                         (int64_t)2 * I * H, (int64_t)H * I,
                                         (!cf.tied_embedding || src.emb_is_q8()) ? (int64_t)cf.vocab * H : 0});
        int8_t* stage_q = nullptr;
        uint16_t* stage_d = nullptr;
        if ((st = dev_alloc(m, &stage_q, (size_t)big)) != LGX_OK) return done(st);
        if ((st = dev_alloc(m, &stage_d, (size_t)(big / 32))) != LGX_OK) return done(st);
        std::vector<int8_t> hq8;
        std::vector<uint16_t> hd16;
        m->qkv.resize(L);
        m->o.resize(L);
        m->gu.resize(L);
        m->dn.resize(L);
        m->bias.resize(L);
        m->kc.resize(L);
        m->vc.resize(L);
        const size_t kv_elems = (size_t)m->num_pages * hkv * LGX_PAGE * d;
        std::vector<float> hb(m->qkv_n);
        m->attn_norm.resize(L);
        m->ffn_norm.resize(L);
        std::vector<float> hn(H);
        // a host vector from the source into a new device buffer
        auto put_vec = [&](int which, int l, int n, float** dst) -> lgx_status {
            std::vector<float>& hv = which == V_BIAS ? hb : hn;
            lgx_status s2 = src.vec(which, l, n, hv.data());
            if (s2 != LGX_OK) return s2;
            if ((s2 = dev_alloc(m, dst, n)) != LGX_OK) return s2;
            LGX_HIP(hipMemcpy(*dst, hv.data(), (size_t)n * 4, hipMemcpyHostToDevice));
            return LGX_OK;
        };
        for (int l = 0; l < L; ++l) {
            if ((st = make_q8(m, src, W_QKV, l, m->qkv_n, H, &m->qkv[l], stage_q, stage_d, hq8, hd16)) ||
                (st = make_q8(m, src, W_O, l, H, hq * d, &m->o[l], stage_q, stage_d, hq8, hd16)) ||
                (st = make_q8(m, src, W_GU, l, 2 * I, H, &m->gu[l], stage_q, stage_d, hq8, hd16)) ||
                (st = make_q8(m, src, W_DN, l, H, I, &m->dn[l], stage_q, stage_d, hq8, hd16)))
                return done(st);
            if ((st = put_vec(V_BIAS, l, m->qkv_n, &m->bias[l])) ||
                (st = put_vec(V_ATTN_NORM, l, H, &m->attn_norm[l])) ||
                (st = put_vec(V_FFN_NORM, l, H, &m->ffn_norm[l])))
                return done(st);
            if ((st = dev_alloc(m, &m->kc[l], kv_elems)) != LGX_OK ||
                (st = dev_alloc(m, &m->vc[l], kv_elems)) != LGX_OK)
                return done(st);
            LGX_HIP(hipMemset(m->kc[l], 0, kv_elems * 2));
            LGX_HIP(hipMemset(m->vc[l], 0, kv_elems * 2));
        }
        if (!cf.tied_embedding &&
            (st = make_q8(m, src, W_LM, 0, cf.vocab, H, &m->lm, stage_q, stage_d, hq8, hd16)) != LGX_OK)
            return done(st);
        if (src.emb_is_q8()) {
            if (cf.vocab % 16)
                return done(fail(LGX_UNSUPPORTED, "Q8_0 embedding needs vocab %% 16 == 0 (got %d)", cf.vocab));
            if ((st = make_q8(m, src, W_EMB, 0, cf.vocab, H, &m->embq, stage_q, stage_d, hq8, hd16)) !=
                LGX_OK)
                return done(st);
            m->emb_q8 = true;
            if (cf.tied_embedding) m->lm = m->embq;
        }
        if ((st = put_vec(V_OUT_NORM, 0, H, &m->out_norm)) != LGX_OK) return done(st);
        hq8.clear();
        hq8.shrink_to_fit();
        if (!m->emb_q8) {
            std::vector<uint16_t> he((size_t)cf.vocab * H);
            if ((st = src.emb(cf.vocab, H, he.data())) != LGX_OK) return done(st);
            if ((st = dev_alloc(m, &m->emb, he.size())) != LGX_OK) return done(st);
            LGX_HIP(hipMemcpy(m->emb, he.data(), he.size() * 2, hipMemcpyHostToDevice));
        }
        if (f16_head(m)) {
            const int64_t nt = lgx_f16_t64_count(cf.vocab, H);
            if ((st = dev_alloc(m, &m->emb_t64, (size_t)nt)) != LGX_OK ||
                (st = dev_alloc(m, &m->xt, (size_t)cdiv(B, 16) * 16 * H)) != LGX_OK)
                return done(st);
            lgx_t64_args ta{m->emb, m->emb_t64, cf.vocab, H};
            if ((st = launch(c, K_REPACK_F16_T64, dim3(cdiv(nt / 8, 256)), dim3(256), ta, nullptr)) !=
                LGX_OK)
                return done(st);
            // the certified greedy lm_head: row constants, and the path only
            // for a finite embedding (a non-finite row has +inf constants)
            if (H % 64 == 0 && H <= LGX_LMC_MAXH && lm_cert_slices(cf.vocab) <= 1024) {
                if ((st = dev_alloc(m, &m->lm_rowc, (size_t)cf.vocab * 4)) != LGX_OK ||
                    (st = dev_alloc(m, &m->lm_summ,
                                    (size_t)std::min(B, LGX_LMC_MAXB) * lm_cert_slices(cf.vocab))) !=
                        LGX_OK ||
                    (st = launch_lm_rowconst(c, m->emb, cf.vocab, H, m->lm_rowc, nullptr)) != LGX_OK)
                    return done(st);
                std::vector<float> rc((size_t)cf.vocab * 4);
                LGX_HIP(hipMemcpy(rc.data(), m->lm_rowc, rc.size() * sizeof(float),
                                  hipMemcpyDeviceToHost));
                m->lm_cert_ok = std::all_of(rc.begin(), rc.end(), [](float f) { return std::isfinite(f); });
            }
        }
        {
            std::vector<float> ct((size_t)cf.max_seq * (d / 2)), stb(ct.size());
            for (int p = 0; p < cf.max_seq; ++p)
                for (int i = 0; i < d / 2; ++i) {
                    const double inv = std::pow(cf.rope_theta, -(2.0 * i) / (double)d);
                    const double ang = (double)p * inv;
                    ct[(size_t)p * (d / 2) + i] = (float)std::cos(ang);
                    stb[(size_t)p * (d / 2) + i] = (float)std::sin(ang);
                }
            if ((st = dev_alloc(m, &m->cos_t, ct.size())) != LGX_OK ||
                (st = dev_alloc(m, &m->sin_t, ct.size())) != LGX_OK)
                return done(st);
            LGX_HIP(hipMemcpy(m->cos_t, ct.data(), ct.size() * 4, hipMemcpyHostToDevice));
            LGX_HIP(hipMemcpy(m->sin_t, stb.data(), stb.size() * 4, hipMemcpyHostToDevice));
            std::vector<int32_t> pt(m->num_pages);
            lgxg::gen_permutation(seed, 4, pt.data(), m->num_pages);
            if ((st = dev_alloc(m, &m->page_table, pt.size())) != LGX_OK) return done(st);
            LGX_HIP(hipMemcpy(m->page_table, pt.data(), pt.size() * 4, hipMemcpyHostToDevice));
        }
        if ((st = dev_alloc(m, &m->seq_len, B)) != LGX_OK) return done(st);
        LGX_HIP(hipMemset(m->seq_len, 0, B * 4));
        const int kmax = std::max({H, I, hq * d});
        int64_t part = 0;
        auto upd = [&](int n, int k) {
            part = std::max<int64_t>(part, (int64_t)nranges_of(k) * B * n);
        };
        upd(m->qkv_n, H);
        upd(H, hq * d);
        upd(2 * I, H);
        upd(H, I);
        if (!f16_head(m)) upd(cf.vocab, H);
        if ((st = dev_alloc(m, &m->h, (size_t)B * H)) || (st = dev_alloc(m, &m->h2, (size_t)B * H)) ||
            (st = dev_alloc(m, &m->xn, (size_t)B * H)) ||
            (st = dev_alloc(m, &m->xq, (size_t)(B + 15) / 16 * 16 * kmax)) ||
            (st = dev_alloc(m, &m->xd, (size_t)B * kmax / 32)) ||
            (st = dev_alloc(m, &m->sq, (size_t)(B + 15) / 16 * 16 * I)) ||
            (st = dev_alloc(m, &m->sd, (size_t)B * I / 32)) ||
            (st = dev_alloc(m, &m->q, (size_t)B * hq * d)) || (st = dev_alloc(m, &m->part, (size_t)part)) ||
            (st = dev_alloc(m, &m->attn_part, (size_t)B * hq * m->nchunk * (d + 2))) ||
            (st = dev_alloc(m, &m->logits,
                            f16_head(m) ? (size_t)nranges_of(H) * B * cf.vocab : 1)) ||
            (st = dev_alloc(m, &m->cand, (size_t)B * argmax_slices(cf.vocab) * 2)) ||
            (cf.vocab <= 64 * LGX_ARGMAX_SLICE &&
             (st = dev_alloc(m, &m->scand, sample_cand_bytes(B, cf.vocab) / 8))))
            return done(st);
        m->hcur = m->h;
        // staging no longer needed
        LGX_HIP(hipDeviceSynchronize());
        for (void* p : {(void*)stage_q, (void*)stage_d}) {
            (void)hipFree(p);
            m->allocs.erase(std::find(m->allocs.begin(), m->allocs.end(), p));
        }
        return done(LGX_OK);
}

}  // namespace

extern "C" {

lgx_status lgx_model_create(lgx_ctx* c, const lgx_qwen_config* cfg, uint64_t seed,
                            lgx_model** out) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!cfg || !out) return fail(LGX_NULL_POINTER, "NULL config or out");
        *out = nullptr;
        if ((st = check_config(cfg)) != LGX_OK) return st;
        GenSource src(seed, cfg->emb_sigma);
        return model_build(c, cfg, seed, src, out);
    });
}

lgx_status lgx_gguf_config(const char* path, int32_t max_batch, int32_t max_seq,
                           lgx_qwen_config* out) {
    return guarded(__func__, [&]() -> lgx_status {
        g_has_error = false;
        if (!path || !out) return fail(LGX_NULL_POINTER, "NULL path or out");
        if (max_batch <= 0 || max_seq <= 0)
            return fail(LGX_INVALID_ARGUMENT, "max_batch %d, max_seq %d", max_batch, max_seq);
        lgxf::Gguf g;
        lgx_status st = g.open(path);
        if (st != LGX_OK) return st;
        return g.config(max_batch, max_seq, out);
    });
}

lgx_status lgx_model_load_gguf(lgx_ctx* c, const char* path, int32_t max_batch, int32_t max_seq,
                               lgx_model** out) {
    return guarded(__func__, [&]() -> lgx_status {
        lgx_status st = enter(c);
        if (st != LGX_OK) return st;
        if (!path || !out) return fail(LGX_NULL_POINTER, "NULL path or out");
        *out = nullptr;
        if (max_batch <= 0 || max_seq <= 0)
            return fail(LGX_INVALID_ARGUMENT, "max_batch %d, max_seq %d", max_batch, max_seq);
        lgxf::Gguf g;
        if ((st = g.open(path)) != LGX_OK) return st;
        lgx_qwen_config cfg{};
        if ((st = g.config(max_batch, max_seq, &cfg)) != LGX_OK) return st;
        if ((st = check_config(&cfg)) != LGX_OK) return st;
        GgufSource src(g, cfg);
        return model_build(c, &cfg, 0, src, out);
    });
}

lgx_status lgx_model_config(const lgx_model* m, lgx_qwen_config* out) {
    return guarded(__func__, [&]() -> lgx_status {
        if (!valid_model(m)) return fail(LGX_INVALID_HANDLE, "invalid lgx_model handle");
        if (!out) return fail(LGX_NULL_POINTER, "NULL out");
        *out = m->c;
        return LGX_OK;
    });
}

lgx_status lgx_model_destroy(lgx_model* m) {
    return guarded(__func__, [&]() -> lgx_status {
        if (!valid_model(m)) return fail(LGX_INVALID_HANDLE, "invalid lgx_model handle");
        (void)hipSetDevice(m->ctx->device);
        (void)hipDeviceSynchronize();
        m->magic = 0;
        delete m;
        return LGX_OK;
    });
}

lgx_status lgx_model_reset(lgx_model* m, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        if (!valid_model(m)) return fail(LGX_INVALID_HANDLE, "invalid lgx_model handle");
        lgx_status st = enter(m->ctx);
        if (st != LGX_OK) return st;
        lgx_advance_args a{m->seq_len, m->c.max_batch, 0, 0};
        if ((st = launch(m->ctx, K_ADVANCE, dim3(cdiv(m->c.max_batch, 64)), dim3(64), a, stream)) != LGX_OK)
            return st;
        std::fill(m->len.begin(), m->len.end(), 0);
        return LGX_OK;
    });
}

lgx_status lgx_qwen_decode_step(lgx_model* m, int32_t B, int32_t* tokens, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        if (!valid_model(m)) return fail(LGX_INVALID_HANDLE, "invalid lgx_model handle");
        lgx_status st = enter(m->ctx);
        if (st != LGX_OK) return st;
        if (!tokens) return fail(LGX_NULL_POINTER, "NULL tokens");
        if (B <= 0 || B > m->c.max_batch)
            return fail(LGX_OUT_OF_BOUNDS, "B = %d outside [1, %d]", B, m->c.max_batch);
        if ((st = check_growth(m, B, 1)) != LGX_OK) return st;
        if ((st = layers(m, B, tokens, 1, stream)) != LGX_OK || (st = head(m, B, tokens, stream)) != LGX_OK)
            return st;
        grow(m, B, 1);
        return LGX_OK;
    });
}

lgx_status lgx_qwen_generate(lgx_model* m, int32_t B, int32_t* tokens, int32_t nsteps,
                             int32_t* history, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        if (!valid_model(m)) return fail(LGX_INVALID_HANDLE, "invalid lgx_model handle");
        lgx_status st = enter(m->ctx);
        if (st != LGX_OK) return st;
        if (!tokens) return fail(LGX_NULL_POINTER, "NULL tokens");
        if (B <= 0 || B > m->c.max_batch)
            return fail(LGX_OUT_OF_BOUNDS, "B = %d outside [1, %d]", B, m->c.max_batch);
        if (nsteps < 0) return fail(LGX_INVALID_ARGUMENT, "nsteps = %d", nsteps);
        if (nsteps == 0) return LGX_OK;
        if ((st = check_growth(m, B, nsteps)) != LGX_OK) return st;
        hipGraphExec_t exec = nullptr;
        // per-kernel timing attaches events to each dispatch, which a graph
        // cannot hold: launch those steps eagerly
        if (!m->ctx->timing && (st = step_graph(m, B, tokens, &exec)) != LGX_OK) return st;
        for (int s = 0; s < nsteps; ++s) {
            if (exec) {
                LGX_HIP(hipGraphLaunch(exec, (hipStream_t)stream));
                if (trace_on())
                    trace_line("graph dev=%d replay B=%d step=%d stream=%p", m->ctx->device, B, s, stream);
            } else if ((st = layers(m, B, tokens, 1, stream)) != LGX_OK ||
                       (st = head(m, B, tokens, stream)) != LGX_OK) {
                return st;
            }
            grow(m, B, 1);
            if (history)
                LGX_HIP(hipMemcpyAsync(history + (int64_t)s * B, tokens, (size_t)B * 4,
                                       hipMemcpyDeviceToDevice, (hipStream_t)stream));
        }
        return LGX_OK;
    });
}

lgx_status lgx_qwen_prefill(lgx_model* m, int32_t B, int32_t P, const int32_t* prompt,
                            int32_t* next, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        if (!valid_model(m)) return fail(LGX_INVALID_HANDLE, "invalid lgx_model handle");
        lgx_status st = enter(m->ctx);
        if (st != LGX_OK) return st;
        if (!prompt || !next) return fail(LGX_NULL_POINTER, "NULL prompt or next");
        if (B <= 0 || B > m->c.max_batch || P <= 0)
            return fail(LGX_OUT_OF_BOUNDS, "B = %d, P = %d", B, P);
        if (!m->ctx->prefill_serial && P > 1) {
            // current lengths (one synchronising read): the prompt must fit,
            // and they bound each chunk's attention grid
            std::vector<int32_t> sl(B);
            LGX_HIP(hipMemcpyAsync(sl.data(), m->seq_len, (size_t)B * 4, hipMemcpyDeviceToHost,
                                   (hipStream_t)stream));
            LGX_HIP(hipStreamSynchronize((hipStream_t)stream));
            int smax = 0;
            for (int32_t v : sl) {
                if (v < 0) return fail(LGX_INVALID_ARGUMENT, "negative sequence length %d", v);
                smax = std::max(smax, (int)v);
            }
            if ((int64_t)smax + P > m->c.max_seq)
                return fail(LGX_OUT_OF_BOUNDS, "prompt of %d tokens after %d exceeds max_seq %d", P,
                            smax, m->c.max_seq);
            std::copy(sl.begin(), sl.end(), m->len.begin());
            if ((st = prefill_alloc(m)) != LGX_OK) return st;
            if (m->fast_prefill && (st = prefill_fast_alloc(m, stream)) != LGX_OK) return st;
            const int chunk = m->pf.chunk;
            for (int p0 = 0; p0 < P - 1; p0 += chunk) {
                const int n = std::min(chunk, P - 1 - p0);
                const int ncg = (int)cdiv(std::min(smax + p0 + n, m->c.max_seq), LGX_ATTN_CHUNK);
                st = m->fast_prefill ? prefill_chunk_fast(m, B, n, prompt + p0, P, stream)
                                     : prefill_chunk(m, B, n, prompt + p0, P, ncg, stream);
                if (st != LGX_OK) return st;
            }
            // the last position through the decode step: its logits give `next`
            if ((st = layers(m, B, prompt + (P - 1), P, stream)) != LGX_OK ||
                (st = head(m, B, next, stream)) != LGX_OK)
                return st;
            grow(m, B, P);
            return LGX_OK;
        }
        if ((st = check_growth(m, B, P)) != LGX_OK) return st;
        for (int p = 0; p < P; ++p) {
            if ((st = layers(m, B, prompt + p, P, stream)) != LGX_OK) return st;
            if (p + 1 < P) {
                lgx_advance_args a{m->seq_len, B, 1, 1};
                if ((st = launch(m->ctx, K_ADVANCE, dim3(cdiv(B, 64)), dim3(64), a, stream)) != LGX_OK)
                    return st;
            } else if ((st = head(m, B, next, stream)) != LGX_OK) {
                return st;
            }
        }
        grow(m, B, P);
        return LGX_OK;
    });
}

lgx_status lgx_model_tensor(lgx_model* m, int32_t layer, int32_t which, const void** dev,
                            size_t* bytes) {
    return guarded(__func__, [&]() -> lgx_status {
        if (!valid_model(m)) return fail(LGX_INVALID_HANDLE, "invalid lgx_model handle");
        if (!dev || !bytes) return fail(LGX_NULL_POINTER, "NULL out pointer");
        if (layer < 0 || layer >= m->c.n_layers) return fail(LGX_OUT_OF_BOUNDS, "layer %d", layer);
        const lgx_qwen_config& cf = m->c;
        auto q8 = [&](const DevQ8& w, bool scales) -> lgx_status {
            if (!w.qs) return fail(LGX_INVALID_ARGUMENT, "tensor %d not present", which);
            *dev = scales ? (const void*)w.d : (const void*)w.qs;
            *bytes = scales ? lgx_q8_scale_count(w.m.n, w.m.k) * 2 : (size_t)w.m.n * w.m.k;
            return LGX_OK;
        };
        switch (which) {
            case LGX_T_EMB:
                if (m->emb_q8) return fail(LGX_INVALID_ARGUMENT, "the embedding is Q8_0 (LGX_T_EMB_Q / _D)");
                *dev = m->emb;
                *bytes = (size_t)cf.vocab * cf.hidden * 2;
                return LGX_OK;
            case LGX_T_EMB_Q: return q8(m->embq, false);
            case LGX_T_EMB_D: return q8(m->embq, true);
            case LGX_T_LM_Q: return q8(m->lm, false);
            case LGX_T_LM_D: return q8(m->lm, true);
            case LGX_T_QKV_Q: return q8(m->qkv[layer], false);
            case LGX_T_QKV_D: return q8(m->qkv[layer], true);
            case LGX_T_O_Q: return q8(m->o[layer], false);
            case LGX_T_O_D: return q8(m->o[layer], true);
            case LGX_T_GU_Q: return q8(m->gu[layer], false);
            case LGX_T_GU_D: return q8(m->gu[layer], true);
            case LGX_T_DOWN_Q: return q8(m->dn[layer], false);
            case LGX_T_DOWN_D: return q8(m->dn[layer], true);
            case LGX_T_QKV_BIAS:
                *dev = m->bias[layer];
                *bytes = (size_t)m->qkv_n * 4;
                return LGX_OK;
            case LGX_T_K_PAGES:
                *dev = m->kc[layer];
                *bytes = (size_t)m->num_pages * cf.n_kv_heads * LGX_PAGE * cf.head_dim * 2;
                return LGX_OK;
            case LGX_T_V_PAGES:
                *dev = m->vc[layer];
                *bytes = (size_t)m->num_pages * cf.n_kv_heads * LGX_PAGE * cf.head_dim * 2;
                return LGX_OK;
            case LGX_T_PAGE_TABLE:
                *dev = m->page_table;
                *bytes = (size_t)m->num_pages * 4;
                return LGX_OK;
            case LGX_T_SEQ_LEN:
                *dev = m->seq_len;
                *bytes = (size_t)cf.max_batch * 4;
                return LGX_OK;
            case LGX_T_HIDDEN:
                *dev = m->xn;
                *bytes = (size_t)cf.max_batch * cf.hidden * 4;
                return LGX_OK;
            case LGX_T_ATTN_NORM:
            case LGX_T_FFN_NORM:
            case LGX_T_OUT_NORM:
                *dev = which == LGX_T_ATTN_NORM ? m->attn_norm[layer]
                       : which == LGX_T_FFN_NORM ? m->ffn_norm[layer] : m->out_norm;
                *bytes = (size_t)cf.hidden * 4;
                return LGX_OK;
            default:
                return fail(LGX_INVALID_ARGUMENT, "unknown tensor id %d", which);
        }
    });
}

lgx_status lgx_model_set_sampling(lgx_model* m, float temperature, int32_t top_k, float top_p,
                                  uint64_t seed) {
    return guarded(__func__, [&]() -> lgx_status {
        if (!valid_model(m)) return fail(LGX_INVALID_HANDLE, "invalid lgx_model handle");
        SampleParams sp;   // greedy
        if (temperature != 0.0f) {
            lgx_status st = sample_check(top_k, top_p, temperature, m->c.vocab, &sp);
            if (st != LGX_OK) return st;
            if (!m->scand) return fail(LGX_UNSUPPORTED, "no sampling buffer for this vocabulary");
            sp.seed = seed;
        }
        // recorded steps hold the old head: drop them (after the device is
        // done with any replay still in flight)
        LGX_HIP(hipSetDevice(m->ctx->device));
        if (!m->graphs.empty()) LGX_HIP(hipDeviceSynchronize());
        for (lgx_model::StepGraph& g : m->graphs) (void)hipGraphExecDestroy(g.exec);
        m->graphs.clear();
        m->samp = sp;
        return LGX_OK;
    });
}

lgx_status lgx_model_set_prefill_mode(lgx_model* m, int32_t mode) {
    return guarded(__func__, [&]() -> lgx_status {
        if (!valid_model(m)) return fail(LGX_INVALID_HANDLE, "invalid lgx_model handle");
        if (mode != LGX_PREFILL_EXACT && mode != LGX_PREFILL_FAST)
            return fail(LGX_INVALID_ARGUMENT, "prefill mode %d", mode);
        if (mode == LGX_PREFILL_EXACT || m->ctx->prefill_serial) {
            m->fast_prefill = mode == LGX_PREFILL_FAST;
            return LGX_OK;
        }
        // the fast mode's one-time work, here rather than in the first
        // prefill: buffers, every layer's weights in binary16, the GEMM
        // library and its plans for full chunks of max_batch sequences.  The
        // mode changes only once all of it has succeeded.
        lgx_status st = enter(m->ctx);
        if (st != LGX_OK) return st;
        if ((st = prefill_alloc(m)) != LGX_OK || (st = prefill_fast_alloc(m, nullptr)) != LGX_OK)
            return st;
        const lgx_qwen_config& cf = m->c;
        const int M = cf.max_batch * m->pf.chunk, H = cf.hidden, I = cf.intermediate,
                  hd = cf.n_heads * cf.head_dim;
        const uint16_t* w = m->pf.w16;
        if ((st = f16gemm_prepare(m->f16, w, m->pf.x16, m->pf.part, false, M, m->qkv_n, H, nullptr)) ||
            (st = f16gemm_prepare(m->f16, w, m->pf.x16, m->pf.part, false, M, H, hd, nullptr)) ||
            (st = f16gemm_prepare(m->f16, w, m->pf.x16, m->pf.gu16, true, M, 2 * I, H, nullptr)) ||
            (st = f16gemm_prepare(m->f16, w, m->pf.x16, m->pf.part, false, M, H, I, nullptr)))
            return st;
        LGX_HIP(hipDeviceSynchronize());
        m->fast_prefill = true;
        return LGX_OK;
    });
}

lgx_status lgx_qwen_logits(lgx_model* m, int32_t B, float* out, void* stream) {
    return guarded(__func__, [&]() -> lgx_status {
        if (!valid_model(m)) return fail(LGX_INVALID_HANDLE, "invalid lgx_model handle");
        lgx_status st = enter(m->ctx);
        if (st != LGX_OK) return st;
        if (!out) return fail(LGX_NULL_POINTER, "NULL out");
        if (B != m->last_B)
            return fail(LGX_INVALID_ARGUMENT, "B = %d, but the last step ran %d sequences", B,
                        m->last_B);
        const int64_t count = (int64_t)B * m->c.vocab;
        if (m->last_cert) {
            // the certified pick left no logits: the exact lm_head of the
            // step's final-norm rows (still in xt) first
            lgx_lmhead_args la{m->xt, m->emb_t64, m->logits, B, m->c.hidden, m->c.vocab};
            if ((st = launch(m->ctx, K_LM_HEAD_T64, dim3(cdiv(m->c.vocab, 64), cdiv(B, 16), 1),
                             dim3(64), la, stream)) != LGX_OK)
                return st;
        }
        lgx_combine_args ca{f16_head(m) ? m->logits : m->part, out, count, m->last_nr};
        return launch(m->ctx, K_COMBINE, dim3(cdiv(count, 256)), dim3(256), ca, stream);
    });
}

}  // extern "C"
