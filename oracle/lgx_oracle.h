/*
 * lgx_oracle.h -- CPU oracle for the lgx Q8 LLM-decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker, never the product:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The product (liblgx.so + lgx_kernels.hsaco) never links, loads or
 * falls back to it.
 *
 * Reference status.  The reference (LOGOS workspace 0.10.1) contains no
 * implementation of any function restated here: it has no CUDA back-end, no
 * tensor types and no LLM code (searches over the whole tree for cuda, gemv,
 * qwen, rmsnorm, softmax, fp16 ... find nothing).  The arithmetic therefore
 * follows the public definitions (GGML Q8_0 block format, Qwen2 decoder
 * architecture) and the canonical reduction schedules written out below.
 * What the reference does contribute are conventions, cited where used:
 *   - SplitMix64 as the portable seeded generator
 *     (crates/logicaffeine_runtime/src/seed.rs:15-38);
 *   - "no implicit FMA, no reassociation" in the oracle tier
 *     (crates/logicaffeine_tests/tests/jit_float_codegen.rs:13-18,
 *      crates/logicaffeine_forge/src/vectorize.rs:9-12): this file is built
 *     with -ffp-contract=off and every fused multiply-add is an explicit
 *     fmaf() at the place the device kernels use one.
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   f32<->f16        exhaustive 2^16 decode vs numpy, RNE encode vs numpy on
 *                    2^20 random + all boundary values
 *   expf             |rel err| < 2 ulp vs numpy float64 exp over the domain;
 *                    exp(0) == 1 exactly; monotone; limits
 *   generators       SplitMix64 published vectors for seed 0 / 1234567; moments
 *   quantize_q8_0    closed forms (ramp, absmax -> +-127, zero block),
 *                    numpy-f64 fixture
 *   q8 block dots    brute-force int64 numpy (exact)
 *   q8 gemv f32      one-hot x (exact column), linearity, numpy-f64 fixture
 *   q8 gemm          per-row equality with the M=1 path (batch invariance),
 *                    numpy-f64 fixture within 1e-5 rel, one-hot closed form
 *   repack t16/s16   round trip + explicit index formula on a tiny case
 *   gqa decode attn  numpy float64 softmax attention on the golden fixture
 *                    (tests/test_oracle_attn.py) within 2e-3, a head-swap
 *                    mutant rejected; single token -> v0 exactly; equal
 *                    scores -> mean; constant V -> V; page-order invariance
 *   rmsnorm          numpy float64 within 3e-6 rel; scale invariance;
 *                    constant row -> sign (the halving-sum order itself is
 *                    checked by tests/test_oracle_attn.py)
 *   rope             norm preservation, position 0 identity, the rotate-half
 *                    pair formula, relative-position property
 *                    <R_p q, R_s k> = f(p - s)
 *   swiglu / silu    silu(0) = 0, large-|g| asymptotes, numpy float64
 *   argmax           first maximum, NaN skipped, all-NaN -> 0, -0 == +0
 *   lm_head_f16      one-hot rows select embedding columns exactly; numpy
 *                    float64 within the chain's error bound
 *   model step       a numpy float64 forward of the same Qwen2 decoder
 *                    (tests/test_oracle_model.py) agrees within 1e-3 of the
 *                    logit scale, an interleaved-RoPE mutant does not; batch
 *                    and slot invariance
 *   model prefill    equal bit for bit (tokens, logits, hidden rows, every
 *                    cached K/V row) to P calls of the model step, over
 *                    several chunks, ragged start lengths and 256-token
 *                    attention-chunk boundaries (tests/test_oracle_model.py)
 *   load_kv          round trip with orc_model_kv; decoding after a loaded
 *                    cache equals decoding after the prefill that made it
 *   sample           top_k = 1 and a tiny top_p give the argmax; equal
 *                    logits pick only the lowest top_k indices, uniformly;
 *                    NaN never drawn; the frequencies of 200k seeded draws
 *                    match a float64 numpy statement of the top-k / nucleus
 *                    distribution (tests/test_oracle_sample.py), and
 *                    SplitMix64 draws follow the published vectors
 * None of these is "parity unpinned": each has the checks above, chosen so
 * that a dropped term, wrong sign or transposed operand fails one of them.
 */
#ifndef LGX_ORACLE_H
#define LGX_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Blocks (of 32) per canonical accumulation range of a Q8 dot product. */
#define ORC_Q8_RANGE_BLOCKS 32

/* ---- scalar formats ---- */
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
void orc_f32_to_f16_array(const float* x, uint16_t* h, int64_t n);
void orc_f16_to_f32_array(const uint16_t* h, float* x, int64_t n);
float orc_expf(float x);
float orc_silu(float x);
void orc_expf_array(const float* x, float* y, int64_t n);

/* ---- seeded generators (SplitMix64 streams) ---- */
uint64_t orc_stream_base(uint64_t seed, uint64_t stream);
void orc_gen_u64(uint64_t seed, uint64_t stream, uint64_t* out, int64_t n);
void orc_splitmix64_seq(uint64_t state, uint64_t* out, int64_t n);
void orc_gen_i8(uint64_t seed, uint64_t stream, int8_t* out, int64_t n);
void orc_gen_normal_f32(uint64_t seed, uint64_t stream, double sigma, float* out, int64_t n);
void orc_gen_normal_f16(uint64_t seed, uint64_t stream, double sigma, uint16_t* out, int64_t n);
void orc_gen_q8_scales(uint64_t seed, uint64_t stream, uint16_t* out, int64_t n);
void orc_gen_below_i32(uint64_t seed, uint64_t stream, uint32_t bound, int32_t* out, int64_t n);

/* ---- Q8_0 ---- */
void orc_quantize_q8_0(const float* x, int64_t m, int32_t k, int8_t* qs, uint16_t* d);
void orc_q8_repack_t16(const int8_t* qs, int32_t n, int32_t k, int8_t* out);
void orc_q8_unpack_t16(const int8_t* t16, int32_t n, int32_t k, int8_t* qs);
int64_t orc_q8_s16_count(int32_t n, int32_t k);
void orc_q8_repack_s16(const uint16_t* d, int32_t n, int32_t k, uint16_t* out);
void orc_q8_gemv_f32(const int8_t* qs, const uint16_t* d, int32_t n, int32_t k,
                     const float* x, float* y);
void orc_q8_blockdots(const int8_t* qs, int32_t n, int32_t k, const int8_t* xq,
                      int32_t* s);
void orc_q8_gemm(const int8_t* qs, const uint16_t* d, int32_t n, int32_t k,
                 const int8_t* xq, const uint16_t* xd, int32_t m, float* y);
float orc_tree_sum(float* p, int32_t g);

/* ---- paged KV cache + GQA decode attention ---- */
float orc_halving_sum(float* p, int32_t n);
void orc_gqa_decode_attn(const float* q, const uint16_t* kpages, const uint16_t* vpages,
                         const int32_t* page_table, const int32_t* seq_len, int32_t B,
                         int32_t hq, int32_t hkv, int32_t d, int32_t maxp, float scale,
                         float* out);
void orc_gen_page_table(uint64_t seed, uint64_t stream, int32_t B, int32_t maxp, int32_t* pt);

/* ---- decode-step glue ---- */
void orc_rmsnorm(const float* x, const float* w, int32_t m, int32_t h, float eps, float* y);
void orc_rope_tables(int32_t max_seq, int32_t d, double theta, float* cos_t, float* sin_t);
void orc_rope(float* x, int32_t nheads, int32_t d, const float* cos_row, const float* sin_row);
void orc_swiglu(const float* gu, int32_t m, int32_t inter, float* a);
int32_t orc_argmax(const float* x, int32_t n);
void orc_lm_head_f16(const float* x, int32_t m, const uint16_t* E, int32_t V, int32_t h,
                     float* logits);

/* ---- random-init Qwen2-shaped Q8_0 model ---- */
typedef struct orc_qwen_config {
    int32_t n_layers, hidden, inter, n_heads, n_kv, head_dim, vocab;
    int32_t tied;              /* 1: logits from the binary16 embedding */
    int32_t max_batch, max_seq;
    float eps;
    double theta;
    double emb_sigma;          /* embedding N(0, emb_sigma) */
} orc_qwen_config;
typedef struct orc_model orc_model;
orc_model* orc_model_create(const orc_qwen_config* cfg, uint64_t seed);
void orc_model_destroy(orc_model* m);
int32_t orc_model_seq_len(const orc_model* m, int32_t slot);
const void* orc_model_tensor(const orc_model* m, int32_t layer, int32_t which);
void orc_model_kv(const orc_model* m, int32_t layer, int32_t kv, int32_t b, int32_t n,
                  uint16_t* out);
void orc_model_step(orc_model* m, int32_t nseq, const int32_t* slots, const int32_t* tokens,
                    int32_t* next, float* hidden_out, float* logits_out);
void orc_model_prefill(orc_model* m, int32_t nseq, const int32_t* slots, int32_t P,
                       const int32_t* tokens, int32_t* next, float* hidden_out,
                       float* logits_out);
void orc_model_load_kv(orc_model* m, int32_t layer, int32_t kv, int32_t b, int32_t n,
                       const uint16_t* rows);
void orc_model_set_seq_len(orc_model* m, int32_t slot, int32_t len);
void orc_model_set_sampling(orc_model* m, float temperature, int32_t top_k, float top_p,
                            uint64_t seed);
void orc_model_set_tensor(orc_model* m, int32_t layer, int32_t which, const void* data);
void orc_model_set_emb_q8(orc_model* m, const int8_t* qs, const uint16_t* d);
void orc_set_threads(int32_t n);
int32_t orc_max_threads(void);

/* ---- seeded top-k / top-p sampling (the rule of lgx_sample) ---- */
int32_t orc_sample_row(const float* logits, int32_t vocab, int32_t top_k, float top_p,
                       float temperature, uint64_t seed, int32_t stream, int32_t pos);
void orc_sample(const float* logits, int32_t m, int32_t vocab, int32_t top_k, float top_p,
                float temperature, uint64_t seed, const int32_t* streams, const int32_t* pos,
                int32_t* out);

#ifdef __cplusplus
}
#endif
#endif
