/*
 * lgx_oracle.c -- CPU restatement of the lgx hot path (TEST INFRASTRUCTURE).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
 * this file, as the checker.  Built with -ffp-contract=off: every fused
 * multiply-add below is an explicit fmaf() standing where the device kernel
 * issues v_fma_f32, and every other float operation is a separately rounded
 * IEEE-754 binary32 operation, so a device kernel that follows the same
 * schedule produces the same bits.
 *
 * The reference contains no implementation of these functions (no GPU
 * back-end, no tensor code); see lgx_oracle.h for the conventions taken from
 * it and for what pins each function.
 */
#include "lgx_oracle.h"

#include <omp.h>

#include <math.h>
#ifdef __AVX2__
#include <immintrin.h>
#endif
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------ */
/* IEEE binary16 <-> binary32                                          */
/* ------------------------------------------------------------------ */

/* Round-to-nearest-even binary32 -> binary16 (IEEE 754-2008 convertFormat).
 * Overflow (|x| >= 65520) gives +-inf; NaN gives the quiet NaN 0x7e00. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {                 /* below 2^-14: binary16 subnormal */
        if (ax <= 0x33000000u) return sign; /* <= 2^-25 rounds (ties-to-even) to 0 */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t sh = 126u - e;             /* value / 2^-24 = m >> sh */
        uint32_t h = (m + (1u << (sh - 1)) - 1u + ((m >> sh) & 1u)) >> sh;
        return (uint16_t)(sign | h);
    }
    ax -= 0x38000000u;                      /* rebias exponent 127 -> 15 */
    ax += 0x0fffu + ((ax >> 13) & 1u);
    return (uint16_t)(sign | (ax >> 13));
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t m = (uint32_t)h & 0x3ffu;
    if (e == 0x1fu) return u2f(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        if (m == 0) return u2f(sign);
        /* subnormal: m * 2^-24, exact in binary32 */
        float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

void orc_f32_to_f16_array(const float* x, uint16_t* h, int64_t n) {
    for (int64_t i = 0; i < n; ++i) h[i] = orc_f32_to_f16(x[i]);
}

void orc_f16_to_f32_array(const uint16_t* h, float* x, int64_t n) {
    for (int64_t i = 0; i < n; ++i) x[i] = orc_f16_to_f32(h[i]);
}

/* ------------------------------------------------------------------ */
/* Canonical exp (binary32)                                            */
/* ------------------------------------------------------------------ */
/* Cody-Waite reduction x = n*ln2 + r with n = rint(x*log2(e)) (rint by the
 * 1.5*2^23 magic constant under round-to-nearest-even), ln2 split into
 * ln2_hi = 0x3f317200 (exact product with n) and ln2_lo; then the degree-7
 * Taylor polynomial of e^r on |r| <= ln2/2 in Horner form with fmaf, and
 * scaling by 2^n through the exponent field.  x < -87.33 returns +0 (no
 * subnormal results), x > 88.72 returns +inf.  exp(0) == 1 exactly. */
float orc_expf(float x) {
    if (x != x) return x;
    if (x > 88.72f) return INFINITY;
    if (x < -87.33f) return 0.0f;
    float t = x * 1.44269504088896341f;
    float nf = (t + 12582912.0f) - 12582912.0f;
    float r = fmaf(-nf, 0.693145751953125f, x);
    r = fmaf(-nf, 1.42860682030941723e-06f, r);
    float p = 1.98412698412698413e-04f;
    p = fmaf(p, r, 1.38888888888888889e-03f);
    p = fmaf(p, r, 8.33333333333333333e-03f);
    p = fmaf(p, r, 4.16666666666666667e-02f);
    p = fmaf(p, r, 1.66666666666666667e-01f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int n = (int)nf;
    if (n > 127) { p = p * 2.0f; n -= 1; }
    return p * u2f((uint32_t)(n + 127) << 23);
}

/* silu(g) = g / (1 + exp(-g)), each step a separately rounded operation. */
float orc_silu(float g) {
    float e = orc_expf(-g);
    float den = 1.0f + e;
    return g / den;
}

void orc_expf_array(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_expf(x[i]);
}

/* ------------------------------------------------------------------ */
/* Seeded generators                                                   */
/* ------------------------------------------------------------------ */
/* SplitMix64 (crates/logicaffeine_runtime/src/seed.rs:30-38): state +=
 * 0x9E3779B97F4A7C15 then the xor-shift-multiply finaliser.  Output i of a
 * sequence started at state s is mix(s + (i+1)*gamma), so every element of a
 * stream is addressable by its index. */
#define SM_GAMMA 0x9E3779B97F4A7C15ull

static inline uint64_t sm_mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void orc_splitmix64_seq(uint64_t state, uint64_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        state += SM_GAMMA;
        out[i] = sm_mix(state);
    }
}

/* Starting state of stream `stream` under `seed`. */
uint64_t orc_stream_base(uint64_t seed, uint64_t stream) {
    return sm_mix(seed + SM_GAMMA) ^ sm_mix((stream + 1ull) * 0xD1B54A32D192ED03ull);
}

static inline uint64_t stream_at(uint64_t base, uint64_t i) {
    return sm_mix(base + (i + 1ull) * SM_GAMMA);
}

void orc_gen_u64(uint64_t seed, uint64_t stream, uint64_t* out, int64_t n) {
    uint64_t b = orc_stream_base(seed, stream);
    for (int64_t i = 0; i < n; ++i) out[i] = stream_at(b, (uint64_t)i);
}

/* Uniform integer in [0, bound) by the multiply-high map of the top 32 bits
 * (bias <= bound / 2^32). */
static inline uint32_t below32(uint64_t u, uint32_t bound) {
    return (uint32_t)(((u >> 32) * (uint64_t)bound) >> 32);
}

/* int8 uniform on [-127, 127]. */
void orc_gen_i8(uint64_t seed, uint64_t stream, int8_t* out, int64_t n) {
    uint64_t b = orc_stream_base(seed, stream);
    for (int64_t i = 0; i < n; ++i) out[i] = (int8_t)((int32_t)below32(stream_at(b, (uint64_t)i), 255u) - 127);
}

void orc_gen_below_i32(uint64_t seed, uint64_t stream, uint32_t bound, int32_t* out, int64_t n) {
    uint64_t b = orc_stream_base(seed, stream);
    for (int64_t i = 0; i < n; ++i) out[i] = (int32_t)below32(stream_at(b, (uint64_t)i), bound);
}

/* Standard normal for element i: Box-Muller on draws 2i and 2i+1 in binary64,
 * u1 in (0,1], u2 in [0,1). */
static inline double normal_at(uint64_t base, uint64_t i) {
    uint64_t a = stream_at(base, 2ull * i);
    uint64_t c = stream_at(base, 2ull * i + 1ull);
    double u1 = (double)((a >> 11) + 1ull) * 0x1.0p-53;
    double u2 = (double)(c >> 11) * 0x1.0p-53;
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

void orc_gen_normal_f32(uint64_t seed, uint64_t stream, double sigma, float* out, int64_t n) {
    uint64_t b = orc_stream_base(seed, stream);
    for (int64_t i = 0; i < n; ++i) out[i] = (float)(sigma * normal_at(b, (uint64_t)i));
}

void orc_gen_normal_f16(uint64_t seed, uint64_t stream, double sigma, uint16_t* out, int64_t n) {
    uint64_t b = orc_stream_base(seed, stream);
    for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_f16((float)(sigma * normal_at(b, (uint64_t)i)));
}

/* Weight block scales: d = |N(0, 0.02)| / 127, rounded to binary32 then to
 * binary16 (RNE). */
void orc_gen_q8_scales(uint64_t seed, uint64_t stream, uint16_t* out, int64_t n) {
    uint64_t b = orc_stream_base(seed, stream);
    for (int64_t i = 0; i < n; ++i) {
        double z = fabs(0.02 * normal_at(b, (uint64_t)i)) / 127.0;
        out[i] = orc_f32_to_f16((float)z);
    }
}

/* ------------------------------------------------------------------ */
/* Q8_0                                                                */
/* ------------------------------------------------------------------ */
/* Activation quantisation, GGML Q8_0 style: per 32-block amax = max|x|,
 * d = amax / 127 (binary32 division), id = d != 0 ? 1/d : 0, q = round half
 * away from zero of x*id clamped to [-127, 127]; the stored scale is
 * binary16(d) (RNE) while q uses the binary32 id. */
void orc_quantize_q8_0(const float* x, int64_t m, int32_t k, int8_t* qs, uint16_t* d) {
    int32_t nb = k / 32;
    /* blocks are independent: rows split over the threads */
#pragma omp parallel for schedule(static) if (m * (int64_t)k >= 65536)
    for (int64_t r = 0; r < m; ++r) {
        for (int32_t b = 0; b < nb; ++b) {
            const float* xb = x + r * k + (int64_t)b * 32;
            float amax = 0.0f;
            for (int i = 0; i < 32; ++i) {
                float a = fabsf(xb[i]);
                if (a > amax) amax = a;
            }
            float dd = amax / 127.0f;
            float id = dd != 0.0f ? 1.0f / dd : 0.0f;
            d[r * nb + b] = orc_f32_to_f16(dd);
            for (int i = 0; i < 32; ++i) {
                float v = roundf(xb[i] * id);
                if (v > 127.0f) v = 127.0f;
                if (v < -127.0f) v = -127.0f;
                qs[r * k + (int64_t)b * 32 + i] = (int8_t)v;
            }
        }
    }
}

/* Device tile layout "T16": 16 rows x 2 blocks (1 KiB) per unit, unit index
 * (row_tile * (k/64) + block_pair); inside a unit lane l = (row%16) + 16*c
 * owns 16 bytes: bytes [0,8) are k = 64p + 8c + j of block 2p and bytes
 * [8,16) the same offsets of block 2p+1.  This is the B-operand order of the
 * 16x16x32 int8 MFMA, so one 128-bit load per lane feeds two MFMAs. */
static inline int64_t t16_index(int32_t row, int32_t kk, int32_t k) {
    int32_t t = row >> 4, r = row & 15;
    int32_t p = kk >> 6, w = kk & 63;
    int32_t hi = w >> 5, c = (w & 31) >> 3, j = w & 7;
    int32_t lane = r + 16 * c;
    return ((int64_t)t * (k >> 6) + p) * 1024 + lane * 16 + hi * 8 + j;
}

void orc_q8_repack_t16(const int8_t* qs, int32_t n, int32_t k, int8_t* out) {
    for (int32_t row = 0; row < n; ++row)
        for (int32_t kk = 0; kk < k; ++kk)
            out[t16_index(row, kk, k)] = qs[(int64_t)row * k + kk];
}

/* Device scale layout "S16": per row tile and half-range (16 blocks) the
 * 16 rows x 16 scales are contiguous, row-major: element
 * ((tile * nhalf + b/16) * 16 + row%16) * 16 + b%16, nhalf = ceil(k/512);
 * entries past k/32 are zero. */
int64_t orc_q8_s16_count(int32_t n, int32_t k) {
    return (int64_t)(n / 16) * ((k + 511) / 512) * 256;
}

void orc_q8_repack_s16(const uint16_t* d, int32_t n, int32_t k, uint16_t* out) {
    int32_t nb = k / 32, nh = (k + 511) / 512;
    memset(out, 0, (size_t)orc_q8_s16_count(n, k) * 2);
    for (int32_t row = 0; row < n; ++row)
        for (int32_t b = 0; b < nb; ++b)
            out[(((int64_t)(row >> 4) * nh + (b >> 4)) * 16 + (row & 15)) * 16 + (b & 15)] =
                d[(int64_t)row * nb + b];
}

void orc_q8_unpack_t16(const int8_t* t16, int32_t n, int32_t k, int8_t* qs) {
    for (int32_t row = 0; row < n; ++row)
        for (int32_t kk = 0; kk < k; ++kk)
            qs[(int64_t)row * k + kk] = t16[t16_index(row, kk, k)];
}

/* y = W x with binary32 x.  Tolerance-checked path (1e-3 rel / 1e-4 abs),
 * so the oracle accumulates in binary64 for accuracy. */
void orc_q8_gemv_f32(const int8_t* qs, const uint16_t* d, int32_t n, int32_t k,
                     const float* x, float* y) {
    int32_t nb = k / 32;
#pragma omp parallel for schedule(static)
    for (int32_t row = 0; row < n; ++row) {
        double acc = 0.0;
        for (int32_t b = 0; b < nb; ++b) {
            const int8_t* q = qs + (int64_t)row * k + (int64_t)b * 32;
            const float* xb = x + (int64_t)b * 32;
            double s = 0.0;
            for (int i = 0; i < 32; ++i) s += (double)q[i] * (double)xb[i];
            acc += (double)orc_f16_to_f32(d[(int64_t)row * nb + b]) * s;
        }
        y[row] = (float)acc;
    }
}

/* orc_f16_to_f32 of every binary16 pattern, for the hot loops (filled once
 * from orc_f16_to_f32 itself, so a lookup returns exactly its bits). */
static float g_f16tab[65536];
__attribute__((constructor)) static void fill_f16tab(void) {
    for (uint32_t h = 0; h < 65536u; ++h) g_f16tab[h] = orc_f16_to_f32((uint16_t)h);
}
static inline float f16f(uint16_t h) { return g_f16tab[h]; }

static inline int32_t block_dot(const int8_t* restrict a, const int8_t* restrict b) {
#ifdef __AVX2__
    /* the same exact integer sum: int8 -> int16, pairwise products summed
     * into int32 lanes (|partial| <= 4 * 127^2, no overflow), then the lanes */
    const __m256i a16lo = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)a));
    const __m256i a16hi = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)(a + 16)));
    const __m256i b16lo = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)b));
    const __m256i b16hi = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)(b + 16)));
    __m256i p = _mm256_add_epi32(_mm256_madd_epi16(a16lo, b16lo), _mm256_madd_epi16(a16hi, b16hi));
    __m128i q = _mm_add_epi32(_mm256_castsi256_si128(p), _mm256_extracti128_si256(p, 1));
    q = _mm_add_epi32(q, _mm_shuffle_epi32(q, 0x4e));
    q = _mm_add_epi32(q, _mm_shuffle_epi32(q, 0xb1));
    return _mm_cvtsi128_si32(q);
#else
    int32_t s = 0;
    for (int i = 0; i < 32; ++i) s += (int32_t)a[i] * (int32_t)b[i];
    return s;
#endif
}

/* Exact int32 block dot products s[row][b] of W with a Q8_0 activation. */
void orc_q8_blockdots(const int8_t* qs, int32_t n, int32_t k, const int8_t* xq, int32_t* s) {
    int32_t nb = k / 32;
#pragma omp parallel for schedule(static)
    for (int32_t row = 0; row < n; ++row)
        for (int32_t b = 0; b < nb; ++b)
            s[(int64_t)row * nb + b] = block_dot(qs + (int64_t)row * k + (int64_t)b * 32, xq + (int64_t)b * 32);
}

/* Pairwise tree with doubling stride: for s = 1, 2, 4, ...: p[i] += p[i+s]
 * for i = 0, 2s, 4s, ... with i+s < g.  Returns p[0]; modifies p. */
float orc_tree_sum(float* p, int32_t g) {
    for (int32_t s = 1; s < g; s <<= 1)
        for (int32_t i = 0; i + s < g; i += 2 * s) p[i] = p[i] + p[i + s];
    return g > 0 ? p[0] : 0.0f;
}

#if defined(__x86_64__) && defined(__GNUC__)
/* AVX-512 VNNI form of orc_q8_gemm for 16+ activation rows (chosen at run
 * time when the host has it): the same exact int32 block dots and the same
 * binary32 chain and tree per output, with 16 activation rows in the 16
 * lanes of a vector.  vpdpbusd multiplies unsigned by signed bytes, so the
 * activation bytes enter as x + 128 (x ^ 0x80) and each block dot starts
 * from -128 * sum(w) of its weight block: sum (x + 128) w - 128 sum w =
 * sum x w, exact in int32 (no saturation: |sum (x + 128) w| <= 32*255*128).
 * Per lane the chain is acc = fmaf((float)s_b, dw_b * dx_b, acc), b
 * ascending inside a range, then orc_tree_sum's pairwise tree over the
 * ranges -- the scalar path's operations on the same values. */
#define ORC_VNNI_ROWS 4       /* weight rows sharing one load of activations */
#define ORC_VNNI_GROUPS 16    /* 16-row activation groups per cache tile */
__attribute__((target("avx512f,avx512bw,avx512vnni")))
static void q8_gemm_vnni(const int8_t* qs, const uint16_t* d, int32_t n, int32_t k,
                         const int8_t* xq, const uint16_t* xd, int32_t m, float* y) {
    const int32_t nb = k / 32, g = (nb + ORC_Q8_RANGE_BLOCKS - 1) / ORC_Q8_RANGE_BLOCKS;
    const int32_t ng = (m + 15) / 16;
    /* activations as [group][block][dword j][16 lanes] of x ^ 0x80, scales
     * as [group][block][16 lanes] binary32; rows past m hold x = 0, d = 0 */
    uint32_t* xu = (uint32_t*)aligned_alloc(64, (size_t)ng * nb * 8 * 64);
    float* dxf = (float*)aligned_alloc(64, (size_t)ng * nb * 64);
    if (!xu || !dxf) abort();
#pragma omp parallel for schedule(static)
    for (int64_t gb = 0; gb < (int64_t)ng * nb; ++gb) {
        const int32_t grp = (int32_t)(gb / nb), b = (int32_t)(gb % nb);
        for (int32_t lane = 0; lane < 16; ++lane) {
            const int32_t row = grp * 16 + lane;
            for (int32_t j = 0; j < 8; ++j) {
                uint32_t v = 0u;
                if (row < m) memcpy(&v, xq + (int64_t)row * k + (int64_t)b * 32 + 4 * j, 4);
                xu[(gb * 8 + j) * 16 + lane] = v ^ 0x80808080u;
            }
            dxf[gb * 16 + lane] = row < m ? f16f(xd[(int64_t)row * nb + b]) : 0.0f;
        }
    }
    const int32_t nrb = (n + ORC_VNNI_ROWS - 1) / ORC_VNNI_ROWS;
#pragma omp parallel
    {
        float* part = (float*)aligned_alloc(64, (size_t)ORC_VNNI_ROWS * g * 64);
        int32_t* wc = (int32_t*)malloc(sizeof(int32_t) * ORC_VNNI_ROWS * nb);
        float* dw = (float*)malloc(sizeof(float) * ORC_VNNI_ROWS * nb);
        if (!part || !wc || !dw) abort();
        for (int32_t g0 = 0; g0 < ng; g0 += ORC_VNNI_GROUPS) {
            const int32_t g1 = g0 + ORC_VNNI_GROUPS < ng ? g0 + ORC_VNNI_GROUPS : ng;
#pragma omp for schedule(dynamic, 4)
            for (int32_t rb = 0; rb < nrb; ++rb) {
                const int8_t* w[ORC_VNNI_ROWS];
                for (int32_t u = 0; u < ORC_VNNI_ROWS; ++u) {
                    int32_t row = rb * ORC_VNNI_ROWS + u;
                    if (row > n - 1) row = n - 1;       /* tail: a repeated row, not stored */
                    w[u] = qs + (int64_t)row * k;
                    for (int32_t b = 0; b < nb; ++b) {
                        int32_t s = 0;
                        for (int32_t i = 0; i < 32; ++i) s += w[u][b * 32 + i];
                        wc[u * nb + b] = -128 * s;
                        dw[u * nb + b] = f16f(d[(int64_t)row * nb + b]);
                    }
                }
                for (int32_t grp = g0; grp < g1; ++grp) {
                    for (int32_t r = 0; r < g; ++r) {
                        __m512 acc[ORC_VNNI_ROWS];
                        for (int32_t u = 0; u < ORC_VNNI_ROWS; ++u) acc[u] = _mm512_setzero_ps();
                        int32_t b1 = (r + 1) * ORC_Q8_RANGE_BLOCKS;
                        if (b1 > nb) b1 = nb;
                        for (int32_t b = r * ORC_Q8_RANGE_BLOCKS; b < b1; ++b) {
                            const int64_t gb = (int64_t)grp * nb + b;
                            const __m512i* xv = (const __m512i*)(xu + gb * 8 * 16);
                            const __m512 dx = _mm512_load_ps(dxf + gb * 16);
                            for (int32_t u = 0; u < ORC_VNNI_ROWS; ++u) {
                                const int32_t* wb = (const int32_t*)(w[u] + (int64_t)b * 32);
                                __m512i s = _mm512_set1_epi32(wc[u * nb + b]);
                                for (int32_t j = 0; j < 8; ++j) {
                                    int32_t wd;
                                    memcpy(&wd, wb + j, 4);
                                    s = _mm512_dpbusd_epi32(s, _mm512_load_si512(xv + j),
                                                            _mm512_set1_epi32(wd));
                                }
                                const __m512 dd = _mm512_mul_ps(_mm512_set1_ps(dw[u * nb + b]), dx);
                                acc[u] = _mm512_fmadd_ps(_mm512_cvtepi32_ps(s), dd, acc[u]);
                            }
                        }
                        for (int32_t u = 0; u < ORC_VNNI_ROWS; ++u)
                            _mm512_store_ps(part + ((int64_t)u * g + r) * 16, acc[u]);
                    }
                    for (int32_t u = 0; u < ORC_VNNI_ROWS; ++u) {
                        const int32_t row = rb * ORC_VNNI_ROWS + u;
                        if (row >= n) break;
                        float* p = part + (int64_t)u * g * 16;
                        /* orc_tree_sum over the ranges, lane by lane */
                        for (int32_t s = 1; s < g; s <<= 1)
                            for (int32_t i = 0; i + s < g; i += 2 * s)
                                _mm512_store_ps(p + i * 16, _mm512_add_ps(_mm512_load_ps(p + i * 16),
                                                                          _mm512_load_ps(p + (i + s) * 16)));
                        for (int32_t lane = 0; lane < 16; ++lane) {
                            const int32_t mi = grp * 16 + lane;
                            if (mi < m) y[(int64_t)mi * n + row] = p[lane];
                        }
                    }
                }
            }
        }
        free(part); free(wc); free(dw);
    }
    free(xu); free(dxf);
}

static int vnni_ok(void) {
    static int ok = -1;
    if (ok < 0) {
        __builtin_cpu_init();
        ok = __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
             __builtin_cpu_supports("avx512vnni") && getenv("ORC_NO_VNNI") == NULL;
    }
    return ok;
}
#endif

/* Canonical Q8 x Q8 product, the schedule every device kernel follows:
 *   s_b  = sum_i qw[32b+i] * qx[32b+i]            (int32, exact)
 *   dd_b = f32(dw_b) * f32(dx_b)                  (exact: 11x11-bit product)
 *   range r covers blocks [32r, min(32r+32, nb)):
 *       P_r = fmaf((float)s_b, dd_b, P_r), P_r starting at +0, b ascending
 *   y = orc_tree_sum(P, ceil(nb/32)).
 * y[m][n] for activation rows m.  Rows are independent (batch invariant). */
void orc_q8_gemm(const int8_t* qs, const uint16_t* d, int32_t n, int32_t k,
                 const int8_t* xq, const uint16_t* xd, int32_t m, float* y) {
    int32_t nb = k / 32;
    int32_t g = (nb + ORC_Q8_RANGE_BLOCKS - 1) / ORC_Q8_RANGE_BLOCKS;
#if defined(__x86_64__) && defined(__GNUC__)
    if (m >= 16 && nb > 0 && vnni_ok()) {
        q8_gemm_vnni(qs, d, n, k, xq, xd, m, y);
        return;
    }
#endif
    float* dxf = (float*)malloc(sizeof(float) * (size_t)m * nb);
    for (int64_t i = 0; i < (int64_t)m * nb; ++i) dxf[i] = f16f(xd[i]);
    /* weight row outer, activation row inner: a thread keeps its weight row
     * and its decoded scales in cache across all m rows; every output is the
     * same chain as the one-row definition above */
#pragma omp parallel
    {
        float* dwf = (float*)malloc(sizeof(float) * (size_t)nb);
        float part[1024];
#pragma omp for schedule(static)
        for (int32_t row = 0; row < n; ++row) {
            const int8_t* w = qs + (int64_t)row * k;
            for (int32_t b = 0; b < nb; ++b) dwf[b] = f16f(d[(int64_t)row * nb + b]);
            int32_t mi = 0;
            /* four activation rows at a time: four independent chains */
            for (; mi + 4 <= m; mi += 4) {
                float p4[4][1024 / ORC_Q8_RANGE_BLOCKS + 1];
                for (int32_t r = 0; r < g; ++r) {
                    float c0 = 0.0f, c1 = 0.0f, c2 = 0.0f, c3 = 0.0f;
                    int32_t b1 = (r + 1) * ORC_Q8_RANGE_BLOCKS;
                    if (b1 > nb) b1 = nb;
                    for (int32_t b = r * ORC_Q8_RANGE_BLOCKS; b < b1; ++b) {
                        const int8_t* wb = w + (int64_t)b * 32;
                        const int8_t* ab = xq + (int64_t)mi * k + (int64_t)b * 32;
                        const float* dxb = dxf + (int64_t)mi * nb + b;
                        c0 = fmaf((float)block_dot(wb, ab), dwf[b] * dxb[0], c0);
                        c1 = fmaf((float)block_dot(wb, ab + k), dwf[b] * dxb[nb], c1);
                        c2 = fmaf((float)block_dot(wb, ab + 2 * (int64_t)k), dwf[b] * dxb[2 * nb], c2);
                        c3 = fmaf((float)block_dot(wb, ab + 3 * (int64_t)k), dwf[b] * dxb[3 * nb], c3);
                    }
                    p4[0][r] = c0;
                    p4[1][r] = c1;
                    p4[2][r] = c2;
                    p4[3][r] = c3;
                }
                for (int32_t u = 0; u < 4; ++u)
                    y[(int64_t)(mi + u) * n + row] = orc_tree_sum(p4[u], g);
            }
            for (; mi < m; ++mi) {
                const int8_t* a = xq + (int64_t)mi * k;
                const float* dx = dxf + (int64_t)mi * nb;
                for (int32_t r = 0; r < g; ++r) {
                    float acc = 0.0f;
                    int32_t b1 = (r + 1) * ORC_Q8_RANGE_BLOCKS;
                    if (b1 > nb) b1 = nb;
                    for (int32_t b = r * ORC_Q8_RANGE_BLOCKS; b < b1; ++b) {
                        int32_t s = block_dot(w + (int64_t)b * 32, a + (int64_t)b * 32);
                        acc = fmaf((float)s, dwf[b] * dx[b], acc);
                    }
                    part[r] = acc;
                }
                y[(int64_t)mi * n + row] = orc_tree_sum(part, g);
            }
        }
        free(dwf);
    }
    free(dxf);
}

/* ------------------------------------------------------------------ */
/* Paged KV cache + GQA decode attention                               */
/* ------------------------------------------------------------------ */
/* Cache layout: K and V pages are binary16 [num_pages][hkv][16][d]; token t
 * of sequence b lives in page page_table[b*maxp + t/16], slot t%16. */
#define ORC_PAGE 16
#define ORC_ATTN_CHUNK 256

static inline const uint16_t* kv_row(const uint16_t* pages, const int32_t* page_table,
                                     int32_t b, int32_t maxp, int32_t t, int32_t g,
                                     int32_t hkv, int32_t d) {
    int32_t page = page_table[(int64_t)b * maxp + t / ORC_PAGE];
    return pages + (((int64_t)page * hkv + g) * ORC_PAGE + (t % ORC_PAGE)) * d;
}

/* Halving tree over a power-of-two count: for s = n/2, n/4, ..., 1:
 * p[j] = p[j] + p[j+s] for j < s.  Returns p[0]; modifies p. */
float orc_halving_sum(float* p, int32_t n) {
    for (int32_t s = n / 2; s >= 1; s /= 2)
        for (int32_t j = 0; j < s; ++j) p[j] = p[j] + p[j + s];
    return p[0];
}

/* Canonical decode attention for one (b, h) over seq_len[b] cached tokens:
 *   s_t  = chain_i fmaf(q[i], f32(K_t[i]), acc) from +0, then * scale
 *   chunks of 256 tokens: m_c = max s_t, p_t = orc_expf(s_t - m_c),
 *   l_c  = halving sum over the chunk's 256 slots (0 past the end),
 *   o_c[i] = chain_t fmaf(p_t, f32(V_t[i]), acc) from +0, t ascending
 *   M = max m_c, w_c = orc_expf(m_c - M),
 *   L = chain_c fmaf(w_c, l_c, L), O[i] = chain_c fmaf(w_c, o_c[i], O[i]),
 *   out[i] = O[i] / L (0 for an empty sequence). */
#if defined(__x86_64__) && defined(__GNUC__)
/* 16 x 16 binary32 transpose: r[j] holds row j on entry, column j on exit
 * (unpacks inside 128-bit lanes, then lane shuffles). */
__attribute__((target("avx512f")))
static inline void tr16x16(__m512 r[16]) {
    __m512 t[16], u[16];
    for (int i = 0; i < 8; ++i) {
        t[2 * i] = _mm512_unpacklo_ps(r[2 * i], r[2 * i + 1]);
        t[2 * i + 1] = _mm512_unpackhi_ps(r[2 * i], r[2 * i + 1]);
    }
    for (int i = 0; i < 4; ++i) {      /* u[4i + c]: column 4L + c of rows 4i..4i+3 in lane L */
        const __m512d a = _mm512_castps_pd(t[4 * i]), b = _mm512_castps_pd(t[4 * i + 2]);
        const __m512d c = _mm512_castps_pd(t[4 * i + 1]), e = _mm512_castps_pd(t[4 * i + 3]);
        u[4 * i] = _mm512_castpd_ps(_mm512_unpacklo_pd(a, b));
        u[4 * i + 1] = _mm512_castpd_ps(_mm512_unpackhi_pd(a, b));
        u[4 * i + 2] = _mm512_castpd_ps(_mm512_unpacklo_pd(c, e));
        u[4 * i + 3] = _mm512_castpd_ps(_mm512_unpackhi_pd(c, e));
    }
    for (int k = 0; k < 4; ++k) {
        const __m512 v0 = _mm512_shuffle_f32x4(u[k], u[4 + k], 0x88);
        const __m512 v1 = _mm512_shuffle_f32x4(u[k], u[4 + k], 0xdd);
        const __m512 w0 = _mm512_shuffle_f32x4(u[8 + k], u[12 + k], 0x88);
        const __m512 w1 = _mm512_shuffle_f32x4(u[8 + k], u[12 + k], 0xdd);
        r[k] = _mm512_shuffle_f32x4(v0, w0, 0x88);
        r[8 + k] = _mm512_shuffle_f32x4(v0, w0, 0xdd);
        r[4 + k] = _mm512_shuffle_f32x4(v1, w1, 0x88);
        r[12 + k] = _mm512_shuffle_f32x4(v1, w1, 0xdd);
    }
}

/* orc_expf on 16 lanes: the same operations lane by lane (NaN passes
 * through, the two range limits are blends after the polynomial). */
__attribute__((target("avx512f")))
static inline __m512 expf16(__m512 x) {
    const __m512 nf = _mm512_sub_ps(_mm512_add_ps(_mm512_mul_ps(x, _mm512_set1_ps(1.44269504088896341f)),
                                                  _mm512_set1_ps(12582912.0f)),
                                    _mm512_set1_ps(12582912.0f));
    __m512 r = _mm512_fnmadd_ps(nf, _mm512_set1_ps(0.693145751953125f), x);
    r = _mm512_fnmadd_ps(nf, _mm512_set1_ps(1.42860682030941723e-06f), r);
    __m512 p = _mm512_set1_ps(1.98412698412698413e-04f);
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(1.38888888888888889e-03f));
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(8.33333333333333333e-03f));
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(4.16666666666666667e-02f));
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(1.66666666666666667e-01f));
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(0.5f));
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(1.0f));
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(1.0f));
    __m512i n = _mm512_cvttps_epi32(nf);
    const __mmask16 big = _mm512_cmpgt_epi32_mask(n, _mm512_set1_epi32(127));
    p = _mm512_mask_mul_ps(p, big, p, _mm512_set1_ps(2.0f));
    n = _mm512_mask_sub_epi32(n, big, n, _mm512_set1_epi32(1));
    __m512 y = _mm512_mul_ps(p, _mm512_castsi512_ps(_mm512_slli_epi32(
                                    _mm512_add_epi32(n, _mm512_set1_epi32(127)), 23)));
    y = _mm512_mask_blend_ps(_mm512_cmp_ps_mask(x, _mm512_set1_ps(-87.33f), _CMP_LT_OQ), y,
                             _mm512_setzero_ps());
    y = _mm512_mask_blend_ps(_mm512_cmp_ps_mask(x, _mm512_set1_ps(88.72f), _CMP_GT_OQ), y,
                             _mm512_set1_ps(INFINITY));
    return _mm512_mask_blend_ps(_mm512_cmp_ps_mask(x, x, _CMP_UNORD_Q), y, x);
}

/* AVX-512 form of orc_gqa_decode_attn for one (sequence b, KV head g) and
 * its gq query heads: the same per-head operations, 16 tokens (scores) or 16
 * dimensions (PV) in the lanes of a vector.  Score lane t runs the chain
 * fmaf(q[i], K_t[i], acc) over i ascending from +0, then * scale; PV lane i
 * runs fmaf(p_t, V_t[i], acc) over t ascending from +0; the binary16 rows are
 * widened with vcvtph2ps (exact: the cache holds no signalling NaN, its
 * values come from RNE conversions).  Softmax, the halving sums and the
 * chunk merge are the scalar code's. */
__attribute__((target("avx512f")))
static void attn_bg_avx512(const float* q, const uint16_t* kpages, const uint16_t* vpages,
                           const int32_t* page_table, int32_t b, int32_t g, int32_t L,
                           int32_t hq, int32_t hkv, int32_t d, int32_t maxp, float scale,
                           float* out, float* vf, float* sbuf, float* oc, float* mc, float* lc) {
    const int32_t gq = hq / hkv, nd = d / 16;
    const int32_t nc = (L + ORC_ATTN_CHUNK - 1) / ORC_ATTN_CHUNK;
    for (int32_t c = 0; c < nc; ++c) {
        const int32_t t0 = c * ORC_ATTN_CHUNK;
        const int32_t n = L - t0 < ORC_ATTN_CHUNK ? L - t0 : ORC_ATTN_CHUNK;
        /* scores: sbuf[hh][t] */
        for (int32_t tb = 0; tb * 16 < n; ++tb) {
            const int32_t nv = n - 16 * tb < 16 ? n - 16 * tb : 16;
            __m512 a[8];
            for (int32_t hh = 0; hh < gq; ++hh) a[hh] = _mm512_setzero_ps();
            for (int32_t ib = 0; ib < nd; ++ib) {
                __m512 r[16];
                for (int32_t j = 0; j < 16; ++j)
                    r[j] = j < nv ? _mm512_cvtph_ps(_mm256_loadu_si256((const __m256i*)(
                                        kv_row(kpages, page_table, b, maxp, t0 + 16 * tb + j, g, hkv, d) +
                                        16 * ib)))
                                  : _mm512_setzero_ps();
                tr16x16(r);
                for (int32_t i = 0; i < 16; ++i)
                    for (int32_t hh = 0; hh < gq; ++hh) {
                        const float qi = q[((int64_t)b * hq + g * gq + hh) * d + 16 * ib + i];
                        a[hh] = _mm512_fmadd_ps(_mm512_set1_ps(qi), r[i], a[hh]);
                    }
            }
            for (int32_t hh = 0; hh < gq; ++hh)
                _mm512_storeu_ps(sbuf + hh * ORC_ATTN_CHUNK + 16 * tb,
                                 _mm512_mul_ps(a[hh], _mm512_set1_ps(scale)));
        }
        /* V rows of the chunk as binary32 */
        for (int32_t t = 0; t < n; ++t) {
            const uint16_t* vr = kv_row(vpages, page_table, b, maxp, t0 + t, g, hkv, d);
            for (int32_t ib = 0; ib < nd; ++ib)
                _mm512_storeu_ps(vf + (int64_t)t * d + 16 * ib,
                                 _mm512_cvtph_ps(_mm256_loadu_si256((const __m256i*)(vr + 16 * ib))));
        }
        for (int32_t hh = 0; hh < gq; ++hh) {
            float* s = sbuf + hh * ORC_ATTN_CHUNK;
            float m = -INFINITY;
            for (int32_t j = 0; j < n; ++j)
                if (s[j] > m) m = s[j];
            for (int32_t j = 0; j < ORC_ATTN_CHUNK; j += 16) {
                const __m512 e = expf16(_mm512_sub_ps(_mm512_loadu_ps(s + j), _mm512_set1_ps(m)));
                const __mmask16 live = j + 16 <= n ? (__mmask16)0xffff
                                     : j >= n ? (__mmask16)0 : (__mmask16)((1u << (n - j)) - 1u);
                _mm512_storeu_ps(s + j, _mm512_maskz_mov_ps(live, e));
            }
            __m512 o[8];
            for (int32_t ib = 0; ib < nd; ++ib) o[ib] = _mm512_setzero_ps();
            for (int32_t t = 0; t < n; ++t) {
                const __m512 p = _mm512_set1_ps(s[t]);
                for (int32_t ib = 0; ib < nd; ++ib)
                    o[ib] = _mm512_fmadd_ps(p, _mm512_loadu_ps(vf + (int64_t)t * d + 16 * ib), o[ib]);
            }
            float* oo = oc + ((int64_t)hh * nc + c) * d;
            for (int32_t ib = 0; ib < nd; ++ib) _mm512_storeu_ps(oo + 16 * ib, o[ib]);
            mc[hh * nc + c] = m;
            lc[hh * nc + c] = orc_halving_sum(s, ORC_ATTN_CHUNK);
        }
    }
    for (int32_t hh = 0; hh < gq; ++hh) {
        const int64_t bh = (int64_t)b * hq + g * gq + hh;
        float M = -INFINITY;
        for (int32_t c = 0; c < nc; ++c) if (mc[hh * nc + c] > M) M = mc[hh * nc + c];
        float Ls = 0.0f;
        for (int32_t c = 0; c < nc; ++c) Ls = fmaf(orc_expf(mc[hh * nc + c] - M), lc[hh * nc + c], Ls);
        for (int32_t i = 0; i < d; ++i) {
            float O = 0.0f;
            for (int32_t c = 0; c < nc; ++c)
                O = fmaf(orc_expf(mc[hh * nc + c] - M), oc[((int64_t)hh * nc + c) * d + i], O);
            out[bh * d + i] = nc > 0 ? O / Ls : 0.0f;
        }
    }
}
#endif

void orc_gqa_decode_attn(const float* q, const uint16_t* kpages, const uint16_t* vpages,
                         const int32_t* page_table, const int32_t* seq_len, int32_t B,
                         int32_t hq, int32_t hkv, int32_t d, int32_t maxp, float scale,
                         float* out) {
    int32_t gq = hq / hkv;
#if defined(__x86_64__) && defined(__GNUC__)
    /* the vector form works on (sequence, KV head) tasks: taken when there
     * are enough of them for the threads (prefill rows, large batches) */
    if (vnni_ok() && d % 16 == 0 && d <= 128 && gq <= 8 &&
        (int64_t)B * hkv >= 4 * (int64_t)omp_get_max_threads()) {
#pragma omp parallel
        {
            float* vf = (float*)malloc(sizeof(float) * ORC_ATTN_CHUNK * d);
            float* sbuf = (float*)malloc(sizeof(float) * 8 * ORC_ATTN_CHUNK);
            int32_t cap = 0;
            float *oc = NULL, *mc = NULL, *lc = NULL;
#pragma omp for schedule(dynamic)
            for (int64_t bg = 0; bg < (int64_t)B * hkv; ++bg) {
                const int32_t b = (int32_t)(bg / hkv), g = (int32_t)(bg % hkv);
                const int32_t L = seq_len[b];
                const int32_t nc = (L + ORC_ATTN_CHUNK - 1) / ORC_ATTN_CHUNK;
                if (nc > cap) {
                    cap = nc;
                    free(oc); free(mc); free(lc);
                    oc = (float*)malloc(sizeof(float) * (size_t)gq * cap * d);
                    mc = (float*)malloc(sizeof(float) * (size_t)gq * cap);
                    lc = (float*)malloc(sizeof(float) * (size_t)gq * cap);
                }
                attn_bg_avx512(q, kpages, vpages, page_table, b, g, L, hq, hkv, d, maxp, scale, out,
                               vf, sbuf, oc, mc, lc);
            }
            free(vf); free(sbuf); free(oc); free(mc); free(lc);
        }
        return;
    }
#endif
#pragma omp parallel for schedule(dynamic)
    for (int64_t bh = 0; bh < (int64_t)B * hq; ++bh) {
        int32_t b = (int32_t)(bh / hq), h = (int32_t)(bh % hq), g = h / gq;
        int32_t L = seq_len[b];
        const float* qv = q + bh * d;
        int32_t nc = (L + ORC_ATTN_CHUNK - 1) / ORC_ATTN_CHUNK;
        float* s = (float*)malloc(sizeof(float) * ORC_ATTN_CHUNK);
        float* pbuf = (float*)malloc(sizeof(float) * ORC_ATTN_CHUNK);
        float* oc = (float*)calloc((size_t)nc * d, sizeof(float));
        float* mc = (float*)malloc(sizeof(float) * (nc > 0 ? nc : 1));
        float* lc = (float*)malloc(sizeof(float) * (nc > 0 ? nc : 1));
        for (int32_t c = 0; c < nc; ++c) {
            int32_t t0 = c * ORC_ATTN_CHUNK, n = L - t0 < ORC_ATTN_CHUNK ? L - t0 : ORC_ATTN_CHUNK;
            float m = -INFINITY;
            /* score chains over i, four tokens' chains interleaved */
            int32_t j = 0;
            for (; j + 4 <= n; j += 4) {
                const uint16_t* k0 = kv_row(kpages, page_table, b, maxp, t0 + j, g, hkv, d);
                const uint16_t* k1 = kv_row(kpages, page_table, b, maxp, t0 + j + 1, g, hkv, d);
                const uint16_t* k2 = kv_row(kpages, page_table, b, maxp, t0 + j + 2, g, hkv, d);
                const uint16_t* k3 = kv_row(kpages, page_table, b, maxp, t0 + j + 3, g, hkv, d);
                float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
                for (int32_t i = 0; i < d; ++i) {
                    a0 = fmaf(qv[i], f16f(k0[i]), a0);
                    a1 = fmaf(qv[i], f16f(k1[i]), a1);
                    a2 = fmaf(qv[i], f16f(k2[i]), a2);
                    a3 = fmaf(qv[i], f16f(k3[i]), a3);
                }
                s[j] = a0 * scale;
                s[j + 1] = a1 * scale;
                s[j + 2] = a2 * scale;
                s[j + 3] = a3 * scale;
            }
            for (; j < n; ++j) {
                const uint16_t* kr = kv_row(kpages, page_table, b, maxp, t0 + j, g, hkv, d);
                float acc = 0.0f;
                for (int32_t i = 0; i < d; ++i) acc = fmaf(qv[i], f16f(kr[i]), acc);
                s[j] = acc * scale;
            }
            for (j = 0; j < n; ++j)
                if (s[j] > m) m = s[j];
            for (j = 0; j < ORC_ATTN_CHUNK; ++j) pbuf[j] = j < n ? orc_expf(s[j] - m) : 0.0f;
            /* PV: chain over tokens for each i (j outer, every i's chain
             * advanced in token order) */
            float* o = oc + (int64_t)c * d;
            for (int32_t i = 0; i < d; ++i) o[i] = 0.0f;
            for (j = 0; j < n; ++j) {
                const uint16_t* vr = kv_row(vpages, page_table, b, maxp, t0 + j, g, hkv, d);
                const float pj = pbuf[j];
                for (int32_t i = 0; i < d; ++i) o[i] = fmaf(pj, f16f(vr[i]), o[i]);
            }
            mc[c] = m;
            lc[c] = orc_halving_sum(pbuf, ORC_ATTN_CHUNK);
        }
        float M = -INFINITY;
        for (int32_t c = 0; c < nc; ++c) if (mc[c] > M) M = mc[c];
        float Ls = 0.0f;
        for (int32_t c = 0; c < nc; ++c) Ls = fmaf(orc_expf(mc[c] - M), lc[c], Ls);
        for (int32_t i = 0; i < d; ++i) {
            float O = 0.0f;
            for (int32_t c = 0; c < nc; ++c) O = fmaf(orc_expf(mc[c] - M), oc[(int64_t)c * d + i], O);
            out[bh * d + i] = nc > 0 ? O / Ls : 0.0f;
        }
        free(s); free(pbuf); free(oc); free(mc); free(lc);
    }
}

/* Random page table: the B * maxp page ids are a seeded permutation of
 * 0..B*maxp-1 (Fisher-Yates with the multiply-high bounded draw). */
void orc_gen_page_table(uint64_t seed, uint64_t stream, int32_t B, int32_t maxp, int32_t* pt) {
    int64_t n = (int64_t)B * maxp;
    uint64_t base = orc_stream_base(seed, stream);
    for (int64_t i = 0; i < n; ++i) pt[i] = (int32_t)i;
    for (int64_t i = n - 1; i > 0; --i) {
        int64_t j = (int64_t)below32(stream_at(base, (uint64_t)(n - 1 - i)), (uint32_t)(i + 1));
        int32_t tmp = pt[i]; pt[i] = pt[j]; pt[j] = tmp;
    }
}

/* ------------------------------------------------------------------ */
/* Decode-step glue                                                    */
/* ------------------------------------------------------------------ */
static int32_t pow2_at_least(int32_t n) {
    int32_t p = 1;
    while (p < n) p <<= 1;
    return p;
}

/* RMSNorm: S = halving sum of x_i*x_i over the next power of two >= h (zeros
 * past h), ms = S / h, r = 1 / sqrtf(ms + eps), y_i = (x_i * r) * w_i. */
void orc_rmsnorm(const float* x, const float* w, int32_t m, int32_t h, float eps, float* y) {
    int32_t n2 = pow2_at_least(h);
    /* rows are independent: split over the threads, one scratch row each */
#pragma omp parallel if (m >= 64)
    {
        float* t = (float*)malloc(sizeof(float) * n2);
#pragma omp for schedule(static)
        for (int32_t r = 0; r < m; ++r) {
            const float* xr = x + (int64_t)r * h;
            for (int32_t i = 0; i < n2; ++i) t[i] = i < h ? xr[i] * xr[i] : 0.0f;
            float ms = orc_halving_sum(t, n2) / (float)h;
            float rr = 1.0f / sqrtf(ms + eps);
            for (int32_t i = 0; i < h; ++i) y[(int64_t)r * h + i] = (xr[i] * rr) * w[i];
        }
        free(t);
    }
}

/* RoPE tables: angle = pos * theta^(-2i/d) in binary64, rounded to binary32
 * after cos / sin.  cos_t, sin_t are [max_seq][d/2]. */
void orc_rope_tables(int32_t max_seq, int32_t d, double theta, float* cos_t, float* sin_t) {
    for (int32_t p = 0; p < max_seq; ++p)
        for (int32_t i = 0; i < d / 2; ++i) {
            double inv = pow(theta, -(2.0 * i) / (double)d);
            double ang = (double)p * inv;
            cos_t[(int64_t)p * (d / 2) + i] = (float)cos(ang);
            sin_t[(int64_t)p * (d / 2) + i] = (float)sin(ang);
        }
}

/* Rotate-half RoPE of nheads vectors of length d in place:
 * x[i] <- x[i]*c - x[i+d/2]*s, x[i+d/2] <- x[i+d/2]*c + x[i]*s. */
void orc_rope(float* x, int32_t nheads, int32_t d, const float* cos_row, const float* sin_row) {
    for (int32_t hh = 0; hh < nheads; ++hh) {
        float* v = x + (int64_t)hh * d;
        for (int32_t i = 0; i < d / 2; ++i) {
            float a = v[i], b = v[i + d / 2], c = cos_row[i], s = sin_row[i];
            float t0 = a * c, t1 = b * s, t2 = b * c, t3 = a * s;
            v[i] = t0 - t1;
            v[i + d / 2] = t2 + t3;
        }
    }
}

/* a_i = silu(g_i) * u_i for gu = [gate(0..I) | up(0..I)]. */
void orc_swiglu(const float* gu, int32_t m, int32_t inter, float* a) {
#pragma omp parallel for schedule(static) if (m >= 16)
    for (int32_t r = 0; r < m; ++r)
        for (int32_t i = 0; i < inter; ++i)
            a[(int64_t)r * inter + i] = orc_silu(gu[(int64_t)r * 2 * inter + i]) *
                                        gu[(int64_t)r * 2 * inter + inter + i];
}

/* First index of the maximum: NaN entries are skipped, ties go to the lowest
 * index, -0 == +0; an all-NaN row gives 0. */
int32_t orc_argmax(const float* x, int32_t n) {
    int32_t best = -1;
    for (int32_t i = 0; i < n; ++i)
        if (x[i] == x[i] && (best < 0 || x[i] > x[best])) best = i;
    return best < 0 ? 0 : best;
}

/* logits[r][v] = canonical dot of binary32 x[r] with binary16 row E[v]:
 * ranges of 1024 elements, each a sequential fmaf chain from +0, then the
 * pairwise tree over ranges. */
void orc_lm_head_f16(const float* x, int32_t m, const uint16_t* E, int32_t V, int32_t h,
                     float* logits) {
    int32_t g = (h + 1023) / 1024;
#pragma omp parallel for schedule(static)
    for (int32_t v = 0; v < V; ++v) {
        float part[64];
        const uint16_t* er = E + (int64_t)v * h;
        for (int32_t r = 0; r < m; ++r) {
            const float* xr = x + (int64_t)r * h;
            for (int32_t q = 0; q < g; ++q) {
                float acc = 0.0f;
                int32_t k1 = (q + 1) * 1024 < h ? (q + 1) * 1024 : h;
                for (int32_t k = q * 1024; k < k1; ++k) acc = fmaf(xr[k], orc_f16_to_f32(er[k]), acc);
                part[q] = acc;
            }
            logits[(int64_t)r * V + v] = orc_tree_sum(part, g);
        }
    }
}

/* ------------------------------------------------------------------ */
/* Random-init Qwen2-shaped Q8_0 model                                 */
/* ------------------------------------------------------------------ */
/* Seed streams (one per tensor; a Q8_0 matrix uses stream s for its quants
 * and s+1 for its scales):
 *   1        embedding, binary16 N(0, emb_sigma)       [vocab][hidden]
 *   2, 3     lm_head Q8_0 (untied models only)          [vocab][hidden]
 *   L+0,1    Wqkv Q8_0, rows q heads | k heads | v heads [(hq+2hkv)d][hidden]
 *   L+2,3    Wo Q8_0                                    [hidden][hq d]
 *   L+4,5    Wgu Q8_0, rows gate | up                   [2 inter][hidden]
 *   L+6,7    Wdown Q8_0                                 [hidden][inter]
 *   L+8      qkv bias, binary32 N(0, 0.02)              [(hq+2hkv)d]
 * with L = 1000 + 16 * layer.  RMSNorm weights are 1.0. */
/* ------------------------------------------------------------------ */
/* Seeded top-k / top-p sampling                                       */
/* ------------------------------------------------------------------ */
/* Candidate order: value descending, then index ascending; NaN is never a
 * candidate and -0 ranks as +0.  The key packs (orderable value bits, 2^32-1
 * - index), so the order is the plain unsigned order of keys. */
static uint64_t sample_key(float x, int32_t v) {
    if (x != x) return 0;
    uint32_t u = f2u(x == 0.0f ? 0.0f : x);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | (uint64_t)(0xffffffffu - (uint32_t)v);
}
static float key_value(uint64_t k) {
    uint32_t u = (uint32_t)(k >> 32);
    u = (u & 0x80000000u) ? (u & 0x7fffffffu) : ~u;
    return u2f(u);
}
static int key_desc(const void* a, const void* b) {
    uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
    return x < y ? 1 : x > y ? -1 : 0;
}

/* One row: the top_k candidates in order j = 0, 1, ...;
 *   e_j = orc_expf((l_j - l_0) * (1/temperature)), c_j = c_{j-1} + e_j
 *   J = first j with c_j >= top_p * c_{n-1}
 *   u = (x >> 40) * 2^-24, x = element pos of SplitMix64 stream `stream` of
 *       seed (orc_stream_base convention)
 *   token = candidate of the first j <= J with c_j > u * c_J (J if none). */
int32_t orc_sample_row(const float* logits, int32_t vocab, int32_t top_k, float top_p,
                       float temperature, uint64_t seed, int32_t stream, int32_t pos) {
    uint64_t* keys = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)(vocab > 0 ? vocab : 1));
    int32_t nv = 0;
    for (int32_t v = 0; v < vocab; ++v) {
        uint64_t k = sample_key(logits[v], v);
        if (k) keys[nv++] = k;
    }
    qsort(keys, (size_t)nv, sizeof(uint64_t), key_desc);
    int32_t n = nv < top_k ? nv : top_k;
    int32_t tok = 0;
    if (n > 0) {
        const float inv_temp = 1.0f / temperature;
        const float v0 = key_value(keys[0]);
        float c[64];
        float acc = 0.0f;
        for (int32_t j = 0; j < n; ++j) {
            acc = acc + orc_expf((key_value(keys[j]) - v0) * inv_temp);
            c[j] = acc;
        }
        const float thr = top_p * acc;
        int32_t J = n - 1;
        for (int32_t j = 0; j < n; ++j)
            if (c[j] >= thr) { J = j; break; }
        uint64_t x = stream_at(orc_stream_base(seed, (uint64_t)stream), (uint64_t)pos);
        const float u = (float)(uint32_t)(x >> 40) * 0x1.0p-24f;
        const float r = u * c[J];
        int32_t pick = J;
        for (int32_t j = 0; j <= J; ++j)
            if (c[j] > r) { pick = j; break; }
        tok = (int32_t)(0xffffffffu - (uint32_t)keys[pick]);
    }
    free(keys);
    return tok;
}

/* m rows; row i uses stream streams[i] and draw index pos[i].  top_k in
 * [1, 64]. */
void orc_sample(const float* logits, int32_t m, int32_t vocab, int32_t top_k, float top_p,
                float temperature, uint64_t seed, const int32_t* streams, const int32_t* pos,
                int32_t* out) {
#pragma omp parallel for schedule(dynamic)
    for (int32_t i = 0; i < m; ++i)
        out[i] = orc_sample_row(logits + (int64_t)i * vocab, vocab, top_k, top_p, temperature,
                                seed, streams[i], pos[i]);
}

struct orc_model {
    orc_qwen_config c;
    uint64_t seed;
    int32_t qkv_n, maxp;
    uint16_t* emb;
    int8_t* emb_qs;        /* a Q8_0 embedding (orc_model_set_emb_q8), else NULL */
    uint16_t* emb_d;
    int8_t* lm_qs;
    uint16_t* lm_d;
    int8_t **qkv_qs, **o_qs, **gu_qs, **dn_qs;
    uint16_t **qkv_d, **o_d, **gu_d, **dn_d;
    float** bias;
    float* ones;
    float **attn_norm, **ffn_norm;   /* RMSNorm weights per layer (1 unless set) */
    float* out_norm;
    float *cos_t, *sin_t;
    uint16_t **kc, **vc;   /* per layer paged [max_batch*maxp][hkv][16][d] */
    int32_t* page_table;   /* identity: slot b page p -> b*maxp + p */
    int32_t* seq_len;
    int32_t s_top_k;       /* 0: greedy argmax; else orc_sample_row with: */
    float s_top_p, s_temp;
    uint64_t s_seed;
};

/* Element k of token v's embedding row: binary16 widened, or Q8_0
 * f32(d) * q (exact). */
static inline float emb_value(const orc_model* m, int32_t v, int32_t k) {
    const int64_t H = m->c.hidden;
    if (m->emb_qs)
        return f16f(m->emb_d[(int64_t)v * (H / 32) + k / 32]) * (float)m->emb_qs[(int64_t)v * H + k];
    return orc_f16_to_f32(m->emb[(int64_t)v * H + k]);
}

static void* xmalloc(size_t n) {
    void* p = malloc(n ? n : 1);
    if (!p) abort();
    return p;
}

static void gen_q8(uint64_t seed, uint64_t stream, int64_t n, int64_t k, int8_t** qs,
                   uint16_t** d) {
    *qs = (int8_t*)xmalloc((size_t)(n * k));
    *d = (uint16_t*)xmalloc((size_t)(n * (k / 32)) * 2);
    /* element-indexed streams, so chunks can be generated in parallel */
    uint64_t bq = orc_stream_base(seed, stream), bd = orc_stream_base(seed, stream + 1);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n * k; ++i)
        (*qs)[i] = (int8_t)((int32_t)below32(stream_at(bq, (uint64_t)i), 255u) - 127);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n * (k / 32); ++i)
        (*d)[i] = orc_f32_to_f16((float)(fabs(0.02 * normal_at(bd, (uint64_t)i)) / 127.0));
}

orc_model* orc_model_create(const orc_qwen_config* cfg, uint64_t seed) {
    orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
    m->c = *cfg;
    m->seed = seed;
    const orc_qwen_config* c = cfg;
    int32_t H = c->hidden, I = c->inter, d = c->head_dim, hq = c->n_heads, hkv = c->n_kv;
    m->qkv_n = (hq + 2 * hkv) * d;
    m->maxp = (c->max_seq + ORC_PAGE - 1) / ORC_PAGE;
    m->emb = (uint16_t*)xmalloc((size_t)c->vocab * H * 2);
    {
        uint64_t be = orc_stream_base(seed, 1);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < (int64_t)c->vocab * H; ++i)
            m->emb[i] = orc_f32_to_f16((float)(c->emb_sigma * normal_at(be, (uint64_t)i)));
    }
    if (!c->tied) gen_q8(seed, 2, c->vocab, H, &m->lm_qs, &m->lm_d);
    int32_t nl = c->n_layers;
    m->qkv_qs = (int8_t**)calloc(nl, sizeof(void*));
    m->o_qs = (int8_t**)calloc(nl, sizeof(void*));
    m->gu_qs = (int8_t**)calloc(nl, sizeof(void*));
    m->dn_qs = (int8_t**)calloc(nl, sizeof(void*));
    m->qkv_d = (uint16_t**)calloc(nl, sizeof(void*));
    m->o_d = (uint16_t**)calloc(nl, sizeof(void*));
    m->gu_d = (uint16_t**)calloc(nl, sizeof(void*));
    m->dn_d = (uint16_t**)calloc(nl, sizeof(void*));
    m->bias = (float**)calloc(nl, sizeof(void*));
    m->kc = (uint16_t**)calloc(nl, sizeof(void*));
    m->vc = (uint16_t**)calloc(nl, sizeof(void*));
    size_t kv_elems = (size_t)c->max_batch * m->maxp * hkv * ORC_PAGE * d;
    for (int32_t l = 0; l < nl; ++l) {
        uint64_t L = 1000 + 16 * (uint64_t)l;
        gen_q8(seed, L + 0, m->qkv_n, H, &m->qkv_qs[l], &m->qkv_d[l]);
        gen_q8(seed, L + 2, H, hq * d, &m->o_qs[l], &m->o_d[l]);
        gen_q8(seed, L + 4, 2 * I, H, &m->gu_qs[l], &m->gu_d[l]);
        gen_q8(seed, L + 6, H, I, &m->dn_qs[l], &m->dn_d[l]);
        m->bias[l] = (float*)xmalloc(sizeof(float) * m->qkv_n);
        orc_gen_normal_f32(seed, L + 8, 0.02, m->bias[l], m->qkv_n);
        m->kc[l] = (uint16_t*)calloc(kv_elems, 2);
        m->vc[l] = (uint16_t*)calloc(kv_elems, 2);
    }
    int32_t mx = H > I ? H : I;
    m->ones = (float*)xmalloc(sizeof(float) * mx);
    for (int32_t i = 0; i < mx; ++i) m->ones[i] = 1.0f;
    m->attn_norm = (float**)calloc(nl, sizeof(void*));
    m->ffn_norm = (float**)calloc(nl, sizeof(void*));
    for (int32_t l = 0; l < nl; ++l) {
        m->attn_norm[l] = (float*)xmalloc(sizeof(float) * H);
        m->ffn_norm[l] = (float*)xmalloc(sizeof(float) * H);
        memcpy(m->attn_norm[l], m->ones, sizeof(float) * H);
        memcpy(m->ffn_norm[l], m->ones, sizeof(float) * H);
    }
    m->out_norm = (float*)xmalloc(sizeof(float) * H);
    memcpy(m->out_norm, m->ones, sizeof(float) * H);
    m->cos_t = (float*)xmalloc(sizeof(float) * (size_t)c->max_seq * (d / 2));
    m->sin_t = (float*)xmalloc(sizeof(float) * (size_t)c->max_seq * (d / 2));
    orc_rope_tables(c->max_seq, d, c->theta, m->cos_t, m->sin_t);
    m->page_table = (int32_t*)xmalloc(sizeof(int32_t) * (size_t)c->max_batch * m->maxp);
    for (int64_t i = 0; i < (int64_t)c->max_batch * m->maxp; ++i) m->page_table[i] = (int32_t)i;
    m->seq_len = (int32_t*)calloc(c->max_batch, sizeof(int32_t));
    return m;
}

void orc_model_destroy(orc_model* m) {
    if (!m) return;
    for (int32_t l = 0; l < m->c.n_layers; ++l) {
        free(m->qkv_qs[l]); free(m->o_qs[l]); free(m->gu_qs[l]); free(m->dn_qs[l]);
        free(m->qkv_d[l]); free(m->o_d[l]); free(m->gu_d[l]); free(m->dn_d[l]);
        free(m->bias[l]); free(m->kc[l]); free(m->vc[l]);
    }
    free(m->qkv_qs); free(m->o_qs); free(m->gu_qs); free(m->dn_qs);
    free(m->qkv_d); free(m->o_d); free(m->gu_d); free(m->dn_d);
    free(m->bias); free(m->kc); free(m->vc);
    for (int32_t l = 0; l < m->c.n_layers; ++l) { free(m->attn_norm[l]); free(m->ffn_norm[l]); }
    free(m->attn_norm); free(m->ffn_norm); free(m->out_norm);
    free(m->emb); free(m->emb_qs); free(m->emb_d); free(m->lm_qs); free(m->lm_d); free(m->ones);
    free(m->cos_t); free(m->sin_t); free(m->page_table); free(m->seq_len);
    free(m);
}

int32_t orc_model_seq_len(const orc_model* m, int32_t slot) { return m->seq_len[slot]; }

/* Host copies of the generated tensors, for comparing the device model's own
 * generator: which = 0 emb, 1 lm q, 2 lm d, 3 qkv q, 4 qkv d, 5 o q, 6 o d,
 * 7 gu q, 8 gu d, 9 down q, 10 down d, 11 bias.  Returns the pointer. */
const void* orc_model_tensor(const orc_model* m, int32_t layer, int32_t which) {
    switch (which) {
        case 0: return m->emb;
        case 1: return m->lm_qs;
        case 2: return m->lm_d;
        case 3: return m->qkv_qs[layer];
        case 4: return m->qkv_d[layer];
        case 5: return m->o_qs[layer];
        case 6: return m->o_d[layer];
        case 7: return m->gu_qs[layer];
        case 8: return m->gu_d[layer];
        case 9: return m->dn_qs[layer];
        case 10: return m->dn_d[layer];
        case 11: return m->bias[layer];
        default: return NULL;
    }
}

/* Copy of the cached K (kv = 0) or V (kv = 1) rows of slot b at layer l,
 * tokens [0, n): out[n][hkv][d] binary16. */
void orc_model_kv(const orc_model* m, int32_t layer, int32_t kv, int32_t b, int32_t n,
                  uint16_t* out) {
    int32_t hkv = m->c.n_kv, d = m->c.head_dim;
    const uint16_t* pages = kv ? m->vc[layer] : m->kc[layer];
    for (int32_t t = 0; t < n; ++t)
        for (int32_t g = 0; g < hkv; ++g)
            memcpy(out + ((int64_t)t * hkv + g) * d,
                   kv_row(pages, m->page_table, b, m->maxp, t, g, hkv, d), (size_t)d * 2);
}

/* One decode step for nseq sequences: sequence slots[i] consumes tokens[i]
 * at position seq_len[slot]; returns the greedy next tokens, the final hidden
 * rows (nullable [nseq][hidden]) and logits (nullable [nseq][vocab]).  Rows
 * are independent, so any subset of slots can be stepped. */
void orc_model_step(orc_model* m, int32_t nseq, const int32_t* slots, const int32_t* tokens,
                    int32_t* next, float* hidden_out, float* logits_out) {
    const orc_qwen_config* c = &m->c;
    int32_t H = c->hidden, I = c->inter, d = c->head_dim, hq = c->n_heads, hkv = c->n_kv;
    int32_t B = nseq, qn = m->qkv_n;
    float* h = (float*)xmalloc(sizeof(float) * B * H);
    float* xn = (float*)xmalloc(sizeof(float) * B * (H > I ? H : I));
    int32_t kmax = H > I ? H : I;
    if (hq * d > kmax) kmax = hq * d;
    int8_t* xq = (int8_t*)xmalloc((size_t)B * kmax);
    uint16_t* xd = (uint16_t*)xmalloc((size_t)B * (kmax / 32) * 2);
    float* qkv = (float*)xmalloc(sizeof(float) * B * qn);
    float* q = (float*)xmalloc(sizeof(float) * B * hq * d);
    float* att = (float*)xmalloc(sizeof(float) * B * hq * d);
    float* y = (float*)xmalloc(sizeof(float) * B * (2 * I > H ? 2 * I : H));
    float* a = (float*)xmalloc(sizeof(float) * B * I);
    int32_t* pt = (int32_t*)xmalloc(sizeof(int32_t) * B * m->maxp);
    int32_t* lens = (int32_t*)xmalloc(sizeof(int32_t) * B);
    float scale = (float)(1.0 / sqrt((double)d));
    for (int32_t i = 0; i < B; ++i) {
        for (int32_t k = 0; k < H; ++k)
            h[(int64_t)i * H + k] = emb_value(m, tokens[i], k);
        memcpy(pt + (int64_t)i * m->maxp, m->page_table + (int64_t)slots[i] * m->maxp,
               sizeof(int32_t) * m->maxp);
        lens[i] = m->seq_len[slots[i]] + 1;
    }
    for (int32_t l = 0; l < c->n_layers; ++l) {
        orc_rmsnorm(h, m->attn_norm[l], B, H, c->eps, xn);
        orc_quantize_q8_0(xn, B, H, xq, xd);
        orc_q8_gemm(m->qkv_qs[l], m->qkv_d[l], qn, H, xq, xd, B, qkv);
        for (int32_t i = 0; i < B; ++i) {
            float* r = qkv + (int64_t)i * qn;
            for (int32_t j = 0; j < qn; ++j) r[j] = r[j] + m->bias[l][j];
            int32_t pos = lens[i] - 1;
            const float* cr = m->cos_t + (int64_t)pos * (d / 2);
            const float* sr = m->sin_t + (int64_t)pos * (d / 2);
            orc_rope(r, hq + hkv, d, cr, sr);         /* q heads then k heads */
            memcpy(q + (int64_t)i * hq * d, r, sizeof(float) * hq * d);
            int32_t b = slots[i];
            for (int32_t g = 0; g < hkv; ++g) {
                int32_t page = m->page_table[(int64_t)b * m->maxp + pos / ORC_PAGE];
                int64_t off = (((int64_t)page * hkv + g) * ORC_PAGE + pos % ORC_PAGE) * d;
                for (int32_t e = 0; e < d; ++e) {
                    m->kc[l][off + e] = orc_f32_to_f16(r[(hq + g) * d + e]);
                    m->vc[l][off + e] = orc_f32_to_f16(r[(hq + hkv + g) * d + e]);
                }
            }
        }
        orc_gqa_decode_attn(q, m->kc[l], m->vc[l], pt, lens, B, hq, hkv, d, m->maxp, scale, att);
        orc_quantize_q8_0(att, B, hq * d, xq, xd);
        orc_q8_gemm(m->o_qs[l], m->o_d[l], H, hq * d, xq, xd, B, y);
        for (int64_t j = 0; j < (int64_t)B * H; ++j) h[j] = h[j] + y[j];
        orc_rmsnorm(h, m->ffn_norm[l], B, H, c->eps, xn);
        orc_quantize_q8_0(xn, B, H, xq, xd);
        orc_q8_gemm(m->gu_qs[l], m->gu_d[l], 2 * I, H, xq, xd, B, y);
        orc_swiglu(y, B, I, a);
        orc_quantize_q8_0(a, B, I, xq, xd);
        orc_q8_gemm(m->dn_qs[l], m->dn_d[l], H, I, xq, xd, B, y);
        for (int64_t j = 0; j < (int64_t)B * H; ++j) h[j] = h[j] + y[j];
    }
    orc_rmsnorm(h, m->out_norm, B, H, c->eps, xn);
    if (hidden_out) memcpy(hidden_out, xn, sizeof(float) * B * H);
    float* logits = (float*)xmalloc(sizeof(float) * (size_t)B * c->vocab);
    if (c->tied && !m->emb_qs) {
        orc_lm_head_f16(xn, B, m->emb, c->vocab, H, logits);
    } else {
        orc_quantize_q8_0(xn, B, H, xq, xd);
        orc_q8_gemm(c->tied ? m->emb_qs : m->lm_qs, c->tied ? m->emb_d : m->lm_d, c->vocab, H,
                    xq, xd, B, logits);
    }
    for (int32_t i = 0; i < B; ++i) {
        next[i] = m->s_top_k > 0
                      ? orc_sample_row(logits + (int64_t)i * c->vocab, c->vocab, m->s_top_k,
                                       m->s_top_p, m->s_temp, m->s_seed, slots[i], lens[i] - 1)
                      : orc_argmax(logits + (int64_t)i * c->vocab, c->vocab);
        m->seq_len[slots[i]] = lens[i];
    }
    if (logits_out) memcpy(logits_out, logits, sizeof(float) * (size_t)B * c->vocab);
    free(logits); free(h); free(xn); free(xq); free(xd); free(qkv); free(q); free(att);
    free(y); free(a); free(pt); free(lens);
}

/* Teacher-forced prefill of nseq sequences, P positions each: row s*P + j is
 * token tokens[s*P + j] of slot slots[s] at position seq_len[slot] + j.
 * Every layer runs its products over all nseq*P rows at once, appends the K/V
 * of all rows, then lets row j attend to the first seq_len + j + 1 tokens of
 * its slot.  Each row goes through exactly the operations orc_model_step
 * applies to it (rows are independent in every product and glue step, and a
 * row never reads cache slots past its own position), so the cache, next
 * tokens, logits and hidden rows equal P calls of orc_model_step; the tests
 * check that bit for bit.  Outputs are those of each slot's last position. */
void orc_model_prefill(orc_model* m, int32_t nseq, const int32_t* slots, int32_t P,
                       const int32_t* tokens, int32_t* next, float* hidden_out,
                       float* logits_out) {
    const orc_qwen_config* c = &m->c;
    int32_t H = c->hidden, I = c->inter, d = c->head_dim, hq = c->n_heads, hkv = c->n_kv;
    int32_t qn = m->qkv_n;
    int64_t R = (int64_t)nseq * P;
    int32_t kmax = H > I ? H : I;
    if (hq * d > kmax) kmax = hq * d;
    float* h = (float*)xmalloc(sizeof(float) * R * H);
    float* xn = (float*)xmalloc(sizeof(float) * R * H);
    int8_t* xq = (int8_t*)xmalloc((size_t)R * kmax);
    uint16_t* xd = (uint16_t*)xmalloc((size_t)R * (kmax / 32) * 2);
    float* qkv = (float*)xmalloc(sizeof(float) * R * qn);
    float* q = (float*)xmalloc(sizeof(float) * R * hq * d);
    float* att = (float*)xmalloc(sizeof(float) * R * hq * d);
    float* y = (float*)xmalloc(sizeof(float) * R * (2 * I > H ? 2 * I : H));
    float* a = (float*)xmalloc(sizeof(float) * R * I);
    int32_t* pt = (int32_t*)xmalloc(sizeof(int32_t) * R * m->maxp);
    int32_t* lens = (int32_t*)xmalloc(sizeof(int32_t) * R);
    float scale = (float)(1.0 / sqrt((double)d));
    for (int64_t r = 0; r < R; ++r) {
        int32_t s = (int32_t)(r / P), j = (int32_t)(r % P);
        for (int32_t k = 0; k < H; ++k)
            h[r * H + k] = emb_value(m, tokens[r], k);
        memcpy(pt + r * m->maxp, m->page_table + (int64_t)slots[s] * m->maxp,
               sizeof(int32_t) * m->maxp);
        lens[r] = m->seq_len[slots[s]] + j + 1;
    }
    for (int32_t l = 0; l < c->n_layers; ++l) {
        orc_rmsnorm(h, m->attn_norm[l], (int32_t)R, H, c->eps, xn);
        orc_quantize_q8_0(xn, R, H, xq, xd);
        orc_q8_gemm(m->qkv_qs[l], m->qkv_d[l], qn, H, xq, xd, (int32_t)R, qkv);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < R; ++i) {
            float* r = qkv + i * qn;
            for (int32_t jj = 0; jj < qn; ++jj) r[jj] = r[jj] + m->bias[l][jj];
            int32_t pos = lens[i] - 1;
            orc_rope(r, hq + hkv, d, m->cos_t + (int64_t)pos * (d / 2),
                     m->sin_t + (int64_t)pos * (d / 2));
            memcpy(q + i * hq * d, r, sizeof(float) * hq * d);
            int32_t b = slots[i / P];
            for (int32_t g = 0; g < hkv; ++g) {
                int32_t page = m->page_table[(int64_t)b * m->maxp + pos / ORC_PAGE];
                int64_t off = (((int64_t)page * hkv + g) * ORC_PAGE + pos % ORC_PAGE) * d;
                for (int32_t e = 0; e < d; ++e) {
                    m->kc[l][off + e] = orc_f32_to_f16(r[(hq + g) * d + e]);
                    m->vc[l][off + e] = orc_f32_to_f16(r[(hq + hkv + g) * d + e]);
                }
            }
        }
        orc_gqa_decode_attn(q, m->kc[l], m->vc[l], pt, lens, (int32_t)R, hq, hkv, d, m->maxp,
                            scale, att);
        orc_quantize_q8_0(att, R, hq * d, xq, xd);
        orc_q8_gemm(m->o_qs[l], m->o_d[l], H, hq * d, xq, xd, (int32_t)R, y);
        for (int64_t j = 0; j < R * H; ++j) h[j] = h[j] + y[j];
        orc_rmsnorm(h, m->ffn_norm[l], (int32_t)R, H, c->eps, xn);
        orc_quantize_q8_0(xn, R, H, xq, xd);
        orc_q8_gemm(m->gu_qs[l], m->gu_d[l], 2 * I, H, xq, xd, (int32_t)R, y);
        orc_swiglu(y, (int32_t)R, I, a);
        orc_quantize_q8_0(a, R, I, xq, xd);
        orc_q8_gemm(m->dn_qs[l], m->dn_d[l], H, I, xq, xd, (int32_t)R, y);
        for (int64_t j = 0; j < R * H; ++j) h[j] = h[j] + y[j];
    }
    /* the head for each slot's last position only */
    float* hl = (float*)xmalloc(sizeof(float) * (size_t)nseq * H);
    for (int32_t s = 0; s < nseq; ++s)
        memcpy(hl + (int64_t)s * H, h + ((int64_t)s * P + P - 1) * H, sizeof(float) * H);
    orc_rmsnorm(hl, m->out_norm, nseq, H, c->eps, xn);
    if (hidden_out) memcpy(hidden_out, xn, sizeof(float) * nseq * H);
    float* logits = (float*)xmalloc(sizeof(float) * (size_t)nseq * c->vocab);
    if (c->tied && !m->emb_qs) {
        orc_lm_head_f16(xn, nseq, m->emb, c->vocab, H, logits);
    } else {
        orc_quantize_q8_0(xn, nseq, H, xq, xd);
        orc_q8_gemm(c->tied ? m->emb_qs : m->lm_qs, c->tied ? m->emb_d : m->lm_d, c->vocab, H,
                    xq, xd, nseq, logits);
    }
    for (int32_t s = 0; s < nseq; ++s) {
        next[s] = m->s_top_k > 0
                      ? orc_sample_row(logits + (int64_t)s * c->vocab, c->vocab, m->s_top_k,
                                       m->s_top_p, m->s_temp, m->s_seed, slots[s],
                                       m->seq_len[slots[s]] + P - 1)
                      : orc_argmax(logits + (int64_t)s * c->vocab, c->vocab);
        m->seq_len[slots[s]] += P;
    }
    if (logits_out) memcpy(logits_out, logits, sizeof(float) * (size_t)nseq * c->vocab);
    free(logits); free(hl); free(h); free(xn); free(xq); free(xd); free(qkv); free(q);
    free(att); free(y); free(a); free(pt); free(lens);
}

/* Writes cached K (kv = 0) or V (kv = 1) rows of slot b at layer l, tokens
 * [0, n), from rows[n][hkv][d] (binary16): the inverse of orc_model_kv.  With
 * orc_model_set_seq_len this loads a cache computed elsewhere (a device
 * prefill the tests have checked bit for bit) so the CPU baseline can decode
 * at the benchmark's context length without re-running the prompt. */
void orc_model_load_kv(orc_model* m, int32_t layer, int32_t kv, int32_t b, int32_t n,
                       const uint16_t* rows) {
    int32_t hkv = m->c.n_kv, d = m->c.head_dim;
    uint16_t* pages = kv ? m->vc[layer] : m->kc[layer];
    for (int32_t t = 0; t < n; ++t)
        for (int32_t g = 0; g < hkv; ++g) {
            int32_t page = m->page_table[(int64_t)b * m->maxp + t / ORC_PAGE];
            memcpy(pages + (((int64_t)page * hkv + g) * ORC_PAGE + t % ORC_PAGE) * d,
                   rows + ((int64_t)t * hkv + g) * d, (size_t)d * 2);
        }
}

void orc_model_set_seq_len(orc_model* m, int32_t slot, int32_t len) { m->seq_len[slot] = len; }

/* OpenMP threads of later oracle calls (the CPU baseline times 1 and all). */
void orc_set_threads(int32_t n) { omp_set_num_threads(n > 0 ? n : 1); }
int32_t orc_max_threads(void) { return omp_get_max_threads(); }

/* Token choice of later steps and prefills: temperature 0 = greedy; else
 * orc_sample_row with stream = slot and draw index = the consumed position. */
void orc_model_set_sampling(orc_model* m, float temperature, int32_t top_k, float top_p,
                            uint64_t seed) {
    m->s_top_k = temperature != 0.0f ? top_k : 0;
    m->s_temp = temperature;
    m->s_top_p = top_p;
    m->s_seed = seed;
}

/* Replace a model tensor (ids of orc_model_tensor, plus 12 attention norm,
 * 13 MLP norm, 14 final norm weight) with `data` of the same size: the
 * tests load a checkpoint's tensors into the oracle this way. */
/* A Q8_0 embedding [vocab][hidden] (row-major quants + scales [vocab][hidden/32])
 * in place of the binary16 one: element k of token v is
 * f32(d[v][k/32]) * q[v][k] (exact in binary32), and a tied model's logits
 * become the canonical Q8 product of the Q8_0 final-norm rows with it (the
 * untied lm_head's operations with this matrix). */
void orc_model_set_emb_q8(orc_model* m, const int8_t* qs, const uint16_t* d) {
    const int64_t V = m->c.vocab, H = m->c.hidden;
    free(m->emb_qs);
    free(m->emb_d);
    m->emb_qs = (int8_t*)xmalloc((size_t)(V * H));
    m->emb_d = (uint16_t*)xmalloc((size_t)(V * (H / 32)) * 2);
    memcpy(m->emb_qs, qs, (size_t)(V * H));
    memcpy(m->emb_d, d, (size_t)(V * (H / 32)) * 2);
}

void orc_model_set_tensor(orc_model* m, int32_t layer, int32_t which, const void* data) {
    const orc_qwen_config* c = &m->c;
    int64_t H = c->hidden, I = c->inter, d = c->head_dim, hq = c->n_heads, V = c->vocab;
    int64_t qn = m->qkv_n;
    void* dst = NULL;
    size_t n = 0;
    switch (which) {
        case 0: dst = m->emb; n = (size_t)(V * H * 2); break;
        case 1: dst = m->lm_qs; n = (size_t)(V * H); break;
        case 2: dst = m->lm_d; n = (size_t)(V * (H / 32) * 2); break;
        case 3: dst = m->qkv_qs[layer]; n = (size_t)(qn * H); break;
        case 4: dst = m->qkv_d[layer]; n = (size_t)(qn * (H / 32) * 2); break;
        case 5: dst = m->o_qs[layer]; n = (size_t)(H * hq * d); break;
        case 6: dst = m->o_d[layer]; n = (size_t)(H * (hq * d / 32) * 2); break;
        case 7: dst = m->gu_qs[layer]; n = (size_t)(2 * I * H); break;
        case 8: dst = m->gu_d[layer]; n = (size_t)(2 * I * (H / 32) * 2); break;
        case 9: dst = m->dn_qs[layer]; n = (size_t)(H * I); break;
        case 10: dst = m->dn_d[layer]; n = (size_t)(H * (I / 32) * 2); break;
        case 11: dst = m->bias[layer]; n = (size_t)(qn * 4); break;
        case 12: dst = m->attn_norm[layer]; n = (size_t)(H * 4); break;
        case 13: dst = m->ffn_norm[layer]; n = (size_t)(H * 4); break;
        case 14: dst = m->out_norm; n = (size_t)(H * 4); break;
        default: return;
    }
    if (dst) memcpy(dst, data, n);
}
