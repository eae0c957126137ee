// lgx_kargs.h -- kernel argument blocks shared by the host launcher and the
// device code.  Every kernel takes exactly one of these structs by value, so
// hipModuleLaunchKernel is called with kernelParams = { &args }.  Plain C
// layout (pointers, int32, float), identical on x86-64 and amdgcn.
#pragma once
#include <stdint.h>

#define LGX_Q8_RANGE_BLOCKS 32   // blocks of 32 per canonical accumulation range
#define LGX_MAX_RANGES 32        // => K <= 32768
#define LGX_WAVE 64

typedef struct {
    const int8_t* src;
    int8_t* dst;
    int32_t n, k;
    int32_t to_t16;  // 1: row-major -> T16, 0: T16 -> row-major
} lgx_repack_args;

typedef struct {
    const uint16_t* src;
    uint16_t* dst;
    int32_t n, k;
    int32_t to_s16;  // 1: row-major [n][k/32] -> S16, 0: S16 -> row-major
} lgx_srepack_args;

typedef struct {
    const float* x;   // [m][k]
    int8_t* qs;       // [m][k]
    uint16_t* d;      // [m][k/32]
    int32_t m, k;
} lgx_quant_args;

// One wave per (row tile of 16, range of 32 blocks[, m-group of 64 rows]).
typedef struct {
    const int8_t* wt;     // T16 weights
    const uint16_t* wd;   // S16 f16 scales
    const float* xf;      // gemv_f32: x [k]
    const int8_t* xq;     // q8 paths: [m][k]
    const uint16_t* xd;   // q8 paths: [m][nb]
    float* y;             // [m][n] when nranges == 1
    float* part;          // [nranges][m][n] when nranges > 1
    int32_t* dbg;         // nullable: [n][nb] int32 block dots (gemv only)
    int8_t* xq_out;       // fused-quantise GEMV: nullable copy of Q8_0(x) quants
    uint16_t* xd_out;     // fused-quantise GEMV: nullable copy of Q8_0(x) scales
    int32_t n, k, m;
    int32_t ntiles, nranges, nmgroups;
    int32_t tpw;          // streaming kernels: row tiles per wave (per workgroup for
                          // the whole-K GEMV)
} lgx_gemv_args;

// Canonical tree over range partials: y[i] = tree(part[0][i], ..., part[g-1][i]).
typedef struct {
    const float* part;    // [nranges][count]
    float* y;             // [count]
    int64_t count;
    int32_t nranges;
} lgx_combine_args;

// Paged GQA decode attention.  K/V pages: binary16 [num_pages][hkv][16][d].
typedef struct {
    const float* q;            // [B][hq][d]
    const uint16_t* kpages;
    const uint16_t* vpages;
    const int32_t* page_table; // [B][maxp]
    const int32_t* seq_len;    // [B]
    float* part;               // [B][hq][nchunk][d + 2]: o_c[0..d), m_c, l_c
    float* out;                // [B][hq][d]
    int32_t B, hq, hkv, maxp, nchunk, num_pages;
    int32_t maxlen;            // tokens beyond min(max_seq_len, maxp*16) are ignored
    float scale;
} lgx_attn_args;

#define LGX_PAGE 16
#define LGX_ATTN_CHUNK 256
