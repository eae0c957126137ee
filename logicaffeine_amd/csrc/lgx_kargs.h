// lgx_kargs.h -- kernel argument blocks shared by the host launcher and the
// device code.  Every kernel takes exactly one of these structs by value, so
// hipModuleLaunchKernel is called with kernelParams = { &args }.  Plain C
// layout (pointers, int32, float), identical on x86-64 and amdgcn.
#pragma once
#include <stdint.h>

#define LGX_Q8_RANGE_BLOCKS 32   // blocks of 32 per canonical accumulation range
#define LGX_MAX_RANGES 32        // => K <= 32768
#define LGX_WAVE 64
#define LGX_GLUE_NT 1024         // threads of the row-wise glue kernels (norm, qkv)

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

// Whole-K GEMV (M = 1): one workgroup per 16-row tile of one matrix of a
// group of independent products in a single launch.
#define LGX_GROUP_MAX 8
typedef struct {
    const int8_t* wt;      // T16 quants
    const uint16_t* wd;    // S16 scales
    const float* xf;       // binary32 activation, quantised in the prologue (or NULL)
    const int8_t* xq;      // Q8_0 activation when xf is NULL
    const uint16_t* xd;
    float* y;              // [n]; the range partials [nranges][n] when part_out
    int8_t* xq_out;        // nullable: Q8_0(xf), written by the matrix's first workgroup
    uint16_t* xd_out;
    int32_t* dbg;          // nullable: int32 block dots [n][k/32]
    int32_t n, k, part_out;
    int32_t pad;           // set by the launcher: log2 of the waves per tile
} lgx_gemv_mat;

typedef struct {
    lgx_gemv_mat mat[LGX_GROUP_MAX];
    int32_t tile0[LGX_GROUP_MAX + 1];  // first workgroup of each matrix; tile0[count] = grid
    int32_t count, pad;                // pad: the activation rows of lgx_k_q8_gemm_grpm16
} lgx_gemv_group_args;
#define LGX_GRPM_ROWS 8                // most activation rows of lgx_k_q8_gemm_grpm16

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
    int32_t len_add;           // attended length = seq_len[b] + len_add (decode step: 1)
    float scale;
    int8_t* xq;                // combine+quantise variant: Q8_0 of out rows [B][hq*d]
    uint16_t* xd;
    // prefill (several queries per sequence): row r = b * qpr + j is the query
    // at position seq_len[b] + j, attending to seq_len[b] + j + len_add
    // tokens; B counts sequences, the q / part / out rows are B * qpr.  0 or
    // 1: one query per sequence (decode).
    int32_t qpr;
    int32_t ncg;               // prefill: chunks covered by the grid
    int32_t xq_t16;            // combine+quantise: xq in T16 tiles instead of row-major
    uint16_t* out16;           // fast prefill attention: binary16 out rows [rows][hq*d] (nullable)
} lgx_attn_args;

// Decode attention merge fused with o_proj (K = hq * d <= 1024, one range):
// workgroup = (sequence, group of `tiles` row tiles of o), 16 waves; see
// lgx_k_attn_merge_o_d*.
typedef struct {
    lgx_attn_args at;          // part, nchunk, hq, seq_len, len_add, maxlen of the merge
    const int8_t* wt;          // o_proj T16 quants [n][k]
    const uint16_t* wd;        // o_proj S16 scales
    float* y;                  // [B][n]
    int32_t n, k, ngroups, tiles;  // tiles: row tiles per workgroup, 1..16
} lgx_merge_o_args;

#define LGX_PAGE 16
#define LGX_ATTN_CHUNK 256

// ---- decode-step glue ----
typedef struct {
    const uint16_t* emb;   // [vocab][n] binary16
    const int32_t* tokens; // token of row r = b * qpr + j at tokens[b * tokens_stride + j]
    float* h;              // [m][n]
    int32_t m, n, vocab, tokens_stride;
    int32_t qpr;           // rows per sequence (0 or 1: one)
} lgx_embed_args;
// Gather of a Q8_0 embedding [vocab][n] in T16 / S16 tiles: h[r][i] =
// f32(d) * q of the token's element i (binary32, exact).
typedef struct {
    const int8_t* wt;      // T16 quants
    const uint16_t* wd;    // S16 scales
    const int32_t* tokens;
    float* h;              // [m][n]
    int32_t m, n, vocab, tokens_stride;
    int32_t qpr;
} lgx_embed_q8_args;

// Q8_0 matrix (T16 quants, S16 scales) to binary16 row-major [n][k]:
// out[r][c] = RNE_f16(f32(d[r][c/32]) * q[r][c]).
typedef struct {
    const int8_t* wt;
    const uint16_t* wd;
    uint16_t* out;
    int32_t n, k;
} lgx_dequant_args;

// seq_len[b] = (keep ? seq_len[b] : 0) + add for b < m
typedef struct {
    int32_t* seq_len;
    int32_t m, add, keep;
} lgx_advance_args;

// h += tree(part) (when part != NULL), then y = RMSNorm(h) * w, written as
// binary32 (xn, nullable), binary32 in T16 column order (xt, nullable:
// xt[((row/16) n + i) 16 + row%16], the lm_head's activation layout) and/or
// Q8_0 (xq/xd, nullable).
typedef struct {
    const float* part;     // [nr][m][n] range partials of the residual update
    int32_t nr;
    float* h;              // [m][n]
    const float* w;        // [n] norm weight
    float* xn;
    int8_t* xq;
    uint16_t* xd;
    int32_t m, n;
    float eps;
    float* xt;
    int32_t xq_t16;        // xq in T16 tiles (the tiled product's operand) instead of row-major
    uint16_t* x16;         // binary16 y [m][n] (nullable; the fast prefill's GEMM operand)
} lgx_norm_args;

// qkv = tree(part) (+ bias, nullable); RoPE on the q and k heads at position seq_len[b];
// q -> q_out (binary32), k and v -> binary16 cache slot (page, pos % 16).
typedef struct {
    const float* part;     // [nr][m][(hq+2hkv)d]
    int32_t nr;
    const float* bias;
    const float* cos_t;    // [max_seq][d/2]
    const float* sin_t;
    const int32_t* seq_len;
    const int32_t* page_table;
    uint16_t* kpages;
    uint16_t* vpages;
    float* q_out;          // [m][hq][d]
    int32_t m, hq, hkv, d, maxp, num_pages, max_seq;
    int32_t qpr;           // rows per sequence: row b * qpr + j is position seq_len[b] + j
                           // of sequence b (0 or 1: one row per sequence)
} lgx_qkv_args;

// Decode residual + RMSNorm + Q8_0 fused with the qkv product and its RoPE /
// KV-append consumer (hidden <= 1024, one range): workgroup = (sequence,
// group of LGX_NQ_TILES row tiles of qkv = 128 columns), one wave per tile;
// see lgx_k_norm_qkv_d*.
#define LGX_NQ_TILES 8
#define LGX_NQ_MAXR 8          // partial ranges of the residual's product
typedef struct {
    lgx_qkv_args q;            // consumer: bias, RoPE tables, cache, q_out, heads
    const float* h;            // residual in [B][H]
    const float* part;         // previous products' range partials [nr][B][H] (nr = 0: none)
    float* h_out;              // residual out [B][H] (written by each sequence's group 0)
    const float* w;            // RMSNorm weight [H]
    const int8_t* wt;          // qkv T16 quants [n][H]
    const uint16_t* wd;        // qkv S16 scales
    int32_t nr, H, n, ngroups;
    float eps;
} lgx_norm_qkv_args;

// a = silu(gate) * up from tree(part) ([nr][m][2*inter]), then Q8_0(a)
// (xq/xd) and/or binary32 a (y); each output nullable.
typedef struct {
    const float* part;
    int32_t nr;
    int8_t* xq;
    uint16_t* xd;
    float* y;
    int32_t m, inter;
    int32_t xq_t16;        // xq in T16 tiles instead of row-major
} lgx_swiglu_args;

// Fast prefill SwiGLU: y[r][i] = RNE_f16(silu(g) * u), g = gu[r][i],
// u = gu[r][inter + i], all binary16 ([m][2 inter] -> [m][inter]).
typedef struct {
    const uint16_t* gu;
    uint16_t* y;
    int32_t m, inter;
} lgx_swiglu16_args;

// 16-row streaming product (K in one range, so each output is final in the
// workgroup that computes it) with its consumer applied in the same
// workgroup: the outputs of the workgroup's tiles go to LDS, then
//   LGX_FUSE_QKV:    workgroup = one head of the qkv rows (d / 16 tiles,
//                    tpw = d / 64): bias + RoPE + q_out and the binary16 K/V
//                    append, as lgx_k_qkv_rope_append (q.part, q.nr unused);
//   LGX_FUSE_SWIGLU: workgroup = 32 * cols32 SwiGLU columns c0..: the gate
//                    tiles of those columns and the up tiles at inter + c0
//                    (2 * cols32 tiles each, tpw = cols32); silu(g) * u and
//                    its Q8_0, as lgx_k_swiglu_quant (s.part, s.nr unused).
#define LGX_FUSE_QKV 1
#define LGX_FUSE_SWIGLU 2
typedef struct {
    lgx_gemv_args g;
    lgx_qkv_args q;
    lgx_swiglu_args s;
} lgx_gemm_fused_args;

// logits[m][v] = canonical dot of binary32 x[m] with binary16 row E[v]
// (1024-element ranges, pairwise tree).
typedef struct {
    const float* x;        // [m][h]
    const uint16_t* emb;   // [vocab][h]
    float* logits;         // [m][vocab]
    int32_t m, h, vocab;
} lgx_lmhead_args;

// Binary16 [rows][h] -> T64 units (lgx_k_repack_f16_t64); binary32
// [rows][h] -> T16 column order (lgx_k_rows_to_t16, src/dst as floats).
typedef struct {
    const void* src;
    void* dst;
    int32_t rows, h;
} lgx_t64_args;

// Certified greedy token of a tied binary16 lm_head (lgx_k_lm_cert, then
// lgx_k_lm_pick).  Per (row b, slice of LGX_LMC_ROWS vocabulary rows) the
// first kernel leaves a summary: L, the largest lower bound of a scaled
// logit in the slice; Umax, the largest upper bound; cnt, the number of rows
// whose upper bound reaches L (their bounds and indices in U/v when cnt <=
// LGX_LMC_CAND; LGX_LMC_EXACT when row b needs exact chains everywhere).
#define LGX_LMC_GROUPS 10                      // 64-row groups (waves) per workgroup
#define LGX_LMC_ROWS (64 * LGX_LMC_GROUPS)      // vocabulary rows per slice
#define LGX_LMC_MAXB 32
#define LGX_LMC_MAXH 1024
#define LGX_LMC_CAND 8
#define LGX_LMC_EXACT 0x7fffffff
typedef struct {
    float L, Umax;
    int32_t cnt, pad;
    float U[LGX_LMC_CAND];
    int32_t v[LGX_LMC_CAND];
} lgx_lmc_summary;
typedef struct {
    const float* x;            // [m][h] binary32 rows
    const uint16_t* emb_t64;   // the binary16 embedding in T64 order
    const float* rowc;         // [vocab][4] (lgx_k_lm_rowconst)
    lgx_lmc_summary* summ;     // [m][nslices]
    float* dbg;                // nullable: [m][vocab][2] scaled approximation, bound
    int32_t m, h, vocab, nslices;
} lgx_lmc_args;
typedef struct {
    const float* x;            // [m][h]
    const uint16_t* emb;       // [vocab][h] row-major binary16
    const lgx_lmc_summary* summ;
    int32_t* tokens;           // [m]
    int32_t* seq_len;          // nullable: += advance
    int32_t m, h, vocab, nslices, advance;
} lgx_lmp_args;
// Per-row constants of a binary16 embedding: rowc[v] = upper bounds of
// (sum_k |e[v][k]|, the same sum over the subnormal entries, ||e[v]||_2),
// then 0; +inf in the first three when the row has a non-finite entry.
typedef struct {
    const uint16_t* emb;       // [vocab][h]
    float* rowc;               // [vocab][4]
    int32_t vocab, h;
} lgx_lmrc_args;

// next[b] = first index of the max of tree(part[.][b][:]) (NaN skipped);
// then tokens[b] = next[b] and seq_len[b] += advance.  Two launches through
// per-slice candidates cand_v/cand_i [m][nslices].
#define LGX_ARGMAX_SLICE 4096
typedef struct {
    const float* part;     // [nr][m][vocab]
    int32_t nr;
    int32_t* tokens;
    int32_t* seq_len;
    float* cand_v;
    int32_t* cand_i;
    int32_t m, vocab, advance, nslices;
} lgx_argmax_args;

// Seeded top-k / top-p sampling of m rows of (range-partial) logits.
// lgx_k_sample_partial: per 4096-logit slice, the slice's top_k keys
// (value descending, index ascending; NaN never a candidate) into
// cand[m][nslices][LGX_SAMPLE_MAX_K] (0 = empty).  lgx_k_sample_final: per
// row the top_k keys of the slice lists, then the canonical draw (see
// lgx_sample in lgx.h); tokens[b] = the drawn index, seq_len[b] += advance.
// The draw index of row b is pos[b], or seq_len[b] before the advance when
// pos is NULL; its SplitMix64 stream is `stream0 + b` of `seed`.
#define LGX_SAMPLE_MAX_K 64
typedef struct {
    const float* part;     // [nr][m][vocab]
    int32_t nr;
    int32_t* tokens;
    int32_t* seq_len;
    const int32_t* pos;
    uint64_t* cand;
    uint64_t seed;
    int32_t m, vocab, nslices, top_k, advance, stream0;
    float top_p, inv_temp;
} lgx_sample_args;

// Large-M Q8_0 product (prefill): one workgroup per (64 weight rows, 128
// activation rows, group of LGX_TG_RANGES ranges).  Activations in the T16
// tile layout of the weights (row tiles of 16, 1 KiB per 64-column pair).
// part[g][m][n] = canonical tree over the ranges of group g, so the tree
// over the groups is the tree over all ranges.  With swiglu = I > 0 (a
// gate|up matrix of n = 2I rows, gate rows first, in one group) the outputs
// are not stored: the workgroup runs SwiGLU + Q8_0 on them and writes the
// quants in T16 tiles to sq ([ceil(m/16)][I/64][64][16]) and the scales to
// sd ([m][I/32]), the lgx_k_swiglu_quant operations.
#define LGX_TG_RANGES 4
#define LGX_TG_N 64
#define LGX_TG_M 128
typedef struct {
    const int8_t* wt;      // T16 weights [n/16][k/64][64][16]
    const uint16_t* wd;    // S16 scales
    const int8_t* xt;      // T16 activations [ceil(m/16)][k/64][64][16]
    const uint16_t* xd;    // activation scales [m][k/32]
    float* part;           // [ngroups][m][n]
    int8_t* sq;            // swiglu: T16 quants of the SwiGLU outputs
    uint16_t* sd;          // swiglu: their scales
    int32_t n, k, m, ngroups;
    int32_t ntn, ntm;      // workgroup tiles along n and m
    int32_t grp;           // ranges per group: 1, 2 or 4 (ngroups = ceil(nranges / grp))
    int32_t swiglu;        // I of a fused SwiGLU consumer, else 0
} lgx_gemm_tiled_args;

// Grouped M > 1 products (lgx_q8_gemm_quantize_group): up to
// LGX_MGROUP_MAX independent matrices, m rows each, in three launches.
#define LGX_MGROUP_MAX 8
// Q8_0 of every x[g] ([m][k[g]] binary32) -> xq[g] (row-major, or T16 tiles
// when t16) and xd[g] [m][k/32]; 8 lanes per 32-block, blocks numbered over
// the matrices (blk0[g] = first block of matrix g).
typedef struct {
    const float* x[LGX_MGROUP_MAX];
    int8_t* xq[LGX_MGROUP_MAX];
    uint16_t* xd[LGX_MGROUP_MAX];
    int32_t k[LGX_MGROUP_MAX];
    int64_t blk0[LGX_MGROUP_MAX + 1];
    int32_t m, count, t16;
} lgx_quant_group_args;
// The tiled product of every matrix in one launch: matrix g takes
// workgroups wg0[g] .. wg0[g+1]-1 (a multiple of 8 from the start, so each
// keeps its XCD-aware order; the padding workgroups exit).
typedef struct {
    lgx_gemm_tiled_args mat[LGX_MGROUP_MAX];
    int32_t wg0[LGX_MGROUP_MAX + 1];
    int32_t count;
} lgx_tiled_group_args;
// The 16-row streaming product of every matrix in one launch: matrix g
// takes workgroups wg0[g] .. as its own (gx[g] x nranges) grid, x fastest.
typedef struct {
    lgx_gemv_args mat[LGX_MGROUP_MAX];
    int32_t wg0[LGX_MGROUP_MAX + 1];
    int32_t gx[LGX_MGROUP_MAX];
    int32_t count;
} lgx_stream_group_args;
// y[g][i] = tree over part[g][0..nr[g]) at element i (count m*n of matrix
// g); elements numbered over the matrices from el0[g].
typedef struct {
    const float* part[LGX_MGROUP_MAX];
    float* y[LGX_MGROUP_MAX];
    int32_t nr[LGX_MGROUP_MAX];
    int64_t el0[LGX_MGROUP_MAX + 1];
    int32_t count;
} lgx_combine_group_args;

// Row-major int8 [rows][k] -> T16 tiles of ceil(rows/16) * 16 rows, the rows
// past `rows` zero.
typedef struct {
    const int8_t* src;
    int8_t* dst;
    int32_t rows, k;
} lgx_act_t16_args;
