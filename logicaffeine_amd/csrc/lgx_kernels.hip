// lgx_kernels.hip -- hand-written CDNA4 (gfx950) kernels of the lgx Q8
// LLM-decode hot path.  Built with
//   hipcc --genco --offload-arch=gfx950 -O3 -ffp-contract=off
//         -fhip-fp32-correctly-rounded-divide-sqrt
//         -Xclang -target-feature -Xclang -packed-fp32-ops
// into lgx_kernels.hsaco, loaded by liblgx.so with hipModuleLoad and launched
// with hipModuleLaunchKernel.  Every kernel is `extern "C"` and takes one
// argument block from lgx_kargs.h.
//
// Float discipline: -ffp-contract=off, so a float expression is evaluated
// exactly as written; fused multiply-adds appear only as explicit fmaf().  The
// canonical schedules (Q8 dot: 32-block ranges of sequential fmaf, pairwise
// tree over ranges) are the ones the CPU oracle restates, so the outputs of the
// q8q8 GEMV and the MFMA GEMM are bit-identical to it and to each other.
//
// Reference status: the reference (LOGOS 0.10.1) has no GPU back-end and no
// kernel for any of these operations; the path is specified by the block
// format (GGML Q8_0: 32 int8 + one f16 scale) and the decode step of a
// Qwen2-style model.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lgx_kargs.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Streaming 128-bit load of weight data (read once per call: non-temporal).
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
    const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Raw buffer descriptors (stride 0, range checked in bytes): a load at or
// past num_records returns zeros and touches no memory.  Word 3 is the gfx9
// raw-buffer format (32-bit data format, no swizzle).
#define LGX_BUF_DWORD3 0x00020000
// The same non-temporal 128-bit load through a buffer descriptor (cache
// policy 2: nt).
__device__ __forceinline__ uint4 ld_buf_stream(__amdgpu_buffer_rsrc_t r, int off) {
    const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// The same load through the caches (cache policy 0): data that other
// workgroups of the launch read again.
__device__ __forceinline__ uint4 ld_buf_cached(__amdgpu_buffer_rsrc_t r, int off) {
    const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float h2f(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

__device__ __forceinline__ uint16_t f2h(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ __forceinline__ int shfl_xor_i(int v, int m) { return __shfl_xor(v, m, 64); }
__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, 64); }

// DPP lane moves for the wave reductions (VALU operations, where a shuffle
// is an LDS round trip): quad_perm [1,0,3,2] (0xB1) and [2,3,0,1] (0x4E),
// row_half_mirror (0x141: lane i <- 7 - i of its 8), row_mirror (0x140:
// lane i <- 15 - i of its 16), row_shl:S (0x100 + S: lane i <- lane i + S of
// its 16-lane row).  A lane without a source keeps its own value.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    const int x = __builtin_bit_cast(int, v);
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(x, x, CTRL, 0xf, 0xf, false));
}
// Maximum over each aligned group of 8 lanes, in every lane of the group
// (fmaxf is order-free, so any pairing gives the same value).
__device__ __forceinline__ float max8(float m) {
    m = fmaxf(m, dpp_f<0xB1>(m));
    m = fmaxf(m, dpp_f<0x4E>(m));
    return fmaxf(m, dpp_f<0x141>(m));
}
// Maximum over the wave, in every lane.
__device__ __forceinline__ float wave_max(float m) {
    m = max8(m);
    m = fmaxf(m, dpp_f<0x140>(m));
    m = fmaxf(m, shfl_xor_f(m, 16));
    return fmaxf(m, shfl_xor_f(m, 32));
}
// The halving tree over the wave's 64 slots, lane i += lane i + s for
// s = 32, 16, ..., 1 (the same pairs and order as the shuffle form); the
// sum is lane 0's.
__device__ __forceinline__ float wave_tree_sum(float l) {
    l = l + __shfl_down(l, 32, 64);
    l = l + __shfl_down(l, 16, 64);
    l = l + dpp_f<0x108>(l);
    l = l + dpp_f<0x104>(l);
    l = l + dpp_f<0x102>(l);
    return l + dpp_f<0x101>(l);
}

__device__ __forceinline__ float4 add4(const float4& x, const float4& y) {
    return make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w);
}
// Largest |f| of a lane's four values (the block maximum is the fmaxf of
// these over the block's lanes, in any order).
__device__ __forceinline__ float absmax4(const float (&f)[4]) {
    return fmaxf(fmaxf(fabsf(f[0]), fabsf(f[1])), fmaxf(fabsf(f[2]), fabsf(f[3])));
}
// The lgx_k_quantize_q8_0 rule for four values of a 32-block whose largest
// |value| is am: the packed quants and the binary16 scale.
__device__ __forceinline__ uint32_t quantize4_am(const float (&f)[4], float am, uint16_t& dh) {
    const float d = am / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint32_t qw = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float q = roundf(f[e] * id);
        q = fminf(fmaxf(q, -127.0f), 127.0f);
        qw |= ((uint32_t)(int32_t)q & 0xffu) << (8 * e);
    }
    dh = f2h(d);
    return qw;
}
// Q8_0 of one 32-block held by 8 consecutive lanes (4 values each).
__device__ __forceinline__ uint32_t quantize4(const float (&f)[4], uint16_t& dh) {
    return quantize4_am(f, max8(absmax4(f)), dh);
}

// ---------------------------------------------------------------------------
// T16 repack / unpack.  One thread per 16-byte lane slot of a 1 KiB unit:
// unit u = tile * (k/64) + pair, lane l = r + 16c; the slot holds bytes
// [64p + 8c, +8) and [64p + 32 + 8c, +8) of row 16*tile + r.
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void lgx_k_repack_t16(const lgx_repack_args a) {
    const int64_t np = a.k >> 6;
    const int64_t total = (int64_t)(a.n >> 4) * np * 64;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int64_t u = i >> 6;
    const int lane = (int)(i & 63);
    const int64_t t = u / np, p = u - t * np;
    const int r = lane & 15, c = lane >> 4;
    const int64_t row = t * 16 + r;
    const int64_t off0 = row * a.k + p * 64 + 8 * c;
    uint64_t* t16 = (uint64_t*)(a.to_t16 ? a.dst : a.src) + i * 2;
    uint64_t* rm0 = (uint64_t*)((a.to_t16 ? a.src : a.dst) + off0);
    uint64_t* rm1 = (uint64_t*)((a.to_t16 ? a.src : a.dst) + off0 + 32);
    if (a.to_t16) {
        uint64_t lo = *rm0, hi = *rm1;
        t16[0] = lo;
        t16[1] = hi;
    } else {
        uint64_t lo = t16[0], hi = t16[1];
        *rm0 = lo;
        *rm1 = hi;
    }
}

// ---------------------------------------------------------------------------
// Q8_0 activation quantisation: one thread per 32-block.
//   amax = max|x|, d = amax/127, id = d ? 1/d : 0, q = clamp(round(x*id)),
//   stored scale f16(d) (RNE).
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void lgx_k_quantize_q8_0(const lgx_quant_args a) {
    const int nb = a.k >> 5;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)a.m * nb) return;
    const int64_t row = i / nb, b = i - row * nb;
    const float4* xp = (const float4*)(a.x + row * a.k + b * 32);
    float v[32];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        float4 f = xp[j];
        v[4 * j + 0] = f.x;
        v[4 * j + 1] = f.y;
        v[4 * j + 2] = f.z;
        v[4 * j + 3] = f.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        float t = fabsf(v[j]);
        amax = t > amax ? t : amax;
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint32_t packed[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float q = roundf(v[4 * j + e] * id);
            q = fminf(fmaxf(q, -127.0f), 127.0f);
            w |= ((uint32_t)(int32_t)q & 0xffu) << (8 * e);
        }
        packed[j] = w;
    }
    uint4* qp = (uint4*)(a.qs + row * a.k + b * 32);
    qp[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    qp[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
    a.d[i] = f2h(d);
}

// Pairwise tree with doubling stride over p[0..g) (s = 1, 2, 4, ...:
// p[i] += p[i+s] for i = 0, 2s, ... with i+s < g).  Indices are compile-time,
// so p stays in registers.
__device__ __forceinline__ float tree_sum(float (&p)[LGX_MAX_RANGES], int g) {
#pragma unroll
    for (int s = 1; s < LGX_MAX_RANGES; s <<= 1) {
#pragma unroll
        for (int i = 0; i + s < LGX_MAX_RANGES; i += 2 * s)
            if (i + s < g) p[i] = p[i] + p[i + s];
    }
    return p[0];
}
template <int R>
__device__ __forceinline__ float tree_sum_r(float (&p)[R], int g) {
#pragma unroll
    for (int s = 1; s < R; s <<= 1) {
#pragma unroll
        for (int i = 0; i + s < R; i += 2 * s)
            if (i + s < g) p[i] = p[i] + p[i + s];
    }
    return p[0];
}

// The same tree over the nr (1 <= nr <= LGX_MAX_RANGES, wave-uniform)
// values get(0), ..., get(nr - 1), over the smallest power-of-two width R
// that holds them.  The R reads are unconditional, at indices clamped to
// nr - 1 (the extra values never enter the sum): reads under per-index
// branches would each wait at their join.
template <int R, class F>
__device__ __forceinline__ float tree_read_r(int nr, F get) {
    float p[R];
#pragma unroll
    for (int j = 0; j < R; ++j) p[j] = get(min(j, nr - 1));
    return tree_sum_r<R>(p, nr);
}
template <class F>
__device__ __forceinline__ float tree_read(int nr, F get) {
    static_assert(LGX_MAX_RANGES == 32, "tree_read widths");
    if (nr <= 2) return tree_read_r<2>(nr, get);
    if (nr <= 4) return tree_read_r<4>(nr, get);
    if (nr <= 8) return tree_read_r<8>(nr, get);
    if (nr <= 16) return tree_read_r<16>(nr, get);
    return tree_read_r<32>(nr, get);
}

// Exact int32 sum of the four k-chunk partials of two blocks.  Lane l = r+16c
// holds s0 (block 2p) and s1 (block 2p+1) for its chunk c.  Two VALU lane
// swaps (v_permlane32_swap, v_permlane16_swap) reduce over c; a third brings
// the block-(2p+1) total next to the block-2p total, so that on return lanes
// 0..15 (c = 0) hold both totals of row r.  Each step adds the two results
// of a swap, which makes it independent of which result is which.
__device__ __forceinline__ void reduce_chunks(int& s0, int& s1) {
    const auto a = __builtin_amdgcn_permlane32_swap(s0, s1, false, false);
    const int t = (int)a[0] + (int)a[1];      // lanes 0-31: s0(c)+s0(c+2); 32-63: s1(c-2)+s1(c)
    const auto b = __builtin_amdgcn_permlane16_swap(t, t, false, false);
    const int u = (int)b[0] + (int)b[1];      // lanes 0-31: total s0; lanes 32-63: total s1
    const auto e = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    s0 = u;                                   // valid in lanes 0-31
    s1 = ((int)e[0] + (int)e[1]) - u;         // lanes 0-31: (s0 + s1) - s0
}

__device__ __forceinline__ float reduce_chunks_f(float v) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float t = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(t), __float_as_uint(t), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// ---------------------------------------------------------------------------
// Scale tile layout S16: the scales of row tile t and half-range u (16
// blocks) are 16 rows x 16 binary16, contiguous and row-major, so the 32
// bytes a lane needs for one half-range are two 16-byte loads and the 64
// lanes of a wave touch 512 contiguous bytes.  nhalf = ceil(k/512).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int s16_nhalf(int k) { return (k + 511) >> 9; }

__device__ __forceinline__ void load_scales_half(const uint16_t* wd, int t, int u, int nh, int r,
                                                 uint32_t (&dw)[8]) {
    const uint4* p = (const uint4*)(wd + (((int64_t)t * nh + u) * 16 + r) * 16);
    const uint4 lo = p[0], hi = p[1];
    dw[0] = lo.x; dw[1] = lo.y; dw[2] = lo.z; dw[3] = lo.w;
    dw[4] = hi.x; dw[5] = hi.y; dw[6] = hi.z; dw[7] = hi.w;
}

extern "C" __global__ __launch_bounds__(256) void lgx_k_repack_s16(const lgx_srepack_args a) {
    const int nb = a.k >> 5, nh = s16_nhalf(a.k);
    const int64_t total = (int64_t)(a.n >> 4) * nh * 256;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int j = (int)(i & 15), r = (int)((i >> 4) & 15);
    const int64_t tu = i >> 8;
    const int64_t t = tu / nh;
    const int u = (int)(tu - t * nh);
    const int b = u * 16 + j;
    const int64_t row = t * 16 + r;
    if (a.to_s16)
        a.dst[i] = b < nb ? a.src[row * nb + b] : (uint16_t)0;
    else if (b < nb)
        a.dst[row * nb + b] = a.src[i];
}

// ---------------------------------------------------------------------------
// Ranges: a range is 32 blocks = 16 T16 units = two half-ranges.  Loops run
// over all 16 units with the address clamped to the last valid unit and the
// contribution of units past the range end forced to zero, so the body is
// branch-free and loads overlap the arithmetic.
// ---------------------------------------------------------------------------
struct RangeInfo {
    int g, p0, npairs, b0, nbr;
};

__device__ __forceinline__ RangeInfo range_info(int g, int k) {
    RangeInfo ri;
    const int np = k >> 6;
    ri.g = g;
    ri.p0 = g * (LGX_Q8_RANGE_BLOCKS / 2);
    ri.npairs = min(LGX_Q8_RANGE_BLOCKS / 2, np - ri.p0);
    ri.b0 = g * LGX_Q8_RANGE_BLOCKS;
    ri.nbr = 2 * ri.npairs;
    return ri;
}

// Q8_0 quantisation of activation blocks [blo, bhi) of row x into LDS in the
// T16 activation order: slot (p*4 + c) holds the 8 bytes of chunk c of block
// 2p, then of block 2p+1 (slots numbered from block blo).  Eight threads per
// block, four values each; the arithmetic is lgx_k_quantize_q8_0's, so quants
// and scales are the same.  Threads of one block iterate together.
__device__ __forceinline__ void quantize_blocks_to_lds(const lgx_gemv_args& a, int blo, int bhi,
                                                       int8_t* xs, float* dxs, bool emit) {
    const int j = threadIdx.x & 7;
    for (int bl = (int)(threadIdx.x >> 3); bl < bhi - blo; bl += (int)(blockDim.x >> 3)) {
        const int b = blo + bl;
        const float4 v = *(const float4*)(a.xf + (int64_t)b * 32 + 4 * j);
        float am = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
        am = max8(am);
        const float d = am / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const float f[4] = {v.x, v.y, v.z, v.w};
        uint32_t qw = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float q = roundf(f[e] * id);
            q = fminf(fmaxf(q, -127.0f), 127.0f);
            qw |= ((uint32_t)(int32_t)q & 0xffu) << (8 * e);
        }
        const int p = bl >> 1, hi = bl & 1, c = j >> 1;
        *(uint32_t*)(xs + (p * 4 + c) * 16 + hi * 8 + 4 * (j & 1)) = qw;
        const uint16_t dh = f2h(d);
        if (j == 0) dxs[bl] = h2f(dh);
        if (emit) {
            if (a.xq_out) *(uint32_t*)(a.xq_out + (int64_t)b * 32 + 4 * j) = qw;
            if (a.xd_out && j == 0) a.xd_out[b] = dh;
        }
    }
}

// Stage pairs [plo, phi) of a pre-quantised activation row into LDS (T16
// order) and the scales of their blocks as binary32.
__device__ __forceinline__ void stage_pairs_q8(const lgx_gemv_args& a, int plo, int phi, int8_t* xs,
                                               float* dxs) {
    for (int s = threadIdx.x; s < 4 * (phi - plo); s += blockDim.x) {
        const int8_t* src = a.xq + (plo + (s >> 2)) * 64 + 8 * (s & 3);
        const uint2 lo = *(const uint2*)src;
        const uint2 hi = *(const uint2*)(src + 32);
        *(uint4*)(xs + s * 16) = make_uint4(lo.x, lo.y, hi.x, hi.y);
    }
    for (int b = threadIdx.x; b < 2 * (phi - plo); b += blockDim.x) dxs[b] = h2f(a.xd[2 * plo + b]);
}

// ---------------------------------------------------------------------------
// Q8 x Q8 GEMV (M = 1) on v_dot4_i32_i8, one wave per (row tile, range):
// 128-bit streaming loads of T16 units, dot4 on each lane's 8-byte chunks,
// exact cross-lane chunk sums (reduce_chunks), then the canonical fmaf chain
// of the range.  Also the only kernel that can emit the int32 block dots.
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void lgx_k_q8q8_gemv(const lgx_gemv_args a) {
    __shared__ __align__(16) int8_t xs[LGX_Q8_RANGE_BLOCKS * 32];
    __shared__ __align__(16) float dxs[LGX_Q8_RANGE_BLOCKS];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const RangeInfo ri = range_info(blockIdx.y, a.k);
    const int nb = a.k >> 5, nh = s16_nhalf(a.k);
    stage_pairs_q8(a, ri.p0, ri.p0 + ri.npairs, xs, dxs);
    __syncthreads();
    const int t = blockIdx.x * 4 + wave;
    if (t >= a.ntiles) return;
    const int r = lane & 15, c = lane >> 4;
    const int row = t * 16 + r;
    const int np = a.k >> 6;
    const int last = ri.npairs - 1;
    const uint4* wp = (const uint4*)a.wt + ((int64_t)t * np + ri.p0) * 64 + lane;
    uint4 w[16];
    uint32_t dw[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) w[i] = ld_stream(wp + min(i, last) * 64);
    {
        uint32_t d0[8], d1[8];
        load_scales_half(a.wd, t, 2 * ri.g, nh, r, d0);
        load_scales_half(a.wd, t, min(2 * ri.g + 1, nh - 1), nh, r, d1);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            dw[i] = d0[i];
            dw[8 + i] = d1[i];
        }
    }
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int ic = min(i, last);
        const int4 xv = *(const int4*)(xs + (ic * 4 + c) * 16);
        int s0 = __builtin_amdgcn_sdot4((int)w[i].x, xv.x, 0, false);
        s0 = __builtin_amdgcn_sdot4((int)w[i].y, xv.y, s0, false);
        int s1 = __builtin_amdgcn_sdot4((int)w[i].z, xv.z, 0, false);
        s1 = __builtin_amdgcn_sdot4((int)w[i].w, xv.w, s1, false);
        reduce_chunks(s0, s1);
        const bool on = i <= last;
        const float d0 = on ? h2f(dw[i] & 0xffffu) * dxs[2 * ic] : 0.0f;
        const float d1 = on ? h2f(dw[i] >> 16) * dxs[2 * ic + 1] : 0.0f;
        acc = fmaf((float)s0, d0, acc);
        acc = fmaf((float)s1, d1, acc);
        if (a.dbg != nullptr && on && c == 0) {
            a.dbg[(int64_t)row * nb + ri.b0 + 2 * i] = s0;
            a.dbg[(int64_t)row * nb + ri.b0 + 2 * i + 1] = s1;
        }
    }
    if (c == 0) {
        if (a.nranges == 1)
            a.y[row] = acc;
        else
            a.part[(int64_t)ri.g * a.n + row] = acc;
    }
}

// ---------------------------------------------------------------------------
// Whole-K Q8 x Q8 GEMV (M = 1).  A workgroup of W waves serves W / Wt
// 16-row tiles of one matrix of a group of independent products, Wt waves
// per tile (Wt per matrix, a power of two <= W, so that a wave owns at most
// about 8-16 of the tile's 64-column pairs); tile0 maps workgroups:
//  * every 128-bit load of the first round (a contiguous stretch of the T16
//    array per tile) and the scales of the range chains are requested first;
//  * prologue: the activation, quantised to Q8_0 from binary32 (the
//    lgx_k_quantize_q8_0 rule) or copied, into LDS in (pair, chunk) order;
//  * exact int32 block dots (v_dot4 on each lane's two 8-byte chunks,
//    reduce_chunks across the chunk lanes) go to LDS;
//  * thread (tile, row, range) runs the canonical fmaf chain of its range
//    and thread (tile, row) the pairwise tree over ranges -> y (no partials,
//    no combine launch), or the chains are stored as range partials.
// LDS (dynamic): k bytes of activation, k/32 scales, then per tile 16 x k/32
// block dots and 16 x ranges partials.
// ---------------------------------------------------------------------------
template <int W, int PS>
__device__ __forceinline__ void q8_gemv_wg_body(const lgx_gemv_group_args& ga) {
    extern __shared__ __align__(16) uint8_t lds_dyn[];
    constexpr int NT = 64 * W;                     // PS: pairs per wave per round
    const int bx = blockIdx.x;
    int g = 0;
#pragma unroll 1
    while (g + 1 < ga.count && bx >= ga.tile0[g + 1]) ++g;
    const lgx_gemv_mat& a = ga.mat[g];
    const int lwt = a.pad;                         // log2 of waves per tile
    const int Wt = 1 << lwt, tpw = W >> lwt;
    const int k = a.k, nb = k >> 5, np = k >> 6, nh = s16_nhalf(k);
    const int nr = (nb + LGX_Q8_RANGE_BLOCKS - 1) / LGX_Q8_RANGE_BLOCKS;
    const int ntiles = a.n >> 4;
    const int tile_base = (bx - ga.tile0[g]) * tpw;
    int8_t* xs = (int8_t*)lds_dyn;                 // k bytes, (pair, chunk) order
    float* dxs = (float*)(lds_dyn + k);            // nb
    int* ss = (int*)(dxs + nb);                    // [tpw][nb][16]
    float* ps = (float*)(ss + tpw * nb * 16);      // [tpw][nr][16]
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r = lane & 15, c = lane >> 4;
    const int ts = wave >> lwt, wt = wave & (Wt - 1);
    const int t = tile_base + ts;
    const bool tile_on = t < ntiles;

    const uint4* wp = (const uint4*)a.wt + (int64_t)t * np * 64 + lane;
    uint4 wv[PS];
    if (tile_on) {
#pragma unroll
        for (int i = 0; i < PS; ++i) {
            const int p = wt + Wt * i;
            if (p < np) wv[i] = ld_stream(wp + (int64_t)p * 64);
        }
    }
    // chain thread q = tid: (tile q / (16 nr), row q % 16, range (q / 16) % nr)
    uint32_t dwa[8], dwb[8];
    {
        const int qt = tid / (16 * nr), qg = (tid >> 4) % nr, qr = tid & 15;
        if (qt < tpw && tile_base + qt < ntiles) {
            load_scales_half(a.wd, tile_base + qt, min(2 * qg, nh - 1), nh, qr, dwa);
            load_scales_half(a.wd, tile_base + qt, min(2 * qg + 1, nh - 1), nh, qr, dwb);
        }
    }

    if (a.xf) {
        const bool first = bx == ga.tile0[g];
        for (int s2 = tid; s2 < nb * 8; s2 += NT) {   // 8 lanes per block, whole groups
            const int bl = s2 >> 3, j = s2 & 7;
            const float4 v = *(const float4*)(a.xf + bl * 32 + 4 * j);
            const float f[4] = {v.x, v.y, v.z, v.w};
            uint16_t dh;
            const uint32_t qw = quantize4(f, dh);
            *(uint32_t*)(xs + ((bl >> 1) * 4 + (j >> 1)) * 16 + (bl & 1) * 8 + 4 * (j & 1)) = qw;
            if (j == 0) dxs[bl] = h2f(dh);
            if (first && a.xq_out) {
                *(uint32_t*)(a.xq_out + bl * 32 + 4 * j) = qw;
                if (j == 0) a.xd_out[bl] = dh;
            }
        }
    } else {
        for (int s2 = tid; s2 < 4 * np; s2 += NT) {
            const int8_t* src = a.xq + (s2 >> 2) * 64 + 8 * (s2 & 3);
            const uint2 lo = *(const uint2*)src;
            const uint2 hi = *(const uint2*)(src + 32);
            *(uint4*)(xs + s2 * 16) = make_uint4(lo.x, lo.y, hi.x, hi.y);
        }
        for (int b = tid; b < nb; b += NT) dxs[b] = h2f(a.xd[b]);
    }
    __syncthreads();

    if (tile_on) {
        int* sst = ss + ts * nb * 16;
        const int row = t * 16 + r;
#pragma unroll 1
        for (int p0 = 0; p0 < np; p0 += PS * Wt) {
            if (p0 > 0) {
#pragma unroll
                for (int i = 0; i < PS; ++i) {
                    const int p = p0 + wt + Wt * i;
                    if (p < np) wv[i] = ld_stream(wp + (int64_t)p * 64);
                }
            }
#pragma unroll
            for (int i = 0; i < PS; ++i) {
                const int p = p0 + wt + Wt * i;
                if (p < np) {                      // wave-uniform
                    const int4 xv = *(const int4*)(xs + (p * 4 + c) * 16);
                    int s0 = __builtin_amdgcn_sdot4((int)wv[i].x, xv.x, 0, false);
                    s0 = __builtin_amdgcn_sdot4((int)wv[i].y, xv.y, s0, false);
                    int s1 = __builtin_amdgcn_sdot4((int)wv[i].z, xv.z, 0, false);
                    s1 = __builtin_amdgcn_sdot4((int)wv[i].w, xv.w, s1, false);
                    reduce_chunks(s0, s1);
                    if (c == 0) {
                        sst[(2 * p) * 16 + r] = s0;
                        sst[(2 * p + 1) * 16 + r] = s1;
                        if (a.dbg) {
                            a.dbg[(int64_t)row * nb + 2 * p] = s0;
                            a.dbg[(int64_t)row * nb + 2 * p + 1] = s1;
                        }
                    }
                }
            }
        }
    }
    __syncthreads();

    // canonical chains
#pragma unroll 1
    for (int q = tid; q < tpw * 16 * nr; q += NT) {
        const int qt = q / (16 * nr), qg = (q >> 4) % nr, qr = q & 15;
        const int tq = tile_base + qt;
        if (tq >= ntiles) continue;
        if (q != tid) {
            load_scales_half(a.wd, tq, min(2 * qg, nh - 1), nh, qr, dwa);
            load_scales_half(a.wd, tq, min(2 * qg + 1, nh - 1), nh, qr, dwb);
        }
        const int* sst = ss + qt * nb * 16;
        const int b0 = qg * LGX_Q8_RANGE_BLOCKS;
        const int nbr = min(LGX_Q8_RANGE_BLOCKS, nb - b0);
        float P = 0.0f;
#pragma unroll
        for (int j = 0; j < LGX_Q8_RANGE_BLOCKS; ++j) {
            if (j < nbr) {
                const uint32_t w2 = j < 16 ? dwa[(j & 15) >> 1] : dwb[(j & 15) >> 1];
                const float dwf = h2f((j & 1) ? (w2 >> 16) : (w2 & 0xffffu));
                P = fmaf((float)sst[(b0 + j) * 16 + qr], dwf * dxs[b0 + j], P);
            }
        }
        if (a.part_out)
            a.y[(int64_t)qg * a.n + tq * 16 + qr] = P;
        else
            ps[(qt * nr + qg) * 16 + qr] = P;
    }
    if (a.part_out) return;
    __syncthreads();
    if (tid < tpw * 16) {
        const int qt = tid >> 4, qr = tid & 15;
        const int tq = tile_base + qt;
        if (tq < ntiles) {
            a.y[tq * 16 + qr] = tree_read(nr, [&](int j) { return ps[(qt * nr + j) * 16 + qr]; });
        }
    }
}

extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_gemv_wg4(const lgx_gemv_group_args a) {
    q8_gemv_wg_body<4, 16>(a);
}
extern "C" __global__ __launch_bounds__(512) void lgx_k_q8_gemv_wg8(const lgx_gemv_group_args a) {
    q8_gemv_wg_body<8, 16>(a);
}
extern "C" __global__ __launch_bounds__(1024) void lgx_k_q8_gemv_wg16(const lgx_gemv_group_args a) {
    q8_gemv_wg_body<16, 10>(a);
}

// ---------------------------------------------------------------------------
// Q8 GEMV with a binary32 activation (tolerance-checked path).  Same T16
// walk; x staged in LDS as floats in T16 activation order (slot (p*4+c) =
// 8 floats of block 2p chunk c, then 8 of block 2p+1).  Per lane an 8-term
// float dot per block scaled by d_w, lane-swap sum over the chunks at the end.
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_gemv_f32(const lgx_gemv_args a) {
    __shared__ __align__(16) float xs[LGX_Q8_RANGE_BLOCKS * 32];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const RangeInfo ri = range_info(blockIdx.y, a.k);
    const int nh = s16_nhalf(a.k);
    {
        // thread i: slot i >> 2 (pair p, chunk c), quarter q = i & 3 of its 16 floats
        const int slot = threadIdx.x >> 2, q = threadIdx.x & 3;
        const int p = slot >> 2, c = slot & 3;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (p < ri.npairs)
            v = *(const float4*)(a.xf + (int64_t)(ri.p0 + p) * 64 + (q >> 1) * 32 + 8 * c + 4 * (q & 1));
        *(float4*)(xs + slot * 16 + 4 * q) = v;
    }
    __syncthreads();
    const int t = blockIdx.x * 4 + wave;
    if (t >= a.ntiles) return;
    const int r = lane & 15, c = lane >> 4;
    const int row = t * 16 + r;
    const int np = a.k >> 6;
    const int last = ri.npairs - 1;
    const uint4* wp = (const uint4*)a.wt + ((int64_t)t * np + ri.p0) * 64 + lane;
    uint4 w[16];
    uint32_t dw[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) w[i] = ld_stream(wp + min(i, last) * 64);
    {
        uint32_t d0[8], d1[8];
        load_scales_half(a.wd, t, 2 * ri.g, nh, r, d0);
        load_scales_half(a.wd, t, min(2 * ri.g + 1, nh - 1), nh, r, d1);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            dw[i] = d0[i];
            dw[8 + i] = d1[i];
        }
    }
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float4* xp = (const float4*)(xs + (i * 4 + c) * 16);
        const float4 xa = xp[0], xb = xp[1], xc = xp[2], xd = xp[3];
        const uint32_t q[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
        const float xv0[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
        const float xv1[8] = {xc.x, xc.y, xc.z, xc.w, xd.x, xd.y, xd.z, xd.w};
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            s0 = fmaf((float)(int8_t)(q[j >> 2] >> (8 * (j & 3))), xv0[j], s0);
            s1 = fmaf((float)(int8_t)(q[2 + (j >> 2)] >> (8 * (j & 3))), xv1[j], s1);
        }
        const bool on = i <= last;
        const float t0 = on ? h2f(dw[i] & 0xffffu) : 0.0f;
        const float t1 = on ? h2f(dw[i] >> 16) : 0.0f;
        acc = fmaf(t0, s0, acc);
        acc = fmaf(t1, s1, acc);
    }
    acc = reduce_chunks_f(acc);
    if (c == 0) {
        if (a.nranges == 1)
            a.y[row] = acc;
        else
            a.part[(int64_t)ri.g * a.n + row] = acc;
    }
}

// ---------------------------------------------------------------------------
// Q8 x Q8 GEMV (M = 1) on int8 MFMA, one wave per (row tile, range).
//
// The wave requests its whole tile-range (16 T16 units, 16 KiB, plus the 32
// S16 scales of each of its rows) before the workgroup stages the range's
// activation (or quantises it, QX) and meets the barrier, so the weight
// stream never waits for the activation.  Per block the MFMA, with the
// activation broadcast to all 16 A rows, yields the exact int32 block dots
// of the wave's 16 rows (the hardware sums the four k-chunks); the c = 0
// lanes run the canonical chain.  One range partial per row goes to `y`
// (single range) or `part` (lgx_k_q8_combine applies the tree).
// ---------------------------------------------------------------------------
template <bool QX>
__device__ __forceinline__ void q8_gemv_mfma_body(const lgx_gemv_args& a) {
    __shared__ __align__(16) int8_t xs[LGX_Q8_RANGE_BLOCKS * 32];
    __shared__ __align__(16) float dxs[LGX_Q8_RANGE_BLOCKS];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const RangeInfo ri = range_info(blockIdx.y, a.k);
    const int nh = s16_nhalf(a.k);
    const int t = blockIdx.x * 4 + wave;
    const int tc = min(t, a.ntiles - 1);
    const int r = lane & 15, c = lane >> 4;
    const int np = a.k >> 6;
    const int last = ri.npairs - 1;
    const uint4* wp = (const uint4*)a.wt + ((int64_t)tc * np + ri.p0) * 64 + lane;
    uint4 w[16];
    uint32_t dw[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) w[i] = ld_stream(wp + min(i, last) * 64);
    {
        uint32_t d0[8], d1[8];
        load_scales_half(a.wd, tc, 2 * ri.g, nh, r, d0);
        load_scales_half(a.wd, tc, min(2 * ri.g + 1, nh - 1), nh, r, d1);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            dw[i] = d0[i];
            dw[8 + i] = d1[i];
        }
    }
    if (QX)
        quantize_blocks_to_lds(a, ri.b0, ri.b0 + ri.nbr, xs, dxs, blockIdx.x == 0);
    else
        stage_pairs_q8(a, ri.p0, ri.p0 + ri.npairs, xs, dxs);
    __syncthreads();
    if (t >= a.ntiles) return;
    const v4i zero = {0, 0, 0, 0};
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int ic = min(i, last);
        const bool on = i <= last;
        const uint4 xv = *(const uint4*)(xs + (ic * 4 + c) * 16);
        const long a0 = (long)(((uint64_t)xv.y << 32) | xv.x);
        const long a1 = (long)(((uint64_t)xv.w << 32) | xv.z);
        long b0 = (long)(((uint64_t)w[i].y << 32) | w[i].x);
        long b1 = (long)(((uint64_t)w[i].w << 32) | w[i].z);
        // keep unit i's MFMAs after unit i-1's chain step (volatile empty asm
        // statements stay in order; b0/b1 pass through one, acc the other),
        // so only one unit's products are live at a time
        asm volatile("" : "+v"(b0), "+v"(b1));
        const v4i d0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, b0, zero, 0, 0, 0);
        const v4i d1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, b1, zero, 0, 0, 0);
        const float e0 = on ? h2f(dw[i] & 0xffffu) * dxs[2 * ic] : 0.0f;
        const float e1 = on ? h2f(dw[i] >> 16) * dxs[2 * ic + 1] : 0.0f;
        acc = fmaf((float)d0[0], e0, acc);
        acc = fmaf((float)d1[0], e1, acc);
        asm volatile("" : "+v"(acc));
    }
    if (c == 0) {
        const int row = t * 16 + r;
        if (a.nranges == 1)
            a.y[row] = acc;
        else
            a.part[(int64_t)ri.g * a.n + row] = acc;
    }
}

extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_gemv_mfma(const lgx_gemv_args a) {
    q8_gemv_mfma_body<false>(a);
}
extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_gemv_mfma_qx(const lgx_gemv_args a) {
    q8_gemv_mfma_body<true>(a);
}

// ---------------------------------------------------------------------------
// Grouped Q8 x Q8 GEMV (M = 1), ranges of a tile inside one workgroup.
// A launch covers independent matrices (tile0 maps workgroups to matrices).
// A workgroup of W waves (4, 8 or 16) serves tpw row tiles of one matrix
// (mat.pad, chosen by the launcher to even out the bytes per workgroup, at
// most W / min(ranges, W)); wave (tile slot, range) streams the 16 units of
// its range (all GRP_WIN = 16 128-bit T16 loads in flight), multiplies on
// int8 MFMA with the activation broadcast (D row = block dot of weight row
// r), and runs the canonical fmaf chain of its range (lanes 0-15 hold row r);
// the pairwise tree over the tile's ranges is applied in LDS -> y, or the
// chains are stored as range partials.  Rows of more than W ranges take
// several ranges per wave.
// The activation is staged in LDS as Q8_0 (of binary32 by the
// lgx_k_quantize_q8_0 rule, or a copy) in (pair, chunk) order.  With several
// tiles per workgroup, the tile-slot-0 wave of each range stages it once for
// all of them (slot = range) behind one workgroup barrier, issued after
// every wave's weight loads; with one tile per workgroup each wave stages
// its own range in its own slot, with no barrier before the products.  LDS
// (dynamic): W x (1 KiB quants + 32 scales), then tpw x ranges x 16 chains.
// ---------------------------------------------------------------------------
#define GRP_WIN 16
#define GRP_XSLOT (1024 + 32 * 4)

// The range's activation, lane l holding the 16 values [16l, 16l + 16) of
// the range (block l/2, half l%2): binary32 (4 x 16 bytes) or Q8_0 (16
// quants + the block scale).
template <bool XF>
__device__ __forceinline__ void grp_x_load(const lgx_gemv_mat& a, const RangeInfo& ri, int lane,
                                           uint4 (&xr)[4], uint32_t& xdr) {
    const int bl = min(lane >> 1, ri.nbr - 1);     // lanes past the range re-read its last block
    const int64_t e0 = (int64_t)(ri.b0 + bl) * 32 + 16 * (lane & 1);
    if constexpr (XF) {
#pragma unroll
        for (int u = 0; u < 4; ++u) xr[u] = *(const uint4*)(a.xf + e0 + 4 * u);
        xdr = 0;
    } else {
        xr[0] = *(const uint4*)(a.xq + e0);
        xdr = a.xd[ri.b0 + bl];
    }
}

// Q8_0 of the loaded values (two lanes per block) into the wave's LDS slot;
// the matrix's first workgroup also writes Q8_0(x) out when asked.
template <bool XF>
__device__ __forceinline__ void grp_x_stage(const lgx_gemv_mat& a, const RangeInfo& ri, int lane,
                                            const uint4 (&xr)[4], uint32_t xdr, int8_t* xsw,
                                            float* dxw, bool emit) {
    const int bl = lane >> 1, h = lane & 1;
    uint32_t q[4];
    float dxv;
    uint16_t dh = 0;
    if constexpr (XF) {
        float f[16];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            f[4 * u + 0] = __uint_as_float(xr[u].x);
            f[4 * u + 1] = __uint_as_float(xr[u].y);
            f[4 * u + 2] = __uint_as_float(xr[u].z);
            f[4 * u + 3] = __uint_as_float(xr[u].w);
        }
        float am = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; ++e) am = fmaxf(am, fabsf(f[e]));
        am = fmaxf(am, dpp_f<0xB1>(am));
        const float d = am / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            uint32_t qw = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float v = roundf(f[4 * u + e] * id);
                v = fminf(fmaxf(v, -127.0f), 127.0f);
                qw |= ((uint32_t)(int32_t)v & 0xffu) << (8 * e);
            }
            q[u] = qw;
        }
        dh = f2h(d);
        dxv = h2f(dh);
    } else {
        q[0] = xr[0].x;
        q[1] = xr[0].y;
        q[2] = xr[0].z;
        q[3] = xr[0].w;
        dxv = h2f(xdr);
    }
    if (bl < ri.nbr) {
        // chunks 2h and 2h + 1 of block bl: 8 bytes each in slot (pair, chunk)
        int8_t* base = xsw + ((bl >> 1) * 4 + 2 * h) * 16 + (bl & 1) * 8;
        *(uint2*)base = make_uint2(q[0], q[1]);
        *(uint2*)(base + 16) = make_uint2(q[2], q[3]);
        if (h == 0) dxw[bl] = dxv;
        if constexpr (XF) {
            if (emit && a.xq_out) {
                *(uint4*)(a.xq_out + (int64_t)(ri.b0 + bl) * 32 + 16 * h) =
                    make_uint4(q[0], q[1], q[2], q[3]);
                if (h == 0) a.xd_out[ri.b0 + bl] = dh;
            }
        }
    }
}

// One wave's range, in two halves around the workgroup barrier of the
// shared staging.  grp_issue: the activation loads (only in a wave that
// stages the range), the scale loads and all GRP_WIN weight units, in that
// issue order; grp_chain: per unit, two MFMAs and the canonical chain step
// over the staged activation (quants xs, block scales dx).
struct GrpRegs {
    uint4 xr[4];
    uint32_t xdr;
    uint32_t dw[16];
    uint4 w[16];
};

template <bool XF>
__device__ __forceinline__ void grp_issue(const lgx_gemv_mat& a, int t, const RangeInfo& ri,
                                          int lane, bool stage, GrpRegs& R) {
    const int np = a.k >> 6, nh = s16_nhalf(a.k);
    const int r = lane & 15;
    if (stage) grp_x_load<XF>(a, ri, lane, R.xr, R.xdr);   // wave-uniform
    {
        uint32_t d0[8], d1[8];
        load_scales_half(a.wd, t, 2 * ri.g, nh, r, d0);
        load_scales_half(a.wd, t, min(2 * ri.g + 1, nh - 1), nh, r, d1);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            R.dw[i] = d0[i];
            R.dw[8 + i] = d1[i];
        }
    }
    // the range's units through a buffer descriptor of npairs KiB: all 16
    // loads are issued (the wait counts stay exact), and those past the
    // range fall outside the descriptor, so they read zeros without any
    // memory access
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((const uint4*)a.wt + ((int64_t)t * np + ri.p0) * 64), 0, ri.npairs * 1024,
        LGX_BUF_DWORD3);
#pragma unroll
    for (int i = 0; i < GRP_WIN; ++i) R.w[i] = ld_buf_stream(wr, (i * 64 + lane) * 16);
    __builtin_amdgcn_sched_barrier(0);            // issue order: activation, scales, weights
}

__device__ __forceinline__ float grp_chain(const RangeInfo& ri, int lane, const GrpRegs& R,
                                           const int8_t* xs, const float* dx) {
    const int c = lane >> 4;
    const v4i zero = {0, 0, 0, 0};
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        if (i < ri.npairs) {                       // wave-uniform
            const uint4 xv = *(const uint4*)(xs + (i * 4 + c) * 16);
            const long a0 = (long)(((uint64_t)xv.y << 32) | xv.x);
            const long a1 = (long)(((uint64_t)xv.w << 32) | xv.z);
            const long b0 = (long)(((uint64_t)R.w[i].y << 32) | R.w[i].x);
            const long b1 = (long)(((uint64_t)R.w[i].w << 32) | R.w[i].z);
            const v4i d0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, b0, zero, 0, 0, 0);
            const v4i d1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, b1, zero, 0, 0, 0);
            const float e0 = h2f(R.dw[i] & 0xffffu) * dx[2 * i];
            const float e1 = h2f(R.dw[i] >> 16) * dx[2 * i + 1];
            acc = fmaf((float)d0[0], e0, acc);
            acc = fmaf((float)d1[0], e1, acc);
        }
        // unit i's MFMAs stay after unit i-1's chain step: one unit live at a
        // time, each waiting only for its own weights (no stores in this
        // loop: a store would share the load counter and make the waits
        // conservative; the block-dot debug output is the dot4 kernel's)
        __builtin_amdgcn_sched_barrier(0);
    }
    return acc;
}

// The fields of ga.mat[g] in two wide scalar loads issued together (one
// round trip; field by field, the compiler waits on each load at its first
// use).  The pointers go back to the global address space.
__device__ __forceinline__ lgx_gemv_mat grp_mat(const lgx_gemv_group_args& ga, int g) {
    static_assert(sizeof(lgx_gemv_mat) == 88, "lgx_gemv_mat layout");
    typedef int v16i_t __attribute__((ext_vector_type(16)));
    typedef int v8i_t __attribute__((ext_vector_type(8)));
    // 64 + 32 bytes from the 88-byte record: the last 8 bytes read belong to
    // the next record or to tile0, inside the argument block either way
    const int* src = (const int*)&ga.mat[g];
    const v16i_t lo = *(const v16i_t*)src;
    const v8i_t hi = *(const v8i_t*)(src + 16);
    asm volatile("" ::"s"(lo), "s"(hi));
    auto p64 = [&](int i) {
        const uint32_t l = (uint32_t)(i < 16 ? lo[i] : hi[i - 16]);
        const uint32_t h = (uint32_t)(i + 1 < 16 ? lo[i + 1] : hi[i + 1 - 16]);
        return ((uint64_t)h << 32) | l;
    };
#define LGX_GLOBAL_PTR(T, v) ((T*)(__attribute__((address_space(1))) T*)(v))
    lgx_gemv_mat a;
    a.wt = LGX_GLOBAL_PTR(const int8_t, p64(0));
    a.wd = LGX_GLOBAL_PTR(const uint16_t, p64(2));
    a.xf = LGX_GLOBAL_PTR(const float, p64(4));
    a.xq = LGX_GLOBAL_PTR(const int8_t, p64(6));
    a.xd = LGX_GLOBAL_PTR(const uint16_t, p64(8));
    a.y = LGX_GLOBAL_PTR(float, p64(10));
    a.xq_out = LGX_GLOBAL_PTR(int8_t, p64(12));
    a.xd_out = LGX_GLOBAL_PTR(uint16_t, p64(14));
    a.dbg = LGX_GLOBAL_PTR(int32_t, p64(16));
#undef LGX_GLOBAL_PTR
    a.n = hi[2];
    a.k = hi[3];
    a.part_out = hi[4];
    a.pad = hi[5];
    return a;
}

template <int W, bool XF>
__device__ __forceinline__ void q8_gemv_grp_body(const lgx_gemv_group_args& ga) {
    extern __shared__ __align__(16) uint8_t lds_dyn[];
    const int bx = blockIdx.x;
    // matrix of this workgroup and its first workgroup: tile0 ascends, so g
    // counts the starts at or below bx (all read in one scalar round trip)
    int g = 0, t0 = 0;
#pragma unroll
    for (int j = 1; j < LGX_GROUP_MAX; ++j) {
        const bool in = j < ga.count && bx >= ga.tile0[j];
        g += in ? 1 : 0;
        t0 = in ? ga.tile0[j] : t0;
    }
    const lgx_gemv_mat a = grp_mat(ga, g);
    const int k = a.k, nb = k >> 5;
    const int nr = (nb + LGX_Q8_RANGE_BLOCKS - 1) / LGX_Q8_RANGE_BLOCKS;
    const int nrs = min(nr, W);
    const int tpw = a.pad;                                // >= 1, set by the launcher
    const int ntiles = a.n >> 4;
    const int tile_base = (bx - t0) * tpw;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    float* ps = (float*)(lds_dyn + W * GRP_XSLOT);        // [tpw][nr][16]
    // wave / nrs without an integer division: wave < 16 and nrs <= 16, so
    // (wave + 1/2) / nrs stays at least 1/32 away from an integer, far more
    // than the error of the reciprocal
    const int ts = __builtin_amdgcn_readfirstlane(
        (int)(((float)wave + 0.5f) * __builtin_amdgcn_rcpf((float)nrs)));
    const int rg = wave - ts * nrs;
    const int t = tile_base + ts;
    const bool on = ts < tpw && t < ntiles;
    const bool emit = bx == t0 && ts == 0;                // one wave per range writes Q8_0(x)
    if (tpw > 1) {
        // several tiles per workgroup (so at most W / 2 ranges per row, one
        // per wave): the tile-slot-0 wave of each range stages it once, in
        // slot rg, for every tile of the workgroup
        const RangeInfo ri = range_info(rg, k);
        int8_t* xs = (int8_t*)lds_dyn + rg * GRP_XSLOT;
        float* dx = (float*)(xs + 1024);
        GrpRegs R;
        if (on) {
            grp_issue<XF>(a, t, ri, lane, ts == 0, R);
            if (ts == 0) grp_x_stage<XF>(a, ri, lane, R.xr, R.xdr, xs, dx, emit);
        }
        __syncthreads();
        if (on) {
            const float acc = grp_chain(ri, lane, R, xs, dx);
            if (lane < 16) {
                if (a.part_out)
                    a.y[(int64_t)rg * a.n + t * 16 + lane] = acc;
                else
                    ps[(ts * nr + rg) * 16 + lane] = acc;
            }
        }
    } else if (on) {
        // one tile per workgroup: each wave stages its own range in its own
        // slot (no barrier before the products); rows of more than W ranges
        // take several ranges per wave
        int8_t* xs = (int8_t*)lds_dyn + wave * GRP_XSLOT;
        float* dx = (float*)(xs + 1024);
#pragma unroll 1
        for (int rg2 = rg; rg2 < nr; rg2 += W) {
            const RangeInfo ri = range_info(rg2, k);
            GrpRegs R;
            grp_issue<XF>(a, t, ri, lane, true, R);
            grp_x_stage<XF>(a, ri, lane, R.xr, R.xdr, xs, dx, emit);
            const float acc = grp_chain(ri, lane, R, xs, dx);
            if (lane < 16) {
                if (a.part_out)
                    a.y[(int64_t)rg2 * a.n + t * 16 + lane] = acc;
                else
                    ps[(ts * nr + rg2) * 16 + lane] = acc;
            }
        }
    }
    if (a.part_out) return;
    __syncthreads();
    if (tid < tpw * 16) {
        const int qt = tid >> 4, qr = tid & 15;
        if (tile_base + qt < ntiles) {
            a.y[(tile_base + qt) * 16 + qr] =
                tree_read(nr, [&](int j) { return ps[(qt * nr + j) * 16 + qr]; });
        }
    }
}

// binary32 activations (quantised in the prologue) ...
extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_gemv_grp4(const lgx_gemv_group_args a) {
    q8_gemv_grp_body<4, true>(a);
}
extern "C" __global__ __launch_bounds__(512) void lgx_k_q8_gemv_grp8(const lgx_gemv_group_args a) {
    q8_gemv_grp_body<8, true>(a);
}
extern "C" __global__ __launch_bounds__(1024) void lgx_k_q8_gemv_grp16(const lgx_gemv_group_args a) {
    q8_gemv_grp_body<16, true>(a);
}
// ... and Q8_0 activations (copied)
extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_gemv_grpq4(const lgx_gemv_group_args a) {
    q8_gemv_grp_body<4, false>(a);
}
extern "C" __global__ __launch_bounds__(512) void lgx_k_q8_gemv_grpq8(const lgx_gemv_group_args a) {
    q8_gemv_grp_body<8, false>(a);
}
extern "C" __global__ __launch_bounds__(1024) void lgx_k_q8_gemv_grpq16(const lgx_gemv_group_args a) {
    q8_gemv_grp_body<16, false>(a);
}

// ---------------------------------------------------------------------------
// Grouped Q8 product of 2..LGX_GRPM_ROWS binary32 activation rows in one
// launch (lgx_q8_gemm_quantize_group at small m): the grouped GEMV's grid
// and layout (workgroup = tpw row tiles of one matrix x all its ranges, one
// wave per (tile slot, range); the launcher keeps the ranges <= 16) with the
// m rows as the MFMA's A operand instead of one broadcast row.  The
// workgroup stages each (range, row) of the binary32 activations as Q8_0
// (the GEMV prologue's rule, one (range, row) per wave at a time) into LDS
// slot (range, row) in the (pair, chunk) order, then every wave requests its
// unit stream and scales; after one barrier each wave's block dots come
// from int8 MFMA (lane l: activation rows 4 (l / 16) + v, weight row l % 16;
// rows past m read zeros), the canonical chain per (row, output) over the
// range's blocks, partials to LDS, and the pairwise tree over the ranges
// gives y[row][16 t + r].  Exact like every product: the int32 block dots do
// not depend on how the rows are packed.
// LDS (dynamic): ranges x LGX_GRPM_ROWS x (1 KiB + 32 scales), then
// [tpw][ranges][LGX_GRPM_ROWS][16] partials.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void grpm_chain(const RangeInfo& ri, int lane, int M, const GrpRegs& R,
                                           const uint8_t* xsr, float (&acc)[4]) {
    const int c = lane >> 4, r = lane & 15;
    const uint32_t keep = r < M ? ~0u : 0u;        // A rows past m are zeros
    const uint8_t* xa = xsr + min(r, LGX_GRPM_ROWS - 1) * GRP_XSLOT;
    const v4i zero = {0, 0, 0, 0};
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[v] = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        if (i < ri.npairs) {                       // wave-uniform
            const uint4 xv = *(const uint4*)(xa + (i * 4 + c) * 16);
            const long a0 = (long)(((uint64_t)(xv.y & keep) << 32) | (xv.x & keep));
            const long a1 = (long)(((uint64_t)(xv.w & keep) << 32) | (xv.z & keep));
            const long b0 = (long)(((uint64_t)R.w[i].y << 32) | R.w[i].x);
            const long b1 = (long)(((uint64_t)R.w[i].w << 32) | R.w[i].z);
            const v4i d0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, b0, zero, 0, 0, 0);
            const v4i d1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, b1, zero, 0, 0, 0);
            const float dw0 = h2f(R.dw[i] & 0xffffu), dw1 = h2f(R.dw[i] >> 16);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float* dxr = (const float*)(xsr + min(4 * c + v, LGX_GRPM_ROWS - 1) * GRP_XSLOT + 1024);
                acc[v] = fmaf((float)d0[v], dw0 * dxr[2 * i], acc[v]);
                acc[v] = fmaf((float)d1[v], dw1 * dxr[2 * i + 1], acc[v]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

template <int W>
__device__ __forceinline__ void q8_gemm_grpm_body(const lgx_gemv_group_args& ga) {
    extern __shared__ __align__(16) uint8_t lds_dyn[];
    constexpr int MR = LGX_GRPM_ROWS;
    const int bx = blockIdx.x;
    int g = 0, t0 = 0;
#pragma unroll
    for (int j = 1; j < LGX_GROUP_MAX; ++j) {
        const bool in = j < ga.count && bx >= ga.tile0[j];
        g += in ? 1 : 0;
        t0 = in ? ga.tile0[j] : t0;
    }
    const lgx_gemv_mat a = grp_mat(ga, g);
    const int M = ga.pad;                                 // activation rows, 2..MR
    const int k = a.k, nb = k >> 5;
    const int nr = (nb + LGX_Q8_RANGE_BLOCKS - 1) / LGX_Q8_RANGE_BLOCKS;   // <= W
    const int tpw = a.pad;                                // tiles per workgroup, tpw * nr <= W
    const int ntiles = a.n >> 4;
    const int tile_base = (bx - t0) * tpw;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    uint8_t* xsl = lds_dyn;                               // [nr][MR] slots
    float* ps = (float*)(lds_dyn + nr * MR * GRP_XSLOT);  // [tpw][nr][MR][16]
    // wave / nr without an integer division (wave < 16, nr <= 16: see
    // q8_gemv_grp_body)
    const int ts = __builtin_amdgcn_readfirstlane((int)(((float)wave + 0.5f) * __builtin_amdgcn_rcpf((float)nr)));
    const int rg = wave - ts * nr;
    const int t = tile_base + ts;
    const bool on = ts < tpw && t < ntiles;
    const RangeInfo ri = range_info(rg, k);
    // (range, row) stagings: staging j on wave W - 1 - j % W (the waves
    // without a tile, the highest, take the first ones), round j / W, all
    // before the unit stream is requested (loads complete in issue order: a
    // staging requested after the units would wait for them; config 1 at
    // m = 8, whose down workgroups stage 9 ranges x 8 rows: 16.5 against
    // 17.2 us with the first staging ahead of the units and the others after)
    const int nst = nr * M;
    auto job = [&](int s) { return (W - 1 - wave) + W * s; };
    auto load_job = [&](int j, uint4 (&xr)[4], uint32_t& xdr) {
        const int r2 = j / M, m = j - r2 * M;
        lgx_gemv_mat am = a;
        am.xf = a.xf + (int64_t)m * k;
        grp_x_load<true>(am, range_info(r2, k), lane, xr, xdr);
    };
    auto stage_job = [&](int j, const uint4 (&xr)[4], uint32_t xdr) {
        const int r2 = j / M, m = j - r2 * M;
        int8_t* xs = (int8_t*)xsl + (r2 * MR + m) * GRP_XSLOT;
        grp_x_stage<true>(a, range_info(r2, k), lane, xr, xdr, xs, (float*)(xs + 1024), false);
    };
    uint4 xa[4];
    uint32_t da = 0;
    GrpRegs R;
    for (int s = 0; job(s) < nst; ++s) {
        load_job(job(s), xa, da);
        stage_job(job(s), xa, da);
    }
    if (on) grp_issue<true>(a, t, ri, lane, false, R);  // units and scales, no activation
    __syncthreads();
    if (on) {
        float acc[4];
        grpm_chain(ri, lane, M, R, xsl + rg * MR * GRP_XSLOT, acc);
        const int c = lane >> 4;
        if (c < MR / 4) {
#pragma unroll
            for (int v = 0; v < 4; ++v) ps[((ts * nr + rg) * MR + 4 * c + v) * 16 + (lane & 15)] = acc[v];
        }
    }
    __syncthreads();
    for (int o = tid; o < tpw * M * 16; o += 64 * W) {
        const int qt = o / (M * 16), rem = o - qt * M * 16, row = rem >> 4, col = rem & 15;
        if (tile_base + qt < ntiles)
            a.y[(int64_t)row * a.n + (tile_base + qt) * 16 + col] =
                tree_read(nr, [&](int jj) { return ps[((qt * nr + jj) * MR + row) * 16 + col]; });
    }
}
extern "C" __global__ __launch_bounds__(1024) void lgx_k_q8_gemm_grpm16(const lgx_gemv_group_args a) {
    q8_gemm_grpm_body<16>(a);
}

// ---------------------------------------------------------------------------
// Streaming Q8 x Q8 GEMM on int8 MFMA (v_mfma_i32_16x16x32_i8), M > 1.
//
// grid = (tile groups, ranges, m-groups of MT*16 rows); 4 waves per
// workgroup.  The workgroup stages its activation range once (LDS, MFMA
// A-operand order; scales transposed to [block][row] as binary32), then each
// wave streams `tpw` row tiles (tile = blockIdx.x*4*tpw + 4*j + wave) of the
// range as 8 KiB halves, the next half requested before the current one is
// consumed.  Per block one MFMA per m-tile gives the exact int32 block dots
// D[m][n] (lane l = r + 16c holds n = r, m = 4c + v); the epilogue runs the
// canonical chain acc = fmaf((float)D, dw*dx, acc).  Range partials go to
// `part` (several ranges) and lgx_k_q8_combine applies the tree.
//
// FUSE (LGX_FUSE_QKV / LGX_FUSE_SWIGLU, MT = 1, one range): the tiles of a
// workgroup are the columns its consumer needs (one qkv head; the gate and
// up tiles of 32 * tpw SwiGLU columns), the chains land in LDS instead of
// `y`, and the consumer runs on them after the stream (lgx_gemm_fused_args).
// ---------------------------------------------------------------------------
constexpr int FUSE_COLS = 128;        // LDS columns of a fused workgroup (d <= 128; 2 * 64)
constexpr int QKV_PE = 8;             // qkv consumer elements per thread: 16 rows x d <= 128 / 256
struct QkvPrep {
    int pos[QKV_PE], page[QKV_PE];
    float b0[QKV_PE], b1[QKV_PE], c[QKV_PE], sn[QKV_PE];
};
__device__ __forceinline__ void fused_qkv_prep1(const lgx_qkv_args& q, int head, int m0, int mrows,
                                                QkvPrep& p);
__device__ __forceinline__ void fused_qkv_prep2(const lgx_qkv_args& q, int head, int m0, int mrows,
                                                QkvPrep& p);
__device__ __forceinline__ void fused_qkv_post(const lgx_qkv_args& q, const float* out_s, int ld,
                                               int head, int m0, int mrows, const QkvPrep& p);
__device__ __forceinline__ void fused_swiglu_post(const lgx_swiglu_args& s, const float* out_s, int ld, int cols,
                                  int c0, int m0, int mrows);

template <int MT, int W, int PB, int FUSE = 0>
__device__ __forceinline__ void q8_stream_body(const lgx_gemv_args& a, const lgx_gemm_fused_args* f,
                                               int bx, int by) {
    constexpr int XSLOTS = MT * 16 * 64;   // 16-byte A-operand slots
    constexpr int DXROWS = MT * 16;
    constexpr int NT = 64 * W;
    constexpr int NB = 16 / PB;            // batches per tile-range (16 pairs)
    static_assert(FUSE == 0 || MT == 1, "fused consumers take 16-row m-groups");
    constexpr int FLD = FUSE_COLS + 1;     // fused output row stride (floats)
    __shared__ __align__(16) uint4 xa_s[XSLOTS];
    __shared__ __align__(16) float dx_s[LGX_Q8_RANGE_BLOCKS * DXROWS];
    __shared__ float out_s[FUSE ? 16 * FLD : 1];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const RangeInfo ri = range_info(by, a.k);
    const int nb = a.k >> 5, nh = s16_nhalf(a.k);
    // m-group fastest along x: the groups of one set of row tiles run
    // together and share the weight stream through L2 / MALL
    const int mg = bx % a.nmgroups, tg = bx / a.nmgroups;
    const int m0 = mg * DXROWS;
    const int mrows = min(DXROWS, a.m - m0);
    const int r = lane & 15, c = lane >> 4;
    const int np = a.k >> 6;
    const int last = ri.npairs - 1;
    const int tbase = tg * W * a.tpw + wave;
    const v4i zero = {0, 0, 0, 0};
    // weight tile of the wave's j-th tile; SwiGLU: logical tiles u < half are
    // gate tiles of the workgroup's columns, the others the up tiles
    const int half = W * a.tpw / 2;
    auto tile_of = [&](int j) {
        if constexpr (FUSE == LGX_FUSE_SWIGLU) {
            const int u = wave + W * j;
            return u < half ? tg * half + u : f->s.inter / 16 + tg * half + (u - half);
        } else {
            return tbase + W * j;
        }
    };

    // batch q of tile j: pairs [PB*(q % NB), +PB) of the range; scales of the
    // batch are 2*PB consecutive blocks of the S16 half-range (q*PB)/8
    auto load_batch = [&](int j, int qb, uint4 (&w)[PB], uint32_t (&dw)[PB]) {
        const int t = min(tile_of(j), a.ntiles - 1);
        const uint4* wp = (const uint4*)a.wt + ((int64_t)t * np + ri.p0) * 64 + lane;
#pragma unroll
        for (int i = 0; i < PB; ++i) w[i] = ld_stream(wp + min(PB * qb + i, last) * 64);
        const int pair0 = PB * qb;                 // first pair of the batch
        const int hh = min(2 * ri.g + pair0 / 8, nh - 1);
        const uint4* sp = (const uint4*)(a.wd + (((int64_t)t * nh + hh) * 16 + r) * 16);
        // 8 pairs (16 scales) per 32-byte row: a PB-pair batch (PB = 4 or 8,
        // pair0 a multiple of PB) is the PB words from word pair0 % 8, i.e.
        // PB / 4 whole 16-byte pieces
        static_assert(PB == 4 || PB == 8, "scale words come in 16-byte pieces");
#pragma unroll
        for (int v = 0; v < PB / 4; ++v) {
            const uint4 q = sp[(pair0 % 8) / 4 + v];
            dw[4 * v] = q.x;
            dw[4 * v + 1] = q.y;
            dw[4 * v + 2] = q.z;
            dw[4 * v + 3] = q.w;
        }
    };
    float acc[MT][4];
    // the LDS operands of unit i + 1 (activation slots and scales) are read
    // while unit i's products run
    auto ld_unit = [&](int pc, uint4 (&xv)[MT], float4 (&x0)[MT], float4 (&x1)[MT]) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            xv[mt] = xa_s[(mt * 16 + pc) * 64 + lane];
            x0[mt] = *(const float4*)(dx_s + (2 * pc) * DXROWS + mt * 16 + 4 * c);
            x1[mt] = *(const float4*)(dx_s + (2 * pc + 1) * DXROWS + mt * 16 + 4 * c);
        }
    };
    auto compute_batch = [&](int qb, const uint4 (&w)[PB], const uint32_t (&dw)[PB]) {
        uint4 xvA[MT], xvB[MT];
        float4 x0A[MT], x1A[MT], x0B[MT], x1B[MT];
        ld_unit(min(PB * qb, last), xvA, x0A, x1A);
#pragma unroll
        for (int i = 0; i < PB; ++i) {
            const int pi = PB * qb + i;
            const bool on = pi <= last;
            if (i + 1 < PB) ld_unit(min(pi + 1, last), xvB, x0B, x1B);
            const float dw0 = on ? h2f(dw[i] & 0xffffu) : 0.0f;
            const float dw1 = on ? h2f(dw[i] >> 16) : 0.0f;
            const long b0 = (long)(((uint64_t)w[i].y << 32) | w[i].x);
            const long b1 = (long)(((uint64_t)w[i].w << 32) | w[i].z);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const uint4 xv = xvA[mt];
                const long a0 = (long)(((uint64_t)xv.y << 32) | xv.x);
                const long a1 = (long)(((uint64_t)xv.w << 32) | xv.z);
                const v4i d0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, b0, zero, 0, 0, 0);
                const v4i d1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, b1, zero, 0, 0, 0);
                const float4 x0 = x0A[mt];
                const float4 x1 = x1A[mt];
                acc[mt][0] = fmaf((float)d0[0], dw0 * x0.x, acc[mt][0]);
                acc[mt][1] = fmaf((float)d0[1], dw0 * x0.y, acc[mt][1]);
                acc[mt][2] = fmaf((float)d0[2], dw0 * x0.z, acc[mt][2]);
                acc[mt][3] = fmaf((float)d0[3], dw0 * x0.w, acc[mt][3]);
                acc[mt][0] = fmaf((float)d1[0], dw1 * x1.x, acc[mt][0]);
                acc[mt][1] = fmaf((float)d1[1], dw1 * x1.y, acc[mt][1]);
                acc[mt][2] = fmaf((float)d1[2], dw1 * x1.z, acc[mt][2]);
                acc[mt][3] = fmaf((float)d1[3], dw1 * x1.w, acc[mt][3]);
            }
            // keep each unit's MFMAs next to their epilogue: bounded live
            // ranges (occupancy) instead of all the batch's MFMA results
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                xvA[mt] = xvB[mt];
                x0A[mt] = x0B[mt];
                x1A[mt] = x1B[mt];
            }
        }
    };
    auto store_tile = [&](int j) {
        if constexpr (FUSE != 0) {
            // logical column tile u of the workgroup: LDS row mm, column 16u + r
            const int u = wave + W * j;
#pragma unroll
            for (int v = 0; v < 4; ++v) out_s[(4 * c + v) * FLD + u * 16 + r] = acc[0][v];
            return;
        }
        const int t = tbase + W * j;
        if (t >= a.ntiles) return;
        const int col = t * 16 + r;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int mm = mt * 16 + 4 * c + v;
                const int m = m0 + mm;
                if (mm < mrows) {
                    if (a.nranges == 1)
                        a.y[(int64_t)m * a.n + col] = acc[mt][v];
                    else
                        a.part[((int64_t)ri.g * a.m + m) * a.n + col] = acc[mt][v];
                }
            }
        }
    };

    uint4 wn[PB], wn2[PB];
    uint32_t dn[PB], dn2[PB];
    QkvPrep qp;
    if constexpr (FUSE == LGX_FUSE_QKV) fused_qkv_prep1(f->q, tg, m0, mrows, qp);
    // batches of the range that hold pairs (the last range may be short);
    // the first is requested before the activations are staged, the second
    // right after the staging loads (before their data is waited for), so a
    // short stream (two batches: the small decode products) waits for one
    // memory round, not two
    const int nbq = min(NB, (ri.npairs + PB - 1) / PB);
    const int nbat = nbq * a.tpw;
    load_batch(0, 0, wn, dn);
    if constexpr (FUSE == LGX_FUSE_QKV) fused_qkv_prep2(f->q, tg, m0, mrows, qp);
    // stage the activation range: every load of a thread is requested before
    // the first LDS store (one L2 round trip, not one per slot)
    {
        constexpr int XS = XSLOTS / NT;            // slots per thread
        uint2 lo[XS], hi[XS];
#pragma unroll
        for (int k = 0; k < XS; ++k) {
            const int s = threadIdx.x + k * NT;
            const int mt = s >> 10, pl = (s >> 6) & 15, l = s & 63;
            const int rr = l & 15, cc = l >> 4;
            const int m = m0 + mt * 16 + rr;
            // unconditional loads at clamped addresses, masked to zero after:
            // a load under a branch makes the compiler wait for every load
            // in flight (the weight batches included) where the paths join
            const bool on = m < a.m && pl < ri.npairs;
            const int8_t* src = a.xq + (int64_t)min(m, a.m - 1) * a.k +
                                (ri.p0 + min(pl, ri.npairs - 1)) * 64 + 8 * cc;
            const uint2 l2 = *(const uint2*)src, h2 = *(const uint2*)(src + 32);
            const uint32_t keep = 0u - (uint32_t)on;
            lo[k] = make_uint2(l2.x & keep, l2.y & keep);
            hi[k] = make_uint2(h2.x & keep, h2.y & keep);
        }
        constexpr int DS = LGX_Q8_RANGE_BLOCKS * DXROWS / NT;   // scales per thread
        uint16_t dh[DS];
#pragma unroll
        for (int k = 0; k < DS; ++k) {
            const int s = threadIdx.x + k * NT;
            const int b = s / DXROWS, m = s - b * DXROWS;
            const uint16_t v = a.xd[(int64_t)(m0 + min(m, mrows - 1)) * nb + ri.b0 + min(b, ri.nbr - 1)];
            // a mask, not a select: the compiler turns a select of a load into
            // a branch around it, with a wait for every load at the join
            dh[k] = v & (uint16_t)(0u - (uint32_t)(m < mrows && b < ri.nbr));
        }
        // unconditional (indices clamped inside): under a branch, the join
        // would wait for every load in flight; and nothing that consumes the
        // staging loads is scheduled above it
        load_batch(1 / nbq, 1 % nbq, wn2, dn2);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < XS; ++k)
            xa_s[threadIdx.x + k * NT] = make_uint4(lo[k].x, lo[k].y, hi[k].x, hi[k].y);
#pragma unroll
        for (int k = 0; k < DS; ++k) dx_s[threadIdx.x + k * NT] = h2f(dh[k]);
    }
    __syncthreads();
    // batch q of the wave's stream: zero the chains at a tile's first batch,
    // store them after its last
    auto run_batch = [&](int q, const uint4 (&w)[PB], const uint32_t (&dw)[PB]) {
        const int qb = q % nbq;
        if (qb == 0) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[mt][v] = 0.0f;
        }
        compute_batch(qb, w, dw);
        if (qb == nbq - 1) store_tile(q / nbq);
    };
    // two buffers in turn (no register copies): batch q + 1 is in flight
    // while batch q is consumed, and batch q + 2 is requested into q's
    // buffer as soon as q is done
#pragma unroll 1
    for (int q = 0; q < nbat; q += 2) {
        run_batch(q, wn, dn);
        if (q + 2 < nbat) load_batch((q + 2) / nbq, (q + 2) % nbq, wn, dn);
        if (q + 1 >= nbat) break;
        run_batch(q + 1, wn2, dn2);
        if (q + 3 < nbat) load_batch((q + 3) / nbq, (q + 3) % nbq, wn2, dn2);
    }
    if constexpr (FUSE == LGX_FUSE_QKV) {
        __syncthreads();
        fused_qkv_post(f->q, out_s, FLD, tg, m0, mrows, qp);
    } else if constexpr (FUSE == LGX_FUSE_SWIGLU) {
        __syncthreads();
        fused_swiglu_post(f->s, out_s, FLD, 16 * half, tg * 16 * half, m0, mrows);
    }
}

extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_gemm_mfma16(const lgx_gemv_args a) {
    q8_stream_body<1, 4, 8>(a, nullptr, blockIdx.x, blockIdx.y);
}
extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_gemm_mfma32(const lgx_gemv_args a) {
    q8_stream_body<2, 4, 8>(a, nullptr, blockIdx.x, blockIdx.y);
}
extern "C" __global__ __launch_bounds__(512) void lgx_k_q8_gemm_mfma64(const lgx_gemv_args a) {
    q8_stream_body<4, 8, 4>(a, nullptr, blockIdx.x, blockIdx.y);
}
extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_gemm_mfma16_qkv(const lgx_gemm_fused_args a) {
    q8_stream_body<1, 4, 8, LGX_FUSE_QKV>(a.g, &a, blockIdx.x, blockIdx.y);
}
extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_gemm_mfma16_swiglu(const lgx_gemm_fused_args a) {
    q8_stream_body<1, 4, 8, LGX_FUSE_SWIGLU>(a.g, &a, blockIdx.x, blockIdx.y);
}
// Grouped 16-row streaming products (lgx_stream_group_args): workgroup ->
// (matrix, its own block coordinates).
template <int MT>
__device__ __forceinline__ void q8_stream_group_body(const lgx_stream_group_args& a) {
    const int bid = blockIdx.x;
    int g = 0;
    while (g + 1 < a.count && bid >= a.wg0[g + 1]) ++g;
    const int local = bid - a.wg0[g];
    q8_stream_body<MT, 4, 8>(a.mat[g], nullptr, local % a.gx[g], local / a.gx[g]);
}
extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_gemm_mfma16_group(const lgx_stream_group_args a) {
    q8_stream_group_body<1>(a);
}

// ---------------------------------------------------------------------------
// Range combine: y[i] = canonical pairwise tree over the range partials.
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_combine(const lgx_combine_args a) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= a.count) return;
    a.y[i] = tree_read(a.nranges, [&](int j) { return a.part[j * a.count + i]; });
}

// ---------------------------------------------------------------------------
// Canonical binary32 exp, the same operation sequence as the CPU oracle:
// Cody-Waite reduction x = n ln2 + r (n by the 1.5*2^23 rounding constant,
// ln2 = 0x3f317200 + 1.42860682e-6), degree-7 Taylor polynomial of e^r in
// Horner form with fmaf, scaling through the exponent field.  x < -87.33
// gives +0, x > 88.72 gives +inf, exp(0) == 1.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float lgx_expf(float x) {
    if (x != x) return x;
    if (x > 88.72f) return __builtin_inff();
    if (x < -87.33f) return 0.0f;
    const float t = x * 1.44269504088896341f;
    const float nf = (t + 12582912.0f) - 12582912.0f;
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
    if (n > 127) {
        p = p * 2.0f;
        n -= 1;
    }
    return p * __uint_as_float((uint32_t)(n + 127) << 23);
}

// p of lane J of the lane's 16-lane row (DPP row_newbcast: J is an immediate)
template <int J>
__device__ __forceinline__ float row_bcast(int v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(v, 0x150 + J, 0xf, 0xf, false));
}
template <int J>
struct IdxC {
    static constexpr int value = J;
};
template <int J, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (J < N) {
        f(IdxC<J>{});
        static_for<J + 1, N>(f);
    }
}

// ---------------------------------------------------------------------------
// Paged GQA decode attention, split over 256-token chunks.
//
// grid = (chunks, B * hkv), 256 threads: one workgroup per (sequence, KV
// head, chunk) serves all GQ query heads of the group, so every K/V row is
// read once per group.  Pages: at D = 64 thread t looks up its own token's
// page (no LDS round or barrier before the K loads), at D = 128 the chunk's
// 16 entries go through LDS.  Loads: thread t requests its token's whole K
// row into registers; once it has landed, the workgroup's direct global->LDS
// loads (global_load_lds_dwordx4, 1 KiB per wave instruction) bring the
// first 32 KiB of the chunk's V rows into LDS in token order (the whole
// chunk at D = 64, tokens 0..127 at D = 128; at D = 128 each thread also
// loads 128 bytes of tokens 128..255 into registers), and V lands while the
// scores are computed.  Phase 1: thread t runs the canonical score chain
// over d for the GQ heads (query rows read as workgroup-uniform values).
// Phase 2: per head the chunk max (exact in any order), p_t =
// lgx_expf(s_t - m), and the halving-tree sum of the 256 slots.  Phase 3:
// the canonical chain over the chunk's tokens, o[i] = fmaf(p_t, V_t[i],
// o[i]), for every (head, i).  Partials (o_c, m_c, l_c) go to `part`;
// lgx_k_attn_combine merges the chunks.  LDS: 32 KiB of V + 1088 bytes per
// head.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void;

// The chunk's first 32 KiB of V rows (KV head g, pages pg_s) into v_s in
// token order: wave instruction j moves bytes [1024 j, +1024), which lie in
// page j / (D/32).  Every instruction is issued, so the compiler can count
// them; one for a page past the last token re-reads the chunk's first page
// (a cache hit) into slots that are never used.
template <int D>
__device__ __forceinline__ void attn_stage_v(const lgx_attn_args& a, int g, int n,
                                             const int* pg_s, uint16_t* v_s, int wave, int lane) {
    constexpr int PER_PAGE = LGX_PAGE * D * 2 / 1024;   // wave instructions per page
    constexpr int NJ = 32768 / 1024;
#pragma unroll
    for (int i = 0; i < NJ / 4; ++i) {
        const int j = wave + 4 * i;
        const int u = j / PER_PAGE;
        const int pg = u * LGX_PAGE < n ? pg_s[u] : pg_s[0];
        const uint16_t* src = a.vpages + ((int64_t)pg * a.hkv + g) * LGX_PAGE * D +
                              (j - u * PER_PAGE) * 512 + lane * 8;
        __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)(v_s + j * 512), 16, 0, 0);
    }
}

template <int D, int GQ>
__device__ __forceinline__ void attn_chunk_body(const lgx_attn_args& a) {
    constexpr int C = LGX_ATTN_CHUNK;
    constexpr int VT = 32768 / (2 * D);          // tokens of V in LDS at once
    constexpr int NVS = C / VT;                   // V stages: 1 (D = 64) or 2 (D = 128)
    constexpr int CPR = D / 8;                    // 16-byte pieces per row
    constexpr int NVB = NVS > 1 ? VT * CPR / 256 : 1;   // register pieces per thread
    static_assert(NVS <= 2 && GQ <= 8, "chunk V in at most two 32 KiB stages, 8 heads");
    __shared__ __align__(16) uint16_t v_s[VT * D];
    // p rows padded by 16 floats: rows of neighbouring heads start 16 banks apart
    __shared__ __align__(16) float p_s[GQ][C + 16];
    __shared__ float mx_s[GQ][4];
    __shared__ int pg_s[C / LGX_PAGE];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = blockIdx.x, bg = blockIdx.y;
    const int b = bg / a.hkv, g = bg - b * a.hkv;
    // one load per 64-byte line of the group's query rows, issued first: the
    // rows (written by the previous kernel) travel from memory while the
    // length, pages and K rows do, and the score chain's scalar loads of
    // them hit the cache
    const float qpf = tid < GQ * D / 16 ? a.q[((int64_t)b * a.hq + g * GQ) * D + 16 * tid] : 0.0f;
    const int L = min(a.seq_len[b] + a.len_add, a.maxlen);
    const int t0 = c * C;
    if (t0 >= L) return;                          // whole workgroup: chunk past the end
    const int n = min(C, L - t0);
    const int h0 = g * GQ;
    // D = 64: every thread looks up its own token's page (the last token's
    // past the end: a real slot, never used), so no LDS round and no barrier
    // stand before the K loads; D = 128 shares the chunk's 16 entries in LDS
    int pgt = 0;
    if constexpr (D == 64) {
        pgt = a.page_table[(int64_t)b * a.maxp + (t0 + min(tid, n - 1)) / LGX_PAGE];
        pgt = min(max(pgt, 0), a.num_pages - 1);
    } else {
        if (tid < C / LGX_PAGE) {
            int pg = 0;
            if (t0 + tid * LGX_PAGE < L) pg = a.page_table[(int64_t)b * a.maxp + t0 / LGX_PAGE + tid];
            pg_s[tid] = min(max(pg, 0), a.num_pages - 1);
        }
        __syncthreads();
        pgt = pg_s[tid >> 4];
    }

    // phase 1: scores.  Thread t owns token t; its whole K row is requested
    // before the first use so all of its loads are in flight together (the
    // row address is a real page slot for every thread: pg_s is clamped).
    float s[GQ];
#pragma unroll
    for (int h = 0; h < GQ; ++h) s[h] = 0.0f;
    const bool valid = tid < n;
    uint4 kv[CPR];
    {
        const uint4* kr = (const uint4*)(a.kpages + (((int64_t)pgt * a.hkv + g) * LGX_PAGE + (tid & 15)) * D);
#pragma unroll
        for (int j = 0; j < CPR; ++j) kv[j] = kr[j];
    }
    // the K row has arrived before V is requested: the compiler waits for
    // every outstanding load before the first use of any of them once the
    // LDS loads are in flight, so V's transfer overlaps the score chain only
    // when it is requested after K is in registers
#pragma unroll
    for (int j = 0; j < CPR; ++j)
        asm volatile("" : "+v"(kv[j].x), "+v"(kv[j].y), "+v"(kv[j].z), "+v"(kv[j].w));
    if constexpr (D == 64) {
        // the whole chunk's V (32 KiB): wave w moves its own tokens
        // 64 w .. 64 w + 63 (wave instructions 8 w .. 8 w + 7, two per page),
        // the page of instruction i taken from lane 16 (i / 2)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int j = 8 * wave + i;
            const int pg = __builtin_amdgcn_readlane(pgt, 16 * (i >> 1));
            const uint16_t* src = a.vpages + ((int64_t)pg * a.hkv + g) * LGX_PAGE * D + (i & 1) * 512 + lane * 8;
            __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)(v_s + j * 512), 16, 0, 0);
        }
    } else {
        attn_stage_v<D>(a, g, n, pg_s, v_s, wave, lane);
    }
    // D = 128: tokens VT.. of V, piece q = 256 i + tid of the second stage
    // (coalesced: 16 lanes per row), stored to v_s after the first stage
    // (rows past the chunk's end read a real page slot: pg_s is clamped)
    u32x4 vb[NVB];
    const bool two = NVS > 1 && n > VT;           // uniform in the workgroup
    if constexpr (NVS > 1) {
#pragma unroll
        for (int i = 0; i < NVB; ++i) {
            const int q = 256 * i + tid, tk = VT + q / CPR;
            vb[i] = *(const u32x4*)(a.vpages + (((int64_t)pg_s[tk >> 4] * a.hkv + g) * LGX_PAGE + (tk & 15)) * D +
                                    (q % CPR) * 8);
        }
    }
    __builtin_amdgcn_sched_barrier(0);           // keep every load ahead of the FMAs
    if (valid) {
        // workgroup-uniform query rows through the scalar cache (the LDS
        // loads above would otherwise keep the compiler from proving them
        // read-only and scalar)
        const __attribute__((address_space(4))) float* qb =
            (const __attribute__((address_space(4))) float*)(a.q + ((int64_t)b * a.hq + h0) * D);
        // the heads run in two passes over the K row (fewer query
        // values live in scalar registers at once); each chain is unchanged
        constexpr int HP = (GQ + 1) / 2;
        static_for<0, (GQ + HP - 1) / HP>([&](auto P) {
            constexpr int hlo = P.value * HP, hhi = hlo + HP < GQ ? hlo + HP : GQ;
#pragma unroll
            for (int j = 0; j < CPR; ++j) {
                const float kf[8] = {h2f(kv[j].x & 0xffffu), h2f(kv[j].x >> 16), h2f(kv[j].y & 0xffffu),
                                     h2f(kv[j].y >> 16),     h2f(kv[j].z & 0xffffu), h2f(kv[j].z >> 16),
                                     h2f(kv[j].w & 0xffffu), h2f(kv[j].w >> 16)};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
#pragma unroll
                    for (int h = hlo; h < hhi; ++h) s[h] = fmaf(qb[h * D + 8 * j + e], kf[e], s[h]);
                }
            }
        });
    }
    // phase 2: max, exp, halving-tree sum.  The wave maxima of the heads
    // advance level by level together (independent shuffles in flight at
    // once, not one chain per head)
    {
        float mw[GQ];
#pragma unroll
        for (int h = 0; h < GQ; ++h) {
            s[h] = valid ? s[h] * a.scale : -__builtin_inff();
            mw[h] = s[h];
        }
#pragma unroll
        for (int h = 0; h < GQ; ++h) mw[h] = wave_max(mw[h]);
        if (lane == 0) {
#pragma unroll
            for (int h = 0; h < GQ; ++h) mx_s[h][wave] = mw[h];
        }
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < GQ; ++h) {
        const float m = fmaxf(fmaxf(mx_s[h][0], mx_s[h][1]), fmaxf(mx_s[h][2], mx_s[h][3]));
        p_s[h][tid] = valid ? lgx_expf(s[h] - m) : 0.0f;
    }
    __builtin_amdgcn_s_waitcnt(0);               // this wave's first-stage V is in LDS
    __syncthreads();                             // ... and every other wave's, and p
    {
        // head h's sum on wave h % 4: levels 128 and 64 of the tree from
        // p_s, the rest across lanes
#pragma unroll
        for (int h0w = 0; h0w < GQ; h0w += 4) {
            const int h = h0w + wave;
            if (h < GQ) {
                float l = (p_s[h][lane] + p_s[h][lane + 128]) + (p_s[h][lane + 64] + p_s[h][lane + 192]);
                l = wave_tree_sum(l);
                if (lane == 0) {
                    const float m = fmaxf(fmaxf(mx_s[h][0], mx_s[h][1]), fmaxf(mx_s[h][2], mx_s[h][3]));
                    float* pp = a.part + (((int64_t)b * a.hq + h0 + h) * a.nchunk + c) * (D + 2);
                    pp[D] = m;
                    pp[D + 1] = l;
                }
            }
        }
    }
    // phase 3: o_c[i] = chain_t fmaf(p_t, V_t[i], o).  n is
    // workgroup-uniform, so the loop bounds do not diverge.
    if constexpr (D == 64) {
        // thread = (dimension pair, head group) reads its pair of each V
        // row from LDS (a wave reads whole rows, conflict-free), four
        // tokens per step with p as one float4
        constexpr int NP = D / 2;                 // dimension pairs
        constexpr int NHG = 256 / NP;             // head groups
        constexpr int HPG = (GQ + NHG - 1) / NHG; // heads per group
        const int ip = tid % NP, hg = tid / NP;
        float o[HPG][2];
#pragma unroll
        for (int k = 0; k < HPG; ++k) o[k][0] = o[k][1] = 0.0f;
        const uint32_t* vs = (const uint32_t*)v_s + ip;
        int t = 0;
        // 16 tokens per step: every read of the step (V pairs, p as float4)
        // issued before the chains
        for (; t + 16 <= n; t += 16) {
            uint32_t vv[16];
            float4 p4[HPG][4];
#pragma unroll
            for (int u = 0; u < 16; ++u) vv[u] = vs[(t + u) * NP];
#pragma unroll
            for (int k = 0; k < HPG; ++k) {
                const int h = min(hg + NHG * k, GQ - 1);
#pragma unroll
                for (int q = 0; q < 4; ++q) p4[k][q] = *(const float4*)&p_s[h][t + 4 * q];
            }
#pragma unroll
            for (int k = 0; k < HPG; ++k) {
                if (hg + NHG * k < GQ) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float pt[4] = {p4[k][q].x, p4[k][q].y, p4[k][q].z, p4[k][q].w};
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            o[k][0] = fmaf(pt[u], h2f(vv[4 * q + u] & 0xffffu), o[k][0]);
                            o[k][1] = fmaf(pt[u], h2f(vv[4 * q + u] >> 16), o[k][1]);
                        }
                    }
                }
            }
        }
        for (; t + 4 <= n; t += 4) {
            uint32_t vv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) vv[u] = vs[(t + u) * NP];
#pragma unroll
            for (int k = 0; k < HPG; ++k) {
                const int h = hg + NHG * k;
                if (h < GQ) {
                    const float4 p4 = *(const float4*)&p_s[h][t];
                    const float pt[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        o[k][0] = fmaf(pt[u], h2f(vv[u] & 0xffffu), o[k][0]);
                        o[k][1] = fmaf(pt[u], h2f(vv[u] >> 16), o[k][1]);
                    }
                }
            }
        }
        for (; t < n; ++t) {
            const uint32_t v = vs[t * NP];
#pragma unroll
            for (int k = 0; k < HPG; ++k) {
                const int h = hg + NHG * k;
                if (h < GQ) {
                    const float pt = p_s[h][t];
                    o[k][0] = fmaf(pt, h2f(v & 0xffffu), o[k][0]);
                    o[k][1] = fmaf(pt, h2f(v >> 16), o[k][1]);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < HPG; ++k) {
            const int h = hg + NHG * k;
            if (h < GQ) {
                float* pp = a.part + (((int64_t)b * a.hq + h0 + h) * a.nchunk + c) * (D + 2) + 2 * ip;
                pp[0] = o[k][0];
                pp[1] = o[k][1];
            }
        }
    } else {
        // D = 128, all four waves: wave w = (head group hgp = w % HGN,
        // dimension slice dq = w / HGN); 16-lane row rho is head 4 hgp + rho,
        // lane k owns DL dimensions of the slice.  The row's p_t comes from
        // lane t%16 of a 16-token register (DPP row_newbcast), V_t from LDS
        // (a row reads 16 DL consecutive halves, the four rows the same ones).
        constexpr int HGN = (GQ + 3) / 4;         // head groups of 4
        constexpr int WPD = 4 / HGN;              // dimension slices
        constexpr int DL = D / WPD / 16;          // dimensions per lane: 1, 2 or 4
        const int hgp = wave % HGN, dq = wave / HGN;
        const int rho = lane >> 4, k = lane & 15;
        const int h = 4 * hgp + rho, hc = min(h, GQ - 1);
        const int dcol = dq * (D / WPD) + DL * k;
        float o[DL];
#pragma unroll
        for (int e = 0; e < DL; ++e) o[e] = 0.0f;
        // a lane's DL halves of V row tl (as 2 words; DL <= 4)
        auto v_load = [&](int tl) -> uint2 {
            if constexpr (DL == 4) return *(const uint2*)(v_s + tl * D + dcol);
            else if constexpr (DL == 2) return make_uint2(*(const uint32_t*)(v_s + tl * D + dcol), 0u);
            else return make_uint2(v_s[tl * D + dcol], 0u);
        };
        auto pv_apply = [&](const uint2 vv, float pb) {
            const float vf[4] = {h2f(vv.x & 0xffffu), h2f(vv.x >> 16), h2f(vv.y & 0xffffu), h2f(vv.y >> 16)};
#pragma unroll
            for (int e = 0; e < DL; ++e) o[e] = fmaf(pb, vf[e], o[e]);
        };
        auto pv_token = [&](int tl, float pb) { pv_apply(v_load(tl), pb); };   // tl: row of the V stage
        auto pv_stage = [&](int tb) {            // tokens [tb, min(n, tb + VT)) from v_s
            const int te = min(n, tb + VT);
            for (int ts = tb; ts < te; ts += 16) {
                // p of the 16 tokens: four 16-byte reads at one address per
                // 16-lane row (LDS broadcast), no VALU work per token
                float pt[16];
                static_for<0, 4>([&](auto Q) {
                    const float4 p4 = *(const float4*)&p_s[hc][ts + 4 * Q.value];
                    pt[4 * Q.value] = p4.x;
                    pt[4 * Q.value + 1] = p4.y;
                    pt[4 * Q.value + 2] = p4.z;
                    pt[4 * Q.value + 3] = p4.w;
                });
                if (ts + 16 <= te) {
                    // the 16 rows' reads issued together, then the chains
                    uint2 vv[16];
                    static_for<0, 16>([&](auto J) { vv[J.value] = v_load(ts + J.value - tb); });
                    static_for<0, 16>([&](auto J) { pv_apply(vv[J.value], pt[J.value]); });
                } else {
                    static_for<0, 16>([&](auto J) {
                        if (ts + J.value < te) pv_token(ts + J.value - tb, pt[J.value]);
                    });
                }
            }
        };
        pv_stage(0);
        if (two) {
            __syncthreads();                      // the first stage is fully read
#pragma unroll
            for (int i = 0; i < NVB; ++i) *(u32x4*)(v_s + (256 * i + tid) * 8) = vb[i];
            __syncthreads();
            pv_stage(VT);
        }
        if (h < GQ) {
            float* pp = a.part + (((int64_t)b * a.hq + h0 + h) * a.nchunk + c) * (D + 2) + dcol;
#pragma unroll
            for (int e = 0; e < DL; ++e) pp[e] = o[e];
        }
    }
    // the prefetch's value is never used; this keeps its load in the code
    if (qpf != qpf && a.len_add == 0x7fffffff) a.part[0] = qpf;
}

// Merge of the chunk partials of one (sequence, query head): M = max m_c,
// w_c = lgx_expf(m_c - M), L = chain fmaf(w_c, l_c), O[i] = chain
// fmaf(w_c, o_c[i]), out = O / L (0 for an empty sequence).  One workgroup of
// D threads per (sequence, head), called by every thread.  The maxima are
// read with one load per thread and chunk stride D (the max is exact in any
// order); w_c and l_c of up to 256 chunks at a time go to LDS, computed once
// per chunk; thread i then runs both chains in chunk order.  Up to 32 chunks,
// every partial a thread needs is requested at once (one memory round); past
// that its o_c[i] are loaded 16 chunks at a time, the next 16 in flight while
// the current 16 enter the chains.
//
// Loads of the partials pp[(c, j)] = pp[c * (D + 2) + j] of chunks c < nch
// through a buffer descriptor: every load is issued (no load under a branch,
// whose join would wait for every load in flight), and those of chunks at or
// past nch read zeros without a memory access.
template <int D>
struct MergeRd {
    __amdgpu_buffer_rsrc_t r;
    __device__ MergeRd(const float* pp, int nch)
        : r(__builtin_amdgcn_make_buffer_rsrc((void*)pp, 0, nch * (D + 2) * 4, LGX_BUF_DWORD3)) {}
    __device__ float operator()(int c, int j) const {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (c * (D + 2) + j) * 4, 0, 0));
    }
};

// One memory round for up to FC (<= D) chunks: every partial this thread may
// need (chunk i's m and l, o_c[i] of every chunk) requested together with
// the length; chunks at or past nc are never used.
template <int D, int FC>
__device__ __forceinline__ float attn_merge_one_round(const lgx_attn_args& a, const float* pp, int row,
                                                      int b, int qpr, float* w_s, float* l_s,
                                                      float* red_s) {
    const int i = threadIdx.x, lane = i & 63, wave = i >> 6;
    const MergeRd<D> rd(pp, a.nchunk);
    const float mc = rd(i, D), lc = rd(i, D + 1);
    float ov[FC];
#pragma unroll
    for (int c = 0; c < FC; ++c) ov[c] = rd(c, i);
    const int L = min(a.seq_len[b] + (row - b * qpr) + a.len_add, a.maxlen);
    const int nc = (max(L, 0) + LGX_ATTN_CHUNK - 1) / LGX_ATTN_CHUNK;
    float M = wave_max(i < nc ? mc : -__builtin_inff());
    if constexpr (D > 64) {
        if (lane == 0) red_s[wave] = M;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < D / 64; ++w) M = fmaxf(M, red_s[w]);
    }
    if (i < nc) {
        w_s[i] = lgx_expf(mc - M);
        l_s[i] = lc;
    }
    __syncthreads();
    float Ls = 0.0f, O = 0.0f;
#pragma unroll
    for (int c = 0; c < FC; ++c) {
        if (c < nc) {                             // uniform
            Ls = fmaf(w_s[c], l_s[c], Ls);
            O = fmaf(w_s[c], ov[c], O);
        }
    }
    return nc > 0 ? O / Ls : 0.0f;
}

template <int D>
__device__ __forceinline__ float attn_merge(const lgx_attn_args& a, int bh) {
    constexpr int TCH = 256;                      // chunks per LDS tile
    __shared__ float w_s[TCH], l_s[TCH], red_s[D / 64];
    const int i = threadIdx.x, lane = i & 63, wave = i >> 6;
    const int qpr = max(a.qpr, 1);
    const int row = bh / a.hq, b = row / qpr;
    const float* pp = a.part + (int64_t)bh * a.nchunk * (D + 2);
    if (a.nchunk <= 16) return attn_merge_one_round<D, 16>(a, pp, row, b, qpr, w_s, l_s, red_s);
    if (a.nchunk <= 32) return attn_merge_one_round<D, 32>(a, pp, row, b, qpr, w_s, l_s, red_s);
    // chunk i's m and l and the first 16 o_c[i] requested with the length
    // (values past nc are never used)
    const MergeRd<D> rd0(pp, a.nchunk);
    const float mc = rd0(i, D), lc = rd0(i, D + 1);
    float ov[16], on[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) ov[u] = rd0(u, i);
    const int L = min(a.seq_len[b] + (row - b * qpr) + a.len_add, a.maxlen);
    const int nc = (max(L, 0) + LGX_ATTN_CHUNK - 1) / LGX_ATTN_CHUNK;
    float M = i < nc ? mc : -__builtin_inff();
    for (int c = i + D; c < nc; c += D) M = fmaxf(M, pp[c * (D + 2) + D]);
    M = wave_max(M);
    if (lane == 0) red_s[wave] = M;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < D / 64; ++w) M = fmaxf(M, red_s[w]);
    float Ls = 0.0f, O = 0.0f;
    for (int c0 = 0; c0 < nc; c0 += TCH) {        // nc is uniform: every thread takes the barriers
        const int cn = min(TCH, nc - c0);
        __syncthreads();                          // the previous tile is consumed
        int c = i;
        if (c0 == 0 && i < cn) {                  // chunk i from the registers
            w_s[i] = lgx_expf(mc - M);
            l_s[i] = lc;
            c += D;
        }
        for (; c < cn; c += D) {
            const float* q = pp + (c0 + c) * (D + 2);
            w_s[c] = lgx_expf(q[D] - M);
            l_s[c] = q[D + 1];
        }
        __syncthreads();
        // o_c[i] 16 chunks at a time, the next 16 requested before the
        // current 16 enter the chains (the values past cn are never used)
        const MergeRd<D> rd(pp + (int64_t)c0 * (D + 2), cn);
        if (c0 > 0) {
#pragma unroll
            for (int u = 0; u < 16; ++u) ov[u] = rd(u, i);
        }
        for (int c = 0; c < cn; c += 16) {
#pragma unroll
            for (int u = 0; u < 16; ++u) on[u] = rd(c + 16 + u, i);
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                if (c + u < cn) {                 // uniform
                    Ls = fmaf(w_s[c + u], l_s[c + u], Ls);
                    O = fmaf(w_s[c + u], ov[u], O);
                }
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) ov[u] = on[u];
        }
    }
    return nc > 0 ? O / Ls : 0.0f;
}

template <int D>
__device__ __forceinline__ void attn_combine_body(const lgx_attn_args& a) {
    const int bh = blockIdx.x;
    a.out[(int64_t)bh * D + threadIdx.x] = attn_merge<D>(a, bh);
}

#define LGX_ATTN_KERNELS(D, G)                                                                    \
    extern "C" __global__ __launch_bounds__(256) void lgx_k_attn_chunk_d##D##_g##G(              \
        const lgx_attn_args a) {                                                                 \
        attn_chunk_body<D, G>(a);                                                                \
    }
LGX_ATTN_KERNELS(64, 1)
LGX_ATTN_KERNELS(64, 2)
LGX_ATTN_KERNELS(64, 3)
LGX_ATTN_KERNELS(64, 4)
LGX_ATTN_KERNELS(64, 5)
LGX_ATTN_KERNELS(64, 6)
LGX_ATTN_KERNELS(64, 7)
LGX_ATTN_KERNELS(64, 8)
LGX_ATTN_KERNELS(128, 1)
LGX_ATTN_KERNELS(128, 2)
LGX_ATTN_KERNELS(128, 3)
LGX_ATTN_KERNELS(128, 4)
LGX_ATTN_KERNELS(128, 5)
LGX_ATTN_KERNELS(128, 6)
LGX_ATTN_KERNELS(128, 7)
LGX_ATTN_KERNELS(128, 8)

extern "C" __global__ __launch_bounds__(128) void lgx_k_attn_combine_d128(const lgx_attn_args a) {
    attn_combine_body<128>(a);
}
extern "C" __global__ __launch_bounds__(64) void lgx_k_attn_combine_d64(const lgx_attn_args a) {
    attn_combine_body<64>(a);
}

// ---------------------------------------------------------------------------
// Decode-step glue.  Each kernel applies the canonical range tree to the
// partials of the product before it (so no separate combine launch), then
// the element-wise step, then (where the next product needs it) the Q8_0
// quantisation of its output row.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float lgx_silu(float g) {
    const float e = lgx_expf(-g);
    const float den = 1.0f + e;
    return g / den;
}

// tree over nr partials of element i (stride = elements per partial)
__device__ __forceinline__ float tree_partials(const float* part, int nr, int64_t stride,
                                               int64_t i) {
    return tree_read(nr, [&](int j) { return part[j * stride + i]; });
}

// Byte offset of element (row m, column i) of an m x k int8 activation held
// in T16 tiles (the tiled product's operand: 1 KiB per 16 rows x 64
// columns, lane (r + 16 c) holding bytes [8c, +8) of both blocks of row r);
// four bytes from a column i % 4 == 0 stay contiguous.
__device__ __forceinline__ int64_t t16_off(int64_t m, int i, int k) {
    return ((m >> 4) * (k >> 6) + (i >> 6)) * 1024 + ((m & 15) + 16 * ((i & 31) >> 3)) * 16 +
           ((i & 63) >> 5) * 8 + (i & 7);
}
__device__ __forceinline__ int64_t xq_off(int64_t m, int i, int k, bool t16) {
    return t16 ? t16_off(m, i, k) : m * k + i;
}

// Quantise row m held in LDS (n floats, n % 32 == 0) into the n-column
// matrix xq (row-major or T16) and its scales xd[m][n/32] with NT threads:
// 8 threads per block, the 8 lanes of a block always active together.
template <int NT>
__device__ __forceinline__ void quantize_row_from_lds(const float* row, int n, int8_t* xq,
                                                      uint16_t* xd, int64_t m, bool t16) {
    const int j = threadIdx.x & 7;
    for (int bl = threadIdx.x >> 3; bl < n / 32; bl += NT / 8) {
        const float f[4] = {row[bl * 32 + 4 * j], row[bl * 32 + 4 * j + 1], row[bl * 32 + 4 * j + 2],
                            row[bl * 32 + 4 * j + 3]};
        uint16_t dh;
        const uint32_t qw = quantize4(f, dh);
        *(uint32_t*)(xq + xq_off(m, bl * 32 + 4 * j, n, t16)) = qw;
        if (j == 0) xd[m * (n / 32) + bl] = dh;
    }
}

// Canonical tree over the nr (1 <= nr <= R, wave-uniform) range partials of
// NE elements i0, i0 + di, ... of one thread (0 where on[e] is false), with
// every load issued before the first add.  The loads are unconditional over
// the smallest power-of-two width W >= nr: partial indices clamped to
// nr - 1, and an element that is off reads element 0 (always present) and
// is dropped at the end; loads under per-element branches would each wait
// at their join.
template <int NE, int W>
__device__ __forceinline__ void tree_partials_w(const float* part, int nr, int64_t stride,
                                                int64_t i0, int64_t di, const bool (&on)[NE],
                                                float (&out)[NE]) {
    float p[NE][W];
#pragma unroll
    for (int j = 0; j < W; ++j)
#pragma unroll
        for (int e = 0; e < NE; ++e)
            p[e][j] = part[min(j, nr - 1) * stride + (on[e] ? i0 + e * di : 0)];
#pragma unroll
    for (int e = 0; e < NE; ++e) out[e] = on[e] ? tree_sum_r<W>(p[e], nr) : 0.0f;
}
template <int NE, int R>
__device__ __forceinline__ void tree_partials_n(const float* part, int nr, int64_t stride,
                                                int64_t i0, int64_t di, const bool (&on)[NE],
                                                float (&out)[NE]) {
    static_assert(R == 8 || R == 32, "tree_partials_n widths");
    if (nr <= 1)
        tree_partials_w<NE, 1>(part, nr, stride, i0, di, on, out);
    else if (nr <= 2)
        tree_partials_w<NE, 2>(part, nr, stride, i0, di, on, out);
    else if (nr <= 4)
        tree_partials_w<NE, 4>(part, nr, stride, i0, di, on, out);
    else if (R == 8 || nr <= 8)
        tree_partials_w<NE, 8>(part, nr, stride, i0, di, on, out);
    else if (nr <= 16)
        tree_partials_w<NE, (R > 16 ? 16 : R)>(part, nr, stride, i0, di, on, out);
    else
        tree_partials_w<NE, R>(part, nr, stride, i0, di, on, out);
}

extern "C" __global__ __launch_bounds__(256) void lgx_k_embed(const lgx_embed_args a) {
    const int row = blockIdx.x, qpr = max(a.qpr, 1), b = row / qpr;
    const int tok = min(max(a.tokens[(int64_t)b * a.tokens_stride + (row - b * qpr)], 0), a.vocab - 1);
    const uint16_t* er = a.emb + (int64_t)tok * a.n;
    for (int i = threadIdx.x; i < a.n; i += 256) a.h[(int64_t)row * a.n + i] = h2f(er[i]);
}

// Q8_0 embedding rows (a checkpoint's token_embd stored as Q8_0): element i
// of token v is f32(d[v][i/32]) * q[v][i], read from the T16 quant tiles
// (byte 8(i%64 >= 32) + i%8 of lane v%16 + 16 (i%32)/8 in unit (v/16, i/64))
// and the S16 scale tiles.
extern "C" __global__ __launch_bounds__(256) void lgx_k_embed_q8(const lgx_embed_q8_args a) {
    const int row = blockIdx.x, qpr = max(a.qpr, 1), b = row / qpr;
    const int tok = min(max(a.tokens[(int64_t)b * a.tokens_stride + (row - b * qpr)], 0), a.vocab - 1);
    const int np = a.n >> 6, nh = s16_nhalf(a.n), t = tok >> 4, r = tok & 15;
    for (int i = threadIdx.x; i < a.n; i += 256) {
        const int kk = i & 63, half = kk >> 5, c = (kk & 31) >> 3;
        const int8_t q = a.wt[((int64_t)t * np + (i >> 6)) * 1024 + (r + 16 * c) * 16 + 8 * half + (kk & 7)];
        const int bl = i >> 5;
        const uint16_t d = a.wd[(((int64_t)t * nh + (bl >> 4)) * 16 + r) * 16 + (bl & 15)];
        a.h[(int64_t)row * a.n + i] = h2f(d) * (float)q;
    }
}

// The canonical pairwise tree over nr (<= R) values, evaluated as they
// arrive in index order: after value j the pending subtrees are the set bits
// of j + 1 (L[k] holds one of 2^k values), merged earlier + later as in the
// level-by-level tree; at the end the pending subtrees fold from the
// smallest (latest) up: T = L[hi] + (... + L[lo]).  j is a compile-time
// constant in the unrolled loop, so every L index is static.
template <int R>
__device__ __forceinline__ float4 tree_stream4(const float4 (&p)[R], int nr) {
    float4 L[6];
#pragma unroll
    for (int k = 0; k < 6; ++k) L[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int j = 0; j < R; ++j) {
        if (j < nr) {
            float4 v = p[j];
            int k = 0;
#pragma unroll
            for (; k < 5; ++k) {
                if (!((j >> k) & 1)) break;
                v = add4(L[k], v);
            }
            L[k] = v;
        }
    }
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    bool have = false;
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        if ((nr >> k) & 1) {
            acc = have ? add4(L[k], acc) : L[k];
            have = true;
        }
    }
    return acc;
}

// Residual combine + RMSNorm (+ Q8_0).  One workgroup of NT threads per row;
// n <= 8192.  Residual: h += tree of the nr range partials (when part is
// set).  S > 0: thread t owns the float4 slots t + NT k (k < S; n % 4 == 0,
// n <= 4 NT S, nr <= R) and requests h and every partial of them at once,
// one round of memory latency; S == 0: thread t owns elements t + NT k,
// partials two elements at a time.  Sum of squares: halving tree over the
// next power of two >= n (zero padded), levels of stride >= NT inside each
// thread (thread t owns slots t + NT k), then across threads (LDS, then wave
// shuffles) -- the oracle's order, whatever the thread count.
#define LGX_NORM_MAX 8192
template <int NT, int S, int R>
__device__ __forceinline__ void norm_body(const lgx_norm_args& a) {
    constexpr int KV = LGX_NORM_MAX / NT;
    __shared__ __align__(16) float row[LGX_NORM_MAX];
    __shared__ float red[NT + 1];   // + the sum of squares
    const int b = blockIdx.x, t = threadIdx.x;
    float* hr = a.h + (int64_t)b * a.n;
    bool on[KV];
#pragma unroll
    for (int k = 0; k < KV; ++k) on[k] = t + NT * k < a.n;
    // the weights of this thread's elements, requested with the row (a load
    // after the barriers below would be one more memory round at the end)
    float wk[KV];
#pragma unroll
    for (int k = 0; k < KV; ++k)
        if (NT * k < a.n) wk[k] = a.w[min(t + NT * k, a.n - 1)];   // uniform test, clamped index
    float v[KV];
    if constexpr (S > 0) {
        // h and the partials through buffer descriptors: every load is
        // issued (the wait counts stay exact), and those of slots past the
        // row or ranges past nr fall outside the descriptor, so they read
        // zeros without a memory access (the launcher keeps the partials'
        // byte span below 2^31)
        const int n4 = a.n >> 2;
        constexpr uint32_t OOB = 0x80000000u;
        const __amdgpu_buffer_rsrc_t hrs =
            __builtin_amdgcn_make_buffer_rsrc((void*)hr, 0, a.n * 4, LGX_BUF_DWORD3);
        float4 x4[S];
#pragma unroll
        for (int k = 0; k < S; ++k)
            x4[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                   hrs, t + NT * k < n4 ? 16u * (t + NT * k) : OOB, 0, 0));
        if (a.part) {
            // every load issued, consumed in order
            float4 pv[S][R];
            const int64_t stride = (int64_t)a.m * a.n;
            const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
                (void*)(a.part + (int64_t)b * a.n), 0, (int)(((a.nr - 1) * stride + a.n) * 4),
                LGX_BUF_DWORD3);
#pragma unroll
            for (int j = 0; j < R; ++j)
#pragma unroll
                for (int k = 0; k < S; ++k) {
                    const uint32_t off = j < a.nr && t + NT * k < n4
                                             ? (uint32_t)((j * stride + 4 * (t + NT * k)) * 4)
                                             : OOB;
                    pv[k][j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(prs, off, 0, 0));
                }
#pragma unroll
            for (int k = 0; k < S; ++k) {
                x4[k] = add4(x4[k], tree_stream4<R>(pv[k], a.nr));
                if (t + NT * k < n4) *(float4*)(hr + 4 * (t + NT * k)) = x4[k];
            }
        }
#pragma unroll
        for (int k = 0; k < S; ++k)
            if (t + NT * k < n4) *(float4*)(row + 4 * (t + NT * k)) = x4[k];
        __syncthreads();
#pragma unroll
        for (int k = 0; k < KV; ++k) {
            const float x = on[k] ? row[t + NT * k] : 0.0f;
            v[k] = x * x;                          // zero past n
        }
    } else {
        float upd[KV];
#pragma unroll
        for (int k = 0; k < KV; ++k) upd[k] = 0.0f;
        if (a.part) {
            // two elements per round: 2 x nr loads in flight, bounded registers
#pragma unroll
            for (int k = 0; k < KV; k += 2) {
                if (on[k]) {
                    const bool o2[2] = {on[k], on[k + 1]};
                    float u2[2];
                    tree_partials_n<2, LGX_MAX_RANGES>(a.part, a.nr, (int64_t)a.m * a.n,
                                                       (int64_t)b * a.n + t + NT * k, NT, o2, u2);
                    upd[k] = u2[0];
                    upd[k + 1] = u2[1];
                }
            }
        }
#pragma unroll
        for (int k = 0; k < KV; ++k) {
            float x = on[k] ? hr[t + NT * k] : 0.0f;
            if (a.part && on[k]) {
                x = x + upd[k];
                hr[t + NT * k] = x;
            }
            if (on[k]) row[t + NT * k] = x;
            v[k] = x * x;                          // zero past n
        }
    }
    int n2 = NT;
    while (n2 < a.n) n2 <<= 1;
    // in-thread levels s = n2/2 ... NT: slot j += slot j + s
    for (int sl = n2 >> 1; sl >= NT; sl >>= 1) {
        const int ks = sl / NT;
#pragma unroll
        for (int k = 0; k < KV; ++k)
            if (k < ks) v[k] = v[k] + v[k + ks];
    }
    red[t] = v[0];
    __syncthreads();
    // levels NT/2 .. 64 across waves, evaluated by wave 0 alone from one
    // LDS round: lane l reads the NT/64 slots l + 64 j and folds them with
    // the same pairs in the same order (slot l + 64 j at level s joins
    // l + 64 j + s), then the lane levels by shuffles
    if (t < 64) {
        constexpr int NS = NT / 64;
        float q[NS];
#pragma unroll
        for (int j = 0; j < NS; ++j) q[j] = red[t + 64 * j];
#pragma unroll
        for (int s = NS / 2; s >= 1; s >>= 1) {
#pragma unroll
            for (int j = 0; j < s; ++j) q[j] = q[j] + q[j + s];
        }
        const float Ssq = wave_tree_sum(q[0]);
        if (t == 0) red[NT] = Ssq;
    }
    __syncthreads();
    const float ms = red[NT] / (float)a.n;
    const float r = 1.0f / sqrtf(ms + a.eps);
#pragma unroll
    for (int k = 0; k < KV; ++k) {
        if (on[k]) {
            const int i = t + NT * k;
            const float y = (row[i] * r) * wk[k];
            row[i] = y;
            if (a.xn) a.xn[(int64_t)b * a.n + i] = y;
            if (a.x16) a.x16[(int64_t)b * a.n + i] = f2h(y);
            if (a.xt) a.xt[((int64_t)(b >> 4) * a.n + i) * 16 + (b & 15)] = y;
        }
    }
    if (a.xq) {
        __syncthreads();
        quantize_row_from_lds<NT>(row, a.n, a.xq, a.xd, b, a.xq_t16 != 0);
    }
}

// Residual combine + RMSNorm (+ Q8_0) on float4 slots held in registers
// throughout: one workgroup of NT threads per row, thread t owns slots
// t + NT k (k < S; slot q = elements 4q .. 4q + 3; n % 4 == 0, n <= 4 NT S,
// nr <= R).  h, the partials and the weights are requested together; the
// sum of squares is the canonical halving tree over the elements (zero
// padded to a power of two), evaluated as element strides >= 4 NT across
// the thread's slots, 256 .. 2 NT across waves (every wave folds them from
// one LDS round, so the workgroup takes a single barrier), 128 .. 4 across
// lanes, 2 and 1 inside the float4 -- the same pairs in the same order (a
// stride at or past the padded width only adds zeros, exactly).  y = (x r) w
// per element and Q8_0 per 32-block from registers (8 consecutive lanes).
template <int NT, int S, int R>
__device__ __forceinline__ void norm4_body(const lgx_norm_args& a) {
    constexpr int NW = NT / 64;
    __shared__ float4 sq_s[NT];
    const int b = blockIdx.x, t = threadIdx.x, lane = t & 63;
    float* hr = a.h + (int64_t)b * a.n;
    const int n4 = a.n >> 2;
    float4 w4[S];
#pragma unroll
    for (int k = 0; k < S; ++k) w4[k] = ((const float4*)a.w)[min(t + NT * k, n4 - 1)];
    // h and the partials through buffer descriptors: every load is issued
    // (the wait counts stay exact), and those of slots past the row or ranges
    // past nr fall outside the descriptor, so they read zeros without a
    // memory access (the launcher keeps the partials' byte span below 2^31)
    constexpr uint32_t OOB = 0x80000000u;
    const __amdgpu_buffer_rsrc_t hrs = __builtin_amdgcn_make_buffer_rsrc((void*)hr, 0, a.n * 4, LGX_BUF_DWORD3);
    float4 x4[S];
#pragma unroll
    for (int k = 0; k < S; ++k)
        x4[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                               hrs, t + NT * k < n4 ? 16u * (t + NT * k) : OOB, 0, 0));
    if (a.part) {
        float4 pv[S][R];
        const int64_t stride = (int64_t)a.m * a.n;
        const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(a.part + (int64_t)b * a.n), 0, (int)(((a.nr - 1) * stride + a.n) * 4), LGX_BUF_DWORD3);
#pragma unroll
        for (int j = 0; j < R; ++j)
#pragma unroll
            for (int k = 0; k < S; ++k) {
                const uint32_t off = j < a.nr && t + NT * k < n4 ? (uint32_t)((j * stride + 4 * (t + NT * k)) * 4)
                                                                 : OOB;
                pv[k][j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(prs, off, 0, 0));
            }
#pragma unroll
        for (int k = 0; k < S; ++k) {
            x4[k] = add4(x4[k], tree_stream4<R>(pv[k], a.nr));
            if (t + NT * k < n4) *(float4*)(hr + 4 * (t + NT * k)) = x4[k];
        }
    }
    // squares (zero past n; slots past the row read zeros above)
    float4 v[S];
#pragma unroll
    for (int k = 0; k < S; ++k)
        v[k] = make_float4(x4[k].x * x4[k].x, x4[k].y * x4[k].y, x4[k].z * x4[k].z, x4[k].w * x4[k].w);
    static_assert(S == 1 || S == 2, "n <= 8 NT: one stride at most inside the thread");
    int n2 = 4;
    while (n2 < a.n) n2 <<= 1;
    if constexpr (S == 2) {
        if (n2 > 4 * NT) v[0] = add4(v[0], v[1]);          // stride 4 NT (n2 = 8 NT)
    }
    sq_s[t] = v[0];
    __syncthreads();
    float4 q[NW];
#pragma unroll
    for (int j = 0; j < NW; ++j) q[j] = sq_s[lane + 64 * j];
#pragma unroll
    for (int s = NW / 2; s >= 1; s >>= 1) {                  // strides 256 s across waves
#pragma unroll
        for (int j = 0; j < s; ++j) q[j] = add4(q[j], q[j + s]);
    }
    float e[4] = {q[0].x, q[0].y, q[0].z, q[0].w};
#pragma unroll
    for (int dl = 32; dl >= 1; dl >>= 1) {                  // strides 4 dl across lanes
#pragma unroll
        for (int c = 0; c < 4; ++c) e[c] = e[c] + __shfl_down(e[c], dl, 64);
    }
    e[0] = e[0] + e[2];
    e[1] = e[1] + e[3];
    e[0] = e[0] + e[1];
    const float ssq = __shfl(e[0], 0, 64);
    const float ms = ssq / (float)a.n;
    const float r = 1.0f / sqrtf(ms + a.eps);
#pragma unroll
    for (int k = 0; k < S; ++k) {
        const int sl = t + NT * k;
        const bool on = sl < n4;
        const float y[4] = {(x4[k].x * r) * w4[k].x, (x4[k].y * r) * w4[k].y, (x4[k].z * r) * w4[k].z,
                            (x4[k].w * r) * w4[k].w};
        if (on && a.xn) *(float4*)(a.xn + (int64_t)b * a.n + 4 * sl) = make_float4(y[0], y[1], y[2], y[3]);
        if (on && a.x16)
            *(uint2*)(a.x16 + (int64_t)b * a.n + 4 * sl) =
                make_uint2(f2h(y[0]) | ((uint32_t)f2h(y[1]) << 16), f2h(y[2]) | ((uint32_t)f2h(y[3]) << 16));
        if (on && a.xt) {
#pragma unroll
            for (int c = 0; c < 4; ++c) a.xt[((int64_t)(b >> 4) * a.n + 4 * sl + c) * 16 + (b & 15)] = y[c];
        }
        if (a.xq && 4 * NT * k < a.n) {      // uniform; whole 8-lane blocks (n % 32 == 0 with Q8_0)
            uint16_t dh;
            const uint32_t qw = quantize4(y, dh);
            if (on) {
                *(uint32_t*)(a.xq + xq_off(b, 4 * sl, a.n, a.xq_t16 != 0)) = qw;
                if ((lane & 7) == 0) a.xd[(int64_t)b * (a.n / 32) + (sl >> 3)] = dh;
            }
        }
    }
}

extern "C" __global__ __launch_bounds__(LGX_GLUE_NT) void lgx_k_add_rmsnorm_quant(const lgx_norm_args a) {
    norm_body<LGX_GLUE_NT, 0, 1>(a);
}
// n % 4 == 0, n <= 4096: 512 threads, two float4 slots each, nr <= 8 / 20;
// n <= 2048: one slot each
extern "C" __global__ __launch_bounds__(512) void lgx_k_add_rmsnorm_quant4s_r8(const lgx_norm_args a) {
    norm4_body<512, 1, 8>(a);
}
extern "C" __global__ __launch_bounds__(512) void lgx_k_add_rmsnorm_quant4_r8(const lgx_norm_args a) {
    norm4_body<512, 2, 8>(a);
}
extern "C" __global__ __launch_bounds__(512) void lgx_k_add_rmsnorm_quant4_r20(const lgx_norm_args a) {
    norm4_body<512, 2, 20>(a);
}

// The same residual combine + RMSNorm (+ Q8_0) with one wave per row, for
// n <= 1024 (n % 4 == 0) and nr <= 8: lane l owns the float4 slots l + 64k
// (elements 256k + 4l .. + 3), requests h and every partial of them at once,
// and the halving tree runs in registers (levels >= 256 across k, 128 .. 4
// across lanes, 2 and 1 inside the float4), so no LDS and no barrier.  The
// 8 lanes of a 32-element block hold it whole: Q8_0 straight from registers.
extern "C" __global__ __launch_bounds__(256) void lgx_k_add_rmsnorm_quant_w(const lgx_norm_args a) {
    constexpr int KS = 4, R = 8;
    const int lane = threadIdx.x & 63;
    const int b = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (b >= a.m) return;                    // whole waves only; no barrier below
    const int n4 = a.n >> 2;
    float4* hr = (float4*)(a.h + (int64_t)b * a.n);
    float4 x4[KS];
#pragma unroll
    for (int k = 0; k < KS; ++k) x4[k] = hr[min(lane + 64 * k, n4 - 1)];
    if (a.part) {
        float4 pv[KS][R];
        const int64_t stride = (int64_t)a.m * n4;
        const float4* pb = (const float4*)a.part + (int64_t)b * n4;
#pragma unroll
        for (int j = 0; j < R; ++j)
#pragma unroll
            for (int k = 0; k < KS; ++k)
                pv[k][j] = pb[min(j, a.nr - 1) * stride + min(lane + 64 * k, n4 - 1)];
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            float px[R], py[R], pz[R], pw[R];
#pragma unroll
            for (int j = 0; j < R; ++j) {
                px[j] = pv[k][j].x;
                py[j] = pv[k][j].y;
                pz[j] = pv[k][j].z;
                pw[j] = pv[k][j].w;
            }
            x4[k].x = x4[k].x + tree_sum_r<R>(px, a.nr);
            x4[k].y = x4[k].y + tree_sum_r<R>(py, a.nr);
            x4[k].z = x4[k].z + tree_sum_r<R>(pz, a.nr);
            x4[k].w = x4[k].w + tree_sum_r<R>(pw, a.nr);
            if (lane + 64 * k < n4) hr[lane + 64 * k] = x4[k];
        }
    }
    float v[KS][4];
#pragma unroll
    for (int k = 0; k < KS; ++k) {
        const bool on = lane + 64 * k < n4;  // zero past n
        v[k][0] = on ? x4[k].x * x4[k].x : 0.0f;
        v[k][1] = on ? x4[k].y * x4[k].y : 0.0f;
        v[k][2] = on ? x4[k].z * x4[k].z : 0.0f;
        v[k][3] = on ? x4[k].w * x4[k].w : 0.0f;
    }
    int n2 = 4;
    while (n2 < a.n) n2 <<= 1;
    // slot i += slot i + sl for i < sl, sl = n2/2 .. 1; element i = 256k + 4 lane + e
    for (int sl = n2 >> 1; sl >= 256; sl >>= 1) {
        const int ks = sl >> 8;
#pragma unroll
        for (int k = 0; k < KS; ++k)
            if (k < ks) {
#pragma unroll
                for (int e = 0; e < 4; ++e) v[k][e] = v[k][e] + v[k + ks][e];
            }
    }
    for (int sl = min(n2 >> 1, 128); sl >= 4; sl >>= 1) {
        const int dl = sl >> 2;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[0][e] = v[0][e] + __shfl_down(v[0][e], dl, 64);
    }
    if (n2 >= 4) {
        v[0][0] = v[0][0] + v[0][2];
        v[0][1] = v[0][1] + v[0][3];
        v[0][0] = v[0][0] + v[0][1];
    }
    const float ssq = __shfl(v[0][0], 0, 64);
    const float ms = ssq / (float)a.n;
    const float r = 1.0f / sqrtf(ms + a.eps);
#pragma unroll
    for (int k = 0; k < KS; ++k) {
        const int s = lane + 64 * k;
        const bool on = s < n4;
        const float4 w4 = ((const float4*)a.w)[min(s, n4 - 1)];
        float y[4] = {(x4[k].x * r) * w4.x, (x4[k].y * r) * w4.y, (x4[k].z * r) * w4.z,
                      (x4[k].w * r) * w4.w};
        if (on && a.xn) *(float4*)(a.xn + (int64_t)b * a.n + 4 * s) = make_float4(y[0], y[1], y[2], y[3]);
        if (on && a.x16)
            *(uint2*)(a.x16 + (int64_t)b * a.n + 4 * s) =
                make_uint2(f2h(y[0]) | ((uint32_t)f2h(y[1]) << 16), f2h(y[2]) | ((uint32_t)f2h(y[3]) << 16));
        if (on && a.xt) {
#pragma unroll
            for (int e = 0; e < 4; ++e) a.xt[((int64_t)(b >> 4) * a.n + 4 * s + e) * 16 + (b & 15)] = y[e];
        }
        if (a.xq && 256 * k < a.n) {         // whole 8-lane blocks (n % 32 == 0 with Q8_0)
            uint16_t dh;
            const uint32_t qw = quantize4(y, dh);
            if (on) {
                *(uint32_t*)(a.xq + xq_off(b, 4 * s, a.n, a.xq_t16 != 0)) = qw;
                if ((lane & 7) == 0) a.xd[(int64_t)b * (a.n / 32) + (s >> 3)] = dh;
            }
        }
    }
}

// QKV combine + bias + RoPE + paged KV append.  One workgroup of 1024
// threads per sequence.
// Tree + bias + RoPE + binary16 K/V append.  grid = (rows of the product,
// ceil(pairs / 256)), 256 threads: thread t of workgroup y owns rotation
// pair p = 256 y + t, i.e. elements (i, i + d/2) of head p / (d/2) of the
// row (q and k heads rotated, v heads copied), whatever d.  The position's
// values (length, then page and cos/sin) are requested first, with the
// pair's partials, so the two dependent rounds they need overlap the
// partials' round.
extern "C" __global__ __launch_bounds__(256) void lgx_k_qkv_rope_append(const lgx_qkv_args a) {
    // workgroup row b of the product (sequence bs, its query j)
    const int b = blockIdx.x, t = threadIdx.x;
    const int qpr = max(a.qpr, 1), bs = b / qpr;
    const int d = a.d, half = d / 2;
    const int nh = a.hq + 2 * a.hkv, nq = nh * d, np = nh * half;
    const int p = blockIdx.y * 256 + t;
    const int pc = min(p, np - 1), hh = pc / half, i = pc - hh * half;
    const int pos = min(max(a.seq_len[bs] + (b - bs * qpr), 0), a.max_seq - 1);
    const int page = min(max(a.page_table[(int64_t)bs * a.maxp + pos / LGX_PAGE], 0), a.num_pages - 1);
    const float c = a.cos_t[(int64_t)pos * half + i], sn = a.sin_t[(int64_t)pos * half + i];
    const int64_t e0 = (int64_t)b * nq + hh * d + i, stride = (int64_t)a.m * nq;
    float x0 = tree_read(a.nr, [&](int j) { return a.part[j * stride + e0]; });
    float x1 = tree_read(a.nr, [&](int j) { return a.part[j * stride + e0 + half]; });
    if (a.bias) {
        x0 = x0 + a.bias[hh * d + i];
        x1 = x1 + a.bias[hh * d + i + half];
    }
    if (p >= np) return;
    const int slot = pos % LGX_PAGE;
    if (hh < a.hq + a.hkv) {
        // rotate-half pair of a q or k head, each product rounded on its own
        const float t0 = x0 * c, t1 = x1 * sn, t2 = x1 * c, t3 = x0 * sn;
        const float y0 = t0 - t1, y1 = t2 + t3;
        if (hh < a.hq) {
            float* qo = a.q_out + ((int64_t)b * a.hq + hh) * d;
            qo[i] = y0;
            qo[i + half] = y1;
        } else {
            const int g = hh - a.hq;
            uint16_t* kd = a.kpages + (((int64_t)page * a.hkv + g) * LGX_PAGE + slot) * d;
            kd[i] = f2h(y0);
            kd[i + half] = f2h(y1);
        }
    } else {
        const int g = hh - a.hq - a.hkv;
        uint16_t* vd = a.vpages + (((int64_t)page * a.hkv + g) * LGX_PAGE + slot) * d;
        vd[i] = f2h(x0);
        vd[i + half] = f2h(x1);
    }
}

// Attention chunk merge for one (sequence, head) + Q8_0 of its D values (D/32
// whole blocks of the attention row, so heads quantise independently).
template <int D>
__device__ __forceinline__ void attn_combine_quant_body(const lgx_attn_args& a) {
    __shared__ float row[D];
    const int bh = blockIdx.x, t = threadIdx.x;
    const float o = attn_merge<D>(a, bh);
    row[t] = o;
    if (a.out) a.out[(int64_t)bh * D + t] = o;
    __syncthreads();
    if (t < D / 4) {                              // 8 lanes per 32-block, all active
        const float f[4] = {row[4 * t], row[4 * t + 1], row[4 * t + 2], row[4 * t + 3]};
        uint16_t dh;
        const uint32_t qw = quantize4(f, dh);
        const int row = bh / a.hq, col = (bh - row * a.hq) * D + 4 * t;
        *(uint32_t*)(a.xq + xq_off(row, col, a.hq * D, a.xq_t16 != 0)) = qw;
        if ((t & 7) == 0) a.xd[(int64_t)bh * (D / 32) + (t >> 3)] = dh;
    }
}
extern "C" __global__ __launch_bounds__(64) void lgx_k_attn_combine_quant_d64(const lgx_attn_args a) {
    attn_combine_quant_body<64>(a);
}
extern "C" __global__ __launch_bounds__(128) void lgx_k_attn_combine_quant_d128(const lgx_attn_args a) {
    attn_combine_quant_body<128>(a);
}

// ---------------------------------------------------------------------------
// Decode attention merge fused with o_proj, for an o_proj of K = hq * d <=
// 1024 (one range: the small models' step).  grid = B * ngroups, 16 waves:
// workgroup = (sequence b, group g of `tiles` 16-row tiles of o, <= 16).
// Wave w requests the partials of head w of sequence b, then (w < the tile
// count) its tile's weights and scales (through the cache: every sequence's
// workgroups read them), and merges heads w, w + 16, ... (one memory round
// up to 16 heads) from the chunk partials with the arithmetic of
// attn_merge_one_round (M = max of the chunk maxima, w_c = lgx_expf(m_c - M),
// L and O chains over the chunks in order, O / L; the chunk weights pass
// between lanes by readlane instead of LDS), the workgroup quantises the row
// to Q8_0 (quantize4, as lgx_k_attn_combine_quant) into LDS in the grouped
// GEMV's (pair, chunk) slot order, and each wave runs grp_chain on its tile:
// y[b][16 t + r] is then what lgx_k_attn_combine_quant followed by the o_proj
// product gives.  The ngroups workgroups of a sequence each merge all of its
// heads: a few KiB of partials per head from L2, where a kernel of its own
// costs a launch and a memory round.  Up to 16 chunks (the launcher checks).
// ---------------------------------------------------------------------------
// One wave's merge of (sequence b, head h), in two halves so that its loads
// can be issued ahead of others: merge_load requests chunk `lane`'s m and l
// and the o_c of the lane's dimensions for the first 16 chunks (loads past
// the sequence's chunk count read zeros through the descriptor);
// merge_finish runs the arithmetic of attn_merge_one_round on them.
template <int D>
struct MergeLd {
    float mc, lc, ov[D / 64][16];
};
template <int D>
__device__ __forceinline__ void merge_load(const lgx_attn_args& a, int b, int h, int lane, MergeLd<D>& m) {
    const float* pp = a.part + ((int64_t)b * a.hq + h) * a.nchunk * (D + 2);
    const MergeRd<D> rd(pp, a.nchunk);
    m.mc = rd(lane, D);
    m.lc = rd(lane, D + 1);
#pragma unroll
    for (int e = 0; e < D / 64; ++e)
#pragma unroll
        for (int c = 0; c < 16; ++c) m.ov[e][c] = rd(c, lane + 64 * e);
}
template <int D>
__device__ __forceinline__ void merge_finish(const lgx_attn_args& a, int b, int lane, const MergeLd<D>& m,
                                             float (&out)[D / 64]) {
    constexpr int E = D / 64;                     // dimensions per lane: lane + 64 e
    const int L = min(a.seq_len[b] + a.len_add, a.maxlen);
    const int nc = (max(L, 0) + LGX_ATTN_CHUNK - 1) / LGX_ATTN_CHUNK;
    const float M = wave_max(lane < nc ? m.mc : -__builtin_inff());
    const float wl = lgx_expf(m.mc - M);          // used by lanes < nc only
    float Ls = 0.0f, O[E];
#pragma unroll
    for (int e = 0; e < E; ++e) O[e] = 0.0f;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
        if (c < nc) {                             // uniform
            const float wc = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), c));
            const float lcc = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, m.lc), c));
            Ls = fmaf(wc, lcc, Ls);
#pragma unroll
            for (int e = 0; e < E; ++e) O[e] = fmaf(wc, m.ov[e][c], O[e]);
        }
    }
#pragma unroll
    for (int e = 0; e < E; ++e) out[e] = nc > 0 ? O[e] / Ls : 0.0f;
}

template <int D, int NW>
__device__ __forceinline__ void attn_merge_o_body(const lgx_merge_o_args& a) {
    const int NT = min(a.tiles, NW);              // tiles per workgroup, one per wave
    __shared__ float row_s[1024];
    __shared__ __align__(16) int8_t xs[GRP_XSLOT];
    float* dx = (float*)(xs + 1024);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = blockIdx.x / a.ngroups, g = blockIdx.x - b * a.ngroups;
    const int k = a.k, np = k >> 6, nh = s16_nhalf(k);
    const int ntiles = a.n >> 4;
    const int t = NT * g + wave;
    const bool on = wave < NT && t < ntiles;      // wave-uniform
    const RangeInfo ri = range_info(0, k);
    const lgx_attn_args& at = a.at;
    // this wave's first head: its partials requested first, so the merge
    // waits for them alone (loads complete in issue order)
    MergeLd<D> ml;
    const bool h0 = wave < at.hq;
    if (h0) merge_load<D>(at, b, wave, lane, ml);
    GrpRegs R;
    if (on) {
        const int r = lane & 15;
        uint32_t d0[8], d1[8];
        load_scales_half(a.wd, t, 0, nh, r, d0);
        load_scales_half(a.wd, t, min(1, nh - 1), nh, r, d1);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            R.dw[i] = d0[i];
            R.dw[8 + i] = d1[i];
        }
        // the tile's units through a buffer descriptor of np KiB (units past
        // it read zeros without a memory access), cache policy 0
        const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)((const uint4*)a.wt + (int64_t)t * np * 64), 0, np * 1024, LGX_BUF_DWORD3);
#pragma unroll
        for (int i = 0; i < GRP_WIN; ++i)
            R.w[i] = ld_buf_cached(wr, (i * 64 + lane) * 16);
    }
    __builtin_amdgcn_sched_barrier(0);            // issue order: partials, then weights
    if (h0) {
        float o[D / 64];
        merge_finish<D>(at, b, lane, ml, o);
#pragma unroll
        for (int e = 0; e < D / 64; ++e) row_s[wave * D + lane + 64 * e] = o[e];
    }
    // heads past NW (more heads than waves): w + NW, w + 2 NW, ...
    for (int h = wave + NW; h < at.hq; h += NW) {
        MergeLd<D> m2;
        merge_load<D>(at, b, h, lane, m2);
        float o[D / 64];
        merge_finish<D>(at, b, lane, m2, o);
#pragma unroll
        for (int e = 0; e < D / 64; ++e) row_s[h * D + lane + 64 * e] = o[e];
    }
    __syncthreads();
    // Q8_0 of the row: thread q holds values 4q .. 4q + 3 (8 threads per
    // block, whole 8-lane groups active since k % 32 == 0)
    if (tid < k / 4) {
        const float f[4] = {row_s[4 * tid], row_s[4 * tid + 1], row_s[4 * tid + 2], row_s[4 * tid + 3]};
        uint16_t dh;
        const uint32_t qw = quantize4(f, dh);
        const int bl = tid >> 3, c = (tid & 7) >> 1;
        *(uint32_t*)(xs + ((bl >> 1) * 4 + c) * 16 + (bl & 1) * 8 + 4 * (tid & 1)) = qw;
        if ((tid & 7) == 0) dx[bl] = h2f(dh);
    }
    __syncthreads();
    if (on) {
        const float acc = grp_chain(ri, lane, R, xs, dx);
        if (lane < 16) a.y[(int64_t)b * a.n + t * 16 + lane] = acc;
    }
}
// ---------------------------------------------------------------------------
// Decode residual + RMSNorm + Q8_0 fused with the qkv product and its RoPE /
// KV-append consumer, for hidden H <= 1024 (one range): grid = B * ngroups,
// 8 waves: workgroup = (sequence b, group g of 8 row tiles of qkv, i.e. 128
// columns: whole heads of d = 64 or 128; two workgroups per CU at 128 VGPRs,
// so config 3's 288 run in one round).  Thread t requests h[b][j] and the
// range partials of the previous product for j = t and t + 512, then wave w
// its tile's weights
// (through the cache) and the consumer's bias, RoPE and page entries are
// requested; x_j = h_j + tree(partials) (group 0 writes it to h_out, a
// buffer other than h: the other groups of the sequence still read h), the
// sum of squares by orc_halving_sum's pairs over 1024 slots (zeros past H,
// which add nothing: x^2 >= 0), evaluated by wave 0 from LDS as the norm
// kernels do, y = (x * r) * w with r = 1 / sqrt(S / H + eps), Q8_0 of y
// (quantize4) into the grouped GEMV's slots, the tile's grp_chain, and the
// lgx_k_qkv_rope_append operations on the 128 columns: bias, rotate-half
// RoPE at position seq_len[b], q to q_out, k and v to the cache.  Each group
// repeats the sequence's norm (H values and their partials, from L2) where
// a kernel of its own costs a launch and a memory round.
// ---------------------------------------------------------------------------
#define NQ_TILES LGX_NQ_TILES
template <int D>
__device__ __forceinline__ void norm_qkv_body(const lgx_norm_qkv_args& a) {
    constexpr int NT = 64 * NQ_TILES;             // one wave per tile
    constexpr int EP = 1024 / NT;                 // row elements per thread
    constexpr int MAXR = LGX_NQ_MAXR;             // partial ranges (the launcher checks)
    __shared__ float row_s[1024];
    __shared__ float sq_s[1024];
    __shared__ float out_s[NQ_TILES * 16];
    __shared__ float rr_s;
    __shared__ __align__(16) int8_t xs[GRP_XSLOT];
    float* dx = (float*)(xs + 1024);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = blockIdx.x / a.ngroups, g = blockIdx.x - b * a.ngroups;
    const int H = a.H, np = H >> 6, nh = s16_nhalf(H);
    const int ntiles = a.n >> 4;
    const int t = NQ_TILES * g + wave;
    const bool on = t < ntiles;                   // wave-uniform
    const lgx_qkv_args& q = a.q;
    // 1. the row and its partials (elements j = tid + NT e), the weights of
    // the thread's four Q8_0 values (4 tid ..), all issued first
    float hv[EP], pv[EP][MAXR];
    const int64_t stride = (int64_t)q.m * H;
#pragma unroll
    for (int e = 0; e < EP; ++e) {
        const int jc = min(tid + NT * e, H - 1);
        hv[e] = a.h[(int64_t)b * H + jc];
        // ranges past nr re-read range nr - 1 (never added: the tree stops at nr)
#pragma unroll
        for (int r = 0; r < MAXR; ++r)
            pv[e][r] = a.part ? a.part[(int64_t)min(r, max(a.nr, 1) - 1) * stride + (int64_t)b * H + jc] : 0.0f;
    }
    const int q4 = min(tid, H / 4 - 1);
    const float4 w4 = *(const float4*)(a.w + 4 * q4);
    // 2. the tile's weights and scales
    const RangeInfo ri = range_info(0, H);
    GrpRegs R;
    if (on) {
        const int r = lane & 15;
        uint32_t d0[8], d1[8];
        load_scales_half(a.wd, t, 0, nh, r, d0);
        load_scales_half(a.wd, t, min(1, nh - 1), nh, r, d1);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            R.dw[i] = d0[i];
            R.dw[8 + i] = d1[i];
        }
        const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
            (void*)((const uint4*)a.wt + (int64_t)t * np * 64), 0, np * 1024, LGX_BUF_DWORD3);
#pragma unroll
        for (int i = 0; i < GRP_WIN; ++i) R.w[i] = ld_buf_cached(wr, (i * 64 + lane) * 16);
    }
    // 3. the consumer's inputs for column cc = tid (< 128) of the group:
    // q / k head columns i < d/2 take the pair (i, i + d/2), v columns one
    // value; the others idle
    const int d = D, half = D / 2;
    const int col = NQ_TILES * 16 * g + min(tid, NQ_TILES * 16 - 1);
    const int head = col / d, ci = col - head * d;
    const bool rot = head < q.hq + q.hkv;
    const bool cact = tid < NQ_TILES * 16 && col < a.n && (rot ? ci < half : true);
    const int pos = min(max(q.seq_len[b], 0), q.max_seq - 1);
    const int page = min(max(q.page_table[(int64_t)b * q.maxp + pos / LGX_PAGE], 0), q.num_pages - 1);
    const float b0 = q.bias ? q.bias[min(col, a.n - 1)] : 0.0f;
    const float b1 = q.bias && rot ? q.bias[min(col + half, a.n - 1)] : 0.0f;
    const float cs = rot ? q.cos_t[(int64_t)pos * half + min(ci, half - 1)] : 0.0f;
    const float sn = rot ? q.sin_t[(int64_t)pos * half + min(ci, half - 1)] : 0.0f;
    __builtin_amdgcn_sched_barrier(0);            // issue order: row, weights, consumer
    // 4. residual and squares
#pragma unroll
    for (int e = 0; e < EP; ++e) {
        const int j = tid + NT * e;
        float x = hv[e];
        if (a.part && a.nr > 0) x = hv[e] + tree_sum_r<MAXR>(pv[e], a.nr);
        if (j < H) {
            row_s[j] = x;
            if (g == 0) a.h_out[(int64_t)b * H + j] = x;
        }
        sq_s[j] = j < H ? x * x : 0.0f;
    }
    __syncthreads();
    if (tid < 64) {
        // orc_halving_sum over the 1024 slots: lane l folds l + 64 j, j < 16
        // (levels 512 .. 64), then the lane levels
        float qv[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) qv[j] = sq_s[tid + 64 * j];
#pragma unroll
        for (int s = 8; s >= 1; s >>= 1) {
#pragma unroll
            for (int j = 0; j < s; ++j) qv[j] = qv[j] + qv[j + s];
        }
        const float Ssq = wave_tree_sum(qv[0]);
        if (tid == 0) rr_s = 1.0f / sqrtf(Ssq / (float)H + a.eps);
    }
    __syncthreads();
    // 5. y = (x * r) * w and its Q8_0 (8 threads per block)
    if (tid < H / 4) {
        const float r = rr_s;
        const float f[4] = {(row_s[4 * tid] * r) * w4.x, (row_s[4 * tid + 1] * r) * w4.y,
                            (row_s[4 * tid + 2] * r) * w4.z, (row_s[4 * tid + 3] * r) * w4.w};
        uint16_t dh;
        const uint32_t qw = quantize4(f, dh);
        const int bl = tid >> 3, c = (tid & 7) >> 1;
        *(uint32_t*)(xs + ((bl >> 1) * 4 + c) * 16 + (bl & 1) * 8 + 4 * (tid & 1)) = qw;
        if ((tid & 7) == 0) dx[bl] = h2f(dh);
    }
    __syncthreads();
    // 6. the tiles' chains
    if (on) {
        const float acc = grp_chain(ri, lane, R, xs, dx);
        if (lane < 16) out_s[wave * 16 + lane] = acc;
    }
    __syncthreads();
    // 7. bias, RoPE, q out, KV append
    if (cact) {
        const int cc = tid;
        const int slot = pos % LGX_PAGE;
        if (rot) {
            const float x0 = q.bias ? out_s[cc] + b0 : out_s[cc];
            const float x1 = q.bias ? out_s[cc + half] + b1 : out_s[cc + half];
            const float t0 = x0 * cs, t1 = x1 * sn, t2 = x1 * cs, t3 = x0 * sn;
            const float y0 = t0 - t1, y1 = t2 + t3;
            if (head < q.hq) {
                float* qo = q.q_out + ((int64_t)b * q.hq + head) * d;
                qo[ci] = y0;
                qo[ci + half] = y1;
            } else {
                uint16_t* kd = q.kpages + (((int64_t)page * q.hkv + (head - q.hq)) * LGX_PAGE + slot) * d;
                kd[ci] = f2h(y0);
                kd[ci + half] = f2h(y1);
            }
        } else {
            const int gv = head - q.hq - q.hkv;
            uint16_t* vd = q.vpages + (((int64_t)page * q.hkv + gv) * LGX_PAGE + slot) * d;
            vd[ci] = f2h(q.bias ? out_s[cc] + b0 : out_s[cc]);
        }
    }
}
extern "C" __global__ __launch_bounds__(64 * LGX_NQ_TILES) void lgx_k_norm_qkv_d64(const lgx_norm_qkv_args a) {
    norm_qkv_body<64>(a);
}
extern "C" __global__ __launch_bounds__(64 * LGX_NQ_TILES) void lgx_k_norm_qkv_d128(const lgx_norm_qkv_args a) {
    norm_qkv_body<128>(a);
}

extern "C" __global__ __launch_bounds__(1024) void lgx_k_attn_merge_o_d64(const lgx_merge_o_args a) {
    attn_merge_o_body<64, 16>(a);
}
extern "C" __global__ __launch_bounds__(1024) void lgx_k_attn_merge_o_d128(const lgx_merge_o_args a) {
    attn_merge_o_body<128, 16>(a);
}

// SwiGLU from gate|up partials + Q8_0.  grid = (rows, ceil(blocks / 32)),
// 256 threads = 32 blocks of 32 values; all partial loads of a thread are
// issued together.
extern "C" __global__ __launch_bounds__(256) void lgx_k_swiglu_quant(const lgx_swiglu_args a) {
    const int b = blockIdx.x;
    const int bl = blockIdx.y * 32 + (threadIdx.x >> 3), j = threadIdx.x & 7;
    const int nbl = a.inter / 32;
    const bool on = bl < nbl;
    const int64_t stride = (int64_t)a.m * 2 * a.inter;
    const int64_t base = (int64_t)b * 2 * a.inter + bl * 32 + 4 * j;
    float gu[8];   // gate 0..3 at base + e, up 4..7 at base + inter + e
    float p[8][8]; // gate|up partials: K = hidden <= 8192, so at most 8 ranges
#pragma unroll
    for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e)
            p[e][r] = (r < a.nr && on) ? a.part[r * stride + base + (e & 3) + (e >> 2) * a.inter] : 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) gu[e] = tree_sum_r<8>(p[e], a.nr);
    float f[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) f[e] = on ? lgx_silu(gu[e]) * gu[4 + e] : 0.0f;
    if (on && a.y) {
        float* yo = a.y + (int64_t)b * a.inter + bl * 32 + 4 * j;
#pragma unroll
        for (int e = 0; e < 4; ++e) yo[e] = f[e];
    }
    uint16_t dh;
    const uint32_t qw = quantize4(f, dh);
    if (on && a.xq) {
        *(uint32_t*)(a.xq + xq_off(b, bl * 32 + 4 * j, a.inter, a.xq_t16 != 0)) = qw;
        if (j == 0) a.xd[(int64_t)b * nbl + bl] = dh;
    }
}

// The fast prefill's SwiGLU on a binary16 gate|up GEMM output: thread per 8
// consecutive outputs of a row (16-byte loads of gate and up, one store).
extern "C" __global__ __launch_bounds__(256) void lgx_k_swiglu_f16(const lgx_swiglu16_args a) {
    const int i8 = a.inter >> 3;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= (int64_t)a.m * i8) return;
    const int64_t r = t / i8;
    const int i = (int)(t - r * i8) * 8;
    const uint16_t* g = a.gu + r * 2 * a.inter + i;
    const uint4 gv = *(const uint4*)g, uv = *(const uint4*)(g + a.inter);
    const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float f0 = lgx_silu(h2f(gw[e] & 0xffffu)) * h2f(uw[e] & 0xffffu);
        const float f1 = lgx_silu(h2f(gw[e] >> 16)) * h2f(uw[e] >> 16);
        o[e] = f2h(f0) | ((uint32_t)f2h(f1) << 16);
    }
    *(uint4*)(a.y + r * a.inter + i) = make_uint4(o[0], o[1], o[2], o[3]);
}

// Consumers of the fused 16-row products (lgx_gemm_fused_args), run by the
// product's workgroup on its outputs in LDS (row mm of the m-group at
// out_s[mm * ld]).  The same operations in the same order as
// lgx_k_qkv_rope_append and lgx_k_swiglu_quant on a one-range product.
// The qkv consumer's loads do not depend on the product, so they are made
// before it (QkvPrep): stage 1, first in the kernel, the length of each
// element's sequence and its bias; stage 2, after the first weight loads are
// issued, the position's cos / sin and page entry.  vmcnt counts in issue
// order, so waiting for stage 1 does not wait for the weight loads behind it.
__device__ __forceinline__ void fused_qkv_prep1(const lgx_qkv_args& q, int head, int m0, int mrows,
                                                QkvPrep& p) {
    const int d = q.d, half = d / 2, qpr = max(q.qpr, 1);
    const int per = head < q.hq + q.hkv ? half : d;
    const float* bias = q.bias ? q.bias + head * d : nullptr;
    // every load unconditional at a valid address (rows past the m-group's
    // read its last row; their values are never used): a load under a
    // per-lane branch makes the compiler wait for all loads at the join
#pragma unroll
    for (int j = 0; j < QKV_PE; ++j) {
        const int e = threadIdx.x + 256 * j, mm = e / per, i = e - mm * per;
        p.pos[j] = q.seq_len[(m0 + min(mm, mrows - 1)) / qpr];
        p.b0[j] = bias ? bias[i] : 0.0f;
        p.b1[j] = bias && per == half ? bias[i + half] : 0.0f;
    }
}
__device__ __forceinline__ void fused_qkv_prep2(const lgx_qkv_args& q, int head, int m0, int mrows,
                                                QkvPrep& p) {
    const int d = q.d, half = d / 2, qpr = max(q.qpr, 1);
    const bool rot = head < q.hq + q.hkv;
    const int per = rot ? half : d;
#pragma unroll
    for (int j = 0; j < QKV_PE; ++j) {
        const int e = threadIdx.x + 256 * j, mm = e / per, i = e - mm * per;
        const int b = m0 + min(mm, mrows - 1), bs = b / qpr;
        const int pos = min(max(p.pos[j] + (b - bs * qpr), 0), q.max_seq - 1);
        p.pos[j] = pos;
        p.page[j] = q.page_table[(int64_t)bs * q.maxp + pos / LGX_PAGE];
        p.c[j] = rot ? q.cos_t[(int64_t)pos * half + i] : 0.0f;
        p.sn[j] = rot ? q.sin_t[(int64_t)pos * half + i] : 0.0f;
    }
}
// Element e = threadIdx.x + 256 j of the head's rows: pair (i, i + d/2) of
// a q / k head, value i of a v head.
__device__ __forceinline__ void fused_qkv_post(const lgx_qkv_args& q, const float* out_s, int ld,
                                               int head, int m0, int mrows, const QkvPrep& p) {
    const int d = q.d, half = d / 2;
    const bool rot = head < q.hq + q.hkv;   // q and k heads rotate, v heads are copied
    const int per = rot ? half : d;
    const bool bias = q.bias != nullptr;
#pragma unroll
    for (int j = 0; j < QKV_PE; ++j) {
        const int e = threadIdx.x + 256 * j, mm = e / per, i = e - mm * per;
        if (mm >= mrows) continue;
        const int b = m0 + mm;
        const int page = min(max(p.page[j], 0), q.num_pages - 1);
        const int slot = p.pos[j] % LGX_PAGE;
        const float* row = out_s + mm * ld;
        if (rot) {
            const float x0 = bias ? row[i] + p.b0[j] : row[i];
            const float x1 = bias ? row[i + half] + p.b1[j] : row[i + half];
            const float c = p.c[j], sn = p.sn[j];
            const float t0 = x0 * c, t1 = x1 * sn, t2 = x1 * c, t3 = x0 * sn;
            const float y0 = t0 - t1, y1 = t2 + t3;
            if (head < q.hq) {
                float* qo = q.q_out + ((int64_t)b * q.hq + head) * d;
                qo[i] = y0;
                qo[i + half] = y1;
            } else {
                uint16_t* kd = q.kpages + (((int64_t)page * q.hkv + (head - q.hq)) * LGX_PAGE + slot) * d;
                kd[i] = f2h(y0);
                kd[i + half] = f2h(y1);
            }
        } else {
            const int g = head - q.hq - q.hkv;
            uint16_t* vd = q.vpages + (((int64_t)page * q.hkv + g) * LGX_PAGE + slot) * d;
            vd[i] = f2h(bias ? row[i] + p.b0[j] : row[i]);
        }
    }
}

// Gate columns at out_s[mm * ld + cc], up at out_s[mm * ld + cols + cc],
// cc < cols; output columns c0 + cc.  8 lanes per 32-block, the 8 lanes of a
// block always active together.
__device__ __forceinline__ void fused_swiglu_post(const lgx_swiglu_args& s, const float* out_s, int ld, int cols,
                                  int c0, int m0, int mrows) {
    const int nbl = cols / 32, j = threadIdx.x & 7;
    for (int e = threadIdx.x >> 3; e < 16 * nbl; e += blockDim.x >> 3) {
        const int mm = e / nbl, bl = e - mm * nbl;
        const bool on = mm < mrows;
        const float* row = out_s + mm * ld + bl * 32 + 4 * j;
        float f[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) f[k] = on ? lgx_silu(row[k]) * row[cols + k] : 0.0f;
        const int64_t m = m0 + mm;
        const int col = c0 + bl * 32 + 4 * j;
        if (on && s.y) {
#pragma unroll
            for (int k = 0; k < 4; ++k) s.y[m * s.inter + col + k] = f[k];
        }
        uint16_t dh;
        const uint32_t qw = quantize4(f, dh);
        if (on && s.xq) {
            *(uint32_t*)(s.xq + xq_off(m, col, s.inter, s.xq_t16 != 0)) = qw;
            if (j == 0) s.xd[m * (s.inter / 32) + col / 32] = dh;
        }
    }
}

// Tied binary16 lm_head (h <= 1024: a single canonical range, so the logit
// is the sequential fmaf chain over the columns).  A workgroup owns 256
// vocabulary rows (one per thread); per 64-column slab, the binary16 rows and
// the activation rows (m <= 64) are staged in LDS with coalesced loads, and
// every thread runs the chain of its vocabulary row for all m rows
// (activation reads are LDS broadcasts).
#define LGX_LM_MAXM 64
extern "C" __global__ __launch_bounds__(256) void lgx_k_lm_head_f16(const lgx_lmhead_args a) {
    __shared__ uint32_t slab[256][33];             // 64 binary16 per row, padded
    __shared__ float4 xs[LGX_LM_MAXM][16];         // 64 columns of each activation row
    const int t = threadIdx.x;
    const int v0 = blockIdx.x * 256;
    const int v = v0 + t;
    // range blockIdx.y: columns [1024 y, min(h, 1024 y + 1024)), its chain
    // to range partial y ([ranges][m][vocab]; one range for h <= 1024)
    const int kb = blockIdx.y * 1024, ke = min(a.h, kb + 1024);
    float* lg = a.logits + (int64_t)blockIdx.y * a.m * a.vocab;
    float acc[LGX_LM_MAXM];
#pragma unroll
    for (int r = 0; r < LGX_LM_MAXM; ++r) acc[r] = 0.0f;
    for (int k0 = kb; k0 < ke; k0 += 64) {
        __syncthreads();
        for (int s2 = t; s2 < 256 * 32; s2 += 256) {
            const int rr = s2 >> 5, cc = s2 & 31;
            const int vv = min(v0 + rr, a.vocab - 1);
            slab[rr][cc] = *(const uint32_t*)(a.emb + (int64_t)vv * a.h + k0 + 2 * cc);
        }
        for (int s2 = t; s2 < a.m * 16; s2 += 256) {
            const int rr = s2 >> 4, q = s2 & 15;
            xs[rr][q] = *(const float4*)(a.x + (int64_t)rr * a.h + k0 + 4 * q);
        }
        __syncthreads();
#pragma unroll 2
        for (int q = 0; q < 16; ++q) {
            const uint32_t w01 = slab[t][2 * q], w23 = slab[t][2 * q + 1];
            const float e0 = h2f(w01 & 0xffffu), e1 = h2f(w01 >> 16);
            const float e2 = h2f(w23 & 0xffffu), e3 = h2f(w23 >> 16);
#pragma unroll
            for (int r = 0; r < LGX_LM_MAXM; ++r) {
                if (r < a.m) {
                    const float4 xv = xs[r][q];
                    acc[r] = fmaf(xv.x, e0, acc[r]);
                    acc[r] = fmaf(xv.y, e1, acc[r]);
                    acc[r] = fmaf(xv.z, e2, acc[r]);
                    acc[r] = fmaf(xv.w, e3, acc[r]);
                }
            }
        }
    }
    if (v >= a.vocab) return;
#pragma unroll
    for (int r = 0; r < LGX_LM_MAXM; ++r)
        if (r < a.m) lg[(int64_t)r * a.vocab + v] = acc[r];
}

// Binary16 rows in T64 order: unit (g, j) = 1 KiB, lane l holds columns
// [8j, 8j+8) of row 64g + l (zero past the last row), so one wave load of a
// unit is one contiguous 1 KiB request.  out has ceil(rows/64) * (h/8)
// units; one thread per 16-byte piece.
extern "C" __global__ __launch_bounds__(256) void lgx_k_repack_f16_t64(const lgx_t64_args a) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int ncg = a.h >> 3;
    const int64_t total = (int64_t)((a.rows + 63) >> 6) * ncg * 64;
    if (i >= total) return;
    const int l = (int)(i & 63);
    const int64_t u = i >> 6;
    const int g = (int)(u / ncg), j = (int)(u - (int64_t)g * ncg);
    const int row = 64 * g + l;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (row < a.rows) v = *(const uint4*)((const uint16_t*)a.src + (int64_t)row * a.h + 8 * j);
    ((uint4*)a.dst)[i] = v;
}

// Binary32 rows [rows][h] -> T16 column order [rows/16][h][16] (the
// activation layout of lgx_k_lm_head_t64); one thread per element.
extern "C" __global__ __launch_bounds__(256) void lgx_k_rows_to_t16(const lgx_t64_args a) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)a.rows * a.h) return;
    const int row = (int)(i / a.h), col = (int)(i - (int64_t)row * a.h);
    ((float*)a.dst)[((int64_t)(row >> 4) * a.h + col) * 16 + (row & 15)] = ((const float*)a.src)[i];
}

// Tied binary16 lm_head over T64 rows: the canonical chain of one
// 1024-column range per blockIdx.z (the sequential fmaf chain over the
// range's columns) into range partial z ([ranges][m][vocab], the consumers
// apply the pairwise tree; h <= 1024 is one range, the logit itself).  One
// wave per (64 vocabulary rows, 16 activation rows, range): lane l owns
// vocabulary row 64g + l and keeps 16 chains.  The activation comes in T16 column order, so the 16
// values of one column are one 64-byte scalar load into SGPRs (wave-uniform,
// no LDS traffic) feeding 16 independent chains; the binary16 units stream
// in as whole 1 KiB wave loads, LGX_LMT_PF units ahead.
#define LGX_LMT_PF 4
extern "C" __global__ __launch_bounds__(64) void lgx_k_lm_head_t64(const lgx_lmhead_args a) {
    typedef const __attribute__((address_space(4))) float* cfloat_p;
    const int g = blockIdx.x, lane = threadIdx.x;
    const int m0 = blockIdx.y * 16, nm = min(16, a.m - m0);
    const int ncg = a.h >> 3;
    // the range's units (8 columns each): [128 z, min(ncg, 128 z + 128))
    const int jb = blockIdx.z * 128, je = min(ncg, jb + 128);
    const uint4* ep = (const uint4*)a.emb + (int64_t)g * ncg * 64 + lane;
    const cfloat_p xt = (cfloat_p)(a.x + (int64_t)blockIdx.y * a.h * 16);
    float acc[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    // h % 32 == 0 (host check): whole groups of LGX_LMT_PF units, and every
    // prefetch is issued (the last unit is re-requested at the tail) so the
    // compiler's wait counts stay exact
    uint4 e[LGX_LMT_PF];
#pragma unroll
    for (int u = 0; u < LGX_LMT_PF; ++u) e[u] = ep[(jb + u) * 64];
    for (int j0 = jb; j0 < je; j0 += LGX_LMT_PF) {
#pragma unroll
        for (int u = 0; u < LGX_LMT_PF; ++u) {
            const int j = j0 + u;
            const uint4 cur = e[u];
            e[u] = ep[min(j + LGX_LMT_PF, je - 1) * 64];
            const float ev[8] = {h2f(cur.x & 0xffffu), h2f(cur.x >> 16), h2f(cur.y & 0xffffu),
                                 h2f(cur.y >> 16),     h2f(cur.z & 0xffffu), h2f(cur.z >> 16),
                                 h2f(cur.w & 0xffffu), h2f(cur.w >> 16)};
            const cfloat_p xc = xt + (int64_t)j * 128;
#pragma unroll
            for (int c = 0; c < 8; ++c) {
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[r] = fmaf(xc[c * 16 + r], ev[c], acc[r]);
            }
        }
    }
    const int v = 64 * g + lane;
    if (v >= a.vocab) return;
    float* lg = a.logits + (int64_t)blockIdx.z * a.m * a.vocab;
#pragma unroll
    for (int r = 0; r < 16; ++r)
        if (r < nm) lg[(int64_t)(m0 + r) * a.vocab + v] = acc[r];
}

// Greedy token, in two launches.  Partial: workgroup (slice, row) takes the
// first maximum of its LGX_ARGMAX_SLICE logits (tree of the range partials,
// NaN skipped) -> candidate (value, index).  Final: per row, the candidate
// with the larger value, on ties the lower index (the first maximum of the
// row; -0 == +0; no candidate -> 0); then tokens[b] = it, seq_len[b] += advance.
__device__ __forceinline__ void better(float& bv, int& bi, float ov, int oi) {
    if (oi != 0x7fffffff && (bi == 0x7fffffff || ov > bv || (ov == bv && oi < bi))) {
        bv = ov;
        bi = oi;
    }
}

__device__ __forceinline__ void wave_best(float& bv, int& bi) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = shfl_xor_f(bv, o);
        const int oi = __shfl_xor(bi, o, 64);
        better(bv, bi, ov, oi);
    }
}

extern "C" __global__ __launch_bounds__(256) void lgx_k_argmax_partial(const lgx_argmax_args a) {
    __shared__ float wv[4];
    __shared__ int wi[4];
    const int sl = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
    const int64_t stride = (int64_t)a.m * a.vocab;
    const int v0 = sl * LGX_ARGMAX_SLICE + t;
    float best = -__builtin_inff();
    int idx = 0x7fffffff;
    for (int k0 = 0; k0 < LGX_ARGMAX_SLICE / 256; k0 += 4) {
        bool on[4];
        float x[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) on[e] = v0 + 256 * (k0 + e) < a.vocab;
        // lm_head partials: K = hidden <= 8192, so at most 8 ranges
        tree_partials_n<4, 8>(a.part, a.nr, stride, (int64_t)b * a.vocab + v0 + 256 * k0, 256, on, x);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (on[e] && x[e] == x[e] && (idx == 0x7fffffff || x[e] > best)) {
                best = x[e];
                idx = v0 + 256 * (k0 + e);
            }
        }
    }
    wave_best(best, idx);
    if ((t & 63) == 0) {
        wv[t >> 6] = best;
        wi[t >> 6] = idx;
    }
    __syncthreads();
    if (t == 0) {
        float bv = wv[0];
        int bi = wi[0];
        for (int w = 1; w < 4; ++w) better(bv, bi, wv[w], wi[w]);
        a.cand_v[(int64_t)b * a.nslices + sl] = bv;
        a.cand_i[(int64_t)b * a.nslices + sl] = bi;
    }
}

extern "C" __global__ __launch_bounds__(64) void lgx_k_argmax_final(const lgx_argmax_args a) {
    const int b = blockIdx.x, l = threadIdx.x;
    float bv = -__builtin_inff();
    int bi = 0x7fffffff;
    for (int s2 = l; s2 < a.nslices; s2 += 64)
        better(bv, bi, a.cand_v[(int64_t)b * a.nslices + s2], a.cand_i[(int64_t)b * a.nslices + s2]);
    wave_best(bv, bi);
    if (l == 0) {
        a.tokens[b] = bi == 0x7fffffff ? 0 : bi;
        if (a.seq_len) a.seq_len[b] += a.advance;
    }
}

// ---------------------------------------------------------------------------
// Certified greedy token of a tied binary16 lm_head: the token of lgx_argmax
// over the canonical logits z[b][v] (sequential fmaf chain over k of
// x[b][k] * e[v][k]) without computing every chain.
//
// lgx_k_lm_cert (workgroup = slice of LGX_LMC_GROUPS 64-row groups, one wave
// per group): row b of x is scaled by s = 2^p (max |x| s in [2^14, 2^15)),
// y = x s and h = f16(y); binary16 MFMAs (f32 accumulation) give
// T = sum_k h e per (v, b).  With S = sum_k |e|, D = the same sum over the
// subnormal e, N >= ||e||_2 (per row, lgx_k_lm_rowconst) and H >= ||h||_2
// (per row of x), |s z - T| <= eps = CA H N + CS S + CD D, taking:
//   - the MFMA accumulation: at most 2^-9 of sum |h| |e| (the sequential
//     round-to-nearest bound for 1024 terms is 2^-14), and sum |h| |e| <=
//     ||h|| ||e|| (Cauchy-Schwarz);
//   - the rounding y -> h: |y - h| <= 2^-11 |h| + 2^-25;
//   - binary16 inputs flushed to zero or not: 2^-14 per flushed h, the
//     subnormal e through D with |h| <= 2^15;
//   - the chain's own rounding: gamma_H = 1024 u / (1 - 1024 u), u = 2^-24,
//     times sum |y| |e|;
// so CA = 2^-9 + 2^-11 + gamma_H (1 + 2^-11), CS = 2^-14 + 2^-25 (+ the
// chain's share), CD = 2^15, each rounded up; eps is then widened for the
// binary32 arithmetic of the bound itself.  The summary of (b, slice): the
// largest lower bound L = T - eps, the largest upper bound U = T + eps, and
// the rows whose U reaches L.
//
// lgx_k_lm_pick (workgroup = row b): L(b) = max over slices; a row v can be
// the first maximum only if U(v) >= L(b) (otherwise s z_v <= U(v) < L(v')
// <= s z_v' for some v').  Those rows get the exact chain (rows of a slice
// holding more than LGX_LMC_CAND of them, or of a row b whose x is not
// finite or outside [2^-60, 2^60] in magnitude: every row of the slice, or
// of the vocabulary); the token is the first maximum of the exact values
// (NaN skipped, none gives 0), then seq_len[b] += advance.
// ---------------------------------------------------------------------------
// binary16 per staged row: h columns, zeros up to the last column of the
// k-steps past h that the prefetch ring runs, and 8 of bank spread
#define LGX_LMC_XS (LGX_LMC_MAXH + 96 + 8)
#define LGX_LMC_CA 2.51e-3f
#define LGX_LMC_CS 6.3e-5f
#define LGX_LMC_CD 32800.0f

// Upper bounds per row: rowc[v] = (sum_k |e|, the same over subnormal e,
// ||e||_2, 0).  The sums of magnitudes are exact in fp64 (binary16
// magnitudes are multiples of 2^-24 below 2^16: 1024 of them need 50 bits);
// the sum of squares has relative error below 2^-42 and is widened before
// the square root.  Each is rounded up to binary32; +inf for a row with a
// non-finite entry.  One wave per row.
__device__ __forceinline__ float f64_to_f32_up(double d) {
    float f = (float)d;
    if ((double)f < d) f = __uint_as_float(__float_as_uint(f) + 1u);   // d >= 0
    return f;
}
extern "C" __global__ __launch_bounds__(256) void lgx_k_lm_rowconst(const lgx_lmrc_args a) {
    const int lane = threadIdx.x & 63;
    const int v = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (v >= a.vocab) return;                   // whole waves; no barrier below
    const uint16_t* er = a.emb + (int64_t)v * a.h;
    double s = 0.0, d = 0.0, q = 0.0;
    int bad = 0;
    for (int k = lane; k < a.h; k += 64) {
        const uint32_t mag = er[k] & 0x7fffu;
        bad |= mag >= 0x7c00u ? 1 : 0;
        const double f = (double)h2f(mag);
        s += f;
        q += f * f;
        if (mag < 0x0400u) d += f;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        s += __shfl_xor(s, o, 64);
        d += __shfl_xor(d, o, 64);
        q += __shfl_xor(q, o, 64);
        bad |= __shfl_xor(bad, o, 64);
    }
    if (lane == 0) {
        const float inf = __builtin_inff();
        ((float4*)a.rowc)[v] = bad ? make_float4(inf, inf, inf, 0.0f)
                                   : make_float4(f64_to_f32_up(s), f64_to_f32_up(d),
                                                 f64_to_f32_up(sqrt(q * (1.0 + 0x1p-40)) * (1.0 + 0x1p-40)),
                                                 0.0f);
    }
}

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
__device__ __forceinline__ v8h as_v8h(uint4 u) { return __builtin_bit_cast(v8h, u); }

#define LGX_LMC_RING 4                  // k-steps in flight: the one in use and three ahead
extern "C" __global__ __launch_bounds__(64 * LGX_LMC_GROUPS) void lgx_k_lm_cert(const lgx_lmc_args a) {
    // rows of the scaled x (binary16 bits), [b][k] with a padded row stride:
    // an MFMA B operand (16 rows x 8 columns) is one conflict-free read
    __shared__ __align__(16) uint16_t xh[LGX_LMC_MAXB * LGX_LMC_XS];
    __shared__ float4 rc[LGX_LMC_GROUPS][64];
    __shared__ float hn[LGX_LMC_MAXB];
    __shared__ float lmx[LGX_LMC_GROUPS][LGX_LMC_MAXB], umx[LGX_LMC_GROUPS][LGX_LMC_MAXB];
    __shared__ float lwg[LGX_LMC_MAXB], uwg[LGX_LMC_MAXB];
    __shared__ int ccnt[LGX_LMC_MAXB], rexact[LGX_LMC_MAXB];
    __shared__ float cu[LGX_LMC_MAXB][LGX_LMC_CAND];
    __shared__ int cv[LGX_LMC_MAXB][LGX_LMC_CAND];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, c = lane >> 4;
    const int ngroups = (a.vocab + 63) >> 6;
    const int g = blockIdx.x * LGX_LMC_GROUPS + w;
    const bool gon = g < ngroups;                          // wave-uniform
    const int ncg = a.h >> 3, ns = a.h >> 5;
    // the group's T64 units (ncg KiB); k-step s, q-block q of lane (r, c):
    // unit 4s + c, position 16q + r (row 16q + r, columns 32s + 8c ..).
    // Past the group (and for a wave without a group) the loads fall outside
    // the descriptor: zeros, no memory access.
    const __amdgpu_buffer_rsrc_t er = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.emb_t64 + (int64_t)min(g, ngroups - 1) * ncg * 512), 0, gon ? ncg * 1024 : 0,
        LGX_BUF_DWORD3);
    uint4 wa[LGX_LMC_RING][4];
    auto ld = [&](int s, uint4 (&dst)[4]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) dst[q] = ld_buf_stream(er, ((4 * s + c) * 64 + 16 * q + r) * 16);
    };
#pragma unroll
    for (int i = 0; i < LGX_LMC_RING - 1; ++i) ld(i, wa[i]);
    // per-row constants of the group's rows
    rc[w][lane] = ((const float4*)a.rowc)[min(64 * g + lane, a.vocab - 1)];
    // stage x: wave w takes rows w, w + GROUPS, ...; lane holds columns
    // 8(lane + 64 i) .. + 7 (i < 3: the h <= 1024 columns and the zeros
    // after them)
    for (int b = w; b < LGX_LMC_MAXB; b += LGX_LMC_GROUPS) {
        const bool brow = b < a.m;                         // wave-uniform
        const float* xr = a.x + (int64_t)min(b, a.m - 1) * a.h;
        float xv[3][8];
        float mx = 0.0f;
        int bad = 0;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const int k8 = lane + 64 * i;
            const bool on = brow && 8 * k8 < a.h;
            const float4* p = (const float4*)(xr + min(8 * k8, a.h - 8));
            const float4 u0 = p[0], u1 = p[1];
            const float t[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                xv[i][e] = on ? t[e] : 0.0f;
                const float ax = fabsf(xv[i][e]);
                bad |= !(ax <= 3.4028234663852886e38f) ? 1 : 0;   // NaN or inf
                mx = fmaxf(mx, ax);
            }
        }
        mx = wave_max(mx);
        const bool anybad = __ballot(bad) != 0;
        const bool exact = anybad || !(mx >= 0x1p-60f) || mx > 0x1p60f;
        // mx = f 2^ex with f in [0.5, 1) (mx normal when not exact)
        const int ex = (int)((__float_as_uint(mx) >> 23) & 0xffu) - 126;
        const int p = exact ? 0 : 15 - ex;                  // mx 2^p in [2^14, 2^15)
        double sq = 0.0;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const int k8 = lane + 64 * i;
            uint32_t hw[4];
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                uint32_t hp[2];
#pragma unroll
                for (int f = 0; f < 2; ++f) {
                    const float y = exact ? 0.0f : ldexpf(xv[i][e + f], p);
                    const uint16_t hb = f2h(y);
                    const double hd = (double)h2f(hb);
                    sq += hd * hd;
                    hp[f] = hb;
                }
                hw[e / 2] = hp[0] | (hp[1] << 16);
            }
            // columns [h, XS) are zero: steps past h read them
            if (8 * k8 + 8 <= LGX_LMC_XS)
                *(uint4*)&xh[b * LGX_LMC_XS + 8 * k8] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) sq += __shfl_xor(sq, o, 64);
        if (lane == 0) {
            rexact[b] = brow && exact ? 1 : 0;
            // ||h||_2 rounded up (the fp64 sum of squares is within 2^-42)
            hn[b] = f64_to_f32_up(sqrt(sq * (1.0 + 0x1p-40)) * (1.0 + 0x1p-40));
        }
    }
    __syncthreads();

    // T[q][t] of batch tile t (rows 16t .. 16t + 15)
    const int nt = a.m > 16 ? 2 : 1;
    const v4f zf = {0.0f, 0.0f, 0.0f, 0.0f};
    v4f T[4][2];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int t = 0; t < 2; ++t) T[q][t] = zf;
    auto step = [&](int s, int slot) {
        uint4 cur[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) cur[q] = wa[slot][q];
        ld(s + LGX_LMC_RING - 1, wa[(slot + LGX_LMC_RING - 1) % LGX_LMC_RING]);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            if (t < nt) {                                   // workgroup-uniform
                const uint4 bh = *(const uint4*)&xh[(16 * t + r) * LGX_LMC_XS + 32 * s + 8 * c];
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    T[q][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_v8h(cur[q]), as_v8h(bh), T[q][t], 0, 0, 0);
            }
        }
    };
#pragma unroll 1
    for (int s0 = 0; s0 < ns; s0 += LGX_LMC_RING) {
        // steps past ns multiply zeros (loads past the group, zero columns)
#pragma unroll
        for (int i = 0; i < LGX_LMC_RING; ++i) step(s0 + i, i);
    }

    // bounds of element (q, t, e): vocabulary row 64g + 16q + 4c + e, batch
    // row 16t + r
    auto bounds = [&](int q, int t, int e, float& lo, float& hi, float& eps) {
        const float4 k4 = rc[w][16 * q + 4 * c + e];
        const float tv = T[q][t][e];
        eps = LGX_LMC_CA * (hn[16 * t + r] * k4.z) + LGX_LMC_CS * k4.x + LGX_LMC_CD * k4.y;
        eps = eps * (1.0f + 0x1p-18f) + fabsf(tv) * 0x1p-21f;
        lo = tv - eps;
        hi = tv + eps;
        // A row with a non-finite entry has infinite constants; its T can be
        // NaN (an inf or NaN entry against a column of x that rounds to 0 in
        // binary16: 0 x inf in the MFMA) and inf - inf is NaN.  A NaN bound
        // certifies nothing: the row stays a candidate for its exact chain.
        if (hi != hi) hi = __builtin_inff();
        if (lo != lo) lo = -__builtin_inff();
        const int v = 64 * g + 16 * q + 4 * c + e;
        if (!gon || v >= a.vocab) lo = hi = -__builtin_inff();
    };
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        if (t < nt) {
            float lm = -__builtin_inff(), um = -__builtin_inff();
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float lo, hi, eps;
                    bounds(q, t, e, lo, hi, eps);
                    lm = fmaxf(lm, lo);
                    um = fmaxf(um, hi);
                    const int b = 16 * t + r, v = 64 * g + 16 * q + 4 * c + e;
                    if (a.dbg && b < a.m && gon && v < a.vocab) {
                        float* dp = a.dbg + ((int64_t)b * a.vocab + v) * 2;
                        dp[0] = T[q][t][e];
                        dp[1] = eps;
                    }
                }
            lm = fmaxf(lm, shfl_xor_f(lm, 16));
            lm = fmaxf(lm, shfl_xor_f(lm, 32));
            um = fmaxf(um, shfl_xor_f(um, 16));
            um = fmaxf(um, shfl_xor_f(um, 32));
            if (c == 0) {
                lmx[w][16 * t + r] = lm;
                umx[w][16 * t + r] = um;
            }
        }
    }
    __syncthreads();
    if (tid < LGX_LMC_MAXB) {
        float lm = -__builtin_inff(), um = -__builtin_inff();
        if (tid < 16 * nt) {
#pragma unroll
            for (int j = 0; j < LGX_LMC_GROUPS; ++j) {
                lm = fmaxf(lm, lmx[j][tid]);
                um = fmaxf(um, umx[j][tid]);
            }
        }
        lwg[tid] = lm;
        uwg[tid] = um;
        ccnt[tid] = 0;
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        if (t < nt) {
            const int b = 16 * t + r;
            const float lb = lwg[b];
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float lo, hi, eps;
                    bounds(q, t, e, lo, hi, eps);
                    if (hi >= lb && hi > -__builtin_inff()) {
                        const int slot = atomicAdd(&ccnt[b], 1);
                        if (slot < LGX_LMC_CAND) {
                            cu[b][slot] = hi;
                            cv[b][slot] = 64 * g + 16 * q + 4 * c + e;
                        }
                    }
                }
        }
    }
    __syncthreads();
    if (tid < a.m) {
        lgx_lmc_summary* o = a.summ + (int64_t)tid * a.nslices + blockIdx.x;
        const int n = ccnt[tid];
        o->L = lwg[tid];
        o->Umax = uwg[tid];
        o->cnt = rexact[tid] ? LGX_LMC_EXACT : n;
        o->pad = 0;
#pragma unroll
        for (int i = 0; i < LGX_LMC_CAND; ++i) {
            o->U[i] = i < n ? cu[tid][i] : -__builtin_inff();
            o->v[i] = i < n ? cv[tid][i] : 0x7fffffff;
        }
    }
}

// The canonical chain of vocabulary row v against the staged row xs, with
// the row itself staged in es (binary32): the wave loads it (one memory
// round), lane 0 chains it, 32 columns per batch of 16-byte LDS reads.
__device__ __forceinline__ float lm_chain_wave(const float* xs, float* es, const uint16_t* emb, int v,
                                               int h, int lane) {
    const uint4* er = (const uint4*)(emb + (int64_t)v * h);
    for (int j = lane; j < (h >> 3); j += 64) {
        const uint4 e = er[j];
        float4* d = (float4*)(es + 8 * j);
        d[0] = make_float4(h2f(e.x & 0xffffu), h2f(e.x >> 16), h2f(e.y & 0xffffu), h2f(e.y >> 16));
        d[1] = make_float4(h2f(e.z & 0xffffu), h2f(e.z >> 16), h2f(e.w & 0xffffu), h2f(e.w >> 16));
    }
    float acc = 0.0f;
    if (lane == 0) {
        for (int k0 = 0; k0 < h; k0 += 32) {
            float4 xa[8], ea[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                xa[i] = *(const float4*)(xs + k0 + 4 * i);
                ea[i] = *(const float4*)(es + k0 + 4 * i);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                acc = fmaf(xa[i].x, ea[i].x, acc);
                acc = fmaf(xa[i].y, ea[i].y, acc);
                acc = fmaf(xa[i].z, ea[i].z, acc);
                acc = fmaf(xa[i].w, ea[i].w, acc);
            }
        }
    }
    return acc;
}

// The canonical chains of 64 consecutive rows v0 + lane (rows >= v1 idle):
// each lane streams its own row in 64-column blocks, one block ahead.
__device__ __forceinline__ float lm_chain_lanes(const float* xs, const uint16_t* emb, int v, int h) {
    const uint4* er = (const uint4*)(emb + (int64_t)v * h);
    const int nb = h >> 6;
    uint4 cur[8], nxt[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) cur[j] = er[j];
    float acc = 0.0f;
    for (int kb = 0; kb < nb; ++kb) {
        const int kn = min(kb + 1, nb - 1);                 // the last block re-reads itself
#pragma unroll
        for (int j = 0; j < 8; ++j) nxt[j] = er[8 * kn + j];
        const float* xk = xs + 64 * kb;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint4 e = cur[j];
            acc = fmaf(xk[8 * j + 0], h2f(e.x & 0xffffu), acc);
            acc = fmaf(xk[8 * j + 1], h2f(e.x >> 16), acc);
            acc = fmaf(xk[8 * j + 2], h2f(e.y & 0xffffu), acc);
            acc = fmaf(xk[8 * j + 3], h2f(e.y >> 16), acc);
            acc = fmaf(xk[8 * j + 4], h2f(e.z & 0xffffu), acc);
            acc = fmaf(xk[8 * j + 5], h2f(e.z >> 16), acc);
            acc = fmaf(xk[8 * j + 6], h2f(e.w & 0xffffu), acc);
            acc = fmaf(xk[8 * j + 7], h2f(e.w >> 16), acc);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) cur[j] = nxt[j];
    }
    return acc;
}

#define LGX_LMP_MAXSL 1024
#define LGX_LMP_MAXC 2048
#define LGX_LMP_WAVES 8
extern "C" __global__ __launch_bounds__(64 * LGX_LMP_WAVES) void lgx_k_lm_pick(const lgx_lmp_args a) {
    constexpr int NT = 64 * LGX_LMP_WAVES;
    __shared__ __align__(16) float xs[LGX_LMC_MAXH];
    __shared__ __align__(16) float es[LGX_LMP_WAVES][LGX_LMC_MAXH];
    __shared__ float rl[LGX_LMP_WAVES];
    __shared__ int cand[LGX_LMP_MAXC];
    __shared__ int dense[LGX_LMP_MAXSL];
    __shared__ int ncand, ndense, exact_row;
    __shared__ float bvs[LGX_LMP_WAVES];
    __shared__ int bis[LGX_LMP_WAVES];
    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const lgx_lmc_summary* sm = a.summ + (int64_t)b * a.nslices;
    for (int k = tid; k < a.h; k += NT) xs[k] = a.x[(int64_t)b * a.h + k];
    // the records of this thread's slices (nslices <= 2 NT) in one memory
    // round: {L, Umax, cnt, pad}, U[0..7], v[0..7]
    static_assert(sizeof(lgx_lmc_summary) == 80 && LGX_LMC_CAND == 8, "record layout");
    uint4 rec[2][5];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint4* rp = (const uint4*)(sm + min(tid + NT * i, a.nslices - 1));
#pragma unroll
        for (int j = 0; j < 5; ++j) rec[i][j] = rp[j];
    }
    float lm = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < 2; ++i)
        if (tid + NT * i < a.nslices) lm = fmaxf(lm, __uint_as_float(rec[i][0].x));
    lm = wave_max(lm);
    if (lane == 0) rl[w] = lm;
    if (tid == 0) {
        ncand = 0;
        ndense = 0;
        exact_row = (int)rec[0][0].z == LGX_LMC_EXACT ? 1 : 0;   // slice 0's record
    }
    __syncthreads();
    float L = rl[0];
#pragma unroll
    for (int j = 1; j < LGX_LMP_WAVES; ++j) L = fmaxf(L, rl[j]);
    if (!exact_row) {
        // the listed rows whose bound reaches L; slices with more rows than
        // listed go to the dense pass
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int s = tid + NT * i;
            const float umax = __uint_as_float(rec[i][0].y);
            const int cnt = (int)rec[i][0].z;
            if (s >= a.nslices || !(umax >= L)) continue;
            if (cnt > LGX_LMC_CAND) {
                dense[atomicAdd(&ndense, 1)] = s;
                continue;
            }
            const uint32_t uu[8] = {rec[i][1].x, rec[i][1].y, rec[i][1].z, rec[i][1].w,
                                    rec[i][2].x, rec[i][2].y, rec[i][2].z, rec[i][2].w};
            const uint32_t vv[8] = {rec[i][3].x, rec[i][3].y, rec[i][3].z, rec[i][3].w,
                                    rec[i][4].x, rec[i][4].y, rec[i][4].z, rec[i][4].w};
            bool full = false;
#pragma unroll
            for (int j = 0; j < LGX_LMC_CAND; ++j)
                if (j < cnt && __uint_as_float(uu[j]) >= L) {
                    const int k = atomicAdd(&ncand, 1);
                    if (k < LGX_LMP_MAXC)
                        cand[k] = (int)vv[j];
                    else
                        full = true;                // (a row listed twice is harmless)
                }
            if (full) dense[atomicAdd(&ndense, 1)] = s;
        }
    }
    __syncthreads();
    float bv = -__builtin_inff();
    int bi = 0x7fffffff;
    auto take = [&](float z, int v) {
        if (z == z) better(bv, bi, z, v);
    };
    // sparse: one candidate per wave at a time
    const int nc = min(ncand, LGX_LMP_MAXC);
    for (int i = w; i < nc; i += LGX_LMP_WAVES) {
        const int v = cand[i];
        const float z = lm_chain_wave(xs, es[w], a.emb, v, a.h, lane);
        if (lane == 0) take(z, v);
    }
    // dense: every row of the listed slices (of every slice for an exact
    // row), one row per lane
    const int nd = exact_row ? a.nslices : ndense;
    for (int i = 0; i < nd; ++i) {
        const int s = exact_row ? i : dense[i];
        const int v0 = s * LGX_LMC_ROWS;
        const int v1 = min(v0 + LGX_LMC_ROWS, a.vocab);
        for (int vb = v0 + 64 * w; vb < v1; vb += NT) {       // wave-uniform
            const int v = vb + lane;
            const float z = lm_chain_lanes(xs, a.emb, min(v, v1 - 1), a.h);
            if (v < v1) take(z, v);
        }
    }
    // first maximum over the threads
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = shfl_xor_f(bv, o);
        const int oi = __shfl_xor(bi, o, 64);
        better(bv, bi, ov, oi);
    }
    if (lane == 0) {
        bvs[w] = bv;
        bis[w] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        float fv = bvs[0];
        int fi = bis[0];
        for (int j = 1; j < LGX_LMP_WAVES; ++j) better(fv, fi, bvs[j], bis[j]);
        a.tokens[b] = fi == 0x7fffffff ? 0 : fi;
        if (a.seq_len) a.seq_len[b] += a.advance;
    }
}

// ---------------------------------------------------------------------------
// Seeded top-k / top-p sampling.  A logit x at vocabulary index v has the key
//   (orderable bits of x, -0 taken as +0) << 32 | (0xffffffff - v)
// so keys sort by value descending, then index ascending; NaN has no key
// (0 marks an empty slot; every real key is larger).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t sample_key(float x, int v) {
    if (x != x) return 0;
    uint32_t u = __float_as_uint(x == 0.0f ? 0.0f : x);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | (uint64_t)(0xffffffffu - (uint32_t)v);
}
__device__ __forceinline__ float key_value(uint64_t k) {
    uint32_t u = (uint32_t)(k >> 32);
    u = (u & 0x80000000u) ? (u & 0x7fffffffu) : ~u;
    return __uint_as_float(u);
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)k, o, 64), hi = __shfl_xor((uint32_t)(k >> 32), o, 64);
        const uint64_t ok = ((uint64_t)hi << 32) | lo;
        k = ok > k ? ok : k;
    }
    return k;
}

// Slice (4096 logits) x row: each wave takes the top_k keys of its 1024
// logits by rounds of wave maxima; thread 0 merges the four sorted lists.
extern "C" __global__ __launch_bounds__(256) void lgx_k_sample_partial(const lgx_sample_args a) {
    __shared__ uint64_t lst[4][LGX_SAMPLE_MAX_K];
    const int sl = blockIdx.x, b = blockIdx.y, t = threadIdx.x, w = t >> 6, l = t & 63;
    const int64_t stride = (int64_t)a.m * a.vocab;
    const int v0 = sl * LGX_ARGMAX_SLICE + w * 1024 + l;
    uint64_t k[16];
#pragma unroll
    for (int c = 0; c < 16; c += 4) {
        bool on[4];
        float x[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) on[e] = v0 + 64 * (c + e) < a.vocab;
        tree_partials_n<4, 8>(a.part, a.nr, stride, (int64_t)b * a.vocab + v0 + 64 * c, 64, on, x);
#pragma unroll
        for (int e = 0; e < 4; ++e) k[c + e] = on[e] ? sample_key(x[e], v0 + 64 * (c + e)) : 0;
    }
    uint64_t lm = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) lm = k[i] > lm ? k[i] : lm;
    for (int r = 0; r < a.top_k; ++r) {
        const uint64_t best = wave_max_u64(lm);
        if (l == 0) lst[w][r] = best;
        if (best == 0) {
            for (int q = r + 1 + l; q < a.top_k; q += 64) lst[w][q] = 0;
            break;                                   // wave-uniform
        }
        if (lm == best) {                            // keys are unique: one lane
            lm = 0;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                k[i] = k[i] == best ? 0 : k[i];
                lm = k[i] > lm ? k[i] : lm;
            }
        }
    }
    __syncthreads();
    if (t == 0) {
        int h[4] = {0, 0, 0, 0};
        uint64_t* out = a.cand + ((int64_t)b * a.nslices + sl) * LGX_SAMPLE_MAX_K;
        for (int r = 0; r < a.top_k; ++r) {
            int wi = 0;
            uint64_t best = 0;
            for (int q = 0; q < 4; ++q) {
                const uint64_t c = h[q] < a.top_k ? lst[q][h[q]] : 0;
                if (c > best) {
                    best = c;
                    wi = q;
                }
            }
            out[r] = best;
            if (best) ++h[wi];
        }
    }
}

__device__ __forceinline__ uint64_t sm_mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Row b: the top_k keys of the slice lists (rounds of wave maxima over the
// list heads), then on lane 0, in key order j = 0, 1, ...:
//   e_j = lgx_expf((v_j - v_0) * inv_temp), c_j = c_{j-1} + e_j (c_{-1} = 0)
//   J   = first j with c_j >= top_p * c_{n-1}
//   u   = (x >> 40) * 2^-24, x = element pos of stream stream0 + b of seed
//   pick the first j <= J with c_j > u * c_J (J if none)
extern "C" __global__ __launch_bounds__(64) void lgx_k_sample_final(const lgx_sample_args a) {
    __shared__ uint64_t top[LGX_SAMPLE_MAX_K];
    const int b = blockIdx.x, l = threadIdx.x;
    const uint64_t* lists = a.cand + (int64_t)b * a.nslices * LGX_SAMPLE_MAX_K;
    int h = 0;
    uint64_t head = l < a.nslices ? lists[(int64_t)l * LGX_SAMPLE_MAX_K] : 0;
    int n = 0;
    for (int r = 0; r < a.top_k; ++r) {
        const uint64_t best = wave_max_u64(head);
        if (best == 0) break;                        // wave-uniform
        if (l == 0) top[r] = best;
        n = r + 1;
        if (head == best) {
            ++h;
            head = h < a.top_k ? lists[(int64_t)l * LGX_SAMPLE_MAX_K + h] : 0;
        }
    }
    __syncthreads();
    if (l != 0) return;
    int tok = 0;
    const int pos = a.pos ? a.pos[b] : a.seq_len[b];
    if (n > 0) {
        const float v0 = key_value(top[0]);
        float c[LGX_SAMPLE_MAX_K];
        float acc = 0.0f;
        for (int j = 0; j < n; ++j) {
            acc = acc + lgx_expf((key_value(top[j]) - v0) * a.inv_temp);
            c[j] = acc;
        }
        const float thr = a.top_p * acc;
        int J = n - 1;
        for (int j = 0; j < n; ++j)
            if (c[j] >= thr) {
                J = j;
                break;
            }
        const uint64_t sb = sm_mix(a.seed + 0x9E3779B97F4A7C15ull) ^
                            sm_mix(((uint64_t)(a.stream0 + b) + 1ull) * 0xD1B54A32D192ED03ull);
        const uint64_t x = sm_mix(sb + ((uint64_t)pos + 1ull) * 0x9E3779B97F4A7C15ull);
        const float u = (float)(uint32_t)(x >> 40) * 0x1.0p-24f;
        const float r = u * c[J];
        int pick = J;
        for (int j = 0; j <= J; ++j)
            if (c[j] > r) {
                pick = j;
                break;
            }
        tok = (int)(0xffffffffu - (uint32_t)top[pick]);
    }
    a.tokens[b] = tok;
    if (a.seq_len) a.seq_len[b] += a.advance;
}

extern "C" __global__ __launch_bounds__(64) void lgx_k_advance(const lgx_advance_args a) {
    const int b = blockIdx.x * 64 + threadIdx.x;
    if (b < a.m) a.seq_len[b] = (a.keep ? a.seq_len[b] : 0) + a.add;
}

// ---------------------------------------------------------------------------
// Activation rows to T16 tiles: thread per 16-byte lane slot of a 1 KiB unit
// (unit = row tile x 64-column pair); rows past `rows` are zero.
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void lgx_k_act_to_t16(const lgx_act_t16_args a) {
    const int64_t np = a.k >> 6;
    const int64_t total = (int64_t)((a.rows + 15) >> 4) * np * 64;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int64_t u = i >> 6;
    const int lane = (int)(i & 63);
    const int64_t t = u / np, p = u - t * np;
    const int64_t row = t * 16 + (lane & 15);
    uint2 lo = make_uint2(0, 0), hi = make_uint2(0, 0);
    if (row < a.rows) {
        const int8_t* s = a.src + row * a.k + p * 64 + 8 * (lane >> 4);
        lo = *(const uint2*)s;
        hi = *(const uint2*)(s + 32);
    }
    *(uint4*)(a.dst + i * 16) = make_uint4(lo.x, lo.y, hi.x, hi.y);
}

// ---------------------------------------------------------------------------
// Q8_0 matrix in T16 / S16 tiles to binary16 row-major (the fast prefill's
// GEMM operand): thread per 8 consecutive columns of a row, i.e. one 8-byte
// piece of a T16 lane slot (columns 64p + 32 half + 8 c .. +7 of row 16 t + r
// sit at byte ((t np + p) 64 + r + 16 c) 16 + 8 half of the tiles).
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void lgx_k_dequant_f16(const lgx_dequant_args a) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int k8 = a.k >> 3;
    if (i >= (int64_t)a.n * k8) return;
    const int row = (int)(i / k8), col = (int)(i - (int64_t)row * k8) * 8;
    const int np = a.k >> 6, nh = s16_nhalf(a.k);
    const int t = row >> 4, r = row & 15, p = col >> 6, half = (col >> 5) & 1, c = (col >> 3) & 3;
    const uint2 q8 = *(const uint2*)(a.wt + (((int64_t)t * np + p) * 64 + r + 16 * c) * 16 + 8 * half);
    const int b = col >> 5;
    const float d = h2f(a.wd[(((int64_t)t * nh + (b >> 4)) * 16 + r) * 16 + (b & 15)]);
    const uint32_t w[2] = {q8.x, q8.y};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int8_t lo = (int8_t)((w[e >> 1] >> (16 * (e & 1))) & 0xff);
        const int8_t hi = (int8_t)((w[e >> 1] >> (16 * (e & 1) + 8)) & 0xff);
        o[e] = f2h(d * (float)lo) | ((uint32_t)f2h(d * (float)hi) << 16);
    }
    *(uint4*)(a.out + (int64_t)row * a.k + col) = make_uint4(o[0], o[1], o[2], o[3]);
}

// ---------------------------------------------------------------------------
// Tiled Q8_0 product (prefill; decode batches of 32 / 64 rows).  Workgroup
// tile: 64 weight rows (4 row tiles) x 32*WM activation rows (2*WM row
// tiles) over one group of a.grp aligned ranges (1, 2 or 4).  Four waves;
// wave (wn, wm) owns weight tiles 2wn, 2wn+1 and activation tiles
// WM*wm .. WM*wm + WM-1.  Per 64-column pair a wave issues one MFMA
// i32_16x16x32_i8 per (block, weight tile, activation tile) with the weight
// tile as A, so lane (r, c) of a result holds weight rows 4c..4c+3 of the
// tile against activation row r; the epilogue runs the canonical chain
// acc = fmaf((float)s, f32(dw) * f32(dx), acc) of each element, the scale
// products of a (block, weight tile, activation tile) coming from one rank-1
// f16 MFMA (16x16x16) with the same lane layout, so the VALU does two
// operations per element (convert, fma).  When a
// range ends its values fold into the group's subtree (a binary counter over
// at most four ranges: earlier + later, as in the level-by-level tree) and
// the group's values go to part[g]: aligned groups of a power-of-two number
// of ranges are subtrees of the canonical tree, so the tree over the groups
// is the tree over all ranges.  A gate|up product in one group can instead
// finish with SwiGLU + Q8_0 in the workgroup (a.swiglu): its tile slots then
// pair each gate tile with the up tile of the same columns.
// Staging: two LDS stages of LGX_TG_S pairs filled by direct global->LDS
// loads, 16-byte lanes for the T16 tiles and 4-byte lanes for the scale
// pairs of a 64-column pair, which land pre-arranged: dw as [pair][64 rows]
// (the four rows of a lane are one 16-byte read), dx as [pair][r][2*WM
// tiles] (the WM tiles of a wave are one read).  Every operand of a stage is
// read into registers before the next stage's loads are issued (the
// compiler would otherwise wait for those loads before the reads).
// Workgroup order: physical ids go round-robin over the 8 XCDs; each XCD
// takes a contiguous run of logical tiles, which walk bands of 8 activation
// tiles, n-tile by n-tile (activation tile fastest), so the tiles in flight
// on one XCD share their operands through its L2.
// ---------------------------------------------------------------------------
// S pairs per stage: 2, or 4 for grids of at most two workgroups per compute
// unit (half the stages, so half the dependent memory rounds)
template <int WM, int S>
struct TgSmem {
    uint4 w[4][S][64];
    uint4 x[2 * WM][S][64];
    uint32_t dw[S][64];
    uint32_t dx[S][16 * 2 * WM];
};

template <int WM, int S = 2>
__device__ __forceinline__ void q8_tiled_body(const lgx_gemm_tiled_args& a, const int P) {
    constexpr int MTILES = 2 * WM;
    // two stage buffers as two variables: a direct load into one is known
    // not to alias reads of the other
    __shared__ TgSmem<WM, S> sm0, sm1;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int wn = wave & 1, wm = wave >> 1;
    const int r = lane & 15, c = lane >> 4;
    // XCD-aware logical id, then (group, band of 8 activation tiles, n tile)
    const int T = a.ntn * a.ntm * a.ngroups;
    const int xcd = P & 7, slot = P >> 3;
    const int q8 = T >> 3, r8 = T & 7;
    const int id = xcd * q8 + min(xcd, r8) + slot;
    const int per_g = a.ntn * a.ntm;
    const int g = id / per_g;
    const int rem = id - g * per_g;
    const int band = rem / (8 * a.ntn);
    const int bsz = min(8, a.ntm - 8 * band);
    const int loc = rem - band * 8 * a.ntn;
    const int tn = loc / bsz, tm = 8 * band + (loc - (loc / bsz) * bsz);
    const int tn0 = tn * 4, tm0 = tm * MTILES;

    const int np = a.k >> 6, nb = a.k >> 5, nh = (a.k + 511) >> 9;
    const int ntw = a.n >> 4, ntx = (a.m + 15) >> 4;
    // Weight row tile of the workgroup's tile slot s (0..3).  With the SwiGLU
    // consumer, slot 2w is the gate tile and slot 2w + 1 the up tile of the
    // same 16 columns 32 tn + 16 w (gate rows [0, I), up rows [I, 2I)), so
    // wave (w, .) holds both factors of its outputs.
    const int swi = a.swiglu;
    auto wtile = [&](int s) {
        return swi ? (s & 1) * (swi >> 4) + 2 * tn + (s >> 1) : min(tn0 + s, ntw - 1);
    };
    const int gpairs = a.grp * (LGX_Q8_RANGE_BLOCKS / 2);
    const int pg0 = g * gpairs;
    const int pend = min(pg0 + gpairs, np);
    const int nst = (pend - pg0 + S - 1) / S;
    const v4i zero = {0, 0, 0, 0};
    const v4f zerof = {0.0f, 0.0f, 0.0f, 0.0f};

    // Direct loads of a stage (pairs pair0 .. pair0 + S - 1, clamped to the
    // group): uniform base + per-lane byte offset fixed over the stages.
    //   weights: 4 tiles x S pairs, units j = wave + 4i (tile j / S, pair j % S)
    //   activations: MTILES tiles x S pairs, likewise
    //   weight scale pairs: [s][64 rows], one 4-byte lane per row (waves < S)
    //   activation scale pairs: [s][r][tile], wave instructions j = wave < WM
    static_assert((S == 2 || S == 4) && WM * S <= 8, "stage layout: scale loads on at most four waves");
    const uint32_t off_t16 = lane * 16;
    const uint32_t off_dw = ((uint32_t)wtile(lane >> 4) * nh * 256 + (lane & 15) * 16) * 2;
    const int dxp = (wave * 64 + lane) % (16 * MTILES);            // position within a pair
    const int dx_ml = (dxp % MTILES) * 16 + dxp / MTILES;
    const uint32_t off_dx = (uint32_t)min(tm0 * 16 + dx_ml, a.m - 1) * nb * 2;
    auto stage = [&](TgSmem<WM, S>& sm, int pair0) {
#pragma unroll
        for (int i = 0; i < S; ++i) {
            const int j = wave + 4 * i;
            const int tile = j / S, s = j - tile * S;
            const int t = wtile(tile), p = min(pair0 + s, pend - 1);
            const char* base = (const char*)a.wt + ((int64_t)t * np + p) * 1024;
            __builtin_amdgcn_global_load_lds((const void*)(base + off_t16), (lds_void*)&sm.w[tile][s][0], 16, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < MTILES * S / 4; ++i) {
            const int j = wave + 4 * i;
            const int tile = j / S, s = j - tile * S;
            const int t = min(tm0 + tile, ntx - 1), p = min(pair0 + s, pend - 1);
            const char* base = (const char*)a.xt + ((int64_t)t * np + p) * 1024;
            __builtin_amdgcn_global_load_lds((const void*)(base + off_t16), (lds_void*)&sm.x[tile][s][0], 16, 0, 0);
        }
        if (wave < S) {
            const int b = 2 * min(pair0 + wave, pend - 1);
            const char* base = (const char*)(a.wd + (b >> 4) * 256 + (b & 15));
            __builtin_amdgcn_global_load_lds((const void*)(base + off_dw), (lds_void*)&sm.dw[wave][0], 4, 0, 0);
        }
        if (wave < WM * S / 2) {                  // 64 words per instruction, 16*MTILES per pair
            const int s = (wave * 64 + lane) / (16 * MTILES);   // uniform unless WM == 1
            const char* src = (const char*)(a.xd + 2 * min(pair0 + s, pend - 1)) + off_dx;
            __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)(&sm.dx[0][0] + wave * 64), 4, 0, 0);
        }
    };

    float acc[2][WM][4], l0[2][WM][4], l1[2][WM][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < WM; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[i][j][v] = l0[i][j][v] = l1[i][j][v] = 0.0f;
    int cnt = 0;

    // One stage: its products from `cur` while the next stage loads into `nxt`.
    auto run = [&](int q, TgSmem<WM, S>& cur, TgSmem<WM, S>& nxt) {
        __syncthreads();                          // stage q landed; stage q-1 fully read
        uint4 A[S][2], B[S][WM];
        uint32_t DWR[S][2], DX[S][WM];
#pragma unroll
        for (int s = 0; s < S; ++s) {
            A[s][0] = cur.w[2 * wn][s][lane];
            A[s][1] = cur.w[2 * wn + 1][s][lane];
#pragma unroll
            for (int j = 0; j < WM; ++j) B[s][j] = cur.x[WM * wm + j][s][lane];
            // weight scale pair of row r of tiles 2wn, 2wn+1 (lanes 16.. read
            // the same rows; their values meet zeros in the scale product)
            DWR[s][0] = cur.dw[s][(2 * wn) * 16 + r];
            DWR[s][1] = cur.dw[s][(2 * wn + 1) * 16 + r];
            const uint32_t* dxr = &cur.dx[s][r * MTILES + WM * wm];
            if constexpr (WM == 4) {
                const uint4 q4 = *(const uint4*)dxr;
                DX[s][0] = q4.x; DX[s][1] = q4.y; DX[s][2] = q4.z; DX[s][3] = q4.w;
            } else if constexpr (WM == 2) {
                const uint2 q2 = *(const uint2*)dxr;
                DX[s][0] = q2.x; DX[s][1] = q2.y;
            } else {
                DX[s][0] = dxr[0];
            }
        }
        if (q + 1 < nst) stage(nxt, pg0 + S * (q + 1));
#pragma unroll
        for (int s = 0; s < S; ++s) {
            if (pg0 + S * q + s >= pend) continue;      // workgroup-uniform
            // product u = (block, weight tile, activation tile); product u + 1
            // is issued before the epilogue of u, so the MFMA latency is
            // covered by that epilogue
            constexpr int NU = 4 * WM;
            auto mf = [&](int u) -> v4i {
                const int blk = u / (2 * WM), i = (u / WM) & 1, j = u % WM;
                const long av = blk ? (long)(((uint64_t)A[s][i].w << 32) | A[s][i].z)
                                    : (long)(((uint64_t)A[s][i].y << 32) | A[s][i].x);
                const long bv = blk ? (long)(((uint64_t)B[s][j].w << 32) | B[s][j].z)
                                    : (long)(((uint64_t)B[s][j].y << 32) | B[s][j].x);
                return __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bv, zero, 0, 0, 0);
            };
            // scale products dw[row 4c+v] x dx[row r] of product u as one
            // rank-1 f16 MFMA with the same lane layout as the int8 result:
            // lanes 0..15 of A and B carry this block's weight and activation
            // scales at k = blk, zeros elsewhere, so D = dw x dx + exact zeros.
            // f16 x f16 is exact in binary32 and the zeros make a -0 product
            // +0, which is fmaf(dw, dx, +0) of the canonical epilogue.
            auto sc = [&](int u) -> v4f {
                const int blk = u / (2 * WM), i = (u / WM) & 1, j = u % WM;
                // both operands keep only this block's half in lanes 0..15, so
                // every other term is 0 x 0 (an infinite or NaN scale of the
                // other block cannot leak in)
                const uint32_t hm = blk ? 0xffff0000u : 0xffffu;
                const uint32_t aw = lane < 16 ? DWR[s][i] & hm : 0u;
                const uint32_t bw = lane < 16 ? DX[s][j] & hm : 0u;
                const v4h av = __builtin_bit_cast(v4h, make_uint2(aw, 0u));
                const v4h bv = __builtin_bit_cast(v4h, make_uint2(bw, 0u));
                return __builtin_amdgcn_mfma_f32_16x16x16f16(av, bv, zerof, 0, 0, 0);
            };
            auto ep = [&](int u, const v4i& d, const v4f& sp) {
                const int i = (u / WM) & 1, j = u % WM;
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[i][j][v] = fmaf((float)d[v], sp[v], acc[i][j][v]);
            };
            v4i dcur = mf(0);
            v4f scur = sc(0);
#pragma unroll
            for (int u = 0; u < NU; ++u) {
                v4i dnext = dcur;
                v4f snext = scur;
                if (u + 1 < NU) {
                    dnext = mf(u + 1);
                    snext = sc(u + 1);
                }
                __builtin_amdgcn_sched_barrier(0);
                ep(u, dcur, scur);
                __builtin_amdgcn_sched_barrier(0);
                dcur = dnext;
                scur = snext;
            }
        }
        const int done = S * (q + 1);
        if (done % (LGX_Q8_RANGE_BLOCKS / 2) == 0 || q == nst - 1) {
            // range end: fold into the group's subtree (cnt is uniform: one
            // branch per fold)
            float* A0 = &acc[0][0][0];
            float* L0 = &l0[0][0][0];
            float* L1 = &l1[0][0][0];
            constexpr int NE = 2 * WM * 4;
            if (cnt == 0 || cnt == 2) {
#pragma unroll
                for (int e = 0; e < NE; ++e) L0[e] = A0[e];
            } else if (cnt == 1) {
#pragma unroll
                for (int e = 0; e < NE; ++e) L1[e] = L0[e] + A0[e];
            } else {
#pragma unroll
                for (int e = 0; e < NE; ++e) L1[e] = L1[e] + (L0[e] + A0[e]);
            }
#pragma unroll
            for (int e = 0; e < NE; ++e) A0[e] = 0.0f;
            ++cnt;
        }
    };

    stage(sm0, pg0);
#pragma unroll 1
    for (int q = 0; q < nst; q += 2) {
        run(q, sm0, sm1);
        if (q + 1 < nst) run(q + 1, sm1, sm0);
    }
    // the group's value of element (i, j, v)
    auto fin = [&](int i, int j, int v) {
        return cnt == 1 ? l0[i][j][v] : cnt == 3 ? l1[i][j][v] + l0[i][j][v] : l1[i][j][v];
    };
    if (swi) {
        // SwiGLU + Q8_0 (the lgx_k_swiglu_quant operations on a one-group
        // product): lane (r, c) of wave (w, wm) holds columns 32 tn + 16 w +
        // 4c .. +3 of activation row r of each tile j; the 32-block of a row
        // is its four lanes c in both waves w, whose maxima meet in LDS
        __shared__ float qm_s[2][WM][16][2];
        const int nbl = swi >> 5;
        float f[WM][4], am[WM];
#pragma unroll
        for (int j = 0; j < WM; ++j) {
#pragma unroll
            for (int v = 0; v < 4; ++v) f[j][v] = lgx_silu(fin(0, j, v)) * fin(1, j, v);
            am[j] = absmax4(f[j]);
            am[j] = fmaxf(am[j], shfl_xor_f(am[j], 16));
            am[j] = fmaxf(am[j], shfl_xor_f(am[j], 32));
            if (c == 0) qm_s[wm][j][r][wn] = am[j];
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < WM; ++j) {
            const int m = (tm0 + WM * wm + j) * 16 + r;
            uint16_t dh;
            const uint32_t qw = quantize4_am(f[j], fmaxf(qm_s[wm][j][r][0], qm_s[wm][j][r][1]), dh);
            if (m >= a.m) continue;
            *(uint32_t*)(a.sq + t16_off(m, 32 * tn + 16 * wn + 4 * c, swi)) = qw;
            if (wn == 0 && c == 0) a.sd[(int64_t)m * nbl + tn] = dh;
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int t = tn0 + 2 * wn + i;
        if (t >= ntw) continue;
        const int n0 = t * 16 + 4 * c;
#pragma unroll
        for (int j = 0; j < WM; ++j) {
            const int m = (tm0 + WM * wm + j) * 16 + r;
            if (m >= a.m) continue;
            float f[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) f[v] = fin(i, j, v);
            *(float4*)(a.part + ((int64_t)g * a.m + m) * a.n + n0) = make_float4(f[0], f[1], f[2], f[3]);
        }
    }
}

extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_gemm_tiled(const lgx_gemm_tiled_args a) {
    q8_tiled_body<4>(a, blockIdx.x);
}
extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_gemm_tiled64(const lgx_gemm_tiled_args a) {
    q8_tiled_body<2>(a, blockIdx.x);
}
extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_gemm_tiled32(const lgx_gemm_tiled_args a) {
    q8_tiled_body<1>(a, blockIdx.x);
}
extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_gemm_tiled64s4(const lgx_gemm_tiled_args a) {
    q8_tiled_body<2, 4>(a, blockIdx.x);
}
extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_gemm_tiled32s4(const lgx_gemm_tiled_args a) {
    q8_tiled_body<1, 4>(a, blockIdx.x);
}
// Grouped tiled products (lgx_tiled_group_args): each matrix's workgroups
// start at a multiple of 8, so the hardware XCD of a workgroup is its
// within-matrix id's & 7, as the XCD-aware order assumes.
template <int WM>
__device__ __forceinline__ void q8_tiled_group_body(const lgx_tiled_group_args& a) {
    const int bid = blockIdx.x;
    int g = 0;
    while (g + 1 < a.count && bid >= a.wg0[g + 1]) ++g;
    const int P = bid - a.wg0[g];
    const lgx_gemm_tiled_args& m = a.mat[g];
    if (P >= m.ntn * m.ntm * m.ngroups) return;   // padding to a multiple of 8
    q8_tiled_body<WM>(m, P);
}
extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_gemm_tiled_group(const lgx_tiled_group_args a) {
    q8_tiled_group_body<4>(a);
}
extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_gemm_tiled64_group(const lgx_tiled_group_args a) {
    q8_tiled_group_body<2>(a);
}
extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_gemm_tiled32_group(const lgx_tiled_group_args a) {
    q8_tiled_group_body<1>(a);
}

// Q8_0 of several activation matrices in one launch (lgx_quant_group_args):
// 8 lanes per 32-block, the lgx_k_quantize_q8_0 rule (quantize4).
extern "C" __global__ __launch_bounds__(256) void lgx_k_quantize_group(const lgx_quant_group_args a) {
    const int64_t blk = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 3;
    if (blk >= a.blk0[a.count]) return;           // whole 8-lane groups
    int g = 0;
    while (g + 1 < a.count && blk >= a.blk0[g + 1]) ++g;
    const int k = a.k[g], nbk = k >> 5, j = threadIdx.x & 7;
    const int64_t local = blk - a.blk0[g];
    const int64_t row = local / nbk;
    const int bl = (int)(local - row * nbk);
    const float4 v = *(const float4*)(a.x[g] + row * k + bl * 32 + 4 * j);
    const float f[4] = {v.x, v.y, v.z, v.w};
    uint16_t dh;
    const uint32_t qw = quantize4(f, dh);
    *(uint32_t*)(a.xq[g] + xq_off(row, bl * 32 + 4 * j, k, a.t16 != 0)) = qw;
    if (j == 0) a.xd[g][row * nbk + bl] = dh;
}

// Range / group trees of several products in one launch (lgx_combine_group_args).
extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_combine_group(const lgx_combine_group_args a) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= a.el0[a.count]) return;
    int g = 0;
    while (g + 1 < a.count && i >= a.el0[g + 1]) ++g;
    const int64_t cnt = a.el0[g + 1] - a.el0[g], e = i - a.el0[g];
    const float* pg = a.part[g];
    a.y[g][e] = tree_read(a.nr[g], [&](int j) { return pg[j * cnt + e]; });
}

// ---------------------------------------------------------------------------
// Causal multi-query attention of a prefill chunk.  Row r = b * qpr + j of q
// is the query at position seq_len[b] + j and attends to its first
// L = seq_len[b] + j + len_add cached tokens.  Every row runs exactly the
// decode schedule (per 256-token chunk: the score chain over d, the chunk
// max, lgx_expf, the halving-tree sum over 256 slots, the PV chain over the
// chunk's tokens; chunks merged by attn_merge), so a prefilled position has
// the bits of a decoded one.
// Workgroup: 512 threads = 8 waves for (sequence b, KV head g, block of
// PFA_QB query rows, chunk c).  The chunk's K rows, then its V rows, pass
// through one 32 KiB LDS tile in stages of PFA_TOK tokens (direct
// global->LDS loads; each row's 16-byte pieces are stored XOR-swizzled by
// the row, so row-wise and column-wise reads are conflict-free) and serve
// the PFA_QB rows x GQ heads.
//   scores:  wave (row qp = w/2, head group hg = w%2) owns heads
//            4 hg .. 4 hg + 3 over the whole chunk, lane l the tokens
//            l + 64 u; the query values come through the scalar cache
//            (uniform in the wave), 4 heads x 8 dimensions per step.
//   softmax: within the wave: per head the max, p to LDS, the halving tree
//            (levels 128 and 64 in-lane, the rest across lanes).
//   PV:      wave (row qp = w/2, head group w%2); 16-lane row rho is head
//            4 (w%2) + rho, lane k owns dims [D/16 k, +D/16); the row's p_t
//            comes from lane t%16 of a 16-token register (DPP row_newbcast).
// ---------------------------------------------------------------------------
#define PFA_QB 4
template <int D>
__device__ __forceinline__ int pfa_swz(int t) {
    return D == 128 ? (t & 15) : ((t >> 1) & 7);
}

template <int D, int GQ>
__device__ __forceinline__ void attn_prefill_body(const lgx_attn_args& a) {
    constexpr int C = LGX_ATTN_CHUNK;
    constexpr int TOK = 32768 / (2 * D);          // tokens per K/V stage
    constexpr int NST = C / TOK;
    constexpr int CPR = D / 8;                    // 16-byte pieces per row
    constexpr int NU = TOK / 128;                 // tokens per lane per stage
    __shared__ __align__(16) uint16_t kv_s[TOK * D];
    // p rows padded by 16 floats: the four heads of a wave read the same
    // token column in four distinct bank groups
    __shared__ __align__(16) float p_s[PFA_QB][GQ][C + 16];
    __shared__ int pg_s[C / LGX_PAGE];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int qpr = max(a.qpr, 1);
    const int nqb = (qpr + PFA_QB - 1) / PFA_QB;
    // XCD-aware logical id, then (sequence x KV head, chunk, query block):
    // the blocks that share a chunk's K/V run on one XCD together
    const int T = a.B * a.hkv * a.ncg * nqb;
    const int P = blockIdx.x, xcd = P & 7, slot = P >> 3;
    const int id = xcd * (T >> 3) + min(xcd, T & 7) + slot;
    const int bg = id / (a.ncg * nqb), rem = id - bg * (a.ncg * nqb);
    const int c = rem / nqb, qb = rem - c * nqb;
    const int b = bg / a.hkv, g = bg - b * a.hkv;
    const int j0 = qb * PFA_QB, t0 = c * C;
    const int sl = a.seq_len[b];
    const int jl = min(j0 + PFA_QB, qpr) - 1;              // last row of the block
    const int Lmax = min(max(sl + jl + a.len_add, 0), a.maxlen);
    if (t0 >= Lmax) return;                       // whole workgroup, before any barrier
    if (tid < C / LGX_PAGE) {
        int pg = 0;
        if (t0 + tid * LGX_PAGE < Lmax) pg = a.page_table[(int64_t)b * a.maxp + t0 / LGX_PAGE + tid];
        pg_s[tid] = min(max(pg, 0), a.num_pages - 1);
    }
    __syncthreads();

    // direct loads of stage kap (tokens [kap TOK, +TOK) of the chunk) of K
    // or V: 32 wave instructions of 1 KiB, wave w issues w, w + 8, ...
    auto stage = [&](const uint16_t* pages, int kap) {
#pragma unroll
        for (int i = 0; i < TOK * CPR / 64 / 8; ++i) {
            const int ins = wave + 8 * i;
            const int pos = ins * 64 + lane;
            const int t = pos / CPR, sp = pos - t * CPR;
            const int tok = kap * TOK + t;
            const uint16_t* src = pages +
                (((int64_t)pg_s[tok >> 4] * a.hkv + g) * LGX_PAGE + (tok & 15)) * D + (sp ^ pfa_swz<D>(t)) * 8;
            __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)(kv_s + ins * 512), 16, 0, 0);
        }
    };

    // ---- scores: wave (row qp, head group hg) owns heads 4 hg + hh (hh < 4)
    // over all C tokens of the chunk, lane l the tokens l + 64 u (u < 4) ----
    constexpr int HW = 4;                         // heads per wave
    constexpr int UPS = TOK / 64;                 // tokens per lane per stage
    const int qp = wave >> 1, hg = wave & 1;
    const int jq = j0 + qp;
    const int row = b * qpr + min(jq, qpr - 1);
    const int nq = jq < qpr ? min(C, min(max(sl + jq + a.len_add, 0), a.maxlen) - t0) : 0;
    typedef const __attribute__((address_space(4))) float* qptr_t;
    const qptr_t q0 = (qptr_t)(a.q + ((int64_t)row * a.hq + g * GQ) * D);
    int qoff[HW];                                 // heads past GQ re-read the last one
#pragma unroll
    for (int hh = 0; hh < HW; ++hh) qoff[hh] = min(4 * hg + hh, GQ - 1) * D;
    auto qh_at = [&](int hh, int i) { return q0[qoff[hh] + i]; };
    float sc[HW][4];
#pragma unroll
    for (int kap = 0; kap < NST; ++kap) {
        if (kap > 0) __syncthreads();             // the previous stage is fully read
        stage(a.kpages, kap);
        __syncthreads();                          // every wave's loads have landed
        float acc[HW][UPS];
#pragma unroll
        for (int hh = 0; hh < HW; ++hh)
#pragma unroll
            for (int v = 0; v < UPS; ++v) acc[hh][v] = 0.0f;
        // 8 dimensions per step (one 16-byte K read per token), the query
        // values in two halves of 4 x 4 scalar registers: each half is
        // requested one half-step before its products
        float qa[HW][4], qb[HW][4];
        auto qload = [&](float (&qv)[HW][4], int s4) {
#pragma unroll
            for (int hh = 0; hh < HW; ++hh)
#pragma unroll
                for (int e = 0; e < 4; ++e) qv[hh][e] = qh_at(hh, 4 * s4 + e);
        };
        auto qk_half = [&](const float (&qv)[HW][4], const float (&kf)[UPS][8], int e0) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int hh = 0; hh < HW; ++hh)
#pragma unroll
                    for (int v = 0; v < UPS; ++v)
                        acc[hh][v] = fmaf(qv[hh][e], kf[v][e0 + e], acc[hh][v]);
        };
        qload(qa, 0);
#pragma unroll 1
        for (int s8 = 0; s8 < CPR; ++s8) {
            float kf[UPS][8];
#pragma unroll
            for (int v = 0; v < UPS; ++v) {
                const int t = lane + 64 * v;
                const uint4 kv = *(const uint4*)(kv_s + t * D + (s8 ^ pfa_swz<D>(t)) * 8);
                const uint32_t w4[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    kf[v][2 * e] = h2f(w4[e] & 0xffffu);
                    kf[v][2 * e + 1] = h2f(w4[e] >> 16);
                }
            }
            qload(qb, 2 * s8 + 1);
            qk_half(qa, kf, 0);
            if (s8 + 1 < CPR) qload(qa, 2 * s8 + 2);
            qk_half(qb, kf, 4);
        }
#pragma unroll
        for (int hh = 0; hh < HW; ++hh)
#pragma unroll
            for (int v = 0; v < UPS; ++v) sc[hh][kap * UPS + v] = acc[hh][v] * a.scale;
    }
    __syncthreads();                              // K fully read: the tile takes V
    stage(a.vpages, 0);

    // ---- softmax, within the wave: max, p to LDS, halving tree (levels
    // 128 and 64 in-lane, the rest across lanes); the wave's heads advance
    // each shuffle level together ----
    {
        float mm[HW], l[HW];
#pragma unroll
        for (int hh = 0; hh < HW; ++hh) {
            mm[hh] = -__builtin_inff();
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                sc[hh][u] = lane + 64 * u < nq ? sc[hh][u] : -__builtin_inff();
                mm[hh] = fmaxf(mm[hh], sc[hh][u]);
            }
        }
#pragma unroll
        for (int hh = 0; hh < HW; ++hh) mm[hh] = wave_max(mm[hh]);
#pragma unroll
        for (int hh = 0; hh < HW; ++hh) {
            const int h = 4 * hg + hh;
            float p[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) p[u] = lane + 64 * u < nq ? lgx_expf(sc[hh][u] - mm[hh]) : 0.0f;
            if (h < GQ) {
#pragma unroll
                for (int u = 0; u < 4; ++u) p_s[qp][h][lane + 64 * u] = p[u];
            }
            l[hh] = (p[0] + p[2]) + (p[1] + p[3]);  // levels 128 and 64
        }
#pragma unroll
        for (int hh = 0; hh < HW; ++hh) l[hh] = wave_tree_sum(l[hh]);
        if (lane == 0 && nq > 0) {
#pragma unroll
            for (int hh = 0; hh < HW; ++hh) {
                const int h = 4 * hg + hh;
                if (h < GQ) {
                    float* pp = a.part + (((int64_t)row * a.hq + g * GQ + h) * a.nchunk + c) * (D + 2);
                    pp[D] = mm[hh];
                    pp[D + 1] = l[hh];
                }
            }
        }
    }

    // ---- PV ----
    constexpr int DL = D / 16;
    const int rho = lane >> 4, k = lane & 15;
    const int h = 4 * hg + rho, hc = min(h, GQ - 1);
    float o[DL];
#pragma unroll
    for (int e = 0; e < DL; ++e) o[e] = 0.0f;
    // a lane's DL halves of V row t of the stage tile (uint4: DL = 8; .xy: DL = 4)
    auto v_load = [&](int t) -> uint4 {
        const int sw = pfa_swz<D>(t);
        if constexpr (D == 128) {
            return *(const uint4*)(kv_s + t * D + (k ^ sw) * 8);
        } else {
            const uint2 vv = *(const uint2*)(kv_s + t * D + ((k >> 1) ^ sw) * 8 + (k & 1) * 4);
            return make_uint4(vv.x, vv.y, 0u, 0u);
        }
    };
    auto pv_apply = [&](const uint4 vv, float pb) {
        const uint32_t w4[4] = {vv.x, vv.y, vv.z, vv.w};
        float vf[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            vf[2 * e] = h2f(w4[e] & 0xffffu);
            vf[2 * e + 1] = h2f(w4[e] >> 16);
        }
#pragma unroll
        for (int e = 0; e < DL; ++e) o[e] = fmaf(pb, vf[e], o[e]);
    };
#pragma unroll
    for (int kap = 0; kap < NST; ++kap) {
        if (kap > 0) {
            __syncthreads();
            stage(a.vpages, kap);
        }
        __syncthreads();                          // V stage kap has landed
        const int tb = kap * TOK, te = min(nq, tb + TOK);   // uniform in the wave
        for (int ts = tb; ts < te; ts += 16) {
            // p of the 16 tokens: four 16-byte reads at one address per
            // 16-lane row (LDS broadcast)
            float pt[16];
            static_for<0, 4>([&](auto Q) {
                const float4 p4 = *(const float4*)&p_s[qp][hc][ts + 4 * Q.value];
                pt[4 * Q.value] = p4.x;
                pt[4 * Q.value + 1] = p4.y;
                pt[4 * Q.value + 2] = p4.z;
                pt[4 * Q.value + 3] = p4.w;
            });
            if (ts + 16 <= te) {
                // 8 rows' reads issued together, then their chains (twice)
                uint4 va[8];
                static_for<0, 8>([&](auto J) { va[J.value] = v_load(ts + J.value - tb); });
                static_for<0, 8>([&](auto J) { pv_apply(va[J.value], pt[J.value]); });
                static_for<0, 8>([&](auto J) { va[J.value] = v_load(ts + 8 + J.value - tb); });
                static_for<0, 8>([&](auto J) { pv_apply(va[J.value], pt[8 + J.value]); });
            } else {
                static_for<0, 16>([&](auto J) {
                    if (ts + J.value < te) pv_apply(v_load(ts + J.value - tb), pt[J.value]);
                });
            }
        }
    }
    if (h < GQ && nq > 0) {
        float* pp = a.part + (((int64_t)row * a.hq + g * GQ + h) * a.nchunk + c) * (D + 2) + DL * k;
#pragma unroll
        for (int e = 0; e < DL; e += 4) *(float4*)(pp + e) = make_float4(o[e], o[e + 1], o[e + 2], o[e + 3]);
    }
}

#define LGX_PFA_KERNELS(D, G)                                                                     \
    extern "C" __global__ __launch_bounds__(512) void lgx_k_attn_prefill_d##D##_g##G(            \
        const lgx_attn_args a) {                                                                 \
        attn_prefill_body<D, G>(a);                                                              \
    }
LGX_PFA_KERNELS(64, 1)
LGX_PFA_KERNELS(64, 2)
LGX_PFA_KERNELS(64, 3)
LGX_PFA_KERNELS(64, 4)
LGX_PFA_KERNELS(64, 5)
LGX_PFA_KERNELS(64, 6)
LGX_PFA_KERNELS(64, 7)
LGX_PFA_KERNELS(64, 8)
LGX_PFA_KERNELS(128, 1)
LGX_PFA_KERNELS(128, 2)
LGX_PFA_KERNELS(128, 3)
LGX_PFA_KERNELS(128, 4)
LGX_PFA_KERNELS(128, 5)
LGX_PFA_KERNELS(128, 6)
LGX_PFA_KERNELS(128, 7)
LGX_PFA_KERNELS(128, 8)

// ---------------------------------------------------------------------------
// Fast prefill attention (opt-in; not the canonical schedule): causal GQA
// flash attention on binary16 MFMA, within 2e-3 of the canonical attention
// (the tests check it against the oracle).  Workgroup =
// (sequence b, KV head g, FPA_Q query positions j0 ..), one wave per query
// head of the group.  Scores are formed transposed, S^T[token][query] =
// K . Q^T with v_mfma_f32_16x16x32_f16 (A: 16 K rows x 32 dimensions from
// LDS; B: the 16 query columns' dimensions in registers, scaled by
// 1/sqrt(d) before their binary16 rounding), so lane l holds tokens
// 4 (l/16) + v of query column l % 16.  The online softmax keeps the running
// maximum and sum per query column (the same in the column's four lanes;
// the sum adds the binary16-rounded weights, so constant V comes out as V);
// P^T in binary16 is then directly the B operand of the PV product
// O^T[dim][query] += V^T . P^T (v_mfma_f32_16x16x16_f16).  V stays in token
// order in LDS; its A operand (16 dimensions x 4 consecutive tokens per
// 16-lane group) comes from the transposing LDS load ds_read_b64_tr_b16:
// the 16 lanes of a group each load 4 halves of a 4 x 16 block (row j / 4,
// columns 4 (j % 4) ..) and lane n receives column n.  Tiles of FPA_T tokens
// pass through LDS once for all the group's heads; V rows past the block's
// last length are cleared (their scores are masked).  Output
// rows: binary32 to `out` and / or Q8_0 (the canonical quantisation rule) to
// xq / xd in row-major or T16 order.
// ---------------------------------------------------------------------------
#define FPA_Q 16
#define FPA_T 64
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s lds_v4s;
typedef __attribute__((address_space(3))) uint16_t lds_u16;
typedef __attribute__((address_space(3))) uint4 lds_u4;
// Tile staging: direct global->LDS loads into two buffers, the next tile's
// issued right after the barrier that publishes the current one, so its
// transfer overlaps the current tile's products.  A wave instruction moves
// 1 KiB = 64 / CH tokens of one page; lane i lands at slot i of it, and its
// source piece is chosen so that the slot holds the swizzled layout.  Rows
// past the block's last length (last tile only) are cleared in V after the
// tile lands (their scores are masked, their weights are 0, and 0 x V must
// stay 0).
template <int D>
struct FpaBuf {
    uint16_t k[FPA_T * D];                    // [token][piece ^ (token % CH)]
    uint16_t v[FPA_T * D];                    // [token][piece ^ 2 (token % (CH / 2))]
};

template <int D, int GQ>
__device__ __forceinline__ void attn_prefill_fast_body(const lgx_attn_args& a) {
    constexpr int CH = D / 8;                 // 16-byte pieces per row
    constexpr int NKS = D / 32;               // k-steps of the score product
    constexpr int NT = 64 * GQ;
    // V pieces swizzled by twice the token mod CH / 2: the four rows of one
    // transposing load (consecutive tokens) fall on different 32-byte pairs
    constexpr int VSW = CH / 2 - 1;
    constexpr int TPI = 64 / CH;              // tokens per 1 KiB wave instruction
    constexpr int NI = FPA_T / TPI;           // wave instructions per tile and tensor
    constexpr int PPT = FPA_T / LGX_PAGE;     // pages per tile
    static_assert(LGX_PAGE % TPI == 0 && PPT <= 64, "a wave instruction stays in one page");
    // two buffers as two variables: a direct load into one is known not to
    // alias reads of the other
    __shared__ __align__(16) FpaBuf<D> sb0, sb1;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int qpr = max(a.qpr, 1), nqb = (qpr + FPA_Q - 1) / FPA_Q;
    // workgroup coordinates as scalars (divisions the compiler may place in
    // vector registers; the page reads below must see a uniform address)
    const int bg = __builtin_amdgcn_readfirstlane(blockIdx.x / nqb), qb = blockIdx.x - bg * nqb;
    const int b = __builtin_amdgcn_readfirstlane(bg / a.hkv), g = bg - b * a.hkv;
    const int j0 = qb * FPA_Q;
    const int sl = a.seq_len[b];
    const int h = g * GQ + w;
    const int qc = lane & 15, kg = lane >> 4;
    const int jq = j0 + qc;
    const bool qvalid = jq < qpr;
    const int Lq = qvalid ? min(max(sl + jq + a.len_add, 0), a.maxlen) : 0;
    const int jl = min(j0 + FPA_Q, qpr) - 1;
    const int Lmax = min(max(sl + jl + a.len_add, 0), a.maxlen);   // workgroup-uniform
    const int row = b * qpr + min(jq, qpr - 1);
    const int ntile = (Lmax + FPA_T - 1) / FPA_T;
    const int32_t* ptab = a.page_table + (int64_t)b * a.maxp;
    // page table entries of tile tt as loaded, through the scalar cache (the
    // row address is uniform): they are first used by the stage after next,
    // and scalar loads do not count against the direct loads in flight;
    // stage() clamps them
    struct Pg {
        int p[PPT];
    };
    const __attribute__((address_space(4))) int32_t* ptab_s =
        (const __attribute__((address_space(4))) int32_t*)ptab;
    auto tile_pages = [&](int tt) {
        Pg r;
#pragma unroll
        for (int i = 0; i < PPT; ++i) r.p[i] = ptab_s[min(tt * PPT + i, a.maxp - 1)];
        return r;
    };
    // the buffers as LDS-space pointers
    lds_u16* const kb0 = (lds_u16*)sb0.k;
    lds_u16* const vb0 = (lds_u16*)sb0.v;
    lds_u16* const kb1 = (lds_u16*)sb1.k;
    lds_u16* const vb1 = (lds_u16*)sb1.v;
    // tile tt's loads into kb / vb (wave instruction j on wave j % GQ), pgv
    // its tile_pages (an entry at or past the length gives slot 0, read but
    // never used unmasked)
    auto stage = [&](lds_u16* kb, lds_u16* vb, int tt, const Pg& pgv) __attribute__((always_inline)) {
        // the lane's token within a wave instruction and its piece slot,
        // derived here from an opaque copy of the lane index: the per-lane
        // addresses are computed at each stage, not held in registers over
        // the tile loop
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int tl = ln / CH, cl = ln % CH;
        auto one = [&](int jj, bool isv) __attribute__((always_inline)) {
            const int t = TPI * jj + tl;
            const int ip = (TPI * jj) / LGX_PAGE;
            const int pg = (tt * PPT + ip) * LGX_PAGE < Lmax ? min(max(pgv.p[ip], 0), a.num_pages - 1) : 0;
            const int c = isv ? cl ^ ((t & VSW) << 1) : cl ^ (t & (CH - 1));
            const uint16_t* src = (isv ? a.vpages : a.kpages) +
                                  (((int64_t)pg * a.hkv + g) * LGX_PAGE + (t & 15)) * D + c * 8;
            __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)((isv ? vb : kb) + jj * 512), 16, 0, 0);
        };
#pragma unroll
        for (int j = 0; j < NI; ++j)
            if (j % GQ == w) one(j, false);       // uniform per wave
#pragma unroll
        for (int j = 0; j < NI; ++j)
            if ((NI + j) % GQ == w) one(j, true);
    };
    // scores in base-2 units: q scaled by log2(e) / sqrt(d), so the weights
    // are exp2(s - m)
    const float qscale = a.scale * 1.44269504088896341f;
    v8h qv[NKS];
    {
        const float* qr = a.q + ((int64_t)row * a.hq + h) * D;
#pragma unroll
        for (int s = 0; s < NKS; ++s) {
            const float4 x0 = *(const float4*)(qr + 32 * s + 8 * kg);
            const float4 x1 = *(const float4*)(qr + 32 * s + 8 * kg + 4);
            const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) qv[s][e] = (_Float16)(xs[e] * qscale);
        }
    }
    float m = -__builtin_inff(), l = 0.0f;
    v4f o[D / 16];
#pragma unroll
    for (int i = 0; i < D / 16; ++i) o[i] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
    // tile tt from k_s / v_s (landed), the next tile's loads into kn / vn
    // with its pages pgn; returns the pages of the tile after that
    auto run = [&](int tt, lds_u16* k_s, lds_u16* v_s, lds_u16* kn, lds_u16* vn, const Pg& pgn)
                   __attribute__((always_inline)) -> Pg {
        const int t0 = tt * FPA_T;
        __syncthreads();                          // tile tt landed (every wave waited); tile tt - 1 read
        if (t0 + FPA_T > Lmax) {                  // uniform: the last tile, rows past Lmax cleared in V
            for (int p = tid; p < FPA_T * CH; p += NT)
                if (t0 + p / CH >= Lmax) *(lds_u4*)(v_s + p * 8) = make_uint4(0u, 0u, 0u, 0u);
            __syncthreads();
        }
        Pg pgnn = pgn;
        if (tt + 1 < ntile) {
            stage(kn, vn, tt + 1, pgn);
            pgnn = tile_pages(min(tt + 2, ntile - 1));
        }
        // S^T of the tile's four 16-token sub-tiles
        v4f st[FPA_T / 16];
#pragma unroll
        for (int u = 0; u < FPA_T / 16; ++u) {
            v4f acc = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
            const int tr = 16 * u + qc;           // the K row of this lane's A operand
#pragma unroll
            for (int s = 0; s < NKS; ++s) {
                const int c = 4 * s + kg;
                const v8h kv = as_v8h(*(const lds_u4*)(k_s + tr * D + (c ^ (tr & (CH - 1))) * 8));
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kv, qv[s], acc, 0, 0, 0);
            }
            st[u] = acc;
        }
        float mt = -__builtin_inff();
#pragma unroll
        for (int u = 0; u < FPA_T / 16; ++u)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float sv = t0 + 16 * u + 4 * kg + v < Lq ? st[u][v] : -__builtin_inff();
                st[u][v] = sv;
                mt = fmaxf(mt, sv);
            }
        mt = fmaxf(mt, shfl_xor_f(mt, 16));
        mt = fmaxf(mt, shfl_xor_f(mt, 32));
        const float mn = fmaxf(m, mt);
        const bool none = mn == -__builtin_inff();          // nothing attended yet
        const float alpha = none ? 1.0f : __builtin_amdgcn_exp2f(m - mn);
        // v_exp_f32 (2^x; results below the normal range give 0): a masked
        // score (-inf) gives 0 against any finite maximum; with nothing
        // attended the reference is 0 (all weights 0)
        const float mref = none ? 0.0f : mn;
        float ps = 0.0f;
        v4h pt[FPA_T / 16];
#pragma unroll
        for (int u = 0; u < FPA_T / 16; ++u)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                pt[u][v] = (_Float16)__builtin_amdgcn_exp2f(st[u][v] - mref);
                ps += (float)pt[u][v];            // the weights the PV product uses
            }
        ps += shfl_xor_f(ps, 16);
        ps += shfl_xor_f(ps, 32);
        l = l * alpha + ps;
        m = mn;
        // o *= alpha only where some lane's alpha differs from 1 (a factor
        // of 1 changes nothing): the running maxima settle after the first
        // tiles
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
            for (int i = 0; i < D / 16; ++i) o[i] *= alpha;
        }
        // lane (qc, kg) loads token 16 u + 4 kg + qc / 4, dimensions
        // 16 i + 4 (qc % 4) .. + 3, and receives dimension 16 i + qc of the
        // tokens 16 u + 4 kg .. + 3
#pragma unroll
        for (int u = 0; u < FPA_T / 16; ++u) {
            const int tv = 16 * u + 4 * kg + (qc >> 2);
#pragma unroll
            for (int i = 0; i < D / 16; ++i) {
                const int cv = 2 * i + ((qc >> 1) & 1);
                const v4s vw = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_v4s*)(v_s + tv * D + (cv ^ ((tv & VSW) << 1)) * 8 + (qc & 1) * 4));
                o[i] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(v4h, vw), pt[u], o[i], 0, 0, 0);
            }
        }
        return pgnn;
    };
    if (ntile > 0) {
        stage(kb0, vb0, 0, tile_pages(0));
        Pg pgn = tile_pages(min(1, ntile - 1));
#pragma unroll 1
        for (int tt = 0; tt < ntile; tt += 2) {
            pgn = run(tt, kb0, vb0, kb1, vb1, pgn);
            if (tt + 1 < ntile) pgn = run(tt + 1, kb1, vb1, kb0, vb0, pgn);
        }
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
    for (int i = 0; i < D / 16; ++i) o[i] *= inv;
    if (a.out && qvalid) {
        float* orow = a.out + ((int64_t)row * a.hq + h) * D;
#pragma unroll
        for (int i = 0; i < D / 16; ++i)
            *(float4*)(orow + 16 * i + 4 * kg) = make_float4(o[i][0], o[i][1], o[i][2], o[i][3]);
    }
    if (a.out16 && qvalid) {
        uint16_t* orow = a.out16 + ((int64_t)row * a.hq + h) * D;
#pragma unroll
        for (int i = 0; i < D / 16; ++i)
            *(uint2*)(orow + 16 * i + 4 * kg) =
                make_uint2(f2h(o[i][0]) | ((uint32_t)f2h(o[i][1]) << 16),
                           f2h(o[i][2]) | ((uint32_t)f2h(o[i][3]) << 16));
    }
    if (a.xq) {
        // block j (dimensions 32 j ..) of query column qc: o[2j] and o[2j+1]
        // in the column's four lanes, 8 values each
#pragma unroll
        for (int j = 0; j < D / 32; ++j) {
            const float f0[4] = {o[2 * j][0], o[2 * j][1], o[2 * j][2], o[2 * j][3]};
            const float f1[4] = {o[2 * j + 1][0], o[2 * j + 1][1], o[2 * j + 1][2], o[2 * j + 1][3]};
            float am = fmaxf(absmax4(f0), absmax4(f1));
            am = fmaxf(am, shfl_xor_f(am, 16));
            am = fmaxf(am, shfl_xor_f(am, 32));
            uint16_t dh;
            const uint32_t q0 = quantize4_am(f0, am, dh), q1 = quantize4_am(f1, am, dh);
            if (qvalid) {
                const int col = h * D + 32 * j + 4 * kg;
                *(uint32_t*)(a.xq + xq_off(row, col, a.hq * D, a.xq_t16 != 0)) = q0;
                *(uint32_t*)(a.xq + xq_off(row, col + 16, a.hq * D, a.xq_t16 != 0)) = q1;
                if (kg == 0) a.xd[(int64_t)row * (a.hq * D / 32) + h * (D / 32) + j] = dh;
            }
        }
    }
}

#define LGX_FPA_KERNELS(D, G)                                                                     \
    extern "C" __global__ __launch_bounds__(64 * G) __attribute__((amdgpu_waves_per_eu(4)))     \
    void lgx_k_attn_prefill_fast_d##D##_g##G(const lgx_attn_args a) {                            \
        attn_prefill_fast_body<D, G>(a);                                                         \
    }
LGX_FPA_KERNELS(64, 1)
LGX_FPA_KERNELS(64, 2)
LGX_FPA_KERNELS(64, 3)
LGX_FPA_KERNELS(64, 4)
LGX_FPA_KERNELS(64, 5)
LGX_FPA_KERNELS(64, 6)
LGX_FPA_KERNELS(64, 7)
LGX_FPA_KERNELS(64, 8)
LGX_FPA_KERNELS(128, 1)
LGX_FPA_KERNELS(128, 2)
LGX_FPA_KERNELS(128, 3)
LGX_FPA_KERNELS(128, 4)
LGX_FPA_KERNELS(128, 5)
LGX_FPA_KERNELS(128, 6)
LGX_FPA_KERNELS(128, 7)
LGX_FPA_KERNELS(128, 8)
