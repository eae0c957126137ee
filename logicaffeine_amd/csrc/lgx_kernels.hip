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
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Streaming 128-bit load of weight data (read once per call: non-temporal).
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
    const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
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

// Cross-workgroup arrival for the range partials of one output slot: release
// this wave's partial stores, count the arrival; the wave that arrives last
// (whichever it is) acquires and runs the tree, so the result does not
// depend on arrival order.  The counter is reset by that wave.
__device__ __forceinline__ bool last_arrival(int32_t* counter, int slot, int nranges, int lane) {
    __threadfence();
    int old = 0;
    if (lane == 0) old = atomicAdd(counter + slot, 1);
    old = __shfl(old, 0, 64);
    if (old != nranges - 1) return false;
    __threadfence();
    return true;
}

// ---------------------------------------------------------------------------
// Shared pieces of the GEMV/GEMM kernels.
//   grid.x = groups of 4 row tiles (one wave each), grid.y = range g,
//   grid.z = m-group (GEMM only).  A range is 32 blocks = 16 T16 units.
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

// End of a GEMV wave (m = 1): one range partial per row in the c == 0 lanes.
__device__ __forceinline__ void finish_gemv(const lgx_gemv_args& a, int g, int t, int row, int c,
                                            int lane, float acc) {
    if (a.nranges == 1) {
        if (c == 0) a.y[row] = acc;
        return;
    }
    if (c == 0) a.part[(int64_t)g * a.n + row] = acc;
    if (!last_arrival(a.counter, t, a.nranges, lane)) return;
    if (c == 0) {
        float p[LGX_MAX_RANGES];
#pragma unroll
        for (int j = 0; j < LGX_MAX_RANGES; ++j)
            p[j] = j < a.nranges ? a.part[(int64_t)j * a.n + row] : 0.0f;
        a.y[row] = tree_sum(p, a.nranges);
    }
    if (lane == 0) a.counter[t] = 0;
}

// ---------------------------------------------------------------------------
// Q8 x Q8 GEMV (M = 1), v_dot4_i32_i8 + cross-lane reduction.
// Each lane holds 8 int8 of block 2p and 8 of block 2p+1 (its k-chunk c) of
// row r; the four k-chunks of a block are summed with two xor-shuffles (exact
// int32), then the range accumulator runs the canonical fmaf chain.
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void lgx_k_q8q8_gemv(const lgx_gemv_args a) {
    __shared__ __align__(16) int8_t xs[LGX_Q8_RANGE_BLOCKS * 32];
    __shared__ float dxs[LGX_Q8_RANGE_BLOCKS];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const RangeInfo ri = range_info(blockIdx.y, a.k);
    const int nb = a.k >> 5;
    {
        const int off = ri.b0 * 32 + 4 * threadIdx.x;
        int v = 0;
        if (4 * (int)threadIdx.x < ri.nbr * 32) v = *(const int*)(a.xq + off);
        *(int*)(xs + 4 * threadIdx.x) = v;
        if (threadIdx.x < LGX_Q8_RANGE_BLOCKS)
            dxs[threadIdx.x] = threadIdx.x < (unsigned)ri.nbr ? h2f(a.xd[ri.b0 + threadIdx.x]) : 0.0f;
    }
    __syncthreads();
    const int t = blockIdx.x * 4 + wave;
    if (t >= a.ntiles) return;
    const int r = lane & 15, c = lane >> 4;
    const int row = t * 16 + r;
    const int np = a.k >> 6;
    const uint4* wp = (const uint4*)a.wt + ((int64_t)t * np + ri.p0) * 64 + lane;
    const uint32_t* dwp = (const uint32_t*)(a.wd + (int64_t)row * nb + ri.b0);
    uint4 w[16];
    uint32_t dw[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        if (i < ri.npairs) {
            w[i] = ld_stream(wp + i * 64);
            dw[i] = dwp[i];
        }
    }
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        if (i < ri.npairs) {
            const int2 xa = *(const int2*)(xs + (2 * i) * 32 + 8 * c);
            const int2 xb = *(const int2*)(xs + (2 * i + 1) * 32 + 8 * c);
            int s0 = __builtin_amdgcn_sdot4((int)w[i].x, xa.x, 0, false);
            s0 = __builtin_amdgcn_sdot4((int)w[i].y, xa.y, s0, false);
            int s1 = __builtin_amdgcn_sdot4((int)w[i].z, xb.x, 0, false);
            s1 = __builtin_amdgcn_sdot4((int)w[i].w, xb.y, s1, false);
            s0 += shfl_xor_i(s0, 16);
            s1 += shfl_xor_i(s1, 16);
            s0 += shfl_xor_i(s0, 32);
            s1 += shfl_xor_i(s1, 32);
            const float d0 = h2f(dw[i] & 0xffffu) * dxs[2 * i];
            const float d1 = h2f(dw[i] >> 16) * dxs[2 * i + 1];
            acc = fmaf((float)s0, d0, acc);
            acc = fmaf((float)s1, d1, acc);
            if (a.dbg != nullptr && c == 0) {
                a.dbg[(int64_t)row * nb + ri.b0 + 2 * i] = s0;
                a.dbg[(int64_t)row * nb + ri.b0 + 2 * i + 1] = s1;
            }
        }
    }
    finish_gemv(a, ri.g, t, row, c, lane, acc);
}

// ---------------------------------------------------------------------------
// Q8 GEMV with a binary32 activation (tolerance-checked path).  Same T16
// walk; per lane an 8-term float dot per block, xor-shuffle sum of the four
// k-chunks, then acc += d_w * dot.
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_gemv_f32(const lgx_gemv_args a) {
    __shared__ __align__(16) float xs[LGX_Q8_RANGE_BLOCKS * 32];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const RangeInfo ri = range_info(blockIdx.y, a.k);
    const int nb = a.k >> 5;
    {
        const int e = 4 * threadIdx.x;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (e < ri.nbr * 32) v = *(const float4*)(a.xf + ri.b0 * 32 + e);
        *(float4*)(xs + e) = v;
    }
    __syncthreads();
    const int t = blockIdx.x * 4 + wave;
    if (t >= a.ntiles) return;
    const int r = lane & 15, c = lane >> 4;
    const int row = t * 16 + r;
    const int np = a.k >> 6;
    const uint4* wp = (const uint4*)a.wt + ((int64_t)t * np + ri.p0) * 64 + lane;
    const uint32_t* dwp = (const uint32_t*)(a.wd + (int64_t)row * nb + ri.b0);
    uint4 w[16];
    uint32_t dw[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        if (i < ri.npairs) {
            w[i] = ld_stream(wp + i * 64);
            dw[i] = dwp[i];
        }
    }
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        if (i < ri.npairs) {
            const float4* x0 = (const float4*)(xs + (2 * i) * 32 + 8 * c);
            const float4* x1 = (const float4*)(xs + (2 * i + 1) * 32 + 8 * c);
            const float4 xa = x0[0], xb = x0[1], xc = x1[0], xd = x1[1];
            const uint32_t q[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
            const float xv0[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
            const float xv1[8] = {xc.x, xc.y, xc.z, xc.w, xd.x, xd.y, xd.z, xd.w};
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float q0 = (float)(int8_t)(q[j >> 2] >> (8 * (j & 3)));
                const float q1 = (float)(int8_t)(q[2 + (j >> 2)] >> (8 * (j & 3)));
                s0 = fmaf(q0, xv0[j], s0);
                s1 = fmaf(q1, xv1[j], s1);
            }
            s0 += shfl_xor_f(s0, 16);
            s1 += shfl_xor_f(s1, 16);
            s0 += shfl_xor_f(s0, 32);
            s1 += shfl_xor_f(s1, 32);
            acc = fmaf(h2f(dw[i] & 0xffffu), s0, acc);
            acc = fmaf(h2f(dw[i] >> 16), s1, acc);
        }
    }
    finish_gemv(a, ri.g, t, row, c, lane, acc);
}

// ---------------------------------------------------------------------------
// Q8 x Q8 GEMM on int8 MFMA (v_mfma_i32_16x16x32_i8), M in m-groups of 64.
// The activation range (up to 64 rows x 32 blocks) is staged in LDS in MFMA
// A-operand order (the T16 order applied to rows of X), the per-block
// activation scales transposed to [block][row] as binary32.  Each wave owns a
// 16-row weight tile; per block one MFMA per 16-row m-tile yields exact int32
// block dots D[m][n] (lane holds m = 4c+v, n = r), and the epilogue runs the
// canonical chain acc = fmaf((float)D, dw*dx, acc).
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void lgx_k_q8_gemm_mfma(const lgx_gemv_args a) {
    __shared__ __align__(16) uint4 xa_s[4 * 16 * 64];             // [mt][pair][lane] 64 KiB
    __shared__ __align__(16) float dx_s[LGX_Q8_RANGE_BLOCKS * 64];   // [block][m]     8 KiB
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const RangeInfo ri = range_info(blockIdx.y, a.k);
    const int nb = a.k >> 5;
    const int m0 = blockIdx.z * 64;
    const int mrows = min(64, a.m - m0);
    const int mtiles = (mrows + 15) >> 4;
    // Stage X: slot (mt, pl, l) holds X[m0+16mt+r][64(p0+pl) + 8c, +8) ++ [.. +32, +8).
    for (int s = threadIdx.x; s < mtiles * 16 * 64; s += 256) {
        const int mt = s >> 10, pl = (s >> 6) & 15, l = s & 63;
        const int r = l & 15, c = l >> 4;
        const int m = m0 + mt * 16 + r;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (m < a.m && pl < ri.npairs) {
            const int8_t* src = a.xq + (int64_t)m * a.k + (ri.p0 + pl) * 64 + 8 * c;
            const uint2 lo = *(const uint2*)src;
            const uint2 hi = *(const uint2*)(src + 32);
            v = make_uint4(lo.x, lo.y, hi.x, hi.y);
        }
        xa_s[s] = v;
    }
    for (int s = threadIdx.x; s < LGX_Q8_RANGE_BLOCKS * 64; s += 256) {
        const int b = s >> 6, m = s & 63;
        float v = 0.0f;
        if (m < mrows && b < ri.nbr) v = h2f(a.xd[(int64_t)(m0 + m) * nb + ri.b0 + b]);
        dx_s[s] = v;
    }
    __syncthreads();
    const int t = blockIdx.x * 4 + wave;
    if (t >= a.ntiles) return;
    const int r = lane & 15, c = lane >> 4;
    const int col = t * 16 + r;
    const int np = a.k >> 6;
    const uint4* wp = (const uint4*)a.wt + ((int64_t)t * np + ri.p0) * 64 + lane;
    const uint32_t* dwp = (const uint32_t*)(a.wd + (int64_t)col * nb + ri.b0);
    uint4 w[16];
    uint32_t dw[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        if (i < ri.npairs) {
            w[i] = ld_stream(wp + i * 64);
            dw[i] = dwp[i];
        }
    }
    float acc[4][4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[mt][v] = 0.0f;
    const v4i zero = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        if (i < ri.npairs) {
            const float dw0 = h2f(dw[i] & 0xffffu), dw1 = h2f(dw[i] >> 16);
            const long b0 = (long)(((uint64_t)w[i].y << 32) | w[i].x);
            const long b1 = (long)(((uint64_t)w[i].w << 32) | w[i].z);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                if (mt < mtiles) {
                    const uint4 xv = xa_s[(mt * 16 + i) * 64 + lane];
                    const long a0 = (long)(((uint64_t)xv.y << 32) | xv.x);
                    const long a1 = (long)(((uint64_t)xv.w << 32) | xv.z);
                    const v4i d0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, b0, zero, 0, 0, 0);
                    const v4i d1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, b1, zero, 0, 0, 0);
                    const float4 x0 = *(const float4*)(dx_s + (2 * i) * 64 + mt * 16 + 4 * c);
                    const float4 x1 = *(const float4*)(dx_s + (2 * i + 1) * 64 + mt * 16 + 4 * c);
                    acc[mt][0] = fmaf((float)d0[0], dw0 * x0.x, acc[mt][0]);
                    acc[mt][1] = fmaf((float)d0[1], dw0 * x0.y, acc[mt][1]);
                    acc[mt][2] = fmaf((float)d0[2], dw0 * x0.z, acc[mt][2]);
                    acc[mt][3] = fmaf((float)d0[3], dw0 * x0.w, acc[mt][3]);
                    acc[mt][0] = fmaf((float)d1[0], dw1 * x1.x, acc[mt][0]);
                    acc[mt][1] = fmaf((float)d1[1], dw1 * x1.y, acc[mt][1]);
                    acc[mt][2] = fmaf((float)d1[2], dw1 * x1.z, acc[mt][2]);
                    acc[mt][3] = fmaf((float)d1[3], dw1 * x1.w, acc[mt][3]);
                }
            }
        }
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        if (mt < mtiles) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int m = m0 + mt * 16 + 4 * c + v;
                if (m < a.m) {
                    if (a.nranges == 1)
                        a.y[(int64_t)m * a.n + col] = acc[mt][v];
                    else
                        a.part[((int64_t)ri.g * a.m + m) * a.n + col] = acc[mt][v];
                }
            }
        }
    }
    if (a.nranges == 1) return;
    const int slot = t * a.nmgroups + blockIdx.z;
    if (!last_arrival(a.counter, slot, a.nranges, lane)) return;
#pragma unroll 1
    for (int o = 0; o < 16; ++o) {
        const int m = m0 + (o >> 2) * 16 + 4 * c + (o & 3);
        if ((o >> 2) < mtiles && m < a.m) {
            float p[LGX_MAX_RANGES];
#pragma unroll
            for (int j = 0; j < LGX_MAX_RANGES; ++j)
                p[j] = j < a.nranges ? a.part[((int64_t)j * a.m + m) * a.n + col] : 0.0f;
            a.y[(int64_t)m * a.n + col] = tree_sum(p, a.nranges);
        }
    }
    if (lane == 0) a.counter[slot] = 0;
}
