// kernels.hip — gfx950 kernels for the routed-expert MoE path, and their
// launchers (extern "C", declared in warp_internal.h).
//
// The expert matvec is decode-then-dot on the matrix cores: each lane reads
// the code word of 4 rows at one vector position (12 bytes, coalesced across
// the wave), gathers the 8-dim fp16 codebook vector of every stage from LDS
// and feeds it as the A operand of v_mfma_f32_16x16x32_f16, whose B operand
// holds the input split into two fp16 halves (hi, lo) per token slot. fp16 x
// fp16 products are exact in fp32, so the result is the fp32 dot product of
// the decoded weights with x to ~22 bits of x. The reference computes the
// same sum through a float LUT (src/model.c:1843-2024); the two agree within
// fp32 rounding.
//
// Built with -ffp-contract=off: every multiply-add that must be fused is an
// explicit __builtin_fmaf, every one that must not be is left as two
// operations, matching the reference's x86 build where it matters (VQ4P).

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include <type_traits>

#include "lds_limit.h"
#include "warp_internal.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u2v __attribute__((ext_vector_type(2)));
typedef unsigned u3v __attribute__((ext_vector_type(3)));

#define CHECK_LAUNCH()                                   \
    do {                                                 \
        hipError_t e_ = hipGetLastError();               \
        if (e_ != hipSuccess) return -(int)e_ - 1000;    \
    } while (0)

// ---- scalar helpers ---------------------------------------------------------

// fp16 bits -> f32 keeping subnormals (src/simd.h:49-67, exponent 31 rebiased
// as a normal number, exactly as the reference does).
__device__ __forceinline__ float f16_keep(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1f, mn = h & 0x3ff;
    if (e == 0) {
        const float f = (float)mn * 5.9604644775390625e-08f;
        return sign ? -f : f;
    }
    return __uint_as_float(sign | ((e + 112u) << 23) | (mn << 13));
}

// fp16 bits (already flushed on upload) -> f32 with the same rebiasing.
__device__ __forceinline__ float f16_flushed(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1f, mn = h & 0x3ff;
    return __uint_as_float(e ? (sign | ((e + 112u) << 23) | (mn << 13)) : sign);
}

// glibc's expf bit for bit (the reference's scores and SiLU call it):
// warp_expf, the table-and-cubic algorithm in double precision.
// A kernel that has issued a long prefetch reads the table from an LDS copy
// (etab): loads complete in issue order, so waiting for a table entry
// loaded after the prefetch would wait for all of it.
#define WARP_EXPF_QUAL __device__ __forceinline__
#include "expf_glibc.h"

__device__ const uint64_t g_exp2_tab[32] = WARP_EXP2_TAB;

__device__ __forceinline__ float expf_ref(float v, const uint64_t *etab) {
    return etab ? warp_expf_t(v, etab) : warp_expf(v);
}

__device__ __forceinline__ float silu_ref(float v, const uint64_t *etab = nullptr) {
    // src/model.c:501: v / (1 + expf(-v))
    return __fdiv_rn(v, __fadd_rn(1.0f, expf_ref(-v, etab)));
}

__device__ __forceinline__ float act_pair(float g, float u, int situ, float beta, float lbeta,
                                          const uint64_t *etab = nullptr) {
    if (!situ) return __fmul_rn(silu_ref(g, etab), u);
    // src/model.c:505-509
    const float a = __fdiv_rn(__fmul_rn(beta, tanhf(__fdiv_rn(g, beta))), __fadd_rn(1.0f, expf_ref(-g, etab)));
    return __fmul_rn(a, lbeta > 0.0f ? __fmul_rn(lbeta, tanhf(__fdiv_rn(u, lbeta))) : u);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// block-wide max of |v| over blockDim.x (a multiple of 64, <= 1024)
__device__ float block_absmax(float v) {
    __shared__ float red[16];
    v = wave_max(fabsf(v));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float m = 0.0f;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) m = fmaxf(m, red[i]);
    __syncthreads();
    return m;
}

// Scale exponent k for the split: max|x| * 2^k in [2^14, 2^15).
__device__ __forceinline__ int split_exp(float mx) {
    if (!(mx > 0.0f) || !isfinite(mx)) return 0;
    int e;
    (void)frexpf(mx, &e);
    return 15 - e;
}

__device__ __forceinline__ void split_store(float x, int k, _Float16 *hi, _Float16 *lo) {
    const float xs = ldexpf(x, k);
    const _Float16 h = (_Float16)xs;
    *hi = h;
    *lo = (_Float16)(xs - (float)h);
}

// ---- split -------------------------------------------------------------------

// One block per vector. Up to 8 values per thread stay in registers between
// the max pass and the store pass (N <= 8192 at 1024 threads).
__global__ __launch_bounds__(1024) void k_split(const float *__restrict__ x, int N,
                                                _Float16 *__restrict__ xs, float *__restrict__ xscale) {
    const int t = blockIdx.x;
    const float *xt = x + (size_t)t * N;
    _Float16 *o = xs + (size_t)t * N * 2;
    float v[8];
    float m = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int i = threadIdx.x + k * 1024;
        v[k] = i < N ? xt[i] : 0.0f;
        m = fmaxf(m, fabsf(v[k]));
    }
    for (int i = threadIdx.x + 8 * 1024; i < N; i += 1024) m = fmaxf(m, fabsf(xt[i]));
    m = block_absmax(m);
    const int e = split_exp(m);
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int i = threadIdx.x + k * 1024;
        if (i < N) split_store(v[k], e, &o[(i >> 3) * 16 + (i & 7)], &o[(i >> 3) * 16 + 8 + (i & 7)]);
    }
    for (int i = threadIdx.x + 8 * 1024; i < N; i += 1024)
        split_store(xt[i], e, &o[(i >> 3) * 16 + (i & 7)], &o[(i >> 3) * 16 + 8 + (i & 7)]);
    if (threadIdx.x == 0) xscale[t] = ldexpf(1.0f, -e);
}

// One wave per row (1 or 4 rows per block) for rows of up to 64 * NP positions of
// 8 values: the row's values stay in registers (two float4 loads per
// position, all issued first), its max |v| is a wave reduction, and each
// position's hi and lo halves leave as one 16-byte store each. ACT: the row
// is act(g, u) of two inputs (the SwiGLU of a batch), optionally also
// written to h_out. Same values as the block-per-row kernels, bit for bit
// (the same exponent from the same maximum). PGM: only the hi halves, in
// the position-group-major order of the reduced-precision products (see
// k_split_pgm), rows p < *nrows, x's row rowmap[p] when rowmap is given.
// Blocks go to the XCDs round-robin. For launches whose neighbouring blocks
// 2x and 2x + 1 read the same data (the two halves of a line, or one
// token's rows), block b of each group of 16 takes work block
// 16 (b / 16) + 2 (b % 8) + (b / 8) % 2, so that blocks b and b + 8, which
// share an XCD, take work blocks 2x and 2x + 1 and the data is fetched into
// one L2. Placement matters only for speed: each block's work is the same
// whatever XCD runs it. The blocks of a last, partial group keep their own.
__device__ __forceinline__ int xcd_pair_block(int b) {
    const int full = (int)gridDim.x & ~15;
    if (b >= full) return b;
    return (b >> 4) * 16 + (b & 7) * 2 + ((b >> 3) & 1);
}

struct PgmOut {
    const int *rowmap, *nrows;
    int R;
    const int *tok_slots;       // by pair in token order: wave q takes x row q / K to slot tok_slots[q]
    int K;
};

// The SwiGLU of the reduced-precision inputs: SiLU with the hardware exp
// (a few ulp of fp32), whose result is then rounded to fp16 (2^-11); SiTU
// keeps the exact form.
__device__ __forceinline__ float act_f16(float g, float u, int situ, float beta, float lbeta) {
    if (situ) return act_pair(g, u, situ, beta, lbeta);
    return g / (1.0f + __expf(-g)) * u;
}

template <int NP, bool ACT, bool PGM>
__global__ __launch_bounds__(256) void k_split_w(const float *__restrict__ g, const float *__restrict__ u, int P, int N,
                                                 int situ, float beta, float lbeta, half8 *__restrict__ xs,
                                                 float *__restrict__ xscale, float *__restrict__ h_out, PgmOut pm) {
    // by pair in token order, a token's neighbouring blocks on one XCD
    const int blk = PGM && pm.tok_slots ? xcd_pair_block((int)blockIdx.x) : (int)blockIdx.x;
    const int lane = threadIdx.x & 63, p = blk * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (p >= P) return;                                    // uniform per wave
    if (PGM && !pm.tok_slots && p >= *pm.nrows) return;    // uniform per wave
    const int nv = N >> 3;
    size_t src = PGM && pm.rowmap ? (size_t)pm.rowmap[p] : (size_t)p;
    int dst = p;                                           // the output row (PGM)
    if (PGM && pm.tok_slots) {
        dst = pm.tok_slots[p];
        if (dst < 0) return;                               // uniform per wave: a pair not computed
        src = (size_t)(p / pm.K);
    }
    const float4 *gp = (const float4 *)(g + src * N), *up = ACT ? (const float4 *)(u + src * N) : nullptr;
    float4 gv[NP][2], uv[NP][2] = {};
#pragma unroll
    for (int j = 0; j < NP; j++) {
        const int pos = min(lane + 64 * j, nv - 1);
        gv[j][0] = gp[2 * pos];
        gv[j][1] = gp[2 * pos + 1];
        if (ACT) {
            uv[j][0] = up[2 * pos];
            uv[j][1] = up[2 * pos + 1];
        }
    }
    float h[NP][8];
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < NP; j++) {
        const float gx[8] = {gv[j][0].x, gv[j][0].y, gv[j][0].z, gv[j][0].w, gv[j][1].x, gv[j][1].y, gv[j][1].z, gv[j][1].w};
        const float ux[8] = {uv[j][0].x, uv[j][0].y, uv[j][0].z, uv[j][0].w, uv[j][1].x, uv[j][1].y, uv[j][1].z, uv[j][1].w};
        const bool in = lane + 64 * j < nv;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            h[j][e] = ACT ? (PGM ? act_f16(gx[e], ux[e], situ, beta, lbeta) : act_pair(gx[e], ux[e], situ, beta, lbeta))
                          : gx[e];
            if (in) m = fmaxf(m, fabsf(h[j][e]));
        }
    }
    m = wave_max(m);
    const int k = split_exp(m);
    half8 *o = xs + (size_t)p * nv * 2;
#pragma unroll
    for (int j = 0; j < NP; j++) {
        const int pos = lane + 64 * j;
        if (pos < nv) {
            half8 hi, lo;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float v = ldexpf(h[j][e], k);
                hi[e] = (_Float16)v;
                lo[e] = (_Float16)(v - (float)hi[e]);
            }
            if constexpr (PGM) {
                xs[((size_t)(pos >> 2) * pm.R + dst) * 4 + (pos & 3)] = hi;
            } else {
                o[2 * pos] = hi;
                o[2 * pos + 1] = lo;
            }
            if (ACT && h_out) {
                float4 *ho = (float4 *)(h_out + (size_t)p * N) + 2 * pos;
                ho[0] = make_float4(h[j][0], h[j][1], h[j][2], h[j][3]);
                ho[1] = make_float4(h[j][4], h[j][5], h[j][6], h[j][7]);
            }
        }
    }
    if (lane == 0) xscale[PGM ? dst : p] = ldexpf(1.0f, -k);
}

template <bool ACT, bool PGM = false>
static int launch_split_w(const float *g, const float *u, int P, int N, int situ, float beta, float lbeta,
                          uint16_t *xs, float *xscale, float *h_out, void *stream, PgmOut pm = PgmOut{}) {
    const int np = (N / 8 + 63) / 64;
    const int rpb = P >= 2048 ? 4 : 1;                    // rows per block: small batches spread over more CUs
    const dim3 grid((P + rpb - 1) / rpb);
#define SPLIT_W(n)                                                                                                  \
    case n:                                                                                                         \
        hipLaunchKernelGGL((k_split_w<n, ACT, PGM>), grid, dim3(64 * rpb), 0, (hipStream_t)stream, g, u, P, N,     \
                           situ, beta, lbeta, (half8 *)xs, xscale, h_out, pm);                                      \
        break;
    switch (np) {
        SPLIT_W(1)
        SPLIT_W(2)
        SPLIT_W(3)
        SPLIT_W(4)
        SPLIT_W(5)
        SPLIT_W(6)
        SPLIT_W(7)
        SPLIT_W(8)
    default: return -1;
    }
#undef SPLIT_W
    CHECK_LAUNCH();
    return 0;
}

// fp16 hi halves of rows in position-group-major order, the B operands of a
// chunk's reduced-precision products: dims 32 pg .. 32 pg + 31 of row p at
// xs[(pg * R + p) * 32 ..], so the consecutive pair slots of a run are side
// by side in every position group. Each row is scaled by a power of two
// (max |v| * 2^k in [2^14, 2^15), 2^-k to xscale[p]) as wk_split does. ACT:
// row p is act_f16(g, u) of pair row p; otherwise row rowmap[p] of x (a chunk's
// pairs in slot order, x replicated per pair). Rows at or past *nrows are
// not written. One 256-thread block per row: a pass for the max, a pass for
// the stores (the row comes from L2 the second time).
template <bool ACT>
__global__ __launch_bounds__(256) void k_split_pgm(const float *__restrict__ g, const float *__restrict__ u,
                                                   const int *__restrict__ rowmap, const int *__restrict__ nrows,
                                                   int N, int R, int situ, float beta, float lbeta,
                                                   half8 *__restrict__ xs, float *__restrict__ xscale) {
    const int p = blockIdx.x;
    if (p >= *nrows) return;                               // uniform per block
    const size_t src = rowmap ? (size_t)rowmap[p] : (size_t)p;
    const float4 *gr = (const float4 *)(g + src * N), *ur = ACT ? (const float4 *)(u + src * N) : nullptr;
    const int nv = N >> 3;
    auto row8 = [&](int v, float (&h)[8]) {
        const float4 a0 = gr[2 * v], a1 = gr[2 * v + 1];
        const float gx[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        if constexpr (ACT) {
            const float4 b0 = ur[2 * v], b1 = ur[2 * v + 1];
            const float ux[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
            for (int e = 0; e < 8; e++) h[e] = act_f16(gx[e], ux[e], situ, beta, lbeta);
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) h[e] = gx[e];
        }
    };
    float m = 0.0f;
    for (int v = threadIdx.x; v < nv; v += blockDim.x) {
        float h[8];
        row8(v, h);
#pragma unroll
        for (int e = 0; e < 8; e++) m = fmaxf(m, fabsf(h[e]));
    }
    const int k = split_exp(block_absmax(m));
    for (int v = threadIdx.x; v < nv; v += blockDim.x) {
        float h[8];
        row8(v, h);
        half8 hi;
#pragma unroll
        for (int e = 0; e < 8; e++) hi[e] = (_Float16)ldexpf(h[e], k);
        xs[((size_t)(v >> 2) * R + p) * 4 + (v & 3)] = hi;
    }
    if (threadIdx.x == 0) xscale[p] = ldexpf(1.0f, -k);
}

extern "C" int wk_split_pgm(const float *g, const float *u, const int *rowmap, const int *nrows, int P, int N,
                            int act, int act_situ, float beta, float lbeta, uint16_t *xs, float *xscale,
                            void *stream) {
    if (P <= 0 || N <= 0 || (N % 32) || !nrows || (act && !u) || (!act && u) ||
        (((uintptr_t)g | (uintptr_t)u | (uintptr_t)xs) & 15))
        return -1;
    // rows of up to 4096 values one wave each, in registers; longer rows a block each
    if (N <= 4096)
        return act ? launch_split_w<true, true>(g, u, P, N, act_situ, beta, lbeta, xs, xscale, nullptr, stream,
                                                PgmOut{nullptr, nrows, P, nullptr, 0})
                   : launch_split_w<false, true>(g, nullptr, P, N, 0, 0.0f, 0.0f, xs, xscale, nullptr, stream,
                                                 PgmOut{rowmap, nrows, P, nullptr, 0});
    if (act)
        hipLaunchKernelGGL(k_split_pgm<true>, dim3(P), dim3(256), 0, (hipStream_t)stream, g, u, rowmap, nrows, N, P,
                           act_situ, beta, lbeta, (half8 *)xs, xscale);
    else
        hipLaunchKernelGGL(k_split_pgm<false>, dim3(P), dim3(256), 0, (hipStream_t)stream, g, u, rowmap, nrows, N, P,
                           0, 0.0f, 0.0f, (half8 *)xs, xscale);
    CHECK_LAUNCH();
    return 0;
}

extern "C" int wk_split_pgm_pairs(const float *x, const int *tok_slots, int T, int K, int N, uint16_t *xs,
                                  float *xscale, void *stream) {
    if (T <= 0 || K <= 0 || N <= 0 || N > 4096 || (N % 32) || !tok_slots || (((uintptr_t)x | (uintptr_t)xs) & 15))
        return -1;
    return launch_split_w<false, true>(x, nullptr, T * K, N, 0, 0.0f, 0.0f, xs, xscale, nullptr, stream,
                                       PgmOut{nullptr, nullptr, T * K, tok_slots, K});
}

extern "C" int wk_split(const float *x, int T, int N, uint16_t *xs, float *xscale, void *stream) {
    if (T <= 0 || N <= 0 || (N & 7)) return -1;
    // rows of up to 4096 values (and 16-byte aligned) one wave each
    if (N <= 4096 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)xs & 15) == 0)
        return launch_split_w<false>(x, nullptr, T, N, 0, 0.0f, 0.0f, xs, xscale, nullptr, stream);
    hipLaunchKernelGGL(k_split, dim3(T), dim3(1024), 0, (hipStream_t)stream, x, N, (_Float16 *)xs, xscale);
    CHECK_LAUNCH();
    return 0;
}

// ---- router logits --------------------------------------------------------------

// One 256-thread block per (token, row): up to eight float4 loads of W and x
// in flight per thread (all issued before the first multiply-add), lane
// partials in ascending index order, then a fixed-order block sum
// (deterministic). Returned in thread 0.
template <int UNR = 8>
__device__ __forceinline__ float router_row_fast(const float *__restrict__ W, const float *__restrict__ x, int E,
                                                 int H, int row) {
    __shared__ float part[4];
    const int t = row / E, e = row % E;
    const float *w = W + (size_t)e * H, *xt = x + (size_t)t * H;
    float acc = 0.0f;
    if ((H & 3) == 0) {
        const float4 *w4 = (const float4 *)w, *x4 = (const float4 *)xt;
        const int n4 = H >> 2;
        for (int i0 = threadIdx.x; i0 < n4; i0 += UNR * 256) {
            float4 a[UNR], b[UNR];
#pragma unroll
            for (int k = 0; k < UNR; k++) {
                const int i = min(i0 + k * 256, n4 - 1);
                a[k] = w4[i];
                b[k] = x4[i];
            }
#pragma unroll
            for (int k = 0; k < UNR; k++) {
                if (i0 + k * 256 < n4) {
                    acc = __builtin_fmaf(a[k].x, b[k].x, acc);
                    acc = __builtin_fmaf(a[k].y, b[k].y, acc);
                    acc = __builtin_fmaf(a[k].z, b[k].z, acc);
                    acc = __builtin_fmaf(a[k].w, b[k].w, acc);
                }
            }
        }
    } else {
        for (int i = threadIdx.x; i < H; i += 256) acc = __builtin_fmaf(w[i], xt[i], acc);
    }
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    return (part[0] + part[1]) + (part[2] + part[3]);
}

__global__ __launch_bounds__(256) void k_router_fast(const float *__restrict__ W, const float *__restrict__ x,
                                                     int E, int H, int T, float *__restrict__ logits) {
    const float v = router_row_fast(W, x, E, H, blockIdx.x);
    if (threadIdx.x == 0) logits[blockIdx.x] = v;
}

// One token: row e's logit, then its sigmoid score and biased score with the
// same operations as the routing's scoring pass (route_pick_lds).
__global__ __launch_bounds__(256) void k_router_scored(const float *__restrict__ W, const float *__restrict__ x,
                                                       int E, int H, const float *__restrict__ bias,
                                                       float *__restrict__ out) {
    const int e = blockIdx.x;
    const float v = router_row_fast(W, x, E, H, e);
    if (threadIdx.x == 0) {
        const float sc = __fdiv_rn(1.0f, __fadd_rn(1.0f, warp_expf(-v)));
        out[e] = sc;
        out[E + e] = __fadd_rn(sc, bias ? bias[e] : 0.0f);
    }
}

// Coherent accesses, for what one block of the fused decode launch writes
// for another, which may run on another XCD (another L2): agent-scope
// atomic stores and loads (relaxed), which the memory model lowers to
// accesses that bypass a stale or write-back copy in the XCD's L2 (sc1), so
// the values reach, and are read from, memory every XCD sees. Nothing here
// rests on how a plain or volatile access is lowered. A wave's stores are
// complete once wait_stores() returns, so with a barrier after it the block
// can raise a count that others poll, without writing back the L2 (which an
// agent-scope release fence does, at a cost that grows with everything the
// XCD's other blocks have written).
__device__ __forceinline__ void st_through4(float *p, float a, float b, float c, float d) {   // p in global memory
    __hip_atomic_store(p + 0, a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(p + 1, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(p + 2, c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(p + 3, d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(float *p, float a) {
    __hip_atomic_store(p, a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0x0F70); }   // vmcnt(0)

// ---- certified routing (decode, sigmoid scores, fp32 router) ---------------------------
//
// The reference's router logit is a sequential, unfused fp32 sum
// (dotf, src/model.c:155-160): s_k = fl(s_{k-1} + fl(w_k x_k)). Its rounding
// errors are bounded by u (sum_k |s_k| + sum_k |w_k x_k|), u = 2^-24. A
// certified row computes the exact sum S* (the fp32 products are exact in
// double, summed in double), the running sums' magnitudes from a prefix
// scan, and that bound B; the reference's logit lies in [S* - B, S* + B].
// The routing ranks the point scores of fp32(S*) and keeps, for each
// expert, the interval its biased score can take (the score function and
// the bias addition are monotone; one ulp is added each way). Where the
// interval of a pick overlaps one ranked after it, the order is not certain
// from the bounds alone: those rows' logits are recomputed with the
// reference's own sequential sum (route_certify) and the picks made again.
// The picks and their order are then the reference's by construction.
constexpr double CERT_U = 5.9604644775390625e-08;         // 2^-24
constexpr int CERT_MAXV = 16;                               // float4 per thread: H <= 16384
constexpr int CERT_EMAX = 4096;                             // experts the certification takes

// The neighbouring floats toward -inf and +inf (NaN and the infinity on that
// side unchanged).
__device__ __forceinline__ float f_down(float v) {
    if (v != v || v == -INFINITY) return v;
    if (v == 0.0f) return -__uint_as_float(1u);
    const uint32_t u = __float_as_uint(v);
    return __uint_as_float(v > 0.0f ? u - 1u : u + 1u);
}
__device__ __forceinline__ float f_up(float v) { return -f_down(-v); }

__device__ __forceinline__ float cert_score(float l, const uint64_t *etab = nullptr) {
    return __fdiv_rn(1.0f, __fadd_rn(1.0f, expf_ref(-l, etab)));
}

// A row's four values for the certifying block, each with this launch's tag
// in the same 64-bit store (tg = NULL: none): the block sees a value and its
// tag together or not at all, so it needs no separate ready word.
struct CertTag {
    unsigned long long *tg;     // [E][4]: point score, biased score, lower, upper bound
    unsigned tag;
};
__device__ __forceinline__ void st_tag(const CertTag &ct, int e, int i, float v) {
    if (ct.tg)
        __hip_atomic_store(ct.tg + 4 * (size_t)e + i, ((unsigned long long)ct.tag << 32) | __float_as_uint(v),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// the four values of row e: the store to out and the tagged one
__device__ __forceinline__ void cert_put(float *out, int E, int e, int i, float v, const CertTag &ct) {
    st_agent(out + (size_t)i * E + e, v);
    st_tag(ct, e, i, v);
}

// Row e's outputs from its exact sum S, the sum of its running sums'
// magnitudes (as) and of its products' magnitudes (ap): the reference's
// rounding errors are bounded by u (as + ap) up to terms of relative size
// n u (its running sums are within that bound of these), plus this code's
// own double arithmetic; products that underflow in fp32 are off by at most
// 2^-149 each. The logit interval is widened to floats outward, and the
// biased-score bounds by one more ulp each way for the score and the sum.
__device__ __forceinline__ void cert_finish(double S, double as, double ap, int H, int E, int e,
                                            const float *__restrict__ bias, float *__restrict__ out,
                                            const CertTag &ct) {
    const double n = (double)H;
    const double B = CERT_U * (as + 1.01 * ap) * (1.0 + 4.0 * n * CERT_U) + 1e-12 * (as + ap) + n * 1.4e-45;
    const float l = (float)S;
    const float lo = f_down((float)(S - B)), hi = f_up((float)(S + B));
    const float bv = bias ? bias[e] : 0.0f;
    const float sc = cert_score(l);
    cert_put(out, E, e, 0, sc, ct);
    cert_put(out, E, e, 1, __fadd_rn(sc, bv), ct);
    const bool ok = isfinite(S) && isfinite(B) && isfinite(lo) && isfinite(hi);
    cert_put(out, E, e, 2, ok ? f_down(__fadd_rn(f_down(cert_score(lo)), bv)) : -INFINITY, ct);
    cert_put(out, E, e, 3, ok ? f_up(__fadd_rn(f_up(cert_score(hi)), bv)) : INFINITY, ct);
}

// The same by three lanes (lane 0 the point score, 1 the lower bound, 2 the
// upper bound), from S and upper bounds as, ap of the sums of magnitudes.
__device__ __forceinline__ void cert_finish3(double S, double as, double ap, int H, int E, int e, int lane,
                                             const float *__restrict__ bias, float *__restrict__ out,
                                             const CertTag &ct) {
    const double n = (double)H;
    const double B = CERT_U * (as + ap) * (1.0 + 4.0 * n * CERT_U) + 1e-12 * (as + ap) + n * 1.4e-45;
    const float lo = f_down((float)(S - B)), hi = f_up((float)(S + B));
    const bool ok = isfinite(S) && isfinite(B) && isfinite(lo) && isfinite(hi);
    const float l = lane == 0 ? (float)S : !ok ? 0.0f : lane == 1 ? lo : hi;
    const float sc = cert_score(l);
    const float bv = bias ? bias[e] : 0.0f;
    if (lane == 0) {
        cert_put(out, E, e, 0, sc, ct);
        cert_put(out, E, e, 1, __fadd_rn(sc, bv), ct);
    } else if (lane == 1) {
        cert_put(out, E, e, 2, ok ? f_down(__fadd_rn(f_down(sc), bv)) : -INFINITY, ct);
    } else {
        cert_put(out, E, e, 3, ok ? f_up(__fadd_rn(f_up(sc), bv)) : INFINITY, ct);
    }
}

// The same by one lane, without the reference's expf, for |S| + B < 30:
// sigma(S) in double from the hardware exponential (relative error at most
// (|S| + 2) 2^-20 for it, with the rounding of S to float), the biased
// score's bounds from sigma' = sigma (1 - sigma) at S and |sigma''| <= 0.1
// over the logit interval: sigma(S +- B) lies within sigma(S) +- (sigma' B +
// 0.05 B^2). The reference's score is sigma of its logit to within a
// relative 2^-22 (its expf, the add and the division, each under an ulp).
// The point score is sigma(S) rounded to float: within the bounds, and
// within a few ulps of the reference's operations on fp32(S).
__device__ __forceinline__ bool cert_finish1(double S, double B, int E, int e, const float *__restrict__ bias,
                                             float *__restrict__ out, const CertTag &ct) {
    if (!(fabs(S) + B < 30.0)) return false;
    const float ef = __expf(-(float)S);
    const double sg = 1.0 / (1.0 + (double)ef);
    const double d1 = sg * (1.0 - sg);
    const double r = (fabs(S) + 2.0) * 0x1p-20 + fabs(S) * 0x1p-23;
    const double err = d1 * r * 1.01 + d1 * B + 0.05 * B * B + (sg + d1 * B) * 0x1p-22 + 1e-300;
    const float bv = bias ? bias[e] : 0.0f;
    const float sc = (float)sg;
    cert_put(out, E, e, 0, sc, ct);
    cert_put(out, E, e, 1, __fadd_rn(sc, bv), ct);
    cert_put(out, E, e, 2, f_down(__fadd_rn(f_down((float)(sg - err)), bv)), ct);
    cert_put(out, E, e, 3, f_up(__fadd_rn(f_up((float)(sg + err)), bv)), ct);
    return true;
}

// out: [0, E) point score, [E, 2E) point biased score, [2E, 3E) the biased
// score's lower bound, [3E, 4E) its upper bound. One 256-thread block per
// row; each thread a contiguous run of the row. H % 4 == 0.
__device__ __forceinline__ void router_row_cert(const float *__restrict__ W, const float *__restrict__ x, int E,
                                                int H, int e, const float *__restrict__ bias, float *__restrict__ out,
                                                const CertTag &ct) {
    __shared__ double r_sum[4], r_abs_s[4];
    __shared__ double r_scan[4];
    __shared__ float r_abs_p[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n4 = H >> 2, per = (n4 + 255) / 256;
    const float4 *w4 = (const float4 *)(W + (size_t)e * H), *x4 = (const float4 *)x;
    float4 a[CERT_MAXV], b[CERT_MAXV];
#pragma unroll
    for (int v = 0; v < CERT_MAXV; v++) {
        const int i = min(tid * per + v, n4 - 1);
        if (v < per) {
            a[v] = w4[i];
            b[v] = x4[i];
        }
    }
    // this thread's run: its exact sum and the magnitudes of its products
    double loc = 0.0;
    float absp = 0.0f;
#pragma unroll
    for (int v = 0; v < CERT_MAXV; v++) {
        if (v < per && tid * per + v < n4) {
            const double p0 = (double)a[v].x * b[v].x, p1 = (double)a[v].y * b[v].y;
            const double p2 = (double)a[v].z * b[v].z, p3 = (double)a[v].w * b[v].w;
            loc += p0; loc += p1; loc += p2; loc += p3;
            absp += fabsf((float)p0) + fabsf((float)p1) + fabsf((float)p2) + fabsf((float)p3);
        }
    }
    // exclusive scan of the runs' sums over the block, in thread order
    double inc = loc;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const double t = __shfl_up(inc, o);
        if (lane >= o) inc += t;
    }
    if (lane == 63) r_scan[wave] = inc;
    __syncthreads();
    double off = inc - loc;
    for (int w = 0; w < wave; w++) off += r_scan[w];
    // sum of the running sums' magnitudes over this run
    double abss = 0.0, s = off;
#pragma unroll
    for (int v = 0; v < CERT_MAXV; v++) {
        if (v < per && tid * per + v < n4) {
            s += (double)a[v].x * b[v].x; abss += fabs(s);
            s += (double)a[v].y * b[v].y; abss += fabs(s);
            s += (double)a[v].z * b[v].z; abss += fabs(s);
            s += (double)a[v].w * b[v].w; abss += fabs(s);
        }
    }
    // block totals (fixed order)
    double tot = loc, ta = abss;
    float tp = absp;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        tot += __shfl_xor(tot, o);
        ta += __shfl_xor(ta, o);
        tp += __shfl_xor(tp, o);
    }
    if (lane == 0) {
        r_sum[wave] = tot;
        r_abs_s[wave] = ta;
        r_abs_p[wave] = tp;
    }
    __syncthreads();
    if (tid == 0) {
        const double S = (r_sum[0] + r_sum[1]) + (r_sum[2] + r_sum[3]);
        const double as = (r_abs_s[0] + r_abs_s[1]) + (r_abs_s[2] + r_abs_s[3]);
        const double ap = ((double)r_abs_p[0] + r_abs_p[1]) + ((double)r_abs_p[2] + r_abs_p[3]);
        cert_finish(S, as, ap, H, E, e, bias, out, ct);
    }
}

// The certification of the selection, by the router's last block
// (cert_last): sync (or NULL: the arrays only; 8-byte aligned) is the launch
// counter (word 0; word 1 pads), then [E][4] 64-bit tagged values (CertTag): a row's blocks tag its
// values with the counter plus one, the certifying block takes a row once
// its four tags are, and then advances the counter (a row a later launch
// writes can never look done to this one, and a late row of this one never
// to the next). K picks, cctr the counters (or NULL), flag the route's
// missing flag.
struct CertTail {
    unsigned *sync;
    int K;
    unsigned long long *cctr;
    int *flag;                  // a wait past the poll limit sets bit 2 (value 4)
    warp_route_args pk;         // pk.idx set: the routing's outputs (idx, w; with pk.table the job lists)
    unsigned polls;             // the poll limit (0: CERT_POLLS)
};
constexpr unsigned CERT_POLLS = 1u << 16;   // polls of the rows' values before the last block gives up

// This launch's tag for the rows' values (the block's threads all read it).
__device__ __forceinline__ CertTag cert_tag(const CertTail &t) {
    CertTag ct = {nullptr, 0u};
    if (t.sync) {
        ct.tg = (unsigned long long *)(t.sync + 2);
        ct.tag = __hip_atomic_load(t.sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    }
    return ct;
}
template <int NT>
__device__ void cert_last(const float *__restrict__ W, const float *__restrict__ x, int E, int H,
                          const float *__restrict__ bias, float *__restrict__ out, const CertTail &t, float *lds,
                          int lds_floats);

__global__ __launch_bounds__(256) void k_router_cert(const float *__restrict__ W, const float *__restrict__ x, int E,
                                                     int H, const float *__restrict__ bias, float *__restrict__ out,
                                                     CertTail t, int lds_floats) {
    extern __shared__ __attribute__((aligned(16))) float rcg_lds[];
    if ((int)blockIdx.x < E) {
        router_row_cert(W, x, E, H, blockIdx.x, bias, out, cert_tag(t));
        return;
    }
    cert_last<256>(W, x, E, H, bias, out, t, rcg_lds, lds_floats);   // block E, with t.sync only
}

// The same arrays, faster: one 256-thread block per row, W's row and x
// staged in LDS by coalesced loads, T = H / (4 R4) threads taking one
// contiguous run of R = 4 R4 columns each (runs padded in LDS so that the
// lanes' 16-byte reads fall on distinct banks). The centre is the exact sum
// of the fp32 products p = fl(w x) -- the reference's own summands -- by
// TwoSum within a run, then in double; the reference's sequential sum s_n of
// them is within u sum_k |S_k| (1 + 2 n u) of it, S_k the exact prefix sums,
// with no term for the products (the same rounded products on both sides).
// sum_k |S_k| is taken from fp32 running sums from each run's offset: each
// is off by at most 2 (R + 2) u sum|p| (the offset rounded once, then R
// roundings of sums of magnitude at most 2 sum|p|), and the fp32 sums of
// magnitudes by a relative (R + 10) u (the run, the wave's six levels, the
// four waves).
template <int R4>
__global__ __launch_bounds__(256) void k_router_cert_b(const float *__restrict__ W, const float *__restrict__ x,
                                                       int E, int H, const float *__restrict__ bias,
                                                       float *__restrict__ out, CertTail t, int lds_floats) {
    constexpr int R = 4 * R4, S4 = R4 + ((R4 & 1) ? 2 : 1);     // run stride: an odd number of float4
    extern __shared__ __attribute__((aligned(16))) float4 rc_lds[];
    __shared__ double rc_wt[4];
    __shared__ float rc_as[4], rc_ap[4];
    if ((int)blockIdx.x == E) {                            // uniform: the certifying block
        cert_last<256>(W, x, E, H, bias, out, t, (float *)rc_lds, lds_floats);
        return;
    }
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n4 = H >> 2, T = n4 / R4, e = blockIdx.x;
    float4 *wl = rc_lds, *xl = rc_lds + 256 * S4;
    const float4 *w4 = (const float4 *)(W + (size_t)e * H), *x4 = (const float4 *)x;
    float4 ws[R4], xs[R4];
#pragma unroll
    for (int v = 0; v < R4; v++) {
        const int i = min(tid + 256 * v, n4 - 1);
        ws[v] = w4[i];
        xs[v] = x4[i];
    }
#pragma unroll
    for (int v = 0; v < R4; v++) {
        const int i = tid + 256 * v;
        if (i < n4) {
            const int r = i / R4, j = i - r * R4;
            wl[r * S4 + j] = ws[v];
            xl[r * S4 + j] = xs[v];
        }
    }
    __syncthreads();
    const bool act = tid < T;
    float p[R], hi = 0.0f, lo = 0.0f, absp = 0.0f;
#pragma unroll
    for (int v = 0; v < R4; v++) {
        const float4 a = act ? wl[tid * S4 + v] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const float4 b = act ? xl[tid * S4 + v] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        p[4 * v] = __fmul_rn(a.x, b.x);
        p[4 * v + 1] = __fmul_rn(a.y, b.y);
        p[4 * v + 2] = __fmul_rn(a.z, b.z);
        p[4 * v + 3] = __fmul_rn(a.w, b.w);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float q = p[4 * v + c];
            const float t = __fadd_rn(hi, q), z = __fsub_rn(t, hi);      // TwoSum: hi + q = t + err exactly
            lo = __fadd_rn(lo, __fadd_rn(__fsub_rn(hi, __fsub_rn(t, z)), __fsub_rn(q, z)));
            hi = t;
            absp = __fadd_rn(absp, fabsf(q));
        }
    }
    // the runs' exclusive prefix over the block (thread order = index order)
    const double run = (double)hi + (double)lo;
    double inc = run;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const double t = __shfl_up(inc, o);
        if (lane >= o) inc += t;
    }
    if (lane == 63) rc_wt[wave] = inc;
    __syncthreads();
    double off = inc - run;
    for (int w = 0; w < wave; w++) off += rc_wt[w];
    float sr = (float)off, abss = 0.0f;
#pragma unroll
    for (int k = 0; k < R; k++) {
        sr = __fadd_rn(sr, p[k]);
        abss = __fadd_rn(abss, fabsf(sr));
    }
    if (!act) abss = 0.0f;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        abss = __fadd_rn(abss, __shfl_xor(abss, o));
        absp = __fadd_rn(absp, __shfl_xor(absp, o));
    }
    if (lane == 0) {
        rc_as[wave] = abss;
        rc_ap[wave] = absp;
    }
    __syncthreads();
    const double S = (rc_wt[0] + rc_wt[1]) + (rc_wt[2] + rc_wt[3]);
    const double g = 1.0 + 2.0 * (R + 10.0) * CERT_U, n = (double)H;
    const double ap = ((double)(rc_ap[0] + rc_ap[1]) + (double)(rc_ap[2] + rc_ap[3])) * g;
    const double dsr = 2.0 * (R + 2.0) * CERT_U * ap;     // the running sums' own error, each
    const double as = ((double)(rc_as[0] + rc_as[1]) + (double)(rc_as[2] + rc_as[3])) * g + n * dsr;
    const double B1 = CERT_U * as * (1.0 + 4.0 * n * CERT_U) + 1e-12 * as + n * 1.4e-45;
    // A tighter bound from the same running sums: the reference's step k
    // rounds a sum t_k with |t_k| <= |sr_k| + dsr + B1 (B1 bounds every
    // earlier partial sum's error too), so its error is at most half an ulp
    // of t_k's binade, 2^(e - 24) for |t_k| in [2^e, 2^(e+1)) -- about 0.7
    // of u |t_k| on average. The binade of fl(|sr_k| + dB) is at least that
    // of |t_k| (rounding to nearest never leaves a binade downward).
    const float dB = (float)((dsr + B1) * (1.0 + 0x1p-20));
    float sr2 = (float)off, hus = 0.0f;
#pragma unroll
    for (int k = 0; k < R; k++) {
        sr2 = __fadd_rn(sr2, p[k]);
        const float y = __fadd_rn(fabsf(sr2), dB);
        const int ex = (__float_as_int(y) >> 23) & 0xff;
        hus = __fadd_rn(hus, ex >= 25 ? __int_as_float((ex - 24) << 23) : 0x1p-126f);   // (below 2^-102: 2^-126)
    }
    if (!act) hus = 0.0f;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) hus = __fadd_rn(hus, __shfl_xor(hus, o));
    if (lane == 0) rc_as[wave] = hus;
    __syncthreads();
    if (tid < 64) {                                       // wave 0 (uniform values)
        const double hsum = ((double)(rc_as[0] + rc_as[1]) + (double)(rc_as[2] + rc_as[3])) * g;
        const double B = fmin(B1, hsum * (1.0 + 4.0 * n * CERT_U) + 1e-12 * as + n * 1.4e-45);
        const CertTag ct = cert_tag(t);
        if (!(fabs(S) + B < 30.0)) {                       // uniform
            if (tid < 3) cert_finish3(S, B / (CERT_U * (1.0 + 4.0 * n * CERT_U) + 1e-12), 0.0, H, E, e, tid,
                                      bias, out, ct);
        } else if (tid == 0) {
            cert_finish1(S, B, E, e, bias, out, ct);
        }
    }
}

// Launches k_router_cert_b<R4> when H / (4 R4) threads of the block make
// whole waves (the callers try the shortest runs first).
// LDS floats of cert_last: the four arrays, the expert table (when it
// writes the job lists), the recompute's row and segments.
static_assert(sizeof(warp_slot) == 24, "warp_slot: six floats of LDS");
static size_t cert_last_floats(int E, int H, bool table) {
    return (size_t)((4 * ((E + 1) & ~1) + 3) & ~3) + (table ? (size_t)6 * ((E + 1) & ~1) : 0) + (size_t)H + 128 * 4 +
           64;
}

template <int R4>
static bool router_cert_b(const float *W, const float *x, int E, int H, const float *bias, float *out,
                          const CertTail &t, hipStream_t s) {
    const int n4 = H >> 2;
    if ((H & 3) || n4 % R4 || n4 / R4 > 256 || (n4 / R4) % 64) return false;
    const size_t lds = std::max((size_t)2 * 256 * (R4 + ((R4 & 1) ? 2 : 1)) * sizeof(float4),
                                t.sync ? cert_last_floats(E, H, t.pk.table) * sizeof(float) : (size_t)0);
    if (lds > 160 * 1024) return false;
    static std::atomic<uint64_t> attr{0};
    if (lds_limit((const void *)k_router_cert_b<R4>, (int)lds, attr, s)) return false;
    hipLaunchKernelGGL(k_router_cert_b<R4>, dim3(E + (t.sync ? 1 : 0)), dim3(256), lds, s, W, x, E, H, bias, out,
                       t, (int)(lds / sizeof(float)));
    return true;
}

extern "C" int wk_router_cert(const float *W, const float *x, int E, int H, const float *bias, float *out,
                              unsigned *sync, int K, unsigned long long *cctr, int *flag,
                              const warp_route_args *pick, unsigned polls, void *stream) {
    if (E <= 0 || H <= 0 || (H & 3) || H > 1024 * CERT_MAXV) return -1;
    if (sync && (K <= 0 || K > WARP_MAX_K || K > E || E > CERT_EMAX || ((uintptr_t)sync & 7))) return -1;
    if (pick && (!sync || !pick->idx || !pick->w || (pick->table && (!pick->jobs || !pick->njobs || !flag))))
        return -1;
    CertTail t = {sync, K, cctr, flag, {}, polls};
    if (pick) t.pk = *pick;
    // hidden sizes of the reference's models (Kimi-Linear 2304, K3 7168) and
    // their neighbours take the staged kernel
    const hipStream_t st = (hipStream_t)stream;
    if (!(router_cert_b<3>(W, x, E, H, bias, out, t, st) || router_cert_b<4>(W, x, E, H, bias, out, t, st) ||
          router_cert_b<5>(W, x, E, H, bias, out, t, st) || router_cert_b<6>(W, x, E, H, bias, out, t, st) ||
          router_cert_b<7>(W, x, E, H, bias, out, t, st) || router_cert_b<8>(W, x, E, H, bias, out, t, st))) {
        const size_t lds = sync ? cert_last_floats(E, H, t.pk.table) * sizeof(float) : 0;
        if (lds > 160 * 1024) return -1;
        static std::atomic<uint64_t> attr{0};
        if (int r_ = lds_limit((const void *)k_router_cert, (int)lds, attr, stream)) return r_;
        hipLaunchKernelGGL(k_router_cert, dim3(E + (sync ? 1 : 0)), dim3(256), lds, st, W, x, E, H, bias, out, t,
                           (int)(lds / sizeof(float)));
    }
    CHECK_LAUNCH();
    return 0;
}

extern "C" int wk_router_scored(const float *W, const float *x, int E, int H, const float *bias, float *out,
                                void *stream) {
    if (E <= 0 || H <= 0) return -1;
    hipLaunchKernelGGL(k_router_scored, dim3(E), dim3(256), 0, (hipStream_t)stream, W, x, E, H, bias, out);
    CHECK_LAUNCH();
    return 0;
}

// A batch of tokens on the matrix cores: logits[t][e] = X[t] . W[e] with
// v_mfma_f32_16x16x4_f32 (fp32 products, fp32 sums). A block of 4 waves owns
// 16 tokens x 16 experts; wave w sums the w-th quarter of H's 16-column
// chunks. Per chunk a lane loads one float4 of its token row and one of its
// expert row (columns 4j..4j+3 of the 16, j = lane / 16) and feeds their
// components to 4 MFMA steps: step s sums column 4j + s, the same column on
// both sides. The quarters meet in LDS and are added in wave order, so each
// logit is a fixed sequence of sums whatever the token's place in the
// batch. Loads run 7 chunks ahead of the multiplies. H is a multiple of 16.
__global__ __launch_bounds__(256) void k_router_mfma(const float *__restrict__ W, const float *__restrict__ x, int E,
                                                     int H, int T, float *__restrict__ logits) {
    __shared__ float red[4][16][16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t0 = blockIdx.x * 16, e0 = blockIdx.y * 16;
    const int r = lane & 15, j = lane >> 4;
    const float4 *xa = (const float4 *)(x + (size_t)min(t0 + r, T - 1) * H) + j;
    const float4 *wb = (const float4 *)(W + (size_t)min(e0 + r, E - 1) * H) + j;
    const int nc = H >> 4, c_lo = wave * nc / 4, c_hi = (wave + 1) * nc / 4;
    constexpr int RING = 8;                                 // 16-column chunks in flight: RING - 1 ahead
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    float4 a[RING], b[RING];
#pragma unroll
    for (int u = 0; u < RING - 1; u++) {
        const int c = min(c_lo + u, nc - 1);
        a[u] = xa[(size_t)c * 4];
        b[u] = wb[(size_t)c * 4];
    }
    for (int c0 = c_lo; c0 < c_hi; c0 += RING) {
#pragma unroll
        for (int u = 0; u < RING; u++) {
            const int c = c0 + u;
            if (c < c_hi) {                                 // uniform
                const int cl = min(c + RING - 1, nc - 1);
                a[(u + RING - 1) % RING] = xa[(size_t)cl * 4];
                b[(u + RING - 1) % RING] = wb[(size_t)cl * 4];
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].x, b[u].x, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].y, b[u].y, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].z, b[u].z, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].w, b[u].w, acc, 0, 0, 0);
            }
        }
    }
    // lane (r, j) holds rows 4j..4j+3 (tokens) of column r (expert)
#pragma unroll
    for (int q = 0; q < 4; q++) red[wave][4 * j + q][r] = acc[q];
    __syncthreads();
    const int tt = threadIdx.x >> 4, ee = threadIdx.x & 15, t = t0 + tt, e = e0 + ee;
    if (t < T && e < E) logits[(size_t)t * E + e] = ((red[0][tt][ee] + red[1][tt][ee]) + red[2][tt][ee]) + red[3][tt][ee];
}

// The reference's dotf on x86 (src/model.c:155-160): one sequential, unfused
// sum per row, bit for bit.
// Strict logits: each (token, expert) row summed in index order, w[i] * x[i]
// rounded and then added (unfused), as the reference's loop does, bit for
// bit. A row's adds form one dependent chain; the rows' chains are
// independent, so a wave runs 16 rows side by side, one per lane: 64
// columns at a time, all 64 lanes form the tile's products from coalesced
// 16-byte loads into LDS (rows 68 floats apart: the 16 lanes' 16-byte reads
// hit distinct banks), the loads of the next RS_D steps in flight (a step's
// adds take far less than a load's latency), and each of lanes 0-15 adds
// its row's 64 products in order, four per LDS read.
constexpr int RS_R = 16;                   // rows per wave
constexpr int RS_C = 64;                   // columns per step
constexpr int RS_P = RS_C + 4;             // LDS row pitch (floats)
constexpr int RS_D = 8;                    // steps whose loads are in flight
__global__ __launch_bounds__(64) void k_router_strict(const float *__restrict__ W, const float *__restrict__ x,
                                                      int E, int H, int T, float *__restrict__ logits) {
    __shared__ __attribute__((aligned(16))) float tp[RS_R * RS_P];
    const int lane = threadIdx.x;
    const int gpt = (E + RS_R - 1) / RS_R;                 // waves per token
    const int t = blockIdx.x / gpt, e0 = (blockIdx.x % gpt) * RS_R;
    const float *xt = x + (size_t)t * H;
    // this lane's share of a step: rows 4 k + lane / 16 (k < 4), columns
    // 4 (lane % 16) .. + 3
    const int lr = lane >> 4, lc = (lane & 15) * 4;
    float4 wv[RS_D][4], xv[RS_D];
    // Every load is a whole, in-bounds 16-byte load (H % 4 == 0): columns
    // past H and steps past the end reload the row's last four columns,
    // and their products are not added. No load sits under a branch, so
    // the waits stay exact and the RS_D steps stay in flight.
    auto load = [&](int d, int c) {
        const int i = min(c + lc, H - 4);
#pragma unroll
        for (int k = 0; k < 4; k++) wv[d][k] = *(const float4 *)(W + (size_t)min(e0 + 4 * k + lr, E - 1) * H + i);
        xv[d] = *(const float4 *)(xt + i);
    };
#pragma unroll
    for (int d = 0; d < RS_D; d++) load(d, d * RS_C);
    float acc = 0.0f;
    for (int cb = 0; cb < H; cb += RS_D * RS_C)
#pragma unroll
    for (int d = 0; d < RS_D; d++) {
        const int c = cb + d * RS_C;
        if (c >= H) break;                                 // uniform
#pragma unroll
        for (int k = 0; k < 4; k++)
            *(float4 *)&tp[(4 * k + lr) * RS_P + lc] =
                make_float4(__fmul_rn(wv[d][k].x, xv[d].x), __fmul_rn(wv[d][k].y, xv[d].y),
                            __fmul_rn(wv[d][k].z, xv[d].z), __fmul_rn(wv[d][k].w, xv[d].w));
        load(d, c + RS_D * RS_C);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane < RS_R) {
            const float *pr = &tp[lane * RS_P];
            const int n = min(RS_C, H - c);
            if (n == RS_C) {
                // all 64 products to registers first, then the adds (reads
                // interleaved with the chain would expose their latency)
                float4 v[RS_C / 4];
#pragma unroll
                for (int i = 0; i < RS_C / 4; i++) v[i] = *(const float4 *)(pr + 4 * i);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < RS_C / 4; i++) {
                    acc = __fadd_rn(acc, v[i].x);
                    acc = __fadd_rn(acc, v[i].y);
                    acc = __fadd_rn(acc, v[i].z);
                    acc = __fadd_rn(acc, v[i].w);
                }
            } else {
                for (int i = 0; i < n; i++) acc = __fadd_rn(acc, pr[i]);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    if (lane < RS_R && e0 + lane < E) logits[(size_t)t * E + e0 + lane] = acc;
}

extern "C" int wk_router_logits(const float *W, const float *x, int E, int H, int T, int strict,
                                float *logits, void *stream) {
    if (E <= 0 || H <= 0 || T <= 0) return -1;
    const int rows = E * T;
    if (strict && (H % 4))
        return -1;
    if (strict)
        hipLaunchKernelGGL(k_router_strict, dim3(T * ((E + RS_R - 1) / RS_R)), dim3(64), 0, (hipStream_t)stream, W, x,
                           E, H, T, logits);
    else if (T >= WARP_ROUTER_MFMA_T && (H & 15) == 0)
        hipLaunchKernelGGL(k_router_mfma, dim3((T + 15) / 16, (E + 15) / 16), dim3(256), 0, (hipStream_t)stream, W, x,
                           E, H, T, logits);
    else
        hipLaunchKernelGGL(k_router_fast, dim3(rows), dim3(256), 0, (hipStream_t)stream, W, x, E, H, T, logits);
    CHECK_LAUNCH();
    return 0;
}

// ---- quantised rows (Q8G / Q4G / Q3G) ------------------------------------------------

__device__ __forceinline__ int q_at(const int8_t *row, int bits, int i) {
    if (bits == 8) return row[i];
    if (bits == 4) {
        const uint8_t b = ((const uint8_t *)row)[i >> 1];
        return (i & 1) ? (int)(b >> 4) - 8 : (int)(b & 0x0F) - 8;
    }
    const uint8_t *p = (const uint8_t *)row;
    const long off = (long)i * 3;
    const int v = (p[off >> 3] >> (off & 7)) | (p[(off >> 3) + 1] << (8 - (off & 7)));
    return (v & 7) - 4;
}

// One wave per (token, output row). Lanes take whole groups; a group's
// partial dot is scaled by its fp16 scale, then the lanes' sums are reduced.
__global__ __launch_bounds__(256) void k_mvq(const int8_t *__restrict__ W, const uint16_t *__restrict__ ws,
                                             size_t rowbytes, int g, int bits, const float *__restrict__ x,
                                             int M, int N, int T, float *__restrict__ y) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M * T) return;
    const int t = row / M, o = row % M;
    const int ng = (N + g - 1) / g;
    const int8_t *wr = W + (size_t)o * rowbytes;
    const uint16_t *sr = ws + (size_t)o * ng;
    const float *xt = x + (size_t)t * N;
    float acc = 0.0f;
    for (int k = lane; k < ng; k += 64) {
        const int lim = (k * g + g <= N) ? g : N - k * g;
        float part = 0.0f;
        for (int i = 0; i < lim; i++) part = __builtin_fmaf((float)q_at(wr, bits, k * g + i), xt[k * g + i], part);
        acc = __builtin_fmaf(f16_keep(sr[k]), part, acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[row] = acc;
}

// ---- decode: the shared expert inside the router and combine launches ---------------------

// One wave's dot of a quantised row (Q8G: 16 weights per 16-byte chunk, Q4G:
// 32) with x in LDS. Lane l takes chunks l, l + 64, ...: load() issues every
// chunk and its group scale (clamped to the row, so no load is
// conditional), dot() multiplies each chunk, scales its sum by the group's
// fp16 scale and sums the lanes. The group is a multiple of a chunk's
// weights, so a chunk never straddles two groups.
template <int BITS, int MAXC>
struct QRow {
    static constexpr int WPC = BITS == 8 ? 16 : 32;
    uint4 w[MAXC];
    uint16_t s[MAXC];
    __device__ __forceinline__ void load(const int8_t *row, const uint16_t *sc, int g, int nc) {
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int k = 0; k < MAXC; k++) {
            const int c = min(lane + 64 * k, nc - 1);
            w[k] = *(const uint4 *)(row + (size_t)c * 16);
            s[k] = sc[c * WPC / g];
        }
    }
    __device__ __forceinline__ float dot(const float *xl, int nc) const {
        const int lane = threadIdx.x & 63;
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < MAXC; k++) {
            if (lane + 64 * k < nc) {
                const float *xv = xl + (lane + 64 * k) * WPC;
                const unsigned u[4] = { w[k].x, w[k].y, w[k].z, w[k].w };
                float p = 0.0f;
                if constexpr (BITS == 8) {
#pragma unroll
                    for (int i = 0; i < 16; i++)
                        p = __builtin_fmaf((float)(int)(int8_t)(u[i >> 2] >> (8 * (i & 3))), xv[i], p);
                } else {
#pragma unroll
                    for (int i = 0; i < 32; i++)
                        p = __builtin_fmaf((float)((int)((u[i >> 3] >> (4 * (i & 7))) & 0xF) - 8), xv[i], p);
                }
                acc = __builtin_fmaf(f16_keep(s[k]), p, acc);
            }
        }
        return wave_sum(acc);
    }
};

constexpr int SH_MAXC = 8;       // chunks per lane: rows up to 8192 (Q8G) or 16384 (Q4G) weights

// Q8G / Q4G rows whose width is a whole number of 16-byte chunks and whose
// group is a whole number of chunks (no chunk straddles a group or the row's
// end), 16-byte aligned: a block of 4 waves takes MQF_RPB rows of one token,
// with x staged in LDS once for them. A wave takes its rows one at a time;
// lane l loads chunks l, l + 64, ... of the row as 16-byte loads (every load
// of the row issued before the first multiply), multiplies each chunk with x
// from LDS, scales the chunk's sum by its group's fp16 scale and the lanes'
// sums are reduced. The loads of the wave's next row are issued before the
// current row's arithmetic, so a wave keeps two rows in flight.
constexpr int MQF_RPW = 4;                 // rows per wave
constexpr int MQF_RPB = 4 * MQF_RPW;       // rows per block
constexpr int MQF_MAXC = 8;                // chunks per lane: rows up to 8192 (Q8G) / 16384 (Q4G) weights

template <int BITS, int MC>
__global__ __launch_bounds__(256) void k_mvq_fast(const int8_t *__restrict__ W, const uint16_t *__restrict__ ws,
                                                  size_t rowbytes, int g, const float *__restrict__ x, int M, int N,
                                                  float *__restrict__ y) {
    extern __shared__ __attribute__((aligned(16))) float xl[];
    using Q = QRow<BITS, MC>;
    const int t = blockIdx.y, wave = threadIdx.x >> 6;
    const int nc = N / Q::WPC, ng = (N + g - 1) / g;
    const int r0 = blockIdx.x * MQF_RPB + wave * MQF_RPW;
    Q cur, nxt;
    {
        const int rr = min(r0, M - 1);
        cur.load(W + (size_t)rr * rowbytes, ws + (size_t)rr * ng, g, nc);
    }
    const float *xt = x + (size_t)t * N;
    for (int i = threadIdx.x; i < N / 4; i += 256) ((float4 *)xl)[i] = ((const float4 *)xt)[i];
    __syncthreads();
#pragma unroll
    for (int q = 0; q < MQF_RPW; q++) {
        if (q + 1 < MQF_RPW) {
            const int rr = min(r0 + q + 1, M - 1);
            nxt.load(W + (size_t)rr * rowbytes, ws + (size_t)rr * ng, g, nc);
        }
        const float v = cur.dot(xl, nc);
        if ((threadIdx.x & 63) == 0 && r0 + q < M) y[(size_t)t * M + r0 + q] = v;
        if (q + 1 < MQF_RPW) cur = nxt;
    }
}

template <int BITS>
static int launch_mvq_fast(const int8_t *W, const uint16_t *ws, size_t rowbytes, int group, const float *x, int M,
                           int N, int T, float *y, void *stream) {
    const int mc = (N / (BITS == 8 ? 16 : 32) + 63) / 64;
    const dim3 grid((M + MQF_RPB - 1) / MQF_RPB, T);
    const size_t lds = (size_t)N * sizeof(float);
#define MQF(n) hipLaunchKernelGGL((k_mvq_fast<BITS, n>), grid, dim3(256), lds, (hipStream_t)stream, W, ws, rowbytes, \
                                  group, x, M, N, y)
    if (mc <= 1) MQF(1);
    else if (mc <= 2) MQF(2);
    else if (mc <= 4) MQF(4);
    else MQF(MQF_MAXC);
#undef MQF
    CHECK_LAUNCH();
    return 0;
}

extern "C" int wk_mvq(const int8_t *W, const uint16_t *ws, size_t rowbytes, int group, int bits,
                      const float *x, int M, int N, int T, float *y, void *stream) {
    if (M <= 0 || N <= 0 || T <= 0 || group <= 0 || (bits != 8 && bits != 4 && bits != 3)) return -1;
    if (bits != 3) {
        const int wpc = bits == 8 ? 16 : 32;
        if (N % wpc == 0 && group % wpc == 0 && N / wpc <= 64 * MQF_MAXC && (size_t)N * sizeof(float) <= 64 * 1024 &&
            (rowbytes & 15) == 0 && ((uintptr_t)W & 15) == 0 && ((uintptr_t)x & 15) == 0 && (N & 3) == 0)
            return bits == 8 ? launch_mvq_fast<8>(W, ws, rowbytes, group, x, M, N, T, y, stream)
                             : launch_mvq_fast<4>(W, ws, rowbytes, group, x, M, N, T, y, stream);
    }
    hipLaunchKernelGGL(k_mvq, dim3((M * T + 3) / 4), dim3(256), 0, (hipStream_t)stream, W, ws, rowbytes, group,
                       bits, x, M, N, T, y);
    CHECK_LAUNCH();
    return 0;
}


extern "C" int wk_shared_fast_ok(int H, const warp_shared_args *sa) {
    if (!sa || (sa->bits != 8 && sa->bits != 4) || H <= 0 || sa->inter <= 0 || (H & 3) || (sa->inter & 3))
        return 0;
    const int wpc = sa->bits == 8 ? 16 : 32;
    if (sa->group <= 0 || sa->group % wpc || H % sa->group || sa->inter % sa->group) return 0;
    if (H / wpc > 64 * SH_MAXC || sa->inter / wpc > 64 * SH_MAXC) return 0;
    for (int k = 0; k < 3; k++)
        if (!sa->q[k] || !sa->s[k] || (sa->rowbytes[k] & 15) || ((uintptr_t)sa->q[k] & 15)) return 0;
    return 1;
}

// Blocks [0, E): one router row each, as k_router_fast. Blocks past E: four
// rows of the shared expert's gate and up each (one wave per row), every
// weight load issued before x is staged in LDS, then h = act(gate, up).
// MC: 16-byte chunks per lane, the fewest that cover a row (no load of a
// chunk past the row's end).
template <int BITS, int MC>
__global__ __launch_bounds__(256) void k_router_shared(const float *__restrict__ W, const float *__restrict__ x, int E,
                                                       int H, float *__restrict__ logits, warp_shared_args sa) {
    if ((int)blockIdx.x < E) {
        // as many float4 steps per thread as a row has (the same sums in the same order)
        constexpr int UNR = BITS == 8 ? MC : (2 * MC < 8 ? 2 * MC : 8);
        const float v = router_row_fast<UNR>(W, x, E, H, blockIdx.x);
        if (threadIdx.x == 0) logits[blockIdx.x] = v;
        return;
    }
    extern __shared__ float xl[];
    using Q = QRow<BITS, MC>;
    const int r = ((int)blockIdx.x - E) * 4 + (int)(threadIdx.x >> 6), rr = min(r, sa.inter - 1);
    const int nc = H / Q::WPC, ng = H / sa.group;
    Q qg, qu;
    qg.load(sa.q[0] + (size_t)rr * sa.rowbytes[0], sa.s[0] + (size_t)rr * ng, sa.group, nc);
    qu.load(sa.q[1] + (size_t)rr * sa.rowbytes[1], sa.s[1] + (size_t)rr * ng, sa.group, nc);
    for (int i = threadIdx.x; i < H / 4; i += 256) ((float4 *)xl)[i] = ((const float4 *)x)[i];
    __syncthreads();
    const float gv = qg.dot(xl, nc), uv = qu.dot(xl, nc);
    if (r < sa.inter && (threadIdx.x & 63) == 0) sa.h[r] = act_pair(gv, uv, sa.situ, sa.beta, sa.lbeta);
}

extern "C" int wk_router_shared(const float *W, const float *x, int E, int H, float *logits, const warp_shared_args *sa,
                                void *stream) {
    if (E <= 0 || !wk_shared_fast_ok(H, sa)) return -1;
    const dim3 grid(E + (sa->inter + 3) / 4);
    const size_t lds = (size_t)H * sizeof(float);
    if (lds > 64 * 1024) return -1;
    const int mc = (H / (sa->bits == 8 ? 16 : 32) + 63) / 64;     // <= SH_MAXC (wk_shared_fast_ok)
#define RS(b, n)                                                                                                   \
    hipLaunchKernelGGL((k_router_shared<b, n>), grid, dim3(256), lds, (hipStream_t)stream, W, x, E, H, logits, *sa)
    if (sa->bits == 8) {
        if (mc <= 1) RS(8, 1);
        else if (mc <= 2) RS(8, 2);
        else if (mc <= 3) RS(8, 3);
        else if (mc <= 4) RS(8, 4);
        else RS(8, SH_MAXC);
    } else {
        if (mc <= 1) RS(4, 1);
        else if (mc <= 2) RS(4, 2);
        else if (mc <= 3) RS(4, 3);
        else if (mc <= 4) RS(4, 4);
        else RS(4, SH_MAXC);
    }
#undef RS
    CHECK_LAUNCH();
    return 0;
}

// Batches of tokens on the matrix cores (the shared expert of a chunk):
// y[t][o] = sum over groups g of scale[o][g] * sum_{i in g} W[o][i] x[t][i],
// as mvq_rows_f32 (src/simd_avx512.c:20-88) per token. v_mfma_f32_16x16x32_f16
// takes 16 rows of 32 weights as A (int8 or 4-bit values, exact in fp16) and
// the fp16 hi/lo halves of x for 8 tokens as B (token t's hi in column 2t, lo
// in 2t + 1; xs from wk_split), so every product is exact and the sums are
// fp32; a group's sums are scaled by its fp16 scale in fp32, and at the end
// the two halves are added and the token's power of two removed.
//
// One launch takes one or two matrices of the same shape that share x
// (blockIdx.z: the shared expert's gate and up). The group scale is folded
// into A: q * s is exact in f32 (8 + 11 significant bits) and splits exactly
// into fp16 hi + lo (|s| < 256, so |q s| stays below the fp16 range; the
// caller checks), so acc += A_hi . B + A_lo . B sums the same exact products
// q s x with no per-group scaling step: the accumulators stay in the matrix
// cores' registers. Block = 4 waves, tile 64 rows x 64 tokens: wave w takes
// tokens 16w .. 16w + 15 (two 16-column tiles) against all 64 rows (four
// 16-row tiles), 16 MFMAs per 32 columns. The block stages 128 columns of
// its rows at a time in LDS as the hi and lo fp16 planes, converted once
// for the 4 waves (rows padded by 16 bytes, so the 16 rows a wave reads at
// one column land in distinct banks), double-buffered, with the raw weights
// of the next 2 slabs in flight in registers. Each wave's x loads run 8
// steps of 32 columns (2 slabs) ahead. The loop has no data-dependent
// branches, so every wait is for the load it needs: the slab count is
// rounded up to even and columns past N are staged as zeros (their x loads
// repeat the last step).
constexpr int MQ_MB = 64, MQ_TB = 64, MQ_KS = 128;
constexpr int MQ_LDA = MQ_KS + 8;                // fp16 per staged row
constexpr int MQ_PLANE = MQ_MB * MQ_LDA;         // fp16 per (buffer, hi/lo) plane

struct MvqMat {
    const int8_t *W;
    const uint16_t *ws;
    size_t rowbytes;
    float *y;
};

template <int BITS>
__global__ __launch_bounds__(256) void k_mvq_gemm(MvqMat m0, MvqMat m1, int group, const half8 *__restrict__ xs,
                                                  const float *__restrict__ xscale, int M, int N, int T) {
    extern __shared__ __attribute__((aligned(16))) unsigned char lds_mq[];
    _Float16 *As = (_Float16 *)lds_mq;           // [2 buffers][hi, lo][MB][LDA]
    const MvqMat mt = blockIdx.z ? m1 : m0;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r0 = blockIdx.x * MQ_MB, t0 = blockIdx.y * MQ_TB;
    const int m = lane & 15, kb = lane >> 4, nv = N >> 3, ng = N / group, nks = N >> 5;
    const int nslab = ((N + MQ_KS - 1) / MQ_KS + 1) & ~1;

    // staging: thread (row sr, part sp) takes 32 columns of a slab, which lie
    // in one group (slabs and parts start at multiples of 32, groups are
    // multiples of 32)
    const int sr = threadIdx.x >> 2, sp = threadIdx.x & 3;
    const size_t grow = (size_t)min(r0 + sr, M - 1);
    const uint8_t *wrow = (const uint8_t *)mt.W + grow * mt.rowbytes;
    const uint16_t *srow = mt.ws + grow * ng;
    constexpr int WB = BITS == 8 ? 8 : 4;        // bytes per load, 4 loads = 32 values
    constexpr int DA = 2;                        // slabs of raw weights in flight
    unsigned raw_r[DA][4][2];
    uint16_t sraw_r[DA];
    auto load_raw = [&](unsigned (&raw)[4][2], uint16_t &sraw, int sl) {
        const int k = min(sl * MQ_KS + 32 * sp, N - 32);   // past N: any valid columns, staged as zeros
        const uint8_t *p = wrow + (size_t)k * BITS / 8;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            if (BITS == 8) {
                const uint2 v = *(const uint2 *)(p + q * WB);
                raw[q][0] = v.x;
                raw[q][1] = v.y;
            } else {
                raw[q][0] = *(const unsigned *)(p + q * WB);
                raw[q][1] = 0u;
            }
        }
        sraw = srow[k / group];                            // (tested at the store: no wait here)
    };
    auto store_raw = [&](const unsigned (&raw)[4][2], uint16_t sraw, int buf, int sl) {
        _Float16 *dh = As + (size_t)(2 * buf) * MQ_PLANE + sr * MQ_LDA + 32 * sp;
        const float sc = sl * MQ_KS + 32 * sp < N ? f16_keep(sraw) : 0.0f;   // past N: zeros
#pragma unroll
        for (int q = 0; q < 4; q++) {
            half8 h, l;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int v = BITS == 8 ? (int)(int8_t)((raw[q][i >> 2] >> (8 * (i & 3))) & 0xFFu)
                                        : (int)((raw[q][0] >> (4 * i)) & 0xFu) - 8;
                const float qs = __fmul_rn((float)v, sc);       // exact
                h[i] = (_Float16)qs;
                l[i] = (_Float16)__fsub_rn(qs, (float)h[i]);    // exact
            }
            *(half8 *)(dh + 8 * q) = h;
            *(half8 *)(dh + MQ_PLANE + 8 * q) = l;
        }
    };

    // x of this wave's two column tiles: token 8 j + m / 2, half m % 2
    const half8 *xr[2];
#pragma unroll
    for (int j = 0; j < 2; j++)
        xr[j] = xs + (size_t)min(t0 + 16 * wave + 8 * j + (m >> 1), T - 1) * nv * 2 + (m & 1);
    constexpr int RB = 4 * DA;                   // x steps in flight
    half8 bq[RB][2];
    auto load_b = [&](half8 (&b)[2], int ks) {
        const int p = min(ks, nks - 1) * 4 + kb;
#pragma unroll
        for (int j = 0; j < 2; j++) b[j] = xr[j][(size_t)p * 2];
    };

#pragma unroll
    for (int d = 0; d < DA; d++) load_raw(raw_r[d], sraw_r[d], d);
#pragma unroll
    for (int u = 0; u < RB; u++) load_b(bq[u], u);
    store_raw(raw_r[0], sraw_r[0], 0, 0);
    load_raw(raw_r[0], sraw_r[0], DA);                     // the slot refilled with slab DA
    __syncthreads();

    f4 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
    // slab sl (d = sl % DA): its 4 steps from LDS buffer d with x from ring
    // slots 4 d .. 4 d + 3; then slab sl + 1's raw weights (ring slot
    // 1 - d) go to the other buffer, which nobody reads until the barrier,
    // and that slot is refilled with slab sl + 1 + DA
    auto slab = [&](int sl, auto dc) {
        constexpr int d = decltype(dc)::value;
        const _Float16 *a_base = As + (size_t)(2 * d) * MQ_PLANE + m * MQ_LDA + 8 * kb;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int ks = sl * 4 + u;
            half8 ah[4], al[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                ah[i] = *(const half8 *)(a_base + 16 * i * MQ_LDA + 32 * u);
                al[i] = *(const half8 *)(a_base + MQ_PLANE + 16 * i * MQ_LDA + 32 * u);
            }
            half8 b[2] = {bq[4 * d + u][0], bq[4 * d + u][1]};
            load_b(bq[4 * d + u], ks + RB);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], b[j], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], b[j], acc[i][j], 0, 0, 0);
        }
        constexpr int dn = (d + 1) % DA;
        store_raw(raw_r[dn], sraw_r[dn], dn, sl + 1);
        load_raw(raw_r[dn], sraw_r[dn], sl + 1 + DA);
        __syncthreads();
    };
    static_assert(DA == 2, "the slab loop below is unrolled by DA");
    for (int sl = 0; sl < nslab; sl += DA) {
        slab(sl, std::integral_constant<int, 0>{});
        slab(sl + 1, std::integral_constant<int, 1>{});
    }
    // lane (kb, m) holds rows 4 kb + r of each 16-row tile; column m holds
    // token m / 2, half m % 2: add the halves, remove 2^k
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int t = t0 + 16 * wave + 8 * j + (m >> 1);
        const float xsc = xscale[min(t, T - 1)];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            f4 v;
#pragma unroll
            for (int r = 0; r < 4; r++) v[r] = (acc[i][j][r] + __shfl_xor(acc[i][j][r], 1)) * xsc;
            const int row = r0 + 16 * i + 4 * kb;
            if ((m & 1) == 0 && t < T) {
                float *yo = mt.y + (size_t)t * M + row;
                if (row + 3 < M && (M & 3) == 0) {
                    *(f4 *)yo = v;
                } else {
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        if (row + r < M) yo[r] = v[r];
                }
            }
        }
    }
}

extern "C" int wk_mvq_gemm(int nmat, const int8_t *const *W, const uint16_t *const *ws, const size_t *rowbytes,
                           int group, int bits, const uint16_t *xs, const float *xscale, int M, int N, int T,
                           float *const *y, void *stream) {
    if (nmat < 1 || nmat > 2 || M <= 0 || N < 32 || T <= 0 || (N % 32) || group <= 0 || (group % 32) ||
        (N % group))
        return -1;
    for (int k = 0; k < nmat; k++) {
        if (!W[k] || !ws[k] || !y[k]) return -1;
        if (bits == 8 && (rowbytes[k] % 8 || rowbytes[k] < (size_t)N)) return -1;
        if (bits == 4 && (rowbytes[k] % 4 || rowbytes[k] < (size_t)N / 2)) return -1;
    }
    const size_t lds = (size_t)4 * MQ_PLANE * sizeof(_Float16);
    const MvqMat a = {W[0], ws[0], rowbytes[0], y[0]};
    const MvqMat b = nmat > 1 ? MvqMat{W[1], ws[1], rowbytes[1], y[1]} : a;
    const dim3 grid((M + MQ_MB - 1) / MQ_MB, (T + MQ_TB - 1) / MQ_TB, nmat);
    if (bits == 8) {
        static std::atomic<uint64_t> attr{0};
        if (int r_ = lds_limit((const void *)k_mvq_gemm<8>, 160 * 1024, attr, stream)) return r_;
        hipLaunchKernelGGL(k_mvq_gemm<8>, grid, dim3(256), lds, (hipStream_t)stream, a, b, group,
                           (const half8 *)xs, xscale, M, N, T);
    } else if (bits == 4) {
        static std::atomic<uint64_t> attr{0};
        if (int r_ = lds_limit((const void *)k_mvq_gemm<4>, 160 * 1024, attr, stream)) return r_;
        hipLaunchKernelGGL(k_mvq_gemm<4>, grid, dim3(256), lds, (hipStream_t)stream, a, b, group,
                           (const half8 *)xs, xscale, M, N, T);
    } else {
        return -1;
    }
    CHECK_LAUNCH();
    return 0;
}

// ---- jobs -----------------------------------------------------------------------------

// Pointers of one matrix inside a record, from the header offsets the table
// holds (waste_expert_hdr, src/waste_format.h:98-130). Row scales are gate
// [I], up [I], down [H].
__device__ __forceinline__ void job_ptrs(warp_job &jb, const warp_slot &sl, int kind, int inter) {
    jb.idx = sl.rec + sl.off[kind];
    const int soff = kind == 0 ? 0 : kind == 1 ? inter : 2 * inter;
    jb.scale = (const uint16_t *)(sl.rec + sl.off[3]) + soff;
}

// ---- routing -----------------------------------------------------------------------

// fl(...fl(fl(0 + v[0]) + v[1]) ... + v[n-1]), one thread: the values of 64
// steps are read at once, so the adds wait for one LDS round trip per 64.
__device__ __forceinline__ float seq_sum_lds(const float *v, int n) {
    float s = 0.0f;
    int e = 0;
    for (; e + 64 <= n; e += 64) {
        float b[64];
#pragma unroll
        for (int i = 0; i < 64; i++) b[i] = v[e + i];
#pragma unroll
        for (int i = 0; i < 64; i++) s = __fadd_rn(s, b[i]);
    }
    for (; e < n; e++) s = __fadd_rn(s, v[e]);
    return s;
}

template <int CTRL, int ROWS>
__device__ __forceinline__ int dpp_src(int v) {
    return __builtin_amdgcn_update_dpp(v, v, CTRL, ROWS, 0xf, false);
}
template <bool MAX>
__device__ __forceinline__ int wave_reduce_i(int v) {
    auto op = [](int a, int b) { return MAX ? max(a, b) : min(a, b); };
    v = op(v, dpp_src<0xB1, 0xf>(v));    // quad_perm 1,0,3,2
    v = op(v, dpp_src<0x4E, 0xf>(v));    // quad_perm 2,3,0,1
    v = op(v, dpp_src<0x141, 0xf>(v));   // row_half_mirror
    v = op(v, dpp_src<0x140, 0xf>(v));   // row_mirror
    v = op(v, dpp_src<0x142, 0xa>(v));   // row_bcast15
    v = op(v, dpp_src<0x143, 0xc>(v));   // row_bcast31
    return __builtin_amdgcn_readlane(v, 63);
}

// Order-preserving int key of a biased score: larger score, larger key.
// -0 counts as +0 (the reference compares floats), and values the
// reference's scan can never pick (at or below -1e30, NaN) get INT_MIN.
__device__ __forceinline__ int route_key(float v) {
    if (!(v > -1e30f)) return INT_MIN;
    const int b = __float_as_int(v + 0.0f);
    return b ^ ((b >> 31) & 0x7fffffff);
}

// Whether a pick has no record: lane j of every wave checks pick j (K <= 64),
// one ballot, no chain of dependent LDS reads.
__device__ __forceinline__ bool picks_missing(const warp_slot *slots, const int *sel, int K) {
    const int l = threadIdx.x & 63;
    const bool m = l < K && slots[sel[min(l, K - 1)]].rec == nullptr;
    return __ballot(m) != 0ull;
}

// Certified selection's test by wave 0 of the picking block (E <= 512, the
// ids lane + 64 m of each lane), with the picks in rank order in lanes
// 0..np-1 (mine) and the biased scores and their bounds in LDS: the
// ambiguous experts, as cert_check defines them, into amb (nonzero bits)
// and their number into *namb, without a block barrier. A non-pick is an
// id whose (key, ~id) is below the last pick's. The usual case is settled
// first with a shorter test: when each pick's lower bound is above the
// next pick's upper bound, the picks' intervals are ordered pairwise (by
// induction along the ranks) and the last pick's lower bound is their
// lowest, so no expert is ambiguous if no non-pick's upper bound reaches it.
__device__ __forceinline__ void route_cert_wave(int E, int np, int mine, const float *biased, const float *lo,
                                                const float *hi, unsigned long long *amb, int *namb) {
    const int lane = threadIdx.x & 63;
    const bool pk = lane < np;
    const float plo = pk ? lo[mine] : INFINITY, phi = pk ? hi[mine] : -INFINITY;
    const int last = __builtin_amdgcn_readlane(mine, max(np, 1) - 1);
    const unsigned long long kmin =
        np > 0 ? ((unsigned long long)((unsigned)route_key(biased[last]) ^ 0x80000000u) << 32) | (unsigned)~last
               : ~0ull;
    float h[8];
    bool non[8];
#pragma unroll
    for (int m = 0; m < 8; m++) {
        const int e = lane + 64 * m, ec = min(e, E - 1);
        const unsigned long long pkd =
            ((unsigned long long)((unsigned)route_key(biased[ec]) ^ 0x80000000u) << 32) | (unsigned)~ec;
        non[m] = e < E && pkd < kmin;
        h[m] = hi[ec];
    }
    // the short test
    const float nhi = __shfl_down(phi, 1);                 // the next pick's upper bound
    const bool sep = lane + 1 >= np || plo > nhi;
    const float lastlo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(plo), max(np, 1) - 1));
    bool reach = false;
#pragma unroll
    for (int m = 0; m < 8; m++) reach |= non[m] && h[m] >= lastlo;
    if (__ballot(!sep || reach) == 0ull) {                 // uniform: nothing ambiguous
        if (lane == 0) *namb = 0;
        return;
    }
    // the full test: every pair
    float pm = plo, sm = phi;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float u = __shfl_up(pm, o), d = __shfl_down(sm, o);
        if (lane >= o) pm = fminf(pm, u);
        if (lane + o < 64) sm = fmaxf(sm, d);
    }
    float before = __shfl_up(pm, 1), after = __shfl_down(sm, 1);
    if (lane == 0) before = INFINITY;
    if (lane == 63) after = -INFINITY;
    const float minlo = __shfl(pm, 63);                   // the lowest lower bound of a pick
    float mnp = -INFINITY;
    bool np_amb[8];
    int n = 0;
#pragma unroll
    for (int m = 0; m < 8; m++) {
        mnp = non[m] ? fmaxf(mnp, h[m]) : mnp;
        np_amb[m] = non[m] && h[m] >= minlo;
    }
    mnp = wave_max(mnp);
    const bool pa = pk && (before <= phi || after >= plo || mnp >= plo);
#pragma unroll
    for (int m = 0; m < 8; m++) {
        const unsigned long long b = __ballot(np_amb[m]);
        n += __popcll(b);
        if (lane == 0 && 64 * m < E) amb[m] = b;
    }
    const unsigned long long pb = __ballot(pa);
    n += __popcll(pb);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (pa) atomicOr(&amb[mine >> 6], 1ull << (mine & 63));
    if (lane == 0) *namb = n;
}

// Decode routing (one token). The logits, the bias and this layer's expert
// table go to LDS in one pass of independent loads; one wave then takes the
// K picks by repeated arg-max -- larger biased score first, the lower id on
// equal scores, never a value at or below -1e30: the reference's scan
// (src/model.c:2727-2739) -- each lane keeping the best of its own ids and
// rescanning them only when that best is taken. The job lists are then
// written from the table in LDS, with no dependent reads of HBM.
// Scores, selection and weights of one token's routing (src/model.c:2723-
// 2745) by a block of NT threads, from the logits and biases already in LDS
// (score[E], biased[E]; both overwritten). On return (all threads past a
// barrier) sel[0..K) holds the picks in order and wsel[0..K) their weights,
// 0 past the picks found; returns the number of picks (< K only when fewer
// than K experts are pickable). want_w (uniform) false: the weights are not
// computed and wsel is left at 0 (a block that only needs the picks).
// scored (uniform): score and biased already hold the sigmoid scores and the
// biased scores (k_router_scored), so the scoring pass is skipped.
// clo/chi (REGS, certified selection): the biased scores' lower and upper
// bounds; wave 0 then also marks the ambiguous experts (as cert_check
// defines them) in camb (E / 64 words) and their number in *namb.
template <bool REGS, int NT>
__device__ __forceinline__ int route_pick_lds(int E, int K, int act, int renorm, float routed_scale, float *score,
                                              float *biased, int *sel, float *wsel, bool want_w = true,
                                              bool scored = false, const uint64_t *etab = nullptr,
                                              const float *clo = nullptr, const float *chi = nullptr,
                                              unsigned long long *camb = nullptr, int *namb = nullptr) {
    __shared__ float red[NT / 64];
    __shared__ int np_s;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid < WARP_MAX_K) { sel[tid] = 0; wsel[tid] = 0.0f; }
    __syncthreads();
    if (!scored) {
        if (act == 1) {
            float mx = -INFINITY;
            for (int e = tid; e < E; e += NT) mx = fmaxf(mx, score[e]);
            mx = wave_max(mx);
            if (lane == 0) red[wave] = mx;
            __syncthreads();
            mx = red[0];
            for (int i = 1; i < NT / 64; i++) mx = fmaxf(mx, red[i]);
            for (int e = tid; e < E; e += NT) score[e] = expf_ref(__fsub_rn(score[e], mx), etab);
            __syncthreads();
            if (tid == 0) red[0] = seq_sum_lds(score, E);   // sequential, as the reference sums
            __syncthreads();
            const float s = red[0];
            for (int e = tid; e < E; e += NT) score[e] = __fdiv_rn(score[e], s);
        } else {
            for (int e = tid; e < E; e += NT) score[e] = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf_ref(-score[e], etab)));
        }
        for (int e = tid; e < E; e += NT) biased[e] = __fadd_rn(score[e], biased[e]);
        __syncthreads();
    }
    if (wave == 0) {
        // Lane l holds the keys of ids l, l + 64, ... (REGS: all in registers,
        // E <= 512; else rescans LDS). The picks of the reference's loop (max
        // each time, strict >, lowest id on ties) are the K largest of
        // (key, -id), in that order.
        constexpr int VPL = REGS ? 8 : 1;
        int mine = 0, npick = 0;
        bool done = false;
        if (REGS) {
            // Order-preserving unsigned keys, 0 for the unpickable. The K-th
            // largest lane maximum t0 bounds the K-th largest key from below
            // (the maxima are K elements of the set), so the picks are among
            // the keys >= max(t0, 1). When those survivors fit one per lane
            // (the usual case), each ranks itself among them by the packed
            // (key, ~id); otherwise the pick loop below runs.
            __shared__ unsigned long long ck[64];
            __shared__ int ord[64];
            unsigned u[VPL], mx = 0;
            float bk[VPL];
#pragma unroll
            for (int m = 0; m < VPL; m++) bk[m] = biased[min(lane + 64 * m, E - 1)];   // all reads in flight
#pragma unroll
            for (int m = 0; m < VPL; m++) {
                const int e = lane + 64 * m;
                u[m] = e < E ? (unsigned)route_key(bk[m]) ^ 0x80000000u : 0u;
                mx = u[m] > mx ? u[m] : mx;
            }
            unsigned t0 = 0;
#pragma unroll
            for (int bit = 31; bit >= 0; bit--) {
                const unsigned cand = t0 | (1u << bit);
                if (__popcll(__ballot(mx >= cand)) >= K) t0 = cand;
            }
            const unsigned lo = t0 ? t0 : 1u;
            const unsigned long long below = (1ull << lane) - 1ull;
            int n = 0;
#pragma unroll
            for (int m = 0; m < VPL; m++) {
                const bool sv = u[m] >= lo;
                const unsigned long long bm = __ballot(sv);
                const int p = n + __popcll(bm & below);
                if (sv && p < 64) ck[p] = ((unsigned long long)u[m] << 32) | (unsigned)~(lane + 64 * m);
                n += __popcll(bm);
            }
            if (n <= 64) {                                 // uniform
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                // each survivor's rank: the others' keys by readlane (no
                // LDS round trip per candidate)
                const unsigned long long me = lane < n ? ck[lane] : 0ull;
                const unsigned mlo = (unsigned)me, mhi = (unsigned)(me >> 32);
                int r = 0;
                for (int i = 0; i < n; i++) {
                    const unsigned long long o =
                        ((unsigned long long)(unsigned)__builtin_amdgcn_readlane((int)mhi, i) << 32) |
                        (unsigned)__builtin_amdgcn_readlane((int)mlo, i);
                    r += o > me;
                }
                if (lane < n && r < K) ord[r] = (int)~(unsigned)me;
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                npick = n < K ? n : K;
                mine = lane < npick ? ord[lane] : 0;
                done = true;
            }
        }
        if (!done) {
            // A pick: the wave max key; the lowest id holding it (one ballot
            // when it is unique, else a min over ids); the owner lane drops it
            // and rescans, the other lanes keep their best (selects, no
            // branches). Pick j stays in lane j.
            int key[VPL];
#pragma unroll
            for (int m = 0; m < VPL; m++) {
                const int e = lane + 64 * m;
                key[m] = REGS && e < E ? route_key(biased[e]) : INT_MIN;
            }
            auto best_of = [&](int &bk, int &bid) {
                bk = INT_MIN;
                bid = 0x7fffffff;
                if (REGS) {
#pragma unroll
                    for (int m = 0; m < VPL; m++) {
                        const bool b = key[m] > bk;
                        bk = b ? key[m] : bk;
                        bid = b ? lane + 64 * m : bid;
                    }
                } else {
                    for (int e = lane; e < E; e += 64) {
                        const int k = route_key(biased[e]);
                        if (k > bk) { bk = k; bid = e; }
                    }
                }
            };
            int bk, bid;
            best_of(bk, bid);
            for (int j = 0; j < K; j++) {
                const int m = wave_reduce_i<true>(bk);
                if (m == INT_MIN) break;          // nothing pickable is left (uniform)
                const unsigned long long hit = __ballot(bk == m);
                int e;
                if (__popcll(hit) == 1) e = __builtin_amdgcn_readlane(bid, __ffsll((long long)hit) - 1);
                else e = wave_reduce_i<false>(bk == m ? bid : 0x7fffffff);
                mine = lane == j ? e : mine;
                npick = j + 1;
                const bool own = (e & 63) == lane;
                if (REGS) {
#pragma unroll
                    for (int q = 0; q < VPL; q++) key[q] = own && q == (e >> 6) ? INT_MIN : key[q];
                    int nk, ni;
                    best_of(nk, ni);
                    bk = own ? nk : bk;
                    bid = own ? ni : bid;
                } else if (own) {
                    biased[e] = -INFINITY;
                    best_of(bk, bid);
                }
            }
        }
        // weights: the sum in pick order (one lane, as the reference), the
        // divisions and the scale in parallel
        if (lane < K) sel[lane] = lane < npick ? mine : 0;
        if (want_w) {
            float wv = lane < npick ? score[mine] : 0.0f;
            float ssum = 0.0f;
            for (int j = 0; j < K; j++)
                ssum = __fadd_rn(ssum, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wv), j)));
            if (renorm && K > 1) wv = __fdiv_rn(wv, __fadd_rn(ssum, 1e-20f));
            wv = __fmul_rn(wv, routed_scale);
            if (lane < K) wsel[lane] = wv;
        }
        if (REGS && clo) route_cert_wave(E, npick, mine, biased, clo, chi, camb, namb);
        if (lane == 0) np_s = npick;
    }
    __syncthreads();
    return np_s;
}

constexpr int CERT_NB = 16;                 // rows recomputed together (lanes of wave 0)
constexpr int CERT_PT = 16;                 // products per thread per chunk

// The certified selection's counters: one routing that recomputed, n rows.
__device__ __forceinline__ void cert_count(const warp_route_args &r, int n) {
    if (threadIdx.x == 0 && r.cctr) {
        __hip_atomic_fetch_add(r.cctr, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_add(r.cctr + 1, (unsigned long long)n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// The recompute of the ambiguous rows cert_check flags (see there), for
// buffers too small for cert_recompute: amb, their mask (nw words,
// consumed); the rows' scores and biased scores are rewritten. Rows in
// batches of up to CERT_NB: the block forms the products fl(w_k x_k) of a
// chunk of columns into stg (the next chunk's loads in flight meanwhile)
// and lanes of wave 0 add them in index order, one row per lane, unfused:
// the reference's dotf (src/model.c:155-160).
template <int NT>
__device__ __forceinline__ void cert_recompute_seq(const warp_route_args &r, float *score, float *biased,
                                                   unsigned long long *amb, int nw, float *stg, int cap,
                                                   const uint64_t *etab) {
    const float *cw = r.cw, *cx = r.cx, *bias = r.bias;
    const int H = r.ch;
    __shared__ int c_ids[CERT_NB];
    __shared__ int c_na;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (;;) {
        if (tid == 0) {                                  // the next batch, ascending ids
            int na = 0;
            for (int i = 0; i < nw && na < CERT_NB; i++) {
                unsigned long long m = amb[i];
                while (m && na < CERT_NB) {
                    c_ids[na++] = i * 64 + __ffsll((long long)m) - 1;
                    m &= m - 1ull;
                }
                amb[i] = m;
            }
            c_na = na;
        }
        __syncthreads();
        const int na = c_na;
        if (na == 0) break;                              // uniform
        // a chunk: na rows of C columns (C % 4 == 0), [C / 4][na][4] in stg
        const int C = min(min(cap / na, NT * CERT_PT / na) & ~3, H);
        float pr[CERT_PT];
        auto load = [&](int k0) {
#pragma unroll
            for (int i = 0; i < CERT_PT; i++) {
                const int t = tid + i * NT, a = t / C, k = t - a * C;
                const bool ok = a < na && k0 + k < H;
                const int kk = ok ? k0 + k : 0;
                const float w = cw[(size_t)c_ids[ok ? a : 0] * H + kk], xv = cx[kk];
                pr[i] = ok ? __fmul_rn(w, xv) : 0.0f;
            }
        };
        load(0);
        float s = 0.0f;
        for (int k0 = 0; k0 < H; k0 += C) {
#pragma unroll
            for (int i = 0; i < CERT_PT; i++) {
                const int t = tid + i * NT, a = t / C, k = t - a * C;
                if (a < na) stg[((k >> 2) * na + a) * 4 + (k & 3)] = pr[i];
            }
            __syncthreads();
            if (k0 + C < H) load(k0 + C);                // in flight while the chain runs
            if (wave == 0 && lane < na) {
                // row lane's products in index order, one unfused add each;
                // the next eight reads in flight while eight are added
                const int n4 = min(C, H - k0) >> 2;
                const float4 *s4 = (const float4 *)stg + lane;
                int q = 0;
                if (n4 >= 8) {
                    float4 c[8];
#pragma unroll
                    for (int j = 0; j < 8; j++) c[j] = s4[(size_t)j * na];
                    for (; q + 8 <= n4; q += 8) {
                        float4 nx[8];
                        const int qn = min(q + 8, n4 - 8);         // (the last group reads itself again)
#pragma unroll
                        for (int j = 0; j < 8; j++) nx[j] = s4[(size_t)(qn + j) * na];
#pragma unroll
                        for (int j = 0; j < 8; j++) {
                            s = __fadd_rn(s, c[j].x);
                            s = __fadd_rn(s, c[j].y);
                            s = __fadd_rn(s, c[j].z);
                            s = __fadd_rn(s, c[j].w);
                        }
#pragma unroll
                        for (int j = 0; j < 8; j++) c[j] = nx[j];
                    }
                }
                for (; q < n4; q++) {
                    const float4 v = s4[(size_t)q * na];
                    s = __fadd_rn(s, v.x);
                    s = __fadd_rn(s, v.y);
                    s = __fadd_rn(s, v.z);
                    s = __fadd_rn(s, v.w);
                }
            }
            __syncthreads();
        }
        if (wave == 0 && lane < na) {
            const int e = c_ids[lane];
            const float sc = cert_score(s, etab);
            score[e] = sc;
            biased[e] = __fadd_rn(sc, bias ? bias[e] : 0.0f);
        }
        __syncthreads();
    }
}

// Floats in order as integers: consecutive floats are consecutive keys
// (-0 just below +0).
__device__ __forceinline__ long long fkey(float f) {
    const int b = __float_as_int(f);
    return b >= 0 ? (long long)b : -(long long)(b & 0x7fffffff) - 1;
}
__device__ __forceinline__ float fkey_inv(long long k) {
    return k >= 0 ? __int_as_float((int)k) : __int_as_float((int)((-(k + 1)) | 0x80000000ll));
}

// v + p[0] + p[1] + ... + p[4 n4 - 1], one fp32 add at a time in that order
// (the reference's dotf chain), p 16-byte aligned in LDS, the next 16
// float4 read while 16 are added: 64 dependent adds cover the LDS latency
// (4 ahead left it exposed: a K3 routing's recompute, 2.1 rows on average,
// took 35 us with 4 ahead and 27 us with 16).
__device__ __forceinline__ float chain_add(float v, const float4 *p, int n4) {
    constexpr int D = 16;
    int q = 0;
    if (n4 >= D) {
        float4 c[D];
#pragma unroll
        for (int j = 0; j < D; j++) c[j] = p[j];
        for (; q + D <= n4; q += D) {
            float4 nx[D];
            const int qn = min(q + D, n4 - D);             // (the last group reads itself again)
#pragma unroll
            for (int j = 0; j < D; j++) nx[j] = p[qn + j];
#pragma unroll
            for (int j = 0; j < D; j++) {
                v = __fadd_rn(v, c[j].x);
                v = __fadd_rn(v, c[j].y);
                v = __fadd_rn(v, c[j].z);
                v = __fadd_rn(v, c[j].w);
            }
#pragma unroll
            for (int j = 0; j < D; j++) c[j] = nx[j];
        }
    }
    for (; q < n4; q++) {
        const float4 c = p[q];
        v = __fadd_rn(v, c.x);
        v = __fadd_rn(v, c.y);
        v = __fadd_rn(v, c.z);
        v = __fadd_rn(v, c.w);
    }
    return v;
}

// One DPP move of a double (its two halves): rows masked out, or lanes with
// no source under bound_ctrl, read 0.
template <int CTRL, int ROWS, bool BC>
__device__ __forceinline__ double dpp_f64(double x) {
    const uint64_t b = __builtin_bit_cast(uint64_t, x);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, ROWS, 0xf, BC);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, ROWS, 0xf, BC);
    return __builtin_bit_cast(double, ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

// The sum over the wave into lane 63 (the other lanes hold partial sums):
// row shifts by 1, 2, 4, 8, then lane 15 of each row added into the next
// (rows 1 and 3) and lane 31 into rows 2 and 3.
__device__ __forceinline__ double wave_sum63_f64(double v) {
    v += dpp_f64<0x111, 0xf, true>(v);
    v += dpp_f64<0x112, 0xf, true>(v);
    v += dpp_f64<0x114, 0xf, true>(v);
    v += dpp_f64<0x118, 0xf, true>(v);
    v += dpp_f64<0x142, 0xa, false>(v);
    v += dpp_f64<0x143, 0xc, false>(v);
    return v;
}

// The sequential sum v + P[0] + ... + P[n - 1] (fp32, one add at a time) by a
// block of NT threads, by speculation over segments: the chain is cut into
// G = NT / 64 segments of L = n / G, and wave g runs segment g from 64
// starts at once -- the 64 floats around the exact prefix sum before it
// (rounded to float), one per lane; the sequential running sum there is
// that prefix plus its rounding so far, usually within a few tens of ulps.
// Wave 0 then follows the chain: from segment 0's end (its start, v, is
// exact) it takes the lane of segment 1 whose start is that value, and so
// on; where the value is not among a segment's starts, it adds that segment
// itself. Returns the sum in every thread (uniform). n % (4 G) == 0; P in
// LDS, 16-byte aligned; U: 64 G floats of LDS.
template <int NT>
__device__ __forceinline__ float spec_chain(float v, const float *P, int n, float *U) {
    constexpr int G = NT / 64;
    __shared__ double sc_seg[G];
    __shared__ float sc_ctr[G], sc_v;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, L = n / G;
    double t = 0.0;                                       // the segments' exact sums
    for (int k = wave * L + lane; k < (wave + 1) * L; k += 64) t += (double)P[k];
    t = wave_sum63_f64(t);
    if (lane == 63) sc_seg[wave] = t;
    __syncthreads();
    if (tid == 0) {
        double acc = (double)v;
        for (int g = 0; g < G; g++) {
            sc_ctr[g] = (float)acc;
            acc += sc_seg[g];
        }
    }
    __syncthreads();
    const float v0 = wave == 0 ? v : fkey_inv(fkey(sc_ctr[wave]) + lane - 32);
    U[wave * 64 + lane] = chain_add(v0, (const float4 *)(P + wave * L), L >> 2);
    __syncthreads();
    if (wave == 0) {                                      // (every lane the same values)
        // lane c holds the end of each segment's start c, lane g the key of
        // segment g's centre
        float ug[G];
#pragma unroll
        for (int g = 0; g < G; g++) ug[g] = U[g * 64 + lane];
        const int kc = (int)fkey(sc_ctr[min(lane, G - 1)]);
        float w = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(ug[0])));
#pragma unroll
        for (int g = 1; g < G; g++) {
            const int c = __builtin_amdgcn_readlane(kc, g);
            const int d = __builtin_amdgcn_readfirstlane((int)((unsigned)fkey(w) - (unsigned)c + 32u));
            // (32-bit keys: a wrapped difference fails the equality test)
            if ((unsigned)d < 64u && isfinite(w) && fkey_inv((long long)c + d - 32) == w)
                w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ug[g]), d));
            else
                w = chain_add(w, (const float4 *)(P + g * L), L >> 2);
        }
        if (lane == 0) sc_v = w;
    }
    __syncthreads();
    return sc_v;
}

// The recompute of the ambiguous rows: as many rows' products fl(w_k x_k)
// as the buffer holds go to LDS at once, then each row's sequential sum by
// spec_chain. H % (4 G) == 0 (G = NT / 64) and cap >= H + 128 G, else the
// chunked single-lane recompute (cert_recompute_seq).
template <int NT>
__device__ __forceinline__ void cert_recompute(const warp_route_args &r, float *score, float *biased,
                                               unsigned long long *amb, int nw, float *stg, int cap,
                                               const uint64_t *etab) {
    constexpr int G = NT / 64;
    constexpr int NR = 4;                                 // rows filled together, at most
    const int H = r.ch;
    if (H % (4 * G) || cap < H + 128 * G) {
        cert_recompute_seq<NT>(r, score, biased, amb, nw, stg, cap, etab);
        return;
    }
    __shared__ int c_rows[NR];
    __shared__ int c_nr;
    const int tid = threadIdx.x;
    const int fit = min(NR, (cap - 128 * G) / H);
    float *U = stg + (size_t)fit * H;
    for (;;) {
        if (tid == 0) {                                  // the next rows, ascending ids
            int n = 0;
            for (int i = 0; i < nw && n < fit; i++) {
                unsigned long long m = amb[i];
                while (m && n < fit) {
                    c_rows[n++] = i * 64 + __ffsll((long long)m) - 1;
                    m &= m - 1ull;
                }
                amb[i] = m;
            }
            c_nr = n;
        }
        __syncthreads();
        const int nr = c_nr;
        if (nr == 0) break;                               // uniform
        const float4 *x4 = (const float4 *)r.cx;
        for (int i = tid; i < nr * (H >> 2); i += NT) {
            const int q = i / (H >> 2), j = i - q * (H >> 2);
            const float4 a = ((const float4 *)(r.cw + (size_t)c_rows[q] * H))[j], b = x4[j];
            ((float4 *)stg)[i] = make_float4(__fmul_rn(a.x, b.x), __fmul_rn(a.y, b.y), __fmul_rn(a.z, b.z),
                                             __fmul_rn(a.w, b.w));
        }
        __syncthreads();
        for (int q = 0; q < nr; q++) {
            const float v = spec_chain<NT>(0.0f, stg + (size_t)q * H, H, U);
            if (tid == 0) {
                const int e = c_rows[q];
                const float sc = cert_score(v, etab);
                score[e] = sc;
                biased[e] = __fadd_rn(sc, r.bias ? r.bias[e] : 0.0f);
            }
        }
        __syncthreads();
    }
}

// Certified selection (sigmoid scores from k_router_cert's bounds). After
// route_pick_lds has picked sel[0..np) by the point biased scores: an expert
// is ambiguous when its biased-score interval [lo, hi] (which holds both the
// point value and the reference's) leaves its order against another expert
// open -- a non-pick whose upper bound reaches the lowest lower bound of a
// pick, a pick whose lower bound is reached by a later pick's upper bound or
// a non-pick's, a pick whose upper bound reaches an earlier pick's lower
// bound. Every pair involving an expert that is not ambiguous is ordered by
// the intervals themselves, so once the ambiguous experts' logits are the
// reference's, the picks made again from these values are the reference's
// picks in the reference's order. The ambiguous rows are recomputed
// (cert_recompute, which the caller runs when this returns non-zero, then
// picks again) in batches of up to CERT_NB: the block forms the products
// fl(w_k x_k) of a chunk of columns into stg (the next chunk's loads in
// flight meanwhile) and lanes of wave 0 add them in index order, one row per
// lane, unfused: the reference's dotf (src/model.c:155-160). The row's score
// and biased score then follow with the routing's own operations.
// Returns the number of ambiguous experts (uniform; 0: the picks stand) and
// their mask in amb. MW: mask words, E <= 64 MW. stg: cap floats of LDS
// (16-byte aligned), cap >= 64 * CERT_NB. count: the block adds to the
// route's counters.
template <int NT, int MW>
__device__ __forceinline__ int cert_check(const warp_route_args &r, int E, int np, float *score, float *biased,
                                          const float *lo, const float *hi, const int *sel, bool count,
                                          unsigned long long *&amb) {
    __shared__ unsigned long long c_pick[MW], c_amb[MW];
    amb = c_amb;
    __shared__ float c_red[NT / 64];
    __shared__ int c_tot;
    __shared__ float c_minlo;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nw = (E + 63) >> 6;
    for (int i = tid; i < nw; i += NT) {
        c_pick[i] = 0ull;
        c_amb[i] = 0ull;
    }
    __syncthreads();
    if (tid < np) atomicOr(&c_pick[sel[tid] >> 6], 1ull << (sel[tid] & 63));
    __syncthreads();
    float mnp = -INFINITY;                               // the highest upper bound of a non-pick
    for (int e = tid; e < E; e += NT)
        if (!((c_pick[e >> 6] >> (e & 63)) & 1ull)) mnp = fmaxf(mnp, hi[e]);
    mnp = wave_max(mnp);
    if (lane == 0) c_red[wave] = mnp;
    // the picks by rank in wave 0, lane j = rank j: the lowest lower bound
    // of the ranks before j, the highest upper bound of those after it
    const bool pk = wave == 0 && lane < np;
    const float plo = pk ? lo[sel[lane]] : INFINITY, phi = pk ? hi[sel[lane]] : -INFINITY;
    float before = INFINITY, after = -INFINITY;
    if (wave == 0) {                                     // uniform per wave
        float pm = plo, sm = phi;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float u = __shfl_up(pm, o), d = __shfl_down(sm, o);
            if (lane >= o) pm = fminf(pm, u);
            if (lane + o < 64) sm = fmaxf(sm, d);
        }
        before = __shfl_up(pm, 1);
        after = __shfl_down(sm, 1);
        if (lane == 0) before = INFINITY;
        if (lane == 63) after = -INFINITY;
        const float mn = -wave_max(-plo);
        if (lane == 0) c_minlo = mn;
    }
    __syncthreads();
    if (pk) {
        float m2 = c_red[0];
        for (int i = 1; i < NT / 64; i++) m2 = fmaxf(m2, c_red[i]);
        if (before <= phi || after >= plo || m2 >= plo) atomicOr(&c_amb[sel[lane] >> 6], 1ull << (sel[lane] & 63));
    }
    {
        const float minlo = c_minlo;
        for (int e = tid; e < E; e += NT)
            if (!((c_pick[e >> 6] >> (e & 63)) & 1ull) && hi[e] >= minlo)
                atomicOr(&c_amb[e >> 6], 1ull << (e & 63));
    }
    __syncthreads();
    if (tid == 0) {
        int n = 0;
        for (int i = 0; i < nw; i++) n += __popcll(c_amb[i]);
        c_tot = n;
    }
    __syncthreads();
    const int total = c_tot;
    if (total == 0) return 0;                            // uniform
    // the picking loop may have taken the picks' biased scores out: their
    // point values again (the router kernel's operations)
    if (tid < np) {
        const int e = sel[tid];
        biased[e] = __fadd_rn(score[e], r.bias ? r.bias[e] : 0.0f);
    }
    if (count) cert_count(r, total);
    return total;
}

// The decode job lists from the picks, by a block of NT threads: jobs[0..K)
// gate, [K..2K) up, [2K..3K) down, njobs[3] = {K, K, K}, or {0, 0, 0} and
// *missing = 1 when a picked expert has no record. slots: the layer's expert
// table (in LDS or global memory).
template <int NT>
__device__ __forceinline__ void route_jobs(const int *sel, int K, const warp_slot *slots, warp_job *__restrict__ jobs,
                                           int *__restrict__ njobs, int *__restrict__ missing, int inter) {
    const int tid = threadIdx.x;
    int miss = 0;
    for (int t = tid; t < 3 * K; t += NT) {          // one thread per (kind, pick), field by field
        const int kind = t / K, j = t - kind * K;
        const warp_slot &sl = slots[sel[j]];
        const uint8_t *rec = sl.rec;
        miss |= rec == nullptr;
        warp_job *jo = jobs + kind * K + j;
        const int soff = kind == 0 ? 0 : kind == 1 ? inter : 2 * inter;
        jo->idx = rec ? rec + sl.off[kind] : nullptr;
        jo->scale = rec ? (const uint16_t *)(rec + sl.off[3]) + soff : nullptr;
        jo->n = 1;
        jo->rsv = 0;
#pragma unroll
        for (int s = 0; s < WARP_TPJ; s++) {
            jo->xi[s] = s == 0 && kind == 2 ? j : 0;
            jo->yi[s] = s == 0 ? j : 0;
        }
    }
    miss = __syncthreads_or(miss);
    if (tid == 0) {
        for (int kind = 0; kind < 3; kind++) njobs[kind] = miss ? 0 : K;
        if (miss) *missing = 1;
    }
}

// One token's routing by a 256-thread block (logits, biases and the expert
// table staged in LDS), idx/w, and the job lists when a table is given.
template <bool REGS>
__device__ __forceinline__ void route1_block(const float *__restrict__ logits, const float *__restrict__ bias,
                                             int E, int K, int act, int renorm, float routed_scale,
                                             int *__restrict__ idx, float *__restrict__ w,
                                             const warp_slot *__restrict__ table, int table_lds,
                                             warp_job *__restrict__ jobs, int *__restrict__ njobs,
                                             int *__restrict__ missing, int inter) {
    extern __shared__ __attribute__((aligned(16))) float lds_r1[];
    float *score = lds_r1;                                     // [E]
    float *biased = lds_r1 + E;                                // [E]
    warp_slot *slots = (warp_slot *)(lds_r1 + 2 * ((E + 1) & ~1));   // [E] when table_lds
    __shared__ int sel[WARP_MAX_K];
    __shared__ float wsel[WARP_MAX_K];
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += 256) {
        score[e] = logits[e];
        biased[e] = bias ? bias[e] : 0.0f;
    }
    if (table && table_lds)
        for (int e = tid; e < E; e += 256) slots[e] = table[e];
    route_pick_lds<REGS, 256>(E, K, act, renorm, routed_scale, score, biased, sel, wsel);
    if (tid < K) {
        idx[tid] = sel[tid];
        w[tid] = wsel[tid];
    }
    if (table) route_jobs<256>(sel, K, table_lds ? slots : table, jobs, njobs, missing, inter);
}

// One block per token (blockIdx.x); the job lists only for a single token.
template <bool REGS>
__global__ __launch_bounds__(256) void k_route1(const float *__restrict__ logits, const float *__restrict__ bias,
                                                int E, int K, int act, int renorm, float routed_scale,
                                                int *__restrict__ idx, float *__restrict__ w,
                                                const warp_slot *__restrict__ table, int table_lds,
                                                warp_job *__restrict__ jobs, int *__restrict__ njobs,
                                                int *__restrict__ missing, int inter) {
    const size_t t = blockIdx.x;
    route1_block<REGS>(logits + t * E, bias, E, K, act, renorm, routed_scale, idx + t * K, w + t * K, table,
                       table_lds, jobs, njobs, missing, inter);
}

extern "C" int wk_route(const float *logits, const float *bias, int E, int K, int T, int act, int renorm,
                        float routed_scale, int *idx, float *w, const warp_slot *table, warp_job *jobs,
                        int *njobs, int *missing, int inter, void *stream) {
    if (E <= 0 || K <= 0 || K > WARP_MAX_K || K > E || T <= 0 || E > 8192) return -1;
    if (table && T != 1) return -1;
    // one block per token; the table is staged in LDS up to 2048 experts (48 KiB)
    const int tl = table && E <= 2048;
    const size_t lds = (size_t)2 * ((E + 1) & ~1) * sizeof(float) + (tl ? (size_t)E * sizeof(warp_slot) : 0);
    if (E <= 512)
        hipLaunchKernelGGL(k_route1<true>, dim3(T), dim3(256), lds, (hipStream_t)stream, logits, bias, E, K, act,
                           renorm, routed_scale, idx, w, table, tl, jobs, njobs, missing, inter);
    else
        hipLaunchKernelGGL(k_route1<false>, dim3(T), dim3(256), lds, (hipStream_t)stream, logits, bias, E, K, act,
                           renorm, routed_scale, idx, w, table, tl, jobs, njobs, missing, inter);
    CHECK_LAUNCH();
    return 0;
}

// The last router block to finish certifies the selection: it loads the
// four arrays every block wrote, picks as the routing will (the larger
// biased score first, the lower id on ties), tests them (route_cert_wave,
// or cert_check above 512 experts), and where that leaves experts
// ambiguous, recomputes their logits in the reference's sequential order
// and writes their exact score and biased score back (both bounds set to
// the biased score). The routing that follows, from these arrays, picks
// the reference's experts in the reference's order. lds: lds_floats of the
// block's dynamic LDS (cert_last_floats).
template <int NT>
__device__ void cert_last(const float *__restrict__ W, const float *__restrict__ x, int E, int H,
                          const float *__restrict__ bias, float *__restrict__ out, const CertTail &t, float *lds,
                          int lds_floats) {
    __shared__ int cl_last, cl_namb;
    __shared__ unsigned long long cl_amb[8], cl_rows[CERT_EMAX / 64];
    __shared__ int sel[WARP_MAX_K];
    __shared__ float wsel[WARP_MAX_K];
    const int tid = threadIdx.x;
    // The certifying block (one more block, gridDim.x - 1 = E, no row of its
    // own) polls the rows' tagged values (CertTag) and takes each row as
    // soon as its four carry this launch's tag; a wait past CERT_POLLS polls
    // raises bit 2 of the flag (the call reports it) and leaves the arrays
    // uncertified. It then advances the launch counter.
    const CertTag ct = cert_tag(t);
    const int E2 = (E + 1) & ~1, nw = (E + 63) >> 6;
    float *score = lds, *biased = lds + E2, *lo = lds + 2 * E2, *hi = lds + 3 * E2;
    // the expert table, for the job lists, staged while the rows come in;
    // the recompute's buffers after it
    warp_slot *slots = (warp_slot *)(lds + ((4 * E2 + 3) & ~3));
    const int s0 = ((4 * E2 + 3) & ~3) + (t.pk.table ? 6 * E2 : 0);
    if (t.pk.table)
        for (int e = tid; e < E; e += NT) {
            const uint2 *src = (const uint2 *)(t.pk.table + e);
            uint2 *dst = (uint2 *)(slots + e);
            const uint2 a0 = src[0], a1 = src[1], a2 = src[2];
            dst[0] = a0;
            dst[1] = a1;
            dst[2] = a2;
        }
    unsigned pend = 0;                                    // this thread's rows not yet loaded
    for (int i = 0; i < CERT_EMAX / NT; i++)
        if (tid + i * NT < E) pend |= 1u << i;
    if (tid == 0) cl_last = 1;
    for (unsigned n = 0;; n++) {
        for (int i = 0; i < CERT_EMAX / NT; i++) {
            const int e = tid + i * NT;
            if ((pend >> i) & 1u) {
                unsigned long long v[4];
#pragma unroll
                for (int k = 0; k < 4; k++)
                    v[k] = __hip_atomic_load(ct.tg + 4 * (size_t)e + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if ((unsigned)(v[0] >> 32) == ct.tag && (unsigned)(v[1] >> 32) == ct.tag &&
                    (unsigned)(v[2] >> 32) == ct.tag && (unsigned)(v[3] >> 32) == ct.tag) {
                    score[e] = __uint_as_float((unsigned)v[0]);
                    biased[e] = __uint_as_float((unsigned)v[1]);
                    lo[e] = __uint_as_float((unsigned)v[2]);
                    hi[e] = __uint_as_float((unsigned)v[3]);
                    pend &= ~(1u << i);
                }
            }
        }
        if (__syncthreads_and(pend == 0)) break;          // uniform
        if (n >= (t.polls ? t.polls : CERT_POLLS)) {
            if (tid == 0) cl_last = 0;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    __syncthreads();
    if (tid == 0) __hip_atomic_store(t.sync, ct.tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // the next launch's
    if (!cl_last) {                                       // (never in practice)
        if (tid == 0 && t.flag) __hip_atomic_fetch_or(t.flag, 4, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // empty job lists: the launches after this one skip their work (and
        // the combine, seeing the flag, writes NaN) rather than read the
        // lists a previous launch left
        if (t.pk.idx && t.pk.table) {
            for (int i = tid; i < 3 * t.K; i += NT) {
                warp_job *jo = t.pk.jobs + i;
                jo->idx = nullptr;
                jo->scale = nullptr;
                jo->n = 0;
            }
            if (tid < 3) t.pk.njobs[tid] = 0;
        }
        return;
    }
    warp_route_args r = {};
    r.bias = bias;
    r.E = E;
    r.cw = W;
    r.cx = x;
    r.ch = H;
    r.cctr = t.cctr;
    unsigned long long *amb = cl_amb;
    const warp_route_args &pk = t.pk;
    const bool want = pk.idx != nullptr;                  // the routing's outputs too (its weights)
    // pass 0 picks and tests; where it recomputed rows, pass 1 picks again
    // from the exact values, for the routing's outputs (one call site per
    // picking kernel: the block's registers are the row blocks' too)
#pragma nounroll
    for (int pass = 0; pass < 2; pass++) {
        int n;
        if (E <= 512) {
            route_pick_lds<true, NT>(E, t.K, 0, pk.renorm, pk.routed_scale, score, biased, sel, wsel, want, true,
                                     nullptr, pass ? nullptr : lo, hi, cl_amb, &cl_namb);
            n = pass ? 0 : cl_namb;
        } else {
            const int np = route_pick_lds<false, NT>(E, t.K, 0, pk.renorm, pk.routed_scale, score, biased, sel, wsel,
                                                     want, true);
            n = pass ? 0 : cert_check<NT, CERT_EMAX / 64>(r, E, np, score, biased, lo, hi, sel, false, amb);
        }
        if (!n) break;                                    // uniform
        cert_count(r, n);
        for (int i = tid; i < nw; i += NT) cl_rows[i] = amb[i];   // (the recompute consumes amb)
        __syncthreads();
        cert_recompute<NT>(r, score, biased, amb, nw, lds + s0, lds_floats - s0, nullptr);
        for (int e = tid; e < E; e += NT)
            if ((cl_rows[e >> 6] >> (e & 63)) & 1ull) {
                out[e] = score[e];
                out[E + e] = biased[e];
                out[2 * E + e] = biased[e];
                out[3 * E + e] = biased[e];
            }
        if (!want) return;                                // uniform
    }
    if (!want) return;                                    // uniform
    // the routing of these arrays, as wk_route does it (route1_block): the
    // picks and weights, and the job lists
    if (tid < t.K) {
        pk.idx[tid] = sel[tid];
        pk.w[tid] = wsel[tid];
    }
    if (pk.table) route_jobs<NT>(sel, t.K, slots, pk.jobs, pk.njobs, t.flag, pk.inter);
}

// Certified routing of one token by a CERT_NT-thread block: the four arrays of
// k_router_cert, the picks, cert_resolve, the picks again where it
// recomputed; idx/w, and the job lists when a table is given. LDS: scores,
// biased scores, bounds [4][E2], the table when table_lds, then the
// recompute buffer (cap floats).
constexpr int CERT_NT = 1024;                // threads of the certified routing block
template <bool REGS>
__global__ __launch_bounds__(CERT_NT) void k_route_cert(warp_route_args r, int K, int table_lds, int cap) {
    extern __shared__ __attribute__((aligned(16))) float lds_rc[];
    const int E = r.E, E2 = (E + 1) & ~1;
    float *score = lds_rc, *biased = lds_rc + E2, *lo = lds_rc + 2 * E2, *hi = lds_rc + 3 * E2;
    warp_slot *slots = (warp_slot *)(lds_rc + 4 * E2);
    float *stg = lds_rc + ((4 * E2 + (table_lds ? 6 * E2 : 0) + 3) & ~3);
    __shared__ int sel[WARP_MAX_K];
    __shared__ float wsel[WARP_MAX_K];
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += CERT_NT) {
        score[e] = r.logits[e];
        biased[e] = r.logits[E + e];
        lo[e] = r.logits[2 * E + e];
        hi[e] = r.logits[3 * E + e];
    }
    if (r.table && table_lds)
        for (int e = tid; e < E; e += CERT_NT) slots[e] = r.table[e];
    __shared__ unsigned long long r_amb[8];
    __shared__ int r_namb;
    const int np = route_pick_lds<REGS, CERT_NT>(E, K, r.act, r.renorm, r.routed_scale, score, biased, sel, wsel, true,
                                             true, nullptr, REGS ? lo : nullptr, hi, r_amb, &r_namb);
    unsigned long long *amb = r_amb;
    int n_amb;
    if (REGS) {
        n_amb = r_namb;
        if (n_amb) cert_count(r, n_amb);
    } else {
        // (above 512 experts: the block's test; the picking loop took the
        // picks' biased scores out, and the test puts them back)
        n_amb = cert_check<CERT_NT, CERT_EMAX / 64>(r, E, np, score, biased, lo, hi, sel, true, amb);
    }
    if (n_amb) {                                           // uniform
        cert_recompute<CERT_NT>(r, score, biased, amb, (E + 63) >> 6, stg, cap, nullptr);
        route_pick_lds<REGS, CERT_NT>(E, K, r.act, r.renorm, r.routed_scale, score, biased, sel, wsel, true, true);
    }
    if (tid < K) {
        r.idx[tid] = sel[tid];
        r.w[tid] = wsel[tid];
    }
    if (r.table) route_jobs<CERT_NT>(sel, K, table_lds ? slots : r.table, r.jobs, r.njobs, r.missing, r.inter);
}

extern "C" int wk_route_cert(const warp_route_args *r, int K, void *stream) {
    if (!r || r->scored != 2 || r->act != 0 || !r->cw || !r->cx || r->ch <= 0 || (r->ch & 3))
        return -1;
    const int E = r->E;
    if (E <= 0 || E > CERT_EMAX || K <= 0 || K > WARP_MAX_K || K > E) return -1;
    const int E2 = (E + 1) & ~1, tl = r->table && E <= 2048;
    const int cap = 16384;                                  // 64 KiB: a row's products up to H = 15360
    const size_t lds = (size_t)(((4 * E2 + (tl ? 6 * E2 : 0) + 3) & ~3) + cap) * sizeof(float);
    if (lds > 160 * 1024) return -1;
    if (E <= 512) {
        static std::atomic<uint64_t> attr{0};
        if (int r_ = lds_limit((const void *)k_route_cert<true>, (int)lds, attr, stream)) return r_;
        hipLaunchKernelGGL(k_route_cert<true>, dim3(1), dim3(CERT_NT), lds, (hipStream_t)stream, *r, K, tl, cap);
    } else {
        static std::atomic<uint64_t> attr{0};
        if (int r_ = lds_limit((const void *)k_route_cert<false>, (int)lds, attr, stream)) return r_;
        hipLaunchKernelGGL(k_route_cert<false>, dim3(1), dim3(CERT_NT), lds, (hipStream_t)stream, *r, K, tl, cap);
    }
    CHECK_LAUNCH();
    return 0;
}

// ---- the MFMA expert matvec --------------------------------------------------------------

template <int FMT> struct FmtT;
template <> struct FmtT<WARP_FMT_VQ3R> { static constexpr int S = 3, E = 256, SB = 3; };
template <> struct FmtT<WARP_FMT_VQ2R> { static constexpr int S = 2, E = 256, SB = 2; };
template <> struct FmtT<WARP_FMT_VQ12> { static constexpr int S = 2, E = 4096, SB = 3; };

// Device memory seen as global (not generic) memory, so that loads through
// pointers read from job lists are global loads.
typedef const __attribute__((address_space(1))) unsigned gu32;

// Code word of 4 consecutive rows at one position, as loaded by a lane.
template <int SB> struct Word;
template <> struct Word<3> {
    u3v w;
    __device__ __forceinline__ void load(const uint8_t *p) {
        const unsigned *q = (const unsigned *)p;
        w = u3v{__builtin_nontemporal_load(q), __builtin_nontemporal_load(q + 1), __builtin_nontemporal_load(q + 2)};
    }
    __device__ __forceinline__ void load_keep(const uint8_t *p) {
        const gu32 *q = (const gu32 *)p;
        w = u3v{q[0], q[1], q[2]};
    }
    __device__ __forceinline__ void mask(unsigned m) { w = u3v{w.x & m, w.y & m, w.z & m}; }
    // 24-bit slot of row t (0..3)
    __device__ __forceinline__ unsigned slot(int t) const {
        switch (t) {
        case 0: return w.x & 0xFFFFFFu;
        case 1: return __builtin_amdgcn_alignbit(w.y, w.x, 24) & 0xFFFFFFu;
        case 2: return __builtin_amdgcn_alignbit(w.z, w.y, 16) & 0xFFFFFFu;
        default: return w.z >> 8;
        }
    }
};
template <> struct Word<2> {
    u2v w;
    __device__ __forceinline__ void load(const uint8_t *p) {
        const unsigned *q = (const unsigned *)p;
        w = u2v{__builtin_nontemporal_load(q), __builtin_nontemporal_load(q + 1)};
    }
    __device__ __forceinline__ void load_keep(const uint8_t *p) {
        const gu32 *q = (const gu32 *)p;
        w = u2v{q[0], q[1]};
    }
    __device__ __forceinline__ void mask(unsigned m) { w = u2v{w.x & m, w.y & m}; }
    __device__ __forceinline__ unsigned slot(int t) const {
        switch (t) {
        case 0: return w.x & 0xFFFFu;
        case 1: return w.x >> 16;
        case 2: return w.y & 0xFFFFu;
        default: return w.y >> 16;
        }
    }
};

// Byte offset in LDS of the codebook vector for (stage, code of this slot).
template <int FMT>
__device__ __forceinline__ unsigned cb_off(unsigned slot, int s) {
    if (FMT == WARP_FMT_VQ12) {
        const unsigned c = s == 0 ? (slot & 0xFFFu) : (slot >> 12);
        return ((unsigned)s * 4096u + c) * 16u;
    }
    const unsigned c = (slot >> (8 * s)) & 0xFFu;
    return ((unsigned)s * 256u + c) * 16u;
}

struct VqArgs {
    const warp_job *jobs;
    const int *njobs;
    int max_jobs;
    int kind_lo;
    const uint16_t *books;      // [3][S][E][8] fp16
    const _Float16 *xs;         // [nx][nv][2][8]
    const float *xscale;        // [nx]
    float *y[3];                // per kind: [ny][M]
    int M, N;
    int xrows;                  // reduced-precision kernel: xs is [N/32][xrows][32] fp16
    unsigned *queue;            // run kernels: per kind, a ticket and a waves-done counter
};

// Units of the run kernels are dealt in chunks of NW consecutive units (a
// block's waves) to RQ_GROUPS queues, one per XCD (blocks go to the XCDs
// round-robin, which matters only for speed: the queues are correct
// wherever the blocks run; the grid is a multiple of RQ_GROUPS): queue g holds
// chunks g, g + 8, g + 16, ... and serves blocks g, g + 8, .... A wave's
// first unit is its block's own chunk (block b, wave w: unit b NW + w);
// after each unit it takes a ticket from its queue, so a wave that finishes
// early takes the next unit of its queue, and the last, partial round
// spreads over the CUs instead of falling on the waves of the first blocks.
// A queue per XCD keeps the atomics off one address (a single counter
// serialised them: 130 us more per layer of 512 tokens). Each unit writes
// only its own outputs, so which wave runs it changes no result bit. Queue
// (kind k, group g) is a ticket counter at line 2 (RQ_GROUPS k + g)
// (RQ_LINE words a line) and a waves-done counter on the next line; the
// last wave of the group out clears both, so every launch (graph replays
// included) starts from zero without a memset.
constexpr int RQ_LINE = 32, RQ_GROUPS = 8;

struct RunQueue {
    unsigned *q;                // the ticket counter; waves done one line on
    int n;                      // units of this queue
    int nwaves;                 // waves of this queue's blocks
};

template <int NW> __device__ __forceinline__ RunQueue rq_open(unsigned *base, int kind, int units) {
    constexpr int span = NW * RQ_GROUPS;
    const int g = blockIdx.x % RQ_GROUPS;
    RunQueue r;
    r.n = (units / span) * NW + min(max(units % span - g * NW, 0), NW);
    r.nwaves = (int)(gridDim.x / RQ_GROUPS) * NW;
    r.q = base + 2 * (kind * RQ_GROUPS + g) * RQ_LINE;
    return r;
}

// this block's first local index, and local index l of its queue -> unit
template <int NW> __device__ __forceinline__ int rq_first() { return (int)(blockIdx.x / RQ_GROUPS) * NW; }
template <int NW> __device__ __forceinline__ int rq_unit(int l) {
    return (l / NW) * NW * RQ_GROUPS + (int)(blockIdx.x % RQ_GROUPS) * NW + l % NW;
}

__device__ __forceinline__ int rq_take(const RunQueue &r, int lane) {
    unsigned t = 0;
    if (lane == 0) t = __hip_atomic_fetch_add(r.q, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return r.nwaves + __builtin_amdgcn_readfirstlane((int)t);
}

// n waves leave (a block that had no unit leaves as one): each wave's
// ticket past the end has returned before it leaves, so the last one out
// clears both counters
__device__ __forceinline__ void rq_leave(const RunQueue &r, int lane, unsigned n) {
    if (lane == 0) {
        unsigned *done = r.q + RQ_LINE;
        const unsigned old = __hip_atomic_fetch_add(done, n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old + n == (unsigned)r.nwaves) {
            __hip_atomic_store(r.q, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <int FMT, int SB>
__device__ __forceinline__ void gather_group(const unsigned char *lds, const Word<SB> &wd, half8 (&a)[4][FmtT<FMT>::S]) {
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const unsigned sl = wd.slot(t);
#pragma unroll
        for (int s = 0; s < FmtT<FMT>::S; s++) a[t][s] = *(const half8 *)(lds + cb_off<FMT>(sl, s));
    }
}

template <int FMT, int TPJ, int WPU, int DB, int VQ_NW, int VQ_D>
__global__ __launch_bounds__(VQ_NW * 64) void k_vq_mfma(VqArgs a) {
    typedef FmtT<FMT> F;
    constexpr int UPW = VQ_NW / WPU;
    extern __shared__ __attribute__((aligned(16))) unsigned char lds_vq[];
    const int kind = a.kind_lo + blockIdx.y;
    const int nj = a.njobs[kind];
    const warp_job *jobs = a.jobs + (size_t)kind * a.max_jobs;
    const int M = a.M, N = a.N, nv = N >> 3, npg = nv >> 2, nrb = (M + 63) >> 6;
    const int units = nj * nrb;
    if ((int)(blockIdx.x * UPW) >= units) return;   // uniform per block

    // codebook of this kind -> LDS
    {
        const uint4 *src = (const uint4 *)(a.books + (size_t)kind * F::S * F::E * 8);
        uint4 *dst = (uint4 *)lds_vq;
        for (int i = threadIdx.x; i < F::S * F::E; i += blockDim.x) dst[i] = src[i];
    }
    float *red = (float *)(lds_vq + (size_t)F::S * F::E * 16);   // [VQ_NW][TPJ][64]
    __syncthreads();

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, jc = lane & 15;
    const int sub = wave / WPU, part = wave % WPU;
    const int pg0 = part * npg / WPU, pg1 = (part + 1) * npg / WPU;
    const int ts = jc >> 1, hl = jc & 1;

    for (int ub = blockIdx.x * UPW; ub < units; ub += gridDim.x * UPW) {
        const int u = ub + sub;
        f4 acc[4];
#pragma unroll
        for (int t = 0; t < 4; t++) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
        if (u < units && pg0 < pg1) {
            const warp_job &jb = jobs[u / nrb];
            const int rb = u % nrb;
            const uint8_t *cp = jb.idx + ((size_t)rb * nv) * 64 * F::SB + (size_t)lane * 4 * F::SB;
            const bool bvalid = ts < jb.n && ts < TPJ;
            const _Float16 *xrow = a.xs + (size_t)(bvalid ? jb.xi[ts] : 0) * nv * 16 + hl * 8 + (size_t)g * 16;
            Word<F::SB> buf[VQ_D];
            half8 bb[VQ_D];
#pragma unroll
            for (int k = 0; k < VQ_D; k++) {
                bb[k] = half8{0, 0, 0, 0, 0, 0, 0, 0};
                if (pg0 + k < pg1) {
                    buf[k].load(cp + (size_t)(pg0 + k) * 256 * F::SB);
                    if (bvalid) bb[k] = *(const half8 *)(xrow + (size_t)(pg0 + k) * 64);
                }
            }
            if (DB) {
                // A operands double-buffered across groups
                half8 av[2][4][F::S];
                gather_group<FMT, F::SB>(lds_vq, buf[0], av[0]);
                for (int pgb = pg0; pgb < pg1; pgb += VQ_D) {
#pragma unroll
                    for (int k = 0; k < VQ_D; k++) {
                        const int pg = pgb + k;
                        if (pg < pg1) {
                            const half8 b = bb[k];
                            const int cur = k & 1;
                            // the next group's gathers go out before this group's MFMAs
                            if (pg + 1 < pg1) gather_group<FMT, F::SB>(lds_vq, buf[(k + 1) % VQ_D], av[cur ^ 1]);
                            if (pg + VQ_D < pg1) {
                                buf[k].load(cp + (size_t)(pg + VQ_D) * 256 * F::SB);
                                if (bvalid) bb[k] = *(const half8 *)(xrow + (size_t)(pg + VQ_D) * 64);
                            }
#pragma unroll
                            for (int t = 0; t < 4; t++)
#pragma unroll
                                for (int s = 0; s < F::S; s++)
                                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[cur][t][s], b, acc[t], 0, 0, 0);
                        }
                    }
                }
            } else {
                for (int pgb = pg0; pgb < pg1; pgb += VQ_D) {
#pragma unroll
                    for (int k = 0; k < VQ_D; k++) {
                        const int pg = pgb + k;
                        if (pg < pg1) {
                            const Word<F::SB> wd = buf[k];
                            const half8 b = bb[k];
                            if (pg + VQ_D < pg1) {
                                buf[k].load(cp + (size_t)(pg + VQ_D) * 256 * F::SB);
                                if (bvalid) bb[k] = *(const half8 *)(xrow + (size_t)(pg + VQ_D) * 64);
                            }
                            half8 av[4][F::S];
                            gather_group<FMT, F::SB>(lds_vq, wd, av);
#pragma unroll
                            for (int t = 0; t < 4; t++)
#pragma unroll
                                for (int s = 0; s < F::S; s++)
                                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[t][s], b, acc[t], 0, 0, 0);
                        }
                    }
                }
            }
        }
        // lane (g, jc) holds C[4g + r][jc] of tile t, i.e. block row 16g + 4r + t,
        // token slot jc/2, half jc%2: fold the halves, park per-wave partials.
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float v = acc[t][r] + __shfl_xor(acc[t][r], 1);
                if (hl == 0 && ts < TPJ) red[(wave * TPJ + ts) * 64 + 16 * g + 4 * r + t] = v;
            }
        __syncthreads();
        for (int q = threadIdx.x; q < UPW * TPJ * 64; q += blockDim.x) {
            const int s = q / (TPJ * 64), tsl = (q / 64) % TPJ, row = q % 64;
            const int uu = ub + s;
            if (uu >= units) continue;
            const warp_job &jb = jobs[uu / nrb];
            const int rg = (uu % nrb) * 64 + row;
            if (tsl >= jb.n || rg >= M) continue;
            float v = 0.0f;
            for (int p = 0; p < WPU; p++) v += red[((s * WPU + p) * TPJ + tsl) * 64 + row];
            v = (v * a.xscale[jb.xi[tsl]]) * f16_keep(jb.scale[rg]);
            a.y[kind][(size_t)jb.yi[tsl] * M + rg] = v;
        }
        __syncthreads();
    }
}

template <int FMT, int TPJ, int WPU, int DB, int NW, int D>
static int launch_vq(const VqArgs &a, int nkinds, int max_units, void *stream) {
    typedef FmtT<FMT> F;
    constexpr int UPW = NW / WPU;
    const size_t lds = (size_t)F::S * F::E * 16 + (size_t)NW * TPJ * 64 * 4;
    if (lds > 163840) return -2;
    static std::atomic<uint64_t> attr{0};
    if (int r_ = lds_limit((const void *)k_vq_mfma<FMT, TPJ, WPU, DB, NW, D>, (int)lds, attr, stream)) return r_;
    int grid = (max_units + UPW - 1) / UPW;
    const int cap = FMT == WARP_FMT_VQ12 ? 256 : 512;
    if (grid > cap) grid = cap;
    if (grid < 1) grid = 1;
    hipLaunchKernelGGL((k_vq_mfma<FMT, TPJ, WPU, DB, NW, D>), dim3(grid, nkinds), dim3(NW * 64), lds,
                       (hipStream_t)stream, a);
    CHECK_LAUNCH();
    return 0;
}

// Waves per unit: up to 4 waves share a unit (four units per 16-wave block,
// which keeps the 64-row units of one launch spread over every CU), fewer
// when a wave would get under 16 position groups. WARP_VQ_WPU overrides it.
static int env_int(const char *name, int dflt) {
    const char *e = getenv(name);
    return e ? atoi(e) : dflt;
}

static int choose_wpu(int npg, int nw) {
    const int forced = env_int("WARP_VQ_WPU", 0);
    if ((forced == 1 || forced == 2 || forced == 4 || forced == 8 || forced == 16) && forced <= nw) return forced;
    int w = nw < 4 ? nw : 4;
    while (w > 1 && npg / w < 16) w >>= 1;
    return w;
}

template <int FMT, int TPJ, int NW, int DB, int D>
static int launch_vq_s(const VqArgs &a, int nkinds, int max_units, int npg, void *stream) {
    switch (choose_wpu(npg, NW)) {
    case 16: return launch_vq<FMT, TPJ, (NW >= 16 ? 16 : NW), DB, NW, D>(a, nkinds, max_units, stream);
    case 8: return launch_vq<FMT, TPJ, 8, DB, NW, D>(a, nkinds, max_units, stream);
    case 4: return launch_vq<FMT, TPJ, 4, DB, NW, D>(a, nkinds, max_units, stream);
    case 2: return launch_vq<FMT, TPJ, 2, DB, NW, D>(a, nkinds, max_units, stream);
    }
    return launch_vq<FMT, TPJ, 1, DB, NW, D>(a, nkinds, max_units, stream);
}

// Kernel shape: 16 waves per block with the next group's codebook gathers
// issued before the current group's MFMAs and 2 code words in flight (the
// fastest measured on gfx950 for the K3 shapes); WARP_VQ_SHAPE=0 selects
// single-buffered gathers with 4 code words in flight.
template <int FMT, int TPJ>
static int launch_vq_w(const VqArgs &a, int nkinds, int max_units, int npg, void *stream) {
    static int shape = -1;
    if (shape < 0) shape = env_int("WARP_VQ_SHAPE", 1);
    if (shape == 0) return launch_vq_s<FMT, TPJ, 16, 0, 4>(a, nkinds, max_units, npg, stream);
    return launch_vq_s<FMT, TPJ, 16, 1, 2>(a, nkinds, max_units, npg, stream);
}

template <int FMT>
static int launch_vq_t(const VqArgs &a, int nkinds, int max_units, int npg, int tpj, void *stream) {
    if (tpj == 1) return launch_vq_w<FMT, 1>(a, nkinds, max_units, npg, stream);
    return launch_vq_w<FMT, WARP_TPJ>(a, nkinds, max_units, npg, stream);
}

// Prefill by runs: one wave per (run, 64-row block), a run being up to
// WARP_RUN_J consecutive jobs of one expert (up to 32 of its tokens, from
// the grouping's run list; njobs[3] runs). The wave gathers the expert's
// codebook vectors (the A operands) once per position group and multiplies
// them with the B operands of every job of the run, so a busy expert's
// records are decoded once per 32 tokens instead of once per 8; only the
// run's own jobs are multiplied. No split over positions: the wave walks
// all of a unit's positions, the next group's gathers issued before the
// current group's MFMAs, then writes its rows (8 waves per block, so each
// holds 4 x 4 accumulator tiles). Code words stream from HBM WD groups
// ahead (8 waves per CU need that many bytes in flight); the B operands
// come from L2, BD groups ahead.
template <int FMT, int WD>
__global__ __launch_bounds__(512) void k_vq_mfma_run(VqArgs a, const int *__restrict__ runs) {
    typedef FmtT<FMT> F;
    constexpr int RJ = WARP_RUN_J;
    extern __shared__ __attribute__((aligned(16))) unsigned char lds_vq[];
    const int kind = a.kind_lo + blockIdx.y;
    const warp_job *jobs = a.jobs + (size_t)kind * a.max_jobs;
    const int M = a.M, N = a.N, nv = N >> 3, npg = nv >> 2, nrb = (M + 63) >> 6;
    const RunQueue rq = rq_open<8>(a.queue, kind, a.njobs[3] * nrb);
    if (rq_first<8>() >= rq.n) {                    // uniform per block
        rq_leave(rq, threadIdx.x, 8);
        return;
    }
    {
        const uint4 *src = (const uint4 *)(a.books + (size_t)kind * F::S * F::E * 8);
        uint4 *dst = (uint4 *)lds_vq;
        for (int i = threadIdx.x; i < F::S * F::E; i += blockDim.x) dst[i] = src[i];
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, jc = lane & 15, ts = jc >> 1, hl = jc & 1;
    for (int l = rq_first<8>() + wave; l < rq.n;) {
        const int u = rq_unit<8>(l);
        const int rv = __builtin_amdgcn_readfirstlane(runs[u / nrb]);   // uniform: u is
        const int j0 = rv >> 3, nt = rv & 7, rb = u % nrb;
        const uint8_t *cp = jobs[j0].idx + ((size_t)rb * nv) * 64 * F::SB + (size_t)lane * 4 * F::SB;
        // B operands of every job of the run; a slot past a job's tokens
        // points at one of its tokens (the grouping fills every slot), so
        // every load is unconditional: its column of the product is not
        // written out. Loads without branches keep the wait counts exact.
        const _Float16 *xrow[RJ];
#pragma unroll
        for (int q = 0; q < RJ; q++)
            xrow[q] = a.xs + (size_t)jobs[j0 + min(q, nt - 1)].xi[ts] * nv * 16 + hl * 8 + (size_t)g * 16;
        f4 acc[RJ][4];
#pragma unroll
        for (int q = 0; q < RJ; q++)
#pragma unroll
            for (int t = 0; t < 4; t++) acc[q][t] = f4{0.f, 0.f, 0.f, 0.f};
        constexpr int BD = 2;
        Word<F::SB> buf[WD];
        half8 bb[BD][RJ];
#pragma unroll
        for (int k = 0; k < WD; k++) buf[k].load_keep(cp + (size_t)min(k, npg - 1) * 256 * F::SB);
#pragma unroll
        for (int k = 0; k < BD; k++)
#pragma unroll
            for (int q = 0; q < RJ; q++) bb[k][q] = *(const half8 *)(xrow[q] + (size_t)min(k, npg - 1) * 64);
        half8 av[2][4][F::S];
        gather_group<FMT, F::SB>(lds_vq, buf[0], av[0]);
        // one position group: the next group's gathers, the loads WD (code
        // words) and BD (B) groups ahead, clamped to the last group, then
        // this group's MFMAs
        auto step = [&](int k, int pg) {
            const int cur = k & 1;                            // = pg & 1: WD is even
            half8 b[RJ];
#pragma unroll
            for (int q = 0; q < RJ; q++) b[q] = bb[k % BD][q];
            gather_group<FMT, F::SB>(lds_vq, buf[(k + 1) % WD], av[cur ^ 1]);
            buf[k].load_keep(cp + (size_t)min(pg + WD, npg - 1) * 256 * F::SB);
#pragma unroll
            for (int q = 0; q < RJ; q++) bb[k % BD][q] = *(const half8 *)(xrow[q] + (size_t)min(pg + BD, npg - 1) * 64);
            // stage-major: the 4 row tiles' chains interleave, no MFMA waits on the previous one
#pragma unroll
            for (int q = 0; q < RJ; q++)
                if (q < nt)                                   // uniform
#pragma unroll
                    for (int s = 0; s < F::S; s++)
#pragma unroll
                        for (int t = 0; t < 4; t++)
                            acc[q][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[cur][t][s], b[q], acc[q][t], 0, 0, 0);
        };
        const int npg_full = npg - npg % WD;
        for (int pgb = 0; pgb < npg_full; pgb += WD) {
#pragma unroll
            for (int k = 0; k < WD; k++) step(k, pgb + k);
        }
#pragma unroll
        for (int k = 0; k < WD; k++)
            if (npg_full + k < npg) step(k, npg_full + k);    // uniform
        l = rq_take(rq, lane);                                // returns while the outputs are stored
        // lane (g, jc) holds C[4g + r][jc] of row tile t: block row 16g + 4r + t,
        // token slot jc / 2 of the job, half jc % 2 -- the 16 consecutive rows
        // 16g .. 16g + 15, stored as four 16-byte runs
#pragma unroll
        for (int q = 0; q < RJ; q++) {
            if (q >= nt) break;                               // uniform
            const warp_job &jq = jobs[j0 + q];
            const bool tv = hl == 0 && ts < jq.n;
            const float xsc = tv ? a.xscale[jq.xi[ts]] : 0.0f;
            const int yrow = tv ? jq.yi[ts] : 0;
            float *yo = a.y[kind] + (size_t)yrow * M;
            if ((M & 63) == 0) {                              // uniform: whole 64-row blocks
                // the same 4 x 4 transpose as the reduced-precision kernel's:
                // store k writes rows 16k .. 16k + 15 as one 64-byte sector
                float w[4][4];
                auto pick = [](const float *u, int i) { return i == 0 ? u[0] : i == 1 ? u[1] : i == 2 ? u[2] : u[3]; };
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    float v[4];                               // rows 16 g + 4 r + t
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        v[r] = ((acc[q][t][r] + __shfl_xor(acc[q][t][r], 1)) * xsc) *
                               f16_keep(jq.scale[rb * 64 + 16 * g + 4 * r + t]);
#pragma unroll
                    for (int d = 0; d < 4; d++) {
                        const float sv = pick(v, g ^ d);
                        w[d][t] = d == 0 ? sv : __shfl_xor(sv, 16 * d);
                    }
                }
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int d = g ^ k;
                    const float4 o = make_float4(d == 0 ? w[0][0] : d == 1 ? w[1][0] : d == 2 ? w[2][0] : w[3][0],
                                                 d == 0 ? w[0][1] : d == 1 ? w[1][1] : d == 2 ? w[2][1] : w[3][1],
                                                 d == 0 ? w[0][2] : d == 1 ? w[1][2] : d == 2 ? w[2][2] : w[3][2],
                                                 d == 0 ? w[0][3] : d == 1 ? w[1][3] : d == 2 ? w[2][3] : w[3][3]);
                    if (tv) *(float4 *)(yo + rb * 64 + 16 * k + 4 * g) = o;
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++)
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        const float v = acc[q][t][r] + __shfl_xor(acc[q][t][r], 1);
                        const int row = rb * 64 + 16 * g + 4 * r + t;
                        if (tv && row < M) yo[row] = (v * xsc) * f16_keep(jq.scale[row]);
                    }
            }
        }
    }
    rq_leave(rq, lane, 1);
}

template <int FMT>
static int launch_vq_run(const VqArgs &a, const int *runs, int nkinds, int max_units, void *stream) {
    typedef FmtT<FMT> F;
    constexpr int WD = F::S == 3 ? 2 : 8;                   // three stages leave room for fewer words
    const size_t lds = (size_t)F::S * F::E * 16;
    static std::atomic<uint64_t> attr{0};
    if (int r_ = lds_limit((const void *)k_vq_mfma_run<FMT, WD>, (int)lds, attr, stream)) return r_;
    int grid = (max_units + 7) / 8;
    const int cap = FMT == WARP_FMT_VQ12 ? 256 : 1024;
    if (grid > cap) grid = cap;
    grid = (grid + RQ_GROUPS - 1) / RQ_GROUPS * RQ_GROUPS;   // the unit queues' groups
    hipLaunchKernelGGL((k_vq_mfma_run<FMT, WD>), dim3(grid, nkinds), dim3(512), lds, (hipStream_t)stream, a, runs);
    CHECK_LAUNCH();
    return 0;
}

// A chunk's reduced-precision mode, by runs as above: the stages' codebook
// vectors of a position are added into one fp16 A operand (v_pk_add_f16,
// each addition rounded once) and B holds only the fp16 hi halves of x, 16
// tokens (two jobs) per MFMA, so a position group takes a quarter of the
// exact kernel's MFMAs: products of fp16 values accumulated in fp32. With
// that few MFMAs the loop is bound by issue and latency, so a block holds
// 16 waves (4 per SIMD, each within 128 VGPRs): the gathers are single-
// buffered (the other waves cover their latency), and the code words and B
// operands are both loaded WD groups ahead. Vector loads retire in issue
// order, so B loaded nearer than the code words would hold the code words
// to its own depth.
// Buffer descriptor word 3 for gfx9 raw buffers (32-bit data format, no
// swizzle); records up to 4 GiB.
constexpr int BUF_RSRC_W3 = 0x00020000;

template <int SB> __device__ __forceinline__ void word_load(Word<SB> &w, __amdgpu_buffer_rsrc_t r, unsigned vo, int so);
template <> __device__ __forceinline__ void word_load<3>(Word<3> &w, __amdgpu_buffer_rsrc_t r, unsigned vo, int so) {
    w.w = __builtin_bit_cast(u3v, __builtin_amdgcn_raw_buffer_load_b96(r, vo, so, 0));
}
template <> __device__ __forceinline__ void word_load<2>(Word<2> &w, __amdgpu_buffer_rsrc_t r, unsigned vo, int so) {
    w.w = __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(r, vo, so, 0));
}

template <int FMT, int WD>
__global__ __launch_bounds__(1024) void k_vq_run_f16(VqArgs a, const int *__restrict__ runs) {
    typedef FmtT<FMT> F;
    constexpr int NWB = 16, RB = WARP_RUN_J / 2;            // waves per block; B operands (2 jobs each) per step
    // the codebook at a fixed LDS address, so the gathers' addresses need no base
    __shared__ uint4 cb_lds[F::S * F::E];
    const unsigned char *lds_vq = (const unsigned char *)cb_lds;
    const int kind = a.kind_lo + blockIdx.y;
    const warp_job *jobs = a.jobs + (size_t)kind * a.max_jobs;
    const int M = a.M, N = a.N, nv = N >> 3, npg = nv >> 2, nrb = (M + 63) >> 6;
    const RunQueue rq = rq_open<NWB>(a.queue, kind, a.njobs[3] * nrb);
    if (rq_first<NWB>() >= rq.n) {                  // uniform per block
        rq_leave(rq, threadIdx.x, NWB);
        return;
    }
    {
        const uint4 *src = (const uint4 *)(a.books + (size_t)kind * F::S * F::E * 8);
        for (int i = threadIdx.x; i < F::S * F::E; i += blockDim.x) cb_lds[i] = src[i];
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, jc = lane & 15;
    // B and the code words through buffer loads: a per-lane offset fixed for
    // the unit and a per-group offset in a scalar register
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void *)a.xs, 0, -1, BUF_RSRC_W3);
    const int pgb_x = a.xrows * 64;                          // bytes per position group of xs
    for (int l = rq_first<NWB>() + wave; l < rq.n;) {
        const int u = rq_unit<NWB>(l);
        const int rv = __builtin_amdgcn_readfirstlane(runs[u / nrb]);   // uniform: u is
        const int j0 = rv >> 3, nt = rv & 7, rb = u % nrb;
        // the unit's code words (uniform: the descriptor lives in scalar registers)
        const uint64_t cba = (uint64_t)(uintptr_t)(jobs[j0].idx + ((size_t)rb * nv) * 64 * F::SB);
        // (readfirstlane returns int: each half goes through unsigned, so the
        // low half is not sign-extended into the high one)
        const uint64_t cbu = ((uint64_t)(unsigned)__builtin_amdgcn_readfirstlane((unsigned)(cba >> 32)) << 32) |
                             (uint64_t)(unsigned)__builtin_amdgcn_readfirstlane((unsigned)cba);
        const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc((void *)(uintptr_t)cbu, 0, -1, BUF_RSRC_W3);
        const unsigned co = (unsigned)lane * 4 * F::SB;
        // B column jc: pair slot jc % 8 of job 2 q + jc / 8 (xs holds the
        // inputs by pair slot, position-group-major, so a run's slots are
        // contiguous); a column past the run's jobs or a job's tokens points
        // at a slot of the run (the grouping fills every slot), so the loads
        // are unconditional and the column is not written out
        unsigned xo[RB];
#pragma unroll
        for (int q = 0; q < RB; q++)
            xo[q] = (unsigned)jobs[j0 + min(2 * q + (jc >> 3), nt - 1)].yi[jc & 7] * 64 + (unsigned)g * 16;
        f4 acc[RB][4];
#pragma unroll
        for (int q = 0; q < RB; q++)
#pragma unroll
            for (int t = 0; t < 4; t++) acc[q][t] = f4{0.f, 0.f, 0.f, 0.f};
        Word<F::SB> buf[WD];
        half8 bb[WD][RB];
#pragma unroll
        for (int k = 0; k < WD; k++) {
            const int pk = min(k, npg - 1);
            word_load<F::SB>(buf[k], cr, co, pk * 256 * F::SB);
#pragma unroll
            for (int q = 0; q < RB; q++)
                bb[k][q] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(xr, xo[q], pk * pgb_x, 0));
        }
        // one position group: its gathers, the code word WD groups ahead,
        // the stage sums and MFMAs, then B WD groups ahead into the slot the
        // MFMAs have read
        auto step = [&](int k, int pg) {
            half8 av[4][F::S];
            gather_group<FMT, F::SB>(lds_vq, buf[k], av);
            const int pn = min(pg + WD, npg - 1);
            word_load<F::SB>(buf[k], cr, co, pn * 256 * F::SB);
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int s = 1; s < F::S; s++) av[t][0] = av[t][0] + av[t][s];
#pragma unroll
            for (int q = 0; q < RB; q++)
                if (2 * q < nt)                               // uniform
#pragma unroll
                    for (int t = 0; t < 4; t++)
                        acc[q][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[t][0], bb[k][q], acc[q][t], 0, 0, 0);
#pragma unroll
            for (int q = 0; q < RB; q++)
                bb[k][q] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(xr, xo[q], pn * pgb_x, 0));
        };
        const int npg_full = npg - npg % WD;
        for (int pgb = 0; pgb < npg_full; pgb += WD) {
#pragma unroll
            for (int k = 0; k < WD; k++) step(k, pgb + k);
        }
#pragma unroll
        for (int k = 0; k < WD; k++)
            if (npg_full + k < npg) step(k, npg_full + k);    // uniform
        l = rq_take(rq, lane);                                // returns while the outputs are stored
        // lane (g, jc) holds C[4g + r][jc] of row tile t: block row
        // 16g + 4r + t, token jc % 8 of job 2 q + jc / 8 -- the 16
        // consecutive rows 16g .. 16g + 15 of one token. The four lanes of a
        // token (g = 0..3) swap their 16-byte runs (a 4 x 4 transpose by
        // lane xors 16, 32, 48), so that store k writes rows 16k .. 16k + 15
        // as one 64-byte sector: stored one float at a time the down launch
        // wrote 3.9x its output, as 16-byte runs 64 B apart 1.75x.
#pragma unroll
        for (int q = 0; q < RB; q++) {
            if (2 * q >= nt) break;                           // uniform
            const int jq_i = 2 * q + (jc >> 3), tk = jc & 7;
            const warp_job &jq = jobs[j0 + min(jq_i, nt - 1)];
            const bool tv = jq_i < nt && tk < jq.n;
            const int yrow = tv ? jq.yi[tk] : 0;
            const float xsc = tv ? a.xscale[yrow] : 0.0f;
            float *yo = a.y[kind] + (size_t)yrow * M;
            if ((M & 63) == 0) {                              // uniform: whole 64-row blocks
                // w[d][t]: what round d brings from lane g ^ d, its row
                // 16 (g ^ d) + 4 g + t
                float w[4][4];
                auto pick = [](const float *u, int i) { return i == 0 ? u[0] : i == 1 ? u[1] : i == 2 ? u[2] : u[3]; };
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    float v[4];                               // rows 16 g + 4 r + t
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        v[r] = (acc[q][t][r] * xsc) * f16_keep(jq.scale[rb * 64 + 16 * g + 4 * r + t]);
#pragma unroll
                    for (int d = 0; d < 4; d++) {             // round d: v[g ^ d] to lane g ^ d
                        const float sv = pick(v, g ^ d);
                        w[d][t] = d == 0 ? sv : __shfl_xor(sv, 16 * d);
                    }
                }
#pragma unroll
                for (int k = 0; k < 4; k++) {                 // rows 16 k + 4 g .. + 3: round g ^ k's
                    const int d = g ^ k;
                    const float4 o = make_float4(d == 0 ? w[0][0] : d == 1 ? w[1][0] : d == 2 ? w[2][0] : w[3][0],
                                                 d == 0 ? w[0][1] : d == 1 ? w[1][1] : d == 2 ? w[2][1] : w[3][1],
                                                 d == 0 ? w[0][2] : d == 1 ? w[1][2] : d == 2 ? w[2][2] : w[3][2],
                                                 d == 0 ? w[0][3] : d == 1 ? w[1][3] : d == 2 ? w[2][3] : w[3][3]);
                    if (tv) *(float4 *)(yo + rb * 64 + 16 * k + 4 * g) = o;
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++)
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        const int row = rb * 64 + 16 * g + 4 * r + t;
                        if (tv && row < M) yo[row] = (acc[q][t][r] * xsc) * f16_keep(jq.scale[row]);
                    }
            }
        }
    }
    rq_leave(rq, lane, 1);
}

template <int FMT>
static int launch_vq_run_f16(const VqArgs &a, const int *runs, int nkinds, int max_units, void *stream) {
    typedef FmtT<FMT> F;
    constexpr int WD = F::S == 3 ? 2 : 3;                   // code words and B operands in flight
    int grid = (max_units + 15) / 16;
    const int cap = FMT == WARP_FMT_VQ12 ? 256 : 512;
    if (grid > cap) grid = cap;
    grid = (grid + RQ_GROUPS - 1) / RQ_GROUPS * RQ_GROUPS;   // the unit queues' groups
    hipLaunchKernelGGL((k_vq_run_f16<FMT, WD>), dim3(grid, nkinds), dim3(1024), 0, (hipStream_t)stream, a, runs);
    CHECK_LAUNCH();
    return 0;
}

extern "C" int wk_vq_runs(int fmt, const warp_job *jobs, const int *njobs, int max_jobs, const int *runs,
                          int kind_lo, int nkinds, const uint16_t *books, const uint16_t *xs, const float *xscale,
                          float *const *y, int M, int N, int fp16_rows, unsigned *queue, void *stream) {
    if (M <= 0 || N <= 0 || (N % 32) || max_jobs <= 0 || !runs || !queue || kind_lo < 0 || nkinds < 1 || kind_lo + nkinds > 3 ||
        fp16_rows < 0 || (size_t)fp16_rows * N * 2 >= ((size_t)1 << 31))
        return -1;
    for (int k = kind_lo; k < kind_lo + nkinds; k++)
        if ((uintptr_t)y[k] & 15) return -1;                // (16-byte row stores)
    const int fp16 = fp16_rows > 0;
    VqArgs a{};
    a.jobs = jobs;
    a.njobs = njobs;
    a.max_jobs = max_jobs;
    a.kind_lo = kind_lo;
    a.books = books;
    a.xs = (const _Float16 *)xs;
    a.xscale = xscale;
    for (int k = 0; k < 3; k++) a.y[k] = y[k];
    a.M = M;
    a.N = N;
    a.xrows = fp16_rows;
    a.queue = queue;
    const int max_units = max_jobs * ((M + 63) / 64);
    switch (fmt) {
#define VR(F)                                                                                                      \
    return fp16 ? launch_vq_run_f16<F>(a, runs, nkinds, max_units, stream)                                         \
                : launch_vq_run<F>(a, runs, nkinds, max_units, stream)
    case WARP_FMT_VQ3R: VR(WARP_FMT_VQ3R);
    case WARP_FMT_VQ2R: VR(WARP_FMT_VQ2R);
    case WARP_FMT_VQ12: VR(WARP_FMT_VQ12);
#undef VR
    }
    return -1;
}

extern "C" int wk_vq_matvec(int fmt, const warp_job *jobs, const int *njobs, int max_jobs, int kind_lo,
                            int nkinds, const uint16_t *books, const uint16_t *xs, const float *xscale,
                            float *const *y, int M, int N, int tokens_per_job, void *stream) {
    if (M <= 0 || N <= 0 || (N % 32) || max_jobs <= 0 || kind_lo < 0 || nkinds < 1 || kind_lo + nkinds > 3)
        return -1;
    if (tokens_per_job != 1 && tokens_per_job != WARP_TPJ) return -1;
    VqArgs a{};
    a.jobs = jobs;
    a.njobs = njobs;
    a.max_jobs = max_jobs;
    a.kind_lo = kind_lo;
    a.books = books;
    a.xs = (const _Float16 *)xs;
    a.xscale = xscale;
    for (int k = 0; k < 3; k++) a.y[k] = y[k];
    a.M = M;
    a.N = N;
    const int npg = N / 32, nrb = (M + 63) / 64, max_units = max_jobs * nrb;
    switch (fmt) {
    case WARP_FMT_VQ3R: return launch_vq_t<WARP_FMT_VQ3R>(a, nkinds, max_units, npg, tokens_per_job, stream);
    case WARP_FMT_VQ2R: return launch_vq_t<WARP_FMT_VQ2R>(a, nkinds, max_units, npg, tokens_per_job, stream);
    case WARP_FMT_VQ12: return launch_vq_t<WARP_FMT_VQ12>(a, nkinds, max_units, npg, tokens_per_job, stream);
    }
    return -1;
}

// ---- the LUT expert matvec (decode) ---------------------------------------------------
//
// The reference's own algorithm (src/model.c:1843-2024), laid out for LDS:
// for every vector position p the table LUT[s][c] = dot(codebook_s[c], x[8p..8p+8])
// is built, and each row sums LUT[0][code0] + LUT[1][code1] (+ LUT[2][code2])
// over its positions, in that order per position as the reference does. A
// random 4-byte LDS read costs about what a random 16-byte codebook gather
// does and replaces a gather plus 16 multiply-adds, so the table wins
// whenever it is amortised over enough rows.
//
// Block = 16 waves, one per CU. A block owns a row group (64 pairs of 64-row
// blocks = 8192 rows, round-robin over the waves; across the jobs of a list
// when they share one input, within one job otherwise) and a split of the
// positions, which it walks 2 positions at a time: the table of the next 2
// positions (2 x S x E floats) is built into one LDS buffer while the rows are
// summed from the other, each pair step of a wave doing a share of the build.
// A lane sums 4 rows of one row block at one position parity; the two
// parities are added at the end and the block writes one partial sum per row
// and split. The splits are added in order by the consumer (k_lut_reduce,
// the down launch's prologue, k_combine_lut), so results are deterministic.
//
// Table build. The codebook of the block's kind sits in registers (fp16, one
// 64-entry group per 64 lanes, 8 groups per wave for 2 x 4096). The build runs
// on the matrix cores: in v_mfma_f32_4x4x4_16b_f16 each lane's entry is one
// column of B (block = 4 lanes = 4 codes), and A holds the split's x scaled
// by 2^ks and split into fp16 hi and lo halves (x*2^ks = hi + lo to ~22
// bits), with the two positions as rows and (dims, hi/lo) as K: four MFMAs
// give sum_d cb[d] * (hi[d] + lo[d]), exact products summed in fp32, and
// every lane ends with both positions of its own entry, which it stores as
// one 8-byte pair (a wave writes 512 contiguous bytes, no bank conflicts).
// The row sums carry the factor 2^ks, removed exactly at the end. Layers whose
// codebooks hold exponent-31 values (finite in the reference, inf for the
// matrix cores) take the X31 variant: the reference's fused d-ascending chain
// on the vector ALUs from f32 x, bit-identical to its table entries.

constexpr int LUT_NW = 16;                 // waves per block
constexpr int LUT_PPW = 4;                 // row-block pairs per wave
constexpr int LUT_PAIRS = LUT_NW * LUT_PPW;
constexpr int LUT_RBG = 2 * LUT_PAIRS;     // row blocks per row group
constexpr int LUT_XCH = 256;               // chunks of x a split stages in LDS (16 KiB)
constexpr int ACT_LD = 8;                  // staged partial-sum loads per thread (down prologue)

struct LutArgs {
    const warp_job *jobs;
    const int *njobs;
    int max_jobs, kind_lo;
    const uint16_t *books;     // [3][S][E][8] fp16, subnormals flushed
    const float *x;            // inputs [*][N]; a job reads x + xi[0] * N
    float *part;               // [nkinds][splits][max_jobs][nrb * 64]
    int M, N, splits, shared_x;
    // when set (down, one input per job): the input of job j is not read
    // from x but made here, h[r] = act(gate[r], up[r]) from the gate/up
    // partial sums (kinds 0 and 1 of the previous launch, act_splits each)
    const float *act_part;
    int act_splits, act_situ;
    float act_beta, act_lbeta;
    // routing in the prologue (gate and up of a decode step): every block
    // picks the experts from the logits itself (the same picks everywhere);
    // block 0 writes idx, w, the job lists of all three kinds (into jobs),
    // njobs and the missing flag for the launches that follow
    warp_route_args r;
    // (routed launches) the blocks of one extra grid row instead compute
    // the shared expert's h = act(gate . x, up . x), one row per wave, as
    // k_router_shared does, when sh.h is set;
    // (down launches, sh_out set) blocks sh_first.. instead compute the
    // shared expert's down rows sh_out = down . sh.h, four rows per wave,
    // as k_combine_lut does
    warp_shared_args sh;
    float *sh_out;
    int sh_first;
};


// Sum of a row's partials over the splits, in split order. Up to 32 splits
// every load is issued before the first add (one memory latency per row).
__device__ __forceinline__ float lut_rowsum(const float *p, int splits, size_t stride) {
    if (splits <= 32) {
        float a[32];
#pragma unroll
        for (int s = 0; s < 32; s++) a[s] = s < splits ? p[(size_t)s * stride] : 0.0f;
        float v = 0.0f;
#pragma unroll
        for (int s = 0; s < 32; s++)
            if (s < splits) v += a[s];
        return v;
    }
    float v = 0.0f;
    for (int s = 0; s < splits; s++) v += p[(size_t)s * stride];
    return v;
}

// The same sum for at most MAXS splits: MAXS loads issued unconditionally
// (indices past the last split repeat it), then the adds in split order.
template <int MAXS>
__device__ __forceinline__ float lut_rowsum_n(const float *p, int splits, size_t stride) {
    float a[MAXS];
#pragma unroll
    for (int s = 0; s < MAXS; s++) a[s] = p[(size_t)min(s, splits - 1) * stride];
    float v = 0.0f;
#pragma unroll
    for (int s = 0; s < MAXS; s++)
        if (s < splits) v += a[s];
    return v;
}

// The same sum with at most 8 loads in flight (few registers); CO: the
// loads are agent-coherent.
template <bool CO = false>
__device__ __forceinline__ float lut_rowsum8(const float *p, int splits, size_t stride) {
    float v = 0.0f;
    for (int s0 = 0; s0 < splits; s0 += 8) {
        float a8[8];
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const float *q = p + (size_t)min(s0 + s, splits - 1) * stride;
            a8[s] = CO ? ld_agent(q) : *q;
        }
#pragma unroll
        for (int s = 0; s < 8; s++)
            if (s0 + s < splits) v += a8[s];
    }
    return v;
}

template <int FMT>
__device__ __forceinline__ unsigned lut_code(unsigned slot, int s) {
    if (FMT == WARP_FMT_VQ12) return s == 0 ? (slot & 0xFFFu) : (slot >> 12);
    return (slot >> (8 * s)) & 0xFFu;
}

typedef _Float16 half4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ half4 half4_of(uint32_t lo, uint32_t hi) {
    return __builtin_bit_cast(half4, make_uint2(lo, hi));
}

// One expert's routing inputs (thread e of a routing block): its score (the
// logit, or with pre-scored logits the sigmoid score), the biased score
// input, and its expert-table entry, loaded together and then staged in LDS.
struct RouteIn {
    float lg, bs;
    const uint8_t *rec;
    uint2 off01, off23;
};
__device__ __forceinline__ RouteIn route_in_load(const warp_route_args &r, int e) {
    RouteIn v = {0.0f, 0.0f, nullptr, make_uint2(0u, 0u), make_uint2(0u, 0u)};
    if (e < r.E) {
        v.lg = r.logits[e];
        v.bs = r.scored ? r.logits[r.E + e] : r.bias ? r.bias[e] : 0.0f;
        // (the slot by fields: an aggregate copy would go through scratch)
        v.rec = r.table[e].rec;
        v.off01 = *(const uint2 *)&r.table[e].off[0];
        v.off23 = *(const uint2 *)&r.table[e].off[2];
    }
    return v;
}
__device__ __forceinline__ void route_in_store(const RouteIn &v, int E, int e, float *score, float *biased,
                                               warp_slot *slots) {
    if (e < E) {
        score[e] = v.lg;
        biased[e] = v.bs;
        slots[e].rec = v.rec;
        *(uint2 *)&slots[e].off[0] = v.off01;
        *(uint2 *)&slots[e].off[2] = v.off23;
    }
}

// The fused decode launch (k_moe_fused) runs gate/up, down and combine work
// items in one grid. Its blocks route the token once and keep the picks'
// records here; its counters say when the inputs of an item are complete.
struct LutPicks {
    const uint8_t *rec[WARP_MAX_K];    // the picks' records, in selection order
    uint32_t off[WARP_MAX_K][4];       // their header offsets (warp_slot.off)
    int nj;                            // K, or 0 when a pick has no record
};
// Counter i of the fused launch is word i * FZ_LINE: one 128-byte line per
// counter, so that its polls and increments load one memory channel each.
constexpr int FZ_LINE = 32;
struct FzSync {
    unsigned *ctr;                     // counters: 0 claims, 1 exits, 2 down items done,
                                       // 3 + g gate/up items of row group g done
    int *flag;                         // the missing flag: bit 2 set when a wait gives up
    unsigned limit;                    // polls before a wait gives up
};

// Thread 0 of a block: wait until counters lo..hi of ctr all reach target. The counted
// items wrote their results with agent-coherent stores that were complete
// before the counts rose, and the block reads them with agent-coherent
// loads once its threads pass the barrier after this. A wait that exceeds
// the poll limit raises bit 2 of the flag and returns, so that every wave
// of the grid ends.
__device__ __forceinline__ void fz_wait(const unsigned *ctr, int lo, int hi, unsigned target, const FzSync &sy) {
    for (int g = lo; g <= hi; g++) {
        unsigned n = 0;
        while (__hip_atomic_load(ctr + g * FZ_LINE, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
            if (++n > sy.limit) {
                __hip_atomic_fetch_or(sy.flag, 4, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                return;
            }
            __builtin_amdgcn_s_sleep(8);
        }
    }
}

// One unit (row group bx / a.splits, split bx % a.splits, kind a.kind_lo +
// by) of a LUT launch, by the whole block.
// SHX = true: the jobs of the list share one input and a row group spans
// them (gate and up); false: one input per job (down). ACT (with SHX false):
// the inputs are made from the gate/up partial sums (a.act_part). RT (with
// SHX): the jobs are picked in the prologue from the router logits (a.r).
// FZ: a work item of the fused launch: the jobs are the picks in pk, and
// (ACT) the gate/up partial sums are read once the row groups that hold
// them are counted complete in sy.
template <int FMT, bool X31, bool SHX, bool ACT, bool RT, bool FZ>
__device__ __forceinline__ void lut_item(const LutArgs &a, const unsigned bx, const unsigned by, const LutPicks *pk,
                                         const FzSync *sy) {
    typedef FmtT<FMT> F;
    constexpr int SE = F::S * F::E;                        // table entries per position
    constexpr int NG = SE / 64;                            // 64-entry groups
    constexpr int GPW = (NG + LUT_NW - 1) / LUT_NW;        // groups per wave
    constexpr int BUF = 2 * SE;                            // floats per buffer
    static_assert(SE % 64 == 0, "table groups");
    // (in the fused launch, opaque per item: what derives from it is
    // computed per item, not held in registers across the item loop)
    unsigned tid = threadIdx.x;
    if constexpr (FZ) asm volatile("" : "+v"(tid));
    // the expf table for the activation and the routing scores, loaded
    // before every other load and kept in LDS (see expf_ref)
    __shared__ uint64_t s_exp[32];
    uint64_t etv = 0;
    if constexpr (ACT || RT) etv = g_exp2_tab[tid & 31];
    extern __shared__ __attribute__((aligned(16))) float lut[];   // [2][S][E][2], then x of the split
    const int kind = a.kind_lo + by;
    const warp_job *jobs = a.jobs + (size_t)kind * a.max_jobs;
    const int nv = a.N >> 3, nrb = (a.M + 63) >> 6, nc = nv >> 1;
    const int grp = bx / a.splits, split = bx % a.splits;
    const int c0 = split * nc / a.splits, c1 = (split + 1) * nc / a.splits;
    const int lane = tid & 63, wave = tid >> 6;
    const int pl = (lane >> 4) & 1, rbsel = lane >> 5, quad = lane & 15;
    int fb0, xj;
    if (SHX) {
        fb0 = grp * LUT_RBG;
        xj = 0;
    } else {
        const int gpj = (nrb + LUT_RBG - 1) / LUT_RBG;
        xj = grp / gpj;
        fb0 = xj * nrb + (grp % gpj) * LUT_RBG;
    }
    constexpr bool act = ACT && !SHX;
    const int nx = (c1 - c0) * 16;                         // inputs of this split
    constexpr int XPT = LUT_XCH * 16 / (LUT_NW * 64);      // inputs per thread, at most

    // The prologue issues its loads in the order their data is needed and
    // waits for no load it does not use (loads complete in issue order).
    constexpr bool rt = RT && SHX;
    const uint8_t *jrec[LUT_PPW];
    const uint8_t *jrec0;
    int xi, nj;
    gu32 *sg = nullptr, *su = nullptr;
    float xr[XPT];
    // The codebook of this kind: group G = vw * GPW + g holds entries
    // 64 G .. 64 G + 63 over [stage][entry], entry 64 G + lane in this lane
    // (128 KiB per block for 2 x 4096 entries). vw rotates the waves' groups
    // by block, so that the blocks of a launch, which all load the same
    // codebook at once, start on different lines.
    const int vw = (wave + (int)bx) & (LUT_NW - 1);
    uint4 cb[GPW];
    auto load_cb = [&]() {
        const uint4 *bk = (const uint4 *)(a.books + (size_t)kind * SE * 8);
#pragma unroll
        for (int g = 0; g < GPW; g++) {
            const int G = vw * GPW + g;
            cb[g] = G < NG ? bk[G * 64 + lane] : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    if constexpr (rt) {
        // 1. The routing inputs (one expert per thread: E <= the block
        //    size), then the token's input and the codebook; the routing
        //    inputs staged in the table buffers, which are not built yet; the
        //    picks; then the record of every pair straight from the staged
        //    expert table.
        const int E = a.r.E, E2 = (E + 1) & ~1, K = a.max_jobs, e = tid;
        float *score = lut, *biased = lut + E2;
        warp_slot *slots = (warp_slot *)(lut + 2 * E2);
        __shared__ int r_sel[WARP_MAX_K];
        __shared__ float r_wsel[WARP_MAX_K];
        const RouteIn ri = route_in_load(a.r, e);
        __builtin_amdgcn_sched_barrier(0);
        const float *xg = a.x + (size_t)c0 * 16;
#pragma unroll
        for (int k = 0; k < XPT; k++) {
            const int i = tid + k * LUT_NW * 64;
            const float v = xg[min(i, nx - 1)];
            xr[k] = i < nx ? v : 0.0f;
        }
        __builtin_amdgcn_sched_barrier(0);
        load_cb();                                         // streams in while the picks are made
        __builtin_amdgcn_sched_barrier(0);
        route_in_store(ri, E, e, score, biased, slots);
        if (tid < 32) s_exp[tid] = etv;
        // only the block that publishes the routing needs the weights
        const bool pub = blockIdx.x == 0 && blockIdx.y == 0;
        route_pick_lds<true, LUT_NW * 64>(E, K, a.r.act, a.r.renorm, a.r.routed_scale, score, biased, r_sel, r_wsel,
                                          pub, a.r.scored != 0, s_exp);
        const bool miss = picks_missing(slots, r_sel, K);  // a pick without a record (the same in every block)
        if (pub) {                                         // uniform per block
            if (tid < K) {
                a.r.idx[tid] = r_sel[tid];
                a.r.w[tid] = r_wsel[tid];
            }
            route_jobs<LUT_NW * 64>(r_sel, K, slots, a.r.jobs, a.r.njobs, a.r.missing, a.r.inter);
        }
#pragma unroll
        for (int q = 0; q < LUT_PPW; q++) {
            const int fb = fb0 + 2 * (q * LUT_NW + wave) + rbsel;
            const warp_slot &sl = slots[r_sel[min(fb / nrb, K - 1)]];
            jrec[q] = sl.rec + sl.off[kind];
        }
        const warp_slot &s0 = slots[r_sel[min(fb0 / nrb, K - 1)]];
        jrec0 = s0.rec + s0.off[kind];
        xi = 0;
        nj = miss ? 0 : K;
        __syncthreads();                                   // the staging area is reused below
    } else if constexpr (FZ) {
        // 1. The records of the block's picks (LDS), the input index and,
        //    for the down items, the gate/up row scales.
        const int K = a.max_jobs;
#pragma unroll
        for (int q = 0; q < LUT_PPW; q++) {
            const int fb = fb0 + 2 * (q * LUT_NW + wave) + rbsel;
            const int j = min(fb / nrb, K - 1);
            jrec[q] = pk->rec[j] + pk->off[j][kind];
        }
        const int j0 = min(fb0 / nrb, K - 1);
        jrec0 = pk->rec[j0] + pk->off[j0][kind];
        xi = 0;
        if constexpr (act) {
            const uint16_t *sc = (const uint16_t *)(pk->rec[xj] + pk->off[xj][3]);
            sg = (gu32 *)sc;
            su = (gu32 *)(sc + a.N);
        }
        nj = pk->nj;
    } else {
        // 1. The job list, written by the routing launch: the record of every
        //    pair (the job of a pair follows from the block's position; the
        //    job count, read alongside, only decides which pairs are real),
        //    the input index and, for the down launch, the gate/up row
        //    scales.
#pragma unroll
        for (int q = 0; q < LUT_PPW; q++) {
            const int fb = fb0 + 2 * (q * LUT_NW + wave) + rbsel;
            jrec[q] = jobs[min(fb / nrb, a.max_jobs - 1)].idx;
        }
        jrec0 = jobs[fb0 / nrb].idx;
        xi = act ? 0 : jobs[xj].xi[0];
        if constexpr (act) {
            sg = (gu32 *)a.jobs[xj].scale;
            su = (gu32 *)a.jobs[(size_t)a.max_jobs + xj].scale;
        }
        nj = a.njobs[kind];
    }

    // 2. Down launch: the gate/up partial sums of this split's inputs, rows
    //    [kind 0, 1][split s] of nx values, spread over the block (one load
    //    per thread per row-chunk; indices past the end are clamped and their
    //    values dropped), to be staged in the table buffers.
    //    (FZ: after step 4, once the row groups are complete.)
    const size_t arows = (size_t)((a.N + 63) >> 6) * 64, astride = (size_t)a.max_jobs * arows;
    const int atot = act ? 2 * a.act_splits * nx : 0;
    const bool astage = act && atot <= ACT_LD * LUT_NW * 64 && atot <= 2 * BUF;   // uniform
    float av[ACT_LD];
    auto stage_partials = [&]() {
        const float *pa = a.act_part + (size_t)xj * arows + (size_t)c0 * 16;
        const int drow = (LUT_NW * 64) / nx, dv = (LUT_NW * 64) % nx, rmax = 2 * a.act_splits - 1;
        int row = tid / nx, v = tid % nx;
#pragma unroll
        for (int k = 0; k < ACT_LD; k++) {
            const float *q = pa + (size_t)min(row, rmax) * astride + v;
            av[k] = FZ ? ld_agent(q) : *q;
            row += drow;
            v += dv;
            if (v >= nx) { v -= nx; row++; }
        }
    };
    if (!FZ && astage) stage_partials();
    __builtin_amdgcn_sched_barrier(0);

    const int fb_end = SHX ? nj * nrb : (xj < nj ? (xj + 1) * nrb : 0);
    if (fb0 >= fb_end || c0 >= c1) return;                 // uniform per block

    // 3. The input: read, or (down launch) the gate/up row scales to make it
    //    with, as the 4-byte words that hold them (the scale arrays of a
    //    record are 4-byte aligned and a split starts at an even input).
    //    Only jobs below the count are dereferenced.
    unsigned gs[XPT], us[XPT];
    if constexpr (act) {
#pragma unroll
        for (int k = 0; k < XPT; k++) {
            const int i = min((int)tid + k * LUT_NW * 64, nx - 1) + c0 * 16;
            gs[k] = sg[i >> 1];
            us[k] = su[i >> 1];
        }
    } else if constexpr (!rt) {
        const float *xg = a.x + (size_t)xi * a.N + (size_t)c0 * 16;
#pragma unroll
        for (int k = 0; k < XPT; k++) {
            const int i = tid + k * LUT_NW * 64;
            const float v = xg[min(i, nx - 1)];
            xr[k] = i < nx ? v : 0.0f;
        }
    }
    // 4. The codebook (unless loaded with the routing inputs), which the
    //    first table build needs, then the code words of the first chunk,
    //    which the loop needs.
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (!rt) load_cb();
    __builtin_amdgcn_sched_barrier(0);
    // Pairs past the group's rows read row block 0 of the block's first job
    // (in bounds), look up entry 0 only and are never written: the loop
    // below has no per-pair branches, so the code-word loads of the next
    // chunk stay in flight across the whole chunk and the LDS reads of all
    // pairs overlap.
    const uint8_t *cp[LUT_PPW];
#pragma unroll
    for (int q = 0; q < LUT_PPW; q++) {
        const int fb = fb0 + 2 * (q * LUT_NW + wave) + rbsel;
        const bool ok = fb < fb_end;
        const int rb = fb - (fb / nrb) * nrb;
        const size_t off = (size_t)(ok ? rb : 0) * nv * 64 * F::SB;
        cp[q] = (ok ? jrec[q] : jrec0) + off + (size_t)pl * 64 * F::SB + (size_t)quad * 4 * F::SB;
    }
    Word<F::SB> wd[LUT_PPW];
#pragma unroll
    for (int q = 0; q < LUT_PPW; q++) wd[q].load_keep(cp[q] + (size_t)(2 * c0) * 64 * F::SB);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (FZ && act) {
        // the gate/up row groups that hold this item's inputs (rows
        // 16 c0 .. 16 c1 - 1 of pick xj), every split of both kinds
        const int nrbg = (a.N + 63) >> 6;
        if (tid == 0)
            fz_wait(sy->ctr + 3 * FZ_LINE, (xj * nrbg + (c0 * 16) / 64) / LUT_RBG, (xj * nrbg + (c1 * 16 - 1) / 64) / LUT_RBG,
                    2u * a.act_splits, *sy);
        __syncthreads();
        if (astage) stage_partials();
    }

    // 5. Down launch: h = act(gate, up) from the partial sums, added over the
    //    splits in split order (through the staging area when it fits).
    if constexpr (act) {
        if (tid < 32) s_exp[tid] = etv;
        if (astage) {
            const int drow = (LUT_NW * 64) / nx, dv = (LUT_NW * 64) % nx;
            int row = tid / nx, v = tid % nx;
#pragma unroll
            for (int k = 0; k < ACT_LD; k++) {
                if (row * nx + v < atot) lut[row * nx + v] = av[k];
                row += drow;
                v += dv;
                if (v >= nx) { v -= nx; row++; }
            }
            __syncthreads();
            // P threads per input (uniform): thread (p, i) adds splits
            // [p S / P, (p + 1) S / P) of input i in split order into LDS
            // after the staged rows, then the P parts are added in part order
            const int S = a.act_splits;
            int P = (LUT_NW * 64) / nx;
            P = P > 8 ? 8 : P;
            while (P > 1 && atot + 2 * P * nx > 2 * BUF) P--;
            float *ps = lut + atot;                        // [gate, up][P][nx]
            if (P > 1) {
                const int i = (int)tid % nx, p = (int)tid / nx;
                if (p < P) {
                    const int s1 = (p + 1) * S / P;
                    float g = 0.0f, u = 0.0f;
                    for (int s2 = p * S / P; s2 < s1; s2++) {
                        g += lut[s2 * nx + i];
                        u += lut[(S + s2) * nx + i];
                    }
                    ps[p * nx + i] = g;
                    ps[(P + p) * nx + i] = u;
                }
                __syncthreads();
            }
#pragma unroll
            for (int k = 0; k < XPT; k++) {
                const int i = tid + k * LUT_NW * 64;
                xr[k] = 0.0f;
                if (i < nx) {
                    float g = 0.0f, u = 0.0f;
                    if (P > 1) {
                        g = ps[i];
                        u = ps[P * nx + i];
                        for (int p = 1; p < P; p++) {
                            g += ps[p * nx + i];
                            u += ps[(P + p) * nx + i];
                        }
                    } else {
                        // the splits in order, 16 LDS reads in flight at a time
                        for (int s0 = 0; s0 < S; s0 += 16) {
                            float ga[16], ua[16];
#pragma unroll
                            for (int t = 0; t < 16; t++) {
                                const int s2 = min(s0 + t, S - 1);
                                ga[t] = lut[s2 * nx + i];
                                ua[t] = lut[(S + s2) * nx + i];
                            }
#pragma unroll
                            for (int t = 0; t < 16; t++)
                                if (s0 + t < S) {
                                    g += ga[t];
                                    u += ua[t];
                                }
                        }
                    }
                    const int sh = 16 * (i & 1);
                    xr[k] = act_pair(g * f16_keep((uint16_t)(gs[k] >> sh)), u * f16_keep((uint16_t)(us[k] >> sh)),
                                     a.act_situ, a.act_beta, a.act_lbeta, s_exp);
                }
            }
        } else {
            __syncthreads();                               // s_exp
            const float *pg = a.act_part + (size_t)xj * arows + (size_t)c0 * 16;
            const float *pu = pg + (size_t)a.act_splits * astride;
#pragma unroll
            for (int k = 0; k < XPT; k++) {
                const int i = tid + k * LUT_NW * 64;
                xr[k] = 0.0f;
                if (i < nx) {
                    const int sh = 16 * (i & 1);
                    const float g = lut_rowsum8<FZ>(pg + i, a.act_splits, astride) * f16_keep((uint16_t)(gs[k] >> sh));
                    const float u = lut_rowsum8<FZ>(pu + i, a.act_splits, astride) * f16_keep((uint16_t)(us[k] >> sh));
                    xr[k] = act_pair(g, u, a.act_situ, a.act_beta, a.act_lbeta, s_exp);
                }
            }
        }
    }
    // -> LDS: f32 [chunk][16] (X31) or the scaled fp16 halves
    // [chunk][position 2][hi, lo][8]
    int ks = 0;
    if constexpr (X31) {
        float *xst = lut + 2 * BUF;
#pragma unroll
        for (int k = 0; k < XPT; k++) {
            const int i = tid + k * LUT_NW * 64;
            if (i < nx) xst[i] = xr[k];
        }
    } else {
        float m = 0.0f;
#pragma unroll
        for (int k = 0; k < XPT; k++) m = fmaxf(m, fabsf(xr[k]));
        ks = split_exp(block_absmax(m));
        _Float16 *xh = (_Float16 *)(lut + 2 * BUF);
#pragma unroll
        for (int k = 0; k < XPT; k++) {
            const int i = tid + k * LUT_NW * 64;
            if (i < nx) {
                const int o = (i >> 4) * 32 + ((i >> 3) & 1) * 16 + (i & 7);
                split_store(xr[k], ks, &xh[o], &xh[o + 8]);
            }
        }
    }

    // A operands (x) of chunk c: row i = lane % 4 is position i (i < 2) or
    // zero; K runs over (hi dims 0-3, hi 4-7, lo 0-3, lo 4-7)
    auto load_b = [&](half4 (&B)[4], int c) {
        const int j = lane & 3;
        const _Float16 *xh = (const _Float16 *)(lut + 2 * BUF) + (c - c0) * 32 + (j & 1) * 16;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const half4 v = *(const half4 *)(xh + (m >> 1) * 8 + (m & 1) * 4);
            B[m] = j < 2 ? v : half4{0, 0, 0, 0};
        }
    };
    // this wave's groups g = q, q + PPW, ... of the table into buffer b: x
    // is A (rows = the 2 positions), this lane's entry the B column, so a
    // lane gets both positions of its own entry and writes them as a pair
    auto build_mfma = [&](const half4 (&X)[4], int b, int q) {
#pragma unroll
        for (int g = q; g < GPW; g += LUT_PPW) {
            const int G = vw * GPW + g;
            if (G < NG) {                                  // uniform per wave
                const half4 clo = half4_of(cb[g].x, cb[g].y), chi = half4_of(cb[g].z, cb[g].w);
                f4 d = {0.f, 0.f, 0.f, 0.f};
                d = __builtin_amdgcn_mfma_f32_4x4x4f16(X[0], clo, d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_4x4x4f16(X[1], chi, d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_4x4x4f16(X[2], clo, d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_4x4x4f16(X[3], chi, d, 0, 0, 0);
                *(float2 *)(lut + b * BUF + (G * 64 + lane) * 2) = make_float2(d[0], d[1]);
            }
        }
    };
    auto load_x = [&](float (&xv)[16], int c) {
        const float *xc = lut + 2 * BUF + (c - c0) * 16;
#pragma unroll
        for (int k = 0; k < 16; k++) xv[k] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(xc[k])));
    };
    auto build_valu = [&](const float (&xv)[16], int b, int q) {
#pragma unroll
        for (int g = q; g < GPW; g += LUT_PPW) {
            const int G = vw * GPW + g;
            if (G < NG) {
                const uint32_t w4[4] = {cb[g].x, cb[g].y, cb[g].z, cb[g].w};
                float t[2];
#pragma unroll
                for (int pp = 0; pp < 2; pp++) {
                    t[pp] = 0.0f;
#pragma unroll
                    for (int d = 0; d < 8; d++)
                        t[pp] = __builtin_fmaf(xv[pp * 8 + d], f16_flushed((uint16_t)(w4[d >> 1] >> (16 * (d & 1)))),
                                               t[pp]);
                }
                *(float2 *)(lut + b * BUF + (G * 64 + lane) * 2) = make_float2(t[0], t[1]);
            }
        }
    };

    float acc[LUT_PPW][4];
#pragma unroll
    for (int q = 0; q < LUT_PPW; q++)
#pragma unroll
        for (int t = 0; t < 4; t++) acc[q][t] = 0.0f;

    half4 B[4];
    float xv[16];
    const int fb_lim = fb_end - fb0;                       // pairs at or past it are not real
    __syncthreads();
    if constexpr (X31) {
        load_x(xv, c0);
#pragma unroll
        for (int q = 0; q < LUT_PPW; q++) build_valu(xv, 0, q);
        load_x(xv, c0 + 1 < c1 ? c0 + 1 : c0);
    } else {
        load_b(B, c0);
#pragma unroll
        for (int q = 0; q < LUT_PPW; q++) build_mfma(B, 0, q);
    }
    __syncthreads();
    for (int c = c0; c < c1; c++) {
        const int b = (c - c0) & 1;
        const bool more = c + 1 < c1;              // uniform
        const int cn = more ? c + 1 : c;
        const float *L = lut + b * BUF + pl;
        if constexpr (!X31) {
            if (more) load_b(B, c + 1);
        }
        // each pair step also builds a share of the next chunk's table
#pragma unroll
        for (int q = 0; q < LUT_PPW; q++) {
            if (more) {
                if constexpr (X31) build_valu(xv, b ^ 1, q);
                else build_mfma(B, b ^ 1, q);
            }
            // a pair past the group's rows looks up entry 0 of each table
            // (one address per position: a broadcast, no bank conflicts)
            Word<F::SB> w = wd[q];
            w.mask(rbsel < fb_lim - 2 * (q * LUT_NW + wave) ? ~0u : 0u);
            wd[q].load_keep(cp[q] + (size_t)(2 * cn) * 64 * F::SB);
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const unsigned sl = w.slot(t);
                float v = L[lut_code<FMT>(sl, 0) * 2];
#pragma unroll
                for (int s = 1; s < F::S; s++) v += L[(s * F::E + lut_code<FMT>(sl, s)) * 2];
                acc[q][t] += v;
            }
        }
        if constexpr (X31) {
            if (more) load_x(xv, c + 2 < c1 ? c + 2 : c + 1);
        }
        __syncthreads();
    }

    // even + odd positions, unscaled: one partial per row of this split
    float *po = a.part + ((size_t)by * a.splits + split) * a.max_jobs * nrb * 64;
#pragma unroll
    for (int q = 0; q < LUT_PPW; q++) {
        float v[4];
#pragma unroll
        for (int t = 0; t < 4; t++) v[t] = ldexpf(acc[q][t] + __shfl_xor(acc[q][t], 16), -ks);
        const int fb = fb0 + 2 * (q * LUT_NW + wave) + rbsel;
        if (pl == 0 && fb < fb_end) {
            float *d = po + fb * 64 + 4 * quad;
            if constexpr (FZ) {
                st_through4(d, v[0], v[1], v[2], v[3]);
            } else {
                *(float4 *)d = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    }
}

// A routed gate/up launch's extra grid row: the shared expert's gate and up
// rows for the token, one row per wave (k_router_shared's loads, sums and
// activation), into sh.h. x is staged in the table buffers.
template <int BITS, int MC>
__device__ __forceinline__ void lut_shared_rows(const LutArgs &a) {
    extern __shared__ __attribute__((aligned(16))) float lut[];
    float *xl = lut;
    using Q = QRow<BITS, MC>;
    const warp_shared_args &sa = a.sh;
    const int H = a.N;
    const int r = (int)blockIdx.x * LUT_NW + (int)(threadIdx.x >> 6), rr = min(r, sa.inter - 1);
    const int nc = H / Q::WPC, ng = H / sa.group;
    Q qg, qu;
    qg.load(sa.q[0] + (size_t)rr * sa.rowbytes[0], sa.s[0] + (size_t)rr * ng, sa.group, nc);
    qu.load(sa.q[1] + (size_t)rr * sa.rowbytes[1], sa.s[1] + (size_t)rr * ng, sa.group, nc);
    for (int i = threadIdx.x; i < H / 4; i += LUT_NW * 64) ((float4 *)xl)[i] = ((const float4 *)a.x)[i];
    __syncthreads();
    const float gv = qg.dot(xl, nc), uv = qu.dot(xl, nc);
    if (r < sa.inter && (threadIdx.x & 63) == 0) sa.h[r] = act_pair(gv, uv, sa.situ, sa.beta, sa.lbeta);
}

__device__ __forceinline__ void lut_shared(const LutArgs &a) {
    const int mc = (a.N / (a.sh.bits == 8 ? 16 : 32) + 63) / 64;
    if (a.sh.bits == 8) {
        if (mc <= 1) lut_shared_rows<8, 1>(a);
        else if (mc <= 2) lut_shared_rows<8, 2>(a);
        else if (mc <= 4) lut_shared_rows<8, 4>(a);
        else lut_shared_rows<8, SH_MAXC>(a);
    } else {
        if (mc <= 1) lut_shared_rows<4, 1>(a);
        else if (mc <= 2) lut_shared_rows<4, 2>(a);
        else if (mc <= 4) lut_shared_rows<4, 4>(a);
        else lut_shared_rows<4, SH_MAXC>(a);
    }
}

// A down launch's appended blocks: the shared expert's down rows, four per
// wave (k_combine_lut's row loads and sums), h staged in the table buffers.
template <int BITS, int MC>
__device__ __forceinline__ void lut_shared_down_rows(const LutArgs &a) {
    extern __shared__ __attribute__((aligned(16))) float lut[];
    using Q = QRow<BITS, MC>;
    const warp_shared_args &sa = a.sh;
    const int M = a.M, snc = sa.inter / Q::WPC, sng = sa.inter / sa.group;
    const int r0 = ((int)blockIdx.x - a.sh_first) * LUT_NW * 4 + (int)(threadIdx.x >> 6) * 4;
    Q qd[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int rr = min(r0 + k, M - 1);
        qd[k].load(sa.q[2] + (size_t)rr * sa.rowbytes[2], sa.s[2] + (size_t)rr * sng, sa.group, snc);
    }
    for (int i = threadIdx.x; i < sa.inter / 4; i += LUT_NW * 64) ((float4 *)lut)[i] = ((const float4 *)sa.h)[i];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float v = qd[k].dot(lut, snc);
        if ((threadIdx.x & 63) == 0 && r0 + k < M) a.sh_out[r0 + k] = v;
    }
}

__device__ __forceinline__ void lut_shared_down(const LutArgs &a) {
    const int mc = (a.sh.inter / (a.sh.bits == 8 ? 16 : 32) + 63) / 64;
    if (a.sh.bits == 8) {
        if (mc <= 1) lut_shared_down_rows<8, 1>(a);
        else if (mc <= 2) lut_shared_down_rows<8, 2>(a);
        else lut_shared_down_rows<8, 4>(a);
    } else {
        if (mc <= 1) lut_shared_down_rows<4, 1>(a);
        else if (mc <= 2) lut_shared_down_rows<4, 2>(a);
        else lut_shared_down_rows<4, 4>(a);
    }
}

template <int FMT, bool X31, bool SHX, bool ACT, bool RT>
__global__ __launch_bounds__(LUT_NW * 64) void k_vq_lut(LutArgs a) {
    if constexpr (RT) {
        if (a.sh.h && blockIdx.y == gridDim.y - 1) {      // uniform per block
            lut_shared(a);
            return;
        }
    }
    if constexpr (ACT && !SHX) {
        if (a.sh_out && (int)blockIdx.x >= a.sh_first) {  // uniform per block
            lut_shared_down(a);
            return;
        }
    }
    lut_item<FMT, X31, SHX, ACT, RT, false>(a, blockIdx.x, blockIdx.y, nullptr, nullptr);
}

// ---- the fused decode launch ---------------------------------------------------------
//
// One launch per decode layer instead of three (gate/up, down, combine): the
// units of the two LUT launches and the combine are work items, claimed in
// order from a counter: [0, n_gu) gate/up (row group major, then kind, then
// split), [n_gu, n_gu + n_d) down (pick major, then split), then the
// combine, 64 output rows each. A down item needs the gate/up row groups of
// its inputs complete, the combine every down item: a block counts each
// item it finishes once the item's partial sums are stored (agent-coherent
// stores, complete), waits for the counts it needs (bounded by a poll
// limit) and reads with agent-coherent loads. Items are claimed in order by running blocks,
// so every item an item waits for was claimed before it by a block that
// runs: the launch completes on however many CUs the device gives it. A
// down item loads its codebook, row scales and first code words before it
// waits. Every block routes the token itself (the same picks everywhere)
// and keeps the picks' records and weights in LDS; block 0 also publishes
// idx, w and the job lists. The last block to leave resets the counters for
// the next launch, so a graph can replay it. Partial sums, their layouts,
// split counts and summation orders are those of the three launches, so the
// results are identical to theirs bit for bit.

struct MoeArgs {
    LutArgs gu, dn;            // the gate/up units (kinds 0, 1; routed, gu.r) and the down units (kind 2, act)
    int groups_gu, groups_d, n_comb;
    const float *add0, *add1;  // added to each output in this order (shared expert, residual), or NULL
    float *out;                // [H]
    FzSync sy;
};

// Rows 64 ci .. 64 ci + 63 of the output: each pick's row (its down partial
// sums added in split order, times its row scale), then the weighted sum in
// selection order, then add0 and add1 (k_combine_lut's arithmetic); NaN when a pick,
// in this or an earlier unreported layer, was not computed. yd: LDS, K x 64.
__device__ __forceinline__ void moe_combine_rows(const MoeArgs &m, int ci, const LutPicks &pk, const float *wl,
                                                 int miss, float *yd) {
    const int H = m.dn.M, I = m.dn.N, K = m.dn.max_jobs, splits = m.dn.splits;
    const int row = threadIdx.x & 63, jq = threadIdx.x >> 6, r0 = ci * 64;
    const int i = min(r0 + row, H - 1);
    const size_t nrows = (size_t)((H + 63) >> 6) * 64, stride = (size_t)K * nrows;
    if (!miss) {
        for (int j = jq; j < K; j += LUT_NW) {
            const float *p = m.dn.part + (size_t)j * nrows + i;
            const float v = lut_rowsum8<true>(p, splits, stride);
            gu32 *sc = (gu32 *)((const uint16_t *)(pk.rec[j] + pk.off[j][3]) + 2 * I);
            yd[j * 64 + row] = v * f16_keep((uint16_t)(sc[i >> 1] >> (16 * (i & 1))));
        }
    }
    __syncthreads();
    if (jq == 0 && r0 + row < H) {
        float s = __builtin_nanf("");
        if (!miss) {
            s = 0.0f;
            for (int j = 0; j < K; j++) s = __fadd_rn(s, __fmul_rn(wl[j], yd[j * 64 + row]));
            if (m.add0) s = __fadd_rn(s, m.add0[i]);
            if (m.add1) s = __fadd_rn(s, m.add1[i]);
        }
        m.out[i] = s;
    }
    __syncthreads();
}

// The launch's arguments, read from the kernel argument segment where they
// are used: the address is opaque to the compiler, so that it loads fields
// per item instead of holding every field of both units in scalar registers
// across the item loop.
__device__ __forceinline__ const MoeArgs &moe_args() {
    uint64_t p = (uint64_t)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(p));
    return *(const MoeArgs *)(const __attribute__((address_space(4))) MoeArgs *)p;
}

template <int FMT, bool X31>
__global__ __launch_bounds__(LUT_NW * 64) void k_moe_fused(MoeArgs) {
    extern __shared__ __attribute__((aligned(16))) float lut[];
    __shared__ LutPicks pk;
    __shared__ int r_sel[WARP_MAX_K];
    __shared__ float r_wsel[WARP_MAX_K];
    __shared__ int s_item, s_miss;
    const int tid = threadIdx.x;
    int total;
    unsigned nxt = 0;
    {
    const MoeArgs &m = moe_args();
    const warp_route_args &r = m.gu.r;
    const int E = r.E, E2 = (E + 1) & ~1, K = m.gu.max_jobs;
    total = 2 * m.groups_gu * m.gu.splits + m.groups_d * m.dn.splits + m.n_comb;
    unsigned *ctr = m.sy.ctr;

    // the first claim, the flag an earlier layer may have left, the routing
    int prev = 0;
    if (tid == 0) {
        nxt = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        prev = *(volatile const int *)r.missing & 3;
    }
    float *score = lut, *biased = lut + E2;
    warp_slot *slots = (warp_slot *)(lut + 2 * E2);
    route_in_store(route_in_load(r, tid), E, tid, score, biased, slots);
    route_pick_lds<true, LUT_NW * 64>(E, K, r.act, r.renorm, r.routed_scale, score, biased, r_sel, r_wsel, true,
                                      r.scored != 0);
    const bool miss = picks_missing(slots, r_sel, K);
    if (tid < K) {
        const warp_slot &sl = slots[r_sel[tid]];
        pk.rec[tid] = sl.rec;
#pragma unroll
        for (int k = 0; k < 4; k++) pk.off[tid][k] = sl.off[k];
    }
    if (blockIdx.x == 0) {                                  // uniform per block
        if (tid < K) {
            r.idx[tid] = r_sel[tid];
            r.w[tid] = r_wsel[tid];
        }
        route_jobs<LUT_NW * 64>(r_sel, K, slots, r.jobs, r.njobs, r.missing, r.inter);
    }
    if (tid == 0) {
        pk.nj = miss ? 0 : K;
        s_miss = prev || miss;
        s_item = (int)nxt;
    }
    }
    __syncthreads();                                       // the staging area is the items' from here

    for (;;) {
        const int item = s_item;
        if (item >= total) break;                          // uniform
        const MoeArgs &m = moe_args();
        const int S = m.gu.splits, n_gu = 2 * m.groups_gu * S, n_d = m.groups_d * m.dn.splits;
        unsigned *ctr = m.sy.ctr;
        if (tid == 0) nxt = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (item < n_gu) {
            const int grp = item / (2 * S), rem = item - grp * 2 * S;
            lut_item<FMT, X31, true, false, false, true>(m.gu, grp * S + rem % S, rem / S, &pk, &m.sy);
            wait_stores();
            __syncthreads();
            if (tid == 0)
                __hip_atomic_fetch_add(ctr + (3 + grp) * FZ_LINE, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else if (item < n_gu + n_d) {
            lut_item<FMT, X31, false, true, false, true>(m.dn, item - n_gu, 0, &pk, &m.sy);
            wait_stores();
            __syncthreads();
            if (tid == 0) __hip_atomic_fetch_add(ctr + 2 * FZ_LINE, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            if (tid == 0) fz_wait(ctr + 2 * FZ_LINE, 0, 0, (unsigned)n_d, m.sy);
            __syncthreads();
            moe_combine_rows(m, item - n_gu - n_d, pk, r_wsel, s_miss, lut);
        }
        if (tid == 0) s_item = (int)nxt;
        __syncthreads();
    }
    if (tid == 0) {
        const MoeArgs &m = moe_args();
        unsigned *ctr = m.sy.ctr;
        const unsigned left = __hip_atomic_fetch_add(ctr + FZ_LINE, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (left == gridDim.x - 1)
            for (int g = 0; g < 3 + m.groups_gu; g++)
                __hip_atomic_store(ctr + g * FZ_LINE, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int FMT, bool X31>
static int launch_moe_fused(const MoeArgs &m, int blocks, void *stream) {
    typedef FmtT<FMT> F;
    const size_t lds = ((size_t)2 * 2 * F::S * F::E + LUT_XCH * 16) * sizeof(float);
    if (lds > 163840) return -2;
    static std::atomic<uint64_t> attr{0};
    if (int r_ = lds_limit((const void *)k_moe_fused<FMT, X31>, (int)lds, attr, stream)) return r_;
    hipLaunchKernelGGL((k_moe_fused<FMT, X31>), dim3(blocks), dim3(LUT_NW * 64), lds, (hipStream_t)stream, m);
    CHECK_LAUNCH();
    return 0;
}

extern "C" int wk_lut_plan(int M, int N, int max_jobs, int nkinds, int shared_x, int target_blocks,
                           size_t cap_floats, int *groups_out, int *splits_out) {
    if (M <= 0 || N <= 0 || (N % 16) || max_jobs <= 0 || nkinds < 1 || nkinds > 3) return -1;
    const long nrb = (M + 63) / 64, nc = N / 16;
    const long groups = shared_x ? ((long)max_jobs * nrb + LUT_RBG - 1) / LUT_RBG
                                 : (long)max_jobs * ((nrb + LUT_RBG - 1) / LUT_RBG);
    const long gt = groups * nkinds;
    long splits = target_blocks > gt ? target_blocks / gt : 1;
    // at least two chunks per split: a block that builds one table pays a
    // whole prologue (routing, codebook, first fill) for it (measured at the
    // Kimi-Linear shape: 80 splits of 144 chunks beat 128 by 3-4%)
    if (splits > nc / 2) splits = nc / 2 > 0 ? nc / 2 : 1;
    if (splits < (nc + LUT_XCH - 1) / LUT_XCH) splits = (nc + LUT_XCH - 1) / LUT_XCH;   // x stash
    while (splits > (nc + LUT_XCH - 1) / LUT_XCH && (size_t)nkinds * splits * max_jobs * nrb * 64 > cap_floats)
        splits--;
    if ((size_t)nkinds * splits * max_jobs * nrb * 64 > cap_floats) return -1;
    if (groups * splits > 0x7fffffffL) return -1;
    if (groups_out) *groups_out = (int)groups;
    if (splits_out) *splits_out = (int)splits;
    return 0;
}

template <int FMT, bool X31, bool SHX, bool ACT, bool RT>
static int launch_lut(const LutArgs &a, int groups, int nkinds, void *stream) {
    typedef FmtT<FMT> F;
    const size_t lds = ((size_t)2 * 2 * F::S * F::E + LUT_XCH * 16) * sizeof(float);
    if (lds > 163840) return -2;
    static std::atomic<uint64_t> attr{0};
    if (int r_ = lds_limit((const void *)k_vq_lut<FMT, X31, SHX, ACT, RT>, (int)lds, attr, stream)) return r_;
    const int gx = groups * a.splits, nsh = a.sh_out ? (a.M + LUT_NW * 4 - 1) / (LUT_NW * 4) : 0;
    hipLaunchKernelGGL((k_vq_lut<FMT, X31, SHX, ACT, RT>), dim3(gx + nsh, nkinds + (a.sh.h && !a.sh_out ? 1 : 0)),
                       dim3(LUT_NW * 64), lds, (hipStream_t)stream, a);
    CHECK_LAUNCH();
    return 0;
}

extern "C" int wk_lut_route_ok(int fmt, int E, int K, int shared_x, int kind_lo, int nkinds) {
    int se;
    switch (fmt) {
    case WARP_FMT_VQ3R: se = FmtT<WARP_FMT_VQ3R>::S * FmtT<WARP_FMT_VQ3R>::E; break;
    case WARP_FMT_VQ2R: se = FmtT<WARP_FMT_VQ2R>::S * FmtT<WARP_FMT_VQ2R>::E; break;
    case WARP_FMT_VQ12: se = FmtT<WARP_FMT_VQ12>::S * FmtT<WARP_FMT_VQ12>::E; break;
    default: return 0;
    }
    // one expert per thread; logits, biases and the expert table staged in
    // the table buffers and the input stash
    const size_t stage = (size_t)2 * ((E + 1) & ~1) * sizeof(float) + (size_t)E * sizeof(warp_slot);
    const size_t room = ((size_t)4 * se + LUT_XCH * 16) * sizeof(float);
    return shared_x && kind_lo == 0 && nkinds == 2 && E > 0 && E <= LUT_NW * 64 && E <= 512 && K > 0 &&
           K <= WARP_MAX_K && K <= E && stage <= room;
}

template <int FMT>
static int launch_lut_x(const LutArgs &a, int groups, int nkinds, int x31, void *stream) {
    if (a.shared_x && a.r.table)
        return x31 ? launch_lut<FMT, true, true, false, true>(a, groups, nkinds, stream)
                   : launch_lut<FMT, false, true, false, true>(a, groups, nkinds, stream);
    if (a.shared_x)
        return x31 ? launch_lut<FMT, true, true, false, false>(a, groups, nkinds, stream)
                   : launch_lut<FMT, false, true, false, false>(a, groups, nkinds, stream);
    if (a.act_part)
        return x31 ? launch_lut<FMT, true, false, true, false>(a, groups, nkinds, stream)
                   : launch_lut<FMT, false, false, true, false>(a, groups, nkinds, stream);
    return x31 ? launch_lut<FMT, true, false, false, false>(a, groups, nkinds, stream)
               : launch_lut<FMT, false, false, false, false>(a, groups, nkinds, stream);
}

extern "C" int wk_vq_lut(int fmt, const warp_job *jobs, const int *njobs, int max_jobs, int kind_lo, int nkinds,
                         const uint16_t *books, int books_x31, const float *x, int shared_x, float *part,
                         size_t cap_floats, int M, int N, int target_blocks, const float *act_part,
                         int act_splits, int act_situ, float act_beta, float act_lbeta,
                         const warp_route_args *route, const warp_shared_args *sh, float *sh_out,
                         int *splits_out, void *stream) {
    if (kind_lo < 0 || kind_lo + nkinds > 3 || !books || !part) return -1;
    if (sh && !sh_out && (!route || !wk_shared_fast_ok(N, sh) || (size_t)N * sizeof(float) > 64 * 1024)) return -1;
    // the shared down rows: M rows of sh->inter weights, four per wave
    const int nsh = sh && sh_out ? (M + LUT_NW * 4 - 1) / (LUT_NW * 4) : 0;
    if (sh_out && (!sh || !act_part || sh->inter / (sh->bits == 8 ? 16 : 32) > 64 * 4 ||
                   (size_t)sh->inter * sizeof(float) > 64 * 1024 || nsh >= target_blocks))
        return -1;
    target_blocks -= nsh;
    if (act_part && (shared_x || kind_lo != 2 || nkinds != 1 || act_splits <= 0)) return -1;
    if (route && !wk_lut_route_ok(fmt, route->E, max_jobs, shared_x, kind_lo, nkinds)) return -1;
    int groups, splits;
    if (wk_lut_plan(M, N, max_jobs, nkinds, shared_x, target_blocks, cap_floats, &groups, &splits)) return -1;
    LutArgs a;
    a.jobs = jobs;
    a.njobs = njobs;
    a.max_jobs = max_jobs;
    a.kind_lo = kind_lo;
    a.books = books;
    a.x = x;
    a.part = part;
    a.M = M;
    a.N = N;
    a.splits = splits;
    a.shared_x = shared_x;
    a.act_part = act_part;
    a.act_splits = act_splits;
    a.act_situ = act_situ;
    a.act_beta = act_beta;
    a.act_lbeta = act_lbeta;
    a.r = route ? *route : warp_route_args{};
    a.sh = sh ? *sh : warp_shared_args{};
    a.sh_out = sh_out;
    a.sh_first = groups * splits;
    if (sh && !sh_out && groups * splits * LUT_NW < sh->inter) return -1;   // one row per wave of the extra grid row
    if (splits_out) *splits_out = splits;
    switch (fmt) {
    case WARP_FMT_VQ3R: return launch_lut_x<WARP_FMT_VQ3R>(a, groups, nkinds, books_x31, stream);
    case WARP_FMT_VQ2R: return launch_lut_x<WARP_FMT_VQ2R>(a, groups, nkinds, books_x31, stream);
    case WARP_FMT_VQ12: return launch_lut_x<WARP_FMT_VQ12>(a, groups, nkinds, books_x31, stream);
    }
    return -1;
}

// ---- few experts: decode-then-dot, whole rows per wave --------------------------------
//
// One row's share at one position: its S codebook vectors (fp16, as the
// codebook holds them) added in fp32, dotted with the position's 8 inputs,
// added to acc.
template <int FMT>
__device__ __forceinline__ float ga_row(const uint4 (&v)[FmtT<FMT>::S], const float4 &x0, const float4 &x1,
                                        float acc) {
    float w[8];
    {
        const half8 h = __builtin_bit_cast(half8, v[0]);
#pragma unroll
        for (int i = 0; i < 8; i++) w[i] = (float)h[i];
    }
#pragma unroll
    for (int s = 1; s < FmtT<FMT>::S; s++) {
        const half8 h = __builtin_bit_cast(half8, v[s]);
#pragma unroll
        for (int i = 0; i < 8; i++) w[i] += (float)h[i];
    }
    acc = __builtin_fmaf(w[0], x0.x, acc);
    acc = __builtin_fmaf(w[1], x0.y, acc);
    acc = __builtin_fmaf(w[2], x0.z, acc);
    acc = __builtin_fmaf(w[3], x0.w, acc);
    acc = __builtin_fmaf(w[4], x1.x, acc);
    acc = __builtin_fmaf(w[5], x1.y, acc);
    acc = __builtin_fmaf(w[6], x1.z, acc);
    return __builtin_fmaf(w[7], x1.w, acc);
}

// The row kernel's jobs and inputs: jobs/njobs (max_jobs per kind) or slot
// (or NULL): one expert's FFN, whose jobs come from its expert-table entry
// (record, header offsets; inter gives the scale arrays' places) instead of
// a job list -- no job-list launch; missing: set when the slot has no
// record.
struct GatherArgs {
    const warp_job *jobs;
    const int *njobs;
    int max_jobs, kind_lo;
    const warp_slot *slot;
    int inter;
    const uint16_t *books;     // [3][S][E][8] fp16, subnormals flushed
    const float *x;
    int M, N, shared_x;
    int act_situ;
    float act_beta, act_lbeta;
    int *missing;
};

// Job j of a kind: its index block, row scales and input row (a job list's
// entry, or the slot's record); false when the record is missing.
__device__ __forceinline__ bool ga_job(const GatherArgs &a, int kind, int j, const uint8_t *&idx,
                                       const uint16_t *&scale, int &xi) {
    if (a.slot) {
        const uint8_t *rec = a.slot->rec;
        if (!rec) return false;
        idx = rec + a.slot->off[kind];
        scale = (const uint16_t *)(rec + a.slot->off[3]) + (kind == 0 ? 0 : kind == 1 ? a.inter : 2 * a.inter);
        xi = 0;
        return true;
    }
    const warp_job &jb = a.jobs[(size_t)kind * a.max_jobs + j];
    idx = jb.idx;
    scale = jb.scale;
    xi = jb.xi[0];
    return true;
}

// One matrix, one expert's FFN, or the few experts of a decode, for one
// token: too few rows share a table to pay for it, and a split over
// positions would need a reduction across blocks. Each block (one job's
// quads; blocks of several jobs in turn) stages its kind's fp16 codebook in LDS (128 KiB
// for 2 x 4096 entries, one block per CU; 12 KiB for 3 x 256) and the input,
// then takes row quads (4 consecutive rows: one code word of the record's
// blocked layout per position) RQ at a time: wave w takes quad w % RQ and
// position slice w / RQ of NS, lane l the slice's positions l, l + 64, ...,
// gathering each row's S codebook vectors from LDS, adding them in fp32 and
// dotting them with the position's 8 inputs. The lanes' sums, then the
// slices' in order, give each row; times its scale it is written out. No
// partial sums leave the block, so a launch is the whole matvec. A codebook
// of at most RW_L1 bytes a kind (3 x 256 or 2 x 256 entries) is read from
// global memory instead, where it stays in the L1 cache, so that the
// gathers need not wait for a staging pass.
constexpr int RW_L1 = 16384;

struct RowsArgs {
    GatherArgs g;              // jobs (or slot), max_jobs, books, x, M, N; act inputs below
    float *y[3];               // per kind: job j's rows out (scaled) at y[kind] + j M; ACT
                               // reads job j's gate and up rows at y[0], y[1] + j N
    float *part;               // or NULL: the rows unscaled at part + j nrb 64 (the table
                               // kernel's one-split partial sums, for k_combine_lut)
    int nkinds, gj;            // kinds; blocks per (job, kind): blockIdx.x = j gj + b
};

template <int FMT, bool ACT, int NW>
__global__ __launch_bounds__(NW * 64) void k_vq_rows(RowsArgs ra) {
    typedef FmtT<FMT> F;
    constexpr bool STAGE = F::S * F::E * 16 > RW_L1;      // the codebook in LDS
    const GatherArgs &a = ra.g;
    extern __shared__ __attribute__((aligned(16))) uint4 rw_lds[];
    const uint4 *bk = (const uint4 *)(a.books + (size_t)(a.kind_lo + (int)blockIdx.y) * F::S * F::E * 8);
    uint4 *cbl = rw_lds;                                   // [S][E] half8 (STAGE)
    const uint4 *cb = STAGE ? (const uint4 *)cbl : bk;
    float *xl = (float *)(rw_lds + (STAGE ? F::S * F::E : 0));   // [N]
    __shared__ float red[NW][4];
    __shared__ uint64_t s_exp[32];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kind = a.kind_lo + (int)blockIdx.y;
    const int nv = a.N >> 3, nrq = (a.M + 3) >> 2;
    const int G = ra.gj, j = (int)blockIdx.x / G, b = (int)blockIdx.x - j * G;
    const uint8_t *jidx;
    const uint16_t *jscale;
    int jxi;
    // this block's quads [q0, q1) of job j: the blocks go to the 8 XCDs in
    // turn (block b to XCD b % 8 when G is a multiple of 8), so each XCD takes
    // a contiguous eighth of the quads, shared by its blocks: the record lines
    // a row block's quads share are then fetched into one XCD's L2, not into
    // each. (Fewer than 8 blocks: contiguous shares.)
    int q0, q1;
    if (G >= 8) {
        const int xcd = b % 8, nb = (G - xcd + 7) / 8, slot = b / 8;
        const int qx0 = xcd * nrq / 8, nqx = (xcd + 1) * nrq / 8 - qx0;
        q0 = qx0 + slot * nqx / nb;
        q1 = qx0 + (slot + 1) * nqx / nb;
    } else {
        q0 = b * nrq / G;
        q1 = (b + 1) * nrq / G;
    }
    const int per = q1 - q0;
    if (!ga_job(a, kind, j, jidx, jscale, jxi)) {          // uniform: the slot has no record
        for (int r = q0 * 4 + tid; r < min(q1 * 4, a.M); r += NW * 64) ra.y[kind][r] = __builtin_nanf("");
        if (blockIdx.x == 0 && blockIdx.y == 0 && tid == 0 && a.missing) *a.missing = 1;
        return;
    }
    if (!a.slot && j >= a.njobs[kind]) return;             // uniform
    if (q0 >= q1) return;                                  // uniform
    const int RQ = min(per, NW), NS = NW / RQ;
    const int qw = wave % RQ, sw = wave / RQ;              // this wave's quad in a round, its slice
    const int p0 = sw * nv / NS, p1 = (sw + 1) * nv / NS;  // the slice's positions
    const bool live = sw < NS;
    constexpr int PPL = 4;                                 // positions a lane holds at once
    // the first round's code words (from HBM) before anything else
    auto word_at = [&](int q, int p) -> const uint8_t * {
        return jidx + ((size_t)(q >> 4) * nv + p) * 64 * F::SB + (size_t)(q & 15) * 4 * F::SB;
    };
    Word<F::SB> wd[PPL];
    {
        const int q = q0 + qw;
#pragma unroll
        for (int k = 0; k < PPL; k++) {
            const int p = p0 + lane + 64 * k;
            if (live && q < q1 && p < p1) wd[k].load_keep(word_at(q, p));
        }
    }
    // the codebook and the input, into LDS
    if constexpr (STAGE)
        for (int i = tid; i < F::S * F::E; i += NW * 64) cbl[i] = bk[i];
    if constexpr (ACT) {
        if (tid < 32) s_exp[tid] = g_exp2_tab[tid];
        __syncthreads();
        const float *g0 = ra.y[0] + (size_t)j * a.N, *u0 = ra.y[1] + (size_t)j * a.N;
        for (int i = tid; i < a.N; i += NW * 64) xl[i] = act_pair(g0[i], u0[i], a.act_situ, a.act_beta, a.act_lbeta, s_exp);
    } else {
        const float *xs = a.x + (a.shared_x ? (size_t)0 : (size_t)jxi * a.N);
        for (int i = tid * 4; i < a.N; i += NW * 64 * 4) *(float4 *)(xl + i) = *(const float4 *)(xs + i);
    }
    __syncthreads();

    for (int qb = q0; qb < q1; qb += RQ) {
        const int q = qb + qw;
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (live && q < q1) {                              // uniform per wave
            for (int pb = p0; pb < p1; pb += 64 * PPL) {
#pragma unroll
                for (int k = 0; k < PPL; k++) {
                    const int p = pb + lane + 64 * k;
                    if (p < p1) {
                        const Word<F::SB> w = wd[k];
                        if (p + 64 * PPL < p1) wd[k].load_keep(word_at(q, p + 64 * PPL));
                        const float4 x0 = *(const float4 *)(xl + 8 * p);
                        const float4 x1 = *(const float4 *)(xl + 8 * p + 4);
#pragma unroll
                        for (int t = 0; t < 4; t++) {
                            const unsigned sl = w.slot(t);
                            uint4 v[F::S];
#pragma unroll
                            for (int s = 0; s < F::S; s++) v[s] = cb[s * F::E + lut_code<FMT>(sl, s)];
                            acc[t] = ga_row<FMT>(v, x0, x1, acc[t]);
                        }
                    }
                }
            }
            // the next round's first code words
            const int qn = q + RQ;
#pragma unroll
            for (int k = 0; k < PPL; k++) {
                const int p = p0 + lane + 64 * k;
                if (qn < q1 && p < p1) wd[k].load_keep(word_at(qn, p));
            }
        }
#pragma unroll
        for (int t = 0; t < 4; t++) acc[t] = wave_sum(acc[t]);
        if (lane == 0) *(float4 *)red[wave] = make_float4(acc[0], acc[1], acc[2], acc[3]);
        __syncthreads();
        if (tid < 4 * RQ) {
            const int qq = qb + tid / 4, r = 4 * qq + (tid & 3);
            if (qq < q1 && r < a.M) {
                float v = red[tid / 4][tid & 3];
                for (int s = 1; s < NS; s++) v += red[s * RQ + tid / 4][tid & 3];
                if (ra.part) ra.part[(size_t)j * (((a.M + 63) >> 6) * 64) + r] = v;
                else ra.y[kind][(size_t)j * a.M + r] = v * f16_keep(jscale[r]);
            }
        }
        __syncthreads();
    }
}

template <int FMT, bool ACT>
static int launch_rows(const RowsArgs &ra, int target_blocks, void *stream) {
    typedef FmtT<FMT> F;
    // a staged codebook: one block of 16 waves per CU; else blocks of 4
    // waves, four per CU
    constexpr bool STAGE = F::S * F::E * 16 > RW_L1;
    constexpr int NW = STAGE ? 16 : 4;
    if (!STAGE) target_blocks *= 4;
    const size_t lds = (F::S * F::E * 16 > RW_L1 ? (size_t)F::S * F::E * 16 : 0) + (size_t)ra.g.N * sizeof(float);
    if (lds > 160 * 1024 - 1024) return -2;
    static std::atomic<uint64_t> attr{0};
    if (int r_ = lds_limit((const void *)k_vq_rows<FMT, ACT, NW>, (int)lds, attr, stream)) return r_;
    const int nrq = (ra.g.M + 3) / 4;
    RowsArgs r = ra;
    int G = target_blocks / (ra.nkinds * ra.g.max_jobs);
    if (G > nrq) G = nrq;
    if (G < 1) G = 1;
    r.gj = G;
    hipLaunchKernelGGL((k_vq_rows<FMT, ACT, NW>), dim3(G * ra.g.max_jobs, ra.nkinds), dim3(NW * 64), lds,
                       (hipStream_t)stream, r);
    CHECK_LAUNCH();
    return 0;
}

extern "C" int wk_vq_rows(int fmt, const warp_job *jobs, const int *njobs, int max_jobs, int kind_lo, int nkinds,
                          const uint16_t *books, const float *x, int M, int N, const warp_slot *slot, int inter,
                          int act_situ, float act_beta, float act_lbeta, float *const *y, float *part, int *missing,
                          int target_blocks, void *stream) {
    if (kind_lo < 0 || kind_lo + nkinds > 3 || !books || !y || M <= 0 || N <= 0 || (N % 32) || max_jobs < 1)
        return -1;
    if (slot ? (inter <= 0 || max_jobs != 1) : (!jobs || !njobs)) return -1;
    const bool act = x == nullptr;                         // down: inputs act(y[0], y[1])
    if (act && (kind_lo != 2 || nkinds != 1 || !y[0] || !y[1])) return -1;
    if (part && (kind_lo != 2 || nkinds != 1)) return -1;
    for (int k = kind_lo; k < kind_lo + nkinds; k++)
        if (!y[k] && !part) return -1;
    RowsArgs ra = {};
    GatherArgs &a = ra.g;
    a.jobs = jobs;
    a.njobs = njobs;
    a.max_jobs = max_jobs;
    ra.part = part;
    a.kind_lo = kind_lo;
    a.slot = slot;
    a.inter = inter;
    a.books = books;
    a.x = x;
    a.M = M;
    a.N = N;
    a.shared_x = 1;
    a.act_situ = act_situ;
    a.act_beta = act_beta;
    a.act_lbeta = act_lbeta;
    a.missing = missing;
    for (int k = 0; k < 3; k++) ra.y[k] = y[k];
    ra.nkinds = nkinds;
    switch (fmt) {
    case WARP_FMT_VQ3R: return act ? launch_rows<WARP_FMT_VQ3R, true>(ra, target_blocks, stream)
                                   : launch_rows<WARP_FMT_VQ3R, false>(ra, target_blocks, stream);
    case WARP_FMT_VQ2R: return act ? launch_rows<WARP_FMT_VQ2R, true>(ra, target_blocks, stream)
                                   : launch_rows<WARP_FMT_VQ2R, false>(ra, target_blocks, stream);
    case WARP_FMT_VQ12: return act ? launch_rows<WARP_FMT_VQ12, true>(ra, target_blocks, stream)
                                   : launch_rows<WARP_FMT_VQ12, false>(ra, target_blocks, stream);
    }
    return -1;
}

extern "C" int wk_moe_fused(int fmt, const uint16_t *books, int books_x31, const float *x, int K, int I, int H,
                            float *part, size_t cap_floats, int n_cu, int act_situ, float act_beta,
                            float act_lbeta, const warp_route_args *route, const float *add0, const float *add1,
                            float *out, unsigned *sync, int sync_words, void *stream) {
    if (!books || !x || !part || !route || !out || !sync || n_cu < 1) return -1;
    if (!wk_lut_route_ok(fmt, route->E, K, 1, 0, 2)) return -1;
    int groups_gu, splits_gu, groups_d, splits_d;
    if (wk_lut_plan(I, H, K, 2, 1, n_cu, cap_floats, &groups_gu, &splits_gu)) return -1;
    const size_t gu_floats = (size_t)2 * splits_gu * K * (((size_t)I + 63) / 64) * 64;
    if (gu_floats > cap_floats || wk_lut_plan(H, I, K, 1, 0, n_cu, cap_floats - gu_floats, &groups_d, &splits_d))
        return -1;
    if ((size_t)(3 + groups_gu) * FZ_LINE > (size_t)sync_words) return -1;
    MoeArgs m = {};
    LutArgs &g = m.gu, &d = m.dn;
    g.jobs = route->jobs;
    g.njobs = route->njobs;
    g.max_jobs = K;
    g.kind_lo = 0;
    g.books = books;
    g.x = x;
    g.part = part;
    g.M = I;
    g.N = H;
    g.splits = splits_gu;
    g.shared_x = 1;
    g.r = *route;
    d = g;
    d.kind_lo = 2;
    d.x = nullptr;
    d.part = part + gu_floats;
    d.M = H;
    d.N = I;
    d.splits = splits_d;
    d.shared_x = 0;
    d.act_part = part;
    d.act_splits = splits_gu;
    d.act_situ = act_situ;
    d.act_beta = act_beta;
    d.act_lbeta = act_lbeta;
    m.groups_gu = groups_gu;
    m.groups_d = groups_d;
    m.n_comb = (H + 63) / 64;
    m.add0 = add0;
    m.add1 = add1;
    m.out = out;
    m.sy.ctr = sync;
    m.sy.flag = route->missing;
    m.sy.limit = 1u << 20;
    const int items = 2 * groups_gu * splits_gu + groups_d * splits_d + m.n_comb;
    const int blocks = n_cu < items ? n_cu : items;
    switch (fmt) {
    case WARP_FMT_VQ3R:
        return books_x31 ? launch_moe_fused<WARP_FMT_VQ3R, true>(m, blocks, stream)
                         : launch_moe_fused<WARP_FMT_VQ3R, false>(m, blocks, stream);
    case WARP_FMT_VQ2R:
        return books_x31 ? launch_moe_fused<WARP_FMT_VQ2R, true>(m, blocks, stream)
                         : launch_moe_fused<WARP_FMT_VQ2R, false>(m, blocks, stream);
    case WARP_FMT_VQ12:
        return books_x31 ? launch_moe_fused<WARP_FMT_VQ12, true>(m, blocks, stream)
                         : launch_moe_fused<WARP_FMT_VQ12, false>(m, blocks, stream);
    }
    return -1;
}


// y_kind[yi][r] = (sum of the partials) * row scale, for every job of each kind.
__global__ __launch_bounds__(256) void k_lut_reduce(const warp_job *__restrict__ jobs, const int *__restrict__ njobs,
                                                    int max_jobs, int kind_lo, const float *__restrict__ part,
                                                    int splits, int M, float *y0, float *y1, float *y2) {
    const int kk = blockIdx.z, kind = kind_lo + kk, j = blockIdx.y, r = blockIdx.x * 256 + threadIdx.x;
    if (j >= njobs[kind] || r >= M) return;
    const size_t nrows = (size_t)((M + 63) >> 6) * 64, stride = (size_t)max_jobs * nrows;
    const warp_job &jb = jobs[(size_t)kind * max_jobs + j];
    const float v = lut_rowsum(part + (size_t)kk * splits * stride + (size_t)j * nrows + r, splits, stride);
    float *y = kind == 0 ? y0 : kind == 1 ? y1 : y2;
    y[(size_t)jb.yi[0] * M + r] = v * f16_keep(jb.scale[r]);
}

extern "C" int wk_lut_reduce(const warp_job *jobs, const int *njobs, int max_jobs, int kind_lo, int nkinds,
                             const float *part, int splits, int M, float *const *y, void *stream) {
    if (M <= 0 || max_jobs <= 0 || splits <= 0 || kind_lo < 0 || nkinds < 1 || kind_lo + nkinds > 3) return -1;
    hipLaunchKernelGGL(k_lut_reduce, dim3((M + 255) / 256, max_jobs, nkinds), dim3(256), 0, (hipStream_t)stream, jobs,
                       njobs, max_jobs, kind_lo, part, splits, M, y[0], y[1], y[2]);
    CHECK_LAUNCH();
    return 0;
}

// Decode: down partials -> out[r] = sum_j w[j] * y_j[r] in selection order
// (unfused, as k_combine), + add0 + add1. One block per 16 rows: the K
// expert outputs of those rows are reduced in parallel into LDS (one thread
// per expert and row), then one thread per row combines them in order. Every
// load that does not depend on another is issued first (the partial sums,
// the weights, the addends); only the row scale waits for its job entry.
// SHB (8 or 4): add0 is the shared expert's down rows of this block against
// sa.h, one wave per 4 rows, their weights loaded first.
// A block of the combine takes 16 rows, half of a 128-byte line of every
// partial-sum row it reads: neighbouring blocks share each line, and
// xcd_pair_block puts them on one XCD, so the line is fetched into one L2.
__device__ __forceinline__ int combine_r0() { return xcd_pair_block((int)blockIdx.x) * 16; }

template <int SHB, int MC>
__global__ __launch_bounds__(256) void k_combine_lut(const warp_job *__restrict__ jobs2, const float *__restrict__ part,
                                                     int splits, int max_jobs, const float *__restrict__ w, int K,
                                                     int H, const float *add0, const float *add1,
                                                     const int *missing, warp_shared_args sa,
                                                     float *__restrict__ out) {
    __shared__ float yd[WARP_MAX_K][16];
    __shared__ float wl[WARP_MAX_K];
    __shared__ float shd[16];
    extern __shared__ float hl[];
    const int r0 = combine_r0(), row = threadIdx.x & 15, jq = threadIdx.x >> 4;
    const int i = min(r0 + row, H - 1);
    using Q = QRow<SHB ? SHB : 8, MC>;
    Q qd[4];
    const int snc = SHB ? sa.inter / Q::WPC : 0;
    if constexpr (SHB != 0) {
        const int sng = sa.inter / sa.group;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int rr = min(r0 + (int)(threadIdx.x >> 6) * 4 + k, H - 1);
            qd[k].load(sa.q[2] + (size_t)rr * sa.rowbytes[2], sa.s[2] + (size_t)rr * sng, sa.group, snc);
        }
        for (int q = threadIdx.x; q < sa.inter / 4; q += 256) ((float4 *)hl)[q] = ((const float4 *)sa.h)[q];
    }
    const size_t nrows = (size_t)((H + 63) >> 6) * 64, stride = (size_t)max_jobs * nrows;
    // (volatile: read here, not after the barrier where it is used)
    const bool miss = missing && *(volatile const int *)missing;
    const float wv = threadIdx.x < K ? w[threadIdx.x] : 0.0f;
    const float a0 = jq == 0 && add0 ? add0[i] : 0.0f;
    const float a1 = jq == 0 && add1 ? add1[i] : 0.0f;
    // expert j's output at row i: its partial sums, then times the row scale
    // (the scale arrays of a record are 4-byte aligned: the word holding row
    // i's scale; a missing expert has no scale pointer)
    auto expert_row = [&](int j, float v) {
        gu32 *sc = (gu32 *)jobs2[j].scale;
        const unsigned sw = sc ? sc[i >> 1] : 0u;
        yd[j][row] = v * f16_keep((uint16_t)(sw >> (16 * (i & 1))));
    };
    if (K <= 16 && splits <= 16) {                         // one expert per thread
        if (jq < K) expert_row(jq, lut_rowsum_n<16>(part + (size_t)jq * nrows + i, splits, stride));
    } else if (K <= 16 && splits <= 32) {                  // the same, 32 loads in flight
        if (jq < K) expert_row(jq, lut_rowsum_n<32>(part + (size_t)jq * nrows + i, splits, stride));
    } else {
        for (int j = jq; j < K; j += 16) expert_row(j, lut_rowsum8(part + (size_t)j * nrows + i, splits, stride));
    }
    if (threadIdx.x < K) wl[threadIdx.x] = wv;
    __syncthreads();
    if constexpr (SHB != 0) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float v = qd[k].dot(hl, snc);
            if ((threadIdx.x & 63) == 0) shd[(threadIdx.x >> 6) * 4 + k] = v;
        }
        __syncthreads();
    }
    if (jq != 0 || r0 + row >= H) return;
    if (miss) {                         // a selected expert was not computed
        out[i] = __builtin_nanf("");
        return;
    }
    float s = 0.0f;
    for (int j = 0; j < K; j++) s = __fadd_rn(s, __fmul_rn(wl[j], yd[j][row]));
    if (SHB) s = __fadd_rn(s, shd[row]);
    else if (add0) s = __fadd_rn(s, a0);
    if (add1) s = __fadd_rn(s, a1);
    out[i] = s;
}

extern "C" int wk_combine_lut(const warp_job *jobs2, const float *part, int splits, int max_jobs, const float *w,
                              int K, int H, const float *add0, const float *add1, const int *missing,
                              const warp_shared_args *sa, float *out, void *stream) {
    if (K <= 0 || K > WARP_MAX_K || H <= 0 || splits <= 0 || K > max_jobs) return -1;
    const dim3 grid((H + 15) / 16);
    if (sa) {
        /* the shared down rows: H rows of sa->inter weights */
        warp_shared_args d = *sa;
        if (!wk_shared_fast_ok(H, sa) || add0 || d.inter / (d.bits == 8 ? 16 : 32) > 64 * 4 ||
            (size_t)d.inter * sizeof(float) > 64 * 1024)
            return -1;
        const size_t lds = (size_t)d.inter * sizeof(float);
        /* chunks per lane: the fewest that cover a shared down row */
        const int mc = (d.inter / (d.bits == 8 ? 16 : 32) + 63) / 64;
#define CL(b, n)                                                                                                   \
    hipLaunchKernelGGL((k_combine_lut<b, n>), grid, dim3(256), lds, (hipStream_t)stream, jobs2, part, splits,       \
                       max_jobs, w, K, H, add0, add1, missing, d, out)
        if (d.bits == 8) {
            if (mc <= 1) CL(8, 1);
            else if (mc <= 2) CL(8, 2);
            else CL(8, 4);
        } else {
            if (mc <= 1) CL(4, 1);
            else if (mc <= 2) CL(4, 2);
            else CL(4, 4);
        }
#undef CL
    } else {
        const warp_shared_args none = {};
        hipLaunchKernelGGL((k_combine_lut<0, 1>), grid, dim3(256), 0, (hipStream_t)stream, jobs2, part, splits,
                           max_jobs, w, K, H, add0, add1, missing, none, out);
    }
    CHECK_LAUNCH();
    return 0;
}

// ---- decoded weights ------------------------------------------------------------------

template <int FMT>
__device__ __forceinline__ unsigned code_at(const uint8_t *p, int s) {
    if (FMT == WARP_FMT_VQ12) {
        const unsigned w = (unsigned)p[0] | ((unsigned)p[1] << 8) | ((unsigned)p[2] << 16);
        return s == 0 ? (w & 0xFFFu) : (w >> 12);
    }
    if (FMT == WARP_FMT_VQ4P) {
        const unsigned b0 = p[0], b1 = p[1], b2 = p[2];
        switch (s) {
        case 0: return b0 & 0x3f;
        case 1: return ((b0 >> 6) | (b1 << 2)) & 0x3f;
        case 2: return ((b1 >> 4) | (b2 << 4)) & 0x3f;
        default: return (b2 >> 2) & 0x3f;
        }
    }
    return p[s];
}

template <int FMT, int S, int E, int SB>
__global__ __launch_bounds__(256) void k_decode(const uint8_t *__restrict__ idx, const uint16_t *__restrict__ scale,
                                                const uint16_t *__restrict__ books, int M, int N,
                                                float *__restrict__ W) {
    const int nv = N >> 3;
    const long q = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= (long)M * nv) return;
    const int r = (int)(q / nv), v = (int)(q % nv);
    const uint8_t *p = idx + (((size_t)(r >> 6) * nv + v) * 64 + (r & 63)) * SB;
    const float sr = f16_keep(scale[r]);
    for (int d = 0; d < 8; d++) {
        float t = f16_flushed(books[((size_t)0 * E + code_at<FMT>(p, 0)) * 8 + d]);
        for (int s = 1; s < S; s++) t = __fadd_rn(t, f16_flushed(books[((size_t)s * E + code_at<FMT>(p, s)) * 8 + d]));
        W[(size_t)r * N + 8 * v + d] = __fmul_rn(t, sr);
    }
}

extern "C" int wk_decode_weights(int fmt, const uint8_t *idx, const uint16_t *scale, const uint16_t *books, int M,
                                 int N, float *W, void *stream) {
    if (M <= 0 || N <= 0 || (N & 7)) return -1;
    const long n = (long)M * (N / 8);
    const dim3 grid((unsigned)((n + 255) / 256)), blk(256);
    hipStream_t s = (hipStream_t)stream;
    switch (fmt) {
    case WARP_FMT_VQ3R: hipLaunchKernelGGL((k_decode<WARP_FMT_VQ3R, 3, 256, 3>), grid, blk, 0, s, idx, scale, books, M, N, W); break;
    case WARP_FMT_VQ2R: hipLaunchKernelGGL((k_decode<WARP_FMT_VQ2R, 2, 256, 2>), grid, blk, 0, s, idx, scale, books, M, N, W); break;
    case WARP_FMT_VQ4P: hipLaunchKernelGGL((k_decode<WARP_FMT_VQ4P, 4, 64, 3>), grid, blk, 0, s, idx, scale, books, M, N, W); break;
    case WARP_FMT_VQ12: hipLaunchKernelGGL((k_decode<WARP_FMT_VQ12, 2, 4096, 3>), grid, blk, 0, s, idx, scale, books, M, N, W); break;
    default: return -1;
    }
    CHECK_LAUNCH();
    return 0;
}

// ---- activation --------------------------------------------------------------------------

__global__ __launch_bounds__(1024) void k_act_split(const float *__restrict__ g, const float *__restrict__ u, int I,
                                                    int situ, float beta, float lbeta, _Float16 *__restrict__ xs,
                                                    float *__restrict__ xscale, float *__restrict__ h_out) {
    const int p = blockIdx.x;
    extern __shared__ float lds_h[];
    const float *gp = g + (size_t)p * I, *up = u + (size_t)p * I;
    float gv[4], uv[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int i = threadIdx.x + k * 1024;
        gv[k] = i < I ? gp[i] : 0.0f;
        uv[k] = i < I ? up[i] : 0.0f;
    }
    float m = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int i = threadIdx.x + k * 1024;
        if (i < I) {
            const float h = act_pair(gv[k], uv[k], situ, beta, lbeta);
            lds_h[i] = h;
            m = fmaxf(m, fabsf(h));
        }
    }
    for (int i = threadIdx.x + 4 * 1024; i < I; i += 1024) {
        const float h = act_pair(gp[i], up[i], situ, beta, lbeta);
        lds_h[i] = h;
        m = fmaxf(m, fabsf(h));
    }
    m = block_absmax(m);
    const int k = split_exp(m);
    _Float16 *o = xs + (size_t)p * I * 2;
    for (int i = threadIdx.x; i < I; i += blockDim.x) {
        const float h = lds_h[i];
        split_store(h, k, &o[(i >> 3) * 16 + (i & 7)], &o[(i >> 3) * 16 + 8 + (i & 7)]);
        if (h_out) h_out[(size_t)p * I + i] = h;
    }
    if (threadIdx.x == 0) xscale[p] = ldexpf(1.0f, -k);
}

extern "C" int wk_act_split(const float *g, const float *u, int P, int I, int act_situ, float beta, float lbeta,
                            uint16_t *xs, float *xscale, float *h_out, void *stream) {
    if (P <= 0 || I <= 0 || (I & 7) || I > 16384) return -1;
    if (I <= 4096 && (((uintptr_t)g | (uintptr_t)u | (uintptr_t)xs | (uintptr_t)h_out) & 15) == 0)
        return launch_split_w<true>(g, u, P, I, act_situ, beta, lbeta, xs, xscale, h_out, stream);
    hipLaunchKernelGGL(k_act_split, dim3(P), dim3(1024), (size_t)I * sizeof(float), (hipStream_t)stream, g, u, I,
                       act_situ, beta, lbeta, (_Float16 *)xs, xscale, h_out);
    CHECK_LAUNCH();
    return 0;
}

__global__ __launch_bounds__(256) void k_act(const float *__restrict__ g, const float *__restrict__ u, long n,
                                             int situ, float beta, float lbeta, float *__restrict__ h) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) h[i] = act_pair(g[i], u[i], situ, beta, lbeta);
}

extern "C" int wk_act(const float *g, const float *u, int P, int I, int act_situ, float beta, float lbeta, float *h,
                      void *stream) {
    if (P <= 0 || I <= 0) return -1;
    const long n = (long)P * I;
    hipLaunchKernelGGL(k_act, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, g, u, n, act_situ,
                       beta, lbeta, h);
    CHECK_LAUNCH();
    return 0;
}

// ---- combine ---------------------------------------------------------------------------------

__global__ __launch_bounds__(256) void k_combine(const float *__restrict__ y, const float *__restrict__ w, int K,
                                                 int H, const float *__restrict__ add0,
                                                 const float *__restrict__ add1, const int *__restrict__ missing,
                                                 float *__restrict__ out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= H) return;
    if (missing && *missing) {          // a selected expert was not computed
        out[i] = __builtin_nanf("");
        return;
    }
    float s = 0.0f;
    for (int j = 0; j < K; j++) s = __fadd_rn(s, __fmul_rn(w[j], y[(size_t)j * H + i]));
    if (add0) s = __fadd_rn(s, add0[i]);
    if (add1) s = __fadd_rn(s, add1[i]);
    out[i] = s;
}

extern "C" int wk_combine(const float *y, const float *w, int K, int H, const float *add0, const float *add1,
                          const int *missing, float *out, void *stream) {
    if (K <= 0 || H <= 0) return -1;
    hipLaunchKernelGGL(k_combine, dim3((H + 255) / 256), dim3(256), 0, (hipStream_t)stream, y, w, K, H, add0, add1,
                       missing, out);
    CHECK_LAUNCH();
    return 0;
}

// ---- VQ4P: int8 LUT and its apply ------------------------------------------------------------

// One block per (vector, 32-position block): the fp32 LUT entries with the
// fused d-ascending chain of the reference's AVX-512 build
// (src/simd_avx512.c:90-123), then max|.|, scale = max/127, ties-to-even
// rounding and the +-127 clamp (src/model.c:2048-2109).
__global__ __launch_bounds__(256) void k_lut_p6(const float *__restrict__ x, int N,
                                                const uint16_t *__restrict__ books, int8_t *__restrict__ lut8,
                                                float *__restrict__ lscale) {
    __shared__ float lut[WARP_LUT_BLK * 256];
    __shared__ float xsh[WARP_LUT_BLK * 8];
    const int vec = blockIdx.y, blk = blockIdx.x, nv = N >> 3;
    const int v0 = blk * WARP_LUT_BLK, v1 = min(v0 + WARP_LUT_BLK, nv), nvb = v1 - v0;
    const float *xv = x + (size_t)vec * N;
    for (int i = threadIdx.x; i < nvb * 8; i += blockDim.x) xsh[i] = xv[v0 * 8 + i];
    __syncthreads();
    float m = 0.0f;
    for (int q = threadIdx.x; q < nvb * 256; q += blockDim.x) {
        const int v = q >> 8, s = (q >> 6) & 3, c = q & 63;
        float t = 0.0f;
        for (int d = 0; d < 8; d++)
            t = __builtin_fmaf(xsh[v * 8 + d], f16_flushed(books[((size_t)s * 64 + c) * 8 + d]), t);
        lut[q] = t;
        m = fmaxf(m, fabsf(t));
    }
    m = block_absmax(m);
    const float inv = m > 0.0f ? __fdiv_rn(127.0f, m) : 0.0f;
    int8_t *dst = lut8 + ((size_t)vec * nv + v0) * 256;
    for (int q = threadIdx.x; q < nvb * 256; q += blockDim.x) {
        int t = (int)rintf(__fmul_rn(lut[q], inv));
        t = t > 127 ? 127 : (t < -127 ? -127 : t);
        dst[q] = (int8_t)t;
    }
    if (threadIdx.x == 0) lscale[(size_t)vec * ((nv + WARP_LUT_BLK - 1) / WARP_LUT_BLK) + blk] = __fdiv_rn(m, 127.0f);
}

extern "C" int wk_lut_p6(const float *x, int V, int N, const uint16_t *books_kind, int8_t *lut8, float *lscale,
                         void *stream) {
    if (V <= 0 || N <= 0 || (N & 7)) return -1;
    const int nv = N / 8, nblk = (nv + WARP_LUT_BLK - 1) / WARP_LUT_BLK;
    hipLaunchKernelGGL(k_lut_p6, dim3(nblk, V), dim3(256), 0, (hipStream_t)stream, x, N, books_kind, lut8, lscale);
    CHECK_LAUNCH();
    return 0;
}

// One wave per (job, 64-row block), lane = row: integer block sums of the
// four int8 lookups, folded into fp32 once per 32 positions in the
// reference's order (src/model.c:2136-2229, portable branch).
__global__ __launch_bounds__(256) void k_apply_p6(const warp_job *__restrict__ jobs, const int *__restrict__ njobs,
                                                  int kind, const int8_t *__restrict__ lut8,
                                                  const float *__restrict__ lscale, float *__restrict__ y, int M,
                                                  int N) {
    const int nv = N >> 3, nrb = (M + 63) >> 6, nblk = (nv + WARP_LUT_BLK - 1) / WARP_LUT_BLK;
    const int unit = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (unit >= njobs[kind] * nrb) return;
    const warp_job &jb = jobs[unit / nrb];
    const int rb = unit % nrb, r = rb * 64 + lane;
    const uint8_t *idx = jb.idx;
    for (int ts = 0; ts < jb.n; ts++) {
    const int8_t *T0 = lut8 + (size_t)jb.xi[ts] * nv * 256;
    const float *ls = lscale + (size_t)jb.xi[ts] * nblk;
    float acc = 0.0f;
    for (int b = 0; b < nblk; b++) {
        const int v0 = b * WARP_LUT_BLK, v1 = min(v0 + WARP_LUT_BLK, nv);
        int sum = 0;
        for (int v = v0; v < v1; v++) {
            const uint8_t *p = idx + (((size_t)rb * nv + v) * 64 + lane) * 3;
            const int8_t *T = T0 + (size_t)v * 256;
            sum += T[code_at<WARP_FMT_VQ4P>(p, 0)] + T[64 + code_at<WARP_FMT_VQ4P>(p, 1)] +
                   T[128 + code_at<WARP_FMT_VQ4P>(p, 2)] + T[192 + code_at<WARP_FMT_VQ4P>(p, 3)];
        }
        acc = __fadd_rn(acc, __fmul_rn(ls[b], (float)sum));
    }
    if (r < M) y[(size_t)jb.yi[ts] * M + r] = __fmul_rn(acc, f16_keep(jb.scale[r]));
    }
}

extern "C" int wk_apply_p6(const warp_job *jobs, const int *njobs, int max_jobs, int kind, const int8_t *lut8,
                           const float *lscale, float *y, int M, int N, void *stream) {
    if (M <= 0 || N <= 0 || (N & 7) || kind < 0 || kind > 2 || max_jobs <= 0) return -1;
    const int nrb = (M + 63) / 64, units = max_jobs * nrb;
    hipLaunchKernelGGL(k_apply_p6, dim3((units + 3) / 4), dim3(256), 0, (hipStream_t)stream,
                       jobs + (size_t)kind * max_jobs, njobs, kind, lut8, lscale, y, M, N);
    CHECK_LAUNCH();
    return 0;
}

// ---- prefill grouping ----------------------------------------------------------------------------

// One block. Counts per expert, exclusive scan, then one thread per expert
// places its pairs in token order and cuts them into jobs of WARP_TPJ.
// A pair (t, k) is computed when it is token t's first pick of its expert
// and its weight is not 0 (moe_chunk takes the first pick's weight and
// skips 0, src/model.c:3631-3636); the others get slot -1.

// Exclusive prefix sum of v over the block (blockDim a multiple of 64, at
// most 1024 threads); *total gets the block's sum. tmp: 16 ints of LDS.
// Every thread of the block calls it.
__device__ __forceinline__ int block_scan_excl(int v, int *tmp, int &total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
    if (lane == 63) tmp[wave] = x;
    __syncthreads();
    int base = 0, tot = 0;
    for (int w = 0; w < nw; w++) {
        const int t = tmp[w];
        base += w < wave ? t : 0;
        tot += t;
    }
    __syncthreads();
    total = tot;
    return base + x - v;
}

// The same for a 64-bit value (three 21-bit counters packed in one: one
// scan instead of three). tmp: 16 64-bit words of LDS.
__device__ __forceinline__ unsigned long long block_scan_excl64(unsigned long long v, unsigned long long *tmp,
                                                                unsigned long long &total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    unsigned long long x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned lo = __shfl_up((unsigned)x, o), hi = __shfl_up((unsigned)(x >> 32), o);
        if (lane >= o) x += ((unsigned long long)hi << 32) | lo;
    }
    if (lane == 63) tmp[wave] = x;
    __syncthreads();
    unsigned long long base = 0, tot = 0;
    for (int w = 0; w < nw; w++) {
        const unsigned long long t = tmp[w];
        base += w < wave ? t : 0ull;
        tot += t;
    }
    __syncthreads();
    total = tot;
    return base + x - v;
}

// One block. The picks are staged in LDS; each expert gets a bitmap of the
// tokens that pick it (in LDS when it fits, else the pairs are found by a
// scan per expert); a pair's place in its expert's list is the number of
// earlier tokens in that bitmap, its slot in its token's list the number
// of the token's computed picks with a lower expert id.
__global__ __launch_bounds__(1024) void k_plan_chunk(const int *__restrict__ idx, const float *__restrict__ w, int T,
                                                     int K, int E, const warp_slot *__restrict__ table,
                                                     int *__restrict__ counts, int *__restrict__ offsets,
                                                     int *__restrict__ pair_tok, int *__restrict__ pair_exp,
                                                     float *__restrict__ pair_w, int *__restrict__ tok_slots,
                                                     warp_job *__restrict__ jobs, int max_jobs,
                                                     int *__restrict__ njobs, int *__restrict__ runs,
                                                     int *__restrict__ missing, int inter, int bitmaps,
                                                     int e_lo, int e_hi, int or_missing) {
    extern __shared__ __attribute__((aligned(16))) int lds_plan[];
    // token bitmap rows of NWP words: an odd stride, so the rows that a
    // wave's pairs read in one step fall on different LDS banks
    const int P = T * K, NWP = ((T + 31) >> 5) | 1;
    warp_slot *stab = (warp_slot *)lds_plan;        // [E] the expert table, read once
    int *pid = (int *)(stab + E);                   // [P]
    int *cnt = pid + P;                             // [E]
    int *off = cnt + E;                             // [E]
    int *tile0 = off + E;                           // [E]
    int *run0 = tile0 + E;                          // [E] place of the expert's first full run
    int *runr = run0 + E;                           // [E] place of its last, partial run
    unsigned *bm = (unsigned *)(runr + E);          // [E][NWP] when bitmaps
    int *ptok = (int *)(bm + (bitmaps ? E * NWP : 0));                    // [P] pair_tok, kept on chip
    unsigned char *pv = (unsigned char *)(ptok + P);                     // [P] pair computed
    // Up to PPT pairs per thread: their picks and weights loaded at once
    // (clamped, so no load waits on another) and the weights kept in
    // registers for the pair loops below; larger batches loop.
    constexpr int PPT = 8;
    const bool regs = P <= PPT * 1024;              // uniform (blockDim 1024)
    float wr[PPT];
    if (regs) {
        int ir[PPT];
#pragma unroll
        for (int i = 0; i < PPT; i++) {
            const int q = min((int)threadIdx.x + i * 1024, P - 1);
            ir[i] = idx[q];
            wr[i] = w[q];
        }
#pragma unroll
        for (int i = 0; i < PPT; i++)
            if ((int)threadIdx.x + i * 1024 < P) pid[threadIdx.x + i * 1024] = ir[i];
    } else {
        for (int q = threadIdx.x; q < P; q += blockDim.x) pid[q] = idx[q];
    }
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        stab[e] = table[e];
        cnt[e] = 0;
    }
    if (bitmaps)
        for (int i = threadIdx.x; i < E * NWP; i += blockDim.x) bm[i] = 0u;
    __syncthreads();
    // each pair's test once (no earlier pick of the token has its expert,
    // and its weight is not 0), kept in LDS for the loops below
    auto count_pair = [&](int q, float wq) {
        const int t = q / K, k = q - t * K, e = pid[q];
        bool v = wq != 0.0f;
        for (int k2 = 0; k2 < k; k2++) v &= pid[t * K + k2] != e;
        pv[q] = v;
        if (v) {
            atomicAdd(&cnt[e], 1);
            if (bitmaps) atomicOr(&bm[e * NWP + (t >> 5)], 1u << (t & 31));
        }
    };
    if (regs) {
#pragma unroll
        for (int i = 0; i < PPT; i++)
            if ((int)threadIdx.x + i * 1024 < P) count_pair(threadIdx.x + i * 1024, wr[i]);
    } else {
        for (int q = threadIdx.x; q < P; q += blockDim.x) count_pair(q, w[q]);
    }
    __syncthreads();
    // per expert, in parallel: pair offset, first job, and the places of
    // its runs -- heaviest first: every full run of WARP_RUN_J jobs, then the
    // partial runs by their job count down to 1 (the launch hands units to
    // waves round-robin, so the long ones start first)
    __shared__ unsigned long long sc_tmp[16];
    __shared__ int miss_s;
    if (threadIdx.x == 0) miss_s = 0;
    int carry[2 + WARP_RUN_J] = {0, 0, 0, 0, 0, 0};   // pairs, jobs, full runs, partial runs by size
    static_assert(WARP_RUN_J == 4, "three partial-run sizes packed in one scan");
    constexpr unsigned long long F = (1ull << 21) - 1ull;   // 21-bit fields: every sum is below P, E < 2^21
    for (int e0 = 0; e0 < E; e0 += blockDim.x) {
        const int e = e0 + threadIdx.x;
        // every pair gets its place; jobs and runs only the window's experts
        const int c = e < E ? cnt[e] : 0, cw = e >= e_lo && e <= e_hi ? c : 0;
        const int nt = (cw + WARP_TPJ - 1) / WARP_TPJ, r = nt % WARP_RUN_J;
        // pairs, jobs and full runs in one scan; the partial runs of 1, 2
        // and 3 jobs in another
        unsigned long long t0, t1;
        const unsigned long long s0 =
            block_scan_excl64((unsigned long long)c | ((unsigned long long)nt << 21) |
                                  ((unsigned long long)(nt / WARP_RUN_J) << 42), sc_tmp, t0);
        const unsigned long long s1 =
            block_scan_excl64((unsigned long long)(r == 1) | ((unsigned long long)(r == 2) << 21) |
                                  ((unsigned long long)(r == 3) << 42), sc_tmp, t1);
        const int pc = (int)(s0 & F) + carry[0];
        const int tc = (int)(t0 & F);
        const int pt = (int)((s0 >> 21) & F) + carry[1];
        carry[1] += (int)((t0 >> 21) & F);
        const int pf = (int)(s0 >> 42) + carry[2];
        carry[2] += (int)(t0 >> 42);
        int pr = 0;
#pragma unroll
        for (int q = 1; q < WARP_RUN_J; q++) {
            if (r == q) pr = (int)((s1 >> (21 * (q - 1))) & F) + carry[2 + q];
            carry[2 + q] += (int)((t1 >> (21 * (q - 1))) & F);
        }
        if (e < E) {
            off[e] = offsets[e] = pc;
            counts[e] = c;
            tile0[e] = pt;
            run0[e] = pf;
            runr[e] = r ? pr : -1;            // rank among the partial runs of its size, placed below
            if (cw && !stab[e].rec) miss_s = 1;
        }
        carry[0] += tc;
    }
    __syncthreads();
    // partial runs after the full ones, by size: WARP_RUN_J - 1 first
    int base[WARP_RUN_J];
    base[WARP_RUN_J - 1] = carry[2];
    for (int q = WARP_RUN_J - 1; q > 1; q--) base[q - 1] = base[q] + carry[2 + q];
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        const int cw = e >= e_lo && e <= e_hi ? cnt[e] : 0;
        const int r = ((cw + WARP_TPJ - 1) / WARP_TPJ) % WARP_RUN_J;
#pragma unroll
        for (int q = 1; q < WARP_RUN_J; q++)
            if (r == q) runr[e] += base[q];
    }
    const int tiles = carry[1], nrun = base[1] + carry[3];
    if (threadIdx.x == 0) {
        offsets[E] = carry[0];
        const int nj = (miss_s || tiles > max_jobs) ? 0 : tiles;
        njobs[0] = njobs[1] = njobs[2] = nj;
        njobs[3] = nj ? nrun : 0;
        // written every call (no clearing needed), except that a later window
        // of one chunk only adds its own failure
        const int m = tiles > max_jobs ? 2 : miss_s ? 1 : 0;
        if (!or_missing || m) *missing = m;
    }
    __syncthreads();
    // every token's K slots: its computed pairs in ascending expert id, then -1
    auto place_pair = [&](int q, float wq) {
        const int t = q / K, k = q - t * K, e = pid[q];
        const bool v = pv[q];
        int r = 0, nv = 0, ninv = 0;
        for (int k2 = 0; k2 < K; k2++) {
            const bool v2 = pv[t * K + k2];
            nv += v2;
            r += v2 && pid[t * K + k2] < e;
            ninv += !v2 && k2 < k;
        }
        if (!v) {
            tok_slots[q - k + nv + ninv] = -1;
            return;
        }
        int pos = off[e];
        if (bitmaps) {
            const unsigned *row = bm + e * NWP;
            for (int i = 0; i < (t >> 5); i++) pos += __popc(row[i]);
            pos += __popc(row[t >> 5] & ((1u << (t & 31)) - 1u));
        } else {
            for (int t2 = 0; t2 < t; t2++)
                for (int k2 = 0; k2 < K; k2++)
                    if (pid[t2 * K + k2] == e && pv[t2 * K + k2]) pos++;
        }
        pair_tok[pos] = t;
        ptok[pos] = t;
        pair_exp[pos] = e;
        pair_w[pos] = wq;
        tok_slots[q - k + r] = pos;
    };
    if (regs) {
#pragma unroll
        for (int i = 0; i < PPT; i++)
            if ((int)threadIdx.x + i * 1024 < P) place_pair(threadIdx.x + i * 1024, wr[i]);
    } else {
        for (int q = threadIdx.x; q < P; q += blockDim.x) place_pair(q, w[q]);
    }
    __syncthreads();
    if (miss_s || tiles > max_jobs) return;          // uniform
    // the runs, one thread per expert (a few entries each)
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        const int ntile = e >= e_lo && e <= e_hi ? (cnt[e] + WARP_TPJ - 1) / WARP_TPJ : 0;
        for (int i = 0; i + WARP_RUN_J <= ntile; i += WARP_RUN_J)
            runs[run0[e] + i / WARP_RUN_J] = ((tile0[e] + i) << 3) | WARP_RUN_J;
        if (ntile % WARP_RUN_J)
            runs[runr[e]] = ((tile0[e] + ntile / WARP_RUN_J * WARP_RUN_J) << 3) | (ntile % WARP_RUN_J);
    }
    // the jobs, one thread per job: its expert is the last one whose first
    // job is not after it (experts without jobs share the next one's first)
    for (int j = threadIdx.x; j < tiles; j += blockDim.x) {
        int lo = 0, hi = E - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (tile0[mid] <= j) lo = mid;
            else hi = mid - 1;
        }
        const int e = lo, i = j - tile0[e], c = cnt[e];
        const int base = off[e] + i * WARP_TPJ, n = min(WARP_TPJ, c - i * WARP_TPJ);
        // the record and the job's tokens, each read once, all loads in flight
        const uint8_t *rec = stab[e].rec;
        const uint4 offs = make_uint4(stab[e].off[0], stab[e].off[1], stab[e].off[2], stab[e].off[3]);
        int tk[WARP_TPJ];
#pragma unroll
        for (int s = 0; s < WARP_TPJ; s++) tk[s] = ptok[base + (s < n ? s : 0)];
#pragma unroll
        for (int kind = 0; kind < 3; kind++) {
            warp_job *jo = jobs + (size_t)kind * max_jobs + j;
            const int soff = kind == 0 ? 0 : kind == 1 ? inter : 2 * inter;
            jo->idx = rec + (kind == 0 ? offs.x : kind == 1 ? offs.y : offs.z);
            jo->scale = (const uint16_t *)(rec + offs.w) + soff;
            jo->n = n;
            jo->rsv = 0;
#pragma unroll
            for (int s = 0; s < WARP_TPJ; s++) {
                const int slot = base + (s < n ? s : 0);
                jo->xi[s] = kind == 2 ? slot : tk[s];
                jo->yi[s] = slot;
            }
        }
    }
}

extern "C" int wk_plan_chunk(const int *idx, const float *w, int T, int K, int E, const warp_slot *table,
                             int *counts, int *offsets, int *pair_tok, int *pair_exp, float *pair_w, int *tok_slots,
                             warp_job *jobs, int max_jobs, int *njobs, int *runs, int *missing, int inter,
                             int e_lo, int e_hi, int or_missing, void *stream) {
    if (T <= 0 || K <= 0 || E <= 0 || max_jobs <= 0 || !runs || e_lo < 0 || e_hi >= E || e_lo > e_hi) return -1;
    // the picks, the per-expert tables, each pair's token and a flag per pair
    // in LDS; the token bitmaps too when they fit
    const size_t base = (size_t)E * sizeof(warp_slot) + ((size_t)2 * T * K + 5 * (size_t)E) * sizeof(int) +
                        (size_t)T * K;
    const size_t bms = (size_t)E * (((T + 31) / 32) | 1) * sizeof(unsigned);
    // dynamic LDS up to 152 KiB: the kernel's static shared memory takes the rest of the 160
    constexpr size_t LDS_MAX = 152 * 1024;
    if (base > LDS_MAX) return -1;
    const int bitmaps = base + bms <= LDS_MAX;
    static std::atomic<uint64_t> attr{0};
    if (int r_ = lds_limit((const void *)k_plan_chunk, (int)LDS_MAX, attr, stream)) return r_;
    hipLaunchKernelGGL(k_plan_chunk, dim3(1), dim3(1024), base + (bitmaps ? bms : 0), (hipStream_t)stream, idx, w, T,
                       K, E, table, counts, offsets, pair_tok, pair_exp, pair_w, tok_slots, jobs, max_jobs, njobs,
                       runs, missing, inter, bitmaps, e_lo, e_hi, or_missing);
    CHECK_LAUNCH();
    return 0;
}

// Per token: the pairs of that token in ascending expert id, each weighted
// and added in that order (moe_chunk's loop order, src/model.c:3601-3656),
// then + add0 (the shared expert) + add1 (the caller's residual).
// V consecutive outputs per thread (float4 when H allows). The token's
// slots, their weights and their rows are read 8 pairs at a time, each kind
// in one batch (clamped to pair 0, so no load waits on another), then added
// in slot order; slots past the computed pairs are -1.
template <int V>
__global__ __launch_bounds__(256) void k_combine_chunk(const float *__restrict__ y, const int *__restrict__ tok_slots,
                                                       const float *__restrict__ pair_w, int T, int K, int H,
                                                       const float *__restrict__ add0, const float *__restrict__ add1,
                                                       float *__restrict__ out) {
    typedef float vec __attribute__((ext_vector_type(V)));
    const int t = blockIdx.y;
    const int i = (blockIdx.x * blockDim.x + threadIdx.x) * V;
    if (i >= H) return;
    const int *sl = tok_slots + (size_t)t * K;
    vec s = {};
    for (int q0 = 0; q0 < K; q0 += 8) {
        int pv[8];
        float wv[8];
        vec yv[8];
#pragma unroll
        for (int j = 0; j < 8; j++) pv[j] = q0 + j < K ? sl[q0 + j] : -1;
#pragma unroll
        for (int j = 0; j < 8; j++) wv[j] = pair_w[max(pv[j], 0)];
#pragma unroll
        for (int j = 0; j < 8; j++) yv[j] = *(const vec *)(y + (size_t)max(pv[j], 0) * H + i);
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (pv[j] >= 0 && wv[j] != 0.0f)
#pragma unroll
                for (int c = 0; c < V; c++) s[c] = __fadd_rn(s[c], __fmul_rn(wv[j], yv[j][c]));
        if (pv[7] < 0) break;                  // uniform: the token's computed pairs come first
    }
    if (add0) {
        const vec a = *(const vec *)(add0 + (size_t)t * H + i);
#pragma unroll
        for (int c = 0; c < V; c++) s[c] = __fadd_rn(s[c], a[c]);
    }
    if (add1) {
        const vec a = *(const vec *)(add1 + (size_t)t * H + i);
#pragma unroll
        for (int c = 0; c < V; c++) s[c] = __fadd_rn(s[c], a[c]);
    }
    *(vec *)(out + (size_t)t * H + i) = s;
}

extern "C" int wk_combine_chunk(const float *y, const int *tok_slots, const float *pair_w, int T, int K, int H,
                                const float *add0, const float *add1, float *out, void *stream) {
    if (T <= 0 || K <= 0 || K > WARP_MAX_K || H <= 0) return -1;
    if (H % 4 == 0 && (((uintptr_t)y | (uintptr_t)add0 | (uintptr_t)add1 | (uintptr_t)out) & 15) == 0)
        hipLaunchKernelGGL(k_combine_chunk<4>, dim3((H / 4 + 255) / 256, T), dim3(256), 0, (hipStream_t)stream, y,
                           tok_slots, pair_w, T, K, H, add0, add1, out);
    else
        hipLaunchKernelGGL(k_combine_chunk<1>, dim3((H + 255) / 256, T), dim3(256), 0, (hipStream_t)stream, y,
                           tok_slots, pair_w, T, K, H, add0, add1, out);
    CHECK_LAUNCH();
    return 0;
}

// ---- the encoder (conversion) ------------------------------------------------------------------
//
// waste_vq_encode (src/vq.c:50-103) for 8-dim vectors: per stage the entry
// nearest the current vector under squared L2, d = sum over j ascending of
// (v[j] - e[j])^2 with every multiply and add rounded on its own (the
// reference's vq.c is built without FMA), the first minimum winning
// (strict <), then the exact residual v - e feeds the next stage. One launch
// per stage: the stage's codebook (entries x 8 fp32, up to 128 KiB) in LDS,
// one thread per vector scanning every entry (all lanes read the same entry
// at once: LDS broadcasts). The residual is kept in `cur`. Blocks of 1024
// threads, so that a 4096-entry codebook (128 KiB, one block per CU) still
// leaves 4 waves per SIMD.
constexpr int ENC_NT = 1024;

__global__ __launch_bounds__(ENC_NT) void k_vq_encode_stage(const float *__restrict__ X, float *__restrict__ cur,
                                                            const float *__restrict__ book, int entries, long n,
                                                            int stage, int stages, uint16_t *__restrict__ codes) {
    extern __shared__ float4 cb4[];                  // [entries][2] float4
    for (int i = threadIdx.x; i < entries * 2; i += ENC_NT) cb4[i] = ((const float4 *)book)[i];
    __syncthreads();
    const long i = (long)blockIdx.x * ENC_NT + threadIdx.x;
    if (i >= n) return;
    const float4 *src = (const float4 *)((stage == 0 ? X : cur) + i * 8);
    const float4 v0 = src[0], v1 = src[1];
    const float v[8] = { v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w };
    int best = 0;
    float bestd = INFINITY;
    for (int c = 0; c < entries; c++) {
        const float4 e0 = cb4[2 * c], e1 = cb4[2 * c + 1];
        const float e[8] = { e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w };
        float d = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float t = __fsub_rn(v[j], e[j]);
            d = __fadd_rn(d, __fmul_rn(t, t));
        }
        if (d < bestd) {
            bestd = d;
            best = c;
        }
    }
    codes[i * stages + stage] = (uint16_t)best;
    if (stage + 1 < stages) {
        const float4 b0 = cb4[2 * best], b1 = cb4[2 * best + 1];
        float4 *dst = (float4 *)(cur + i * 8);
        dst[0] = make_float4(__fsub_rn(v[0], b0.x), __fsub_rn(v[1], b0.y), __fsub_rn(v[2], b0.z), __fsub_rn(v[3], b0.w));
        dst[1] = make_float4(__fsub_rn(v[4], b1.x), __fsub_rn(v[5], b1.y), __fsub_rn(v[6], b1.z), __fsub_rn(v[7], b1.w));
    }
}

extern "C" int wk_vq_encode(const float *X, long n, const float *books, int stages, int entries, float *cur,
                            uint16_t *codes, void *stream) {
    if (n <= 0 || stages < 1 || entries < 1 || entries > 4096) return -1;
    if (((uintptr_t)X | (uintptr_t)books | (uintptr_t)cur) & 15) return -1;
    const size_t lds = (size_t)entries * 8 * sizeof(float);
    static std::atomic<uint64_t> attr{0};
    if (int r_ = lds_limit((const void *)k_vq_encode_stage, 4096 * 8 * (int)sizeof(float), attr, stream)) return r_;
    const unsigned grid = (unsigned)((n + ENC_NT - 1) / ENC_NT);
    for (int s = 0; s < stages; s++) {
        hipLaunchKernelGGL(k_vq_encode_stage, dim3(grid), dim3(ENC_NT), lds, (hipStream_t)stream, X, cur,
                           books + (size_t)s * entries * 8, entries, n, s, stages, codes);
        CHECK_LAUNCH();
    }
    return 0;
}

// One Lloyd iteration (waste_vq_lloyd, src/vq.c:109-136) after the
// assignment: per cluster, the mean of its members, summed in double in
// ascending member index as the reference does, so the new centroids are
// bit-identical to it. A stable counting sort by cluster gives each
// cluster its members in index order: counts per chunk of ENC_CH vectors,
// per-cluster offsets (cluster-major, chunk-minor), then one wave per chunk
// places its members in order.
constexpr int ENC_CH = 4096;

__global__ __launch_bounds__(256) void k_lloyd_count(const uint16_t *__restrict__ asg, long n, int entries,
                                                     int *__restrict__ counts) {
    extern __shared__ int hist[];
    for (int c = threadIdx.x; c < entries; c += 256) hist[c] = 0;
    __syncthreads();
    const long i0 = (long)blockIdx.x * ENC_CH;
    for (int k = threadIdx.x; k < ENC_CH && i0 + k < n; k += 256) atomicAdd(&hist[asg[i0 + k]], 1);
    __syncthreads();
    for (int c = threadIdx.x; c < entries; c += 256) counts[(size_t)blockIdx.x * entries + c] = hist[c];
}

// per cluster: running offsets over the chunks (in place) and its total
__global__ __launch_bounds__(256) void k_lloyd_offsets(int *__restrict__ counts, int nchunk, int entries,
                                                       int *__restrict__ total) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= entries) return;
    int run = 0;
    for (int b = 0; b < nchunk; b++) {
        const int v = counts[(size_t)b * entries + c];
        counts[(size_t)b * entries + c] = run;
        run += v;
    }
    total[c] = run;
}

// exclusive scan of the totals (one block) and the number of live clusters
__global__ __launch_bounds__(1024) void k_lloyd_scan(const int *__restrict__ total, int entries, int *__restrict__ base,
                                                     int *__restrict__ live) {
    __shared__ int tmp[16];
    int carry = 0, nlive = 0;
    for (int c0 = 0; c0 < entries; c0 += 1024) {
        const int c = c0 + threadIdx.x;
        const int v = c < entries ? total[c] : 0;
        int tot;
        const int ex = block_scan_excl(v, tmp, tot);
        if (c < entries) base[c] = carry + ex;
        carry += tot;
        int lv;
        (void)block_scan_excl(v > 0 ? 1 : 0, tmp, lv);
        nlive += lv;
    }
    if (threadIdx.x == 0) *live = nlive;
}

// one wave per chunk, its vectors in index order, 64 at a time: a lane's
// place among the equal clusters of its step is the number of earlier lanes
// with its cluster; the chunk's running count per cluster is in LDS
__global__ __launch_bounds__(64) void k_lloyd_scatter(const uint16_t *__restrict__ asg, long n, int entries,
                                                      const int *__restrict__ rel, const int *__restrict__ base,
                                                      int *__restrict__ sorted) {
    extern __shared__ int ctr[];
    const int lane = threadIdx.x;
    for (int c = lane; c < entries; c += 64) ctr[c] = 0;
    __syncthreads();
    const long i0 = (long)blockIdx.x * ENC_CH;
    const unsigned long long below = (1ull << lane) - 1ull;
    for (int k0 = 0; k0 < ENC_CH && i0 + k0 < n; k0 += 64) {
        const long i = i0 + k0 + lane;
        const bool ok = i < n;
        const int c = ok ? (int)asg[i] : -1;
        unsigned long long peers = 0;
        for (int j = 0; j < 64; j++)
            if (__builtin_amdgcn_readlane(c, j) == c) peers |= 1ull << j;
        const int rank = __popcll(peers & below), cnt = __popcll(peers);
        const int seen = ok ? ctr[c] : 0;
        __syncthreads();
        if (ok) {
            sorted[base[c] + rel[(size_t)blockIdx.x * entries + c] + seen + rank] = (int)i;
            if (rank == 0) ctr[c] = seen + cnt;
        }
        __syncthreads();
    }
}

// one thread per (cluster, dim): its members' values in index order, in double
__global__ __launch_bounds__(256) void k_lloyd_mean(const float *__restrict__ X, const int *__restrict__ sorted,
                                                    const int *__restrict__ base, const int *__restrict__ total,
                                                    int entries, int dim, float *__restrict__ C) {
    const int q = blockIdx.x * 256 + threadIdx.x;
    if (q >= entries * dim) return;
    const int c = q / dim, d = q - c * dim, n = total[c];
    if (!n) return;                                   // an empty cluster keeps its centroid
    const int *m = sorted + base[c];
    double s = 0.0;
    for (int k = 0; k < n; k++) s = __dadd_rn(s, (double)X[(size_t)m[k] * dim + d]);
    C[q] = (float)__ddiv_rn(s, (double)n);
}

extern "C" int wk_vq_lloyd(const float *X, long n, float *C, int entries, int dim, uint16_t *asg, int *counts,
                           int *total, int *base, int *sorted, int *live, void *stream) {
    if (n <= 0 || entries < 1 || entries > 4096 || dim != 8) return -1;
    int rc = wk_vq_encode(X, n, C, 1, entries, nullptr, asg, stream);
    if (rc) return rc;
    const int nchunk = (int)((n + ENC_CH - 1) / ENC_CH);
    const size_t lds = (size_t)entries * sizeof(int);
    hipLaunchKernelGGL(k_lloyd_count, dim3(nchunk), dim3(256), lds, (hipStream_t)stream, asg, n, entries, counts);
    CHECK_LAUNCH();
    hipLaunchKernelGGL(k_lloyd_offsets, dim3((entries + 255) / 256), dim3(256), 0, (hipStream_t)stream, counts,
                       nchunk, entries, total);
    CHECK_LAUNCH();
    hipLaunchKernelGGL(k_lloyd_scan, dim3(1), dim3(1024), 0, (hipStream_t)stream, total, entries, base, live);
    CHECK_LAUNCH();
    hipLaunchKernelGGL(k_lloyd_scatter, dim3(nchunk), dim3(64), lds, (hipStream_t)stream, asg, n, entries, counts, base,
                       sorted);
    CHECK_LAUNCH();
    hipLaunchKernelGGL(k_lloyd_mean, dim3((entries * dim + 255) / 256), dim3(256), 0, (hipStream_t)stream, X, sorted,
                       base, total, entries, dim, C);
    CHECK_LAUNCH();
    return 0;
}

// ---- synthetic data ---------------------------------------------------------------------------

__device__ __forceinline__ uint64_t splitmix(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void k_fill(uint8_t *__restrict__ p, size_t n, uint64_t seed) {
    const size_t nw = n / 8;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < nw; i += (size_t)gridDim.x * blockDim.x)
        ((uint64_t *)p)[i] = splitmix(seed ^ (i * 0xD1B54A32D192ED03ull));
    if (blockIdx.x == 0 && threadIdx.x < (n & 7)) p[nw * 8 + threadIdx.x] = (uint8_t)splitmix(seed + n + threadIdx.x);
}

extern "C" int wk_fill_random(uint8_t *p, size_t n, uint64_t seed, void *stream) {
    if (!n) return 0;
    if (((uintptr_t)p) & 7) return -1;
    hipLaunchKernelGGL(k_fill, dim3(4096), dim3(256), 0, (hipStream_t)stream, p, n, seed);
    CHECK_LAUNCH();
    return 0;
}

__global__ __launch_bounds__(256) void k_set_slots(warp_slot *__restrict__ table, const warp_slot_upd *__restrict__ u,
                                                   int n, int8_t *__restrict__ crc_bad,
                                                   warp_crc_err *__restrict__ err) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int key = u[i].key;
    warp_slot v = u[i].v;
    if (u[i].checked && crc_bad && crc_bad[key]) {
        v.rec = nullptr;                       // refused: the record stays out of the table
        const int k = atomicAdd(&err->n, 1);
        if (k < WARP_CRC_ERR_KEYS) err->keys[k] = key;
    } else if (!u[i].checked && crc_bad) {
        crc_bad[key] = 0;                      // an unchecked entry (eviction, synthetic record) is no refusal
    }
    table[key] = v;
}

extern "C" int wk_set_slots(warp_slot *table, const warp_slot_upd *u, int n, int8_t *crc_bad, warp_crc_err *err,
                            void *stream) {
    if (n <= 0) return 0;
    if (crc_bad && !err) return -1;
    hipLaunchKernelGGL(k_set_slots, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, table, u, n, crc_bad,
                       err);
    CHECK_LAUNCH();
    return 0;
}

// ---- the latent MoE's tail ----------------------------------------------------------
//
// waste_rmsnorm (src/model.c:132-138) per token, in place allowed: o = x *
// r * w with r = 1 / sqrt(sum x^2 / n + eps). The sum runs in a fixed tree
// (each thread a strided partial, then the waves, in order), so it is
// deterministic; it differs from the reference's sequential sum by fp32
// rounding only. One block per token.
__global__ __launch_bounds__(256) void k_rmsnorm(const float *__restrict__ x, const float *__restrict__ w, int n,
                                                 float eps, float *__restrict__ o) {
    __shared__ float red[4];
    const float *xt = x + (size_t)blockIdx.x * n;
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) s = __fadd_rn(s, __fmul_rn(xt[i], xt[i]));
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    s = __fadd_rn(__fadd_rn(red[0], red[1]), __fadd_rn(red[2], red[3]));
    const float r = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(s, (float)n), eps)));
    float *ot = o + (size_t)blockIdx.x * n;
    for (int i = threadIdx.x; i < n; i += 256) ot[i] = __fmul_rn(__fmul_rn(xt[i], r), w[i]);
}

extern "C" int wk_rmsnorm(const float *x, const float *w, int T, int n, float eps, float *o, void *stream) {
    if (!x || !w || !o || T <= 0 || n <= 0) return -1;
    hipLaunchKernelGGL(k_rmsnorm, dim3(T), dim3(256), 0, (hipStream_t)stream, x, w, n, eps, o);
    CHECK_LAUNCH();
    return 0;
}

// out = (y + a0) + a1 elementwise, each addend optional: the routed part, then
// the shared expert, then the caller's residual (src/model.c:2934-2939).
__global__ __launch_bounds__(256) void k_add3(const float *__restrict__ y, const float *a0, const float *a1, size_t n,
                                              float *out) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        float v = y[i];
        if (a0) v = __fadd_rn(v, a0[i]);
        if (a1) v = __fadd_rn(v, a1[i]);
        out[i] = v;
    }
}

extern "C" int wk_add3(const float *y, const float *a0, const float *a1, size_t n, float *out, void *stream) {
    if (!y || !out || n == 0) return -1;
    const size_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(k_add3, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, (hipStream_t)stream, y,
                       a0, a1, n, out);
    CHECK_LAUNCH();
    return 0;
}

// One expert's three matvec jobs from its device table entry (one input,
// one output row block each), its combine weight 1 and the job counts:
// the single-expert FFN without routing.
__global__ __launch_bounds__(64) void k_expert_jobs(const warp_slot *__restrict__ entry, int inter,
                                                    warp_job *__restrict__ jobs, int *__restrict__ njobs,
                                                    float *__restrict__ w, int *__restrict__ missing) {
    const int kind = threadIdx.x;
    const warp_slot s = *entry;
    if (kind < 3) {
        warp_job jb = {};
        jb.idx = s.rec ? s.rec + s.off[kind] : nullptr;
        jb.scale = s.rec ? (const uint16_t *)(s.rec + s.off[3]) + (kind == 0 ? 0 : kind == 1 ? inter : 2 * inter)
                         : nullptr;
        jb.n = 1;
        jobs[kind] = jb;
        njobs[kind] = s.rec ? 1 : 0;
    }
    if (kind == 3) {
        w[0] = 1.0f;
        njobs[3] = 0;
        if (!s.rec) *missing = 1;     // sticky until reported
    }
}

extern "C" int wk_expert_jobs(const warp_slot *entry, int inter, warp_job *jobs, int *njobs, float *w, int *missing,
                              void *stream) {
    if (!entry || !jobs || !njobs || !w || !missing || inter <= 0) return -1;
    hipLaunchKernelGGL(k_expert_jobs, dim3(1), dim3(64), 0, (hipStream_t)stream, entry, inter, jobs, njobs, w,
                       missing);
    CHECK_LAUNCH();
    return 0;
}

extern "C" int wk_device_arch(int device, char *buf, int n) {
    hipDeviceProp_t pr;
    if (hipGetDeviceProperties(&pr, device) != hipSuccess) return -1;
    int i = 0;
    for (; i < n - 1 && pr.gcnArchName[i]; i++) buf[i] = pr.gcnArchName[i];
    if (n > 0) buf[i] = 0;
    return 0;
}
