// kda.hip — the Kimi Delta Attention recurrence on the device: the
// kda_step slot of the reference's dispatch table (src/waste_backend.h:69-72,
// src/kda.c:26-68) and a T-step forward that keeps the state on chip.
//
// Per head h, with state S [K][V]: q and k are L2-normalised (k by
// 1/sqrt(sum k^2 + 1e-12), q by the same and by 1/sqrt(K)); pass A decays
// every row kk of S by exp(g[kk]) and accumulates u = S^T k; then
// d = beta (v - u); pass B adds k d^T to S and accumulates o = S^T q. Every
// column i of S depends only on per-row scalars, so a thread owns a column:
// a block of V threads takes one head, its S in LDS for the call, read and
// written once. The arithmetic is the reference's, operation by operation
// (separate multiplies and adds in row order, IEEE sqrt and division,
// glibc's expf), so S and o are bit-identical to waste_kda_step.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lds_limit.h"
#include "warp_internal.h"

#define WARP_EXPF_QUAL __device__ __forceinline__
#include "expf_glibc.h"

constexpr int KDA_MAX_K = 256;

// 1 / sqrt(sum x^2 + 1e-12): the sum sequential in index order (l2_rnorm,
// src/kda.c:19-24), by thread 0; the result broadcast through LDS.
__device__ inline float kda_rnorm(const float *x, int n, float *tmp) {
    if (threadIdx.x == 0) {
        float s = 0.0f;
        for (int i = 0; i < n; i++) s = __fadd_rn(s, __fmul_rn(x[i], x[i]));
        *tmp = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(s, 1e-12f)));
    }
    __syncthreads();
    const float r = *tmp;
    __syncthreads();
    return r;
}

// T steps of one head (blockIdx.x) per launch: inputs of step t at
// q + t*qs etc.; the state stays in LDS between steps.
__global__ __launch_bounds__(1024) void k_kda(int T, int H, int K, int V, const float *__restrict__ q,
                                              const float *__restrict__ k, const float *__restrict__ v,
                                              const float *__restrict__ g, const float *__restrict__ beta,
                                              float *__restrict__ S, float *__restrict__ o) {
    extern __shared__ float Sl[];                 // [K][V]
    __shared__ float dk[KDA_MAX_K], kv[KDA_MAX_K], qv[KDA_MAX_K], red;
    const int h = blockIdx.x, i = threadIdx.x;
    float *Sh = S + (size_t)h * K * V;
    for (int kk = 0; kk < K; kk++) Sl[kk * V + i] = Sh[(size_t)kk * V + i];
    const float qscale = __fdiv_rn(1.0f, __fsqrt_rn((float)K));
    for (int t = 0; t < T; t++) {
        const size_t hk = ((size_t)t * H + h) * K, hv = ((size_t)t * H + h) * V;
        const float *qh = q + hk, *kh = k + hk, *gh = g + hk;
        const float qn = __fmul_rn(kda_rnorm(qh, K, &red), qscale);
        const float kn = kda_rnorm(kh, K, &red);
        for (int kk = i; kk < K; kk += V) {
            dk[kk] = warp_expf(gh[kk]);
            kv[kk] = __fmul_rn(kh[kk], kn);
            qv[kk] = __fmul_rn(qh[kk], qn);
        }
        __syncthreads();
        // pass A: decay the column, u = sum over rows of row * kv
        float u = 0.0f;
        for (int kk = 0; kk < K; kk++) {
            const float r = __fmul_rn(Sl[kk * V + i], dk[kk]);
            Sl[kk * V + i] = r;
            u = __fadd_rn(u, __fmul_rn(r, kv[kk]));
        }
        const float d = __fmul_rn(beta[(size_t)t * H + h], __fsub_rn(v[hv + i], u));
        // pass B: the rank-1 update of the column, o = sum of row * qv
        float acc = 0.0f;
        for (int kk = 0; kk < K; kk++) {
            const float r = __fadd_rn(Sl[kk * V + i], __fmul_rn(d, kv[kk]));
            Sl[kk * V + i] = r;
            acc = __fadd_rn(acc, __fmul_rn(r, qv[kk]));
        }
        o[hv + i] = acc;
        __syncthreads();                           // dk/kv/qv of the next step
    }
    for (int kk = 0; kk < K; kk++) Sh[(size_t)kk * V + i] = Sl[kk * V + i];
}

extern "C" int wk_kda(int T, int H, int K, int V, const float *q, const float *k, const float *v, const float *g,
                      const float *beta, float *S, float *o, void *stream) {
    if (T <= 0 || H <= 0 || K <= 0 || K > KDA_MAX_K || V <= 0 || V > 1024) return -1;
    const size_t lds = (size_t)K * V * sizeof(float);
    if (lds > 150 * 1024) return -1;
    static std::atomic<uint64_t> attr{0};
    if (int r_ = lds_limit((const void *)k_kda, 150 * 1024, attr, stream)) return r_;
    hipLaunchKernelGGL(k_kda, dim3(H), dim3(V), lds, (hipStream_t)stream, T, H, K, V, q, k, v, g, beta, S, o);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : -(int)e - 1000;
}
