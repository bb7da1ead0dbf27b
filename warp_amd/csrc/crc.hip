// crc.hip — zlib's crc32 on the device: the checksum of expert records
// (waste_expert_hdr.crc32 over the payload after the header,
// src/waste_format.h:116-127; src/model.c:1742-1744), and the reference's
// waste_crc32 (src/crc32.c:176) on device memory.
//
// The CRC register update is linear over GF(2), so the checksum of a long
// buffer is assembled from independent pieces. With R(M) the register after
// M from a zero start ("raw"), R(A B) = R(A) * x^(8|B|) + R(B) mod P (the
// product in the reflected polynomial representation zlib uses, P =
// 0xEDB88320), and zlib's crc32 is R(M) + 0xFFFFFFFF * x^(8|M|) + 0xFFFFFFFF
// (its initial register and final complement). Each thread takes the raw CRC
// of 64 contiguous bytes with byte tables in LDS (slicing by 4); a block of
// 1024 threads folds its 64 KiB in a tree of such products; one more block
// folds the blocks' results.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "warp_internal.h"

#define CRC_POLY 0xEDB88320u
constexpr int CRC_NT = 1024;                   // threads per block
constexpr int CRC_SEG = 64;                    // bytes per thread
constexpr int CRC_BLK = CRC_NT * CRC_SEG;      // bytes per block (64 KiB)

// a(x) b(x) mod P, reflected (bit 31 is x^0): for each power of a, add b,
// then b times x; 32 fixed steps, no branches.
__host__ __device__ inline uint32_t gf2_mulmod(uint32_t a, uint32_t b) {
    uint32_t p = 0;
#pragma unroll
    for (int i = 31; i >= 0; i--) {
        p ^= b & (0u - ((a >> i) & 1u));
        b = (b >> 1) ^ (CRC_POLY & (0u - (b & 1u)));
    }
    return p;
}

// x^(2^k) mod P for k = 0..63: x^(8n) is the product of those k where bit
// (k - 3) of n is set.
struct CrcPow {
    uint32_t p[64];
};

__device__ inline uint32_t x8n_mod(uint64_t n, const CrcPow &pw) {
    uint32_t r = 1u << 31;                     // x^0
    for (int k = 3; n; k++, n >>= 1)
        if (n & 1) r = gf2_mulmod(r, pw.p[k]);
    return r;
}

// LDS tables for slicing by 4: T0[b] = R of byte b; Tk[b] = Tk-1[b] shifted
// by a zero byte.
__device__ inline void crc_tables(uint32_t (*T)[256]) {
    for (int i = threadIdx.x; i < 256; i += blockDim.x) {
        uint32_t c = (uint32_t)i;
#pragma unroll
        for (int k = 0; k < 8; k++) c = (c >> 1) ^ (CRC_POLY & (0u - (c & 1u)));
        T[0][i] = c;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 256; i += blockDim.x) {
        uint32_t c = T[0][i];
#pragma unroll
        for (int k = 1; k < 4; k++) {
            c = (c >> 8) ^ T[0][c & 0xFFu];
            T[k][i] = c;
        }
    }
    __syncthreads();
}

// Fold the block's (crc, len) pairs, in order, into thread 0: a tree whose
// right operand's length is a full power-of-two span except on the last
// (partial) path, where x^(8 len) is computed.
__device__ inline uint32_t crc_fold(uint32_t c, uint64_t len, uint64_t span0, const CrcPow &pw,
                                    uint32_t *sc, uint64_t *sl) {
    const int t = threadIdx.x;
    sc[t] = c;
    sl[t] = len;
    __syncthreads();
    uint64_t span = span0;
    uint32_t xs = x8n_mod(span, pw);           // x^(8 span): the full right operand
    for (int s = 1; s < (int)blockDim.x; s <<= 1) {
        if ((t & (2 * s - 1)) == 0 && t + s < (int)blockDim.x) {
            const uint64_t lr = sl[t + s];
            const uint32_t xr = lr == span ? xs : x8n_mod(lr, pw);
            sc[t] = gf2_mulmod(sc[t], xr) ^ sc[t + s];
            sl[t] += lr;
        }
        __syncthreads();
        span *= 2;
        xs = gf2_mulmod(xs, xs);
    }
    return sc[0];
}

// Raw CRC of each 64 KiB block of p[0, n): part[b].
__global__ __launch_bounds__(CRC_NT) void k_crc_blocks(const uint8_t *__restrict__ p, uint64_t n, CrcPow pw,
                                                       uint32_t *__restrict__ part) {
    __shared__ uint32_t T[4][256];
    __shared__ uint32_t sc[CRC_NT];
    __shared__ uint64_t sl[CRC_NT];
    const uint64_t beg = (uint64_t)blockIdx.x * CRC_BLK + (uint64_t)threadIdx.x * CRC_SEG;
    const uint64_t len = beg < n ? (n - beg < CRC_SEG ? n - beg : CRC_SEG) : 0;
    // the segment's bytes, loaded before the tables are built
    uint32_t w[CRC_SEG / 4];
    if (len == CRC_SEG && ((uintptr_t)(p + beg) & 15) == 0) {
        const uint4 *q = (const uint4 *)(p + beg);
#pragma unroll
        for (int i = 0; i < CRC_SEG / 16; i++) {
            const uint4 v = q[i];
            w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < CRC_SEG / 4; i++) {
            uint32_t v = 0;
            for (int b = 0; b < 4; b++) {
                const uint64_t o = 4 * (uint64_t)i + b;
                if (o < len) v |= (uint32_t)p[beg + o] << (8 * b);
            }
            w[i] = v;
        }
    }
    crc_tables(T);
    uint32_t c = 0;
    const int whole = (int)(len / 4);
#pragma unroll
    for (int i = 0; i < CRC_SEG / 4; i++)
        if (i < whole) {
            c ^= w[i];
            c = T[3][c & 0xFFu] ^ T[2][(c >> 8) & 0xFFu] ^ T[1][(c >> 16) & 0xFFu] ^ T[0][c >> 24];
        }
    for (int b = 4 * whole; b < (int)len; b++) {
        const uint32_t byte = (w[b >> 2] >> (8 * (b & 3))) & 0xFFu;
        c = T[0][(c ^ byte) & 0xFFu] ^ (c >> 8);
    }
    const uint32_t r = crc_fold(c, len, CRC_SEG, pw, sc, sl);
    if (threadIdx.x == 0) part[blockIdx.x] = r;
}

// Folds the nb block CRCs into zlib's crc32 of the n bytes: *out; with key
// >= 0 also compares it with *expect (the record header's field) and sets
// bad[key] to 1 on a mismatch, 0 otherwise.
__global__ __launch_bounds__(CRC_NT) void k_crc_final(const uint32_t *__restrict__ part, int nb, uint64_t n,
                                                      CrcPow pw, uint32_t *__restrict__ out,
                                                      const uint32_t *__restrict__ expect, int key,
                                                      int8_t *__restrict__ bad) {
    __shared__ uint32_t sc[CRC_NT];
    __shared__ uint64_t sl[CRC_NT];
    // thread t folds blocks [t * per, (t + 1) * per) in order first
    const int per = (nb + CRC_NT - 1) / CRC_NT;
    const uint32_t xb = x8n_mod(CRC_BLK, pw);
    uint32_t c = 0;
    uint64_t len = 0;
    for (int b = threadIdx.x * per; b < (threadIdx.x + 1) * per && b < nb; b++) {
        const uint64_t lb = (uint64_t)b * CRC_BLK + CRC_BLK <= n ? CRC_BLK : n - (uint64_t)b * CRC_BLK;
        c = gf2_mulmod(c, lb == CRC_BLK ? xb : x8n_mod(lb, pw)) ^ part[b];
        len += lb;
    }
    const uint32_t r = crc_fold(c, len, (uint64_t)per * CRC_BLK, pw, sc, sl);
    if (threadIdx.x == 0) {
        const uint32_t crc = r ^ gf2_mulmod(0xFFFFFFFFu, x8n_mod(n, pw)) ^ 0xFFFFFFFFu;
        if (out) *out = crc;
        if (key >= 0) bad[key] = crc != *expect;
    }
}

static CrcPow make_pow() {
    CrcPow pw;
    uint32_t x = 1u << 30;                     // x^1
    for (int k = 0; k < 64; k++) {
        pw.p[k] = x;
        x = gf2_mulmod(x, x);
    }
    return pw;
}

static CrcPow crc_pow() {
    static const CrcPow pw = make_pow();       // initialised once, thread-safe
    return pw;
}

extern "C" size_t wk_crc32_tmp_words(size_t n) { return (n + CRC_BLK - 1) / CRC_BLK; }

extern "C" int wk_crc32(const uint8_t *p, size_t n, uint32_t *tmp, uint32_t *out, const uint32_t *expect, int key,
                        int8_t *bad, void *stream) {
    if (!p || !tmp || n == 0 || (key >= 0 && (!expect || !bad)) || (key < 0 && !out)) return -1;
    const size_t nb = wk_crc32_tmp_words(n);
    if (nb > 0x7fffffff) return -1;
    const CrcPow pw = crc_pow();
    hipLaunchKernelGGL(k_crc_blocks, dim3((unsigned)nb), dim3(CRC_NT), 0, (hipStream_t)stream, p, (uint64_t)n, pw,
                       tmp);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return -(int)e - 1000;
    hipLaunchKernelGGL(k_crc_final, dim3(1), dim3(CRC_NT), 0, (hipStream_t)stream, tmp, (int)nb, (uint64_t)n, pw, out,
                       expect, key, bad);
    e = hipGetLastError();
    return e == hipSuccess ? 0 : -(int)e - 1000;
}
