// Small helper kernels of the GEMM library: tile-to-row weight re-layout,
// fp32 -> bf16 rounding of A, greedy argmax, copies and fills.
// Included by hip_gemm.hip, whose host code launches them.
#ifndef QH_MISC_KERNELS_H
#define QH_MISC_KERNELS_H

#include "gemm_common.h"

// ---------------------------------------------------------------------------
// misc kernels
// ---------------------------------------------------------------------------
// dst[n][k] = src[tile(n,k)], tile-major as in kernels_ame.c:212-215,269
__global__ void k_tile_to_row(uint16_t *__restrict__ dst, const uint16_t *__restrict__ src,
                              int N, int K, int tn, int tk) {
    const size_t total = (size_t)N * K;
    const size_t ktiles = (size_t)(K / tk);
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int n = (int)(i / K), k = (int)(i % K);
        const size_t t = (size_t)(n / tn) * ktiles + (size_t)(k / tk);
        dst[i] = src[t * (size_t)tn * tk + (size_t)(n % tn) * tk + (k % tk)];
    }
}

// (value, index) argmax: larger value wins, ties -> lower index; NaN never
// wins a comparison (matches the strict ">" scan of ops_scalar.c:57-62 except
// that a NaN at index 0 is not returned when any value is ordered).
__device__ __forceinline__ void am_merge(float &v, int &i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i) || (v != v && v2 == v2)) { v = v2; i = i2; }
}

__global__ __launch_bounds__(NTHREADS) void k_argmax_partial(float *__restrict__ pv,
                                                            int *__restrict__ pi,
                                                            const float *__restrict__ v, int n) {
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int i = blockIdx.x * NTHREADS + threadIdx.x; i < n; i += gridDim.x * NTHREADS)
        am_merge(bv, bi, v[i], i);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        float ov = __shfl_xor(bv, m);
        int oi = __shfl_xor(bi, m);
        am_merge(bv, bi, ov, oi);
    }
    __shared__ float sv[4];
    __shared__ int si[4];
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { sv[wave] = bv; si[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) am_merge(bv, bi, sv[w], si[w]);
        pv[blockIdx.x] = bv;
        pi[blockIdx.x] = bi;
    }
}

__global__ __launch_bounds__(WAVE) void k_argmax_final(int *__restrict__ out,
                                                      const float *__restrict__ pv,
                                                      const int *__restrict__ pi, int np,
                                                      const float *__restrict__ v) {
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int i = threadIdx.x; i < np; i += WAVE) am_merge(bv, bi, pv[i], pi[i]);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        float ov = __shfl_xor(bv, m);
        int oi = __shfl_xor(bi, m);
        am_merge(bv, bi, ov, oi);
    }
    // the reference's scan starts from v[0]; a NaN there is never beaten
    if (threadIdx.x == 0) out[0] = (bi == 0x7FFFFFFF || v[0] != v[0]) ? 0 : bi;
}

// plain 16-byte-vector copy: a kernel of known traffic (bytes read = bytes
// written = n16 * 16) against which HBM traffic counters are calibrated
__global__ __launch_bounds__(NTHREADS) void k_copy16(u32x4 *__restrict__ dst,
                                                    const u32x4 *__restrict__ src, size_t n16) {
    for (size_t i = (size_t)blockIdx.x * NTHREADS + threadIdx.x; i < n16;
         i += (size_t)gridDim.x * NTHREADS)
        dst[i] = __builtin_nontemporal_load(src + i);
}

// Reads n16 16-byte chunks once and writes nothing: the decode GEMVs' load
// form (buffer loads, non-temporal, a wave covering 1 KB per instruction),
// four loads in flight per lane per step.  The reference for read-traffic
// counters: its traffic is exactly the bytes read.  n16 * 16 < 2^31.
__global__ __launch_bounds__(NTHREADS) void k_read16(const u32x4 *__restrict__ src, size_t n16) {
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(src, n16 * 16);
    const uint32_t stride = gridDim.x * NTHREADS;
    u32x4 acc = {0u, 0u, 0u, 0u};
    for (uint32_t i = blockIdx.x * NTHREADS + threadIdx.x; i < n16; i += 4 * stride) {
        u32x4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const uint32_t q = i + u * stride;
            v[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, q < n16 ? q * 16u : BUF_OOB, 0, 2);
        }
#pragma unroll
        for (int u = 0; u < 4; u++) acc ^= v[u];
    }
    asm volatile("" ::"v"(acc.x), "v"(acc.y), "v"(acc.z), "v"(acc.w));
}

// dst[i] = bf16 RNE of src[i]; 8 elements per lane per step (n % 8 == 0,
// 16-byte aligned src and dst)
__global__ __launch_bounds__(NTHREADS) void k_cvt_bf16(uint16_t *__restrict__ dst,
                                                       const float *__restrict__ src, size_t n8) {
    for (size_t i = (size_t)blockIdx.x * NTHREADS + threadIdx.x; i < n8; i += (size_t)gridDim.x * NTHREADS) {
        const f32x4 x0 = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(src) + 2 * i);
        const f32x4 x1 = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(src) + 2 * i + 1);
        u32x4 w;
        w.x = pack_bf16x2(x0.x, x0.y);
        w.y = pack_bf16x2(x0.z, x0.w);
        w.z = pack_bf16x2(x1.x, x1.y);
        w.w = pack_bf16x2(x1.z, x1.w);
        reinterpret_cast<u32x4 *>(dst)[i] = w;
    }
}

__global__ __launch_bounds__(NTHREADS) void k_fill_zero(float *__restrict__ c, size_t n) {
    for (size_t i = (size_t)blockIdx.x * NTHREADS + threadIdx.x; i < n;
         i += (size_t)gridDim.x * NTHREADS)
        c[i] = 0.0f;
}

#endif  // QH_MISC_KERNELS_H
