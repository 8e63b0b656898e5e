// GEMV kernels for M <= 16: the M = 1 decode GEMV with its fused prologues
// (RMSNorm, residual add, embedding row, attention merge, activation row in
// the kernel arguments), the 2 <= M <= 4 GEMV and the small-batch GEMV.
// Included by hip_gemm.hip, whose host code launches them.
#ifndef QH_GEMV_KERNELS_H
#define QH_GEMV_KERNELS_H

#include "gemm_common.h"
#include "fp_pinned.h"

// ---------------------------------------------------------------------------
// GEMV: M <= 4
// ---------------------------------------------------------------------------
// One halving step per template level, so that every index below is a
// constant (a loop over a run-time `half` would index v dynamically).
template <int HALF, int MASK>
__device__ __forceinline__ void wave_halving_steps(float *v, int lane) {
    if constexpr (HALF >= 1) {
        const bool hi = (lane & MASK) != 0;
#pragma unroll
        for (int i = 0; i < HALF; i++) {
            const float send = hi ? v[i] : v[i + HALF];
            const float keep = hi ? v[i + HALF] : v[i];
            v[i] = keep + __shfl_xor(send, MASK);
        }
        wave_halving_steps<HALF / 2, MASK / 2>(v, lane);
    }
}
// After this, lane l holds the 64-lane total of value index l >> (6 - log2 V).
// Each halving step trades half of the values with the partner lane, so a
// lane ends up owning one value after log2(V) exchanges instead of V*6.
template <int V>
__device__ __forceinline__ float wave_transpose_reduce(float (&v)[V], int lane) {
    static_assert(V >= 1 && V <= 64 && (V & (V - 1)) == 0, "V must be a power of 2 <= 64");
    wave_halving_steps<V / 2, 32>(v, lane);
    constexpr int L = (V >= 64) ? 6 : (V >= 32) ? 5 : (V >= 16) ? 4 : (V >= 8) ? 3 : (V >= 4) ? 2 : (V >= 2) ? 1 : 0;
    float x = v[0];
#pragma unroll
    for (int mask = 32 >> L; mask >= 1; mask >>= 1) x += __shfl_xor(x, mask);
    return x;
}

template <int X> struct pow2_ceil { static constexpr int v = (X <= 1) ? 1 : 2 * pow2_ceil<(X + 1) / 2>::v; };
template <> struct pow2_ceil<1> { static constexpr int v = 1; };

// grid.x = ceil(N / (4 * ROWS)); block = 256 (4 waves); dynamic LDS = MR*K*4.
// Requires K % 8 == 0 and 16-byte aligned a and b.  Rows >= N are clamped
// for loading and never stored.
template <int MR, int ROWS, int CU>
__global__ __launch_bounds__(NTHREADS) void k_gemv(float *__restrict__ c,
                                                  const float *__restrict__ a,
                                                  const uint16_t *__restrict__ b,
                                                  int K, int N) {
    extern __shared__ float sA[];   // [MR][K], rounded to bf16
    const int tid = threadIdx.x;
    {
        const f32x4 *a4 = reinterpret_cast<const f32x4 *>(a);
        f32x4 *s4 = reinterpret_cast<f32x4 *>(sA);
        const int n4 = (MR * K) >> 2;
        for (int i = tid; i < n4; i += NTHREADS) {
            f32x4 v = a4[i];
            v.x = round_bf16(v.x); v.y = round_bf16(v.y);
            v.z = round_bf16(v.z); v.w = round_bf16(v.w);
            s4[i] = v;
        }
    }
    __syncthreads();

    const int wave = tid >> 6, lane = tid & 63;
    const int row0 = (blockIdx.x * 4 + wave) * ROWS;
    if (row0 >= N) return;             // no barrier below this point
    const int nch = K >> 3;            // 16-byte chunks per row
    const u32x4 *b4 = reinterpret_cast<const u32x4 *>(b);

    constexpr int V = pow2_ceil<MR * ROWS>::v;
    float acc[V];
#pragma unroll
    for (int i = 0; i < V; i++) acc[i] = 0.0f;

    for (int c0 = lane; c0 < nch; c0 += WAVE * CU) {
        u32x4 bv[CU][ROWS];
#pragma unroll
        for (int u = 0; u < CU; u++) {
            const int ch = c0 + WAVE * u;
#pragma unroll
            for (int r = 0; r < ROWS; r++) {
                const int row = min(row0 + r, N - 1);
                if (ch < nch)
                    bv[u][r] = __builtin_nontemporal_load(b4 + (size_t)row * nch + ch);
                else
                    bv[u][r] = u32x4{0u, 0u, 0u, 0u};
            }
        }
#pragma unroll
        for (int u = 0; u < CU; u++) {
            const int ch = c0 + WAVE * u;
            if (ch < nch) {
#pragma unroll
                for (int m = 0; m < MR; m++) {
                    const f32x4 *ap = reinterpret_cast<const f32x4 *>(sA + m * K + ch * 8);
                    const f32x4 x0 = ap[0], x1 = ap[1];
                    const float av[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                    for (int r = 0; r < ROWS; r++) {
                        float s = acc[m * ROWS + r];
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            s = fmaf(av[2 * e], bf16_lo(bv[u][r][e]), s);
                            s = fmaf(av[2 * e + 1], bf16_hi(bv[u][r][e]), s);
                        }
                        acc[m * ROWS + r] = s;
                    }
                }
            }
        }
    }

    constexpr int LV = (V >= 64) ? 6 : (V >= 32) ? 5 : (V >= 16) ? 4 : (V >= 8) ? 3 : (V >= 4) ? 2 : (V >= 2) ? 1 : 0;
    const float tot = wave_transpose_reduce<V>(acc, lane);
    const int idx = lane >> (6 - LV);
    if ((lane & ((64 >> LV) - 1)) == 0) {
        const int m = idx / ROWS, r = idx % ROWS;
        if (m < MR && row0 + r < N) c[(size_t)m * N + row0 + r] = tot;
    }
}

// GEMV-shaped GEMM for 5 <= M <= MR (8 or 16) and K <= 512 * CPL: every
// weight row is read once, with each load instruction covering 1 KB of one
// row (lane l owns the 16-byte chunks l, l + 64, ... of every row), and the
// M rows of A are applied to it from registers with v_dot2_f32_bf16.  The
// block's NWV waves first load A once between them (fp32, from L2) and
// round it to bf16 into LDS, then every wave issues its ROWS * CPL weight
// loads, and A is passed to the lanes while the weights are in flight: a
// launch costs one HBM round trip.  The ROWS * MR sums of a wave are reduced
// across its lanes by halving exchanges, one value per lane at the end.
// Rows of A past M are zeros; weight rows past N read zeros and are not
// stored.  Dynamic LDS: MR * K * 2 bytes.
template <int MR, int ROWS, int CPL, int NWV>
__global__ __launch_bounds__(NWV * WAVE) void k_gemv_m(float *__restrict__ c, const float *__restrict__ a,
                                                      const uint16_t *__restrict__ b, int M, int K, int N) {
    constexpr int NT = NWV * WAVE;                    // threads per block
    extern __shared__ u32x4 sa_m[];                   // [MR][K / 8] bf16 chunks
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nch = K >> 3;
    const int row0 = (blockIdx.x * NWV + wave) * ROWS;

    // 1. A -> registers (fp32, from L2): MR rows of nch chunks over the block
    const __amdgpu_buffer_rsrc_t ra = buf_rsrc(a, (size_t)M * K * 4);
    constexpr int AQ = (MR * WAVE * CPL + NT - 1) / NT;  // chunks per thread at K = 512 CPL
    u32x4 alo[AQ], ahi[AQ];
#pragma unroll
    for (int i = 0; i < AQ; i++) {
        const int q = tid + NT * i;
        const int m = q / nch, ch = q - m * nch;
        const bool ok = q < MR * nch && m < M;
        const uint32_t off = ((uint32_t)m * K + 8 * ch) * 4u;   // M * K * 4 < 2^31
        alo[i] = __builtin_amdgcn_raw_buffer_load_b128(ra, ok ? off : BUF_OOB, 0, 0);
        ahi[i] = __builtin_amdgcn_raw_buffer_load_b128(ra, ok ? off + 16u : BUF_OOB, 0, 0);
    }
    // 2. this wave's weights: rows row0 + r, chunks lane + 64 j (non-temporal)
    const __amdgpu_buffer_rsrc_t rb = buf_rsrc(b, (size_t)N * K * 2);
    u32x4 bw[ROWS][CPL];
#pragma unroll
    for (int r = 0; r < ROWS; r++)
#pragma unroll
        for (int j = 0; j < CPL; j++) {
            const int ch = lane + WAVE * j;
            const bool ok = row0 + r < N && ch < nch;
            const uint32_t off = ((uint32_t)(row0 + r) * K + 8 * ch) * 2u;   // N * K * 2 < 2^31
            bw[r][j] = __builtin_amdgcn_raw_buffer_load_b128(rb, ok ? off : BUF_OOB, 0, 2);
        }
    __builtin_amdgcn_sched_barrier(0);
    // 3. A rounded to bf16 (RNE) into LDS while the weights are in flight
#pragma unroll
    for (int i = 0; i < AQ; i++) {
        const int q = tid + NT * i;
        u32x4 v;
        v.x = pack_bf16x2(__uint_as_float(alo[i].x), __uint_as_float(alo[i].y));
        v.y = pack_bf16x2(__uint_as_float(alo[i].z), __uint_as_float(alo[i].w));
        v.z = pack_bf16x2(__uint_as_float(ahi[i].x), __uint_as_float(ahi[i].y));
        v.w = pack_bf16x2(__uint_as_float(ahi[i].z), __uint_as_float(ahi[i].w));
        if (q < MR * nch) sa_m[q] = v;
    }
    __syncthreads();
    // 4. sums: acc[r * MR + m] over this lane's chunks
    constexpr int V = pow2_ceil<ROWS * MR>::v;
    float acc[V];
#pragma unroll
    for (int i = 0; i < V; i++) acc[i] = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; j++) {
        // chunks past K: the weights read zeros, so any A chunk will do
        const int ch = min(lane + WAVE * j, nch - 1);
#pragma unroll
        for (int m = 0; m < MR; m++) {
            const u32x4 x = sa_m[m * nch + ch];
#pragma unroll
            for (int r = 0; r < ROWS; r++) {
                float t = acc[r * MR + m];
                t = bf16_dot2(bw[r][j].x, x.x, t);
                t = bf16_dot2(bw[r][j].y, x.y, t);
                t = bf16_dot2(bw[r][j].z, x.z, t);
                t = bf16_dot2(bw[r][j].w, x.w, t);
                acc[r * MR + m] = t;
            }
        }
    }
    // 5. reduce over the lanes; value index r * MR + m ends in lane group idx
    constexpr int LV = (V >= 64) ? 6 : (V >= 32) ? 5 : (V >= 16) ? 4 : (V >= 8) ? 3 : (V >= 4) ? 2 : (V >= 2) ? 1 : 0;
    const float tot = wave_transpose_reduce<V>(acc, lane);
    const int idx = lane >> (6 - LV);
    if ((lane & ((64 >> LV) - 1)) == 0 && idx < ROWS * MR) {
        const int r = idx / MR, m = idx % MR;
        if (m < M && row0 + r < N) c[(size_t)m * N + row0 + r] = tot;
    }
}

__device__ const int k_zero_token = 0;     // token read by prologues without an embedding

// Activation prologue of the M = 1 GEMV (decode): the GEMV input is
//   a = rmsnorm(x + r) * nw       (fpga_bringup/src/src/ops_scalar.c:11-16,
//                                  residual add ops_scalar.c:53-55)
// where x is either an fp32 row or, when emb is set, the bf16 embedding row
// emb[*tok] (qwen3.c:295-298).  Block 0 stores x + r to x_out when x_out is
// set (the updated residual stream).
struct GemvPro {
    const float *x;
    const uint16_t *emb;
    const int *tok;
    int emb_rows;
    const float *r;
    const uint16_t *nw;
    float *x_out;
    float eps;
};

// M = 1 fast path (decode).  One wave owns ROWS output rows; lane l owns the
// 16-byte chunks l, l+64, ..., l+64*(CPL-1) of every row (CPL = chunks per
// lane, K <= 512*CPL).  The block's 256 threads first load the activation
// row once between them (a quarter per wave, 16 B per thread per 4 KB of
// row), then every wave issues all of its ROWS*CPL non-temporal weight
// loads; the activation (rounded to bf16, and for PRO normalised first) is
// exchanged through LDS while the weights are still in flight, so a launch
// costs one HBM round trip and each block reads the activation from L2
// once instead of once per wave.  GATED: rows of Wg and Wu with the same
// index are both loaded and the epilogue writes silu(gate) * up.  PRO: the
// activation row comes from the GemvPro prologue instead of a.
// Dynamic LDS: (K + 8) floats.  Waves without rows still take part in the
// barriers.
// MERGE: a holds split attention partials (qh_gemv_merge) and the activation
// row is their softmax merge; their loads go out before the weight loads,
// the merge arithmetic after them.
// KA: the activation row arrives already rounded to packed bf16 pairs in the
// kernel arguments (ka: the kernel-argument segment, GemvKaRow first) -- the
// host-pointer path's M = 1 calls with K <= 3072, which then need no copy of
// A to the device before the GEMV.
template <int ROWS, int CPL, bool GATED, bool PRO, bool MERGE, bool KA>
__device__ __forceinline__ void gemv1_body(float *__restrict__ c, const float *__restrict__ a,
                                           const uint16_t *__restrict__ b, const uint16_t *__restrict__ b2,
                                           int K, int N, GemvPro pro, const uint2 *__restrict__ ka) {
    constexpr int NB = GATED ? 2 * ROWS : ROWS;     // weight rows per wave
    constexpr int NQ = CPL * 2 * WAVE;               // 4-element groups of the padded row (512*CPL)
    constexpr int QMAX = (NQ + NTHREADS - 1) / NTHREADS;
    extern __shared__ __align__(16) uint32_t sx[];   // [2*NQ] bf16 pairs of the padded row, then [4] floats
    float *sred = reinterpret_cast<float *>(sx + 2 * NQ);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int row0 = (blockIdx.x * (NTHREADS / WAVE) + wave) * ROWS;
    // MERGE is launched for K = 2048 only (the 16 x 128 attention output),
    // whose 512 groups the 256 threads cover exactly: its merge has no tail
    static_assert(!MERGE || (CPL == 4 && QMAX == 2), "MERGE expects K = 2048");
    const int nch = K >> 3, nq = K >> 2;

    // 1. this thread's share of the activation row (issued before the
    //    weights; groups past K read zeros)
    f32x4 xa[QMAX];
    uint2 wn[QMAX];
    f32x4 xv[PRO ? QMAX : 1], rv[PRO ? QMAX : 1];    // prologue sources (x, r, embedding row)
    uint2 e[PRO ? QMAX : 1];
    constexpr int MS = MERGE ? QH_ATT_SPLITS : 1;
    f32x4 mo[MERGE ? QMAX : 1][MS];
    float2 mml[MERGE ? QMAX : 1][MS];
    // Scheduling barriers keep the activation-side loads ahead of the weight
    // loads and their arithmetic behind them, so a wave waits for the
    // activation alone before its LDS store.
    if constexpr (MERGE) {
        // group i = dims 4i .. 4i+3 of the 2048-vector: head i/32 (kv head
        // i/64, query head (i/32)&1 of the group), d4 = i%32
        const __amdgpu_buffer_rsrc_t rp = buf_rsrc(a, (size_t)8 * QH_ATT_SPLITS * 2 * QH_ATT_PART * 4);
#pragma unroll
        for (int q = 0; q < QMAX; q++) {
            const int ii = tid + NTHREADS * q;       // < 512 = nq: no tail for K = 2048
            const uint32_t pb = (uint32_t)(((ii >> 6) * QH_ATT_SPLITS * 2 + ((ii >> 5) & 1)) * QH_ATT_PART) * 4u;
#pragma unroll
            for (int s = 0; s < MS; s++) {
                const uint32_t ps = pb + (uint32_t)(s * 2 * QH_ATT_PART) * 4u;
                mml[q][s] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rp, ps, 0, 0));
                mo[q][s] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                         rp, ps + 16u + (uint32_t)(ii & 31) * 16u, 0, 0));
            }
        }
    } else if constexpr (KA) {
        // nothing to load ahead: the row is in the kernel arguments
    } else if constexpr (!PRO) {
        const __amdgpu_buffer_rsrc_t ra = buf_rsrc(a, (size_t)K * 4);
#pragma unroll
        for (int q = 0; q < QMAX; q++) {
            const int i = tid + NTHREADS * q;
            xa[q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  ra, i < nq ? (uint32_t)i * 16 : BUF_OOB, 0, 0));
        }
    } else {
        // x + r, or the embedding row of the device-held token: every source
        // is loaded, absent ones from empty buffers, which read as zeros, so
        // the prologue has no branch
        const bool emb = pro.emb != nullptr;
        int t = *(emb ? pro.tok : &k_zero_token);
        t = t < 0 ? 0 : (t >= pro.emb_rows ? pro.emb_rows - 1 : t);
        const __amdgpu_buffer_rsrc_t re = buf_rsrc(emb ? pro.emb + (size_t)t * K : nullptr, emb ? (size_t)K * 2 : 0);
        const __amdgpu_buffer_rsrc_t rx = buf_rsrc(pro.x, (pro.x && !emb) ? (size_t)K * 4 : 0);
        const __amdgpu_buffer_rsrc_t rr = buf_rsrc(pro.r, (pro.r && !emb) ? (size_t)K * 4 : 0);
        const __amdgpu_buffer_rsrc_t rw = buf_rsrc(pro.nw, (size_t)K * 2);
#pragma unroll
        for (int q = 0; q < QMAX; q++) {
            const int i = tid + NTHREADS * q;
            const uint32_t o16 = i < nq ? (uint32_t)i * 16 : BUF_OOB, o8 = i < nq ? (uint32_t)i * 8 : BUF_OOB;
            xv[q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, o16, 0, 0));
            rv[q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rr, o16, 0, 0));
            e[q] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(re, o8, 0, 0));
            wn[q] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rw, o8, 0, 0));
        }
    }
    __builtin_amdgcn_sched_barrier(0);               // the activation loads go out first

    // 2. all weight loads of this wave; rows past N and chunks past K read
    //    zeros (the caller keeps N*K*2 below 2 GiB)
    const __amdgpu_buffer_rsrc_t rb = buf_rsrc(b, (size_t)N * K * 2);
    const __amdgpu_buffer_rsrc_t rb2 = buf_rsrc(GATED ? b2 : b, (size_t)N * K * 2);
    u32x4 bv[NB][CPL];
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
        const int row = row0 + r;
#pragma unroll
        for (int j = 0; j < CPL; j++) {
            const int ch = lane + WAVE * j;
            const uint32_t off = (row < N && ch < nch) ? (uint32_t)row * (uint32_t)K * 2u + (uint32_t)ch * 16u
                                                       : BUF_OOB;
            bv[r][j] = __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 2);      // nt: read once
            if constexpr (GATED) bv[ROWS + r][j] = __builtin_amdgcn_raw_buffer_load_b128(rb2, off, 0, 2);
        }
    }
    __builtin_amdgcn_sched_barrier(0);               // ... then every weight load

    // 3. activation through LDS as bf16 (RNE), normalised first for PRO;
    //    zeros past K
    uint2 *sx2 = reinterpret_cast<uint2 *>(sx);
    if constexpr (KA) {
        // the host rounded the row and zeroed it past K
#pragma unroll
        for (int q = 0; q < QMAX; q++) {
            const int i = tid + NTHREADS * q;
            if (NQ % NTHREADS == 0 || i < NQ) sx2[i] = ka[i];
        }
    } else if constexpr (PRO) {
#pragma unroll
        for (int q = 0; q < QMAX; q++)
            xa[q] = f32x4{bf16_lo(e[q].x), bf16_hi(e[q].x), bf16_lo(e[q].y), bf16_hi(e[q].y)} + (xv[q] + rv[q]);
        float ss = 0.0f;
#pragma unroll
        for (int q = 0; q < QMAX; q++)
            ss += sumsq4(xa[q].x, xa[q].y, xa[q].z, xa[q].w);
        ss = wave_sum(ss);
        if (lane == 0) sred[wave] = ss;
        if (pro.x_out && blockIdx.x == 0) {
#pragma unroll
            for (int q = 0; q < QMAX; q++) {
                const int i = tid + NTHREADS * q;
                if (i < nq) reinterpret_cast<f32x4 *>(pro.x_out)[i] = xa[q];
            }
        }
        __syncthreads();
        ss = (sred[0] + sred[1]) + (sred[2] + sred[3]);
        const float scale = 1.0f / sqrtf(ss / (float)K + pro.eps);
#pragma unroll
        for (int q = 0; q < QMAX; q++) {
            const int i = tid + NTHREADS * q;
            if (NQ % NTHREADS == 0 || i < NQ)
                sx2[i] = uint2{pack_bf16x2((xa[q].x * scale) * bf16_lo(wn[q].x), (xa[q].y * scale) * bf16_hi(wn[q].x)),
                               pack_bf16x2((xa[q].z * scale) * bf16_lo(wn[q].y), (xa[q].w * scale) * bf16_hi(wn[q].y))};
        }
    } else {
        if constexpr (MERGE) {
#pragma unroll
            for (int q = 0; q < QMAX; q++) {
                float mx = mml[q][0].x;
#pragma unroll
                for (int s = 1; s < MS; s++) mx = fmaxf(mx, mml[q][s].x);
                float den = 0.0f;
                f32x4 num = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < MS; s++) {
                    const float w = mml[q][s].x == -INFINITY ? 0.0f : expf(mml[q][s].x - mx);
                    den = fmaf(w, mml[q][s].y, den);
                    num.x = fmaf(w, mo[q][s].x, num.x);
                    num.y = fmaf(w, mo[q][s].y, num.y);
                    num.z = fmaf(w, mo[q][s].z, num.z);
                    num.w = fmaf(w, mo[q][s].w, num.w);
                }
                const float inv = 1.0f / den;
                xa[q] = num * inv;
            }
        }
#pragma unroll
        for (int q = 0; q < QMAX; q++) {
            const int i = tid + NTHREADS * q;
            if (NQ % NTHREADS == 0 || i < NQ)
                sx2[i] = uint2{pack_bf16x2(xa[q].x, xa[q].y), pack_bf16x2(xa[q].z, xa[q].w)};
        }
    }
    __syncthreads();

    // 4. this lane's activation chunks, then packed bf16 dot products
    u32x4 xc[CPL];
#pragma unroll
    for (int j = 0; j < CPL; j++) xc[j] = reinterpret_cast<const u32x4 *>(sx)[lane + WAVE * j];
    float acc[NB];
#pragma unroll
    for (int r = 0; r < NB; r++) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) s = bf16_dot2(bv[r][j][e], xc[j][e], s);
        acc[r] = s;
    }

    // 5. wave sums (every lane holds every row's total); lane r stores row r
    float tot = 0.0f, up = 0.0f;
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
        const float t = wave_sum(acc[r]);
        tot = lane == r ? t : tot;
        if constexpr (GATED) {
            const float u = wave_sum(acc[ROWS + r]);
            up = lane == r ? u : up;
        }
    }
    if (lane < ROWS && row0 + lane < N) c[row0 + lane] = GATED ? silu_mul(tot, up) : tot;
}

template <int ROWS, int CPL, bool GATED, bool PRO = false, bool MERGE = false>
__global__ __launch_bounds__(NTHREADS) void k_gemv1(float *__restrict__ c,
                                                   const float *__restrict__ a,
                                                   const uint16_t *__restrict__ b,
                                                   const uint16_t *__restrict__ b2,
                                                   int K, int N, GemvPro pro) {
    gemv1_body<ROWS, CPL, GATED, PRO, MERGE, false>(c, a, b, b2, K, N, pro, nullptr);
}

// the activation row of a KA launch: K <= 512 CPL bf16 values (at least
// 1024), zero past K (first kernel argument, so it sits at offset 0 of the
// argument segment; 6 KB at K = 3072, within what gfx950 launches accept)
template <int CPL>
struct GemvKaRow {
    static constexpr int WORDS = CPL <= 2 ? 512 : 256 * CPL;
    uint32_t w[WORDS];
};
template <int ROWS, int CPL, bool GATED>
__global__ __launch_bounds__(NTHREADS) void k_gemv1_ka(GemvKaRow<CPL> row, float *__restrict__ c,
                                                      const uint16_t *__restrict__ b,
                                                      const uint16_t *__restrict__ b2, int K, int N) {
    (void)row;   // read in place, through the argument segment
    const uint2 *ka = (const uint2 *)__builtin_amdgcn_kernarg_segment_ptr();   // address space 4 to generic
    gemv1_body<ROWS, CPL, GATED, false, false, true>(c, nullptr, b, b2, K, N, GemvPro{}, ka);
}

// Fused gate/up GEMV: rows of Wg and Wu with the same index share a wave, and
// the epilogue writes silu(gate) * up.  Same constraints as k_gemv.
template <int MR, int ROWS, int CU>
__global__ __launch_bounds__(NTHREADS) void k_gemv_gated(float *__restrict__ h,
                                                        const float *__restrict__ x,
                                                        const uint16_t *__restrict__ wg,
                                                        const uint16_t *__restrict__ wu,
                                                        int K, int N) {
    extern __shared__ float sA[];
    const int tid = threadIdx.x;
    {
        const f32x4 *a4 = reinterpret_cast<const f32x4 *>(x);
        f32x4 *s4 = reinterpret_cast<f32x4 *>(sA);
        const int n4 = (MR * K) >> 2;
        for (int i = tid; i < n4; i += NTHREADS) {
            f32x4 v = a4[i];
            v.x = round_bf16(v.x); v.y = round_bf16(v.y);
            v.z = round_bf16(v.z); v.w = round_bf16(v.w);
            s4[i] = v;
        }
    }
    __syncthreads();

    const int wave = tid >> 6, lane = tid & 63;
    const int row0 = (blockIdx.x * 4 + wave) * ROWS;
    if (row0 >= N) return;
    const int nch = K >> 3;
    const u32x4 *g4 = reinterpret_cast<const u32x4 *>(wg);
    const u32x4 *u4 = reinterpret_cast<const u32x4 *>(wu);

    constexpr int V = pow2_ceil<2 * MR * ROWS>::v;
    float acc[V];
#pragma unroll
    for (int i = 0; i < V; i++) acc[i] = 0.0f;

    for (int c0 = lane; c0 < nch; c0 += WAVE * CU) {
        u32x4 bv[CU][2 * ROWS];
#pragma unroll
        for (int u = 0; u < CU; u++) {
            const int ch = c0 + WAVE * u;
#pragma unroll
            for (int r = 0; r < ROWS; r++) {
                const int row = min(row0 + r, N - 1);
                if (ch < nch) {
                    bv[u][r] = __builtin_nontemporal_load(g4 + (size_t)row * nch + ch);
                    bv[u][ROWS + r] = __builtin_nontemporal_load(u4 + (size_t)row * nch + ch);
                } else {
                    bv[u][r] = u32x4{0u, 0u, 0u, 0u};
                    bv[u][ROWS + r] = u32x4{0u, 0u, 0u, 0u};
                }
            }
        }
#pragma unroll
        for (int u = 0; u < CU; u++) {
            const int ch = c0 + WAVE * u;
            if (ch < nch) {
#pragma unroll
                for (int m = 0; m < MR; m++) {
                    const f32x4 *ap = reinterpret_cast<const f32x4 *>(sA + m * K + ch * 8);
                    const f32x4 x0 = ap[0], x1 = ap[1];
                    const float av[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                    for (int r = 0; r < 2 * ROWS; r++) {
                        float s = acc[m * 2 * ROWS + r];
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            s = fmaf(av[2 * e], bf16_lo(bv[u][r][e]), s);
                            s = fmaf(av[2 * e + 1], bf16_hi(bv[u][r][e]), s);
                        }
                        acc[m * 2 * ROWS + r] = s;
                    }
                }
            }
        }
    }

    constexpr int LV = (V >= 64) ? 6 : (V >= 32) ? 5 : (V >= 16) ? 4 : (V >= 8) ? 3 : (V >= 4) ? 2 : (V >= 2) ? 1 : 0;
    const float tot = wave_transpose_reduce<V>(acc, lane);
    // value index idx = m*2*ROWS + r (r < ROWS: gate, r >= ROWS: up); bring
    // the up total to the lane that holds the matching gate total
    const int idx = lane >> (6 - LV);
    const int step = 64 >> LV;                       // lanes per value
    const float up = __shfl(tot, (lane + ROWS * step) & 63);
    if ((lane & (step - 1)) == 0) {
        const int m = idx / (2 * ROWS), r = idx % (2 * ROWS);
        if (m < MR && r < ROWS && row0 + r < N)
            h[(size_t)m * N + row0 + r] = silu_mul(tot, up);
    }
}

#endif  // QH_GEMV_KERNELS_H
