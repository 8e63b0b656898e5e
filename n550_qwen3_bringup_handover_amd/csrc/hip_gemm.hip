// CDNA4 (gfx950) kernels for the Qwen3-0.6B projection GEMMs and the shim
// functions that launch them.  Semantics follow the reference GEMM plug-in
// (fpga_bringup/src/src/kernels.h:44-57): C[M,N] = A[M,K] . B[N,K]^T with A
// fp32 row-major, B bf16 bits row-major [out, in], C fp32 row-major,
// C overwritten.  A is rounded to bf16 with round-to-nearest-even on the
// load path (the AME kernel does the same, kernels_ame.c:219-236), products
// of two bf16 values are exact in fp32, and accumulation is fp32.
//
// Kernels:
//   k_gemv<MR,ROWS,CU>   M <= 4: streams B once with 128-bit non-temporal
//                        loads; A staged in LDS; a transposing wave
//                        reduction of ROWS*MR partial sums per lane.
//   k_gemm<...>          M > 4: 256-thread workgroups, 4 waves, bf16 MFMA
//                        16x16x32 with fp32 accumulate, A/B tiles staged
//                        through XOR-swizzled LDS, double-buffered; optional
//                        gated epilogue h = silu(gate) * up.
//   k_tile_to_row        weight re-layout for the tile-major blob format.
//   k_argmax_*           first-max reduction for greedy decoding.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "hip_shim.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

#define WAVE 64
#define NTHREADS 256

// ---------------------------------------------------------------------------
// bf16 helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// two fp32 -> packed bf16 pair (low half = first), RNE (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pack_bf16x2(float x, float y) {
    uint32_t lo = __builtin_bit_cast(uint16_t, (__bf16)x);
    uint32_t hi = __builtin_bit_cast(uint16_t, (__bf16)y);
    return lo | (hi << 16);
}
__device__ __forceinline__ float round_bf16(float x) {
    return __uint_as_float((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x) << 16);
}

__device__ __forceinline__ float silu_mul(float g, float u) {
    // reference: (g / (1 + expf(-g))) * u  (ops_scalar.c:46-51)
    return (g / (1.0f + expf(-g))) * u;
}

// ---------------------------------------------------------------------------
// GEMV: M <= 4
// ---------------------------------------------------------------------------
// After this, lane l holds the 64-lane total of value index l >> (6 - log2 V).
// Each halving step trades half of the values with the partner lane, so a
// lane ends up owning one value after log2(V) exchanges instead of V*6.
template <int V>
__device__ __forceinline__ float wave_transpose_reduce(float (&v)[V], int lane) {
    static_assert(V >= 1 && V <= 64 && (V & (V - 1)) == 0, "V must be a power of 2 <= 64");
#pragma unroll
    for (int s = 0, half = V / 2; half >= 1; s++, half /= 2) {
        const int mask = 32 >> s;
        const bool hi = (lane & mask) != 0;
#pragma unroll
        for (int i = 0; i < half; i++) {
            float send = hi ? v[i] : v[i + half];
            float keep = hi ? v[i + half] : v[i];
            v[i] = keep + __shfl_xor(send, mask);
        }
    }
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

// M = 1 fast path (decode).  One wave owns ROWS output rows; lane l owns the
// 16-byte chunks l, l+64, ..., l+64*(CPL-1) of every row (CPL = chunks per
// lane, K <= 512*CPL).  All ROWS*CPL weight loads and the 2*CPL activation
// loads are issued before the first use, so a launch costs one memory round
// trip; there is no LDS and no barrier.  GATED: rows of Wg and Wu with the
// same index are both loaded and the epilogue writes silu(gate) * up.
template <int ROWS, int CPL, bool GATED>
__global__ __launch_bounds__(NTHREADS) void k_gemv1(float *__restrict__ c,
                                                   const float *__restrict__ a,
                                                   const uint16_t *__restrict__ b,
                                                   const uint16_t *__restrict__ b2,
                                                   int K, int N) {
    constexpr int NB = GATED ? 2 * ROWS : ROWS;     // weight rows per wave
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * (NTHREADS / WAVE) + wave) * ROWS;
    if (row0 >= N) return;
    const int nch = K >> 3;
    const u32x4 *b4 = reinterpret_cast<const u32x4 *>(b);
    const u32x4 *u4 = reinterpret_cast<const u32x4 *>(b2);

    u32x4 bv[NB][CPL];
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
        const size_t rb = (size_t)min(row0 + r, N - 1) * nch;
#pragma unroll
        for (int j = 0; j < CPL; j++) {
            const int ch = lane + WAVE * j;
            if (ch < nch) {
                bv[r][j] = __builtin_nontemporal_load(b4 + rb + ch);
                if constexpr (GATED) bv[ROWS + r][j] = __builtin_nontemporal_load(u4 + rb + ch);
            } else {
                bv[r][j] = u32x4{0u, 0u, 0u, 0u};
                if constexpr (GATED) bv[ROWS + r][j] = u32x4{0u, 0u, 0u, 0u};
            }
        }
    }
    float av[CPL][8];
#pragma unroll
    for (int j = 0; j < CPL; j++) {
        const int ch = lane + WAVE * j;
        if (ch < nch) {
            const f32x4 *ap = reinterpret_cast<const f32x4 *>(a + ch * 8);
            const f32x4 x0 = ap[0], x1 = ap[1];
            av[j][0] = x0.x; av[j][1] = x0.y; av[j][2] = x0.z; av[j][3] = x0.w;
            av[j][4] = x1.x; av[j][5] = x1.y; av[j][6] = x1.z; av[j][7] = x1.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) av[j][e] = 0.0f;
        }
    }
#pragma unroll
    for (int j = 0; j < CPL; j++)
#pragma unroll
        for (int e = 0; e < 8; e++) av[j][e] = round_bf16(av[j][e]);

    constexpr int V = pow2_ceil<NB>::v;
    float acc[V];
#pragma unroll
    for (int i = 0; i < V; i++) acc[i] = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; j++)
#pragma unroll
        for (int r = 0; r < NB; r++) {
            float s = acc[r];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                s = fmaf(av[j][2 * e], bf16_lo(bv[r][j][e]), s);
                s = fmaf(av[j][2 * e + 1], bf16_hi(bv[r][j][e]), s);
            }
            acc[r] = s;
        }

    constexpr int LV = (V >= 64) ? 6 : (V >= 32) ? 5 : (V >= 16) ? 4 : (V >= 8) ? 3 : (V >= 4) ? 2 : (V >= 2) ? 1 : 0;
    const float tot = wave_transpose_reduce<V>(acc, lane);
    const int idx = lane >> (6 - LV);
    const int step = 64 >> LV;                       // lanes holding each value
    if constexpr (!GATED) {
        if ((lane & (step - 1)) == 0 && idx < ROWS && row0 + idx < N) c[row0 + idx] = tot;
    } else {
        const float up = __shfl(tot, (lane + ROWS * step) & 63);
        if ((lane & (step - 1)) == 0 && idx < ROWS && row0 + idx < N) c[row0 + idx] = silu_mul(tot, up);
    }
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

// ---------------------------------------------------------------------------
// MFMA GEMM: M > 4
// ---------------------------------------------------------------------------
// LDS tiles hold rows of BK bf16 (CPR = BK/8 chunks of 16 bytes).  Chunk c of
// row r lives at chunk slot c ^ f(r).  f makes the 16-byte fragment reads of
// 16 consecutive rows at one chunk hit distinct banks for 64 four-byte banks
// (16 lanes/pass) and for 32 banks (8 lanes/pass).
template <int CPR>
__device__ __forceinline__ int lds_slot(int row, int ch) {
    if constexpr (CPR == 16) return row * 16 + (ch ^ (row & 15));
    else return row * 8 + (ch ^ ((row ^ (row >> 3)) & 7));
}

template <int BM, int BN, int BK, int WM, int WN, bool GATED, bool VEC>
struct GemmCfg {
    static constexpr int CPR = BK / 8;                 // 16-byte chunks per row
    static constexpr int A_TOTAL = BM * CPR, B_TOTAL = BN * CPR;
    static constexpr int A_CHUNKS = (A_TOTAL + NTHREADS - 1) / NTHREADS;
    static constexpr int B_CHUNKS = (B_TOTAL + NTHREADS - 1) / NTHREADS;
    static constexpr int WTM = BM / WM, WTN = BN / WN;  // wave tile
    static constexpr int TM = WTM / 16, TN = WTN / 16;  // MFMA tiles per wave
    static constexpr int BNO = GATED ? BN / 2 : BN;     // output columns per block
    static_assert(WM * WN == 4, "4 waves");
    static_assert(A_TOTAL % NTHREADS == 0 || A_TOTAL < NTHREADS, "chunk split");
    static_assert(B_TOTAL % NTHREADS == 0 || B_TOTAL < NTHREADS, "chunk split");
    static_assert(TM >= 1 && TN >= 1, "wave tile");
    static_assert(!GATED || (TN % 2 == 0), "gated needs paired column tiles");
};

// Gated column mapping: the wave's TN column tiles are TN/2 gate tiles and
// the TN/2 up tiles of the same output columns.  B-tile rows [0, BN/2) hold
// Wg rows, [BN/2, BN) hold Wu rows.
template <int BN, int WN, int TN, bool GATED>
__device__ __forceinline__ int b_tile_row(int wn, int j) {
    if constexpr (!GATED) {
        return wn * (BN / WN) + 16 * j;
    } else {
        constexpr int BNO = BN / 2, TNO = TN / 2;
        const int base = wn * (BNO / WN);
        return (j < TNO) ? base + 16 * j : BNO + base + 16 * (j - TNO);
    }
}

template <int BM, int BN, int BK, int WM, int WN, bool GATED, bool VEC>
__global__ __launch_bounds__(NTHREADS, 2) void k_gemm(float *__restrict__ c,
                                                     const float *__restrict__ a,
                                                     const uint16_t *__restrict__ b,
                                                     const uint16_t *__restrict__ b2,
                                                     int M, int K, int N) {
    using C = GemmCfg<BM, BN, BK, WM, WN, GATED, VEC>;
    __shared__ u32x4 sA[2][BM * C::CPR];
    __shared__ u32x4 sB[2][BN * C::CPR];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = wave / WN, wn = wave % WN;
    const int m0 = blockIdx.y * BM;
    const int n0 = blockIdx.x * C::BNO;

    // ---- global -> register staging ----
    float ra[C::A_CHUNKS][8];
    u32x4 rb[C::B_CHUNKS];

    auto load_a = [&](int k0) {
#pragma unroll
        for (int i = 0; i < C::A_CHUNKS; i++) {
            const int q = tid + NTHREADS * i;
            if (C::A_TOTAL < NTHREADS && q >= C::A_TOTAL) break;
            const int row = q / C::CPR, ch = q % C::CPR;
            const int gm = m0 + row, gk = k0 + ch * 8;
            if constexpr (VEC) {
                if (gm < M && gk < K) {
                    const f32x4 *p = reinterpret_cast<const f32x4 *>(a + (size_t)gm * K + gk);
                    const f32x4 x0 = p[0], x1 = p[1];
                    ra[i][0] = x0.x; ra[i][1] = x0.y; ra[i][2] = x0.z; ra[i][3] = x0.w;
                    ra[i][4] = x1.x; ra[i][5] = x1.y; ra[i][6] = x1.z; ra[i][7] = x1.w;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; e++) ra[i][e] = 0.0f;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++)
                    ra[i][e] = (gm < M && gk + e < K) ? a[(size_t)gm * K + gk + e] : 0.0f;
            }
        }
    };
    auto load_b = [&](int k0) {
#pragma unroll
        for (int i = 0; i < C::B_CHUNKS; i++) {
            const int q = tid + NTHREADS * i;
            if (C::B_TOTAL < NTHREADS && q >= C::B_TOTAL) break;
            const int row = q / C::CPR, ch = q % C::CPR;
            const uint16_t *src;
            int gn;
            if constexpr (GATED) {
                const bool up = row >= C::BNO;
                gn = n0 + (up ? row - C::BNO : row);
                src = up ? b2 : b;
            } else {
                gn = n0 + row;
                src = b;
            }
            const int gk = k0 + ch * 8;
            if constexpr (VEC) {
                if (gn < N && gk < K)
                    rb[i] = *reinterpret_cast<const u32x4 *>(src + (size_t)gn * K + gk);
                else
                    rb[i] = u32x4{0u, 0u, 0u, 0u};
            } else {
                uint32_t w[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    uint32_t lo = (gn < N && gk + 2 * e < K) ? src[(size_t)gn * K + gk + 2 * e] : 0u;
                    uint32_t hi = (gn < N && gk + 2 * e + 1 < K) ? src[(size_t)gn * K + gk + 2 * e + 1] : 0u;
                    w[e] = lo | (hi << 16);
                }
                rb[i] = u32x4{w[0], w[1], w[2], w[3]};
            }
        }
    };
    auto store_tiles = [&](int buf) {
#pragma unroll
        for (int i = 0; i < C::A_CHUNKS; i++) {
            const int q = tid + NTHREADS * i;
            if (C::A_TOTAL < NTHREADS && q >= C::A_TOTAL) break;
            const int row = q / C::CPR, ch = q % C::CPR;
            u32x4 w;
            w.x = pack_bf16x2(ra[i][0], ra[i][1]);
            w.y = pack_bf16x2(ra[i][2], ra[i][3]);
            w.z = pack_bf16x2(ra[i][4], ra[i][5]);
            w.w = pack_bf16x2(ra[i][6], ra[i][7]);
            sA[buf][lds_slot<C::CPR>(row, ch)] = w;
        }
#pragma unroll
        for (int i = 0; i < C::B_CHUNKS; i++) {
            const int q = tid + NTHREADS * i;
            if (C::B_TOTAL < NTHREADS && q >= C::B_TOTAL) break;
            const int row = q / C::CPR, ch = q % C::CPR;
            sB[buf][lds_slot<C::CPR>(row, ch)] = rb[i];
        }
    };

    f32x4 acc[C::TM][C::TN];
#pragma unroll
    for (int i = 0; i < C::TM; i++)
#pragma unroll
        for (int j = 0; j < C::TN; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nk = (K + BK - 1) / BK;
    load_a(0);
    load_b(0);
    store_tiles(0);
    __syncthreads();

    const int lrow = lane & 15, lgrp = lane >> 4;
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) {
            load_a((kt + 1) * BK);
            load_b((kt + 1) * BK);
        }
#pragma unroll
        for (int s = 0; s < BK / 32; s++) {
            const int ch = 4 * s + lgrp;
            bf16x8 af[C::TM], bfr[C::TN];
#pragma unroll
            for (int i = 0; i < C::TM; i++) {
                const int row = wm * C::WTM + 16 * i + lrow;
                af[i] = __builtin_bit_cast(bf16x8, sA[cur][lds_slot<C::CPR>(row, ch)]);
            }
#pragma unroll
            for (int j = 0; j < C::TN; j++) {
                const int row = b_tile_row<BN, WN, C::TN, GATED>(wn, j) + lrow;
                bfr[j] = __builtin_bit_cast(bf16x8, sB[cur][lds_slot<C::CPR>(row, ch)]);
            }
#pragma unroll
            for (int i = 0; i < C::TM; i++)
#pragma unroll
                for (int j = 0; j < C::TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) store_tiles(cur ^ 1);
        __syncthreads();
    }

    // ---- epilogue: lane holds rows 4*(lane>>4)+r, column lane&15 of each tile
#pragma unroll
    for (int i = 0; i < C::TM; i++) {
        const int rbase = m0 + wm * C::WTM + 16 * i + 4 * lgrp;
        if constexpr (!GATED) {
#pragma unroll
            for (int j = 0; j < C::TN; j++) {
                const int col = n0 + wn * C::WTN + 16 * j + lrow;
                if (col < N) {
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int row = rbase + r;
                        if (row < M) c[(size_t)row * N + col] = acc[i][j][r];
                    }
                }
            }
        } else {
            constexpr int TNO = C::TN / 2;
#pragma unroll
            for (int j = 0; j < TNO; j++) {
                const int col = n0 + wn * (C::BNO / WN) + 16 * j + lrow;
                if (col < N) {
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int row = rbase + r;
                        if (row < M) c[(size_t)row * N + col] = silu_mul(acc[i][j][r], acc[i][j + TNO][r]);
                    }
                }
            }
        }
    }
}

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

__global__ __launch_bounds__(NTHREADS) void k_fill_zero(float *__restrict__ c, size_t n) {
    for (size_t i = (size_t)blockIdx.x * NTHREADS + threadIdx.x; i < n;
         i += (size_t)gridDim.x * NTHREADS)
        c[i] = 0.0f;
}

// ---------------------------------------------------------------------------
// host side of the shim
// ---------------------------------------------------------------------------
static int g_inited = 0;
static int g_device = -1;
static hipStream_t g_stream = nullptr;
static hipError_t g_last_hip = hipSuccess;
static char g_devname[256];
static hipEvent_t g_ev[64];
static int g_ev_made[64];
static int g_forced_plan = 0;
#define QH_MAX_GRAPHS 16
static hipGraphExec_t g_graph_exec[QH_MAX_GRAPHS];
static int g_capturing = 0;
static float *g_am_v = nullptr;   // argmax partials (allocated at init)
static int *g_am_i = nullptr;
static const int AM_BLOCKS = 1024;

static int fail(hipError_t e, int code) {
    g_last_hip = e;
    (void)hipGetLastError();
    return code;
}
#define HCHECK(expr, code)                       \
    do {                                         \
        hipError_t _e = (expr);                  \
        if (_e != hipSuccess) return fail(_e, code); \
    } while (0)

extern "C" int qh_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

extern "C" int qh_init(int device) {
    if (g_inited) return (device < 0 || device == g_device) ? QH_OK : QH_ESTATE;
    int n = 0;
    HCHECK(hipGetDeviceCount(&n), QH_ENODEV);
    if (n <= 0) return QH_ENODEV;
    if (device < 0) device = 0;
    if (device >= n) return QH_EINVAL;
    HCHECK(hipSetDevice(device), QH_ENODEV);
    hipDeviceProp_t prop;
    HCHECK(hipGetDeviceProperties(&prop, device), QH_ENODEV);
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        g_last_hip = hipErrorInvalidDeviceFunction;
        return QH_ENODEV;             // the code objects are built for gfx950 only
    }
    strncpy(g_devname, prop.gcnArchName, sizeof g_devname - 1);
    HCHECK(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking), QH_ERUNTIME);
    HCHECK(hipMalloc((void **)&g_am_v, AM_BLOCKS * sizeof(float)), QH_ENOMEM);
    HCHECK(hipMalloc((void **)&g_am_i, AM_BLOCKS * sizeof(int)), QH_ENOMEM);
    g_device = device;
    g_inited = 1;
    return QH_OK;
}

extern "C" void qh_shutdown(void) {
    if (!g_inited) return;
    (void)hipStreamSynchronize(g_stream);
    for (int i = 0; i < QH_MAX_GRAPHS; i++)
        if (g_graph_exec[i]) { (void)hipGraphExecDestroy(g_graph_exec[i]); g_graph_exec[i] = nullptr; }
    for (int i = 0; i < 64; i++)
        if (g_ev_made[i]) { (void)hipEventDestroy(g_ev[i]); g_ev_made[i] = 0; }
    (void)hipFree(g_am_v);
    (void)hipFree(g_am_i);
    g_am_v = nullptr;
    g_am_i = nullptr;
    (void)hipStreamDestroy(g_stream);
    g_stream = nullptr;
    g_inited = 0;
    g_device = -1;
}

extern "C" int qh_device(void) { return g_device; }
extern "C" const char *qh_device_name(void) { return g_inited ? g_devname : ""; }
extern "C" int qh_last_hip_error(void) { return (int)g_last_hip; }
extern "C" const char *qh_last_hip_error_string(void) { return hipGetErrorString(g_last_hip); }
extern "C" void *qh_stream(void) { return (void *)g_stream; }

extern "C" int qh_malloc(void **p, size_t bytes) {
    if (!g_inited) return QH_ESTATE;
    if (!p) return QH_EINVAL;
    *p = nullptr;
    if (bytes == 0) bytes = 256;
    HCHECK(hipMalloc(p, bytes), QH_ENOMEM);
    return QH_OK;
}
extern "C" int qh_free(void *p) {
    if (!p) return QH_OK;
    HCHECK(hipFree(p), QH_ERUNTIME);
    return QH_OK;
}
extern "C" int qh_host_alloc(void **p, size_t bytes) {
    if (!g_inited) return QH_ESTATE;
    if (!p) return QH_EINVAL;
    *p = nullptr;
    if (bytes == 0) bytes = 256;
    HCHECK(hipHostMalloc(p, bytes, hipHostMallocDefault), QH_ENOMEM);
    return QH_OK;
}
extern "C" int qh_host_free(void *p) {
    if (!p) return QH_OK;
    HCHECK(hipHostFree(p), QH_ERUNTIME);
    return QH_OK;
}
extern "C" int qh_h2d(void *dst, const void *src, size_t bytes) {
    if (!g_inited) return QH_ESTATE;
    if (bytes == 0) return QH_OK;
    HCHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream), QH_ERUNTIME);
    return QH_OK;
}
extern "C" int qh_d2h(void *dst, const void *src, size_t bytes) {
    if (!g_inited) return QH_ESTATE;
    if (bytes == 0) return QH_OK;
    HCHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream), QH_ERUNTIME);
    return QH_OK;
}
extern "C" int qh_d2d(void *dst, const void *src, size_t bytes) {
    if (!g_inited) return QH_ESTATE;
    if (bytes == 0) return QH_OK;
    HCHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_stream), QH_ERUNTIME);
    return QH_OK;
}
extern "C" int qh_sync(void) {
    if (!g_inited) return QH_ESTATE;
    HCHECK(hipStreamSynchronize(g_stream), QH_ERUNTIME);
    return QH_OK;
}

extern "C" int qh_timer_record(int slot) {
    if (!g_inited) return QH_ESTATE;
    if (slot < 0 || slot >= 64) return QH_EINVAL;
    if (!g_ev_made[slot]) {
        HCHECK(hipEventCreate(&g_ev[slot]), QH_ERUNTIME);
        g_ev_made[slot] = 1;
    }
    HCHECK(hipEventRecord(g_ev[slot], g_stream), QH_ERUNTIME);
    return QH_OK;
}
extern "C" int qh_timer_elapsed_ms(int a, int b, float *ms) {
    if (!g_inited) return QH_ESTATE;
    if (a < 0 || a >= 64 || b < 0 || b >= 64 || !g_ev_made[a] || !g_ev_made[b] || !ms) return QH_EINVAL;
    HCHECK(hipEventSynchronize(g_ev[b]), QH_ERUNTIME);
    HCHECK(hipEventElapsedTime(ms, g_ev[a], g_ev[b]), QH_ERUNTIME);
    return QH_OK;
}

// ---- plans ------------------------------------------------------------------
enum {
    PLAN_AUTO = 0,
    PLAN_GEMV = 1,
    PLAN_T128x128 = 2,
    PLAN_T64x128 = 3,
    PLAN_T64x64 = 4,
    PLAN_T32x128 = 5,
    PLAN_T16x64 = 6,
    PLAN_SCALAR64 = 7,     // MFMA 64x64 with element-wise loads (any K, any alignment)
    PLAN_COUNT = 8
};
static const char *k_plan_names[PLAN_COUNT] = {
    "auto", "gemv", "mfma128x128", "mfma64x128", "mfma64x64", "mfma32x128", "mfma16x64", "mfma64x64-scalar"};

static inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

static int choose_plan(int M, int K, int N, int gated, bool vec) {
    if (!vec) return PLAN_SCALAR64;
    if (M <= 4 && (size_t)M * K * 4 <= 64 * 1024) return PLAN_GEMV;
    const int bno = gated ? 2 : 1;   // gated tiles produce half as many output columns
    auto blocks = [&](int bm, int bn) {
        return (long)((M + bm - 1) / bm) * (long)((N + bn / bno - 1) / (bn / bno));
    };
    if (M <= 16) return PLAN_T16x64;
    if (M <= 32) return PLAN_T32x128;
    if (M <= 64) return (blocks(64, 128) >= 256) ? PLAN_T64x128 : PLAN_T64x64;
    if (blocks(128, 128) >= 256) return PLAN_T128x128;
    if (blocks(64, 128) >= 256) return PLAN_T64x128;
    return PLAN_T64x64;
}

extern "C" const char *qh_gemm_plan(int M, int K, int N, int gated) {
    int p = g_forced_plan ? g_forced_plan : choose_plan(M, K, N, gated, (K % 8) == 0);
    return k_plan_names[p];
}

extern "C" int qh_force_plan(int plan_id) {
    if (plan_id < 0 || plan_id >= PLAN_COUNT) return QH_EINVAL;
    g_forced_plan = plan_id;
    return QH_OK;
}

template <int ROWS, bool GATED>
static int launch_gemv1_rows(float *c, const float *a, const uint16_t *b, const uint16_t *b2,
                             int K, int N, int cpl) {
    const int grid = (N + (NTHREADS / WAVE) * ROWS - 1) / ((NTHREADS / WAVE) * ROWS);
    // only the (ROWS, CPL) pairs launch_gemv1 can pick: <= 16 loads per lane
#define QH_GEMV1_CASE(P)                                                                     \
    case P:                                                                                  \
        if constexpr (ROWS == 1 || ROWS * P * (GATED ? 2 : 1) <= 16)                         \
            hipLaunchKernelGGL((k_gemv1<ROWS, P, GATED>), dim3(grid), dim3(NTHREADS), 0,     \
                               g_stream, c, a, b, b2, K, N);                                 \
        else                                                                                 \
            return QH_EINVAL;                                                                \
        break;
    switch (cpl) {
        QH_GEMV1_CASE(1)
        QH_GEMV1_CASE(2)
        QH_GEMV1_CASE(3)
        QH_GEMV1_CASE(4)
        QH_GEMV1_CASE(5)
        QH_GEMV1_CASE(6)
        QH_GEMV1_CASE(7)
        QH_GEMV1_CASE(8)
        default: return QH_EINVAL;
    }
#undef QH_GEMV1_CASE
    HCHECK(hipGetLastError(), QH_ELAUNCH);
    return QH_OK;
}

// M = 1 with K <= 4096.  Rows per wave: as many as keep >= 2048 waves in the
// grid (8 per CU) and <= 16 weight loads of 16 B in flight per lane.
static int launch_gemv1(float *c, const float *a, const uint16_t *b, const uint16_t *b2,
                        int K, int N, bool gated) {
    const int cpl = (K / 8 + WAVE - 1) / WAVE;
    const int per_row = gated ? 2 * cpl : cpl;
    int rows = 8;
    while (rows > 1 && (long)(N + rows - 1) / rows < 2048) rows /= 2;
    while (rows > 1 && rows * per_row > 16) rows /= 2;
    if (gated && rows > 4) rows = 4;
    switch (rows) {
        case 1: return gated ? launch_gemv1_rows<1, true>(c, a, b, b2, K, N, cpl)
                             : launch_gemv1_rows<1, false>(c, a, b, b2, K, N, cpl);
        case 2: return gated ? launch_gemv1_rows<2, true>(c, a, b, b2, K, N, cpl)
                             : launch_gemv1_rows<2, false>(c, a, b, b2, K, N, cpl);
        case 4: return gated ? launch_gemv1_rows<4, true>(c, a, b, b2, K, N, cpl)
                             : launch_gemv1_rows<4, false>(c, a, b, b2, K, N, cpl);
        case 8: return launch_gemv1_rows<8, false>(c, a, b, b2, K, N, cpl);
        default: return QH_EINVAL;
    }
}

template <int MR>
static int launch_gemv_mr(float *c, const float *a, const uint16_t *b, const uint16_t *b2,
                          int K, int N, bool gated) {
    if (MR == 1 && K <= 8 * WAVE * 8) return launch_gemv1(c, a, b, b2, K, N, gated);
    const size_t lds = (size_t)MR * K * sizeof(float);
    // rows per wave: enough waves to cover the GPU for small N, and up to 8
    // rows (16 loads of 16 B in flight per lane at K = 1024) for large N
    const int cpl = (K / 8 + WAVE - 1) / WAVE;       // chunks per lane
    int rows = 8;
    while (rows > 1 && (long)(N + rows - 1) / rows < 2048) rows /= 2;
    while (rows > 1 && rows * cpl > 16) rows /= 2;
    if (gated && rows > 4) rows = 4;
    const int grid = (N + 4 * rows - 1) / (4 * rows);
#define QH_GEMV_CASE(R)                                                                      \
    case R:                                                                                  \
        hipLaunchKernelGGL((k_gemv<MR, R, 2>), dim3(grid), dim3(NTHREADS), lds, g_stream,     \
                           c, a, b, K, N);                                                   \
        break;
#define QH_GEMV_GATED_CASE(R)                                                                \
    case R:                                                                                  \
        hipLaunchKernelGGL((k_gemv_gated<MR, R, 2>), dim3(grid), dim3(NTHREADS), lds,         \
                           g_stream, c, a, b, b2, K, N);                                     \
        break;
    if (gated) {
        switch (rows) {
            QH_GEMV_GATED_CASE(1)
            QH_GEMV_GATED_CASE(2)
            QH_GEMV_GATED_CASE(4)
            default: return QH_EINVAL;
        }
    } else {
        switch (rows) {
            QH_GEMV_CASE(1)
            QH_GEMV_CASE(2)
            QH_GEMV_CASE(4)
            QH_GEMV_CASE(8)
            default: return QH_EINVAL;
        }
    }
#undef QH_GEMV_CASE
#undef QH_GEMV_GATED_CASE
    HCHECK(hipGetLastError(), QH_ELAUNCH);
    return QH_OK;
}

template <int BM, int BN, int BK, int WM, int WN, bool GATED, bool VEC>
static int launch_tile(float *c, const float *a, const uint16_t *b, const uint16_t *b2,
                       int M, int K, int N) {
    constexpr int BNO = GATED ? BN / 2 : BN;
    const dim3 grid((N + BNO - 1) / BNO, (M + BM - 1) / BM);
    if (grid.y > 65535u) return QH_ETOOBIG;
    hipLaunchKernelGGL((k_gemm<BM, BN, BK, WM, WN, GATED, VEC>), grid, dim3(NTHREADS), 0,
                       g_stream, c, a, b, b2, M, K, N);
    HCHECK(hipGetLastError(), QH_ELAUNCH);
    return QH_OK;
}

template <bool GATED>
static int dispatch(int plan, float *c, const float *a, const uint16_t *b, const uint16_t *b2,
                    int M, int K, int N) {
    switch (plan) {
        case PLAN_GEMV:
            switch (M) {
                case 1: return launch_gemv_mr<1>(c, a, b, b2, K, N, GATED);
                case 2: return launch_gemv_mr<2>(c, a, b, b2, K, N, GATED);
                case 3: return launch_gemv_mr<3>(c, a, b, b2, K, N, GATED);
                case 4: return launch_gemv_mr<4>(c, a, b, b2, K, N, GATED);
                default: return QH_EINVAL;
            }
        case PLAN_T128x128: return launch_tile<128, 128, 64, 2, 2, GATED, true>(c, a, b, b2, M, K, N);
        case PLAN_T64x128:  return launch_tile<64, 128, 64, 2, 2, GATED, true>(c, a, b, b2, M, K, N);
        case PLAN_T64x64:   return launch_tile<64, 64, 64, 2, 2, GATED, true>(c, a, b, b2, M, K, N);
        case PLAN_T32x128:  return launch_tile<32, 128, 64, 2, 2, GATED, true>(c, a, b, b2, M, K, N);
        case PLAN_T16x64:   return launch_tile<16, 128, 64, 1, 4, GATED, true>(c, a, b, b2, M, K, N);
        case PLAN_SCALAR64: return launch_tile<64, 64, 64, 2, 2, GATED, false>(c, a, b, b2, M, K, N);
        default: return QH_EINVAL;
    }
}

static int gemm_common(float *c, const float *a, const uint16_t *b, const uint16_t *b2,
                       int M, int K, int N, bool gated) {
    if (!g_inited) return QH_ESTATE;
    if (M < 0 || K < 0 || N < 0) return QH_EINVAL;
    if (M == 0 || N == 0) return QH_OK;
    if (!c || !b || !a || (gated && !b2)) return QH_EINVAL;
    if (K == 0) {   // empty sum: the reference writes 0.0f (and silu(0)*0 = 0)
        // a kernel, not hipMemsetAsync: this may be recorded into a graph
        const size_t n = (size_t)M * N;
        const size_t want = (n + NTHREADS - 1) / NTHREADS;
        hipLaunchKernelGGL(k_fill_zero, dim3((unsigned)(want < 4096 ? want : 4096)), dim3(NTHREADS), 0,
                           g_stream, c, n);
        HCHECK(hipGetLastError(), QH_ELAUNCH);
        return QH_OK;
    }
    const bool vec = (K % 8) == 0 && aligned16(a) && aligned16(b) && (!gated || aligned16(b2));
    int plan = g_forced_plan ? g_forced_plan : choose_plan(M, K, N, gated, vec);
    if (!vec) plan = PLAN_SCALAR64;   // forced plans still need vector-safe inputs
    if (plan == PLAN_GEMV && (M > 4 || (size_t)M * K * 4 > 64 * 1024)) plan = PLAN_T64x64;
    return gated ? dispatch<true>(plan, c, a, b, b2, M, K, N)
                 : dispatch<false>(plan, c, a, b, nullptr, M, K, N);
}

extern "C" int qh_gemm(float *c, const float *a, const uint16_t *b, int M, int K, int N) {
    return gemm_common(c, a, b, nullptr, M, K, N, false);
}

extern "C" int qh_gemm_gate_up_silu(float *h, const float *x, const uint16_t *wg,
                                    const uint16_t *wu, int M, int K, int N) {
    return gemm_common(h, x, wg, wu, M, K, N, true);
}

extern "C" int qh_tile_to_row(uint16_t *dst, const uint16_t *src, int N, int K, int tn, int tk) {
    if (!g_inited) return QH_ESTATE;
    if (N <= 0 || K <= 0 || tn <= 0 || tk <= 0 || !dst || !src) return QH_EINVAL;
    if (N % tn || K % tk) return QH_ELAYOUT;
    const size_t total = (size_t)N * K;
    const int grid = (int)((total + NTHREADS - 1) / NTHREADS < 8192 ? (total + NTHREADS - 1) / NTHREADS : 8192);
    hipLaunchKernelGGL(k_tile_to_row, dim3(grid), dim3(NTHREADS), 0, g_stream, dst, src, N, K, tn, tk);
    HCHECK(hipGetLastError(), QH_ELAUNCH);
    return QH_OK;
}

// ---- stream capture into HIP graphs ------------------------------------------

extern "C" int qh_capture_begin(void) {
    if (!g_inited) return QH_ESTATE;
    if (g_capturing) return QH_ESTATE;
    HCHECK(hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal), QH_ERUNTIME);
    g_capturing = 1;
    return QH_OK;
}

extern "C" int qh_capture_end(int *graph_id) {
    if (!g_inited || !g_capturing) return QH_ESTATE;
    g_capturing = 0;
    hipGraph_t graph = nullptr;
    HCHECK(hipStreamEndCapture(g_stream, &graph), QH_ERUNTIME);
    int slot = -1;
    for (int i = 0; i < QH_MAX_GRAPHS; i++)
        if (!g_graph_exec[i]) { slot = i; break; }
    if (slot < 0) {
        (void)hipGraphDestroy(graph);
        return QH_ETOOBIG;
    }
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return fail(e, QH_ERUNTIME);
    g_graph_exec[slot] = exec;
    if (graph_id) *graph_id = slot;
    return QH_OK;
}

extern "C" int qh_graph_launch(int id) {
    if (!g_inited) return QH_ESTATE;
    if (id < 0 || id >= QH_MAX_GRAPHS || !g_graph_exec[id]) return QH_EINVAL;
    HCHECK(hipGraphLaunch(g_graph_exec[id], g_stream), QH_ERUNTIME);
    return QH_OK;
}

extern "C" int qh_graph_destroy(int id) {
    if (id < 0 || id >= QH_MAX_GRAPHS || !g_graph_exec[id]) return QH_EINVAL;
    HCHECK(hipGraphExecDestroy(g_graph_exec[id]), QH_ERUNTIME);
    g_graph_exec[id] = nullptr;
    return QH_OK;
}

extern "C" int qh_copy(void *dst, const void *src, size_t bytes) {
    if (!g_inited) return QH_ESTATE;
    if (!dst || !src || (bytes & 15u) || !aligned16(dst) || !aligned16(src)) return QH_EINVAL;
    if (bytes == 0) return QH_OK;
    const size_t n16 = bytes / 16;
    const size_t want = (n16 + NTHREADS - 1) / NTHREADS;
    const int grid = (int)(want < 4096 ? want : 4096);
    hipLaunchKernelGGL(k_copy16, dim3(grid), dim3(NTHREADS), 0, g_stream, (u32x4 *)dst,
                       (const u32x4 *)src, n16);
    HCHECK(hipGetLastError(), QH_ELAUNCH);
    return QH_OK;
}

extern "C" int qh_argmax(int *out, const float *v, int n) {
    if (!g_inited) return QH_ESTATE;
    if (n <= 0 || !out || !v) return QH_EINVAL;
    int blocks = (n + NTHREADS * 4 - 1) / (NTHREADS * 4);
    if (blocks > AM_BLOCKS) blocks = AM_BLOCKS;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(k_argmax_partial, dim3(blocks), dim3(NTHREADS), 0, g_stream, g_am_v, g_am_i, v, n);
    HCHECK(hipGetLastError(), QH_ELAUNCH);
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(WAVE), 0, g_stream, out, g_am_v, g_am_i, blocks, v);
    HCHECK(hipGetLastError(), QH_ELAUNCH);
    return QH_OK;
}
