// Tiled MFMA GEMM kernels for M > 4: the 64 x 64 - 128 x 128 double-buffered
// tiles, the LDS ring fed by global_load_lds (software-pipelined, k groups)
// and the large 64 x 64 - 256 x 256 tiles with two stages in flight.
// Included by hip_gemm.hip, whose host code launches them.
#ifndef QH_TILE_KERNELS_H
#define QH_TILE_KERNELS_H

#include "gemm_common.h"

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

// Output-tile order for a 1-D grid.  Workgroups are handed to the 8 XCDs
// round-robin (workgroup b runs on XCD b % 8) and each XCD has its own L2, so
// the MT x NT tile grid is cut into rm x rn = 8 regions, one per XCD, and the
// workgroups of an XCD walk their region m-major (consecutive ones share an A
// panel).  Each XCD then pulls only its A and B slabs into its L2.  rm == 0
// means plain row-major order (used when the grid does not split evenly).
struct TileMap {
    int MT, NT, rm, rn;
};

__device__ __forceinline__ void tile_of(int bid, const TileMap &map, int &tm, int &tn) {
    if (map.rm == 0) {
        tm = bid / map.NT;
        tn = bid % map.NT;
        return;
    }
    const int xcd = bid & 7, local = bid >> 3;
    const int rmt = map.MT / map.rm, rnt = map.NT / map.rn;    // tiles per region
    tm = (xcd / map.rn) * rmt + local / rnt;
    tn = (xcd % map.rn) * rnt + local % rnt;
}

template <int BM, int BN, int BK, int WM, int WN, bool GATED, bool VEC>
__global__ __launch_bounds__(NTHREADS, 2) void k_gemm(float *__restrict__ c,
                                                     const float *__restrict__ a,
                                                     const uint16_t *__restrict__ b,
                                                     const uint16_t *__restrict__ b2,
                                                     int M, int K, int N, TileMap map) {
    using C = GemmCfg<BM, BN, BK, WM, WN, GATED, VEC>;
    __shared__ u32x4 sA[2][BM * C::CPR];
    __shared__ u32x4 sB[2][BN * C::CPR];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = wave / WN, wn = wave % WN;
    int tm, tn;
    tile_of(blockIdx.x, map, tm, tn);
    const int m0 = tm * BM;
    const int n0 = tn * C::BNO;

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
// Ring-pipelined MFMA GEMM (K % 32 == 0, 16-byte aligned operands)
// ---------------------------------------------------------------------------
// A k-loop that waits for one global round trip per step is latency-bound
// (~0.7 us per step on MI355X).  Here every 32-wide k step of the A tile
// (fp32) and B tile (bf16) is copied straight from global memory into a ring
// of STAGES LDS slots by global_load_lds_dwordx4 (no registers involved), and
// STAGES-1 steps are always in flight.  Per step each wave waits only for its
// own oldest copies (s_waitcnt vmcnt), one barrier publishes the slot and
// frees the previous one, the next copy is issued, then MFMAs run on the
// slot; A is converted to bf16 (RNE) as its fragments are read.
//
// LDS slot layout (one step): A rows of 32 fp32 (128 B = 8 chunks of 16 B),
// then B rows of 32 bf16 (64 B = 4 chunks).  Chunk c of row r sits at
// c ^ swzA(r) / c ^ swzB(r); both swizzles keep 16 consecutive rows at one
// logical chunk on distinct banks (checked for 8- and 16-lane LDS passes).
// A wave's LDS copy always fills 1 KB contiguously (lane i -> bytes 16i..),
// so each lane picks the global chunk that belongs at its LDS position.
// Swizzle for rows of CH 16-byte chunks (64, 128, 256 or 512 bytes).
template <int CH>
__device__ __forceinline__ int swz(int r) {
    if constexpr (CH == 4) return ((r >> 1) ^ (r >> 3)) & 3;
    else if constexpr (CH == 8) return (r ^ (r >> 3)) & 7;
    else return r & 15;                       // 16 or 32 chunks
}

// s_waitcnt immediate for "at most n vector-memory ops outstanding" (gfx9
// encoding: vmcnt bits [3:0] and [15:14]; expcnt and lgkmcnt left at max)
#define QH_VMCNT(n) ((((n) & 15) | (((n) >> 4) << 14)) | (7 << 4) | (15 << 8))

template <int BM, int BN, int WM, int WN, int STAGES, bool GATED, int BK_ = 32, int KG = 1>
struct RingCfg {
    static constexpr int BK = BK_;                      // k per stage (32, 64, 128)
    static constexpr int KS = BK / 32;                  // MFMA k-steps per stage
    static constexpr int KSG = KS / KG;                 // ... per wave group
    static constexpr int CA = BK / 4, CB = BK / 8;      // 16-byte chunks per A / B row
    static constexpr int A_BYTES = BM * BK * 4, B_BYTES = BN * BK * 2;
    static constexpr int STAGE = A_BYTES + B_BYTES;
    static constexpr int NW = WM * WN * KG;             // waves: KG groups of WM x WN
    static constexpr int A_DMA = A_BYTES / 1024 / NW;  // 1 KB copies per wave per step
    static constexpr int B_DMA = B_BYTES / 1024 / NW;
    static constexpr int LPS = A_DMA + B_DMA;           // copies per wave per step
    static constexpr int WTM = BM / WM, WTN = BN / WN;
    static constexpr int TM = WTM / 16, TN = WTN / 16;
    static constexpr int BNO = GATED ? BN / 2 : BN;
    static constexpr int LDS = STAGES * STAGE;
    static constexpr int vm(int k) { return k * LPS > 63 ? 63 : k * LPS; }
    static_assert(NW == 4 || NW == 8 || NW == 16, "4, 8 or 16 waves");
    static_assert((KG == 1 || KG == 2 || KG == 4) && KSG * KG == KS, "wave groups split a stage's k-steps");
    static_assert(A_DMA * NW * 1024 == A_BYTES && B_DMA * NW * 1024 == B_BYTES, "every wave issues the same number of copies");
    static_assert(A_DMA >= 1 && B_DMA >= 1, "copies per wave");
    static_assert(TM >= 1 && TN >= 1 && (!GATED || TN % 2 == 0), "wave tile");
    static_assert(STAGES >= 2 && (STAGES - 2) * LPS <= 63, "vmcnt range");
};

// ---------------------------------------------------------------------------
// Software-pipelined ring GEMM
// ---------------------------------------------------------------------------
template <int V> struct IC { static constexpr int value = V; };

// A and B stream straight into an LDS ring of STAGES slots with
// global_load_lds (16-byte copies, explicit vmcnt waits, one barrier per
// stage), and the phases of consecutive stages overlap inside each wave: while the MFMAs of stage `it` run on
// fragments already in registers, the LDS reads of stage it+1 fill a second
// register set and the copies of stage it+STAGES-1 are in flight.  Per stage:
//   wait (own copies of it+1) -> barrier -> issue copies of it+STAGES-1 ->
//   read fragments of it+1 -> MFMAs of it.
// The copy into slot (it-1) % STAGES is safe after the barrier: every wave
// consumed stage it-1 (its MFMAs ran) before reaching it.  LDS destinations
// of the copies are wave-uniform and computed from a scalar wave index.
// KG groups of WM x WN waves: with KG = 2 or 4 (the 32 x 64 tiles with
// 128-deep stages, one block per CU) the groups split each stage's k-steps
// and the others add their sums into the first group's through LDS at the
// end, in group order, so that two or four waves share each SIMD (measured
// on MI355X, graph-replayed, against one group of 2 x 2: 512 x {1024, 2048,
// 3072} x 1024 6.9 / 10.9 / 15.0 -> 6.4 / 9.65 / 12.8 us with two groups,
// 128 x 1024 x 4096 6.7 -> 6.2, gate|up + SiLU 64 x 1024 x 3072 6.74 ->
// 6.27; four groups from K = 2048: 512 x {2048, 3072} x 1024 9.5 / 12.7 ->
// 9.1 / 12.2, but at K = 1024 they lose, 6.24 -> 6.35; 2 x 4 waves on the
// plain tiles instead reached 6.75 / 10.6 / 14.5).
template <int BM, int BN, int WM, int WN, int STAGES, bool GATED, int BK_, int KG>
__global__ __launch_bounds__(64 * WM * WN * KG, 1) void k_gemm_pipe(float *__restrict__ c,
                                                          const float *__restrict__ a,
                                                          const uint16_t *__restrict__ b,
                                                          const uint16_t *__restrict__ b2,
                                                          int M, int K, int N, TileMap map) {
    using R = RingCfg<BM, BN, WM, WN, STAGES, GATED, BK_, KG>;
    static_assert(STAGES >= 3, "one stage being read, one in use, one or more in flight");
    extern __shared__ __align__(16) unsigned char smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);     // scalar
    const int kg = wave / (WM * WN), wq = wave % (WM * WN);   // k group, wave within it
    const int wm = wq / WN, wn = wq % WN;
    int tm, tn;
    tile_of(blockIdx.x, map, tm, tn);
    const int m0 = tm * BM;
    const int n0 = tn * R::BNO;
    const int nk = K / R::BK;

    const float *asrc[R::A_DMA];
    const uint16_t *bsrc[R::B_DMA];
#pragma unroll
    for (int i = 0; i < R::A_DMA; i++) {
        const int seg = wave * R::A_DMA + i;
        const int r = seg * (64 / R::CA) + lane / R::CA;
        const int cl = (lane % R::CA) ^ swz<R::CA>(r);
        const int gm = min(m0 + r, M - 1);
        asrc[i] = a + (size_t)gm * K + cl * 4;
    }
#pragma unroll
    for (int i = 0; i < R::B_DMA; i++) {
        const int seg = wave * R::B_DMA + i;
        const int r = seg * (64 / R::CB) + lane / R::CB;
        const int cl = (lane % R::CB) ^ swz<R::CB>(r);
        const uint16_t *src = b;
        int gn;
        if constexpr (GATED) {
            const bool up = r >= R::BNO;
            gn = n0 + (up ? r - R::BNO : r);
            src = up ? b2 : b;
        } else {
            gn = n0 + r;
        }
        gn = min(gn, N - 1);
        bsrc[i] = src + (size_t)gn * K + cl * 8;
    }
    // wave-uniform LDS byte offsets of this wave's copies within a slot
    const int a_dst = wave * R::A_DMA * 1024;
    const int b_dst = R::A_BYTES + wave * R::B_DMA * 1024;

    auto issue = [&](int step) {
        unsigned char *slot = smem + (step % STAGES) * R::STAGE;
        const int k0 = step * R::BK;
#pragma unroll
        for (int i = 0; i < R::A_DMA; i++)
            __builtin_amdgcn_global_load_lds(
                (const void *)(asrc[i] + k0),
                (__attribute__((address_space(3))) void *)(slot + a_dst + i * 1024), 16, 0, 0);
#pragma unroll
        for (int i = 0; i < R::B_DMA; i++)
            __builtin_amdgcn_global_load_lds(
                (const void *)(bsrc[i] + k0),
                (__attribute__((address_space(3))) void *)(slot + b_dst + i * 1024), 16, 0, 0);
    };

    const int lrow = lane & 15, lgrp = lane >> 4;
    // per-lane LDS offsets of this lane's fragment rows (within a slot)
    int arow_off[R::TM], arow_sw[R::TM], brow_off[R::TN], brow_sw[R::TN];
#pragma unroll
    for (int i = 0; i < R::TM; i++) {
        const int row = wm * R::WTM + 16 * i + lrow;
        arow_off[i] = row * (R::CA * 16);
        arow_sw[i] = swz<R::CA>(row);
    }
#pragma unroll
    for (int j = 0; j < R::TN; j++) {
        const int row = b_tile_row<BN, WN, R::TN, GATED>(wn, j) + lrow;
        brow_off[j] = R::A_BYTES + row * (R::CB * 16);
        brow_sw[j] = swz<R::CB>(row);
    }

    u32x4 fa[2][R::KSG][R::TM][2], fb[2][R::KSG][R::TN];
    // `SET` selects the register set at compile time (IC<0> / IC<1>)
    auto read_frags = [&](int step, auto SET) {
        constexpr int set = decltype(SET)::value;
        const unsigned char *slot = smem + (step % STAGES) * R::STAGE;
#pragma unroll
        for (int tt = 0; tt < R::KSG; tt++) {
            const int t = kg * R::KSG + tt;                   // this group's k-steps
#pragma unroll
            for (int i = 0; i < R::TM; i++) {
                const u32x4 *rowp = reinterpret_cast<const u32x4 *>(slot + arow_off[i]);
                fa[set][tt][i][0] = rowp[(8 * t + 2 * lgrp) ^ arow_sw[i]];
                fa[set][tt][i][1] = rowp[(8 * t + 2 * lgrp + 1) ^ arow_sw[i]];
            }
#pragma unroll
            for (int j = 0; j < R::TN; j++) {
                const u32x4 *rowp = reinterpret_cast<const u32x4 *>(slot + brow_off[j]);
                fb[set][tt][j] = rowp[(4 * t + lgrp) ^ brow_sw[j]];
            }
        }
    };

    f32x4 acc[R::TM][R::TN];
#pragma unroll
    for (int i = 0; i < R::TM; i++)
#pragma unroll
        for (int j = 0; j < R::TN; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto mfmas = [&](auto SET) {
        constexpr int set = decltype(SET)::value;
#pragma unroll
        for (int t = 0; t < R::KSG; t++) {
            bf16x8 af[R::TM];
#pragma unroll
            for (int i = 0; i < R::TM; i++) {
                const f32x4 x0 = __builtin_bit_cast(f32x4, fa[set][t][i][0]);
                const f32x4 x1 = __builtin_bit_cast(f32x4, fa[set][t][i][1]);
                u32x4 w;
                w.x = pack_bf16x2(x0.x, x0.y);
                w.y = pack_bf16x2(x0.z, x0.w);
                w.z = pack_bf16x2(x1.x, x1.y);
                w.w = pack_bf16x2(x1.z, x1.w);
                af[i] = __builtin_bit_cast(bf16x8, w);
            }
#pragma unroll
            for (int i = 0; i < R::TM; i++)
#pragma unroll
                for (int j = 0; j < R::TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        af[i], __builtin_bit_cast(bf16x8, fb[set][t][j]), acc[i][j], 0, 0, 0);
        }
    };

    // prologue: copies of stages 0 .. STAGES-2 in flight; stage 0 read
    const int pro = nk < STAGES - 1 ? nk : STAGES - 1;
    for (int s = 0; s < pro; s++) issue(s);
    {
        const int later = min(nk - 1, STAGES - 2);      // stages issued after stage 0
        switch (later) {
            case 0: __builtin_amdgcn_s_waitcnt(QH_VMCNT(0)); break;
            case 1: __builtin_amdgcn_s_waitcnt(QH_VMCNT(R::vm(1))); break;
            case 2: __builtin_amdgcn_s_waitcnt(QH_VMCNT(R::vm(2))); break;
            case 3: __builtin_amdgcn_s_waitcnt(QH_VMCNT(R::vm(3))); break;
            case 4: __builtin_amdgcn_s_waitcnt(QH_VMCNT(R::vm(4))); break;
            default: __builtin_amdgcn_s_waitcnt(QH_VMCNT(R::vm(5))); break;
        }
        __builtin_amdgcn_s_barrier();
        read_frags(0, IC<0>{});
    }

    // one pipeline step: MFMAs on register set CUR while stage it+1 is read
    // into the other set
    auto step = [&](int it, auto CUR) {
        constexpr int cur = decltype(CUR)::value;
        if (it + 1 < nk) {
            // own copies of stage it+1 landed: stages it+2 .. it+STAGES-2 may
            // still be in flight
            const int later = min(nk - 2 - it, STAGES - 3);
            switch (later) {
                case 0: __builtin_amdgcn_s_waitcnt(QH_VMCNT(0)); break;
                case 1: __builtin_amdgcn_s_waitcnt(QH_VMCNT(R::vm(1))); break;
                case 2: __builtin_amdgcn_s_waitcnt(QH_VMCNT(R::vm(2))); break;
                case 3: __builtin_amdgcn_s_waitcnt(QH_VMCNT(R::vm(3))); break;
                default: __builtin_amdgcn_s_waitcnt(QH_VMCNT(R::vm(4))); break;
            }
            __builtin_amdgcn_s_barrier();
            if (it + STAGES - 1 < nk) issue(it + STAGES - 1);
            read_frags(it + 1, IC<cur ^ 1>{});
        }
        mfmas(CUR);
    };
    // the same step where stage it+1 exists, a copy is due and STAGES-3
    // later stages stay in flight: straight-line code, so that the compiler
    // waits before the MFMAs only for the older fragment set (lgkmcnt of
    // the reads just issued) instead of every LDS read (the branches of
    // `step` leave it with lgkmcnt(0), which serialises the reads of stage
    // it+1 with the MFMAs of stage it)
    auto full_step = [&](int it, auto CUR) {
        constexpr int cur = decltype(CUR)::value;
        __builtin_amdgcn_s_waitcnt(QH_VMCNT(R::vm(STAGES - 3)));
        __builtin_amdgcn_s_barrier();
        issue(it + STAGES - 1);
        read_frags(it + 1, IC<cur ^ 1>{});
        mfmas(CUR);
        __builtin_amdgcn_sched_barrier(0);             // no MFMA moves past the next barrier
    };
    int it = 0;
    for (; it + STAGES < nk; it += 2) {
        full_step(it, IC<0>{});
        full_step(it + 1, IC<1>{});
    }
    for (; it < nk; it += 2) {
        step(it, IC<0>{});
        if (it + 1 < nk) step(it + 1, IC<1>{});
    }

    // two wave groups: the second adds its sums into the first's through LDS
    if constexpr (KG > 1) {
        constexpr int PER_G = WM * WN * R::TM * R::TN * 64;   // f32x4 per group
        f32x4 *xred = reinterpret_cast<f32x4 *>(smem);
        __syncthreads();                                   // every wave is done with the ring
        if (kg > 0) {
#pragma unroll
            for (int i = 0; i < R::TM; i++)
#pragma unroll
                for (int j = 0; j < R::TN; j++)
                    xred[(kg - 1) * PER_G + ((wq * R::TM + i) * R::TN + j) * 64 + lane] = acc[i][j];
        }
        __syncthreads();
        if (kg > 0) return;
#pragma unroll
        for (int q = 1; q < KG; q++)                       // the groups' sums in group order
#pragma unroll
            for (int i = 0; i < R::TM; i++)
#pragma unroll
                for (int j = 0; j < R::TN; j++)
                    acc[i][j] += xred[(q - 1) * PER_G + ((wq * R::TM + i) * R::TN + j) * 64 + lane];
    }

    // epilogue: lane holds rows 4*(lane>>4)+r, column lane&15 of each tile
#pragma unroll
    for (int i = 0; i < R::TM; i++) {
        const int rbase = m0 + wm * R::WTM + 16 * i + 4 * lgrp;
        if constexpr (!GATED) {
#pragma unroll
            for (int j = 0; j < R::TN; j++) {
                const int col = n0 + wn * R::WTN + 16 * j + lrow;
                if (col < N) {
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        if (rbase + r < M) __builtin_nontemporal_store(acc[i][j][r], &c[(size_t)(rbase + r) * N + col]);
                }
            }
        } else {
            constexpr int TNO = R::TN / 2;
#pragma unroll
            for (int j = 0; j < TNO; j++) {
                const int col = n0 + wn * (R::BNO / WN) + 16 * j + lrow;
                if (col < N) {
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        if (rbase + r < M)
                            __builtin_nontemporal_store(silu_mul(acc[i][j][r], acc[i][j + TNO][r]),
                                                        &c[(size_t)(rbase + r) * N + col]);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Large-tile MFMA GEMM: 32x32x16 bf16 MFMA, 2 x 2 waves (2 x 4 on 256 x 256
// tiles), two stages in flight
// ---------------------------------------------------------------------------
// Block tile BM x BN, k stages of BK (32 or 64).  Each wave owns a
// (BM/WMW) x (BN/WNW) tile of TM x TN 32x32 accumulators (fp32, 16 per lane).
// 256 x 256 tiles run eight waves (two per SIMD, 128 x 64 each): with one
// wave per SIMD the MFMA pipe idles whenever that wave waits (measured on
// MI355X, graph-replayed: 4096 x 1024 x 4096 45.2 -> 43.3 us, gated 4096 x
// 1024 x 3072 84.8 -> 72.4 us, 8192 x 1024 x 4096 bf16 A 88.2 -> 83.9 us).
// Operands move global -> registers -> LDS with 16-byte buffer loads (a
// fixed 32-bit offset per lane and load, the stage's k offset in a scalar
// register): A as fp32, rounded to bf16 (RNE) on the way into LDS; B as
// bf16.  Registers hold two stages (two sets), LDS two slots; stage `it` is
// one scheduling region in which the MFMAs of stage it (fragments from slot
// it&1), the loads of stage it+2 and the conversion and LDS stores of stage
// it+1 (into the other slot) are interleaved, followed by one barrier.
// With one wave per SIMD the MFMA pipe only stays busy if the loads and
// stores issue between MFMAs; run back to back they leave it idle half the
// time.  Two stages of loads stay in flight, which covers the ~1 us load
// latency seen under load.
// Register sets and LDS slots are picked at compile time (loop unrolled by
// two; each slot is its own LDS array), so the compiler can tell that the
// stores of stage it+1 do not touch what the MFMAs of stage it read, and its
// wait analysis follows each register.
// LDS rows are BK bf16 (CPR = BK/8 chunks of 16 bytes); chunk c of row r
// sits at slot c ^ f(r), f chosen so that the 32-row fragment reads are
// conflict-free (SQ_LDS_BANK_CONFLICT reads 0 on MI355X for both row
// widths; for 64-byte rows f(r) = ((r >> 1) ^ (r >> 3)) & 3 left 37% of the
// LDS busy cycles to conflicts, 4096 x 1024 x 4096 43.3 -> 42.2 us).
// Per block per stage the CU moves (4*BM + 2*BN)*BK bytes through its vector
// memory path for 2*BM*BN*BK flops: 256 x 256 tiles need 3/256 byte per
// flop, inside the ~64 B/clk a CU loads against its 4096 flop/clk.
// Requires K % BK == 0, 16-byte aligned a, b, b2, and fewer than 2^32 bytes
// in A and in each weight matrix.  Rows >= M and columns >= N are clamped for
// loading and never stored.
// waves of a large-tile block along N: four on 256 x 256 tiles, else two;
// along M (WMW): two, or four for gated 128 x 128 tiles when they do not
// outnumber the CUs (a wave's gate and up columns stay together)
constexpr int xl_wn(int bm, int bn) { return bm == 256 && bn == 256 ? 4 : 2; }
template <int BM, int BN, int BK, bool GATED, bool ABF16 = false, int SETS = 2, int WMW = 2, int KG = 1>
struct XlCfg {
    static constexpr int WNW = xl_wn(BM, BN);
    static constexpr int NT = 64 * WMW * WNW * KG;              // threads: KG groups of WMW x WNW waves
    static constexpr int KSG = BK / 16 / KG;                    // k-steps of a stage per wave group
    static constexpr int CPR = BK / 8;                          // 16-byte chunks per LDS row
    static constexpr int WTM = BM / WMW, WTN = BN / WNW;        // wave tile
    static constexpr int TM = WTM / 32, TN = WTN / 32;          // 32x32 blocks per wave
    static constexpr int BNO = GATED ? BN / 2 : BN;             // output columns per block
    static constexpr int A_SLOT = BM * BK * 2, B_SLOT = BN * BK * 2;
    static constexpr int LDS = 2 * (A_SLOT + B_SLOT);
    static constexpr int A_CPR = ABF16 ? CPR : BK / 4;          // 16-byte A chunks per row
    static constexpr int A_LOADS = BM * A_CPR / NT;             // 16-byte A loads per lane
    static constexpr int B_LOADS = BN * CPR / NT;               // 16-byte bf16 loads per lane
    static constexpr int B_ROWS_PER_LOAD = NT / CPR;
    static constexpr int MFMAS = TM * TN * KSG;                 // per wave per stage
    static constexpr int LOADS = A_LOADS + B_LOADS;             // per lane per stage
    static_assert(BK == 32 || BK == 64, "k stage");
    static_assert((KG == 1 || KG == 2) && KSG * KG == BK / 16, "wave groups split a stage's k-steps");
    static_assert(SETS >= 1 && SETS <= 3, "register sets");
    static_assert(TM >= 1 && TN >= 1 && (!GATED || TN % 2 == 0), "wave tile");
    static_assert(A_LOADS >= 1 && B_LOADS >= 1, "loads per lane");
    static_assert(!GATED || BNO % B_ROWS_PER_LOAD == 0, "a load never mixes Wg and Wu rows");
    static_assert(LDS <= 160 * 1024, "LDS");
};

template <int CPR>
__device__ __forceinline__ int xl_swz(int r) {
    if constexpr (CPR == 8) return (r ^ (r >> 3)) & 7;
    else return (r ^ (r >> 2)) & 3;
}

// B-tile row of 32-column block j of wave column wn (gated: the first TN/2
// blocks are Wg rows, the rest the Wu rows of the same outputs)
template <int BN, int TN, bool GATED, int WNW>
__device__ __forceinline__ int xl_brow(int wn, int j) {
    if constexpr (!GATED) {
        return wn * (BN / WNW) + 32 * j;
    } else {
        constexpr int TNO = TN / 2;
        const int base = wn * (BN / (2 * WNW));
        return (j < TNO) ? base + 32 * j : BN / 2 + base + 32 * (j - TNO);
    }
}

// Scheduling pattern of one stage (one wave's instruction order).  The
// fragments of the first k-step are read first; then every MFMA is followed
// by its share of: the fragment reads of the next k-step (spread over the
// MFMAs of the k-step before), the global loads (first half of the MFMAs)
// and the LDS stores (second half).  Waiting on a fragment read right before
// its MFMA would expose the LDS latency on every MFMA pair.
template <int N, int SLOTS, int I>
struct XlShare {   // how many of N items go after MFMA I of SLOTS (even spread)
    static constexpr int v = ((I + 1) * N) / SLOTS - (I * N) / SLOTS;
};
// STORE_FIRST (one register set): the stores of stage it+1 go in the first
// half, the loads of stage it+2 (into the registers the stores freed) in the
// second half.
template <int I, int MFMAS, int KS, int FR, int LOADS, bool STORE_FIRST = false>
struct XlSched {
    static constexpr int PER_K = MFMAS / KS;           // MFMAs per k-step
    static constexpr int H = MFMAS / 2;
    static constexpr int FIRST = STORE_FIRST ? 0x200 : 0x020, SECOND = STORE_FIRST ? 0x020 : 0x200;
    static __device__ __forceinline__ void run() {
        if constexpr (I == 0) __builtin_amdgcn_sched_group_barrier(0x100, FR, 0);   // first fragments
        if constexpr (I < MFMAS) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                      // MFMA
            if constexpr (I < MFMAS - PER_K) {                                      // next fragments
                constexpr int n = XlShare<FR * (KS - 1), MFMAS - PER_K, I>::v;
                if constexpr (n > 0) __builtin_amdgcn_sched_group_barrier(0x100, n, 0);
            }
            if constexpr (I < H) {
                constexpr int n = XlShare<LOADS, H, I>::v;
                if constexpr (n > 0) __builtin_amdgcn_sched_group_barrier(FIRST, n, 0);
            } else {
                constexpr int n = XlShare<LOADS, MFMAS - H, I - H>::v;
                if constexpr (n > 0) __builtin_amdgcn_sched_group_barrier(SECOND, n, 0);
            }
            XlSched<I + 1, MFMAS, KS, FR, LOADS, STORE_FIRST>::run();
        }
    }
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t xl_rsrc(const void *p, size_t bytes) {
    // raw buffer: stride 0, num_records = bytes, default data format
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)(uint32_t)bytes, 0x00020000);
}

// ABF16: A is already bf16 (a points to uint16_t bits): it is copied into LDS
// like B, with no conversion.
// 64-row tiles (batched decode) are bandwidth kernels: two blocks per CU
// double the loads in flight
// SETS = 1: one register set; each stage stores stage it+1 first and then
// loads stage it+2 into the freed registers (one stage of latency cover, for
// tiles whose two register sets would not fit).
template <int BM, int BN, int BK, bool GATED, bool ABF16, int SETS, int WMW, int KG>
__global__ __launch_bounds__(64 * WMW * xl_wn(BM, BN) * KG, WMW * xl_wn(BM, BN) * KG == 8 ? 1 : (BM * BN <= 128 * 128 ? 2 : 1)) void k_gemm_xl(float *__restrict__ c,
                                                        const void *__restrict__ a,
                                                        const uint16_t *__restrict__ b,
                                                        const uint16_t *__restrict__ b2,
                                                        int M, int K, int N, TileMap map) {
    using X = XlCfg<BM, BN, BK, GATED, ABF16, SETS, WMW, KG>;
    constexpr int CPR = X::CPR;
    __shared__ __align__(16) unsigned char sa0[X::A_SLOT];
    __shared__ __align__(16) unsigned char sa1[X::A_SLOT];
    __shared__ __align__(16) unsigned char sb0[X::B_SLOT];
    __shared__ __align__(16) unsigned char sb1[X::B_SLOT];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kg = wave / (WMW * X::WNW), wq = wave % (WMW * X::WNW);   // k group, wave within it
    const int wm = wq / X::WNW, wn = wq % X::WNW;
    int tm, tn;
    tile_of(blockIdx.x, map, tm, tn);
    const int m0 = tm * BM;
    const int n0 = tn * X::BNO;
    const int nk = K / BK;

    const __amdgpu_buffer_rsrc_t ra = xl_rsrc(a, (size_t)M * K * (ABF16 ? 2 : 4));
    const __amdgpu_buffer_rsrc_t rb = xl_rsrc(b, (size_t)N * K * 2);
    const __amdgpu_buffer_rsrc_t rb2 = GATED ? xl_rsrc(b2, (size_t)N * K * 2) : rb;

    // A: load i of this lane is fp32 chunk q = i*256 + tid of the tile (BK/4
    // chunks of 4 floats per row); B: bf16 chunk q (CPR chunks of 8 per row)
    uint32_t aoffs[X::A_LOADS];
    int adst[X::A_LOADS];
#pragma unroll
    for (int i = 0; i < X::A_LOADS; i++) {
        const int q = i * X::NT + tid;
        const int r = q / X::A_CPR, cq = q % X::A_CPR;
        const uint32_t row = (uint32_t)min(m0 + r, M - 1) * (uint32_t)K;
        if constexpr (ABF16) {
            aoffs[i] = (row + (uint32_t)cq * 8u) * 2u;
            adst[i] = r * (BK * 2) + ((cq ^ xl_swz<CPR>(r)) << 4);
        } else {
            aoffs[i] = (row + (uint32_t)cq * 4u) * 4u;
            adst[i] = r * (BK * 2) + (((cq >> 1) ^ xl_swz<CPR>(r)) << 4) + ((cq & 1) << 3);
        }
    }
    uint32_t boffs[X::B_LOADS];
    int bdst[X::B_LOADS];
#pragma unroll
    for (int i = 0; i < X::B_LOADS; i++) {
        const int q = i * X::NT + tid;
        const int r = q / CPR, ch = q % CPR;
        int gn = n0 + r;
        if constexpr (GATED) {
            if (i * X::B_ROWS_PER_LOAD >= X::BNO) gn = n0 + r - X::BNO;   // Wu rows
        }
        boffs[i] = ((uint32_t)min(gn, N - 1) * (uint32_t)K + (uint32_t)ch * 8u) * 2u;
        bdst[i] = r * (BK * 2) + ((ch ^ xl_swz<CPR>(r)) << 4);
    }

    // fragment read offsets (bytes within an A / B slot) and swizzles
    const int lrow = lane & 31, lk = lane >> 5;
    int aoff[X::TM], asw[X::TM], boff[X::TN], bsw[X::TN];
#pragma unroll
    for (int i = 0; i < X::TM; i++) {
        const int r = wm * X::WTM + 32 * i + lrow;
        aoff[i] = r * (BK * 2);
        asw[i] = xl_swz<CPR>(r);
    }
#pragma unroll
    for (int j = 0; j < X::TN; j++) {
        const int r = xl_brow<BN, X::TN, GATED, X::WNW>(wn, j) + lrow;
        boff[j] = r * (BK * 2);
        bsw[j] = xl_swz<CPR>(r);
    }

    u32x4 areg[SETS][X::A_LOADS];
    u32x4 breg[SETS][X::B_LOADS];
    // SET: register set (and, for store and compute, LDS slot), compile-time
    auto load = [&](int step, auto SET) {
        constexpr int set = SETS == 1 ? 0 : decltype(SET)::value % SETS;
        const int ka = step * BK * (ABF16 ? 2 : 4), kb = step * BK * 2;   // scalar byte offsets
#pragma unroll
        for (int i = 0; i < X::A_LOADS; i++)
            areg[set][i] = __builtin_amdgcn_raw_buffer_load_b128(ra, aoffs[i], ka, 0);
#pragma unroll
        for (int i = 0; i < X::B_LOADS; i++) {
            const bool up = GATED && i * X::B_ROWS_PER_LOAD >= X::BNO;
            breg[set][i] = __builtin_amdgcn_raw_buffer_load_b128(up ? rb2 : rb, boffs[i], kb, 0);
        }
    };
    // RSET: the register set that holds the stage (SETS = 3: not the slot)
    auto store = [&](auto SLOT, auto RSET) {
        constexpr int slot = decltype(SLOT)::value;
        constexpr int set = SETS == 1 ? 0 : SETS == 2 ? slot : decltype(RSET)::value % SETS;
        unsigned char *as = slot ? sa1 : sa0;
        unsigned char *bs = slot ? sb1 : sb0;
#pragma unroll
        for (int i = 0; i < X::A_LOADS; i++) {
            if constexpr (ABF16) {
                *reinterpret_cast<u32x4 *>(as + adst[i]) = areg[set][i];
            } else {
                const f32x4 x = __builtin_bit_cast(f32x4, areg[set][i]);
                uint2 w;
                w.x = pack_bf16x2(x.x, x.y);
                w.y = pack_bf16x2(x.z, x.w);
                *reinterpret_cast<uint2 *>(as + adst[i]) = w;
            }
        }
#pragma unroll
        for (int i = 0; i < X::B_LOADS; i++)
            *reinterpret_cast<u32x4 *>(bs + bdst[i]) = breg[set][i];
    };

    typedef float f32x16 __attribute__((ext_vector_type(16)));
    f32x16 acc[X::TM][X::TN];
#pragma unroll
    for (int i = 0; i < X::TM; i++)
#pragma unroll
        for (int j = 0; j < X::TN; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0.f;

    // fragments double-buffered across k-steps: those of k-step t+1 are read
    // while the MFMAs of k-step t run
    auto compute = [&](auto SET) {
        constexpr int set = decltype(SET)::value;
        constexpr int KS = X::KSG;                               // this group's k-steps: kg KS ..
        const unsigned char *as = set ? sa1 : sa0;
        const unsigned char *bs = set ? sb1 : sb0;
        bf16x8 fa[2][X::TM], fb[2][X::TN];
        auto read = [&](int t, int f) {
            const int ch = 2 * (kg * KS + t) + lk;
#pragma unroll
            for (int i = 0; i < X::TM; i++)
                fa[f][i] = *reinterpret_cast<const bf16x8 *>(as + aoff[i] + ((ch ^ asw[i]) << 4));
#pragma unroll
            for (int j = 0; j < X::TN; j++)
                fb[f][j] = *reinterpret_cast<const bf16x8 *>(bs + boff[j] + ((ch ^ bsw[j]) << 4));
        };
        read(0, 0);
#pragma unroll
        for (int t = 0; t < KS; t++) {
            if (t + 1 < KS) read(t + 1, (t + 1) & 1);
#pragma unroll
            for (int i = 0; i < X::TM; i++)
#pragma unroll
                for (int j = 0; j < X::TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[t & 1][i], fb[t & 1][j], acc[i][j], 0, 0, 0);
        }
    };

    // prologue: stage 0 stored, stage 1 (and with two sets stage 1 too)
    // in flight
    if constexpr (SETS == 3) {
        load(0, IC<0>{});
        if (nk > 1) load(1, IC<1>{});
        if (nk > 2) load(2, IC<2>{});
        store(IC<0>{}, IC<0>{});
    } else if constexpr (SETS == 2) {
        load(0, IC<0>{});
        if (nk > 1) load(1, IC<1>{});
        store(IC<0>{}, IC<0>{});
    } else {
        load(0, IC<0>{});
        store(IC<0>{}, IC<0>{});
        if (nk > 1) load(1, IC<0>{});
    }
    __syncthreads();

    // steady state (it + 2 < nk): SET = it & 1 is the LDS slot of stage it.
    // The loads are unconditional here (conditional loads make the
    // compiler's wait analysis wait for all of them).
    auto steady = [&](int it, auto SET) {
        constexpr int set = decltype(SET)::value;
        if constexpr (SETS == 2) {
            load(it + 2, IC<set>{});
            compute(IC<set>{});
            store(IC<set ^ 1>{}, IC<set ^ 1>{});
        } else {
            store(IC<set ^ 1>{}, IC<0>{});
            load(it + 2, IC<0>{});
            compute(IC<set>{});
        }
        XlSched<0, X::MFMAS, X::KSG, X::TM + X::TN, X::LOADS, SETS == 1>::run();
        __syncthreads();
    };
    auto tail = [&](int it, auto SET) {
        constexpr int set = decltype(SET)::value;
        if constexpr (SETS == 2) {
            if (it + 2 < nk) load(it + 2, IC<set>{});
            compute(IC<set>{});
            if (it + 1 < nk) store(IC<set ^ 1>{}, IC<set ^ 1>{});
        } else {
            if (it + 1 < nk) store(IC<set ^ 1>{}, IC<0>{});
            if (it + 2 < nk) load(it + 2, IC<0>{});
            compute(IC<set>{});
        }
        __syncthreads();
    };
    // three register sets (SETS = 3): stage it + 3 is loaded while stage it
    // is computed, so three stages are in flight; R = it mod 6 fixes the LDS
    // slot (R & 1) and the register sets (R mod 3 loaded, R + 1 mod 3 stored)
    auto steady3 = [&](int it, auto R) {
        constexpr int r = decltype(R)::value;
        load(it + 3, IC<r % 3>{});
        compute(IC<r & 1>{});
        store(IC<(r + 1) & 1>{}, IC<(r + 1) % 3>{});
        XlSched<0, X::MFMAS, X::KSG, X::TM + X::TN, X::LOADS, false>::run();
        __syncthreads();
    };
    auto tail3 = [&](int it, auto R) {
        constexpr int r = decltype(R)::value;
        if (it + 3 < nk) load(it + 3, IC<r % 3>{});
        compute(IC<r & 1>{});
        if (it + 1 < nk) store(IC<(r + 1) & 1>{}, IC<(r + 1) % 3>{});
        __syncthreads();
    };
    int it = 0;
    if constexpr (SETS == 3) {
        for (; it + 8 < nk; it += 6) {
            steady3(it, IC<0>{});
            steady3(it + 1, IC<1>{});
            steady3(it + 2, IC<2>{});
            steady3(it + 3, IC<3>{});
            steady3(it + 4, IC<4>{});
            steady3(it + 5, IC<5>{});
        }
        // at most 8 stages left, it a multiple of 6
        tail3(it, IC<0>{});
        if (it + 1 < nk) tail3(it + 1, IC<1>{});
        if (it + 2 < nk) tail3(it + 2, IC<2>{});
        if (it + 3 < nk) tail3(it + 3, IC<3>{});
        if (it + 4 < nk) tail3(it + 4, IC<4>{});
        if (it + 5 < nk) tail3(it + 5, IC<5>{});
        if (it + 6 < nk) tail3(it + 6, IC<0>{});
        if (it + 7 < nk) tail3(it + 7, IC<1>{});
    } else {
        for (; it + 3 < nk; it += 2) {
            steady(it, IC<0>{});
            steady(it + 1, IC<1>{});
        }
        // 1 to 3 stages left, it even
        tail(it, IC<0>{});
        if (it + 1 < nk) tail(it + 1, IC<1>{});
        if (it + 2 < nk) tail(it + 2, IC<0>{});
    }

    // two wave groups: the second adds its sums into the first's through LDS
    if constexpr (KG == 2) {
        __shared__ float xred[(X::NT / 2) * X::TM * X::TN * 16];
        __syncthreads();
        if (kg == 1) {
#pragma unroll
            for (int i = 0; i < X::TM; i++)
#pragma unroll
                for (int j = 0; j < X::TN; j++)
#pragma unroll
                    for (int v = 0; v < 16; v++) xred[(((wq * X::TM + i) * X::TN + j) * 16 + v) * 64 + lane] = acc[i][j][v];
        }
        __syncthreads();
        if (kg == 1) return;
#pragma unroll
        for (int i = 0; i < X::TM; i++)
#pragma unroll
            for (int j = 0; j < X::TN; j++)
#pragma unroll
                for (int v = 0; v < 16; v++) acc[i][j][v] += xred[(((wq * X::TM + i) * X::TN + j) * 16 + v) * 64 + lane];
    }

    // epilogue: value v of a 32x32 block sits at row 8*(v/4) + 4*(lane/32) + v%4,
    // column lane%32
#pragma unroll
    for (int i = 0; i < X::TM; i++) {
        const int rbase = m0 + wm * X::WTM + 32 * i + 4 * lk;
        if constexpr (!GATED) {
#pragma unroll
            for (int j = 0; j < X::TN; j++) {
                const int col = n0 + wn * X::WTN + 32 * j + lrow;
                if (col < N) {
#pragma unroll
                    for (int v = 0; v < 16; v++) {
                        const int row = rbase + 8 * (v >> 2) + (v & 3);
                        if (row < M) __builtin_nontemporal_store(acc[i][j][v], &c[(size_t)row * N + col]);
                    }
                }
            }
        } else {
            constexpr int TNO = X::TN / 2;
#pragma unroll
            for (int j = 0; j < TNO; j++) {
                const int col = n0 + wn * (X::BNO / X::WNW) + 32 * j + lrow;
                if (col < N) {
#pragma unroll
                    for (int v = 0; v < 16; v++) {
                        const int row = rbase + 8 * (v >> 2) + (v & 3);
                        if (row < M)
                            __builtin_nontemporal_store(silu_mul(acc[i][j][v], acc[i][j + TNO][v]),
                                                        &c[(size_t)row * N + col]);
                    }
                }
            }
        }
    }
}

#endif  // QH_TILE_KERNELS_H
