// MFMA GEMM kernels for decode batches, 5 <= M <= 64: weight-streaming,
// skinny (small N), narrow (K-heavy, 16/32-column blocks), wide (the tied
// lm_head) and the 16-row kernel.
// Included by hip_gemm.hip, whose host code launches them.
#ifndef QH_SMALL_M_KERNELS_H
#define QH_SMALL_M_KERNELS_H

#include "gemm_common.h"

// ---------------------------------------------------------------------------
// Weight-streaming MFMA GEMM for 5 <= M <= 64 (small decode batches)
// ---------------------------------------------------------------------------
// For M <= 64 the weights are almost all of the traffic, and the tile kernels
// above keep too few of their bytes in flight per CU to stream them at HBM
// rate.  Here a block of 8 waves owns 16-row tiles of B (the weights) and a
// K slice of 256*KS (blockIdx.y picks the slice).  Wave w owns k range
// [slice + 32*KS*w, +32*KS): it holds its A fragments (MT m-tiles of 16 rows,
// rounded to bf16 RNE) in registers for the whole kernel and loads its B
// fragments straight from memory into registers, ST tiles ahead, with
// v_mfma_f32_16x16x32_bf16 (A operand = activations, B operand = weights).
// Lane (r, g) = (lane % 16, lane / 16) holds k = 32s + 8g .. 32s + 8g + 7 of
// step s for row r of both operands.  The 8 partial tiles are summed through
// LDS in wave order (one barrier per tile, two LDS buffers).  Blocks walk
// tiles blockIdx.x, +gridDim.x, ... so one launch of <= 256 blocks streams any
// N.  Every load is an unconditional buffer load: rows past N and tiles past
// a block's last one read at an offset beyond the buffer, which returns zeros
// and touches no memory, so the loop has no branches around its loads.
// part == nullptr: C (or silu(gate)*up) is written; otherwise the fp32 sums
// of slice ks go to part[ks][j][M][N] (j = 0, or gate/up for GATED) and
// k_stream_reduce adds the slices in order.
#define STREAM_THREADS 512

template <int MT, int KS, int ST, bool GATED>
__global__ __launch_bounds__(STREAM_THREADS, 1) void k_gemm_stream(float *__restrict__ c,
                                                                float *__restrict__ part,
                                                                const float *__restrict__ a,
                                                                const uint16_t *__restrict__ b,
                                                                const uint16_t *__restrict__ b2,
                                                                int M, int K, int N, int ntiles) {
    constexpr int NJ = GATED ? 2 : 1;
    constexpr int SLOTS = MT * NJ;                       // f32x4 accumulators per lane
    __shared__ f32x4 red[2][STREAM_THREADS / WAVE][SLOTS][WAVE];

    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    const int r16 = lane & 15, g = lane >> 4;
    const int kw0 = blockIdx.y * (256 * KS) + w * (32 * KS) + 8 * g;     // this lane's first k
    const int first = blockIdx.x, stride = gridDim.x;
    const int nmine = first < ntiles ? (ntiles - 1 - first) / stride + 1 : 0;
    if (nmine == 0) return;                              // uniform over the block

    // ---- A fragments: the fp32 loads go out first, then the first B tiles'
    //      loads (below), and only then is A rounded (loads complete in order,
    //      so waiting for A does not wait for B): one memory round trip
    //      before the first MFMA instead of two
    const __amdgpu_buffer_rsrc_t ra = xl_rsrc(a, (size_t)M * K * 4);
    u32x4 alo[MT][KS], ahi[MT][KS];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int m = 16 * mt + r16;
        const uint32_t off = m < M ? (uint32_t)(((size_t)m * K + kw0) * 4) : BUF_OOB;
#pragma unroll
        for (int s = 0; s < KS; s++) {
            alo[mt][s] = __builtin_amdgcn_raw_buffer_load_b128(ra, off + 128 * s, 0, 0);
            ahi[mt][s] = __builtin_amdgcn_raw_buffer_load_b128(ra, off + 128 * s + 16, 0, 0);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    bf16x8 af[MT][KS];                                   // rounded after the B loads below

    // ---- B fragments: ST tiles in flight
    const __amdgpu_buffer_rsrc_t rb = xl_rsrc(b, (size_t)N * K * 2);
    const __amdgpu_buffer_rsrc_t rb2 = xl_rsrc(GATED ? b2 : b, (size_t)N * K * 2);
    u32x4 bq[ST][NJ][KS];
    auto boff = [&](int i) -> uint32_t {                  // byte offset of this lane's row of tile i
        const int n = 16 * (first + stride * i) + r16;
        return (i < nmine && n < N) ? (uint32_t)(((size_t)n * K + kw0) * 2) : BUF_OOB;
    };
    auto load = [&](u32x4 (&q)[NJ][KS], int i) {
        const uint32_t off = boff(i);
#pragma unroll
        for (int s = 0; s < KS; s++) {
            q[0][s] = __builtin_amdgcn_raw_buffer_load_b128(rb, off + 64 * s, 0, 0);
            if constexpr (GATED) q[1][s] = __builtin_amdgcn_raw_buffer_load_b128(rb2, off + 64 * s, 0, 0);
        }
    };

    const size_t MN = (size_t)M * N;
    auto tile = [&](const u32x4 (&q)[NJ][KS], int i) {
        f32x4 acc[NJ][MT];
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) acc[j][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; s++)
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const bf16x8 bf = __builtin_bit_cast(bf16x8, q[j][s]);
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
                    acc[j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt][s], bf, acc[j][mt], 0, 0, 0);
            }
        const int buf = i & 1;
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) red[buf][w][j * MT + mt][lane] = acc[j][mt];
        __syncthreads();
        // thread q < 64*MT sums slot (mt, lane p) over the 8 waves in order:
        // rows 16*mt + 4*(p/16) + 0..3, column 16*tile + p%16
        const int t = threadIdx.x;
        if (t < WAVE * MT) {
            const int mt = t / WAVE, p = t % WAVE;
            f32x4 sum[NJ];
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                sum[j] = red[buf][0][j * MT + mt][p];
#pragma unroll
                for (int v = 1; v < STREAM_THREADS / WAVE; v++) sum[j] += red[buf][v][j * MT + mt][p];
            }
            const int n = 16 * (first + stride * i) + (p & 15);
            const int m0 = 16 * mt + 4 * (p >> 4);
            if (n < N) {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int m = m0 + r;
                    if (m < M) {
                        const size_t o = (size_t)m * N + n;
                        if (part) {
                            float *pp = part + (size_t)blockIdx.y * NJ * MN + o;
                            pp[0] = sum[0][r];
                            if constexpr (GATED) pp[MN] = sum[1][r];
                        } else if constexpr (GATED) {
                            c[o] = silu_mul(sum[0][r], sum[1][r]);
                        } else {
                            c[o] = sum[0][r];
                        }
                    }
                }
            }
        }
    };

#pragma unroll
    for (int d = 0; d < ST; d++) load(bq[d], d);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int s = 0; s < KS; s++) {
            u32x4 p;
            p.x = pack_bf16x2(__uint_as_float(alo[mt][s].x), __uint_as_float(alo[mt][s].y));
            p.y = pack_bf16x2(__uint_as_float(alo[mt][s].z), __uint_as_float(alo[mt][s].w));
            p.z = pack_bf16x2(__uint_as_float(ahi[mt][s].x), __uint_as_float(ahi[mt][s].y));
            p.w = pack_bf16x2(__uint_as_float(ahi[mt][s].z), __uint_as_float(ahi[mt][s].w));
            af[mt][s] = __builtin_bit_cast(bf16x8, p);
        }
    for (int base = 0; base < nmine; base += ST) {
#pragma unroll
        for (int d = 0; d < ST; d++) {
            if (base + d < nmine) tile(bq[d], base + d);     // uniform over the block
            load(bq[d], base + d + ST);
        }
    }
}

// ---------------------------------------------------------------------------
// Skinny GEMM for M <= 64 with small N (batched-decode projections)
// ---------------------------------------------------------------------------
// C[M,N] = A[M,K]·B[N,K]^T with A short: blockIdx.x owns 64 rows of B (four
// waves, 16 rows each), blockIdx.y a K slice of KSL (a multiple of 64, at
// most 256) and blockIdx.z a slab of 64 rows of A and C.  The block stages its slice of A once in LDS as bf16 (RNE), rows
// of 16-byte chunks XOR-swizzled by row, so that the four waves read their
// v_mfma_f32_16x16x32_bf16 A fragments from one copy instead of each block
// re-reading A per 16-row tile; each wave issues all of its B loads before
// the staging wait, so the weight stream is in flight while A is converted.
// The weights are loaded in row order (8 rows x 128 contiguous bytes per
// instruction) and pass through the wave's own LDS rows; straight into
// registers in the MFMA fragment order (16 rows x 64 bytes per instruction)
// they took longer (measured on MI355X, graph-replayed: 16 x {3072, 4096} x
// 1024 6.53 / 6.81 -> 6.14 / 6.41 us, 64 x 3072 x 1024 10.3 -> 9.2, 48 x
// 2048 x 1024 9.06 -> 8.26; 8 x 2048 x 1024 5.73 -> 5.84).  No cross-wave
// reduction: a wave
// owns its 16 output columns.  With more than one slice the fp32 sums go to
// part[slice][j][M][N] (j = gate/up when GATED) and k_stream_reduce adds the
// slices in order; otherwise C (or silu(gate)*up) is written directly.
// Loads past M and past N are buffer loads at out-of-range offsets (zeros).
template <int MT, bool GATED>
__global__ __launch_bounds__(NTHREADS) void k_gemm_skinny(float *__restrict__ c, float *__restrict__ part,
                                                          const float *__restrict__ a,
                                                          const uint16_t *__restrict__ b,
                                                          const uint16_t *__restrict__ b2,
                                                          int M, int K, int N, int ksl) {
    constexpr int NJ = GATED ? 2 : 1;
    constexpr int KSMAX = 256 / 32;                      // 32-deep steps per slice, at most
    __shared__ __align__(16) u32x4 sa[MT * 16 * (256 / 8)];   // [row][chunk ^ swz(row)], bf16
    __shared__ __align__(16) u32x4 sbw[NTHREADS / WAVE][NJ * 16 * 32];   // each wave's weight rows
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int k0 = blockIdx.y * ksl;
    const int m0 = blockIdx.z * 64;                    // this block's 64-row slab of A and C
    const int ncs = ksl >> 3;                           // 16-byte chunks per row of the slice
    const int nst = ksl >> 5;                           // 32-deep steps

    // 1. the block's A slice first (8 floats per chunk, CPT chunks per
    //    thread; chunks past the slice or rows past M read zeros) ...
    constexpr int CPT = MT * 16 * (256 / 8) / NTHREADS;
    const __amdgpu_buffer_rsrc_t ra = buf_rsrc(a, (size_t)M * K * 4);
    const int total = MT * 16 * ncs;                     // chunks of the staged slice
    u32x4 alo[CPT], ahi[CPT];
#pragma unroll
    for (int i = 0; i < CPT; i++) {
        const int q = tid + NTHREADS * i;
        const int m = q / ncs, ch = q % ncs;
        const uint32_t off = (q < total && m0 + m < M) ? (uint32_t)(((size_t)(m0 + m) * K + k0 + 8 * ch) * 4)
                                                         : BUF_OOB;
        alo[i] = __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0);
        ahi[i] = __builtin_amdgcn_raw_buffer_load_b128(ra, off + 16, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2. ... then this wave's B chunks: row n of its 16, k = k0 + 32 s + 8 g
    //    (in flight while A is converted; loads complete in order, so a wait
    //    for A does not wait for these)
    const __amdgpu_buffer_rsrc_t rb = buf_rsrc(b, (size_t)N * K * 2);
    const __amdgpu_buffer_rsrc_t rb2 = buf_rsrc(GATED ? b2 : b, (size_t)N * K * 2);
    const int n = blockIdx.x * 64 + w * 16 + r16;
    // in row order: load s covers rows 8 (s % 2) + lane / 8 of the wave's 16,
    // chunks 8 (s / 2) + lane % 8 of the slice (8 rows x 128 bytes)
    u32x4 bq[NJ][KSMAX];
#pragma unroll
    for (int s = 0; s < KSMAX; s++) {
        const int row = 8 * (s & 1) + (lane >> 3), ch = 8 * (s >> 1) + (lane & 7);
        const int nr = blockIdx.x * 64 + w * 16 + row;
        const uint32_t off = (ch < ncs && nr < N) ? (uint32_t)(((size_t)nr * K + k0 + 8 * ch) * 2) : BUF_OOB;
        bq[0][s] = __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 2);
        if constexpr (GATED) bq[1][s] = __builtin_amdgcn_raw_buffer_load_b128(rb2, off, 0, 2);
    }
    __builtin_amdgcn_sched_barrier(0);

    // the A slice -> LDS as bf16 (RNE), 16-byte chunks XOR-swizzled by row
#pragma unroll
    for (int i = 0; i < CPT; i++) {
        const int q = tid + NTHREADS * i;
        const int m = q / ncs, ch = q % ncs;
        u32x4 v;
        v.x = pack_bf16x2(__uint_as_float(alo[i].x), __uint_as_float(alo[i].y));
        v.y = pack_bf16x2(__uint_as_float(alo[i].z), __uint_as_float(alo[i].w));
        v.z = pack_bf16x2(__uint_as_float(ahi[i].x), __uint_as_float(ahi[i].y));
        v.w = pack_bf16x2(__uint_as_float(ahi[i].z), __uint_as_float(ahi[i].w));
        if (q < total) sa[m * ncs + (ch ^ (m & 7))] = v;
    }
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int s = 0; s < KSMAX; s++) {
            const int row = 8 * (s & 1) + (lane >> 3), ch = 8 * (s >> 1) + (lane & 7);
            sbw[w][(j * 16 + row) * 32 + (ch ^ (row & 15))] = bq[j][s];
        }
    __syncthreads();

    // 3. MFMA over the slice: A fragment rows 16 mt + r16, chunk 4 s + g
    f32x4 acc[NJ][MT];
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[j][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KSMAX; s++) {
        if (s < nst) {                                   // uniform
            bf16x8 af[MT];
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const int m = 16 * mt + r16;
                af[mt] = __builtin_bit_cast(bf16x8, sa[m * ncs + ((4 * s + g) ^ (m & 7))]);
            }
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const bf16x8 bf = __builtin_bit_cast(bf16x8, sbw[w][(j * 16 + r16) * 32 + ((4 * s + g) ^ (r16 & 15))]);
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
                    acc[j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt], bf, acc[j][mt], 0, 0, 0);
            }
        }
    }

    // 4. lane holds rows 16 mt + 4 g + r, column n
    if (n < N) {
        const size_t MN = (size_t)M * N;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + 16 * mt + 4 * g + r;
                if (m < M) {
                    const size_t o = (size_t)m * N + n;
                    if (part) {
                        float *pp = part + (size_t)blockIdx.y * NJ * MN + o;
                        pp[0] = acc[0][mt][r];
                        if constexpr (GATED) pp[MN] = acc[1][mt][r];
                    } else if constexpr (GATED) {
                        c[o] = silu_mul(acc[0][mt][r], acc[1][mt][r]);
                    } else {
                        c[o] = acc[0][mt][r];
                    }
                }
            }
    }
}

// C = sum over the KSPLIT slices of part, in slice order (gated: silu(gate)*up).
// Four outputs per thread; the loads of every slice (at most RMAX) go out
// before the first add, so the pass costs one memory round trip, not one per
// slice.  Requires MN % 4 == 0 and 16-byte aligned c and part (else the
// scalar tail below handles the last MN % 4).
#define RMAX 16
template <bool GATED>
__global__ __launch_bounds__(NTHREADS) void k_stream_reduce(float *__restrict__ c,
                                                            const float *__restrict__ part,
                                                            size_t MN, int ksplit) {
    constexpr int NJ = GATED ? 2 : 1;
    const __amdgpu_buffer_rsrc_t rp = buf_rsrc(part, (size_t)ksplit * NJ * MN * 4);
    const size_t n4 = MN / 4;
    for (size_t i = (size_t)blockIdx.x * NTHREADS + threadIdx.x; i < n4; i += (size_t)gridDim.x * NTHREADS) {
        f32x4 v[NJ][RMAX];
#pragma unroll
        for (int ks = 0; ks < RMAX; ks++)
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const size_t e = ((size_t)ks * NJ + j) * MN + 4 * i;     // element offset
                v[j][ks] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                               rp, ks < ksplit && e * 4 < 0x80000000ull ? (uint32_t)(e * 4) : BUF_OOB, 0, 0));
            }
        f32x4 s0 = v[0][0], s1 = GATED ? v[NJ - 1][0] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 1; ks < RMAX; ks++)
            if (ks < ksplit) {
                s0 += v[0][ks];
                if constexpr (GATED) s1 += v[1][ks];
            }
        f32x4 o = s0;
        if constexpr (GATED) o = f32x4{silu_mul(s0.x, s1.x), silu_mul(s0.y, s1.y), silu_mul(s0.z, s1.z), silu_mul(s0.w, s1.w)};
        if (((uintptr_t)c & 15) == 0) {
            reinterpret_cast<f32x4 *>(c)[i] = o;
        } else {                                     // C only 4-byte aligned
            c[4 * i] = o.x; c[4 * i + 1] = o.y; c[4 * i + 2] = o.z; c[4 * i + 3] = o.w;
        }
    }
    if (blockIdx.x == 0 && threadIdx.x < MN % 4) {       // tail
        const size_t i = n4 * 4 + threadIdx.x;
        float t0 = part[i], t1 = GATED ? part[MN + i] : 0.f;
        for (int ks = 1; ks < ksplit; ks++) {
            t0 += part[(size_t)ks * NJ * MN + i];
            if constexpr (GATED) t1 += part[(size_t)ks * NJ * MN + MN + i];
        }
        c[i] = GATED ? silu_mul(t0, t1) : t0;
    }
}

// ---------------------------------------------------------------------------
// Narrow GEMM for M <= 64 and K-heavy shapes (o, down of a decode batch)
// ---------------------------------------------------------------------------
// blockIdx.y owns NCOL = 32 or 16 columns of C (16-column MFMA tiles; with
// GATED the same columns of both weights), blockIdx.z a slab of ROWS = 16 MT
// rows and blockIdx.x a K slice of KSL = 32 * NWV * KPW for NWV waves of KPW
// steps (slice-major, so with a multiple of 8 slices each XCD reads one
// slice of A).  Every thread issues all of its
// loads at once: the block's slice of A first (from L2), then its wave's
// weights (from HBM); the slice is rounded to bf16 (RNE) into LDS (16-byte
// chunks XOR-swizzled by row) while the weights are in flight.  Where the
// block's LDS also holds them (even KPW), the weights are loaded in row order
// -- every instruction 8 rows x 128 contiguous bytes -- and pass through the
// wave's own LDS rows, instead of straight into registers in the MFMA
// fragment order (16 rows x 64 bytes per instruction; measured on MI355X,
// graph-replayed, M = 64: q 4.9 -> 4.25 us, q|k|v 5.74 -> 5.6, k/v 5.88 ->
// 5.62, o 6.66 -> 6.49, down 7.39 -> 7.25; M = 128 k/v 4.4 -> 4.05, q 5.5 ->
// 5.05).  The NWV
// waves split the slice (wave w: KPW steps of 32 from k0 + 32 KPW w) and
// their partial tiles are added through LDS (reusing the A slice's space) in
// wave order.  With one slice the block writes C (silu(gate) * up when
// GATED).  With several, each block writes its slice sums [slice][j][M][N]
// with agent-scope (write-through) stores, waits for them, and takes a ticket
// from its tile's counter; the block that draws the last ticket reads every
// slice's sums (agent-scope loads), adds them in slice order --
// deterministic, whatever the arrival order -- writes C and resets the
// counter to zero for the next call.  No block waits for another and there
// is no second launch.  Loads past M and N read zeros at out-of-range
// offsets.
#define NARROW_COLS 32                // the widest column block (NCOL); 16 is the other
template <int MT, int KPW, bool GATED, int NCOL = NARROW_COLS, int NWV = 4>
__global__ __launch_bounds__(64 * NWV, 1) void k_gemm_narrow(float *__restrict__ c, float *__restrict__ part,
                                                            unsigned *__restrict__ cnt,
                                                            const float *__restrict__ a,
                                                            const uint16_t *__restrict__ b,
                                                            const uint16_t *__restrict__ b2, int M, int K, int N) {
    constexpr int NJ = GATED ? 2 : 1;
    constexpr int NTH = 64 * NWV, NW = NWV;              // threads and waves of a block
    constexpr int KSL = 32 * NW * KPW, CH = KSL / 8;     // slice depth, 16-byte chunks per row
    constexpr int NT = NCOL / 16, ROWS = 16 * MT;
    constexpr int RSTRIDE = NCOL + 4;                     // +4: conflict-free column writes, 16-byte aligned rows
    constexpr int SA_U4 = ROWS * CH, RED_U4 = NW * NJ * ROWS * RSTRIDE / 4;
    static_assert(CH % 16 == 0, "the row swizzle stays inside a row");
    __shared__ __align__(16) u32x4 smem[SA_U4 > RED_U4 ? SA_U4 : RED_U4];
    // weights in row order through per-wave LDS rows where they fit
    constexpr int BR = NJ * NT * 16, CW = 4 * KPW;        // a wave's weight rows, 16-byte chunks per row
    constexpr bool BROW = KPW % 2 == 0 &&
        ((SA_U4 > RED_U4 ? SA_U4 : RED_U4) + NW * BR * CW) * 16 + 64 <= 160 * 1024;
    constexpr int BSW = CW % 16 == 0 ? 15 : 7;            // row swizzle within a row's chunks
    __shared__ __align__(16) u32x4 sbw[BROW ? NW * BR * CW : 1];
    u32x4 *const sa = smem;                               // the A slice, then
    float *const red = reinterpret_cast<float *>(smem);   // [wave][j][row][RSTRIDE] wave partials
    __shared__ unsigned last_s;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int k0 = blockIdx.x * KSL, ks = gridDim.x;
    const int n0 = blockIdx.y * NCOL, m0 = blockIdx.z * ROWS;
    const size_t MN = (size_t)M * N;

    // 1. every load at once: first the block's A slice (rows past M read
    //    zeros; it comes from L2), then this wave's weights (rows
    //    n0 + 16 nt + r16, k = k0 + 32 (KPW w + s) + 8 g; from HBM), so that the
    //    slice is rounded into LDS while the weights are still in flight
    constexpr int PER = ROWS * CH / NTH;             // 32-byte pieces of A per thread
    // Where A's pieces and the weights together would pass 48 loads in
    // flight (the 16-wide blocks with one 3072-deep slice), A comes in two
    // halves: the second is loaded once the first is in LDS, while the
    // weights are still on their way from HBM.
    constexpr int PA = (2 * PER + NJ * NT * KPW > 48) ? (PER + 1) / 2 : PER;
    static_assert(PER >= 1 && ROWS * CH % NTH == 0 && 2 * PA + NJ * NT * KPW <= 64, "loads in flight");
    const __amdgpu_buffer_rsrc_t ra = xl_rsrc(a, (size_t)M * K * 4);
    u32x4 lo[PA], hi[PA];
    auto load_a = [&](int i, int slot) {                  // piece i into register slot
        const int q = tid + NTH * i;
        const int m = m0 + q / CH, ch = q % CH;
        const uint32_t off = (uint32_t)(((size_t)m * K + k0 + 8 * ch) * 4);
        lo[slot] = __builtin_amdgcn_raw_buffer_load_b128(ra, m < M ? off : BUF_OOB, 0, 0);
        hi[slot] = __builtin_amdgcn_raw_buffer_load_b128(ra, m < M ? off + 16u : BUF_OOB, 0, 0);
    };
#pragma unroll
    for (int i = 0; i < PA; i++) load_a(i, i);
    const __amdgpu_buffer_rsrc_t rb = xl_rsrc(b, (size_t)N * K * 2);
    const __amdgpu_buffer_rsrc_t rb2 = xl_rsrc(GATED ? b2 : b, (size_t)N * K * 2);
    u32x4 bq[NJ][NT][KPW];
    if constexpr (BROW) {
        // load i: rows 8 (i % (BR / 8)) + lane / 8 of the wave's BR rows (Wg rows,
        // then Wu rows), chunks 8 (i / (BR / 8)) + lane % 8: 8 rows x 128 bytes
        u32x4 *const flat = &bq[0][0][0];
#pragma unroll
        for (int i = 0; i < NJ * NT * KPW; i++) {
            const int row = 8 * (i % (BR / 8)) + (lane >> 3), ch = 8 * (i / (BR / 8)) + (lane & 7);
            const int j = row / (NT * 16), n = n0 + row % (NT * 16);
            const uint32_t off = n < N ? (uint32_t)(((size_t)n * K + k0 + 32 * KPW * w + 8 * ch) * 2) : BUF_OOB;
            flat[i] = __builtin_amdgcn_raw_buffer_load_b128(j ? rb2 : rb, off, 0, 2);
        }
    } else {                                              // fragment order: rows n0 + 16 nt + r16
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int n = n0 + 16 * nt + r16;
            const uint32_t base = (uint32_t)(((size_t)n * K + k0 + 32 * KPW * w + 8 * g) * 2);
#pragma unroll
            for (int s = 0; s < KPW; s++) {
                const uint32_t off = n < N ? base + 64u * s : BUF_OOB;
                bq[0][nt][s] = __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 2);
                if constexpr (GATED) bq[NJ - 1][nt][s] = __builtin_amdgcn_raw_buffer_load_b128(rb2, off, 0, 2);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    u32x4 *const sbwave = sbw + (BROW ? w * BR * CW : 0);
    if constexpr (BROW) {
        const u32x4 *const flat = &bq[0][0][0];
#pragma unroll
        for (int i = 0; i < NJ * NT * KPW; i++) {
            const int row = 8 * (i % (BR / 8)) + (lane >> 3), ch = 8 * (i / (BR / 8)) + (lane & 7);
            sbwave[row * CW + (ch ^ (row & BSW))] = flat[i];
        }
    }

    // 2. A rounded to bf16 (RNE) into LDS (the second half, if any, loaded
    //    and rounded after the first)
    auto store_a = [&](int i, int slot) {
        const int q = tid + NTH * i;
        const int m = q / CH, ch = q % CH;
        u32x4 v;
        v.x = pack_bf16x2(__uint_as_float(lo[slot].x), __uint_as_float(lo[slot].y));
        v.y = pack_bf16x2(__uint_as_float(lo[slot].z), __uint_as_float(lo[slot].w));
        v.z = pack_bf16x2(__uint_as_float(hi[slot].x), __uint_as_float(hi[slot].y));
        v.w = pack_bf16x2(__uint_as_float(hi[slot].z), __uint_as_float(hi[slot].w));
        sa[m * CH + (ch ^ (m & 15))] = v;
    };
#pragma unroll
    for (int i = 0; i < PA; i++) store_a(i, i);
    if constexpr (PA < PER) {
#pragma unroll
        for (int i = PA; i < PER; i++) load_a(i, i - PA);
#pragma unroll
        for (int i = PA; i < PER; i++) store_a(i, i - PA);
    }
    __syncthreads();

    // 3. MFMA over this wave's steps: A fragment rows 16 mt + r16, chunk 4 (KPW w + s) + g
    f32x4 acc[NJ][NT][MT];
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) acc[j][nt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KPW; s++) {
        bf16x8 af[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const int m = 16 * mt + r16;
            af[mt] = __builtin_bit_cast(bf16x8, sa[m * CH + ((4 * (KPW * w + s) + g) ^ (m & 15))]);
        }
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
                {
                    u32x4 wf;
                    if constexpr (BROW) {
                        const int row = (j * NT + nt) * 16 + r16, ch = 4 * s + g;
                        wf = sbwave[row * CW + (ch ^ (row & BSW))];
                    } else {
                        wf = bq[j][nt][s];
                    }
                    acc[j][nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        af[mt], __builtin_bit_cast(bf16x8, wf), acc[j][nt][mt], 0, 0, 0);
                }
    }
    __syncthreads();                                      // every wave is done reading the A slice

    // 4. wave partials -> LDS: lane holds rows 16 mt + 4 g + r, column 16 nt + r16
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    red[((w * NJ + j) * ROWS + 16 * mt + 4 * g + r) * RSTRIDE + 16 * nt + r16] =
                        acc[j][nt][mt][r];
    __syncthreads();

    // 5. quads of 4 columns, q = tid + NTH i: row m0 + q / QR, columns
    //    4 (q % QR) .. +3 (QR = NCOL / 4 quads per row), summed over the
    //    waves in order; N % 4 == 0, so a quad is wholly in or out
    constexpr int QR = NCOL / 4;
    constexpr int NQ = ROWS * QR, QPT = NQ >= NTH ? NQ / NTH : 1;
    static_assert(NQ % NTH == 0 || NQ < NTH, "quads per thread");
    f32x4 v[NJ][QPT];
    uint32_t coff[QPT];                                   // byte offset of the quad in C, or BUF_OOB
#pragma unroll
    for (int i = 0; i < QPT; i++) {
        const bool live = tid + NTH * i < NQ;        // MT = 1: half of the threads
        const int q = live ? tid + NTH * i : 0;
        const int m = q / QR, cq = 4 * (q % QR), n = n0 + cq;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            f32x4 t = *reinterpret_cast<const f32x4 *>(&red[(j * ROWS + m) * RSTRIDE + cq]);
#pragma unroll
            for (int ww = 1; ww < NW; ww++)
                t += *reinterpret_cast<const f32x4 *>(&red[((ww * NJ + j) * ROWS + m) * RSTRIDE + cq]);
            v[j][i] = t;
        }
        coff[i] = (live && m0 + m < M && n < N) ? (uint32_t)(((size_t)(m0 + m) * N + n) * 4) : BUF_OOB;
    }
    auto finish = [&](const f32x4 &x, const f32x4 &y) -> u32x4 {
        if constexpr (GATED)
            return __builtin_bit_cast(u32x4, f32x4{silu_mul(x[0], y[0]), silu_mul(x[1], y[1]),
                                                   silu_mul(x[2], y[2]), silu_mul(x[3], y[3])});
        else
            return __builtin_bit_cast(u32x4, x);
    };
    const __amdgpu_buffer_rsrc_t rc = xl_rsrc(c, MN * 4);
    if (ks == 1) {
#pragma unroll
        for (int i = 0; i < QPT; i++)
            __builtin_amdgcn_raw_buffer_store_b128(finish(v[0][i], v[NJ - 1][i]), rc, coff[i], 0, 0);
        return;
    }
    // 6. slice sums out (write-through, agent scope), then a ticket; the last
    //    block adds the slices
    const __amdgpu_buffer_rsrc_t rp = xl_rsrc(part, (size_t)ks * NJ * MN * 4);
    const uint32_t j_bytes = (uint32_t)(MN * 4), sl_bytes = NJ * j_bytes;
#pragma unroll
    for (int i = 0; i < QPT; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
            __builtin_amdgcn_raw_buffer_store_b128(
                __builtin_bit_cast(u32x4, v[j][i]), rp,
                coff[i] == BUF_OOB ? BUF_OOB : coff[i] + blockIdx.x * sl_bytes + j * j_bytes, 0, AUX_SC1);
    __builtin_amdgcn_s_waitcnt(0);                        // this thread's sums have landed
    __syncthreads();                                      // ... and every thread's
    unsigned *const tick = cnt + blockIdx.z * gridDim.y + blockIdx.y;
    if (tid == 0)
        last_s = __hip_atomic_fetch_add(tick, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)ks - 1u;
    __syncthreads();
    if (!last_s) return;                                  // uniform over the block
    f32x4 sum[NJ][QPT];
#pragma unroll
    for (int i = 0; i < QPT; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
            sum[j][i] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           rp, coff[i] == BUF_OOB ? BUF_OOB : coff[i] + j * j_bytes, 0, AUX_SC1));
    for (int sl0 = 1; sl0 < ks; sl0 += 8) {               // 8 slices of every quad in flight, added in order
        u32x4 t[NJ][QPT][8];
#pragma unroll
        for (int i = 0; i < QPT; i++)
#pragma unroll
            for (int j = 0; j < NJ; j++)
#pragma unroll
                for (int u = 0; u < 8; u++)
                    t[j][i][u] = __builtin_amdgcn_raw_buffer_load_b128(
                        rp, (coff[i] == BUF_OOB || sl0 + u >= ks)
                                ? BUF_OOB : coff[i] + (uint32_t)(sl0 + u) * sl_bytes + j * j_bytes,
                        0, AUX_SC1);
#pragma unroll
        for (int i = 0; i < QPT; i++)
#pragma unroll
            for (int j = 0; j < NJ; j++)
#pragma unroll
                for (int u = 0; u < 8; u++)
                    if (sl0 + u < ks) sum[j][i] += __builtin_bit_cast(f32x4, t[j][i][u]);
    }
#pragma unroll
    for (int i = 0; i < QPT; i++)
        __builtin_amdgcn_raw_buffer_store_b128(finish(sum[0][i], sum[NJ - 1][i]), rc, coff[i], 0, 0);
    if (tid == 0) __hip_atomic_store(tick, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Wide GEMM for M <= 64 and very wide N (the tied lm_head of a decode batch)
// ---------------------------------------------------------------------------
// One block per CU, four independent waves.  The block's 16 MT rows of A sit
// in LDS as bf16 for the whole launch (RNE; 16-byte chunks XOR-swizzled by
// row); each wave walks its own 32-column tiles (DEF = 0: tile t = wave + j
// waves)
// over the whole of K, in chunks of 64 k.  A chunk's weights -- 32 rows x
// 128 bytes -- are read with every load instruction covering 8 rows x 128
// contiguous bytes (the MFMA fragment order, 16 rows x 64 bytes per
// instruction, streams about 15% slower from HBM), passed through the wave's
// own 4 KB of LDS, and read back as 16x16x32 MFMA fragments.  WIDE_D chunks
// are in flight per wave; no block or wave waits for another.  Loads past N
// read zeros at out-of-range offsets; rows past M are zeros in LDS.
// DEF > 0 (every wave has at most DEF tiles, as for the 151,936-column
// lm_head): wave gw takes the DEF consecutive tiles from DEF gw, holds each
// finished tile's sums in registers and writes them all after its last one,
// so that C goes out in rows of DEF x 128 contiguous bytes after the weight
// stream instead of interleaved with it (measured on MI355X, graph-replayed,
// 64 / 32 / 8 x 1024 x 151936: 66.0 / 58.9 / 50.7 -> 59.6 / 52.0 / 47.8 us;
// holding the tiles but keeping the strided tile order: 64.2 / 54.8 / 48.9).
#define WIDE_KC 64            // k per chunk
#define WIDE_D 4              // chunks in flight per wave (K / WIDE_KC must be a multiple)
#define WIDE_A_BYTES (128 * 1024)
#define WIDE_B_U4 (32 * WIDE_KC / 8)   // 16-byte chunks of one wave's staged weights
__device__ __forceinline__ int wide_key(int row) { return (row ^ (row >> 3)) & 7; }

template <int MT, int NCH, int DEF>
__global__ __launch_bounds__(NTHREADS, 1) void k_gemm_wide(float *__restrict__ c, const float *__restrict__ a,
                                                          const uint16_t *__restrict__ b, int M, int N,
                                                          int ntiles) {
    extern __shared__ __align__(16) u32x4 wide_lds[];
    constexpr int ROWS = 16 * MT, NW = NTHREADS / WAVE, K = NCH * WIDE_KC, CHA = K / 8;
    static_assert(NCH % WIDE_D == 0 && CHA % 16 == 0 && ROWS * CHA * 16 <= WIDE_A_BYTES, "wide geometry");
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    u32x4 *const sa = wide_lds;                            // [ROWS][CHA] A, swizzled
    u32x4 *const sb = wide_lds + ROWS * CHA + w * WIDE_B_U4;   // this wave's staged chunk
    const int gw = blockIdx.x * NW + w, nwaves = gridDim.x * NW;
    // tiles of this wave: gw, gw + nwaves, ...; with DEF, the DEF consecutive
    // tiles from gw DEF (their C rows then go out DEF x 128 contiguous bytes)
    const int my_tiles = DEF > 0 ? min(max(ntiles - gw * DEF, 0), DEF)
                                 : (gw < ntiles ? (ntiles - gw + nwaves - 1) / nwaves : 0);
    auto tile_index = [&](int ti) { return DEF > 0 ? gw * DEF + ti : gw + ti * nwaves; };
    const __amdgpu_buffer_rsrc_t rb = xl_rsrc(b, (size_t)N * K * 2);

    // the loads of chunk kc of tile number ti (of this wave): instruction i
    // covers rows 32 t + 8 i + lane / 8, bytes 128 kc + 16 (lane % 8)
    // (32-bit offsets, N * K * 2 < 2^31; computed without branches so that
    // every load is issued where it stands)
    auto issue = [&](u32x4 (&dst)[4], int ti, int kc) {
        const int t = tile_index(ti);
        const bool live = ti < my_tiles;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = 32 * t + 8 * i + (lane >> 3);
            const uint32_t off = ((uint32_t)n * K + WIDE_KC * kc + 8 * (lane & 7)) * 2u;
            dst[i] = __builtin_amdgcn_raw_buffer_load_b128(rb, (live && n < N) ? off : BUF_OOB, 0, 2);
        }
    };
    u32x4 ring[WIDE_D][4];
#pragma unroll
    for (int d = 0; d < WIDE_D; d++) issue(ring[d], 0, d);
    __builtin_amdgcn_sched_barrier(0);

    // A -> LDS once: rows past M read zeros
    {
        const __amdgpu_buffer_rsrc_t ra = xl_rsrc(a, (size_t)M * K * 4);
        constexpr int TOTAL = ROWS * CHA;
#pragma unroll 1
        for (int q0 = 0; q0 < TOTAL; q0 += 8 * NTHREADS) {
            u32x4 lo[8], hi[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int q = q0 + tid + NTHREADS * i;
                const int m = q / CHA, ch = q % CHA;
                const bool ok = q < TOTAL && m < M;
                const uint32_t off = (uint32_t)(((size_t)m * K + 8 * ch) * 4);
                lo[i] = __builtin_amdgcn_raw_buffer_load_b128(ra, ok ? off : BUF_OOB, 0, 0);
                hi[i] = __builtin_amdgcn_raw_buffer_load_b128(ra, ok ? off + 16u : BUF_OOB, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int q = q0 + tid + NTHREADS * i;
                const int m = q / CHA, ch = q % CHA;
                u32x4 v;
                v.x = pack_bf16x2(__uint_as_float(lo[i].x), __uint_as_float(lo[i].y));
                v.y = pack_bf16x2(__uint_as_float(lo[i].z), __uint_as_float(lo[i].w));
                v.z = pack_bf16x2(__uint_as_float(hi[i].x), __uint_as_float(hi[i].y));
                v.w = pack_bf16x2(__uint_as_float(hi[i].z), __uint_as_float(hi[i].w));
                if (q < TOTAL) sa[m * CHA + (ch ^ (m & 15))] = v;
            }
        }
    }
    __syncthreads();

    // The tile out through the wave's staging space (see below)
    auto store_half = [&](const f32x4 (&acc)[2][MT], int ti, const int h) {
        // The tile out through the wave's staging space, 32 rows at a time, so
        // that every store instruction writes 8 rows x 128 contiguous bytes
        // (4-byte stores straight from the MFMA layout, 4 rows x 64 bytes per
        // instruction, write back at well under half the speed).  Lane holds
        // rows 16 mt + 4 g + r, column 16 nt + r16; LDS row-major [32][32]
        // fp32 with the 16-byte chunk XOR-swizzled by row.
        const int t = tile_index(ti);
        float *const sc = reinterpret_cast<float *>(sb);
        const __amdgpu_buffer_rsrc_t rc = xl_rsrc(c, (size_t)M * N * 4);
        {
#pragma unroll
            for (int mh = 0; mh < 2 && 2 * h + mh < MT; mh++)
#pragma unroll
                for (int nt = 0; nt < 2; nt++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int row = 16 * mh + 4 * g + r, col = 16 * nt + r16;
                        sc[row * 32 + ((((col >> 2) ^ (row & 7)) << 2) | (col & 3))] = acc[nt][2 * h + mh][r];
                    }
#pragma unroll
            for (int i = 0; i < (MT >= 2 ? 4 : 2); i++) {
                const int row = 8 * i + (lane >> 3), cq = lane & 7;
                const f32x4 v = *reinterpret_cast<const f32x4 *>(&sc[row * 32 + ((cq ^ (row & 7)) << 2)]);
                const int m = 32 * h + row, n = 32 * t + 4 * cq;
                const uint32_t off = (m < M && n < N) ? (uint32_t)(((size_t)m * N + n) * 4) : BUF_OOB;
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rc, off, 0, 2);   // nt
            }
        }
    };
    auto store_tile = [&](const f32x4 (&acc)[2][MT], int ti) {
#pragma unroll
        for (int h = 0; h < (MT + 1) / 2; h++) store_half(acc, ti, h);
    };
    f32x4 held[DEF > 0 ? DEF : 1][2][MT];                 // finished tiles, written after the last one
    // one iteration per tile, its NCH chunks unrolled: chunk kc always uses
    // ring slot kc % WIDE_D, and the accumulators live inside the iteration
    for (int ti = 0; ti < my_tiles; ti++) {
        f32x4 acc[2][MT];
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) acc[nt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kc = 0; kc < NCH; kc++) {
            const int d = kc % WIDE_D;
            // stage this chunk: row 8 i + lane / 8, chunk lane % 8 (swizzled)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int row = 8 * i + (lane >> 3);
                sb[row * 8 + ((lane & 7) ^ wide_key(row))] = ring[d][i];
            }
            // refill the slot WIDE_D chunks ahead (into the next tile near the end)
            if (kc + WIDE_D < NCH) issue(ring[d], ti, kc + WIDE_D);
            else issue(ring[d], ti + 1, kc + WIDE_D - NCH);
            __builtin_amdgcn_sched_barrier(0);            // keep the ring's order of issue
            // two k-steps of 32: A rows 16 mt + r16, B rows 16 nt + r16, chunk 4 s + g
#pragma unroll
            for (int s = 0; s < 2; s++) {
                const int ka = 4 * (WIDE_KC / 32 * kc + s) + g;         // chunk of A's row
                bf16x8 af[MT], bfr[2];
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    const int m = 16 * mt + r16;
                    af[mt] = __builtin_bit_cast(bf16x8, sa[m * CHA + (ka ^ (m & 15))]);
                }
#pragma unroll
                for (int nt = 0; nt < 2; nt++) {
                    const int row = 16 * nt + r16;
                    bfr[nt] = __builtin_bit_cast(bf16x8, sb[row * 8 + ((4 * s + g) ^ wide_key(row))]);
                }
#pragma unroll
                for (int nt = 0; nt < 2; nt++)
#pragma unroll
                    for (int mt = 0; mt < MT; mt++)
                        acc[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt], bfr[nt], acc[nt][mt], 0, 0, 0);
            }
        }
        if constexpr (DEF == 0) {
            store_tile(acc, ti);
        } else {
#pragma unroll
            for (int q = 0; q < DEF; q++)
                if (q == ti) {
#pragma unroll
                    for (int nt = 0; nt < 2; nt++)
#pragma unroll
                        for (int mt = 0; mt < MT; mt++) held[q][nt][mt] = acc[nt][mt];
                }
        }
    }
    if constexpr (DEF > 0) {
#pragma unroll
        for (int h = 0; h < (MT + 1) / 2; h++)
#pragma unroll
            for (int q = 0; q < DEF; q++)
                if (q < my_tiles) store_half(held[q], q, h);
    }
}

// ---------------------------------------------------------------------------
// 16-row GEMM for M <= 16 (small decode batches)
// ---------------------------------------------------------------------------
// blockIdx.x owns 16 CT columns of C (16 CT rows of B); the block's NWV waves
// split K = KT (wave w: k range [w KW, (w + 1) KW)), each computing 16 x 16
// tiles with v_mfma_f32_16x16x32_bf16 (A operand = activations, B operand =
// weights), and the NWV tiles are added through LDS in wave order.  Each lane
// issues all of its loads at once: its share of the wave's weights, then its
// share of the wave's 16 x KW slice of A (fp32; rows past M read zeros) --
// both in row order, every load instruction covering whole 128-byte lines (8
// rows x 128 bytes of weights, 2 rows x 512 bytes of A at KW = 128).  Loading
// A in the MFMA fragment order instead (16 rows x two 16-byte pieces 32 bytes
// apart per instruction) made A the larger part of the kernel (measured on
// MI355X, graph-replayed per call: 16 x 1024 x 3072 3.87 -> 3.01 us, 16 x
// 2048 x 2048 5.74 -> 3.68, 8 x 1024 x 3072 3.24 -> 2.82).  Both pass through
// the wave's own LDS rows (16-byte chunks XOR-swizzled by row; A rounded to
// bf16 (RNE) on the way in) and come back as fragments; only the wave itself
// reads its rows, so a wave-scope fence, not a block barrier, orders the
// writes and reads.  Where the block's LDS does not hold weights and A side
// by side (m16_asep false), the wave reads its weight fragments into
// registers first and A then reuses the same rows.  Lane (r, g) =
// (lane % 16, lane / 16) holds k = 32s + 8g .. 32s + 8g + 7 of step s for
// row r of both operands.  Rows of B past N read zeros and their columns of C
// are not stored.  GATED: the block's two tiles are the Wg and the Wu rows of
// the same 16 columns (CT = 2), and C = silu(x Wg^T) * (x Wu^T).
constexpr bool m16_asep(int nwv, int kt, int ct) {
    return ct * 16 * kt * 2 + 16 * kt * 2 + nwv * ct * 16 * 17 * 4 <= 160 * 1024;
}
constexpr size_t m16_lds_bytes(int nwv, int kt, int ct) {   // weights, A (if separate), wave tiles
    return (size_t)ct * 16 * kt * 2 + (m16_asep(nwv, kt, ct) ? (size_t)16 * kt * 2 : 0) +
           (size_t)nwv * ct * 16 * 17 * 4;
}
template <int NWV, int KT, int CT, bool GATED = false>
__global__ __launch_bounds__(NWV * WAVE) void k_gemm_m16(float *__restrict__ c, const float *__restrict__ a,
                                                        const uint16_t *__restrict__ b,
                                                        const uint16_t *__restrict__ b2, int M, int N) {
    constexpr int KW = KT / NWV, CHW = KW / 8, STEPS = KW / 32, NBL = 16 * CHW / WAVE;
    constexpr int PPR = KW / 4, APL = 16 * PPR / WAVE;   // 16-byte fp32 pieces of A per row / per lane
    constexpr int SW = CHW >= 16 ? 15 : CHW - 1;           // swizzle mask: within the row's chunks
    constexpr bool ASEP = m16_asep(NWV, KT, CT);
    static_assert(KW * NWV == KT && CHW % 8 == 0 && NBL * WAVE == 16 * CHW && APL * WAVE == 16 * PPR &&
                  NWV * WAVE >= 256 * CT && (!GATED || CT == 2), "k split");
    constexpr int COLS = GATED ? 16 : 16 * CT;             // columns of C per block
    // LDS: [NWV][CT][16][CHW] weights, [NWV][16][CHW] A if separate, [NWV][CT][16][17] fp32 tiles
    extern __shared__ __align__(16) u32x4 m16_lds[];
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    const int r16 = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * COLS;
    u32x4 *const sb = m16_lds + w * CT * 16 * CHW;
    u32x4 *const sa = ASEP ? m16_lds + NWV * CT * 16 * CHW + w * 16 * CHW : sb;
    float *const red = reinterpret_cast<float *>(m16_lds + NWV * CT * 16 * CHW + (ASEP ? NWV * 16 * CHW : 0));

    // weights: load i of tile t covers rows 16 t + 8 (i % 2) + lane / 8 (GATED: rows
    // 8 (i % 2) + lane / 8 of Wg for t = 0, of Wu for t = 1), chunks 8 (i / 2) + lane % 8
    const __amdgpu_buffer_rsrc_t rb = buf_rsrc(b, (size_t)N * KT * 2);
    const __amdgpu_buffer_rsrc_t rb2 = buf_rsrc(GATED ? b2 : b, (size_t)N * KT * 2);
    u32x4 bw[CT][NBL];
#pragma unroll
    for (int t = 0; t < CT; t++)
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int row = 8 * (i & 1) + (lane >> 3), ch = 8 * (i >> 1) + (lane & 7);
            const int n = n0 + (GATED ? 0 : 16 * t) + row;
            const uint32_t off = n < N ? ((uint32_t)n * KT + w * KW + 8 * ch) * 2u : BUF_OOB;
            bw[t][i] = __builtin_amdgcn_raw_buffer_load_b128(GATED && t ? rb2 : rb, off, 0, 0);
        }
    // A: piece q = j WAVE + lane is row q / PPR, floats 4 (q % PPR) .. + 3 of the wave's k range
    const __amdgpu_buffer_rsrc_t ra = buf_rsrc(a, (size_t)M * KT * 4);
    u32x4 ap[APL];
#pragma unroll
    for (int j = 0; j < APL; j++) {
        const int q = j * WAVE + lane, row = q / PPR, pc = q % PPR;
        const uint32_t off = row < M ? ((uint32_t)row * KT + w * KW + 4 * pc) * 4u : BUF_OOB;
        ap[j] = __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    auto wave_sync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    auto store_a = [&] {        // rounded to bf16, 8 bytes = half a 16-byte chunk per piece
#pragma unroll
        for (int j = 0; j < APL; j++) {
            const int q = j * WAVE + lane, row = q / PPR, pc = q % PPR;
            uint2 v;
            v.x = pack_bf16x2(__uint_as_float(ap[j].x), __uint_as_float(ap[j].y));
            v.y = pack_bf16x2(__uint_as_float(ap[j].z), __uint_as_float(ap[j].w));
            *reinterpret_cast<uint2 *>(reinterpret_cast<unsigned char *>(sa + row * CHW + ((pc >> 1) ^ (row & SW))) +
                                       8 * (pc & 1)) = v;
        }
    };
#pragma unroll
    for (int t = 0; t < CT; t++)
#pragma unroll
        for (int i = 0; i < NBL; i++) {
            const int row = 8 * (i & 1) + (lane >> 3), ch = 8 * (i >> 1) + (lane & 7);
            sb[(16 * t + row) * CHW + (ch ^ (row & SW))] = bw[t][i];
        }
    if constexpr (ASEP) store_a();
    wave_sync();
    bf16x8 bf[ASEP ? 1 : STEPS][CT];
    if constexpr (!ASEP) {      // weight fragments to registers, then A into the same rows
#pragma unroll
        for (int s = 0; s < STEPS; s++)
#pragma unroll
            for (int t = 0; t < CT; t++)
                bf[s][t] = __builtin_bit_cast(bf16x8, sb[(16 * t + r16) * CHW + ((4 * s + g) ^ (r16 & SW))]);
        wave_sync();
        store_a();
        wave_sync();
    }

    f32x4 acc[CT];
#pragma unroll
    for (int t = 0; t < CT; t++) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < STEPS; s++) {
        const int ch = 4 * s + g;
        const bf16x8 af = __builtin_bit_cast(bf16x8, sa[r16 * CHW + (ch ^ (r16 & SW))]);
#pragma unroll
        for (int t = 0; t < CT; t++) {
            bf16x8 wf;
            if constexpr (ASEP) wf = __builtin_bit_cast(bf16x8, sb[(16 * t + r16) * CHW + (ch ^ (r16 & SW))]);
            else wf = bf[s][t];
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, wf, acc[t], 0, 0, 0);
        }
    }
    // lane (r, g) holds rows 4g .. 4g + 3 of C, column 16 t + r of the block's
#pragma unroll
    for (int t = 0; t < CT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) red[((w * CT + t) * 16 + 4 * g + r) * 17 + r16] = acc[t][r];
    __syncthreads();
    if constexpr (GATED) {
        if (threadIdx.x < 256) {
            const int m = (threadIdx.x >> 4) & 15, col = threadIdx.x & 15;
            float sg = red[m * 17 + col], su = red[(16 + m) * 17 + col];
#pragma unroll
            for (int v = 1; v < NWV; v++) {
                sg += red[((v * 2) * 16 + m) * 17 + col];
                su += red[((v * 2 + 1) * 16 + m) * 17 + col];
            }
            const int n = n0 + col;
            if (m < M && n < N) c[(size_t)m * N + n] = silu_mul(sg, su);
        }
    } else if (threadIdx.x < 256 * CT) {
        const int t = threadIdx.x >> 8, m = (threadIdx.x >> 4) & 15, col = threadIdx.x & 15;
        float sum = red[(t * 16 + m) * 17 + col];
#pragma unroll
        for (int v = 1; v < NWV; v++) sum += red[((v * CT + t) * 16 + m) * 17 + col];
        const int n = n0 + 16 * t + col;
        if (m < M && n < N) c[(size_t)m * N + n] = sum;
    }
}

#endif  // QH_SMALL_M_KERNELS_H
