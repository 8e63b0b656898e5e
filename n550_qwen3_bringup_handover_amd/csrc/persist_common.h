// Device helpers shared by the persistent decode kernels (hip_persist.hip:
// the 112 layer GEMVs; hip_model_persist.hip: the whole decoder stack):
// the packed-bf16 GEMV rows of a compute wave (the same sums in the same
// order as the per-call k_gemv1, so outputs are bit-identical), the paced
// weight prefetch, and the exchange between workgroups -- tagged words
// {fp32, epoch} written by the producers, polled across the XCD boundary by
// PS_RELAYS relay workgroups per XCD, which copy them into their XCD's copy
// and raise a flag per part; every workgroup of the XCD polls the flags and
// reads the copy.  Every wait is bounded (PS_SPIN rounds), after which it
// records an error flag and goes on, so every wave always finishes.
#ifndef QH_PERSIST_COMMON_H
#define QH_PERSIST_COMMON_H

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define WAVE 64
#define PS_CWAVES 4                          // compute waves per workgroup
#define PS_THREADS ((PS_CWAVES + 1) * WAVE)  // + the poller wave
#define PS_BLOCKS 256
#define PS_GW (PS_BLOCKS * PS_CWAVES)        // compute waves of a launch
#define PS_SPIN (1 << 15)                    // poll rounds before giving up (~30 ms)
#define PS_LDS_U32 1536                      // one input buffer: 3072 bf16 values

// s_sleep units between consecutive weight loads of a stage's prefetch (load_wts).
// Measured on MI355X, the 112 layer GEMVs with the relays' first poll after
// 24 units: 293 us unpaced, 289 / 286 / 286 us at 3 / 4 / 5 units everywhere,
// 284 us at these (8 units everywhere: 319 us, the waves reach the barrier late)
#define PACE_QKV 4
#define PACE_O 3
#define PACE_GU 5
#define PACE_D 3

// ---- helpers (the same arithmetic as the per-call GEMV kernels) -----------
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *p, size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)(uint32_t)bytes, 0x00020000);
}
#define AUX_NT 2       // non-temporal: each weight is read once per step
#define AUX_SC1 16     // agent scope: coherent across the XCDs' L2 caches

__device__ __forceinline__ uint32_t pack_bf16x2(float x, float y) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const f32x2_t f = {x, y};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}
__device__ __forceinline__ float bf16_dot2(uint32_t w, uint32_t x, float acc) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w), __builtin_bit_cast(bf16x2_t, x), acc,
                                           false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_partner(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
// sum over the 64 lanes, the same bits in every lane (as wave_sum of gemm_common.h)
__device__ __forceinline__ float wave_sum(float x) {
    x += dpp_partner<0xB1>(x);
    x += dpp_partner<0x4E>(x);
    x += dpp_partner<0x141>(x);
    x += dpp_partner<0x140>(x);
    const auto p16 = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, x), __builtin_bit_cast(int, x), false, false);
    x = __builtin_bit_cast(float, (int)p16[0]) + __builtin_bit_cast(float, (int)p16[1]);
    const auto p32 = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, x), __builtin_bit_cast(int, x), false, false);
    return __builtin_bit_cast(float, (int)p32[0]) + __builtin_bit_cast(float, (int)p32[1]);
}
__device__ __forceinline__ float silu_mul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

// ---- compute waves -----------------------------------------------------------
// Weights of ROWS consecutive rows (and the matching rows of b2 when GATED)
// starting at row0, K = 512 * CPL: every row and chunk is in range (the
// stage shapes divide evenly), so the loads are unconditional.  PACE s_sleep
// units (64 clocks) separate consecutive loads: a stage's output exchange
// queues behind the weight loads issued just after its stores (a relay's
// one poll took 1.65 / 0.62 / 1.18 / 0.42 us after q, o, h and x, the time
// to stream the 12.6 / 6.3 / 8.4 / 4.2 MB issued then), so the loads are
// spread over the exchange instead of issued as one burst.
template <int ROWS, int CPL, bool GATED>
struct Wts {
    u32x4 v[GATED ? 2 * ROWS : ROWS][CPL];
};

template <int ROWS, int CPL, bool GATED, int PACE>
__device__ __forceinline__ void load_wts(Wts<ROWS, CPL, GATED> &w, const uint16_t *b, const uint16_t *b2, int row0,
                                         int nrows, int lane) {
    constexpr int K = 512 * CPL;
    const __amdgpu_buffer_rsrc_t rb = rsrc(b, (size_t)nrows * K * 2);
    const __amdgpu_buffer_rsrc_t rb2 = rsrc(GATED ? b2 : b, (size_t)nrows * K * 2);
#pragma unroll
    for (int r = 0; r < ROWS; r++)
#pragma unroll
        for (int j = 0; j < CPL; j++) {
            const uint32_t off = (uint32_t)(row0 + r) * (uint32_t)(K * 2) + (uint32_t)(lane + WAVE * j) * 16u;
            w.v[r][j] = __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, AUX_NT);
            if (PACE > 0) __builtin_amdgcn_s_sleep(PACE);
            if constexpr (GATED) {
                w.v[ROWS + r][j] = __builtin_amdgcn_raw_buffer_load_b128(rb2, off, 0, AUX_NT);
                if (PACE > 0) __builtin_amdgcn_s_sleep(PACE);
            }
        }
}

// rows row0 .. row0+ROWS-1 of one GEMV against the bf16 input in LDS: lane r
// returns row r's output (silu(gate) * up when GATED), other lanes garbage
template <int ROWS, int CPL, bool GATED>
__device__ __forceinline__ float gemv_rows(const Wts<ROWS, CPL, GATED> &w, const uint32_t *act, int lane) {
    constexpr int NB = GATED ? 2 * ROWS : ROWS;
    u32x4 xc[CPL];
#pragma unroll
    for (int j = 0; j < CPL; j++) xc[j] = reinterpret_cast<const u32x4 *>(act)[lane + WAVE * j];
    float acc[NB];
#pragma unroll
    for (int r = 0; r < NB; r++) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) s = bf16_dot2(w.v[r][j][e], xc[j][e], s);
        acc[r] = s;
    }
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
    return GATED ? silu_mul(tot, up) : tot;
}

// ---- poller wave -------------------------------------------------------------
#define PS_RELAYS 8                  // relay workgroups per XCD (of 32)
#define PS_XCDS 8
// s_sleep units (64 clocks) a relay waits after the stage's barrier before
// its first poll: polls that reach the words before their producers' stores
// slow the exchange down.  Measured on MI355X, the 112 layer GEMVs with
// unpaced weight loads: 333 us polling at once, 296 / 293 / 292 / 308 / 340
// us after 8 / 16 / 32 / 48 / 64 units (sleeping between polls instead: 341
// us); with the paced loads (PACE_*) 287 / 286 / 286 us after 20 / 24 / 28
#define PS_PRE 24
// relay poll: wait until the VP words of src carry `tag` (agent-scope
// loads, two words per 16-byte piece, lane l takes pieces l, l + 64, ...;
// bounded); d receives the pieces
template <int VP, int NL>
__device__ __forceinline__ void relay_wait(const uint64_t *src, unsigned tag, u32x4 (&d)[NL], unsigned *state,
                                           int lane, bool &gave_up) {
    static_assert(VP % 2 == 0 && NL == (VP + 127) / 128 && NL <= 32, "relay parts");
    const __amdgpu_buffer_rsrc_t rs = rsrc(src, (size_t)VP * 8);
    uint32_t ready = 0;
#pragma unroll
    for (int i = 0; i < NL; i++) {                 // lanes past the part: nothing to wait for
        d[i] = u32x4{0u, 0u, 0u, 0u};
        if ((uint32_t)(lane + WAVE * i) * 16u >= (uint32_t)VP * 8u) ready |= 1u << i;
    }
    const uint32_t all = (NL >= 32) ? 0xFFFFFFFFu : ((1u << NL) - 1u);
    __builtin_amdgcn_s_sleep(PS_PRE);
    for (int spin = 0;; spin++) {
#pragma unroll
        for (int i = 0; i < NL; i++)
            if (!(ready >> i & 1u))
                d[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, (uint32_t)(lane + WAVE * i) * 16u, 0, AUX_SC1);
#pragma unroll
        for (int i = 0; i < NL; i++)
            if (d[i].y == tag && d[i].w == tag) ready |= 1u << i;
        if (__all(ready == all)) break;
        if (gave_up || spin >= PS_SPIN) {
            if (lane == 0) atomicOr(state + 1, 1u);
            gave_up = true;
            break;
        }
    }
}
// the VP words of relay_wait into dst as packed bf16 pairs (pair q = words
// 2q, 2q+1, RNE); then, once the stores are acknowledged by the XCD's L2,
// `tag` into flag[r]
template <int VP, int NL>
__device__ __forceinline__ void relay_put_pairs(const u32x4 (&d)[NL], uint32_t *dst, unsigned *flag, int r,
                                                unsigned tag, int lane) {
    const __amdgpu_buffer_rsrc_t rd = rsrc(dst, (size_t)VP * 2);
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const uint32_t q = (uint32_t)(lane + WAVE * i);
        if (q * 16u < (uint32_t)VP * 8u)
            __builtin_amdgcn_raw_buffer_store_b32(pack_bf16x2(__uint_as_float(d[i].x), __uint_as_float(d[i].z)), rd,
                                                  q * 4u, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0);                // the wave's pairs are in the XCD's L2 ...
    if (lane == 0)                                // ... before its flag
        __builtin_amdgcn_raw_buffer_store_b32(tag, rsrc(flag, PS_RELAYS * 4), (uint32_t)r * 4u, 0, 0);
}
// the same as fp32 words (word q = value of source word q)
template <int VP, int NL>
__device__ __forceinline__ void relay_put_f32(const u32x4 (&d)[NL], float *dst, unsigned *flag, int r, unsigned tag,
                                              int lane) {
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    const __amdgpu_buffer_rsrc_t rd = rsrc(dst, (size_t)VP * 4);
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const uint32_t q = (uint32_t)(lane + WAVE * i);
        if (q * 16u < (uint32_t)VP * 8u) __builtin_amdgcn_raw_buffer_store_b64(u32x2{d[i].x, d[i].z}, rd, q * 8u, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0);
    if (lane == 0) __builtin_amdgcn_raw_buffer_store_b32(tag, rsrc(flag, PS_RELAYS * 4), (uint32_t)r * 4u, 0, 0);
}
// wait until the PS_RELAYS flags of a stage carry `tag` (bounded)
__device__ __forceinline__ void wait_flags(const unsigned *flag, unsigned tag, unsigned *state, int lane,
                                           bool &gave_up) {
    for (int spin = 0;; spin++) {
        const unsigned f =
            lane < PS_RELAYS ? __hip_atomic_load(flag + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : tag;
        if (__all(f == tag)) break;
        if (gave_up || spin >= PS_SPIN) {
            if (lane == 0) atomicOr(state + 1, 1u);
            gave_up = true;
            break;
        }
    }
}

#endif
