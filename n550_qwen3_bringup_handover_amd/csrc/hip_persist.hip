// Persistent decode step of the M = 1 GEMV set on CDNA4 (gfx950): the 4 x L
// dependent GEMVs of L decoder layers (fused q|k|v 1024 -> 4096, o 2048 ->
// 1024 on the q part, fused gate|up 1024 -> 2 x 3072 with silu(gate) * up,
// down 3072 -> 1024; fpga_bringup/src/src/qwen3.c:477-540 calls them as
// separate qwen3_gemm calls) in one launch instead of 4 x L.
//
// Why: each GEMV streams 4-12 MB of weights, which at ~6.5 TB/s takes
// 0.6-1.9 us, while a dependent kernel launch costs ~1.6 us on MI355X and
// cannot start streaming its weights before its predecessor has finished.
// Here every workgroup stays resident for the whole step and loads the next
// GEMV's weights while it waits for that GEMV's input, so the weight stream
// overlaps the exchange of activations between GEMVs.
//
// Layout of one launch: 256 workgroups (one per CU), each 4 compute waves
// and 1 poller wave.  Stage s of layer l has N output rows split evenly over
// the 1024 compute waves (4, 1, 3 (gate and up) and 1 rows per wave).  A
// compute wave holds its rows' weights in registers (lane l owns the
// 16-byte chunks l, l+64, ... of each row, as k_gemv1 does, so every output
// is the same sum in the same order and bit-identical to the per-call GEMV
// path), issues the next stage's weight loads, then waits at the workgroup
// barrier for the stage's input.
//
// Activations leave the compute waves as 64-bit words {fp32 value, tag}
// written with agent-scope (sc1) stores; the tag is the launch's epoch, so a
// word is valid exactly when its tag matches and no counter or cache flush
// is needed (a 64-bit access is single-copy atomic).  Only the poller wave
// of a workgroup waits for a stage's input (below); every wait is bounded:
// after PS_SPIN rounds it records an error and goes on, so every wave always
// finishes.  The input reaches an LDS buffer as bf16 pairs (RNE) and the
// poller joins the barrier.  The compute waves' memory counter then holds
// only weight loads, so waiting for one stage's weights never waits for the
// input, and the poll never waits for the weights.  LDS holds two input
// buffers: stage s reads buffer s % 2 while the poller fills buffer
// (s + 1) % 2; one barrier per stage separates them.
//
// Relays: reading words that another XCD has just written is slow when all
// 256 workgroups poll them (measured on MI355X: 2.2-3.1 us from the last
// store to the median poll).  So the words cross the XCD boundary once per
// XCD: at launch, the first PS_RELAYS workgroups on each XCD (an
// agent-scope ticket per XCD, the XCD read from HW_REG_XCC_ID) become its
// relays.  Relay r polls part r of every stage's words from the exchange,
// stores the part into its XCD's copy as packed bf16 pairs (the LDS format),
// waits for those stores to be acknowledged by the XCD's L2 and then stores
// the launch's epoch into its flag for the stage.  Every workgroup of the
// XCD, relays included, polls the stage's PS_RELAYS flags (32 bytes) and
// then reads the copy once -- all inside the XCD's L2.  Measured on MI355X,
// the 112 layer GEMVs: 412 us with every workgroup polling the exchange,
// 366-369 us with the relays' copies polled word by word (tagged), 332-333
// us with flags and bf16 copies, 292-294 us when the relays' first poll of a
// stage waits ~0.85 us (PS_PRE), 284 us with the weight prefetch paced
// (PACE_*), against ~350 us as per-call launches.
// A workgroup on an XCD with no relay, or a part no relay took, can only
// make the bounded polls give up with the error flag set.
//
// Residency: the 256 workgroups must be resident together (each waits for
// the others' outputs).  The host checks the occupancy (one workgroup of
// PS_THREADS threads per CU on all 256 CUs); the bounded polls guarantee
// termination even if another stream's kernels delayed a workgroup, with
// the error flag set.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hip_shim.h"

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define WAVE 64
#define PS_CWAVES 4                          // compute waves per workgroup
#define PS_THREADS ((PS_CWAVES + 1) * WAVE)  // + the poller wave
#define PS_BLOCKS 256
#define PS_GW (PS_BLOCKS * PS_CWAVES)        // compute waves of a launch
#define PS_SPIN (1 << 15)                    // poll rounds before giving up (~30 ms)
#define PS_LDS_U32 1536                      // one input buffer: 3072 bf16 values

#define H_DIM 1024
#define QKV_N 4096
#define Q_N 2048
#define I_N 3072

// per-layer fp32 outputs: q|k|v (4096), o (1024), h (3072), x (1024)
#define OUT_QKV 0
#define OUT_O 4096
#define OUT_H 5120
#define OUT_X 8192
#define OUT_LD 9216
// per-layer exchange slots of XCH_LD words: q (2048), o (1024), h (3072), x (1024)
#define XCH_LD 3072

// s_sleep units between consecutive weight loads of a stage's prefetch (load_wts).
// Measured on MI355X, the 112 layer GEMVs with the relays' first poll after
// 24 units: 293 us unpaced, 289 / 286 / 286 us at 3 / 4 / 5 units everywhere,
// 284 us at these (8 units everywhere: 319 us, the waves reach the barrier late)
#define PACE_QKV 4
#define PACE_O 3
#define PACE_GU 5
#define PACE_D 3

#define PS_MAX_LAYERS 32
struct PersistArgs {
    // per layer: q|k|v, o, gate, up, down (row-major bf16).  Held in the kernel
    // arguments, so each layer's pointers come from scalar loads: a pointer
    // fetched by a vector load would make every weight load wait for it
    // (the memory counter is in order) and would not be known to be uniform
    const uint16_t *w[PS_MAX_LAYERS][5];
    const float *x0;            // input of layer 0 (1024 fp32)
    float *out;                 // [layers][OUT_LD]
    uint64_t *xch;              // [layers][4][XCH_LD] exchange words
    unsigned *state;            // [0] epoch of the last launch, [1] error flags (1 = poll gave up),
                                // [2] arrivals, [4 + x] relay tickets of XCD x
    uint32_t *relay;            // [8 XCDs][PS_MAX_LAYERS * 4][XCH_LD / 2]: each XCD's copy, bf16 pairs
    unsigned *flags;            // [8 XCDs][PS_MAX_LAYERS * 4][PS_RELAYS]: epoch of each relay part copied
    int layers;
};

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

// lane r < ROWS writes row row0 + r: fp32 output, and (xch set) its
// exchange word {value, tag}
template <int ROWS>
__device__ __forceinline__ void put_rows(float v, float *out, uint64_t *xch, int row0, unsigned tag, int lane) {
    if (lane < ROWS) {
        out[row0 + lane] = v;
        if (xch) {
            const uint64_t word = ((uint64_t)tag << 32) | __float_as_uint(v);
            __hip_atomic_store(xch + row0 + lane, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
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
// relay part r: wait until the V / PS_RELAYS words of part r of src carry
// `tag` (agent-scope loads, two words per 16-byte load; bounded), store them
// into dst as packed bf16 pairs (pair q of the part = words 2q, 2q+1, RNE),
// wait for the stores, then store `tag` in flag[r]
template <int V>
__device__ __forceinline__ void relay_copy(const uint64_t *src, uint32_t *dst, unsigned *flag, unsigned tag, int r,
                                           unsigned *state, int lane, bool &gave_up) {
    constexpr int VP = V / PS_RELAYS, NL = (VP + 127) / 128;   // words of a part, 16-byte loads per lane
    static_assert(V % PS_RELAYS == 0 && VP % 2 == 0 && NL <= 32, "relay parts");
    const __amdgpu_buffer_rsrc_t rs = rsrc(src + (size_t)r * VP, (size_t)VP * 8);
    u32x4 d[NL];
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
    const __amdgpu_buffer_rsrc_t rd = rsrc(dst + (size_t)r * (VP / 2), (size_t)VP * 2);
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

// V words' copy on this XCD: wait until the PS_RELAYS flags of the stage
// carry `tag` (bounded), then read the V / 2 bf16 pairs into act
template <int V>
__device__ __forceinline__ void poll_copy(const uint32_t *src, const unsigned *flag, unsigned tag, uint32_t *act,
                                          unsigned *state, int lane, bool &gave_up) {
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
    constexpr int NQ = V / 8, NL = (NQ + WAVE - 1) / WAVE;   // 16-byte pieces of 4 pairs, per lane
    const __amdgpu_buffer_rsrc_t rs = rsrc(src, (size_t)V * 2);
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int q = lane + WAVE * i;
        if (q < NQ)
            reinterpret_cast<u32x4 *>(act)[q] = __builtin_amdgcn_raw_buffer_load_b128(rs, (uint32_t)q * 16u, 0, AUX_SC1);
    }
}

// the first layer's input: plain fp32, written before the launch
__device__ __forceinline__ void load_input(const float *x0, uint32_t *act, int lane) {
    const __amdgpu_buffer_rsrc_t rx = rsrc(x0, H_DIM * 4);
#pragma unroll
    for (int i = 0; i < H_DIM / (4 * WAVE); i++) {
        const f32x4 v = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      rx, (uint32_t)(lane + WAVE * i) * 16u, 0, 0));
        act[2 * (lane + WAVE * i)] = pack_bf16x2(v.x, v.y);
        act[2 * (lane + WAVE * i) + 1] = pack_bf16x2(v.z, v.w);
    }
}

__global__ __launch_bounds__(PS_THREADS, 1) void k_decode_persist(PersistArgs p) {
    __shared__ __align__(16) uint32_t act[2][PS_LDS_U32];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const unsigned tag = __hip_atomic_load(p.state, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    // this workgroup's XCD and, for the first PS_RELAYS to arrive there, its relay part
    __shared__ int s_xcd, s_part;
    if (tid == 0) {
        unsigned xr;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xr));
        const int xcd = (int)(xr & (PS_XCDS - 1));
        const unsigned t = __hip_atomic_fetch_add(p.state + 4 + xcd, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_xcd = xcd;
        s_part = t < PS_RELAYS ? (int)t : -1;
    }
    __syncthreads();

    if (wave == PS_CWAVES) {
        // ---- poller: one input per stage, then the barrier -----------------
        bool gave_up = false;
        const int part = s_part;
        // this XCD's copy (bf16 pairs, XCH_LD / 2 per stage slot) and flags
        uint32_t *const copy = p.relay + (size_t)s_xcd * PS_MAX_LAYERS * 4 * (XCH_LD / 2);
        unsigned *const flags = p.flags + (size_t)s_xcd * PS_MAX_LAYERS * 4 * PS_RELAYS;
        auto slot = [&](int si) { return copy + (size_t)si * (XCH_LD / 2); };
        auto flag = [&](int si) { return flags + (size_t)si * PS_RELAYS; };
        for (int l = 0; l < p.layers; l++) {
            const uint64_t *x = p.xch + (size_t)l * 4 * XCH_LD;      // the exchange words of layer l
            const int si = 4 * l;                                     // slots si .. si+3: q, o, h, x
            if (l == 0) {
                load_input(p.x0, act[0], lane);
            } else {                                                  // x of layer l-1
                if (part >= 0) relay_copy<H_DIM>(x - XCH_LD, slot(si - 1), flag(si - 1), tag, part, p.state, lane, gave_up);
                poll_copy<H_DIM>(slot(si - 1), flag(si - 1), tag, act[0], p.state, lane, gave_up);
            }
            __syncthreads();
            if (part >= 0) relay_copy<Q_N>(x, slot(si), flag(si), tag, part, p.state, lane, gave_up);     // q
            poll_copy<Q_N>(slot(si), flag(si), tag, act[1], p.state, lane, gave_up);
            __syncthreads();
            if (part >= 0) relay_copy<H_DIM>(x + XCH_LD, slot(si + 1), flag(si + 1), tag, part, p.state, lane, gave_up);   // o
            poll_copy<H_DIM>(slot(si + 1), flag(si + 1), tag, act[0], p.state, lane, gave_up);
            __syncthreads();
            if (part >= 0) relay_copy<I_N>(x + 2 * XCH_LD, slot(si + 2), flag(si + 2), tag, part, p.state, lane, gave_up);   // h
            poll_copy<I_N>(slot(si + 2), flag(si + 2), tag, act[1], p.state, lane, gave_up);
            __syncthreads();
        }
    } else {
        // ---- compute waves ------------------------------------------------
        const int gw = blockIdx.x * PS_CWAVES + wave;     // 0 .. 1023
        Wts<4, 2, false> wa;    // q|k|v: rows 4gw .. 4gw+3 of 4096, K 1024
        Wts<1, 4, false> wb;    // o: row gw of 1024, K 2048
        Wts<3, 2, true> wc;     // gate|up: rows 3gw .. 3gw+2 of 3072, K 1024
        Wts<1, 6, false> wd;    // down: row gw of 1024, K 3072
        load_wts<4, 2, false, 0>(wa, p.w[0][0], nullptr, 4 * gw, QKV_N, lane);
        for (int l = 0; l < p.layers; l++) {
            const uint16_t *const *wl = p.w[l];
            float *out = p.out + (size_t)l * OUT_LD;
            uint64_t *x = p.xch + (size_t)l * 4 * XCH_LD;
            load_wts<1, 4, false, PACE_O>(wb, wl[1], nullptr, gw, H_DIM, lane);
            __syncthreads();
            float v = gemv_rows(wa, act[0], lane);
            put_rows<4>(v, out + OUT_QKV, 4 * gw < Q_N ? x : nullptr, 4 * gw, tag, lane);

            load_wts<3, 2, true, PACE_GU>(wc, wl[2], wl[3], 3 * gw, I_N, lane);
            __syncthreads();
            v = gemv_rows(wb, act[1], lane);
            put_rows<1>(v, out + OUT_O, x + XCH_LD, gw, tag, lane);

            load_wts<1, 6, false, PACE_D>(wd, wl[4], nullptr, gw, H_DIM, lane);
            __syncthreads();
            v = gemv_rows(wc, act[0], lane);
            put_rows<3>(v, out + OUT_H, x + 2 * XCH_LD, 3 * gw, tag, lane);

            // the next layer's q|k|v, unconditionally: after the last layer the
            // resource is empty (its loads read zeros and touch no memory), so
            // the compiler counts the loads exactly and stage D waits for its
            // own weights only
            const bool more = l + 1 < p.layers;
            load_wts<4, 2, false, PACE_QKV>(wa, p.w[more ? l + 1 : l][0], nullptr, 4 * gw, more ? QKV_N : 0, lane);
            __syncthreads();
            v = gemv_rows(wd, act[1], lane);
            put_rows<1>(v, out + OUT_X, x + 3 * XCH_LD, gw, tag, lane);
        }
    }
    // the next launch's epoch is published by the last workgroup to finish
    // (an arrival count in state[2]): every workgroup read this launch's
    // epoch before it arrives, so none -- not even one that started late,
    // after another gave up waiting -- can tag its words with the next one
    if (tid == 0) {
        const unsigned arrived =
            __hip_atomic_fetch_add(p.state + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (arrived == gridDim.x - 1) {
            for (int xd = 0; xd < PS_XCDS; xd++)      // the relay tickets, for the next launch
                __hip_atomic_store(p.state + 4 + xd, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(p.state + 2, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(p.state, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ---- host side ------------------------------------------------------------------
static uint64_t *g_xch = nullptr;     // [PS_MAX_LAYERS][4][XCH_LD] exchange words
static unsigned *g_state = nullptr;   // epoch, error flags, arrivals, relay tickets
static uint32_t *g_relay = nullptr;   // [PS_XCDS] bf16 copies of the exchange words
static unsigned *g_flags = nullptr;   // their relay flags
static int g_ps_ok = 0;               // 1 = the device keeps the grid resident

// at library init (device current): the exchange words start at tag 0,
// which no launch uses
extern "C" int qh_persist_init(void) {
    int dev = 0, cus = 0, nb = 0;
    g_ps_ok = hipGetDevice(&dev) == hipSuccess &&
              hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
              hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_decode_persist, PS_THREADS, 0) == hipSuccess &&
              cus == PS_BLOCKS && nb >= 1;
    (void)hipGetLastError();
    const size_t xb = (size_t)PS_MAX_LAYERS * 4 * XCH_LD * sizeof(uint64_t);
    const size_t fb = (size_t)PS_XCDS * PS_MAX_LAYERS * 4 * PS_RELAYS * sizeof(unsigned);
    if (hipMalloc((void **)&g_xch, xb) != hipSuccess || hipMalloc((void **)&g_state, 64) != hipSuccess ||
        hipMalloc((void **)&g_relay, PS_XCDS * xb / 4) != hipSuccess ||
        hipMemset(g_relay, 0, PS_XCDS * xb / 4) != hipSuccess ||
        hipMalloc((void **)&g_flags, fb) != hipSuccess || hipMemset(g_flags, 0, fb) != hipSuccess ||
        hipMemset(g_xch, 0, xb) != hipSuccess || hipMemset(g_state, 0, 64) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
        (void)hipGetLastError();
        return QH_ENOMEM;
    }
    return QH_OK;
}

extern "C" void qh_persist_shutdown(void) {
    (void)hipFree(g_xch);
    (void)hipFree(g_state);
    (void)hipFree(g_relay);
    (void)hipFree(g_flags);
    g_xch = nullptr;
    g_state = nullptr;
    g_relay = nullptr;
    g_flags = nullptr;
    g_ps_ok = 0;
}

extern "C" int qh_persist_supported(void) { return g_ps_ok; }
extern "C" int qh_persist_out_ld(void) { return OUT_LD; }

extern "C" int qh_decode_persist(const uint16_t *const *w, const float *x0_d, float *out_d, int layers) {
    if (!w || !x0_d || !out_d || layers < 1) return QH_EINVAL;
    if (layers > PS_MAX_LAYERS) return QH_ETOOBIG;
    if (!g_xch || !g_ps_ok) return QH_ENODEV;
    PersistArgs a;
    for (int l = 0; l < PS_MAX_LAYERS; l++)
        for (int k = 0; k < 5; k++) {
            a.w[l][k] = l < layers ? w[5 * l + k] : nullptr;
            if (l < layers && !a.w[l][k]) return QH_EINVAL;
        }
    a.x0 = x0_d;
    a.out = out_d;
    a.xch = g_xch;
    a.state = g_state;
    a.relay = g_relay;
    a.flags = g_flags;
    a.layers = layers;
    hipLaunchKernelGGL(k_decode_persist, dim3(PS_BLOCKS), dim3(PS_THREADS), 0, (hipStream_t)qh_stream(), a);
    return hipGetLastError() == hipSuccess ? QH_OK : QH_ELAUNCH;
}

// error flags raised by launches since the last call (synchronises the stream)
extern "C" int qh_persist_errors(unsigned *flags) {
    if (!g_state || !flags) return QH_ESTATE;
    unsigned h[2] = {0u, 0u};
    if (hipStreamSynchronize((hipStream_t)qh_stream()) != hipSuccess ||
        hipMemcpy(h, g_state, sizeof h, hipMemcpyDeviceToHost) != hipSuccess) {
        (void)hipGetLastError();
        return QH_ERUNTIME;
    }
    *flags = h[1];
    if (h[1] && hipMemset(g_state + 1, 0, sizeof(unsigned)) != hipSuccess) {
        (void)hipGetLastError();
        return QH_ERUNTIME;
    }
    return QH_OK;
}
