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
#include <string.h>

#include "hip_shim.h"
#include "persist_common.h"

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

// relay part r: wait until the V / PS_RELAYS words of part r of src carry
// `tag`, store them into dst as packed bf16 pairs (pair q of the part =
// words 2q, 2q+1, RNE), wait for the stores, then store `tag` in flag[r]
template <int V>
__device__ __forceinline__ void relay_copy(const uint64_t *src, uint32_t *dst, unsigned *flag, unsigned tag, int r,
                                           unsigned *state, int lane, bool &gave_up) {
    constexpr int VP = V / PS_RELAYS, NL = (VP + 127) / 128;
    static_assert(V % PS_RELAYS == 0, "relay parts");
    u32x4 d[NL];
    relay_wait<VP>(src + (size_t)r * VP, tag, d, state, lane, gave_up);
    relay_put_pairs<VP>(d, dst + (size_t)r * (VP / 2), flag, r, tag, lane);
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
    memset(&a, 0, sizeof a);          // no stray stack bytes in the kernel arguments' padding
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
