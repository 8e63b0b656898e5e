// CDNA4 (gfx950) GEMM / GEMV library for the Qwen3-0.6B projection GEMMs:
// the host side of the shim (device and stream, workspaces, the plan table
// that picks a kernel per M x K x N, the launchers, graph capture) and the
// extern "C" entry points.  Semantics follow the reference GEMM plug-in
// (fpga_bringup/src/src/kernels.h:44-57): C[M,N] = A[M,K] . B[N,K]^T with A
// fp32 row-major, B bf16 bits row-major [out, in], C fp32 row-major,
// C overwritten.  A is rounded to bf16 with round-to-nearest-even on the
// load path (the AME kernel does the same, kernels_ame.c:219-236), products
// of two bf16 values are exact in fp32, and accumulation is fp32.
//
// The kernels live in headers by family, all compiled into this unit:
//   gemm_common.h      types, constants, bf16 / wave-reduction / SiLU helpers
//   gemv_kernels.h     M = 1 decode GEMV (fused prologues), M <= 4, M <= 16
//   tile_kernels.h     tiled MFMA GEMMs for M > 4: double-buffered tiles,
//                      the global_load_lds ring, the large tiles
//   misc_kernels.h     weight re-layout, A rounding, argmax, copies
//   small_m_kernels.h  decode-batch GEMMs, 5 <= M <= 64: weight-streaming,
//                      skinny, narrow, wide (lm_head), 16-row
#include "gemm_common.h"
#include "gemv_kernels.h"
#include "tile_kernels.h"
#include "misc_kernels.h"
#include "small_m_kernels.h"

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
static int g_last_plan = 0;        // the plan the last GEMM call launched (PLAN_AUTO: none yet)
#define QH_MAX_GRAPHS 16
static hipGraphExec_t g_graph_exec[QH_MAX_GRAPHS];
static void *g_graph_ws[QH_MAX_GRAPHS][2];   // library workspaces each graph uses (abf, part)
// Workspaces replaced while a graph exists: a captured graph keeps the device
// addresses it was recorded with, so a grown workspace's old buffer stays
// allocated until no graph is left (or the library shuts down).
#define QH_MAX_RETIRED 64
static void *g_retired[QH_MAX_RETIRED];
static int g_n_retired = 0;
static void free_retired(void);
static int g_capturing = 0;
static float *g_am_v = nullptr;   // argmax partials (allocated at init)
static int *g_am_i = nullptr;
static const int AM_BLOCKS = 1024;
// bf16 copy of an fp32 A for the large-tile GEMMs (grown outside graph capture)
static uint16_t *g_abf = nullptr;
static size_t g_abf_elems = 0;
static int g_cus = 256;            // compute units of the device (set at init)
#define PART_INIT_BYTES ((size_t)32 << 20)
static float *g_part = nullptr;    // K-slice sums of the skinny, stream and narrow kernels (grown on demand)
static size_t g_part_bytes = 0;
// tickets of the narrow kernel's K split, one per 32-column block: zero
// between calls (each call's last block resets the ones it used)
#define NARROW_CNT 2048
static unsigned *g_cnt = nullptr;
static const size_t ABF_INIT_ELEMS = (size_t)8192 * 3072;   // 48 MiB: M x K up to 8192 x 3072

// the no-allocation entry point's workspace (see qh_gemm_noalloc)
#define QH_SCRATCH_BYTES ((size_t)32 << 20)
__device__ __align__(256) unsigned char scratch[QH_SCRATCH_BYTES];
// its last NARROW_CNT words hold the narrow kernel's tickets (zeroed at init);
// the rest is the bf16 copy of A or the slice sums
#define QH_SCRATCH_WS_BYTES (QH_SCRATCH_BYTES - NARROW_CNT * sizeof(unsigned))
#define QH_MAX_DEVICES 64
static void *g_scratch_dev[QH_MAX_DEVICES];   // per device: its copy of `scratch`

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
    if (prop.multiProcessorCount > 0) g_cus = prop.multiProcessorCount;
    HCHECK(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking), QH_ERUNTIME);
    HCHECK(hipMalloc((void **)&g_am_v, AM_BLOCKS * sizeof(float)), QH_ENOMEM);
    HCHECK(hipMalloc((void **)&g_am_i, AM_BLOCKS * sizeof(int)), QH_ENOMEM);
    HCHECK(hipMalloc((void **)&g_abf, ABF_INIT_ELEMS * sizeof(uint16_t)), QH_ENOMEM);
    g_abf_elems = ABF_INIT_ELEMS;
    // split-K partials: 32 MiB covers the Qwen3-0.6B projection shapes up to M = 2048
    // (e.g. 4 slices x 1024 x 1024 fp32); grown outside graph capture if needed
    HCHECK(hipMalloc((void **)&g_part, PART_INIT_BYTES), QH_ENOMEM);
    g_part_bytes = PART_INIT_BYTES;
    HCHECK(hipMalloc((void **)&g_cnt, NARROW_CNT * sizeof(unsigned)), QH_ENOMEM);
    HCHECK(hipMemset(g_cnt, 0, NARROW_CNT * sizeof(unsigned)), QH_ERUNTIME);
    // the no-allocation entry point's workspace: this device's copy of the
    // file-scope array (device current here)
    if (device < QH_MAX_DEVICES && !g_scratch_dev[device])
        HCHECK(hipGetSymbolAddress(&g_scratch_dev[device], HIP_SYMBOL(scratch)), QH_ERUNTIME);
    if (device < QH_MAX_DEVICES)
        HCHECK(hipMemset((unsigned char *)g_scratch_dev[device] + QH_SCRATCH_WS_BYTES, 0,
                         NARROW_CNT * sizeof(unsigned)), QH_ERUNTIME);
    g_device = device;
    {
        const int rc = qh_persist_init();
        if (rc) return rc;
    }
    g_inited = 1;
    return QH_OK;
}

extern "C" void qh_shutdown(void) {
    if (!g_inited) return;
    (void)hipStreamSynchronize(g_stream);
    for (int i = 0; i < QH_MAX_GRAPHS; i++) {
        if (g_graph_exec[i]) { (void)hipGraphExecDestroy(g_graph_exec[i]); g_graph_exec[i] = nullptr; }
        g_graph_ws[i][0] = g_graph_ws[i][1] = nullptr;
    }
    free_retired();
    for (int i = 0; i < 64; i++)
        if (g_ev_made[i]) { (void)hipEventDestroy(g_ev[i]); g_ev_made[i] = 0; }
    (void)hipFree(g_abf);
    g_abf = nullptr;
    g_abf_elems = 0;
    (void)hipFree(g_part);
    g_part = nullptr;
    g_part_bytes = 0;
    (void)hipFree(g_cnt);
    g_cnt = nullptr;
    (void)hipFree(g_am_v);
    (void)hipFree(g_am_i);
    g_am_v = nullptr;
    g_am_i = nullptr;
    qh_persist_shutdown();
    qm_persist_shutdown();
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
// Every plan below is one that choose_plan / choose_bf16a_plan returns, or the
// fall-back (mfma64x64) taken when a plan's alignment or size conditions fail.
enum {
    PLAN_AUTO = 0,
    PLAN_GEMV = 1,             // M <= 4: HBM-streaming GEMV
    PLAN_T128x128 = 2,         // register-staged 16x16x32 MFMA tiles (K % 8 == 0)
    PLAN_T64x128 = 3,
    PLAN_T64x64 = 4,           // the fall-back
    PLAN_T32x128 = 5,
    PLAN_T16x64 = 6,
    PLAN_SCALAR64 = 7,         // MFMA 64x64 with element-wise loads (any K, any alignment)
    // software-pipelined LDS ring (K % BK == 0): tile, k per stage, LDS stages
    PLAN_P32x64k128s4 = 8,
    PLAN_P32x64k64s4 = 9,
    PLAN_P64x64k64s3 = 10,
    // large tiles, 32x32x16 MFMA, fp32 A rounded on the load path (K % BK == 0)
    PLAN_X128x128 = 11,        // BK 64
    PLAN_X256x256 = 12,        // BK 32
    PLAN_X64x128 = 13,         // BK 64
    // A rounded to bf16 by one extra pass into the workspace, then bf16 x bf16
    PLAN_XB256x256k32 = 14,
    PLAN_XB128x128 = 15,       // BK 64
    PLAN_XB256x256s1 = 16,     // BK 64, one register set
    // weight-streaming MFMA GEMM for M <= 64 (K % 256 == 0): KS chosen per
    // shape, or forced (wave k range 32*KS; K / (256*KS) block slices)
    PLAN_STREAM = 17,
    PLAN_STREAM_KS1 = 18,
    PLAN_STREAM_KS2 = 19,
    PLAN_STREAM_KS4 = 20,
    PLAN_STREAM_KS8 = 21,
    // skinny M <= 64: A slice staged in LDS, K split over blocks (K % 64 == 0)
    PLAN_SKINNY = 22,
    // narrow M <= 64 (K % 128 == 0): 32-column blocks, K split over blocks and
    // the slices added inside the same launch
    PLAN_NARROW = 23,
    // wide M <= 64 (K % 512 == 0, A within 128 KB of LDS as bf16): A resident
    // in LDS, each wave streaming its own 32-column tiles
    PLAN_WIDE = 24,
    // 5 <= M <= 16, K <= 1024: every weight row read once, dot2 with A from registers
    PLAN_GEMV16 = 25,
    // large-tile kernel on 64 x 64 tiles, BK 64, three register sets (three
    // stages in flight; not gated): two blocks per CU
    PLAN_X64x64s3 = 26,
    // M <= 16, K = 1024, 2048 or 3072: 16-column blocks, K split over the
    // block's waves, v_mfma_f32_16x16x32_bf16 (not gated)
    PLAN_M16 = 27,
    PLAN_COUNT = 28
};
static const char *k_plan_names[PLAN_COUNT] = {
    "auto", "gemv", "mfma128x128", "mfma64x128", "mfma64x64", "mfma32x128", "mfma16x64", "mfma64x64-scalar",
    "pipe32x64k128s4", "pipe32x64k64s4", "pipe64x64k64s3",
    "xl128x128", "xl256x256", "xl64x128",
    "xb256x256k32", "xb128x128", "xb256x256s1",
    "stream", "stream-ks1", "stream-ks2", "stream-ks4", "stream-ks8", "skinny", "narrow", "wide",
    "gemv16", "xl64x64s3", "m16"};
static inline bool is_pipe_plan(int p) { return p >= PLAN_P32x64k128s4 && p <= PLAN_P64x64k64s3; }
static inline bool is_xl_plan(int p) {
    return (p >= PLAN_X128x128 && p <= PLAN_XB256x256s1) || p == PLAN_X64x64s3;
}
static inline bool is_xb_plan(int p) { return p >= PLAN_XB256x256k32 && p <= PLAN_XB256x256s1; }
static inline bool is_stream_plan(int p) { return p >= PLAN_STREAM && p <= PLAN_STREAM_KS8; }
static inline bool is_narrow_plan(int p) { return p == PLAN_NARROW; }
static inline int stream_mt(int M) { return M <= 16 ? 1 : M <= 32 ? 2 : 4; }
// the stream kernel's limits: M <= 64, whole 256-deep block slices, byte
// offsets below 2 GiB (its out-of-range marker), 16-byte aligned rows
static inline bool stream_fits(int M, int K, int N) {
    return M >= 1 && M <= 64 && K > 0 && K % 256 == 0 && (size_t)M * K * 4 < (1ull << 31) &&
           (size_t)N * K * 2 < (1ull << 31);
}
// the 16-row kernel's limits: M <= 16, K one of its instantiations, byte
// offsets below 2 GiB
static inline bool m16_fits(int M, int K, int N) {
    return M >= 1 && M <= 16 && (K == 1024 || K == 2048 || K == 3072) && N >= 1 &&
           (size_t)N * K * 2 < (1ull << 31);
}
// the 16-row kernel's column tiles per block: two once one-tile blocks would
// outnumber the CUs (halves the blocks' re-reads of A; measured on MI355X,
// graph-replayed, 16 x 1024 x 8192 / 16384: 5.8 / 10.1 -> 4.5 / 7.7 us, and
// 16 x 1024 x 4096: 3.8 -> 4.0 us the other way)
static inline int m16_ct(int K, int N) { return K <= 2048 && (N + 15) / 16 > g_cus ? 2 : 1; }
// the narrow kernel's limits: M <= 256, whole 128-deep slices, whole quads
// of columns, byte offsets below 2 GiB; its geometry search also keeps the
// tiles (row slab x 32 columns, a ticket each) within NARROW_CNT
static inline bool narrow_fits(int M, int K, int N) {
    return M >= 1 && M <= 256 && K > 0 && K % 128 == 0 && N % 4 == 0 && (N + NARROW_COLS - 1) / NARROW_COLS <= NARROW_CNT &&
           (size_t)M * K * 4 < (1ull << 31) && (size_t)N * K * 2 < (1ull << 31);
}
// the wide kernel's limits: M <= 64, K = 512 or 1024 (whole groups of
// WIDE_D chunks, instantiated depths), whole quads of columns, the bf16 rows
// of A within WIDE_A_BYTES, byte offsets below 2 GiB
static inline bool wide_fits(int M, int K, int N) {
    return M >= 1 && M <= 64 && N > 0 && N % 4 == 0 && (K == 512 || K == 1024) && (size_t)M * N * 4 < (1ull << 31) &&
           (size_t)16 * stream_mt(M) * K * 2 <= WIDE_A_BYTES && (size_t)M * K * 4 < (1ull << 31) &&
           (size_t)N * K * 2 < (1ull << 31);
}
// the GEMV-shaped kernel for M <= 16: K <= 1024 (two chunks per lane),
// byte offsets below 2 GiB
static inline bool gemv16_fits(int M, int K, int N) {
    return M >= 1 && M <= 16 && N > 0 && K > 0 && K % 8 == 0 && K <= 1024 && (size_t)M * K * 4 < (1ull << 31) &&
           (size_t)N * K * 2 < (1ull << 31);
}
// k steps of 32 per wave (KS must divide K/256, and the A fragments, 4*MT*KS
// registers, must fit in 64): no K split while there are >= 128 tiles of 16
// rows; else the largest KS whose slices still give >= 192 blocks (measured
// on MI355X: a split costs a reduction pass, ~2 us, but 64 blocks leave
// three quarters of the chip idle)
static int stream_ks(int M, int K, int N, int cus) {
    (void)cus;
    const int mt = stream_mt(M), kb = K / 256;
    const long ntiles = (N + 15) / 16;
    int smallest = 0;
    for (int ks = 8; ks >= 1; ks /= 2) {
        if (mt * ks > 16 || kb % ks) continue;
        const long blocks = ntiles * (kb / ks);
        if ((kb / ks == 1 && ntiles >= 128) || blocks >= 192) return ks;
        smallest = ks;
    }
    return smallest;
}
static inline int xl_bk(int p) { return (p == PLAN_X256x256 || p == PLAN_XB256x256k32) ? 32 : 64; }
static inline int pipe_bk(int p) { return p == PLAN_P32x64k128s4 ? 128 : 64; }

static inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// bf16-A shapes: 256 x 256 tiles when they fill the chip, else the smaller
// tiles (measured on MI355X for the Qwen3-0.6B projection shapes)
static int choose_bf16a_plan(int M, int K, int N, int gated) {
    (void)K;
    const int bno = gated ? 2 : 1;
    auto blocks = [&](int bm, int bn) {
        return (long)((M + bm - 1) / bm) * (long)((N + bn / bno - 1) / (bn / bno));
    };
    if (!gated && blocks(256, 256) >= 256) return PLAN_XB256x256k32;
    return PLAN_XB128x128;
}

static int choose_plan(int M, int K, int N, int gated, bool vec) {
    if (!vec) return PLAN_SCALAR64;
    // 2 <= M <= 16 (config 1's gate_proj, small decode batches): the 16-row
    // kernel, 16 or 32 columns per block and K split over its waves, where a
    // sweep of M 2..16 x K 1024..3072 x N 1024..16384 measured it fastest
    // (MI355X, graph-replayed per call: 16 x 1024 x 3072 3.3 us against 5.3 on
    // the GEMV-shaped kernel; 16 x 3072 x {1024, 3072} 5.5 / 5.9 against 6.3
    // on the narrow and 15.7 on the weight-streaming kernel; 4 x 2048 x 3072
    // 4.2 against 6.2 on the GEMV).  Not at N > 8192 with K >= 2048, where
    // every block re-reads all of A (the GEMV at M <= 4, the weight-streaming
    // kernel above: 16 x 2048 x 16384 17.6 against 18.4 us), nor at M = 2
    // with K = 2048, N <= 2048 or K = 3072, N > 4096, or at N > 8192, where
    // the GEMV is as fast or faster.
    if (!gated && M >= 2 && m16_fits(M, K, N) &&
        (M >= 4 ? (N <= 8192 || (K == 1024 && N <= 16384))
                : ((K == 1024 && N <= 8192) || (K == 2048 && N > 2048 && N <= 8192) ||
                   (K == 3072 && N <= 4096))))
        return PLAN_M16;
    // gated (gate|up + SiLU of a small decode batch) above M = 4: the same
    // kernel with the Wg and the Wu rows of 16 columns as a block's two tiles
    // (K <= 2048), where measured faster (graph-replayed: 16 x 1024 x 3072 3.7
    // us against 5.8 on the 32x64 ring tiles, 16 x 2048 x 3072 5.9 against
    // 7.9; not at N = 8192 beyond M = 8 or K = 1024; batched decode of 16 / 8
    // sequences 13.7k / 7.6k -> 14.5k / 8.1k tok/s).  At M <= 4 the GEMV stays:
    // alone the 16-row kernel was faster there too (4 x 1024 x 3072 3.6 against
    // 5.1 us), but decode of 4 sequences lost 1% with it.
    if (gated && M > 4 && K <= 2048 && m16_fits(M, K, N) &&
        (N <= 4096 || (K == 1024 && M <= 8 && N <= 8192)))
        return PLAN_M16;
    if (M <= 4 && (size_t)M * K * 4 <= 64 * 1024) return PLAN_GEMV;
    // 16 < M <= 64, not gated (every projection of a decode batch but
    // gate|up): the narrow kernel, 32-column blocks in row slabs with K split
    // over blocks where that fills the chip, the slices added in the same
    // launch (measured on MI355X, graph-replayed, M = 64: q|k|v 1024 -> 4096
    // 6.3 -> 4.7 us, q 6.0 -> 4.4, k 6.0 -> 5.4, o 9.7 -> 6.2, down 9.7 ->
    // 6.9, gate alone 6.0 -> 5.1; M = 32 and 48 alike).  Gated, its two weight
    // streams make it slower than the 32x64 tiles (64x1024x3072: 7.8 against
    // 6.3 us).
    if (!gated && narrow_fits(M, K, N) && M > 16 && M <= 64 && N >= 512 && N <= 4096 && K >= 1024 && K <= 4096)
        return PLAN_NARROW;
    // and at M <= 16 where it beats the stream and skinny kernels below
    // (16x3072x2048 7.7 -> 6.4 us)
    if (!gated && narrow_fits(M, K, N) && M <= 16 && K >= 2048 && K <= 4096 && N > 1024 && N <= 2048)
        return PLAN_NARROW;
    // 64 < M <= 256 (prefill chunks through the drop-in call, one projection
    // at a time), where its slabs beat the 32x64 tiles: N <= 1024 up to 128
    // rows, and N <= 2048 at K = 1024; K = 1024, N <= 1024 up to 256 rows
    // (measured on MI355X, graph-replayed, M = 128: k/v 1024 -> 1024 6.2 ->
    // 4.1 us, q 1024 -> 2048 6.3 -> 4.9, o 2048 -> 1024 9.8 -> 7.2, down 3072
    // -> 1024 13.3 -> 8.8; M = 256 k/v 6.2 -> 4.8; slower at N = 4096, at K =
    // 2048 with N = 2048, and above 128 rows at K >= 2048)
    if (!gated && narrow_fits(M, K, N) && M > 64 && K >= 1024 && K <= 3072 &&
        ((M <= 128 && (N <= 1024 || (K == 1024 && N <= 2048))) || (K == 1024 && N <= 1024)))
        return PLAN_NARROW;
    // the rest of them at M <= 64: the skinny kernel, A slices staged once
    // per block and K split over blocks, the slices added by a second launch
    // (measured on MI355X: 16x3072x1024 8.1 -> 5.5 us against the tiles); at
    // K = 1024 the slices' partial sums cost more than they save
    if (!gated && M <= 64 && K >= 2048 && K <= 4096 && K % 64 == 0 && N <= 2048 &&
        (size_t)M * K * 4 < (1ull << 31) && (size_t)N * K * 2 < (1ull << 31))
        return PLAN_SKINNY;
    // the tied lm_head of a decode batch (N very wide, K = 512 or 1024): the
    // wide kernel, A resident in LDS and every wave streaming its own tiles
    // (measured on MI355X, graph-replayed, 64 / 48 / 32 / 16 / 8 x 1024 x
    // 151936: 65.6 / 62.7 / 58.5 / 53.2 / 50.5 us against 79.0 / 72.2 / 66.9
    // / 60.1 / 55.9 on the weight-streaming kernel; at M = 64 it moves 311 MB
    // of weights in and 39 MB of C out, 5.3 TB/s of mixed traffic)
    if (!gated && N >= 32768 && wide_fits(M, K, N)) return PLAN_WIDE;
    // 5 <= M <= 16, K < 1024 (K = 1024 takes the 16-row kernel above): the
    // GEMV-shaped kernel, each weight row read once in 1 KB pieces and dot2
    // against A held in registers (measured on MI355X, graph-replayed, at K =
    // 1024 before the 16-row kernel: 16 x 1024 x {1024, 2048, 3072, 4096}
    // 3.5 / 3.7 / 4.8 / 4.9 us against 5.2 / 5.1 / 5.2 / 5.2 on the narrow and
    // weight-streaming kernels)
    if (!gated && gemv16_fits(M, K, N) && M >= 5 && N <= 4096) return PLAN_GEMV16;
    // the weight-streaming kernel for 5 <= M <= 16, and up to M = 32 where
    // N <= 2048 leaves the 32x64 tiles few blocks (measured on MI355X, e.g.
    // 16x1024x3072 5.7 vs 6.5 us, 16x3072x1024 7.7 vs 13.5 us); gated shapes
    // stay on the tiles, which hold both weight rows of a block in one pass
    if (!gated && stream_fits(M, K, N) && (M <= 16 || (M <= 32 && N <= 2048))) return PLAN_STREAM;
    // and for every M <= 64 when N is very wide and the wide kernel does not
    // fit (measured on MI355X, 64 / 48 / 32 x 1024 x 151936: 76-79 / 70-73 /
    // 62-63 us against 81-84 / 74-75 / 68-70 on the 64- and 32-row tiles)
    if (!gated && stream_fits(M, K, N) && N >= 32768) return PLAN_STREAM;
    const int bno = gated ? 2 : 1;   // gated tiles produce half as many output columns
    auto blocks = [&](int bm, int bn) {
        return (long)((M + bm - 1) / bm) * (long)((N + bn / bno - 1) / (bn / bno));
    };
    // Measured on MI355X (Qwen3-0.6B projection shapes, M = 16 .. 4096): the
    // software-pipelined 32x64 tile with 128-deep stages wins while its tiles
    // fit one round on the 256 CUs (it holds 128 KB of LDS, one block per
    // CU); with 64-deep stages (64 KB, two blocks per CU) up to two rounds;
    // larger grids and large M do better with the register-staged 64- and
    // 128-wide tiles.
    // Large-tile kernels (32x32x16 MFMA, two stages of loads in flight) win
    // from M = 1024 on, and at M = 512 wherever 128 x 128 tiles still give
    // half the chip a tile (fused q|k|v, gate|up): 256 x 256 when they fill
    // all 256 CUs, gate|up from M = 2048 with A rounded to bf16 by one pass
    // first, 128 x 128 otherwise.
    if (K % 64 == 0 && (size_t)M * K * 4 < (1ull << 32) && (size_t)N * K * 2 < (1ull << 32)) {
        // One round of 64 x 128 tiles (192 .. 256 of them, eight waves per
        // block in two k groups), else of 128 x 128 tiles from M = 512, else
        // of 64 x 64 tiles (measured on MI355X, graph-replayed: 512 x 1024 x
        // 4096 13.6 -> 11.7 us, 384 x 1024 x 4096 12.4 -> 10.8, 1024 x 1024 x
        // 2048 13.0 -> 11.4, 2048 x 2048 x 1024 21.9 -> 18.1, 2048 x 3072 x 1024
        // 30.2 -> 23.8 against the 64 x 64 tiles; 768 x 1024 x 4096 19.3 ->
        // 17.0 on 128 x 128; 256 / 192 x 1024 x 4096 10.3 / 9.6 -> 8.7 / 8.2
        // against the 32 x 64 ring tiles)
        if (!gated && M >= 256 && blocks(64, 128) >= 192 && blocks(64, 128) <= g_cus) return PLAN_X64x128;
        if (!gated && M >= 512 && blocks(128, 128) >= 192 && blocks(128, 128) <= g_cus) return PLAN_X128x128;
        if (!gated && M > 128 && blocks(64, 64) >= 192 && blocks(64, 64) <= g_cus) return PLAN_X64x64s3;
        // gated between 128 and 512 rows where 128 x 128 tiles would leave
        // half the chip idle, and between 512 and 1024: 64 x 128 tiles (256 x
        // 1024 x 3072: 15.3 -> 10.4 us against the 64 x 64 tiles; 768 / 1024
        // rows 25.6 / 26.7 -> 24.2 / 25.7 against 128 x 128)
        if (gated && M > 128 && blocks(128, 128) < 128 && blocks(64, 128) >= 128) return PLAN_X64x128;
        if (gated && M > 512 && M <= 1024) return PLAN_X64x128;
        // 64 x 64 tiles (two blocks per CU, three stages in flight) where they
        // make one or two rounds at K = 1024 (measured on MI355X: 512x1024x2048
        // 9.3 -> 8.2 us, 512x1024x4096 12.8 -> 12.2, 1024x1024x2048 12.4 -> 11.5,
        // 1024x1024x1024 8.5 -> 8.0; at 512x1024x1024 they lose, 7.6 vs 6.6)
        if (!gated && M >= 256 && M <= 1024 && K <= 1024 && blocks(64, 64) >= 256 && blocks(64, 64) <= 512)
            return PLAN_X64x64s3;
        // and for the K-heavy narrow shapes (o, down) at M = 1024 .. 2048, where
        // the third stage in flight pays (1024x2048x1024 15.8 -> 13.9 us,
        // 1024x3072x1024 21.6 -> 18.7, 2048x3072x1024 30.4 -> 28.4)
        if (!gated && M >= 1024 && M <= 2048 && K >= 2048 && N <= 1024 && blocks(64, 64) >= 256)
            return PLAN_X64x64s3;
        if (M >= 1024) {
            // Fewer than 256 tiles of 128x128 (measured on MI355X, every plan at
            // M = 1024 and 2048 on the Qwen3-0.6B shapes): the 32x64 tiles while
            // they fit two rounds (1024 x {1024,2048,3072} -> 1024: 9.1, 15.1,
            // 21.3 us against 13.9, 19.6, 21.7 on 128x128 / split K), 64x128
            // tiles at K = 1024 (1024x1024x2048 12.7 vs 15.4 us, 2048x1024x1024
            // 12.7 vs 15.0), 64x64 tiles while they fit two rounds (2048x2048
            // x1024 21.9 vs 27.2 us), else K split over the idle CUs
            if (!gated && blocks(128, 128) < 256) {
                if (blocks(32, 64) <= 512) return PLAN_P32x64k64s4;
                if (K <= 1024 && blocks(64, 128) >= 256) return PLAN_X64x128;
                if (blocks(64, 64) <= 512) return PLAN_P64x64k64s3;
            }
            // 256 x 256 tiles; below M = 8192 without the bf16 rounding pass of A
            // (measured on MI355X, 4096 x 1024 x 4096: 42.3 vs 45.6 us)
            if (!gated && blocks(256, 256) >= 256) return M >= 8192 ? PLAN_XB256x256s1 : PLAN_X256x256;
            // gated from M = 2048: one round of 256 x 256 tiles on eight waves
            // where they fit, and from M = 8192 (2048 / 8192 x 1024 x 3072: 39.4 /
            // 136 -> 37.3 / 120.6 us), else A rounded to bf16 first and 128 x 128
            // tiles (4096 rows: 68 against 75 us on 256 x 256)
            if (gated && M >= 2048)
                return (blocks(256, 256) <= g_cus || M >= 8192) ? PLAN_X256x256 : PLAN_XB128x128;
            return PLAN_X128x128;
        }
        if (M > 128 && blocks(128, 128) >= 128)
            return (!gated && blocks(64, 128) >= 256) ? PLAN_X64x128 : PLAN_X128x128;
    }
    if (M <= 128 || (!gated && M <= 512)) {
        const long t = blocks(32, 64);
        if (K % 128 == 0 && t <= 256) return PLAN_P32x64k128s4;
        if (K % 64 == 0 && t <= 512) return PLAN_P32x64k64s4;
    }
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

template <int ROWS, bool GATED, bool PRO, bool MERGE = false>
static int launch_gemv1_rows(float *c, const float *a, const uint16_t *b, const uint16_t *b2,
                             int K, int N, int cpl, const GemvPro &pro) {
    const int grid = (N + (NTHREADS / WAVE) * ROWS - 1) / ((NTHREADS / WAVE) * ROWS);
    const size_t lds = (size_t)(4 * WAVE * cpl + 8) * sizeof(uint32_t);   // bf16 row padded to 512*cpl, partials
    // only the (ROWS, CPL) pairs launch_gemv1 can pick: <= 16 loads per lane
#define QH_GEMV1_CASE(P)                                                                     \
    case P:                                                                                  \
        if constexpr ((ROWS == 1 || ROWS * P * (GATED ? 2 : 1) <= 16) && (!MERGE || P == 4)) \
            hipLaunchKernelGGL((k_gemv1<ROWS, P, GATED, PRO, MERGE>), dim3(grid), dim3(NTHREADS), \
                               lds, g_stream, c, a, b, b2, K, N, pro);                       \
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

// M = 1 with K <= 4096.  Rows per wave: at most 4, as many as keep >= 4096
// waves in the grid (16 per CU) and <= 16 weight loads of 16 B in flight per
// lane (measured on MI355X: lm_head 1024 -> 151936 streams 6.5 TB/s with 8
// rows per wave, 7.1-7.2 TB/s with 4, 2 or 1; q|k|v 1024 -> 4096 at one row
// per wave instead of two: the 113-launch decode step 2,486-2,492 ->
// 2,504 tok/s)
template <bool PRO>
static int launch_gemv1_t(float *c, const float *a, const uint16_t *b, const uint16_t *b2,
                          int K, int N, bool gated, const GemvPro &pro) {
    const int cpl = (K / 8 + WAVE - 1) / WAVE;
    const int per_row = gated ? 2 * cpl : cpl;
    int rows = 4;
    while (rows > 1 && (long)(N + rows - 1) / rows < 4096) rows /= 2;
    while (rows > 1 && rows * per_row > 16) rows /= 2;
    switch (rows) {
        case 1: return gated ? launch_gemv1_rows<1, true, PRO>(c, a, b, b2, K, N, cpl, pro)
                             : launch_gemv1_rows<1, false, PRO>(c, a, b, b2, K, N, cpl, pro);
        case 2: return gated ? launch_gemv1_rows<2, true, PRO>(c, a, b, b2, K, N, cpl, pro)
                             : launch_gemv1_rows<2, false, PRO>(c, a, b, b2, K, N, cpl, pro);
        case 4: return gated ? launch_gemv1_rows<4, true, PRO>(c, a, b, b2, K, N, cpl, pro)
                             : launch_gemv1_rows<4, false, PRO>(c, a, b, b2, K, N, cpl, pro);
        default: return QH_EINVAL;
    }
}
static int launch_gemv1(float *c, const float *a, const uint16_t *b, const uint16_t *b2,
                        int K, int N, bool gated) {
    return launch_gemv1_t<false>(c, a, b, b2, K, N, gated, GemvPro{});
}

// M = 1 with K <= 3072 (K % 8 == 0) and the activation row already rounded
// to bf16 on the host (`row`: max(1024, 512 CPL) bf16 values, zero past K):
// the row goes in the launch's kernel arguments, so nothing is copied to the
// device before the GEMV.  Same kernel body, row choice and results as
// launch_gemv1_t.
template <int ROWS, int CPL>
static int launch_gemv1_ka(float *c, const uint16_t *row_bf16, const uint16_t *b, const uint16_t *b2, int K, int N) {
    GemvKaRow<CPL> row;
    memcpy(row.w, row_bf16, sizeof row.w);
    const int grid = (N + (NTHREADS / WAVE) * ROWS - 1) / ((NTHREADS / WAVE) * ROWS);
    const size_t lds = (size_t)(4 * WAVE * CPL + 8) * sizeof(uint32_t);
    if (b2) {
        if constexpr (ROWS * CPL * 2 <= 16)
            hipLaunchKernelGGL((k_gemv1_ka<ROWS, CPL, true>), dim3(grid), dim3(NTHREADS), lds, g_stream, row, c, b,
                               b2, K, N);
        else
            return QH_EINVAL;
    } else {
        hipLaunchKernelGGL((k_gemv1_ka<ROWS, CPL, false>), dim3(grid), dim3(NTHREADS), lds, g_stream, row, c, b,
                           nullptr, K, N);
    }
    HCHECK(hipGetLastError(), QH_ELAUNCH);
    return QH_OK;
}
// cpl 5 and 6 run at most 2 rows per wave (launch_gemv1_t's <= 16 loads per lane)
template <int ROWS>
static int launch_gemv1_ka_cpl(int cpl, float *c, const uint16_t *row, const uint16_t *b, const uint16_t *b2, int K,
                               int N) {
    switch (cpl) {
        case 1: return launch_gemv1_ka<ROWS, 1>(c, row, b, b2, K, N);
        case 2: return launch_gemv1_ka<ROWS, 2>(c, row, b, b2, K, N);
        case 3: return launch_gemv1_ka<ROWS, 3>(c, row, b, b2, K, N);
        case 4: return launch_gemv1_ka<ROWS, 4>(c, row, b, b2, K, N);
        case 5: if constexpr (ROWS <= 2) return launch_gemv1_ka<ROWS, 5>(c, row, b, b2, K, N); else return QH_EINVAL;
        case 6: if constexpr (ROWS <= 2) return launch_gemv1_ka<ROWS, 6>(c, row, b, b2, K, N); else return QH_EINVAL;
        default: return QH_EINVAL;
    }
}
extern "C" int qh_gemv_ka(float *c, const uint16_t *row_bf16, const uint16_t *b, const uint16_t *b2, int K, int N) {
    if (!g_inited) return QH_ESTATE;
    if (!c || !row_bf16 || !b || K <= 0 || K > 3072 || (K % 8) || N <= 0 || !aligned16(b) || (b2 && !aligned16(b2)))
        return QH_EINVAL;
    if ((size_t)N * K * 2 >= (1ull << 31)) return QH_ETOOBIG;
    const int cpl = (K / 8 + WAVE - 1) / WAVE;
    const int per_row = b2 ? 2 * cpl : cpl;
    int rows = 4;
    while (rows > 1 && (long)(N + rows - 1) / rows < 4096) rows /= 2;
    while (rows > 1 && rows * per_row > 16) rows /= 2;
    g_last_plan = PLAN_GEMV;
    switch (rows) {
        case 1: return launch_gemv1_ka_cpl<1>(cpl, c, row_bf16, b, b2, K, N);
        case 2: return launch_gemv1_ka_cpl<2>(cpl, c, row_bf16, b, b2, K, N);
        case 4: return launch_gemv1_ka_cpl<4>(cpl, c, row_bf16, b, b2, K, N);
        default: return QH_EINVAL;
    }
}

extern "C" int qh_gemv_merge(float *c, const float *part, const uint16_t *b, int K, int N) {
    if (!g_inited) return QH_ESTATE;
    if (!c || !part || !b || K != 2048 || N <= 0 || !aligned16(part) || !aligned16(b)) return QH_EINVAL;
    if ((size_t)N * K * 2 >= (1ull << 31)) return QH_ETOOBIG;
    // K = 2048: 256 chunks of 16 bytes per row, 4 per lane; one row per wave
    // keeps >= 2048 waves for N = 1024 and 16 weight loads in flight per lane
    const int cpl = K / 8 / WAVE;
    const int rc = launch_gemv1_rows<1, false, false, true>(c, part, b, nullptr, K, N, cpl, GemvPro{});
    return rc;
}

template <int MR>
static int launch_gemv_mr(float *c, const float *a, const uint16_t *b, const uint16_t *b2,
                          int K, int N, bool gated) {
    if (MR == 1 && K <= 8 * WAVE * 8 && (size_t)N * K * 2 < (1ull << 31))   // k_gemv1's 32-bit offsets
        return launch_gemv1(c, a, b, b2, K, N, gated);
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

// Tile grid of an M x N output in BM x BNO tiles, with the 8-way XCD split
// whose per-XCD A + B slabs are smallest (row-major order when no split
// divides the grid).  Returns the number of tiles, or -1 if too many.
static long make_map(TileMap &map, int M, int N, int K, int BM, int BN, int BNO) {
    map.MT = (M + BM - 1) / BM;
    map.NT = (N + BNO - 1) / BNO;
    const long tiles = (long)map.MT * map.NT;
    if (tiles > 0x7FFFFFFFL) return -1;
    map.rm = 0;
    map.rn = 0;
    double best = 0.0;
    for (int rm = 1; rm <= 8; rm *= 2) {
        const int rn = 8 / rm;
        if (map.MT % rm || map.NT % rn) continue;
        const double slab = (double)(map.MT / rm) * BM * K * 4.0 + (double)(map.NT / rn) * BN * K * 2.0;
        if (map.rm == 0 || slab < best) { best = slab; map.rm = rm; map.rn = rn; }
    }
    return tiles;
}

template <int BM, int BN, int BK, int WM, int WN, bool GATED, bool VEC>
static int launch_tile(float *c, const float *a, const uint16_t *b, const uint16_t *b2,
                       int M, int K, int N) {
    TileMap map;
    const long tiles = make_map(map, M, N, K, BM, BN, GATED ? BN / 2 : BN);
    if (tiles < 0) return QH_ETOOBIG;
    hipLaunchKernelGGL((k_gemm<BM, BN, BK, WM, WN, GATED, VEC>), dim3((unsigned)tiles),
                       dim3(NTHREADS), 0, g_stream, c, a, b, b2, M, K, N, map);
    HCHECK(hipGetLastError(), QH_ELAUNCH);
    return QH_OK;
}

// requires K % BK == 0 and 16-byte aligned a, b, b2 (checked by the caller)
template <int BM, int BN, int WM, int WN, int STAGES, bool GATED, int BK = 32, int KG = 1>
static int launch_pipe(float *c, const float *a, const uint16_t *b, const uint16_t *b2,
                       int M, int K, int N) {
    using R = RingCfg<BM, BN, WM, WN, STAGES, GATED, BK, KG>;
    static int attr_dev = -1;              // dynamic LDS above 64 KB must be opted into, per device
    if (attr_dev != g_device) {
        HCHECK(hipFuncSetAttribute((const void *)k_gemm_pipe<BM, BN, WM, WN, STAGES, GATED, BK, KG>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, R::LDS),
               QH_ELAUNCH);
        attr_dev = g_device;
    }
    TileMap map;
    const long tiles = make_map(map, M, N, K, BM, BN, R::BNO);
    if (tiles < 0) return QH_ETOOBIG;
    hipLaunchKernelGGL((k_gemm_pipe<BM, BN, WM, WN, STAGES, GATED, BK, KG>), dim3((unsigned)tiles),
                       dim3(64 * WM * WN * KG), R::LDS, g_stream, c, a, b, b2, M, K, N, map);
    HCHECK(hipGetLastError(), QH_ELAUNCH);
    return QH_OK;
}

// ---- workspace ----------------------------------------------------------------
// Device memory beyond a GEMM's inputs and outputs: the bf16 copy of A (xb
// plans) or the fp32 slice sums of a K split (skinny, stream).  No plan uses
// both at once.  The library's own pair (g_abf, g_part) grows on demand
// outside graph capture; the no-allocation entry point passes the fixed
// `scratch` array instead (both fields point at it; `grow` false).
struct Ws {
    uint16_t *abf;
    size_t abf_elems;
    float *part;
    size_t part_bytes;
    bool grow;
    unsigned *cnt;     // NARROW_CNT zeroed tickets (narrow plan)
};

// A captured graph keeps the device addresses it was recorded with.  Each
// graph slot lists the library workspace buffers its kernels use; a buffer
// replaced by a larger one is freed at once when no live graph lists it, and
// otherwise parked in g_retired until the last graph listing it is destroyed.
static bool g_cap_abf = false, g_cap_part = false;   // used by the graph being captured

static bool graph_holds(const void *p) {
    for (int i = 0; i < QH_MAX_GRAPHS; i++)
        if (g_graph_exec[i] && (g_graph_ws[i][0] == p || g_graph_ws[i][1] == p)) return true;
    return false;
}

// a library workspace about to be written by a launch on the stream
static uint16_t *use_abf(const Ws &ws) {
    if (ws.grow && g_capturing) g_cap_abf = true;
    return ws.abf;
}
static float *use_part(const Ws &ws) {
    if (ws.grow && g_capturing) g_cap_part = true;
    return ws.part;
}

// drop a replaced workspace buffer: freed now unless a live graph uses it;
// false (nothing changed) when it must be parked and the list is full
static bool retire_buffer(void *p) {
    if (!p) return true;
    if (!graph_holds(p)) {
        (void)hipStreamSynchronize(g_stream);   // the old buffer may still be read
        (void)hipFree(p);
        return true;
    }
    if (g_n_retired >= QH_MAX_RETIRED) return false;
    g_retired[g_n_retired++] = p;
    return true;
}

// free every parked buffer that no live graph uses any more
static void free_retired(void) {
    int j = 0;
    bool synced = false;
    for (int i = 0; i < g_n_retired; i++) {
        if (graph_holds(g_retired[i])) {
            g_retired[j++] = g_retired[i];
            continue;
        }
        if (!synced) { (void)hipStreamSynchronize(g_stream); synced = true; }
        (void)hipFree(g_retired[i]);
    }
    g_n_retired = j;
}

// ws holds at least `bytes` of slice sums: the library's grows (outside
// capture only), a fixed workspace does not
static bool part_ensure(Ws &ws, size_t bytes) {
    if (bytes >= (1ull << 31)) return false;           // the reduction's 32-bit offsets
    if (bytes <= ws.part_bytes) return true;
    if (!ws.grow || g_capturing) return false;
    if (graph_holds(g_part) && g_n_retired >= QH_MAX_RETIRED) return false;
    float *p = nullptr;
    if (hipMalloc((void **)&p, bytes) != hipSuccess) { (void)hipGetLastError(); return false; }
    (void)retire_buffer(g_part);               // cannot fail: room checked above
    g_part = p;
    g_part_bytes = bytes;
    ws.part = p;
    ws.part_bytes = bytes;
    return true;
}

// ws holds at least n bf16 elements
static bool abf_ensure(Ws &ws, size_t n) {
    if (n <= ws.abf_elems) return true;
    if (!ws.grow || g_capturing) return false;
    if (graph_holds(g_abf) && g_n_retired >= QH_MAX_RETIRED) return false;
    uint16_t *p = nullptr;
    if (hipMalloc((void **)&p, n * sizeof(uint16_t)) != hipSuccess) { (void)hipGetLastError(); return false; }
    (void)retire_buffer(g_abf);                // cannot fail: room checked above
    g_abf = p;
    g_abf_elems = n;
    ws.abf = p;
    ws.abf_elems = n;
    return true;
}

static Ws lib_ws(void) { return Ws{g_abf, g_abf_elems, g_part, g_part_bytes, true, g_cnt}; }

// requires K % BK == 0, 16-byte aligned a, b, b2 and operands below 4 GiB
// (checked by the caller)
// When one round of blocks covers the tiles, a block with one wave per SIMD
// leaves the MFMA pipe idle while that wave waits, so two layouts run eight
// waves instead: gated 128 x 128 tiles as 4 x 2 waves, and the other tiles
// up to 128 x 128 (BK = 64; gated 64 x 128 too: 256 x 1024 -> 3072 gate|up +
// SiLU 12.1 -> 10.4 us) as two groups of 2 x 2 waves that split each
// stage's k-steps, the second group adding its sums into the first's
// through LDS at the end (measured on MI355X, graph-replayed: gate|up + SiLU
// 512 x 1024 -> 3072 18.0 -> 16.7 us, 256 rows 15.8 -> 13.7-14.9; 64 x 64
// tiles 512 x 1024 x 2048 8.46 -> 7.83 us, 1024 x 2048 x 1024 13.65 ->
// 12.7, 1024 x 1024 x 1024 8.2 -> 7.7; 128 x 128 tiles 4096 x {1024, 2048,
// 3072} x 1024 19.2 / 32 / 44 -> 17.8 / 27 / 37.8, 2048 x 1024 x 2048 18.9
// -> 17.6; 64 x 128 tiles 2048 x 1024 x 1024 12.8 -> 11.3).  With more
// tiles than CUs, two blocks of four waves per CU stay faster (gated M =
// 1024 26.4 against 33.3 us).
template <int BM, int BN, int BK, bool GATED, bool ABF16 = false, int SETS = 2>
static int launch_xl(float *c, const void *a, const uint16_t *b, const uint16_t *b2,
                     int M, int K, int N) {
    using X = XlCfg<BM, BN, BK, GATED, ABF16, SETS>;
    TileMap map;
    const long tiles = make_map(map, M, N, K, BM, BN, X::BNO);
    if (tiles < 0) return QH_ETOOBIG;
    if constexpr (GATED && BM == 128 && BN == 128) {
        if (tiles <= g_cus) {
            hipLaunchKernelGGL((k_gemm_xl<BM, BN, BK, GATED, ABF16, SETS, 4, 1>), dim3((unsigned)tiles, 1),
                               dim3(XlCfg<BM, BN, BK, GATED, ABF16, SETS, 4>::NT), 0, g_stream, c, a, b, b2, M, K, N,
                               map);
            HCHECK(hipGetLastError(), QH_ELAUNCH);
            return QH_OK;
        }
    }
    if constexpr (BK == 64 && BM * BN <= 128 * 128 && (!GATED || BM * BN < 128 * 128)) {
        if (tiles <= g_cus) {
            hipLaunchKernelGGL((k_gemm_xl<BM, BN, BK, GATED, ABF16, SETS, 2, 2>), dim3((unsigned)tiles, 1),
                               dim3(XlCfg<BM, BN, BK, GATED, ABF16, SETS, 2, 2>::NT), 0, g_stream, c, a, b, b2, M, K, N,
                               map);
            HCHECK(hipGetLastError(), QH_ELAUNCH);
            return QH_OK;
        }
    }
    hipLaunchKernelGGL((k_gemm_xl<BM, BN, BK, GATED, ABF16, SETS, 2, 1>), dim3((unsigned)tiles, 1), dim3(X::NT), 0,
                       g_stream, c, a, b, b2, M, K, N, map);
    HCHECK(hipGetLastError(), QH_ELAUNCH);
    return QH_OK;
}

// fp32 -> bf16 (RNE) on the stream; n % 8 == 0, 16-byte aligned pointers
static int launch_cvt_bf16(uint16_t *dst, const float *src, size_t n) {
    const size_t n8 = n / 8;
    size_t blocks = (n8 + NTHREADS - 1) / NTHREADS;
    if (blocks > 2048) blocks = 2048;
    if (blocks == 0) return QH_OK;
    hipLaunchKernelGGL(k_cvt_bf16, dim3((unsigned)blocks), dim3(NTHREADS), 0, g_stream, dst, src, n8);
    HCHECK(hipGetLastError(), QH_ELAUNCH);
    return QH_OK;
}

// fp32 bytes of the slice sums a stream plan with KS needs (0: no K split)
static inline size_t stream_part_bytes(int M, int K, int N, int ks, bool gated) {
    const int ksplit = K / (256 * ks);
    return ksplit > 1 ? (size_t)ksplit * (gated ? 2 : 1) * M * N * sizeof(float) : 0;
}

// weight-streaming GEMM: K % (256*KS) == 0, M <= 64, 16-byte aligned a, b,
// b2, sizes within stream_fits and the slice sums within ws (checked by the
// caller).  K / (256*KS) > 1 slices sum through ws and one k_stream_reduce pass.
template <int MT, int KS, bool GATED>
static int launch_stream_t(const Ws &ws, float *c, const float *a, const uint16_t *b, const uint16_t *b2,
                           int M, int K, int N) {
    constexpr int ST = KS >= 8 ? 2 : KS >= 4 ? 3 : KS >= 2 ? 4 : 8;   // tiles in flight per wave
    const int ksplit = K / (256 * KS);
    const int ntiles = (N + 15) / 16;
    const int gx = ntiles < g_cus ? ntiles : g_cus;
    float *part = nullptr;
    const size_t MN = (size_t)M * N;
    if (ksplit > 1) {
        if (stream_part_bytes(M, K, N, KS, GATED) > ws.part_bytes) return QH_ETOOBIG;
        part = use_part(ws);
    }
    hipLaunchKernelGGL((k_gemm_stream<MT, KS, ST, GATED>), dim3(gx, ksplit), dim3(STREAM_THREADS), 0,
                       g_stream, c, part, a, b, b2, M, K, N, ntiles);
    HCHECK(hipGetLastError(), QH_ELAUNCH);
    if (ksplit > 1) {
        size_t blocks = (MN + NTHREADS - 1) / NTHREADS;
        if (blocks > 1024) blocks = 1024;
        hipLaunchKernelGGL((k_stream_reduce<GATED>), dim3((unsigned)blocks), dim3(NTHREADS), 0, g_stream,
                           c, part, MN, ksplit);
        HCHECK(hipGetLastError(), QH_ELAUNCH);
    }
    return QH_OK;
}

// K slices of the skinny kernel: multiples of 64, at most 256 deep; the
// fewest that give every CU a 64-row block (else the most)
#define SKINNY_MMAX 256          // rows of A the skinny plan takes (slabs of 64)
static int skinny_slices(int K, int N, int M = 64) {
    const long nblk = (long)((N + 63) / 64) * ((M + 63) / 64);
    int best = 0;
    for (int ks = 1; ks <= K / 64 && ks <= RMAX; ks++) {
        if (K % ks || (K / ks) % 64 || K / ks > 256) continue;
        best = ks;
        if (nblk * ks >= g_cus) return ks;
    }
    return best;
}

// skinny GEMM: M <= SKINNY_MMAX, K % 64 == 0, 16-byte aligned a, b, b2 and
// sizes below 2 GiB (checked by the caller); more than one slice needs the
// slice sums in ws
template <int MT, bool GATED>
static int launch_skinny_t(const Ws &ws, float *c, const float *a, const uint16_t *b, const uint16_t *b2,
                           int M, int K, int N, bool reduce = true) {
    const int ks = skinny_slices(K, N, M);
    if (ks <= 0) return QH_EINVAL;
    const int nblk = (N + 63) / 64;
    const int mslab = (M + 63) / 64;
    const size_t MN = (size_t)M * N;
    float *part = nullptr;
    if (ks > 1) {
        if ((size_t)ks * (GATED ? 2 : 1) * MN * sizeof(float) > ws.part_bytes) return QH_ETOOBIG;
        part = use_part(ws);
    }
    hipLaunchKernelGGL((k_gemm_skinny<MT, GATED>), dim3(nblk, ks, mslab), dim3(NTHREADS), 0, g_stream, c, part, a,
                       b, b2, M, K, N, K / ks);
    HCHECK(hipGetLastError(), QH_ELAUNCH);
    if (ks > 1 && reduce) {
        size_t blocks = (MN + NTHREADS - 1) / NTHREADS;
        if (blocks > 2048) blocks = 2048;
        hipLaunchKernelGGL((k_stream_reduce<GATED>), dim3((unsigned)blocks), dim3(NTHREADS), 0, g_stream,
                           c, part, MN, ks);
        HCHECK(hipGetLastError(), QH_ELAUNCH);
    }
    return QH_OK;
}
template <bool GATED>
static int launch_skinny(const Ws &ws, float *c, const float *a, const uint16_t *b, const uint16_t *b2,
                         int M, int K, int N) {
    switch (stream_mt(M)) {
        case 1: return launch_skinny_t<1, GATED>(ws, c, a, b, b2, M, K, N);
        case 2: return launch_skinny_t<2, GATED>(ws, c, a, b, b2, M, K, N);
        default: return launch_skinny_t<4, GATED>(ws, c, a, b, b2, M, K, N);
    }
}

// The narrow kernel's geometry: 16 mt rows per block in `slabs` row slabs,
// K slices of 128 kpw (ks of them).  kpw is capped so that a thread's loads
// in flight (2 mt kpw of A, 2 nj kpw of weights) stay within 64.  The search
// runs over mt (from the rows M needs down to 16) and kpw for the grid that
// fills the most CUs in one round (one block per CU); among those it prefers
// one slice (no slice sums at all), then the fewest bytes a block moves: its
// A slice (fp32), its weights, and twice the slice sums its last block reads
// (they sit on the critical path).  Measured on MI355X, M = 64, graph-
// replayed: 64x1024x4096 6.1 us (32x64 tiles) -> 4.9 (32-row slabs, one
// slice), 64x1024x2048 6.0 -> 4.2 (16-row slabs), 64x2048x1024 7.4 (64 rows,
// 8 slices) -> 6.2 (32 rows, 4 slices), 64x3072x1024 7.9 -> 6.9.
struct NarrowGeom {
    int mt, slabs, kpw, ks, ncol;
};
static inline int narrow_kmax(int mt, bool gated) {
    const int lim = 64 / (2 * mt + 2 * (gated ? 2 : 1));
    return lim >= 8 ? 8 : lim >= 6 ? 6 : lim >= 4 ? 4 : lim >= 3 ? 3 : lim >= 2 ? 2 : 1;
}
// The geometry of a narrow launch, searched per shape: the most CUs filled in
// one round, then one slice (no sums at all), then the fewest bytes a block
// moves, counting the sums its last block reads twice.  Column blocks are 32
// wide, or 16 wide with 16-row slabs, not gated, and slices of 1024, 2048 or
// 3072: that form takes K = 1024 - 3072 in one slice where the 32-wide
// blocks need 2-8 (64 x {1024, 2048, 3072} x 1024: 256 blocks and no slice
// sums; measured on MI355X, graph-replayed: k/v 5.3 -> 3.1 us, o 6.3 -> 4.4).
static NarrowGeom narrow_geom(int M, int K, int N, bool gated) {
    static const int opts[] = {8, 6, 4, 3, 2, 1};
    static const int opts16[] = {24, 16, 8};
    const int nj = gated ? 2 : 1;
    const int auto_mt = stream_mt(M);
    NarrowGeom best{0, 0, 0, 0, 0};
    long best_blocks = 0, best_cost = 0;
    auto consider = [&](int mt, int kpw, int ncol) {
        const long ncb = (N + ncol - 1) / ncol;
        const int slabs = (M + 16 * mt - 1) / (16 * mt);
        const long tiles = ncb * slabs;
        if (tiles > NARROW_CNT || K % (128 * kpw)) return;
        const int ks = K / (128 * kpw);
        const long blocks = tiles * ks;
        const long ksl = 128L * kpw, rows = 16L * mt;
        const long cost = rows * ksl * 4 + nj * ncol * ksl * 2 + (ks > 1 ? 2L * ks * rows * ncol * 4 * nj : 0);
        // one round: blocks <= CUs, else (nothing fits) the fewest blocks
        const bool fits = blocks <= g_cus, best_fits = best_blocks <= g_cus;
        bool take;
        if (!best.kpw) take = true;
        else if (fits != best_fits) take = fits;
        else if (!fits) take = blocks < best_blocks;
        // one slice (no slice sums, no tickets) once it gives at least half
        // the CUs a block (measured on MI355X, 96 x 1024 x 1024: 6.4 us on
        // 256 blocks of 4 slices, 4.0 on 192 of one)
        else if ((ks == 1 && 2 * blocks >= g_cus) != (best.ks == 1 && 2 * best_blocks >= g_cus))
            take = ks == 1 && 2 * blocks >= g_cus;
        else if (blocks != best_blocks) take = blocks > best_blocks;
        else if ((ks == 1) != (best.ks == 1)) take = ks == 1;
        else take = cost < best_cost;
        if (take) {
            best = NarrowGeom{mt, slabs, kpw, ks, ncol};
            best_blocks = blocks;
            best_cost = cost;
        }
    };
    for (int mt = auto_mt; mt >= 1; mt /= 2)
        for (int kpw : opts)
            if (kpw <= narrow_kmax(mt, gated)) consider(mt, kpw, NARROW_COLS);
    if (!gated)
        for (int kpw : opts16) consider(1, kpw, 16);
    return best;
}
static inline size_t narrow_part_bytes(const NarrowGeom &g, int M, int N, bool gated) {
    return g.ks > 1 ? (size_t)g.ks * (gated ? 2 : 1) * M * N * sizeof(float) : 0;
}
// the instantiated (mt, kpw, gated, ncol, waves) combinations: loads in
// flight within 64.  The 16-wide blocks with a 3072-deep slice (geometry kpw
// 24) run 8 waves of 12 steps each, the same K slice: A and the weights then
// all go out at entry (24 A loads + 12 weight loads per lane; with 4 waves,
// 48 + 24, A had to come in two halves).  Measured on MI355X, graph-replayed:
// 64 x 3072 x 1024 6.51 -> 6.18 us; at kpw 8 and 16 (one phase either way)
// 8 waves were no faster (64 x 2048 x 1024 4.40 -> 4.49 us), so those stay 4.
template <int MT, int KPW, bool GATED, int NCOL, int NWV>
constexpr bool narrow_ok() {
    return NCOL == 16 ? (MT == 1 && !GATED && ((NWV == 4 && (KPW == 8 || KPW == 16)) || (NWV == 8 && KPW == 12)))
                      : NWV == 4 && 2 * MT * KPW + 2 * (GATED ? 2 : 1) * KPW <= 64;
}

template <int MT, int KPW, bool GATED, int NCOL = NARROW_COLS, int NWV = 4>
static int launch_narrow_t(const Ws &ws, const NarrowGeom &g, float *c, const float *a, const uint16_t *b,
                           const uint16_t *b2, int M, int K, int N) {
    if constexpr (!narrow_ok<MT, KPW, GATED, NCOL, NWV>()) {
        return QH_EINVAL;
    } else {
        const int ncb = (N + NCOL - 1) / NCOL;
        float *part = nullptr;
        if (g.ks > 1) {
            if (narrow_part_bytes(g, M, N, GATED) > ws.part_bytes || !ws.cnt) return QH_ETOOBIG;
            part = use_part(ws);
        }
        hipLaunchKernelGGL((k_gemm_narrow<MT, KPW, GATED, NCOL, NWV>),
                           dim3((unsigned)g.ks, (unsigned)ncb, (unsigned)g.slabs), dim3(64 * NWV), 0, g_stream, c,
                           part, ws.cnt, a, b, b2, M, K, N);
        HCHECK(hipGetLastError(), QH_ELAUNCH);
        return QH_OK;
    }
}
// narrow GEMM for plan p: sizes within narrow_fits, 16-byte aligned a, b, b2
// and the slice sums within ws (checked by the caller)
template <bool GATED>
static int launch_narrow(const Ws &ws, float *c, const float *a, const uint16_t *b, const uint16_t *b2,
                         int M, int K, int N) {
    const NarrowGeom g = narrow_geom(M, K, N, GATED);
    if (g.ncol == 16) {
        switch (g.kpw) {
            case 8: return launch_narrow_t<1, 8, GATED, 16>(ws, g, c, a, b, b2, M, K, N);
            case 16: return launch_narrow_t<1, 16, GATED, 16>(ws, g, c, a, b, b2, M, K, N);
            case 24: return launch_narrow_t<1, 12, GATED, 16, 8>(ws, g, c, a, b, b2, M, K, N);   // 8 waves
            default: return QH_EINVAL;
        }
    }
#define QH_NARROW_CASES(MT)                                                                  \
    switch (g.kpw) {                                                                         \
        case 1: return launch_narrow_t<MT, 1, GATED>(ws, g, c, a, b, b2, M, K, N);           \
        case 2: return launch_narrow_t<MT, 2, GATED>(ws, g, c, a, b, b2, M, K, N);           \
        case 3: return launch_narrow_t<MT, 3, GATED>(ws, g, c, a, b, b2, M, K, N);           \
        case 4: return launch_narrow_t<MT, 4, GATED>(ws, g, c, a, b, b2, M, K, N);           \
        case 6: return launch_narrow_t<MT, 6, GATED>(ws, g, c, a, b, b2, M, K, N);           \
        case 8: return launch_narrow_t<MT, 8, GATED>(ws, g, c, a, b, b2, M, K, N);           \
        default: return QH_EINVAL;                                                           \
    }
    switch (g.mt) {
        case 1: QH_NARROW_CASES(1)
        case 2: QH_NARROW_CASES(2)
        default: QH_NARROW_CASES(4)
    }
#undef QH_NARROW_CASES
}

// wide GEMM: sizes within wide_fits, 16-byte aligned a and b (checked by the caller)
template <int MT, int NCH>
static int launch_wide_t(float *c, const float *a, const uint16_t *b, int M, int N) {
    const int nw = NTHREADS / WAVE;
    const size_t lds = (size_t)16 * MT * NCH * WIDE_KC * 2 + (size_t)nw * WIDE_B_U4 * 16;
    static int attr_dev = -1;              // dynamic LDS above 64 KB must be opted into, per device
    if (attr_dev != g_device) {
        HCHECK(hipFuncSetAttribute((const void *)k_gemm_wide<MT, NCH, 0>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (int)lds),
               QH_ELAUNCH);
        HCHECK(hipFuncSetAttribute((const void *)k_gemm_wide<MT, NCH, 5>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (int)lds),
               QH_ELAUNCH);
        attr_dev = g_device;
    }
    const int ntiles = (N + 31) / 32;
    int blocks = (ntiles + nw - 1) / nw;
    if (blocks > g_cus) blocks = g_cus;
    if ((ntiles + (long)blocks * nw - 1) / ((long)blocks * nw) <= 5)
        hipLaunchKernelGGL((k_gemm_wide<MT, NCH, 5>), dim3((unsigned)blocks), dim3(NTHREADS), lds, g_stream, c, a, b,
                           M, N, ntiles);
    else
        hipLaunchKernelGGL((k_gemm_wide<MT, NCH, 0>), dim3((unsigned)blocks), dim3(NTHREADS), lds, g_stream, c, a, b,
                           M, N, ntiles);
    HCHECK(hipGetLastError(), QH_ELAUNCH);
    return QH_OK;
}
static int launch_wide(float *c, const float *a, const uint16_t *b, int M, int K, int N) {
    const int mt = stream_mt(M);
    if (K == 1024) return mt == 1 ? launch_wide_t<1, 16>(c, a, b, M, N) : mt == 2 ? launch_wide_t<2, 16>(c, a, b, M, N)
                                                                                 : launch_wide_t<4, 16>(c, a, b, M, N);
    if (K == 512) return mt == 1 ? launch_wide_t<1, 8>(c, a, b, M, N) : mt == 2 ? launch_wide_t<2, 8>(c, a, b, M, N)
                                                                               : launch_wide_t<4, 8>(c, a, b, M, N);
    return QH_EINVAL;
}

template <int NWV, int KT, int CT, bool GATED = false>
static int launch_m16_t(float *c, const float *a, const uint16_t *b, const uint16_t *b2, int M, int N) {
    const size_t lds = m16_lds_bytes(NWV, KT, CT);
    static int attr_dev = -1;              // dynamic LDS above 64 KB must be opted into, per device
    if (attr_dev != g_device) {
        HCHECK(hipFuncSetAttribute((const void *)k_gemm_m16<NWV, KT, CT, GATED>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
               QH_ELAUNCH);
        attr_dev = g_device;
    }
    const int cols = GATED ? 16 : 16 * CT;
    hipLaunchKernelGGL((k_gemm_m16<NWV, KT, CT, GATED>), dim3((unsigned)((N + cols - 1) / cols)), dim3(NWV * WAVE),
                       lds, g_stream, c, a, b, b2, M, N);
    HCHECK(hipGetLastError(), QH_ELAUNCH);
    return QH_OK;
}
// sizes within m16_fits (gated: K <= 2048), 16-byte aligned a, b, b2 (checked by the caller)
template <bool GATED>
static int launch_m16(float *c, const float *a, const uint16_t *b, const uint16_t *b2, int M, int K, int N) {
    if constexpr (GATED) {
        switch (K) {
            case 1024: return launch_m16_t<8, 1024, 2, true>(c, a, b, b2, M, N);
            case 2048: return launch_m16_t<8, 2048, 2, true>(c, a, b, b2, M, N);
            default: return QH_EINVAL;
        }
    } else {
        const int ct = m16_ct(K, N);
        switch (K * 10 + ct) {
            case 10241: return launch_m16_t<8, 1024, 1>(c, a, b, nullptr, M, N);
            case 10242: return launch_m16_t<8, 1024, 2>(c, a, b, nullptr, M, N);
            case 20481: return launch_m16_t<8, 2048, 1>(c, a, b, nullptr, M, N);
            case 20482: return launch_m16_t<8, 2048, 2>(c, a, b, nullptr, M, N);
            case 30721: return launch_m16_t<8, 3072, 1>(c, a, b, nullptr, M, N);
            default: return QH_EINVAL;
        }
    }
}

template <int MR, int ROWS, int CPL, int NWV>
static int launch_gemv_m_t(float *c, const float *a, const uint16_t *b, int M, int K, int N) {
    const int per_block = NWV * ROWS;
    const unsigned grid = (unsigned)((N + per_block - 1) / per_block);
    hipLaunchKernelGGL((k_gemv_m<MR, ROWS, CPL, NWV>), dim3(grid), dim3(NWV * WAVE), (size_t)MR * K * 2, g_stream, c,
                       a, b, M, K, N);
    HCHECK(hipGetLastError(), QH_ELAUNCH);
    return QH_OK;
}
// sizes within gemv16_fits, 16-byte aligned a and b (checked by the caller).
// 8 waves per block share one staged copy of A (its L2 reads, 2-4 KB per
// row of A per block, are the kernel's main cost after the weights); rows per
// wave: 4 at M <= 8, else 2, halved while that leaves fewer than 192 blocks
// (measured on MI355X, 16 x 1024 x {3072, 2048, 1024}: 4.9 / 3.8 / 3.5 us
// with 8 waves against 5.4 / 4.5 / 3.6 with 4 and 5.0 / 4.8 / 4.6 with 16)
static int launch_gemv16(float *c, const float *a, const uint16_t *b, int M, int K, int N) {
    constexpr int NWV = 8;
    int rows = M <= 8 ? 4 : 2;
    while (rows > 1 && (long)N / (NWV * rows) < 192) rows /= 2;
    const int key = (M <= 8 ? 100 : 200) + (K <= 512 ? 10 : 20) + rows;
    switch (key) {
        case 111: return launch_gemv_m_t<8, 1, 1, NWV>(c, a, b, M, K, N);
        case 112: return launch_gemv_m_t<8, 2, 1, NWV>(c, a, b, M, K, N);
        case 114: return launch_gemv_m_t<8, 4, 1, NWV>(c, a, b, M, K, N);
        case 121: return launch_gemv_m_t<8, 1, 2, NWV>(c, a, b, M, K, N);
        case 122: return launch_gemv_m_t<8, 2, 2, NWV>(c, a, b, M, K, N);
        case 124: return launch_gemv_m_t<8, 4, 2, NWV>(c, a, b, M, K, N);
        case 211: return launch_gemv_m_t<16, 1, 1, NWV>(c, a, b, M, K, N);
        case 212: return launch_gemv_m_t<16, 2, 1, NWV>(c, a, b, M, K, N);
        case 221: return launch_gemv_m_t<16, 1, 2, NWV>(c, a, b, M, K, N);
        case 222: return launch_gemv_m_t<16, 2, 2, NWV>(c, a, b, M, K, N);
        default: return QH_EINVAL;
    }
}

template <bool GATED>
static int launch_stream(const Ws &ws, float *c, const float *a, const uint16_t *b, const uint16_t *b2,
                         int M, int K, int N, int ks) {
    switch (stream_mt(M) * 100 + ks) {
        case 101: return launch_stream_t<1, 1, GATED>(ws, c, a, b, b2, M, K, N);
        case 102: return launch_stream_t<1, 2, GATED>(ws, c, a, b, b2, M, K, N);
        case 104: return launch_stream_t<1, 4, GATED>(ws, c, a, b, b2, M, K, N);
        case 108: return launch_stream_t<1, 8, GATED>(ws, c, a, b, b2, M, K, N);
        case 201: return launch_stream_t<2, 1, GATED>(ws, c, a, b, b2, M, K, N);
        case 202: return launch_stream_t<2, 2, GATED>(ws, c, a, b, b2, M, K, N);
        case 204: return launch_stream_t<2, 4, GATED>(ws, c, a, b, b2, M, K, N);
        case 208: return launch_stream_t<2, 8, GATED>(ws, c, a, b, b2, M, K, N);
        case 401: return launch_stream_t<4, 1, GATED>(ws, c, a, b, b2, M, K, N);
        case 402: return launch_stream_t<4, 2, GATED>(ws, c, a, b, b2, M, K, N);
        case 404: return launch_stream_t<4, 4, GATED>(ws, c, a, b, b2, M, K, N);
        default: return QH_EINVAL;
    }
}

// bf16-A large-tile GEMM for plan p (an xb plan); a is bf16 bits
template <bool GATED>
static int dispatch_bf16a(int p, float *c, const uint16_t *a, const uint16_t *b, const uint16_t *b2,
                          int M, int K, int N) {
    switch (p) {
        case PLAN_XB256x256k32: return launch_xl<256, 256, 32, GATED, true>(c, a, b, b2, M, K, N);
        case PLAN_XB128x128:    return launch_xl<128, 128, 64, GATED, true>(c, a, b, b2, M, K, N);
        case PLAN_XB256x256s1:  return launch_xl<256, 256, 64, GATED, true, 1>(c, a, b, b2, M, K, N);
        default: return QH_EINVAL;
    }
}


template <bool GATED>
static int dispatch(int plan, const Ws &ws, float *c, const float *a, const uint16_t *b, const uint16_t *b2,
                    int M, int K, int N) {
    g_last_plan = plan;
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
        case PLAN_P32x64k128s4:   // four k groups (16 waves) from K = 2048, two below (see k_gemm_pipe)
            return K >= 2048 ? launch_pipe<32, 64, 2, 2, 4, GATED, 128, 4>(c, a, b, b2, M, K, N)
                             : launch_pipe<32, 64, 2, 2, 4, GATED, 128, 2>(c, a, b, b2, M, K, N);
        case PLAN_P32x64k64s4:  return launch_pipe<32, 64, 2, 2, 4, GATED, 64>(c, a, b, b2, M, K, N);
        case PLAN_P64x64k64s3:  return launch_pipe<64, 64, 2, 2, 3, GATED, 64>(c, a, b, b2, M, K, N);
        case PLAN_XB256x256k32: case PLAN_XB128x128: case PLAN_XB256x256s1: {
            if ((size_t)M * K > ws.abf_elems) return QH_ETOOBIG;
            uint16_t *abf = use_abf(ws);
            const int rc = launch_cvt_bf16(abf, a, (size_t)M * K);
            if (rc) return rc;
            return dispatch_bf16a<GATED>(plan, c, abf, b, b2, M, K, N);
        }
        case PLAN_X128x128: return launch_xl<128, 128, 64, GATED>(c, a, b, b2, M, K, N);
        case PLAN_X256x256: return launch_xl<256, 256, 32, GATED>(c, a, b, b2, M, K, N);
        case PLAN_X64x128:  return launch_xl<64, 128, 64, GATED>(c, a, b, b2, M, K, N);
        case PLAN_X64x64s3: return launch_xl<64, 64, 64, false, false, 3>(c, a, b, b2, M, K, N);   // not gated
        case PLAN_SKINNY: return launch_skinny<GATED>(ws, c, a, b, b2, M, K, N);
        case PLAN_NARROW:
            return launch_narrow<GATED>(ws, c, a, b, b2, M, K, N);
        case PLAN_WIDE:
            if constexpr (GATED) return QH_EINVAL;
            else return launch_wide(c, a, b, M, K, N);
        case PLAN_GEMV16:
            if constexpr (GATED) return QH_EINVAL;
            else return launch_gemv16(c, a, b, M, K, N);
        case PLAN_M16: return launch_m16<GATED>(c, a, b, b2, M, K, N);
        case PLAN_STREAM_KS1: return launch_stream<GATED>(ws, c, a, b, b2, M, K, N, 1);
        case PLAN_STREAM_KS2: return launch_stream<GATED>(ws, c, a, b, b2, M, K, N, 2);
        case PLAN_STREAM_KS4: return launch_stream<GATED>(ws, c, a, b, b2, M, K, N, 4);
        case PLAN_STREAM_KS8: return launch_stream<GATED>(ws, c, a, b, b2, M, K, N, 8);
        default: return QH_EINVAL;
    }
}

// The plan for an M x K x N call and the workspace it needs in ws (grown
// there when ws is the library's).  A plan whose conditions fail falls back
// to the 64x64 tiles, or to the fp32-A large tiles when the bf16 copy of A
// has no room; with a fixed workspace (`strict`) a plan that needs more than
// it holds is QH_ETOOBIG instead of a fall-back.  Returns the plan, or
// -QH_E* on error.
static int resolve_plan(Ws &ws, int M, int K, int N, bool gated, bool vec, bool strict) {
    int plan = g_forced_plan ? g_forced_plan : choose_plan(M, K, N, gated, vec);
    if (!vec) plan = PLAN_SCALAR64;   // forced plans still need vector-safe inputs
    if (plan == PLAN_GEMV && (M > 4 || (size_t)M * K * 4 > 64 * 1024)) plan = PLAN_T64x64;
    if (is_pipe_plan(plan) && (K % pipe_bk(plan)) != 0) plan = PLAN_T64x64;   // whole k stages
    if (plan == PLAN_X64x64s3 && gated) plan = PLAN_T64x64;   // one B block per wave tile
    if (is_xl_plan(plan) && ((K % xl_bk(plan)) != 0 ||           // xl copies whole k stages and
                             (size_t)M * K * 4 >= (1ull << 32) ||   // addresses with 32-bit offsets
                             (size_t)N * K * 2 >= (1ull << 32)))
        plan = PLAN_T64x64;
    if (is_xb_plan(plan) && !abf_ensure(ws, (size_t)M * K)) {     // no room for the bf16 copy of A
        if (strict) return -QH_ETOOBIG;
        plan = PLAN_X128x128;
    }
    if (plan == PLAN_SKINNY) {
        const int ks = (M <= SKINNY_MMAX && K % 64 == 0 && (size_t)M * K * 4 < (1ull << 31) &&
                        (size_t)N * K * 2 < (1ull << 31)) ? skinny_slices(K, N, M) : 0;
        const size_t part = (size_t)ks * (gated ? 2 : 1) * M * N * sizeof(float);
        if (ks > 1 && !part_ensure(ws, part)) {
            if (strict) return -QH_ETOOBIG;
            plan = PLAN_T64x64;
        } else if (ks <= 0) {
            plan = PLAN_T64x64;
        }
    }
    if (plan == PLAN_WIDE && (gated || !wide_fits(M, K, N))) plan = PLAN_T64x64;
    if (plan == PLAN_GEMV16 && (gated || !gemv16_fits(M, K, N))) plan = PLAN_T64x64;
    if (plan == PLAN_M16 && (!m16_fits(M, K, N) || (gated && K > 2048))) plan = PLAN_T64x64;
    if (is_narrow_plan(plan)) {
        // the slice sums need room in the workspace
        const NarrowGeom g = narrow_fits(M, K, N) ? narrow_geom(M, K, N, gated) : NarrowGeom{0, 0, 0, 0, 0};
        if (g.kpw <= 0) {
            plan = PLAN_T64x64;
        } else {
            const size_t part = narrow_part_bytes(g, M, N, gated);
            if (part && (!ws.cnt || !part_ensure(ws, part))) {
                if (strict) return -QH_ETOOBIG;
                plan = PLAN_T64x64;
            }
        }
    }
    if (is_stream_plan(plan)) {
        // KS must divide the slices and fit the A registers; more than one
        // slice needs workspace for the fp32 partial sums
        const bool fits = stream_fits(M, K, N);
        const int ks = plan != PLAN_STREAM ? 1 << (plan - PLAN_STREAM_KS1) : fits ? stream_ks(M, K, N, g_cus) : 0;
        bool ok = fits && ks > 0 && (K / 256) % ks == 0 && stream_mt(M) * ks <= 16 && K / (256 * ks) <= RMAX;
        if (ok) {
            const size_t part = stream_part_bytes(M, K, N, ks, gated);
            if (part && !part_ensure(ws, part)) {
                if (strict) return -QH_ETOOBIG;
                ok = false;
            }
        }
        if (!ok) plan = PLAN_T64x64;
        else plan = ks == 1 ? PLAN_STREAM_KS1 : ks == 2 ? PLAN_STREAM_KS2 : ks == 4 ? PLAN_STREAM_KS4 : PLAN_STREAM_KS8;
    }
    return plan;
}

static int gemm_common(Ws ws, bool strict, float *c, const float *a, const uint16_t *b, const uint16_t *b2,
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
    const int plan = resolve_plan(ws, M, K, N, gated, vec, strict);
    if (plan < 0) return -plan;
    return gated ? dispatch<true>(plan, ws, c, a, b, b2, M, K, N)
                 : dispatch<false>(plan, ws, c, a, b, nullptr, M, K, N);
}

// C = A.B^T with A already bf16 (bits), for callers that hold bf16
// activations: the large-tile kernels without the conversion pass.  Needs
// K % 64 == 0 and 16-byte aligned a, b, b2.
static int gemm_bf16a_common(float *c, const uint16_t *a, const uint16_t *b, const uint16_t *b2,
                             int M, int K, int N, bool gated) {
    if (!g_inited) return QH_ESTATE;
    if (M < 0 || K < 0 || N < 0) return QH_EINVAL;
    if (M == 0 || N == 0) return QH_OK;
    if (!c || !a || !b || (gated && !b2)) return QH_EINVAL;
    if (K % 64 != 0 || K == 0 || !aligned16(a) || !aligned16(b) || (gated && !aligned16(b2)))
        return QH_EINVAL;
    if ((size_t)M * K * 2 >= (1ull << 32) || (size_t)N * K * 2 >= (1ull << 32)) return QH_ETOOBIG;
    int plan = g_forced_plan;
    if (!is_xb_plan(plan)) plan = choose_bf16a_plan(M, K, N, gated);
    g_last_plan = plan;
    return gated ? dispatch_bf16a<true>(plan, c, a, b, b2, M, K, N)
                 : dispatch_bf16a<false>(plan, c, a, b, nullptr, M, K, N);
}

extern "C" int qh_gemm_bf16a(float *c, const uint16_t *a, const uint16_t *b, int M, int K, int N) {
    return gemm_bf16a_common(c, a, b, nullptr, M, K, N, false);
}

extern "C" int qh_gemm_gate_up_silu_bf16a(float *h, const uint16_t *x, const uint16_t *wg,
                                          const uint16_t *wu, int M, int K, int N) {
    return gemm_bf16a_common(h, x, wg, wu, M, K, N, true);
}

extern "C" int qh_gemm(float *c, const float *a, const uint16_t *b, int M, int K, int N) {
    return gemm_common(lib_ws(), false, c, a, b, nullptr, M, K, N, false);
}

extern "C" const char *qh_last_plan(void) { return k_plan_names[g_last_plan]; }

// ---- the no-allocation entry point ------------------------------------------
// qh_gemm with a fixed workspace, for callers that cannot allocate (code
// under graph capture, tight serving loops): the file-scope device array
// `scratch` (QH_SCRATCH_BYTES, one copy per GPU for the life of the process)
// replaces the library's growable workspace; a plan that would need more is
// QH_ETOOBIG, and nothing is allocated or freed.  Host code reaches the array
// only through the per-device address hipGetSymbolAddress returned at init
// (g_scratch_dev), never through its name.  Every plan writes all of the
// workspace it reads, except the narrow plan's tickets in the array's last
// NARROW_CNT words: zeroed at init, and each call leaves the ones it used at
// zero again, so nothing needs clearing between calls.  Calls that overlap on
// one GPU (another stream, another process's graph) race on the array.
extern "C" size_t qh_scratch_bytes(void) { return QH_SCRATCH_BYTES; }

extern "C" int qh_gemm_noalloc(float *c, const float *a, const uint16_t *b, int M, int K, int N) {
    if (!g_inited) return QH_ESTATE;
    void *s = g_scratch_dev[g_device];
    if (!s) return QH_ESTATE;
    const Ws ws{(uint16_t *)s, QH_SCRATCH_WS_BYTES / sizeof(uint16_t), (float *)s, QH_SCRATCH_WS_BYTES, false,
                (unsigned *)((unsigned char *)s + QH_SCRATCH_WS_BYTES)};
    return gemm_common(ws, true, c, a, b, nullptr, M, K, N, false);
}

// qh_gemm, except that when the skinny kernel splits K the slices' fp32 sums
// are left in the split-K workspace ([ks][M][N], *part) for the caller to add
// in slice order -- the sums k_stream_reduce would form -- instead of a second
// launch.  Taken where the automatic plan is the skinny kernel, and for
// M <= 128, K >= 2048, N <= 2048, where the kernel in 64-row slabs ties or
// beats the 32x64 tiles once the reduction launch is gone (measured at
// M = 96 / 128: down 13.2 / 13.2 -> ~9 us, o 9.6 / 9.8 -> ~6.5 us) -- but
// not where the automatic plan is the narrow kernel, which writes C itself
// (at M = 128 its o and down, with the plain residual + RMSNorm after them,
// beat the split sums and the norm that adds them: 128-token prefill 1.68
// -> 1.65 ms, 2,014-token prefill 40.3 -> 39.5 ms).
// Otherwise C is written and *ks = 0.  The partials last until the next call
// that uses the workspace.
extern "C" int qh_gemm_split(float *c, const float *a, const uint16_t *b, int M, int K, int N,
                             const float **part, int *ks) {
    if (!part || !ks) return QH_EINVAL;
    *part = nullptr;
    *ks = 0;
    if (!g_inited) return QH_ESTATE;
    const bool vec = M > 0 && K > 0 && N > 0 && a && b && c && (K % 8) == 0 && aligned16(a) && aligned16(b);
    const int auto_plan = vec ? choose_plan(M, K, N, false, vec) : PLAN_SCALAR64;
    const bool take = vec && !g_forced_plan && auto_plan != PLAN_NARROW &&
                      (auto_plan == PLAN_SKINNY || (M <= 128 && K >= 2048 && N <= 2048));
    Ws ws = lib_ws();
    if (take && M <= SKINNY_MMAX && K % 64 == 0 && (size_t)M * K * 4 < (1ull << 31) &&
        (size_t)N * K * 2 < (1ull << 31)) {
        const int s = skinny_slices(K, N, M);
        if (s > 1 && part_ensure(ws, (size_t)s * M * N * sizeof(float))) {
            int rc;
            g_last_plan = PLAN_SKINNY;
            switch (stream_mt(M)) {
                case 1: rc = launch_skinny_t<1, false>(ws, c, a, b, nullptr, M, K, N, false); break;
                case 2: rc = launch_skinny_t<2, false>(ws, c, a, b, nullptr, M, K, N, false); break;
                default: rc = launch_skinny_t<4, false>(ws, c, a, b, nullptr, M, K, N, false); break;
            }
            if (rc == QH_OK) {
                *part = ws.part;
                *ks = s;
            }
            return rc;
        }
    }
    return gemm_common(ws, false, c, a, b, nullptr, M, K, N, false);
}

extern "C" int qh_gemm_gate_up_silu(float *h, const float *x, const uint16_t *wg,
                                    const uint16_t *wu, int M, int K, int N) {
    return gemm_common(lib_ws(), false, h, x, wg, wu, M, K, N, true);
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
    g_cap_abf = g_cap_part = false;
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
    // the workspace buffers its kernels read or write stay allocated while it lives
    g_graph_ws[slot][0] = g_cap_abf ? (void *)g_abf : nullptr;
    g_graph_ws[slot][1] = g_cap_part ? (void *)g_part : nullptr;
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
    // a launch of this graph may still run: wait for the stream first, so
    // no caller has to
    HCHECK(hipStreamSynchronize(g_stream), QH_ERUNTIME);
    HCHECK(hipGraphExecDestroy(g_graph_exec[id]), QH_ERUNTIME);
    g_graph_exec[id] = nullptr;
    g_graph_ws[id][0] = g_graph_ws[id][1] = nullptr;
    free_retired();
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

extern "C" int qh_read(const void *src, size_t bytes) {
    if (!g_inited) return QH_ESTATE;
    if (!src || (bytes & 15u) || !aligned16(src) || bytes >= ((size_t)1 << 31)) return QH_EINVAL;
    if (bytes == 0) return QH_OK;
    const size_t n16 = bytes / 16;
    const size_t want = (n16 + NTHREADS - 1) / NTHREADS;
    const int grid = (int)(want < 4096 ? want : 4096);
    hipLaunchKernelGGL(k_read16, dim3(grid), dim3(NTHREADS), 0, g_stream, (const u32x4 *)src, n16);
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

// Greedy step bookkeeping on the device (so a decode step can be replayed as
// a graph with no host round trip): token = argmax, out[*step] = token when
// *step < cap, *step += 1, *pos += adv.
__global__ __launch_bounds__(WAVE) void k_argmax_step(int *__restrict__ tok, int *__restrict__ out,
                                                     int *__restrict__ step, int cap,
                                                     int *__restrict__ pos, int adv,
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
    if (threadIdx.x == 0) {
        const int t = (bi == 0x7FFFFFFF || v[0] != v[0]) ? 0 : bi;
        tok[0] = t;
        const int s = step[0];
        if (s >= 0 && s < cap) out[s] = t;
        step[0] = s + 1;
        pos[0] += adv;
    }
}

extern "C" int qh_argmax_step(int *tok, int *out, int *step, int cap, int *pos, int adv,
                              const float *v, int n) {
    if (!g_inited) return QH_ESTATE;
    if (n <= 0 || !tok || !out || !step || !pos || !v || cap < 0) return QH_EINVAL;
    int blocks = (n + NTHREADS * 4 - 1) / (NTHREADS * 4);
    if (blocks > AM_BLOCKS) blocks = AM_BLOCKS;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(k_argmax_partial, dim3(blocks), dim3(NTHREADS), 0, g_stream, g_am_v, g_am_i, v, n);
    HCHECK(hipGetLastError(), QH_ELAUNCH);
    hipLaunchKernelGGL(k_argmax_step, dim3(1), dim3(WAVE), 0, g_stream, tok, out, step, cap, pos, adv,
                       g_am_v, g_am_i, blocks, v);
    HCHECK(hipGetLastError(), QH_ELAUNCH);
    return QH_OK;
}

// M = 1 GEMV whose activation row comes from the rmsnorm prologue (GemvPro).
// Requires K % 8 == 0, K <= 4096 and 16-byte aligned pointers.
extern "C" int qh_gemv_pro(float *c, const qh_gemv_pro_t *p, const uint16_t *b, const uint16_t *b2,
                           int K, int N, int gated) {
    if (!g_inited) return QH_ESTATE;
    if (!c || !p || !b || (gated && !b2) || !p->nw || (!p->x && !(p->emb && p->tok))) return QH_EINVAL;
    if (K <= 0 || N <= 0 || K % 8 || K > 8 * WAVE * 8) return QH_EINVAL;
    if ((size_t)N * K * 2 >= (1ull << 31)) return QH_ETOOBIG;      // 32-bit weight offsets
    if (p->emb && p->emb_rows <= 0) return QH_EINVAL;
    if (!aligned16(c) || !aligned16(b) || (gated && !aligned16(b2)) || !aligned16(p->nw) ||
        (p->x && !aligned16(p->x)) || (p->r && !aligned16(p->r)) ||
        (p->x_out && !aligned16(p->x_out)) || (p->emb && !aligned16(p->emb)))
        return QH_EINVAL;
    GemvPro pro;
    memset(&pro, 0, sizeof pro);     // no stray stack bytes in the kernel arguments' padding
    pro.x = p->emb ? nullptr : p->x;
    pro.emb = p->emb;
    pro.tok = p->tok;
    pro.emb_rows = p->emb_rows;
    pro.r = p->emb ? nullptr : p->r;
    pro.nw = p->nw;
    pro.x_out = p->x_out;
    pro.eps = p->eps;
    return launch_gemv1_t<true>(c, nullptr, b, b2, K, N, gated != 0, pro);
}

