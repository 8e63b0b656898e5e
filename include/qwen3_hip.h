/* MI355X (gfx950) GEMM plug-in for the Qwen3-0.6B C runtime — public C ABI.
 *
 * Link libqwen3_hip.so in place of a kernels_$(KERNEL).c and the model
 * forward (fpga_bringup/src/src/qwen3.c) calls the GPU through the same four
 * symbols it already uses.  Paths below are relative to the reference root;
 * SRC = fpga_bringup/src/src.
 *
 * Semantics shared by every GEMM entry point:
 *   C[M,N] = A[M,K] . B[N,K]^T, A fp32 row-major (lda = K), B bf16 bits
 *   row-major [out_features, in_features] (ldb = K), C fp32 row-major
 *   (ldc = N), C fully overwritten.  A is rounded to bf16 (round to nearest
 *   even, as SRC/qwen3.h:31-37 and the AME kernel SRC/kernels_ame.c:219-236
 *   do), each bf16 x bf16 product is exact, accumulation is fp32.
 *   Any M, K, N >= 0 (no hidden caps, no read past the end of B, unlike
 *   SRC/kernels_ame.c:221 and SRC/kernels.h:25-42).
 *
 * Host-pointer entry points are synchronous: on return C is complete in host
 * memory (SRC/kernels_ame.c:426-444 gives the same guarantee).
 *
 * Weights: B is read-only during a call (SRC/qwen3.h:203-207).
 *   - B inside a range given to qwen3_hip_map_weights() is served from one
 *     device copy of that whole range (the model blob), at zero per-call cost;
 *     the range must stay unchanged until it is unmapped;
 *   - any other B is copied to the device on every call (default), so, as
 *     with the reference kernels, a caller may change B between calls;
 *   - opt-in (qwen3_hip_set_weight_cache(1) or QWEN3_HIP_WEIGHT_CACHE=1):
 *     other B are instead cached by address and verified on each call against
 *     a sampled fingerprint of their contents (shape, first/last 256 bytes and
 *     512 sampled 8-byte words); a buffer changed only outside the sampled
 *     words is NOT detected, so call qwen3_hip_forget_weights() after
 *     modifying a cached weight buffer in place.
 *
 * Errors: the reference ABI is void, so a failure inside qwen3_gemm /
 * qwen3_gemm_row / qwen3_gemm_gate_up_silu prints one line to stderr and
 * aborts the process by default; after qwen3_hip_set_abort(0) it instead
 * leaves C unwritten and records a sticky code for qwen3_hip_last_error().
 *
 * Threading: not thread-safe and not reentrant (one stream, shared staging),
 * like the reference kernels (SRC/kernels_ame.c:56).
 */
#ifndef QWEN3_HIP_H
#define QWEN3_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- the reference GEMM plug-in (SRC/kernels.h) ---------------------------- */

/* replaces qwen3_gemm, SRC/kernels.h:56-57 (portable version
 * SRC/kernels_scalar.c:9-21, AME version SRC/kernels_ame.c:449-452).
 * B is addressed in the layout set by qwen3_set_weight_layout(). */
void qwen3_gemm(float *c, const float *a, const uint16_t *b,
                int M, int K, int N);

/* replaces qwen3_gemm_row, SRC/kernels.h:79-80 (weak default
 * SRC/qwen3.c:60-65, AME SRC/kernels_ame.c:456-459): B is always row-major
 * (the tied embedding table used as lm_head). */
void qwen3_gemm_row(float *c, const float *a, const uint16_t *b,
                    int M, int K, int N);

/* replaces qwen3_set_weight_layout, SRC/kernels.h:89 (weak default
 * SRC/qwen3.c:67-73, AME SRC/kernels_ame.c:189-207).  layout 0 = ROW,
 * 1 = TILE (tile_n x tile_k sub-blocks stored contiguously, n-major,
 * SRC/kernels_ame.c:212-215).  Accepts ROW, and TILE with tile sizes that
 * divide every model dimension (SRC/kernels_ame.c:196-205); returns -1
 * otherwise, which qwen3_init turns into QWEN3_ERR_LAYOUT (SRC/qwen3.c:113-116).
 * TILE weights are re-laid out to row-major once, on the device, on upload. */
int qwen3_set_weight_layout(int layout, int tile_n, int tile_k);

/* replaces qwen3_kernel_name, SRC/kernels.h:92: "hip-gfx950". */
const char *qwen3_kernel_name(void);

/* ---- extensions for the same call sites ------------------------------------ */

/* h[M,N] = silu(X.Wg^T) * (X.Wu^T) in one pass: replaces the gate GEMM, up
 * GEMM and qwen3_op_silu_mul sequence of SRC/qwen3.c:531-537 (silu_mul as in
 * SRC/ops_scalar.c:46-51).  Wg, Wu in the current weight layout. */
void qwen3_gemm_gate_up_silu(float *h, const float *x, const uint16_t *wg,
                             const uint16_t *wu, int M, int K, int N);

/* ---- runtime control ------------------------------------------------------- */

/* error codes returned by qwen3_hip_* and kept by qwen3_hip_last_error() */
enum {
    QWEN3_HIP_OK = 0,
    QWEN3_HIP_EINVAL = 1,
    QWEN3_HIP_ENODEV = 2,
    QWEN3_HIP_ENOMEM = 3,
    QWEN3_HIP_ELAUNCH = 4,
    QWEN3_HIP_ERUNTIME = 5,
    QWEN3_HIP_ELAYOUT = 6,
    QWEN3_HIP_ESTATE = 7,
    QWEN3_HIP_ETOOBIG = 8
};

/* Select the device and create the library's stream.  Called implicitly by
 * the first GEMM with device -1 (= device 0, or $QWEN3_HIP_DEVICE). */
int qwen3_hip_init(int device);
/* Free every device copy of weights, staging buffers and the stream. */
void qwen3_hip_release(void);
/* First error since the last call (then cleared). */
int qwen3_hip_last_error(void);
const char *qwen3_hip_strerror(int err);
/* 1 (default) = abort on error inside the void reference entry points. */
void qwen3_hip_set_abort(int on);
/* Upload [blob, blob+size) once; later B pointers inside it use that copy.
 * The range must stay allocated and unchanged until it is unmapped. */
int qwen3_hip_map_weights(const void *blob, size_t size);
/* Drop the device copy of a range mapped at blob (and copies derived from
 * it); QWEN3_HIP_EINVAL if nothing is mapped there. */
int qwen3_hip_unmap_weights(const void *blob);
/* Drop the cached device copy for B (or every unmapped copy if b == NULL). */
void qwen3_hip_forget_weights(const void *b);
/* 1 = cache unmapped B by address (sampled fingerprint, see above); 0 (the
 * default, unless QWEN3_HIP_WEIGHT_CACHE=1) = copy unmapped B on every call.
 * Turning it off drops the cached copies. */
void qwen3_hip_set_weight_cache(int on);
/* Bytes of device memory held for weights (mapped ranges + cached copies). */
size_t qwen3_hip_weight_bytes(void);

/* ---- device-pointer API (inputs and outputs already in HBM) ----------------
 * Asynchronous on the library stream; return a QWEN3_HIP_* code and never
 * abort.  Pointers ending in _d are device pointers. */
int qwen3_hip_gemm_dev(float *c_d, const float *a_d, const uint16_t *b_d,
                       int M, int K, int N);
int qwen3_hip_gemm_gate_up_silu_dev(float *h_d, const float *x_d,
                                    const uint16_t *wg_d, const uint16_t *wu_d,
                                    int M, int K, int N);
/* The same two products with A already bf16 (uint16_t bits, [M,K]
 * row-major): for callers that hold bf16 activations, so no rounding pass
 * is needed.  Results equal the fp32-A calls on A = bf16(A).  Large-tile
 * MFMA kernels; K % 64 == 0 and 16-byte aligned pointers, else
 * QWEN3_HIP_EINVAL.  No counterpart in the reference ABI
 * (SRC/kernels.h:44-57 takes fp32 A only). */
int qwen3_hip_gemm_bf16a_dev(float *c_d, const uint16_t *a_d, const uint16_t *b_d,
                             int M, int K, int N);
int qwen3_hip_gemm_gate_up_silu_bf16a_dev(float *h_d, const uint16_t *x_d,
                                          const uint16_t *wg_d, const uint16_t *wu_d,
                                          int M, int K, int N);
/* qwen3_hip_gemm_dev that allocates nothing: no counterpart in the
 * reference ABI; for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Its workspace (the bf16 copy of A or the fp32 K-slice sums some plans use)
 * is a fixed device array of qwen3_hip_scratch_bytes() = 32 MiB, one per GPU,
 * held until the process ends; a call whose plan would need more returns
 * QWEN3_HIP_ETOOBIG and launches nothing.  Results equal qwen3_hip_gemm_dev's.
 * The library must be initialised first (qwen3_hip_init: QWEN3_HIP_ESTATE
 * otherwise).  Every call on a GPU shares that GPU's array, which keeps the
 * last call's contents; calls that overlap on one GPU (graphs replayed on
 * another stream, other threads or processes) race on it. */
int qwen3_hip_gemm_noalloc_dev(float *c_d, const float *a_d, const uint16_t *b_d,
                               int M, int K, int N);
size_t qwen3_hip_scratch_bytes(void);
/* The M = 1 GEMV set of one decode token for `layers` (1..32) decoder
 * layers in ONE persistent launch: the q|k|v, o, gate, up and down calls of
 * SRC/qwen3.c:477-540 with their Qwen3-0.6B shapes, chained as a decode step
 * chains them when the ops between them are left out (x -> q|k|v; its q part
 * -> o; o -> silu(gate) * up; that -> down -> x of the next layer).
 * w: HOST array [layers][5] of device pointers, per layer q|k|v [4096][1024]
 * (q, k, v rows stacked), o [1024][2048], gate [3072][1024], up [3072][1024],
 * down [1024][3072] (bf16, row-major [out, in]); x0_d: layer 0's input (1024
 * fp32); out_d: [layers][qwen3_hip_decode_set_out_ld()] fp32, per layer
 * q|k|v at 0, o at 4096, silu(gate)*up at 5120, down at 8192.  Every output
 * equals, bit for bit, the qwen3_hip_gemm_dev / _gate_up_silu_dev call
 * chain on the same inputs.  Asynchronous on the library stream; may be
 * captured into a graph.  QWEN3_HIP_ENODEV where the device cannot keep the
 * launch's 256 workgroups resident (qwen3_hip_decode_set_supported() == 0).
 * No counterpart in the reference ABI (its GEMMs are separate calls). */
int qwen3_hip_decode_set_dev(const uint16_t *const *w, const float *x0_d, float *out_d, int layers);
int qwen3_hip_decode_set_supported(void);
int qwen3_hip_decode_set_out_ld(void);
/* error flags of decode-set launches since the last call (synchronises):
 * 1 = a workgroup stopped waiting for its input (results not valid) */
int qwen3_hip_decode_set_errors(unsigned *flags);
/* device counterpart of qwen3_op_argmax (SRC/ops.h:36-37,
 * SRC/ops_scalar.c:57-62): first index of the maximum, ties -> lowest index,
 * a NaN at index 0 wins as in the reference's strict ">" scan */
int qwen3_hip_argmax_dev(int *out_d, const float *v_d, int n);
int qwen3_hip_tile_to_row_dev(uint16_t *dst_d, const uint16_t *src_d,
                              int N, int K, int tile_n, int tile_k);

/* device-to-device copy by a plain streaming kernel (bytes a multiple of 16,
 * 16-byte aligned pointers); its traffic is exactly bytes read + bytes
 * written, which makes it the reference for HBM traffic counters */
int qwen3_hip_copy_dev(void *dst_d, const void *src_d, size_t bytes);
/* reads bytes (a multiple of 16, below 2 GiB, 16-byte aligned pointer) once
 * with the decode GEMVs' load form and writes nothing: the reference for
 * read-traffic counters (no counterpart in the reference; for measurement) */
int qwen3_hip_read_dev(const void *src_d, size_t bytes);

/* HIP graphs: device-pointer calls made between capture_begin and
 * capture_end are recorded, not run; graph_launch replays them on the
 * library stream (a decode step becomes one submission).  Only the _dev
 * entry points may be captured (the host-pointer ones synchronise). */
int qwen3_hip_capture_begin(void);
int qwen3_hip_capture_end(int *graph_id);
int qwen3_hip_graph_launch(int graph_id);
int qwen3_hip_graph_destroy(int graph_id);

int qwen3_hip_malloc(void **p_d, size_t bytes);
int qwen3_hip_free(void *p_d);
int qwen3_hip_memcpy_h2d(void *dst_d, const void *src, size_t bytes);
int qwen3_hip_memcpy_d2h(void *dst, const void *src_d, size_t bytes);
int qwen3_hip_sync(void);
/* HIP events on the library stream: record slot s, elapsed ms from a to b */
int qwen3_hip_timer_record(int slot);
int qwen3_hip_timer_elapsed_ms(int a, int b, float *ms);
/* which kernel a shape goes to ("gemv", "mfma64x64", ...), and a test hook
 * to force one (0 = automatic) */
const char *qwen3_hip_plan(int M, int K, int N, int gated);
int qwen3_hip_force_plan(int plan_id);
/* the plan the last GEMM call launched (after any fall-back) */
const char *qwen3_hip_last_plan(void);
/* name of the device in use (gfx arch string), "" before init */
const char *qwen3_hip_device_name(void);

#ifdef __cplusplus
}
#endif
#endif /* QWEN3_HIP_H */
