/* Thin C-ABI shim between the C host code (kernels_hip.c) and HIP.
 *
 * Everything here takes plain pointers and sizes.  Device pointers are
 * marked _d.  Launchers are asynchronous on the shim's single stream and
 * return 0 or a QH_E* error code; nothing here aborts.
 */
#ifndef QWEN3_HIP_SHIM_H
#define QWEN3_HIP_SHIM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    QH_OK = 0,
    QH_EINVAL = 1,      /* bad argument (sizes, pointers, alignment) */
    QH_ENODEV = 2,      /* no HIP device / init failed */
    QH_ENOMEM = 3,      /* device or pinned allocation failed */
    QH_ELAUNCH = 4,     /* kernel launch failed */
    QH_ERUNTIME = 5,    /* any other HIP runtime error (copy, sync, event) */
    QH_ELAYOUT = 6,     /* weight layout not usable for this shape */
    QH_ESTATE = 7,      /* call order (e.g. use before init) */
    QH_ETOOBIG = 8      /* size beyond a documented maximum */
};

int         qh_init(int device);        /* idempotent; creates the stream */
void        qh_shutdown(void);
int         qh_device(void);
const char *qh_device_name(void);
int         qh_device_count(void);      /* initialises HIP */
int         qh_last_hip_error(void);    /* raw hipError_t of the last failure */
const char *qh_last_hip_error_string(void);

int qh_malloc(void **p_d, size_t bytes);
int qh_free(void *p_d);
int qh_host_alloc(void **p, size_t bytes);     /* pinned host memory */
int qh_host_free(void *p);
int qh_h2d(void *dst_d, const void *src, size_t bytes);   /* async on the stream */
int qh_d2h(void *dst, const void *src_d, size_t bytes);   /* async on the stream */
int qh_d2d(void *dst_d, const void *src_d, size_t bytes); /* async on the stream */
int qh_sync(void);
void *qh_stream(void);                                    /* hipStream_t */

/* C[M,N] = A[M,K] . B[N,K]^T;  A fp32, B bf16 bits, C fp32; row-major,
 * lda = ldb = K, ldc = N.  A is rounded to bf16 (RNE) on the load path. */
int qh_gemm(float *c_d, const float *a_d, const uint16_t *b_d,
            int M, int K, int N);
/* qh_gemm, but when the automatic plan splits K over the skinny kernel's
 * blocks the ks > 1 fp32 slice sums are left in library workspace
 * (*part_d: [ks][M][N]) for the caller to add in slice order instead of a
 * reduction launch; otherwise C is written and *ks = 0.  The partials are
 * valid until the next library call that uses the split-K workspace. */
int qh_gemm_split(float *c_d, const float *a_d, const uint16_t *b_d, int M, int K, int N,
                  const float **part_d, int *ks);
/* qh_gemm with the fixed device array `scratch` (qh_scratch_bytes()) as
 * workspace: allocates and frees nothing; QH_ETOOBIG when the plan needs
 * more workspace than the array holds.  Results equal qh_gemm's. */
int qh_gemm_noalloc(float *c_d, const float *a_d, const uint16_t *b_d, int M, int K, int N);
size_t qh_scratch_bytes(void);
/* The M = 1 GEMV set of `layers` (<= 32) decoder layers in one persistent
 * launch (hip_persist.hip): w = HOST array [layers][5] of device pointers to
 * q|k|v [4096][1024],
 * o [1024][2048], gate [3072][1024], up [3072][1024], down [1024][3072];
 * layer 0 reads x0 (1024 fp32), layer l > 0 the previous down output, o
 * reads the q part; out_d = [layers][qh_persist_out_ld()] fp32: q|k|v, o,
 * silu(gate)*up, down at 0, 4096, 5120, 8192.  Outputs equal the per-call
 * GEMV kernels' bit for bit.  QH_ENODEV if the device cannot keep the grid
 * resident (256 CUs, one workgroup each). */
int qh_decode_persist(const uint16_t *const *w, const float *x0_d, float *out_d, int layers);
int qh_persist_supported(void);
int qh_persist_out_ld(void);
/* error flags of launches since the last call (1 = an input poll gave up);
 * synchronises the stream */
int qh_persist_errors(unsigned *flags);
int qh_persist_init(void);
void qh_persist_shutdown(void);
/* the persistent decoder-stack launch's buffers (hip_model_persist.hip),
 * allocated by the first model that uses it, freed at shutdown */
void qm_persist_shutdown(void);
/* name of the plan the last GEMM call launched */
const char *qh_last_plan(void);
/* h[M,N] = silu(X.Wg^T) * (X.Wu^T) */
int qh_gemm_gate_up_silu(float *h_d, const float *x_d, const uint16_t *wg_d,
                         const uint16_t *wu_d, int M, int K, int N);
/* the same with A already bf16 bits [M,K] (no rounding pass): large-tile
 * MFMA kernels; K % 64 == 0 and 16-byte aligned pointers */
int qh_gemm_bf16a(float *c_d, const uint16_t *a_d, const uint16_t *b_d,
                  int M, int K, int N);
int qh_gemm_gate_up_silu_bf16a(float *h_d, const uint16_t *x_d, const uint16_t *wg_d,
                               const uint16_t *wu_d, int M, int K, int N);
/* tile-major [N/tn][K/tk][tn][tk] -> row-major [N][K] */
int qh_tile_to_row(uint16_t *dst_d, const uint16_t *src_d, int N, int K,
                   int tile_n, int tile_k);
/* first index of the maximum of v[0..n) (ties -> lowest index) */
int qh_argmax(int *out_d, const float *v_d, int n);
/* greedy-step bookkeeping on the device: *tok = argmax(v), out[*step] = *tok
 * when *step < cap, then *step += 1 and *pos += adv */
int qh_argmax_step(int *tok_d, int *out_d, int *step_d, int cap, int *pos_d, int adv,
                   const float *v_d, int n);

/* M = 1 GEMV with an rmsnorm prologue: the activation row is
 *   a = rmsnorm(x + r) * nw     (x fp32, or the bf16 row emb[*tok] when emb
 *                                is set, in which case r is ignored)
 * and, when x_out is set, x + r is stored there (one writer).  c[N] =
 * a . B^T, or silu(a . Wg^T) * (a . Wu^T) when gated (b2 = Wu).  K % 8 == 0,
 * K <= 4096, 16-byte aligned pointers. */
typedef struct {
    const float *x;
    const uint16_t *emb;
    const int *tok;
    int emb_rows;
    const float *r;
    const uint16_t *nw;
    float *x_out;
    float eps;
} qh_gemv_pro_t;
int qh_gemv_pro(float *c_d, const qh_gemv_pro_t *pro, const uint16_t *b_d, const uint16_t *b2_d,
                int K, int N, int gated);

/* M = 1 GEMV whose activation row is decode attention merged from split
 * softmax partials (the o projection): part holds, for 8 kv heads x
 * QH_ATT_SPLITS position ranges x 2 query heads, QH_ATT_PART floats
 * {m, l, -, -, o[128]} (max score, sum of exp(score - m), sum of
 * exp(score - m) * v); the activation is sum_s e^(m_s-M) o_s / sum_s
 * e^(m_s-M) l_s per head, M = max_s m_s.  K = 2048 (16 heads x 128). */
#define QH_ATT_SPLITS 8
#define QH_ATT_PART (4 + 128)
int qh_gemv_merge(float *c_d, const float *part_d, const uint16_t *b_d, int K, int N);

/* M = 1 GEMV (b2: gated, silu(gate) * up) whose activation row is given on
 * the host already rounded to bf16 (row_bf16: max(1024, K rounded up to a
 * multiple of 512) values, zero past K) and travels in the launch's kernel
 * arguments: K <= 3072, K % 8 == 0.  c may be pinned host memory; each
 * element of c is written exactly once. */
int qh_gemv_ka(float *c, const uint16_t *row_bf16, const uint16_t *b_d, const uint16_t *b2_d, int K, int N);

/* device copy by a plain 16-byte-vector kernel (bytes % 16 == 0, 16-byte
 * aligned pointers): the known-traffic reference for HBM counter calibration */
int qh_copy(void *dst_d, const void *src_d, size_t bytes);
/* reads bytes (% 16 == 0, < 2 GiB, 16-byte aligned) once with the decode
 * GEMVs' buffer-load form and writes nothing: the known-traffic reference for
 * read counters */
int qh_read(const void *src_d, size_t bytes);

/* stream capture: launches between begin and end are recorded (not run)
 * into a graph that qh_graph_launch replays on the shim stream */
int qh_capture_begin(void);
int qh_capture_end(int *graph_id);
int qh_graph_launch(int graph_id);
int qh_graph_destroy(int graph_id);

/* kernel choice for a GEMM shape (for logs/tests): returns a static name */
const char *qh_gemm_plan(int M, int K, int N, int gated);
/* override the automatic choice: 0 = auto, otherwise a plan id (see
 * qh_gemm_plan names); for tests and sweeps */
int qh_force_plan(int plan_id);

/* HIP events on the shim stream, for timing what this stream runs */
int   qh_timer_record(int slot);            /* slot in [0, 64) */
int   qh_timer_elapsed_ms(int a, int b, float *ms);

#ifdef __cplusplus
}
#endif
#endif /* QWEN3_HIP_SHIM_H */
