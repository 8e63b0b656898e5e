/* Threaded RTL-numerics GEMM — TEST INFRASTRUCTURE (oracle), never shipped.
 *
 * The plug-in symbols qwen3_gemm / qwen3_kernel_name with the arithmetic of
 * fpga_bringup/src/src/kernels_hwsim.c:22-56 (the AME target's numerics, as
 * orc_gemm_hw16 in oracle.c restates them): A rounded to bf16 with the
 * hwsim RNE (Inf/NaN passed through, kernels_hwsim.c:22-28), each run of 16
 * products along K summed exactly (in double: a bf16 x bf16 product has at
 * most 16 significant bits, so a 16-term block is exact for the operand
 * ranges of the model and the golden vectors), and the running fp32 sum
 * rounded after every block, blocks in K order.
 *
 * The only difference from orc_gemm_hw16 is that the N output columns are
 * split over threads; every output is computed by one thread in the same
 * order, so the result does not depend on the thread count.  It exists so
 * that the reference forward (qwen3.c) built with a long context can be run
 * in minutes when the long-context fixtures are written; it is pinned
 * bit-exact to the compiled kernels_hwsim.c by tests/test_oracle.py.
 *
 * Threads: $ORC_THREADS, else the number of online CPUs (at most 64).
 */
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define HW_BLOCK 16
#define MAX_THREADS 64

/* kernels_hwsim.c:22-28: RNE to bf16, Inf and NaN kept as they are */
static uint16_t hw_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7F800000u) == 0x7F800000u) return (uint16_t)(u >> 16);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

static double bf16_to_double(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return (double)f;
}

typedef struct {
    float *c;
    const double *at;         /* [K][M]: A rounded to bf16, transposed */
    const uint16_t *b;
    int M, K, N, n0, n1;
} job_t;

/* Per output column n, the M rows advance together through the K blocks:
 * blk[m] += a[m][k] * b[n][k] in k order, then acc[m] = fp32(acc[m] + blk[m])
 * after each block -- for every output the same operations in the same order
 * as orc_gemm_hw16, with the loop over m (independent outputs) innermost so
 * that the compiler can keep several outputs in one vector register. */
static void *work(void *arg) {
    const job_t *j = (const job_t *)arg;
    const int M = j->M, K = j->K, N = j->N;
    double *blk = (double *)malloc((size_t)M * sizeof(double));
    float *acc = (float *)malloc((size_t)M * sizeof(float));
    if (!blk || !acc) abort();
    for (int n = j->n0; n < j->n1; n++) {
        const uint16_t *brow = j->b + (size_t)n * (size_t)K;
        for (int m = 0; m < M; m++) acc[m] = 0.0f;
        for (int k0 = 0; k0 < K; k0 += HW_BLOCK) {
            const int k1 = k0 + HW_BLOCK < K ? k0 + HW_BLOCK : K;
            for (int m = 0; m < M; m++) blk[m] = 0.0;
            for (int k = k0; k < k1; k++) {
                const double bk = bf16_to_double(brow[k]);
                const double *ak = j->at + (size_t)k * (size_t)M;
                for (int m = 0; m < M; m++) blk[m] += ak[m] * bk;
            }
            for (int m = 0; m < M; m++) acc[m] = (float)((double)acc[m] + blk[m]);
        }
        for (int m = 0; m < M; m++) j->c[(size_t)m * (size_t)N + n] = acc[m];
    }
    free(blk);
    free(acc);
    return NULL;
}

static int n_threads(void) {
    const char *e = getenv("ORC_THREADS");
    long t = e ? atol(e) : sysconf(_SC_NPROCESSORS_ONLN);
    if (t < 1) t = 1;
    if (t > MAX_THREADS) t = MAX_THREADS;
    return (int)t;
}

void qwen3_gemm(float *c, const float *a, const uint16_t *b, int M, int K, int N) {
    if (M <= 0 || N <= 0) return;
    if (K <= 0) {
        memset(c, 0, (size_t)M * (size_t)N * sizeof(float));
        return;
    }
    double *at = (double *)malloc((size_t)M * (size_t)K * sizeof(double));
    if (!at) abort();
    for (int m = 0; m < M; m++)
        for (int k = 0; k < K; k++)
            at[(size_t)k * (size_t)M + m] = bf16_to_double(hw_f32_to_bf16(a[(size_t)m * (size_t)K + k]));
    int t = n_threads();
    if (t > N) t = N;
    pthread_t th[MAX_THREADS];
    job_t jobs[MAX_THREADS];
    for (int i = 0; i < t; i++) {
        jobs[i] = (job_t){c, at, b, M, K, N, (int)((long)N * i / t), (int)((long)N * (i + 1) / t)};
        if (i > 0 && pthread_create(&th[i], NULL, work, &jobs[i]) != 0) abort();
    }
    work(&jobs[0]);
    for (int i = 1; i < t; i++) pthread_join(th[i], NULL);
    free(at);
}

const char *qwen3_kernel_name(void) { return "hwsim-threaded"; }
