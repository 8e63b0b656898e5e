/* CPU oracle for the Qwen3-0.6B GEMM/GEMV hot path — TEST INFRASTRUCTURE ONLY.
 *
 * Loaded only by tests/, the smoke check and bench.py's cpu_baseline leg, as
 * the checker.  Built "gcc -O2 -std=c11 -ffp-contract=off" so that every
 * float multiply and add is a separate IEEE operation in source order, as the
 * reference's own build does (fpga_bringup/src/src/Makefile:10).
 * Citations: SRC = fpga_bringup/src/src (relative to the reference root).
 */
#define _POSIX_C_SOURCE 199309L
#include "oracle.h"

#include <math.h>
#include <string.h>
#include <time.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* SRC/qwen3.h:21-26: bf16 is the top half of an fp32 word. */
float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* SRC/qwen3.h:28-35: round-to-nearest-even by adding 0x7FFF plus the lsb of
 * the kept half, then truncating.  No NaN/Inf special case (a NaN whose
 * payload carries into the sign bit comes out as -0, exactly as there). */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    uint32_t bias = 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)((u + bias) >> 16);
}

/* SRC/kernels_hwsim.c:22-28: the same recipe, but exponent-all-ones words
 * (Inf and NaN) are truncated instead of rounded. */
uint16_t orc_f32_to_bf16_hw(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7F800000u) == 0x7F800000u) return (uint16_t)(u >> 16);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* Independent restatement used only to pin the two recipes above: round |f|
 * to the bf16 grid with the FPU's round-half-even (nearbyint in double, where
 * every step is exact), then put the sign back.  bf16 keeps 8 significant
 * bits for normals; below 2^-126 the grid is the fixed subnormal spacing
 * 2^-133. */
uint16_t orc_f32_to_bf16_fpu(float f) {
    uint32_t u = f2u(f);
    uint32_t sign = u & 0x80000000u;
    if (isnan(f)) return (uint16_t)((u >> 16) | 0x0040u);
    if (isinf(f) || f == 0.0f) return (uint16_t)(u >> 16);
    double ax = fabs((double)f);
    double ulp;
    if (ax < 0x1p-126) {
        ulp = 0x1p-133;
    } else {
        int e;
        (void)frexp(ax, &e);          /* ax = m * 2^e, m in [0.5, 1) */
        ulp = ldexp(1.0, e - 8);
    }
    double q = nearbyint(ax / ulp) * ulp;
    float qf = (float)q;              /* exact, or +Inf past the top binade */
    return (uint16_t)((sign | f2u(qf)) >> 16);
}

uint64_t orc_bf16_rne_selfcheck(const uint16_t *lo_list, int n_lo) {
    uint64_t bad = 0;
    for (uint32_t hi = 0; hi < 65536u; hi++) {
        for (int j = 0; j < n_lo; j++) {
            uint32_t bits = (hi << 16) | lo_list[j];
            float f = u2f(bits);
            if (isnan(f)) continue;
            if (orc_f32_to_bf16(f) != orc_f32_to_bf16_fpu(f)) bad++;
            if (!isinf(f) && orc_f32_to_bf16_hw(f) != orc_f32_to_bf16_fpu(f)) bad++;
        }
    }
    return bad;
}

void orc_round_bf16_f32(float *dst, const float *src, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = orc_bf16_to_f32(orc_f32_to_bf16(src[i]));
}

void orc_f32_to_bf16_array(uint16_t *dst, const float *src, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = orc_f32_to_bf16(src[i]);
}

void orc_bf16_to_f32_array(float *dst, const uint16_t *src, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = orc_bf16_to_f32(src[i]);
}

/* SRC/kernels_scalar.c:9-21.  One fp32 product, one fp32 add, k ascending;
 * A is used exactly as given (callers pass bf16-representable activations
 * when they want the "bf16 inputs" semantics of the GPU path). */
void orc_gemm_scalar_cols(float *c, const float *a, const uint16_t *b,
                          int M, int K, int N, int n0, int n1) {
    for (int m = 0; m < M; m++) {
        const float *arow = a + (size_t)m * (size_t)K;
        float *crow = c + (size_t)m * (size_t)N;
        for (int n = n0; n < n1; n++) {
            const uint16_t *brow = b + (size_t)n * (size_t)K;
            float sum = 0.0f;
            for (int k = 0; k < K; k++) {
                float p = arow[k] * orc_bf16_to_f32(brow[k]);
                sum = sum + p;
            }
            crow[n] = sum;
        }
    }
}

void orc_gemm_scalar(float *c, const float *a, const uint16_t *b,
                     int M, int K, int N) {
    orc_gemm_scalar_cols(c, a, b, M, K, N, 0, N);
}

/* SRC/kernels_hwsim.c:31-56.  A is rounded to bf16 (hwsim recipe); each
 * block of 16 consecutive k is summed exactly (double holds 16 products of
 * 8-bit significands exactly for inputs of sane range), and the running
 * accumulator is rounded to fp32 after every block. */
#define ORC_HW_BLOCK 16
void orc_gemm_hw16(float *c, const float *a, const uint16_t *b,
                   int M, int K, int N) {
    for (int m = 0; m < M; m++) {
        const float *arow = a + (size_t)m * (size_t)K;
        float *crow = c + (size_t)m * (size_t)N;
        for (int n = 0; n < N; n++) {
            const uint16_t *brow = b + (size_t)n * (size_t)K;
            float acc = 0.0f;
            for (int k0 = 0; k0 < K; k0 += ORC_HW_BLOCK) {
                int k1 = k0 + ORC_HW_BLOCK < K ? k0 + ORC_HW_BLOCK : K;
                double blk = 0.0;
                for (int k = k0; k < k1; k++) {
                    double av = (double)orc_bf16_to_f32(orc_f32_to_bf16_hw(arow[k]));
                    blk += av * (double)orc_bf16_to_f32(brow[k]);
                }
                acc = (float)((double)acc + blk);
            }
            crow[n] = acc;
        }
    }
}

/* SRC/test_kernels.c:19-29 (double accumulation), plus the magnitude sum
 * that normalises errors the way rtl_verification/check.py:158-215 uses
 * c_peak: an error is judged against what the accumulation went through. */
void orc_gemm_exact(double *c, double *absum, const float *a,
                    const uint16_t *b, int M, int K, int N) {
    for (int m = 0; m < M; m++) {
        const float *arow = a + (size_t)m * (size_t)K;
        for (int n = 0; n < N; n++) {
            const uint16_t *brow = b + (size_t)n * (size_t)K;
            double s = 0.0, sa = 0.0;
            for (int k = 0; k < K; k++) {
                double p = (double)arow[k] * (double)orc_bf16_to_f32(brow[k]);
                s += p;
                sa += fabs(p);
            }
            if (c) c[(size_t)m * N + n] = s;
            if (absum) absum[(size_t)m * N + n] = sa;
        }
    }
}

/* SRC/ops_scalar.c:46-51 */
void orc_silu_mul(float *gate, const float *up, int n) {
    for (int i = 0; i < n; i++) {
        float g = gate[i];
        float den = 1.0f + expf(-g);
        gate[i] = (g / den) * up[i];
    }
}

/* SRC/ops_scalar.c:57-62: ties resolve to the lowest index; NaNs never win
 * a strict comparison (so a NaN at index 0 stays the answer only if nothing
 * compares greater than it, which nothing does). */
int orc_argmax(const float *v, int n) {
    int best = 0;
    float bv = v[0];
    for (int i = 1; i < n; i++) {
        if (v[i] > bv) { bv = v[i]; best = i; }
    }
    return best;
}

/* SRC/qwen3.c:531-537: gate GEMM, up GEMM, then silu(gate) * up in place. */
void orc_gate_up_silu(float *h, const float *x, const uint16_t *wg,
                      const uint16_t *wu, int M, int K, int N) {
    /* h doubles as the gate buffer; up needs its own M*N scratch, which the
     * caller cannot provide through this signature, so do it per row. */
    for (int m = 0; m < M; m++) {
        const float *xr = x + (size_t)m * K;
        float *hr = h + (size_t)m * N;
        for (int n = 0; n < N; n++) {
            const uint16_t *gr = wg + (size_t)n * K;
            const uint16_t *ur = wu + (size_t)n * K;
            float sg = 0.0f, su = 0.0f;
            for (int k = 0; k < K; k++) {
                float pg = xr[k] * orc_bf16_to_f32(gr[k]);
                sg = sg + pg;
            }
            for (int k = 0; k < K; k++) {
                float pu = xr[k] * orc_bf16_to_f32(ur[k]);
                su = su + pu;
            }
            float den = 1.0f + expf(-sg);
            hr[n] = (sg / den) * su;
        }
    }
}

/* SRC/kernels_ame.c:212-215 (tile index) and :269 (rows inside a tile are
 * tile_k elements apart). */
size_t orc_tile_offset(int n, int k, int K, int tile_n, int tile_k) {
    size_t tile = (size_t)(n / tile_n) * (size_t)(K / tile_k) + (size_t)(k / tile_k);
    return tile * (size_t)tile_n * (size_t)tile_k
         + (size_t)(n % tile_n) * (size_t)tile_k + (size_t)(k % tile_k);
}

void orc_row_to_tile(uint16_t *dst, const uint16_t *src, int N, int K,
                     int tile_n, int tile_k) {
    for (int n = 0; n < N; n++)
        for (int k = 0; k < K; k++)
            dst[orc_tile_offset(n, k, K, tile_n, tile_k)] = src[(size_t)n * K + k];
}

/* SplitMix64 (Steele, Lea, Flood 2014; constants as published). */
uint64_t orc_splitmix64(uint64_t *state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Box-Muller on 53-bit uniforms; both outputs of each pair are used. */
static void fill_normal_f32(float *dst, size_t n, uint64_t seed, float sigma) {
    uint64_t st = seed;
    const double two_pi = 6.283185307179586476925286766559;
    size_t i = 0;
    while (i < n) {
        double u1 = ((double)(orc_splitmix64(&st) >> 11) + 1.0) * 0x1p-53; /* (0,1] */
        double u2 = (double)(orc_splitmix64(&st) >> 11) * 0x1p-53;         /* [0,1) */
        double r = sqrt(-2.0 * log(u1));
        dst[i++] = (float)(r * cos(two_pi * u2) * (double)sigma);
        if (i < n) dst[i++] = (float)(r * sin(two_pi * u2) * (double)sigma);
    }
}

void orc_fill_bf16_normal(uint16_t *dst, size_t n, uint64_t seed, float sigma) {
    /* generate in blocks so no large temporary is needed */
    float tmp[256];
    uint64_t st = seed;
    size_t i = 0;
    while (i < n) {
        size_t m = n - i < 256 ? n - i : 256;
        /* one seed per block derived from the stream keeps it O(1) memory */
        fill_normal_f32(tmp, m, orc_splitmix64(&st), sigma);
        for (size_t j = 0; j < m; j++) dst[i + j] = orc_f32_to_bf16(tmp[j]);
        i += m;
    }
}

void orc_fill_f32_bf16_normal(float *dst, size_t n, uint64_t seed, float sigma) {
    float tmp[256];
    uint64_t st = seed;
    size_t i = 0;
    while (i < n) {
        size_t m = n - i < 256 ? n - i : 256;
        fill_normal_f32(tmp, m, orc_splitmix64(&st), sigma);
        for (size_t j = 0; j < m; j++)
            dst[i + j] = orc_bf16_to_f32(orc_f32_to_bf16(tmp[j]));
        i += m;
    }
}

/* SRC/test_kernels.c:31-35 */
void orc_test_lcg_fill(float *dst, size_t n, uint32_t *state) {
    for (size_t i = 0; i < n; i++) {
        *state = *state * 1664525u + 1013904223u;
        dst[i] = (float)((*state >> 8) & 0xFFFFu) / 32768.0f - 1.0f;
    }
}

double orc_now_seconds(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}
