/* CPU oracle for the Qwen3-0.6B GEMM/GEMV hot path — TEST INFRASTRUCTURE ONLY.
 *
 * This library is the checker, never the product: only tests/, the smoke
 * check in __graft_entry__.py and the cpu_baseline leg of bench.py may load
 * it.  The product path (libqwen3_hip.so) never links or calls it.
 *
 * Every function restates one piece of the reference's algorithm, written
 * from scratch, and cites the reference file:line it follows.  Paths are
 * relative to the reference root; SRC = fpga_bringup/src/src.
 *
 * Pinning (what proves each function right, besides reading it):
 *   orc_f32_to_bf16        boundary-complete comparison with an independent
 *                          FPU-based rounding (orc_f32_to_bf16_fpu) + the
 *                          reference's own compiled qwen3.h (oracle/_ref)
 *   orc_gemm_scalar        bit-exact vs the compiled reference kernels_scalar.c
 *                          (oracle/_ref) and vs fixtures it wrote
 *                          (tests/golden/scalar_*.bin)
 *   orc_gemm_hw16          bit-exact vs all 12 shipped RTL golden vectors
 *                          (rtl_verification/cases/STAR/c_ref.bin) and vs the
 *                          compiled reference kernels_hwsim.c
 *   orc_gemm_exact         closed forms (ones -> K, bringup.c 1x1x32 = 32.0f)
 *                          and Python Fraction brute force on tiny inputs
 *   orc_silu_mul           vs compiled reference ops_scalar.c + special cases
 *   orc_argmax             vs numpy first-argmax + compiled ops_scalar.c
 *   orc_tile_offset        vs the formula's defining property (each (n,k)
 *                          maps to a distinct slot; a row-major tile round trip)
 *   RNG                    SplitMix64 published test vector
 */
#ifndef QWEN3_ORACLE_H
#define QWEN3_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- bf16 <-> fp32 (SRC/qwen3.h:21-37, SRC/kernels_hwsim.c:22-28) ---- */
float    orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);          /* RNE by integer add; no NaN special case */
uint16_t orc_f32_to_bf16_hw(float f);       /* same, but Inf/NaN pass through (hwsim) */
uint16_t orc_f32_to_bf16_fpu(float f);      /* independent formulation, for pinning */
void     orc_round_bf16_f32(float *dst, const float *src, size_t n);
void     orc_f32_to_bf16_array(uint16_t *dst, const float *src, size_t n);
void     orc_bf16_to_f32_array(float *dst, const uint16_t *src, size_t n);
/* count mismatches of orc_f32_to_bf16 vs orc_f32_to_bf16_fpu over every
 * (hi16, lo16) with hi16 in [0,65536) and lo16 from lo_list (NaNs skipped) */
uint64_t orc_bf16_rne_selfcheck(const uint16_t *lo_list, int n_lo);

/* ---- GEMM semantics: C[M,N] = A[M,K] . B[N,K]^T ---- */
/* SRC/kernels_scalar.c:9-21 — fp32 multiply, then fp32 add, k ascending */
void orc_gemm_scalar(float *c, const float *a, const uint16_t *b,
                     int M, int K, int N);
/* same, restricted to output columns [n0, n1): for bounded samples */
void orc_gemm_scalar_cols(float *c, const float *a, const uint16_t *b,
                          int M, int K, int N, int n0, int n1);
/* SRC/kernels_hwsim.c:33-56 — A->bf16 RNE, exact 16-element block sums,
 * fp32 rounding between blocks */
void orc_gemm_hw16(float *c, const float *a, const uint16_t *b,
                   int M, int K, int N);
/* fp64 GEMM (SRC/test_kernels.c:19-29) plus sum_k |a||b| for the
 * normalised error metric; either output may be NULL */
void orc_gemm_exact(double *c, double *absum, const float *a,
                    const uint16_t *b, int M, int K, int N);

/* ---- ops on the GEMM path ---- */
/* SRC/ops_scalar.c:46-51: gate[i] = (g / (1 + expf(-g))) * up[i] */
void orc_silu_mul(float *gate, const float *up, int n);
/* SRC/ops_scalar.c:57-62: first index of the maximum (strict >) */
int  orc_argmax(const float *v, int n);
/* SRC/qwen3.c:531-537: h = silu(x.Wg^T) * (x.Wu^T) with scalar GEMMs */
void orc_gate_up_silu(float *h, const float *x, const uint16_t *wg,
                      const uint16_t *wu, int M, int K, int N);

/* ---- weight layouts (SRC/kernels.h:59-68, SRC/kernels_ame.c:212-215) ---- */
/* element offset of B[n][k] in the tile-major layout with tiles of
 * tile_n x tile_k, tiles ordered n-major then k */
size_t orc_tile_offset(int n, int k, int K, int tile_n, int tile_k);
void   orc_row_to_tile(uint16_t *dst, const uint16_t *src, int N, int K,
                       int tile_n, int tile_k);

/* ---- deterministic inputs ---- */
uint64_t orc_splitmix64(uint64_t *state);
/* N(0,1)*sigma, rounded to bf16 (RNE); bits out */
void orc_fill_bf16_normal(uint16_t *dst, size_t n, uint64_t seed, float sigma);
/* N(0,1)*sigma, rounded to bf16 then widened: exactly bf16-representable fp32 */
void orc_fill_f32_bf16_normal(float *dst, size_t n, uint64_t seed, float sigma);
/* SRC/test_kernels.c:31-35 LCG: uniform [-1, 1) with 16 random bits */
void orc_test_lcg_fill(float *dst, size_t n, uint32_t *state);

/* ---- helpers for timing the CPU baseline ---- */
double orc_now_seconds(void);

#ifdef __cplusplus
}
#endif
#endif /* QWEN3_ORACLE_H */
