/* C-ABI launchers of the model kernels in hip_model.hip (device pointers,
 * asynchronous on the shim stream, QH_* return codes).  Internal header. */
#ifndef QWEN3_HIP_MODEL_SHIM_H
#define QWEN3_HIP_MODEL_SHIM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QM_MAX_CHUNK 128     /* tokens per forward call (QWEN3_MAX_BATCH, qwen3.h:145) */
#define QM_MAX_SEQ 8192      /* positions; bounded by the attention kernel's LDS */

/* x[row] = emb[tok[row]] (emb set) or x[row] += r[row] (r set);
 * xb[row] = rmsnorm(x[row]) * nw;  nt rows of K floats */
int qm_rows_norm(float *x_d, const float *r_d, const uint16_t *emb_d, const int *tok_d, int emb_rows,
                 const uint16_t *nw_d, float *xb_d, int nt, int K, float eps);

/* fused QK-norm + RoPE + KV-cache write + causal GQA attention for nt tokens
 * at positions *pos_d .. *pos_d + nt - 1 of one layer */
int qm_attention(const float *qkv_d, float *out_d, float *kc_d, float *vc_d, const uint16_t *qn_d,
                 const uint16_t *kn_d, const float *rcos_d, const float *rsin_d, const int *pos_d,
                 int nt, int max_seq, float eps);
size_t qm_attention_lds_bytes(int nt, int max_seq);

/* *p = v, as a kernel (safe inside stream capture) */
int qm_set_i32(int *p_d, int v);

#ifdef __cplusplus
}
#endif
#endif
