/* C-ABI launchers of the model kernels in hip_model.hip (device pointers,
 * asynchronous on the shim stream, QH_* return codes).  Internal header. */
#ifndef QWEN3_HIP_MODEL_SHIM_H
#define QWEN3_HIP_MODEL_SHIM_H

#include <stddef.h>
#include <stdint.h>

#include "hip_shim.h"

#ifdef __cplusplus
extern "C" {
#endif

#define QM_MAX_CHUNK 128     /* tokens per forward call (QWEN3_MAX_BATCH, qwen3.h:145) */
#define QM_MAX_SEQ 8192      /* positions; the attention kernels keep 2 x max_seq scores in LDS */

/* x[row] = emb[tok[row]] (emb set) or x[row] += r[row] (r set);
 * xb[row] = rmsnorm(x[row]) * nw;  nt rows of K floats */
int qm_rows_norm(float *x_d, const float *r_d, const uint16_t *emb_d, const int *tok_d, int emb_rows,
                 const uint16_t *nw_d, float *xb_d, int nt, int K, float eps);
/* the same with x[row] += sum of ks (<= 16) split-K slices of part_d
 * ([ks][nt][K], added in slice order) instead of r (r_d and emb_d NULL) */
int qm_rows_norm_split(float *x_d, const float *r_d, const uint16_t *emb_d, const int *tok_d, int emb_rows,
                       const uint16_t *nw_d, float *xb_d, int nt, int K, float eps, const float *part_d,
                       int ks);

/* QK-norm + RoPE + KV-cache write, then causal GQA attention, for nt tokens
 * at positions *pos_d .. *pos_d + nt - 1 of one layer (two launches); the
 * q part of qkv is left normalised and roped.  ctx_bound (host-known,
 * nt .. max_seq) must be >= *pos_d + nt: it sizes the scores in LDS (tokens
 * whose context exceeds it are skipped) */
int qm_attention(float *qkv_d, float *out_d, float *kc_d, float *vc_d, const uint16_t *qn_d,
                 const uint16_t *kn_d, const float *rcos_d, const float *rsin_d, const int *pos_d,
                 int nt, int max_seq, int ctx_bound, float eps);
/* dynamic LDS of the chunk attention with qt tokens per block and score
 * rows of ldp floats */
size_t qm_attention_lds_bytes(int qt, int ldp);

/* decode attention split into QM_ATT_SPLITS position ranges per kv head:
 * writes softmax partials (m, l, o[128] per head and range, QM_ATT_PART
 * floats each, [kv head][split][2 heads]) for the o-projection GEMV to merge
 * (qh_gemv_merge); also writes the new k/v to the cache */
#define QM_ATT_SPLITS QH_ATT_SPLITS
#define QM_ATT_PART QH_ATT_PART
#define QM_ATT_PART_FLOATS (8 * QM_ATT_SPLITS * 2 * QM_ATT_PART)
int qm_attention_decode_part(const float *qkv_d, float *part_d, float *kc_d, float *vc_d,
                             const uint16_t *qn_d, const uint16_t *kn_d, const float *rcos_d,
                             const float *rsin_d, const int *pos_d, int max_seq, float eps);

/* batched decode attention for n_seq sequences, one token each: row s of
 * qkv is sequence s's token at position pos[s]; its cache starts kv_seq
 * floats after sequence s-1's (same layout as above); each kv head's
 * positions are split into QM_BATCH_SPLITS ranges, whose partials (part:
 * QM_BATCH_PART_FLOATS per sequence) are merged into att[n_seq][2048]
 * (two launches) */
#ifndef QM_BATCH_SPLITS
#define QM_BATCH_SPLITS 8
#endif
#define QM_BATCH_PART_FLOATS (8 * QM_BATCH_SPLITS * 2 * QM_ATT_PART)
int qm_attention_decode_batch(const float *qkv_d, float *att_d, float *part_d, float *kc_d, float *vc_d,
                              size_t kv_seq, const uint16_t *qn_d, const uint16_t *kn_d,
                              const float *rcos_d, const float *rsin_d, const int *pos_d, int n_seq,
                              int max_seq, float eps);

/* greedy step of n_rows sequences: tok[r] = argmax of logits row r (n
 * floats, first index on ties); out[r*out_ld + pos[r] - plen[r] + 1] =
 * tok[r] when that index is in [0, out_ld); pos[r] += 1 */
int qm_argmax_rows(const float *logits_d, int n, int n_rows, int *tok_d, int *pos_d, const int *plen_d,
                   int *out_d, int out_ld);

/* One decode token's 28 decoder layers as one persistent launch
 * (hip_model_persist.hip), the same bits as the per-layer launches of
 * model_hip.c decode_step: w holds 9 weight pointers per layer (input norm,
 * q|k|v, q norm, k norm, o, post-attention norm, gate, up, down); the token
 * and position come from state[0], state[1]; writes each layer's new K/V
 * cache entry, the residual after the last layer's o add to x_out and the
 * last down output to dn_out.  qm_persist_init allocates its buffers once
 * (device current); qm_persist_supported says whether the device keeps the
 * launch's 256 workgroups resident; qm_persist_errors returns (and clears)
 * the error flags of launches that gave up waiting on an exchange. */
int qm_persist_init(void);
int qm_persist_supported(void);
int qm_decode_layers_persist(const uint16_t *const *w, int layers, const uint16_t *embed, int vocab,
                             const int *state, float *kc, float *vc, size_t kv_layer, const float *rcos,
                             const float *rsin, int max_seq, float eps, float *x_out, float *dn_out);
int qm_persist_errors(unsigned *flags);

/* *p = v, as a kernel (safe inside stream capture) */
int qm_set_i32(int *p_d, int v);
/* p[0..n) = 0, as a kernel */
int qm_zero_i32(int *p_d, int n);

#ifdef __cplusplus
}
#endif
#endif
