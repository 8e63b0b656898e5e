/* MI355X (gfx950) device-resident Qwen3-0.6B forward and the QW3M weight
 * blob — public C ABI of libqwen3_hip (same library as qwen3_hip.h).
 *
 * Paths are relative to the reference root; SRC = fpga_bringup/src/src.
 *
 * The reference runs its forward on the host (SRC/qwen3.c:455-576) and hands
 * only the GEMMs to the plug-in.  This forward keeps the weights, the
 * activations and the KV cache in HBM and runs every op on the GPU: the
 * projections through the same GEMM/GEMV kernels as qwen3_gemm, the other
 * ops (SRC/ops.h:21-49: rmsnorm, rope, softmax, silu_mul, residual_add,
 * argmax, bf16_to_f32, dot, axpy) as GPU kernels fused around them.  Greedy
 * decoding keeps the token, the position and the output list on the device,
 * so each generated token is one replay of a captured HIP graph.
 *
 * Numerics: as the reference forward with an A-bf16 GEMM (the AME kernel,
 * SRC/kernels_ame.c:219-236): GEMM/GEMV inputs are rounded to bf16, products
 * are exact, sums are fp32; other ops are fp32 as in SRC/ops_scalar.c, with
 * parallel reduction orders.
 *
 * Errors: functions return 0, a QWEN3_HIP_E* code (> 0, qwen3_hip.h) for a
 * device/argument problem, or one of the reference's QWEN3_ERR_* values
 * (< 0, SRC/qwen3.h:188-200) for a blob that does not parse.
 *
 * Threading: not thread-safe; shares the library's single stream.  Close
 * every model before qwen3_hip_release().
 */
#ifndef QWEN3_HIP_MODEL_H
#define QWEN3_HIP_MODEL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* QW3M blob layouts (header offset 76, SRC/kernels.h:67-68) */
#define QWEN3_HIP_LAYOUT_ROW 0
#define QWEN3_HIP_LAYOUT_TILE 1

/* ---- QW3M blob (SRC/qwen3_config.h:33-81) ---------------------------------- */

/* Exact file size of a Qwen3-0.6B blob in the given layout (row: align 128,
 * 1,192,100,096 B; tile: 128x32 tiles, align 4096, 1,192,433,664 B), or 0. */
size_t qwen3_hip_qw3m_size(int layout);

/* Write a complete random-init blob into blob[0..size): header as
 * SRC/qwen3_config.h:41-62, tensors in the order of :63-78, every
 * projection and embed_tokens ~ N(0, 0.02) in bf16, every norm weight 1.0.
 * Tensor t (0 = embed_tokens .. 309 = final norm) draws from seed + t.
 * Deterministic for (seed, layout) whatever `threads` is.  No reference
 * counterpart: the reference exports real weights, which are not available
 * offline.  Returns 0 or QWEN3_HIP_EINVAL (size must equal qw3m_size). */
int qwen3_hip_qw3m_write_random(void *blob, size_t size, uint64_t seed, int layout,
                                int threads);

/* Validate a blob the way qwen3_init does (SRC/qwen3.c:87-146: magic,
 * version, dtype, shapes, align, layout, theta/eps, exact size); returns 0 or
 * the reference's QWEN3_ERR_* code. */
int qwen3_hip_qw3m_check(const void *blob, size_t size);

/* ---- device-resident forward -------------------------------------------- */

typedef struct qwen3_hip_model qwen3_hip_model;

/* Mirrors qwen3_init (SRC/qwen3.c:87-146): parses the blob, uploads every
 * tensor to the device (tile-major matrices are re-laid row-major there) and
 * allocates activations and a KV cache for max_seq positions (0 = 4096;
 * at most 8192).  The blob may be freed after this returns. */
int qwen3_hip_model_open(qwen3_hip_model **model, const void *blob, size_t size, int max_seq);

void qwen3_hip_model_close(qwen3_hip_model *model);

int qwen3_hip_model_max_seq(const qwen3_hip_model *model);

/* Mirrors qwen3_forward_batch (SRC/qwen3.c:455-576): n_token tokens (1 ..
 * 128, the reference's QWEN3_MAX_BATCH) at positions pos0 .. pos0+n_token-1;
 * writes their K/V into the cache and leaves the last token's logits on the
 * device.  Unlike the reference, out-of-range sizes return QWEN3_HIP_EINVAL
 * instead of silently doing nothing. */
int qwen3_hip_model_forward(qwen3_hip_model *model, const int *tokens, int n_token, int pos0);

/* Copy the last logits (vocab floats) to host memory (synchronous). */
int qwen3_hip_model_logits(qwen3_hip_model *model, float *out);

/* argmax of the last logits, first index on ties (SRC/ops_scalar.c:57-62). */
int qwen3_hip_model_argmax(qwen3_hip_model *model, int *token);

/* Greedy generation as SRC/main.c:227-256: prefill of the prompt in chunks
 * of 128, out[0] = argmax of the prefill logits, then n_decode steps, step i
 * feeding out[i] at position n_prompt + i and producing out[i + 1].  With
 * stop_at_eos, generation ends after the first EOS (151645 or 151643,
 * SRC/qwen3_config.h:28-30), which is included.  out needs n_decode + 1
 * ints; *n_out receives the count.  n_prompt + n_decode <= max_seq. */
int qwen3_hip_model_generate(qwen3_hip_model *model, const int *prompt, int n_prompt, int n_decode,
                             int stop_at_eos, int *out, int *n_out);

/* Wall-clock split of the last generate call (ms): prefill including the
 * first argmax, and the n_decode decode steps. */
int qwen3_hip_model_timing(const qwen3_hip_model *model, double *prefill_ms, double *decode_ms);

/* Decode steps as one graph replay each (1, the default) or as eager
 * launches (0); both compute the same thing. */
int qwen3_hip_model_set_graph(qwen3_hip_model *model, int on);

/* Decode steps with the 28 decoder layers as one persistent launch (1) or
 * as five launches per layer (0, the default; QWEN3_HIP_MODEL_PERSIST=1 in
 * the environment makes 1 the default); both give the same bits (no
 * counterpart in the reference, which has no launches).  On MI355X the
 * persistent launch measured 3% slower (1,720-1,750 against 1,780-1,805
 * tok/s for 128 greedy steps after a 128-token prompt).  Turning it on where
 * the device cannot keep the launch's 256 workgroups resident returns
 * QWEN3_HIP_ENODEV.  qwen3_hip_model_persistent returns the mode. */
int qwen3_hip_model_set_persistent(qwen3_hip_model *model, int on);
int qwen3_hip_model_persistent(const qwen3_hip_model *model);
/* Error flags raised by persistent decode launches since the last call
 * (nonzero: a launch gave up waiting for another workgroup's outputs, and
 * the tokens it produced are invalid); synchronises the device. */
int qwen3_hip_model_persist_errors(qwen3_hip_model *model, unsigned *flags);

/* Intermediate-activation dumps, as qwen3_set_dump (SRC/qwen3.h:166-178):
 * during qwen3_hip_model_forward the callback receives, in host memory and
 * under the reference's names, every tensor this forward materialises:
 * "embed_out" (layer -1); per layer "input_layernorm_out", "q_proj_out",
 * "k_proj_out", "v_proj_out", "attn_out", "o_proj_out",
 * "x_after_attn_residual", "post_attn_norm_out", "silu_gate_mul_up",
 * "down_proj_out", "layer_out"; and "logits" (layer -1).  The reference's
 * other names (q/k norm and rope outputs, separate gate/up outputs, the
 * final norm) are fused into kernels here and are not produced.  Each dump
 * synchronises the device; NULL (the default) turns dumping off. */
typedef void (*qwen3_hip_dump_fn)(void *ctx, int layer, const char *name, const float *data,
                                  size_t n);
int qwen3_hip_model_set_dump(qwen3_hip_model *model, qwen3_hip_dump_fn fn, void *ctx);

/* ---- multi-sequence batched decode ----------------------------------------
 *
 * No counterpart in the reference, whose forward holds one sequence
 * (SRC/qwen3.h:234-241).  n_seq independent sequences share the model's
 * weights; each has its own KV cache of max_ctx positions (229,376 bytes per
 * position: 28 layers x 8 kv heads x 128 dims x fp32 K and V).  A sequence
 * is prefilled on its own through the forward of qwen3_hip_model_forward; a
 * decode step then feeds one token of every sequence, each at its own
 * position, so each projection is one GEMM with M = n_seq rows (the same
 * qwen3_gemm kernels) instead of n_seq GEMVs, and attention runs over every
 * sequence's cache in one launch.  Greedy selection as
 * qwen3_hip_model_generate (first index of the maximum).
 *
 * The batch borrows the model's weights, rope tables and activation
 * buffers: close it before the model.  If the model is closed first, the
 * batch's later calls return QWEN3_HIP_ESTATE (qwen3_hip_batch_close still
 * frees it).  Its calls, like the model's, are synchronous; a batch call
 * discards the model's last logits. */
typedef struct qwen3_hip_batch qwen3_hip_batch;

/* n_seq in 1 .. 128 (QWEN3_MAX_BATCH rows per GEMM); max_ctx in 2 ..
 * qwen3_hip_model_max_seq(model). */
int qwen3_hip_batch_open(qwen3_hip_batch **batch, qwen3_hip_model *model, int n_seq, int max_ctx);

void qwen3_hip_batch_close(qwen3_hip_batch *batch);

/* Prefill sequence seq (0 .. n_seq-1) with n_prompt tokens (1 .. max_ctx-1)
 * at positions 0 .. n_prompt-1, in chunks of 128, replacing whatever the
 * sequence held; its next token is the argmax of the last prompt row's
 * logits.  Sequences may have prompts of different lengths. */
int qwen3_hip_batch_prefill(qwen3_hip_batch *batch, int seq, const int *prompt, int n_prompt);

/* n_decode greedy steps of every sequence at once (every sequence must be
 * prefilled).  out[s * (n_decode + 1) + 0] receives the token sequence s is
 * fed first (after a prefill: the prefill's argmax), out[s * (n_decode + 1)
 * + i] the token generated by step i.  A later call continues where the
 * previous one ended.  Each sequence's positions must stay below max_ctx:
 * n_prompt + tokens decoded since its prefill + n_decode <= max_ctx.  EOS
 * does not stop a sequence (callers cut at it). */
int qwen3_hip_batch_decode(qwen3_hip_batch *batch, int n_decode, int *out);

/* Logits of the last decode step, n_seq x vocab floats (synchronous copy). */
int qwen3_hip_batch_logits(qwen3_hip_batch *batch, float *out);

/* Decode steps as one graph replay each (1, the default; the first step of
 * the first call runs eagerly, then the step is captured) or as eager
 * launches (0); both compute the same thing. */
int qwen3_hip_batch_set_graph(qwen3_hip_batch *batch, int on);

/* Wall-clock ms of the last qwen3_hip_batch_decode call. */
int qwen3_hip_batch_timing(const qwen3_hip_batch *batch, double *decode_ms);

#ifdef __cplusplus
}
#endif
#endif
