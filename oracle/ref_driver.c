/* Greedy-generation driver around the reference forward — TEST INFRASTRUCTURE.
 *
 * Compiled only together with the reference's own qwen3.c + a kernels_*.c +
 * ops_scalar.c into oracle/_ref/ (see the "ref" target of the Makefile here),
 * so that tests can run the reference model on a random-init QW3M blob.
 * The loop follows fpga_bringup/src/src/main.c:227-256: one batched prefill
 * of the prompt (chunked by QWEN3_MAX_BATCH), argmax of the last logits,
 * then one qwen3_forward per generated token.
 */
#define _POSIX_C_SOURCE 199309L
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "qwen3.h"

/* wall-clock seconds of the last refdrv_generate's prefill and decode loops */
static double g_t_prefill, g_t_decode;
static double now_s(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec + 1e-9 * (double)t.tv_nsec;
}
void refdrv_last_times(double *prefill_s, double *decode_s) {
    *prefill_s = g_t_prefill;
    *decode_s = g_t_decode;
}

size_t refdrv_scratch_bytes(void) { return qwen3_scratch_bytes(); }
int refdrv_max_seq(void) { return QWEN3_MAX_SEQ; }
int refdrv_max_batch(void) { return QWEN3_MAX_BATCH; }

/* ---- intermediate dumps (qwen3_set_dump, qwen3.h:166-178) ---------------- */
typedef struct {
    int layer;
    char name[44];
    size_t off, n;
} refdrv_rec_t;

typedef struct {
    float *buf;
    size_t cap, used;
    refdrv_rec_t *recs;
    int max_recs, n_recs, overflow;
} capture_t;

static void capture_cb(void *ctx, int layer, const char *name, const float *data, size_t n) {
    capture_t *c = (capture_t *)ctx;
    if (c->n_recs >= c->max_recs || c->used + n > c->cap) { c->overflow = 1; return; }
    refdrv_rec_t *r = &c->recs[c->n_recs++];
    r->layer = layer;
    strncpy(r->name, name, sizeof r->name - 1);
    r->name[sizeof r->name - 1] = 0;
    r->off = c->used;
    r->n = n;
    memcpy(c->buf + c->used, data, n * sizeof(float));
    c->used += n;
}

/* One qwen3_forward_batch of tokens[0..n_token) at position 0 with every
 * EMIT of qwen3.c captured into buf (records in recs).  Returns the number
 * of records, -100 if buf or recs were too small, or a QWEN3_ERR_* code. */
int refdrv_forward_dump(const void *blob, size_t blob_size, const int *tokens, int n_token,
                        float *buf, size_t cap, refdrv_rec_t *recs, int max_recs) {
    static qwen3_t m;
    void *scratch = malloc(qwen3_scratch_bytes());
    if (!scratch) return QWEN3_ERR_OOM;
    int rc = qwen3_init(&m, blob, blob_size, scratch, qwen3_scratch_bytes());
    if (rc != QWEN3_OK) { free(scratch); return rc; }
    if (n_token < 1 || n_token > QWEN3_MAX_BATCH) { free(scratch); return QWEN3_ERR_SHAPE; }
    capture_t c = {buf, cap, 0, recs, max_recs, 0, 0};
    qwen3_set_dump(&m, capture_cb, &c);
    qwen3_forward_batch(&m, tokens, n_token, 0);
    qwen3_set_dump(&m, NULL, NULL);
    free(scratch);
    return c.overflow ? -100 : c.n_recs;
}

/* logit gap between the best and the runner-up, for divergence reports */
static float top2_margin(const float *v, int n) {
    float b1 = v[0], b2 = -3.0e38f;
    for (int i = 1; i < n; i++) {
        if (v[i] > b1) { b2 = b1; b1 = v[i]; }
        else if (v[i] > b2) b2 = v[i];
    }
    return b1 - b2;
}

/* Returns the number of tokens written to out (<= n_decode + 1), or a
 * negative QWEN3_ERR_* code.  out[0] comes from the prefill logits; each
 * decode step i feeds out[i] at position n_prompt + i and yields out[i+1].
 * If logits_out is non-NULL, the last logits row after the prefill is copied
 * there (VOCAB floats). */
int refdrv_generate(const void *blob, size_t blob_size,
                    const int *prompt, int n_prompt, int n_decode,
                    int stop_at_eos, int *out, float *margins,
                    float *logits_out) {
    static qwen3_t m;
    void *scratch = malloc(qwen3_scratch_bytes());
    if (!scratch) return QWEN3_ERR_OOM;
    int rc = qwen3_init(&m, blob, blob_size, scratch, qwen3_scratch_bytes());
    if (rc != QWEN3_OK) { free(scratch); return rc; }
    if (n_prompt < 1 || n_prompt + n_decode > QWEN3_MAX_SEQ) {
        free(scratch);
        return QWEN3_ERR_SHAPE;
    }

    const double t0 = now_s();
    for (int p0 = 0; p0 < n_prompt; p0 += QWEN3_MAX_BATCH) {
        int nt = n_prompt - p0 < QWEN3_MAX_BATCH ? n_prompt - p0 : QWEN3_MAX_BATCH;
        qwen3_forward_batch(&m, prompt + p0, nt, p0);
    }
    if (logits_out)
        memcpy(logits_out, qwen3_last_logits(&m), sizeof(float) * QWEN3_VOCAB_SIZE);

    int n_out = 0;
    int next = qwen3_argmax(qwen3_last_logits(&m), QWEN3_VOCAB_SIZE);
    if (margins) margins[n_out] = top2_margin(qwen3_last_logits(&m), QWEN3_VOCAB_SIZE);
    out[n_out++] = next;
    const double t1 = now_s();
    for (int step = 0; step < n_decode; step++) {
        if (stop_at_eos &&
            (next == QWEN3_EOS_TOKEN_ID_0 || next == QWEN3_EOS_TOKEN_ID_1))
            break;
        qwen3_forward(&m, next, n_prompt + step);
        next = qwen3_argmax(qwen3_last_logits(&m), QWEN3_VOCAB_SIZE);
        if (margins) margins[n_out] = top2_margin(qwen3_last_logits(&m), QWEN3_VOCAB_SIZE);
        out[n_out++] = next;
    }
    g_t_prefill = t1 - t0;
    g_t_decode = now_s() - t1;
    free(scratch);
    return n_out;
}

/* refdrv_generate, and also the logits after chosen decode steps: for each
 * step s in log_steps[0..n_log) (1 <= s <= n_decode: the forward that
 * produces out[s]), VOCAB floats go to step_logits + i * VOCAB. */
int refdrv_generate_steps(const void *blob, size_t blob_size,
                          const int *prompt, int n_prompt, int n_decode,
                          int *out, float *margins, float *logits_out,
                          const int *log_steps, int n_log, float *step_logits) {
    static qwen3_t m;
    void *scratch = malloc(qwen3_scratch_bytes());
    if (!scratch) return QWEN3_ERR_OOM;
    int rc = qwen3_init(&m, blob, blob_size, scratch, qwen3_scratch_bytes());
    if (rc != QWEN3_OK) { free(scratch); return rc; }
    if (n_prompt < 1 || n_prompt + n_decode > QWEN3_MAX_SEQ) {
        free(scratch);
        return QWEN3_ERR_SHAPE;
    }
    for (int p0 = 0; p0 < n_prompt; p0 += QWEN3_MAX_BATCH) {
        int nt = n_prompt - p0 < QWEN3_MAX_BATCH ? n_prompt - p0 : QWEN3_MAX_BATCH;
        qwen3_forward_batch(&m, prompt + p0, nt, p0);
    }
    if (logits_out)
        memcpy(logits_out, qwen3_last_logits(&m), sizeof(float) * QWEN3_VOCAB_SIZE);
    int n_out = 0;
    int next = qwen3_argmax(qwen3_last_logits(&m), QWEN3_VOCAB_SIZE);
    if (margins) margins[n_out] = top2_margin(qwen3_last_logits(&m), QWEN3_VOCAB_SIZE);
    out[n_out++] = next;
    for (int step = 0; step < n_decode; step++) {
        qwen3_forward(&m, next, n_prompt + step);
        const float *lg = qwen3_last_logits(&m);
        for (int i = 0; i < n_log; i++)
            if (log_steps[i] == step + 1)
                memcpy(step_logits + (size_t)i * QWEN3_VOCAB_SIZE, lg, sizeof(float) * QWEN3_VOCAB_SIZE);
        next = qwen3_argmax(lg, QWEN3_VOCAB_SIZE);
        if (margins) margins[n_out] = top2_margin(lg, QWEN3_VOCAB_SIZE);
        out[n_out++] = next;
    }
    free(scratch);
    return n_out;
}
