/* Host side of the device-resident Qwen3-0.6B forward, in C11.
 *
 * The forward follows fpga_bringup/src/src/qwen3.c:455-576 op for op; what
 * changes is where the data lives and how ops are grouped into launches:
 *
 *   chunk (prefill, n tokens)           decode step (1 token, graph-replayed)
 *   ------------------------------     --------------------------------------
 *   embed + rmsnorm        rows_norm    [rmsnorm prologue + qkv GEMV]  (layer 0
 *   qkv GEMM (q|k|v, N=4096)  gemm       gathers the embedding row itself)
 *   qk-norm, rope, KV write,            [qk-norm, rope, KV write, attention]
 *     attention            attention    [o GEMV]
 *   o GEMM                 gemm         [residual + rmsnorm prologue +
 *   residual + rmsnorm     rows_norm     gate/up GEMV + silu*up]
 *   gate/up GEMM + silu*up gemm (gated) [down GEMV]
 *   down GEMM              gemm         ... next layer's prologue adds down
 *   (next layer's rows_norm adds down)  [residual + final norm + lm_head GEMV]
 *   residual + final norm + lm_head     [argmax + token/pos/out bookkeeping]
 *     GEMV on the last row
 *
 * The residual stream of a decode step ping-pongs between x0 and x1: each
 * prologue reads one and its single writer stores x + r into the other.
 */
#define _POSIX_C_SOURCE 200809L   /* clock_gettime under -std=c11 */
#include "qwen3_hip_model.h"
#include "qwen3_hip.h"
#include "hip_shim.h"
#include "model_shim.h"
#include "qw3m.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#define H QW3M_HIDDEN
#define QKV_N (QW3M_Q_DIM + 2 * QW3M_KV_DIM)
#define NL QW3M_N_LAYERS
#define V QW3M_VOCAB
#define DEFAULT_MAX_SEQ 4096

typedef struct {
    uint16_t *in_norm, *wqkv, *qn, *kn, *wo, *post_norm, *wg, *wu, *wd;
} layer_t;

struct qwen3_hip_model {
    int max_seq;
    uint16_t *wbuf;                    /* all weights, one allocation */
    uint16_t *embed, *final_norm;
    layer_t L[NL];
    float *kc, *vc;                    /* [NL][KVH][..] see hip_model.hip */
    float *rcos, *rsin;                /* [max_seq][64] */
    float *x, *x0, *x1, *xb, *qkv, *att, *ob, *hb, *dn, *logits;
    float *apart;                      /* decode attention partials [QM_ATT_PART_FLOATS] */
    int *tok_in;                       /* [QM_MAX_CHUNK] */
    int *state;                        /* [0] token, [1] position, [2] step */
    int *out_tok;                      /* [max_seq + 1] */
    int use_graph;
    int use_persist;                   /* decode layers as one persistent launch */
    int graph_id;                      /* -1 until captured */
    qwen3_hip_dump_fn dump;            /* chunk-path intermediate dumps (NULL = off) */
    void *dump_ctx;
    float *dump_host;                  /* staging for dumps */
    int have_logits;
    double t_prefill_ms, t_decode_ms;
    struct qwen3_hip_batch *batches;   /* open batches on this model (linked by next) */
};

static void detach_batches(qwen3_hip_model *m);

static double now_ms(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec * 1e3 + (double)ts.tv_nsec * 1e-6;
}

/* ---- QW3M -------------------------------------------------------------------- */

size_t qwen3_hip_qw3m_size(int layout) { return qw3m_size(layout); }

int qwen3_hip_qw3m_write_random(void *blob, size_t size, uint64_t seed, int layout, int threads) {
    return qw3m_write_random(blob, size, seed, layout, threads) == 0 ? QWEN3_HIP_OK : QWEN3_HIP_EINVAL;
}

int qwen3_hip_qw3m_check(const void *blob, size_t size) { return qw3m_parse(blob, size, NULL); }

/* ---- open / close ------------------------------------------------------------ */

static size_t up256(size_t x) { return (x + 255) & ~(size_t)255; }

/* bytes of each device tensor, in allocation order */
static size_t dev_weight_bytes(void) {
    size_t b = up256((size_t)V * H * 2) + up256(H * 2);
    const size_t per = up256(H * 2) + up256((size_t)QKV_N * H * 2) + 2 * up256(QW3M_HEAD_DIM * 2) +
                       up256((size_t)H * QW3M_Q_DIM * 2) + up256(H * 2) +
                       2 * up256((size_t)QW3M_INTER * H * 2) + up256((size_t)H * QW3M_INTER * 2);
    return b + (size_t)NL * per;
}

/* upload tensor t of the blob into dst (row-major [rows][cols]); tile-major
 * matrices go through stage and are re-laid on the device */
static int upload(const uint8_t *blob, const qw3m_info_t *info, int t, uint16_t *dst, uint16_t *stage) {
    int rows, cols, mat;
    qw3m_tensor_shape(t, &rows, &cols, &mat);
    const size_t bytes = (size_t)rows * cols * 2;
    const void *src = blob + info->offset[t];
    if (info->layout == QW3M_LAYOUT_TILE && mat) {
        int rc = qh_h2d(stage, src, bytes);
        if (!rc) rc = qh_tile_to_row(dst, stage, rows, cols, info->tile_n, info->tile_k);
        /* the next upload overwrites stage: wait here (pageable source too) */
        if (!rc) rc = qh_sync();
        return rc;
    }
    int rc = qh_h2d(dst, src, bytes);
    if (!rc) rc = qh_sync();
    return rc;
}

static void rope_tables(float *c, float *s, int max_seq) {
    /* ops_scalar.c:21-35: inv_freq = 1 / theta^(2i / head_dim), angle = pos * inv_freq */
    const int half = QW3M_HEAD_DIM / 2;
    for (int i = 0; i < half; i++) {
        const float inv_freq = 1.0f / powf(QW3M_ROPE_THETA, (float)(2 * i) / (float)QW3M_HEAD_DIM);
        for (int p = 0; p < max_seq; p++) {
            const float ang = (float)p * inv_freq;
            c[(size_t)p * half + i] = cosf(ang);
            s[(size_t)p * half + i] = sinf(ang);
        }
    }
}

void qwen3_hip_model_close(qwen3_hip_model *m) {
    if (!m) return;
    (void)qh_sync();
    detach_batches(m);
    if (m->graph_id >= 0) (void)qh_graph_destroy(m->graph_id);
    void *bufs[] = {m->wbuf, m->kc, m->vc, m->rcos, m->rsin, m->x, m->x0, m->x1, m->xb, m->qkv,
                    m->att, m->ob, m->hb, m->dn, m->logits, m->apart, m->tok_in, m->state, m->out_tok};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++) (void)qh_free(bufs[i]);
    free(m->dump_host);
    free(m);
}

int qwen3_hip_model_open(qwen3_hip_model **out, const void *blob, size_t size, int max_seq) {
    if (!out) return QWEN3_HIP_EINVAL;
    *out = NULL;
    qw3m_info_t info;
    int rc = qw3m_parse(blob, size, &info);
    if (rc) return rc;
    if (max_seq == 0) max_seq = DEFAULT_MAX_SEQ;
    if (max_seq < 1 || max_seq > QM_MAX_SEQ) return QWEN3_HIP_EINVAL;
    rc = qwen3_hip_init(-1);
    if (rc) return rc;

    qwen3_hip_model *m = (qwen3_hip_model *)calloc(1, sizeof *m);
    if (!m) return QWEN3_HIP_ENOMEM;
    m->max_seq = max_seq;
    m->use_graph = 1;
    m->graph_id = -1;
    {
        /* the persistent decode launch, opt-in: measured slower than the
         * per-layer launches (1,720-1,750 against 1,780-1,805 tok/s).  Its
         * buffers, shared by every model, are allocated when first wanted;
         * failing to get them only leaves it off. */
        const char *env = getenv("QWEN3_HIP_MODEL_PERSIST");
        m->use_persist = env && strcmp(env, "1") == 0 && qm_persist_init() == 0 && qm_persist_supported();
    }

#define DEV(ptr, bytes)                                                   \
    do {                                                                  \
        if ((rc = qh_malloc((void **)&(ptr), (bytes))) != 0) goto fail;   \
    } while (0)
    DEV(m->wbuf, dev_weight_bytes());
    const size_t kv_bytes = (size_t)NL * QW3M_N_KV_HEADS * max_seq * QW3M_HEAD_DIM * sizeof(float);
    DEV(m->kc, kv_bytes);
    DEV(m->vc, kv_bytes);
    const size_t rope_bytes = (size_t)max_seq * (QW3M_HEAD_DIM / 2) * sizeof(float);
    DEV(m->rcos, rope_bytes);
    DEV(m->rsin, rope_bytes);
    const size_t B = QM_MAX_CHUNK;
    DEV(m->x, B * H * 4);
    DEV(m->x0, H * 4);
    DEV(m->x1, H * 4);
    DEV(m->xb, B * H * 4);
    DEV(m->qkv, B * QKV_N * 4);
    DEV(m->att, B * QW3M_Q_DIM * 4);
    DEV(m->ob, B * H * 4);
    DEV(m->hb, B * QW3M_INTER * 4);
    DEV(m->dn, B * H * 4);
    DEV(m->logits, (size_t)V * 4);
    DEV(m->apart, (size_t)QM_ATT_PART_FLOATS * 4);
    DEV(m->tok_in, B * sizeof(int));
    DEV(m->state, 4 * sizeof(int));
    DEV(m->out_tok, ((size_t)max_seq + 1) * sizeof(int));
#undef DEV

    /* carve the weight allocation */
    {
        uint8_t *p = (uint8_t *)m->wbuf;
#define CARVE(dst, bytes) do { (dst) = (uint16_t *)p; p += up256(bytes); } while (0)
        CARVE(m->embed, (size_t)V * H * 2);
        CARVE(m->final_norm, H * 2);
        for (int l = 0; l < NL; l++) {
            layer_t *L = &m->L[l];
            CARVE(L->in_norm, H * 2);
            CARVE(L->wqkv, (size_t)QKV_N * H * 2);
            CARVE(L->qn, QW3M_HEAD_DIM * 2);
            CARVE(L->kn, QW3M_HEAD_DIM * 2);
            CARVE(L->wo, (size_t)H * QW3M_Q_DIM * 2);
            CARVE(L->post_norm, H * 2);
            CARVE(L->wg, (size_t)QW3M_INTER * H * 2);
            CARVE(L->wu, (size_t)QW3M_INTER * H * 2);
            CARVE(L->wd, (size_t)H * QW3M_INTER * 2);
        }
#undef CARVE
    }

    /* upload; the tile stage holds the largest matrix (6 MiB) */
    {
        uint16_t *stage = NULL;
        if (info.layout == QW3M_LAYOUT_TILE &&
            (rc = qh_malloc((void **)&stage, (size_t)QW3M_INTER * H * 2)) != 0)
            goto fail;
        const uint8_t *b = (const uint8_t *)blob;
        rc = upload(b, &info, 0, m->embed, stage);
        for (int l = 0; l < NL && !rc; l++) {
            const int t0 = 1 + 11 * l;
            layer_t *L = &m->L[l];
            if (!rc) rc = upload(b, &info, t0 + QW3M_T_IN_NORM, L->in_norm, stage);
            if (!rc) rc = upload(b, &info, t0 + QW3M_T_WQ, L->wqkv, stage);
            if (!rc) rc = upload(b, &info, t0 + QW3M_T_WK, L->wqkv + (size_t)QW3M_Q_DIM * H, stage);
            if (!rc) rc = upload(b, &info, t0 + QW3M_T_WV, L->wqkv + (size_t)(QW3M_Q_DIM + QW3M_KV_DIM) * H, stage);
            if (!rc) rc = upload(b, &info, t0 + QW3M_T_QNORM, L->qn, stage);
            if (!rc) rc = upload(b, &info, t0 + QW3M_T_KNORM, L->kn, stage);
            if (!rc) rc = upload(b, &info, t0 + QW3M_T_WO, L->wo, stage);
            if (!rc) rc = upload(b, &info, t0 + QW3M_T_POST_NORM, L->post_norm, stage);
            if (!rc) rc = upload(b, &info, t0 + QW3M_T_WGATE, L->wg, stage);
            if (!rc) rc = upload(b, &info, t0 + QW3M_T_WUP, L->wu, stage);
            if (!rc) rc = upload(b, &info, t0 + QW3M_T_WDOWN, L->wd, stage);
        }
        if (!rc) rc = upload(b, &info, QW3M_N_TENSORS - 1, m->final_norm, stage);
        if (stage) (void)qh_free(stage);
        if (rc) goto fail;
    }

    /* rope tables */
    {
        float *c = (float *)malloc(rope_bytes), *s = (float *)malloc(rope_bytes);
        if (!c || !s) { free(c); free(s); rc = QWEN3_HIP_ENOMEM; goto fail; }
        rope_tables(c, s, max_seq);
        rc = qh_h2d(m->rcos, c, rope_bytes);
        if (!rc) rc = qh_h2d(m->rsin, s, rope_bytes);
        if (!rc) rc = qh_sync();
        free(c);
        free(s);
        if (rc) goto fail;
    }
    *out = m;
    return QWEN3_HIP_OK;
fail:
    qwen3_hip_model_close(m);
    return rc;
}

int qwen3_hip_model_max_seq(const qwen3_hip_model *m) { return m ? m->max_seq : 0; }

int qwen3_hip_model_set_dump(qwen3_hip_model *m, qwen3_hip_dump_fn fn, void *ctx) {
    if (!m) return QWEN3_HIP_EINVAL;
    if (fn && !m->dump_host) {
        m->dump_host = (float *)malloc((size_t)QM_MAX_CHUNK * QKV_N * sizeof(float));
        if (!m->dump_host) return QWEN3_HIP_ENOMEM;
    }
    m->dump = fn;
    m->dump_ctx = ctx;
    return QWEN3_HIP_OK;
}

/* copy rows x cols floats at column col0 of a [rows][ld] device matrix to the
 * host and hand them to the dump callback (same names as qwen3.c's EMITs) */
static int dump_dev(qwen3_hip_model *m, int layer, const char *name, const float *dev, int rows,
                    int ld, int col0, int cols) {
    float *h = m->dump_host;
    int rc = qh_d2h(h, dev, (size_t)rows * ld * sizeof(float));
    if (!rc) rc = qh_sync();
    if (rc) return rc;
    if (col0 != 0 || cols != ld)
        for (int r = 0; r < rows; r++) memmove(h + (size_t)r * cols, h + (size_t)r * ld + col0, cols * sizeof(float));
    m->dump(m->dump_ctx, layer, name, h, (size_t)rows * cols);
    return QWEN3_HIP_OK;
}

int qwen3_hip_model_set_graph(qwen3_hip_model *m, int on) {
    if (!m) return QWEN3_HIP_EINVAL;
    m->use_graph = on ? 1 : 0;
    return QWEN3_HIP_OK;
}

int qwen3_hip_model_set_persistent(qwen3_hip_model *m, int on) {
    if (!m) return QWEN3_HIP_EINVAL;
    if (on) {
        const int rc = qm_persist_init();   /* once: the launch's buffers and the residency check */
        if (rc) return rc;
        if (!qm_persist_supported()) return QWEN3_HIP_ENODEV;
    }
    if ((on ? 1 : 0) != m->use_persist && m->graph_id >= 0) {   /* the captured step is the other kind */
        int rc = qh_sync();
        if (!rc) rc = qh_graph_destroy(m->graph_id);
        if (rc) return rc;
        m->graph_id = -1;
    }
    m->use_persist = on ? 1 : 0;
    return QWEN3_HIP_OK;
}

int qwen3_hip_model_persistent(const qwen3_hip_model *m) { return m ? m->use_persist : 0; }

int qwen3_hip_model_persist_errors(qwen3_hip_model *m, unsigned *flags) {
    if (!m || !flags) return QWEN3_HIP_EINVAL;
    *flags = 0;
    return qm_persist_supported() ? qm_persist_errors(flags) : QWEN3_HIP_OK;
}

/* ---- forward ----------------------------------------------------------------- */

static size_t kv_layer_floats(const qwen3_hip_model *m) {
    return (size_t)QW3M_N_KV_HEADS * m->max_seq * QW3M_HEAD_DIM;
}

/* where a chunk's K/V go: layer l's cache of one sequence starts at
 * kc + l * layer_stride (layout in hip_model.hip, max_seq positions) */
typedef struct {
    float *kc, *vc;
    size_t layer_stride;
    int max_seq;
} kv_t;

static kv_t model_kv(qwen3_hip_model *m) {
    const kv_t kv = {m->kc, m->vc, kv_layer_floats(m), m->max_seq};
    return kv;
}

/* nt tokens already in tok_in at positions pos0.. (pos0 also set by the
 * caller in state[1]) of the sequence whose cache is kv; logits of the last
 * row when want_logits */
static int run_chunk(qwen3_hip_model *m, const kv_t *kv, int nt, int pos0, int want_logits) {
    int rc;
    const float eps = QW3M_RMS_EPS;
    /* with a dump callback the residual add of down_proj is done at the end
       of its layer (to materialise "layer_out"), not in the next prologue */
    const int dumping = m->dump != NULL;
#define DUMP(layer, name, ptr, ld, col0, cols) \
    do { if (!rc && dumping) rc = dump_dev(m, (layer), (name), (ptr), nt, (ld), (col0), (cols)); } while (0)
    /* without dumps, the o and down projections may leave split-K slice sums
       (qh_gemm_split) that the next residual + RMSNorm adds itself; the last
       layer's down is written out for the lm_head GEMV's prologue */
    const float *opart = NULL, *dpart = NULL;
    int oks = 0, dks = 0;
    for (int l = 0; l < NL; l++) {
        const layer_t *L = &m->L[l];
        if (l == 0) {
            rc = qm_rows_norm(m->x, NULL, m->embed, m->tok_in, V, L->in_norm, m->xb, nt, H, eps);
            DUMP(-1, "embed_out", m->x, H, 0, H);
        } else {
            rc = qm_rows_norm_split(m->x, dumping || dks ? NULL : m->dn, NULL, NULL, 0, L->in_norm, m->xb, nt, H,
                                    eps, dpart, dks);
        }
        DUMP(l, "input_layernorm_out", m->xb, H, 0, H);
        if (!rc) rc = qh_gemm(m->qkv, m->xb, L->wqkv, nt, H, QKV_N);
        DUMP(l, "q_proj_out", m->qkv, QKV_N, 0, QW3M_Q_DIM);
        DUMP(l, "k_proj_out", m->qkv, QKV_N, QW3M_Q_DIM, QW3M_KV_DIM);
        DUMP(l, "v_proj_out", m->qkv, QKV_N, QW3M_Q_DIM + QW3M_KV_DIM, QW3M_KV_DIM);
        if (!rc) rc = qm_attention(m->qkv, m->att, kv->kc + l * kv->layer_stride,
                                   kv->vc + l * kv->layer_stride, L->qn, L->kn, m->rcos, m->rsin,
                                   m->state + 1, nt, kv->max_seq, pos0 + nt, eps);
        DUMP(l, "attn_out", m->att, QW3M_Q_DIM, 0, QW3M_Q_DIM);
        if (!rc) rc = dumping ? qh_gemm(m->ob, m->att, L->wo, nt, QW3M_Q_DIM, H)
                              : qh_gemm_split(m->ob, m->att, L->wo, nt, QW3M_Q_DIM, H, &opart, &oks);
        DUMP(l, "o_proj_out", m->ob, H, 0, H);
        if (!rc) rc = qm_rows_norm_split(m->x, oks ? NULL : m->ob, NULL, NULL, 0, L->post_norm, m->xb, nt, H, eps,
                                         opart, oks);
        DUMP(l, "x_after_attn_residual", m->x, H, 0, H);
        DUMP(l, "post_attn_norm_out", m->xb, H, 0, H);
        if (!rc) rc = qh_gemm_gate_up_silu(m->hb, m->xb, L->wg, L->wu, nt, H, QW3M_INTER);
        DUMP(l, "silu_gate_mul_up", m->hb, QW3M_INTER, 0, QW3M_INTER);
        dks = 0;
        if (!rc) rc = (dumping || l == NL - 1) ? qh_gemm(m->dn, m->hb, L->wd, nt, QW3M_INTER, H)
                                               : qh_gemm_split(m->dn, m->hb, L->wd, nt, QW3M_INTER, H, &dpart, &dks);
        DUMP(l, "down_proj_out", m->dn, H, 0, H);
        if (!rc && dumping) {
            /* x += down (xb is scratch here; the next layer recomputes it) */
            rc = qm_rows_norm(m->x, m->dn, NULL, NULL, 0, L->in_norm, m->xb, nt, H, eps);
            DUMP(l, "layer_out", m->x, H, 0, H);
        }
        if (rc) return rc;
    }
#undef DUMP
    if (!want_logits) return QWEN3_HIP_OK;
    const qh_gemv_pro_t pro = {m->x + (size_t)(nt - 1) * H, NULL, NULL, 0,
                               dumping ? NULL : m->dn + (size_t)(nt - 1) * H, m->final_norm, NULL, eps};
    rc = qh_gemv_pro(m->logits, &pro, m->embed, NULL, H, V, 0);
    if (!rc && dumping) {
        rc = qh_d2h(m->dump_host, m->logits, (size_t)V * sizeof(float));
        if (!rc) rc = qh_sync();
        if (!rc) m->dump(m->dump_ctx, -1, "logits", m->dump_host, V);
    }
    return rc;
}

/* one greedy decode step on the device: token state[0] at position
 * state[1]; appends the next token to out_tok[state[2]] */
static int decode_step(qwen3_hip_model *m) {
    int rc = QWEN3_HIP_OK;
    const float eps = QW3M_RMS_EPS;
    if (m->use_persist) {
        /* the 28 layers in one launch: x0 and dn as the per-layer launches leave them */
        const uint16_t *w[NL * 9];
        for (int l = 0; l < NL; l++) {
            const layer_t *L = &m->L[l];
            const uint16_t *lw[9] = {L->in_norm, L->wqkv, L->qn, L->kn, L->wo, L->post_norm, L->wg, L->wu, L->wd};
            memcpy(w + 9 * l, lw, sizeof lw);
        }
        rc = qm_decode_layers_persist(w, NL, m->embed, V, m->state, m->kc, m->vc, kv_layer_floats(m), m->rcos,
                                      m->rsin, m->max_seq, eps, m->x0, m->dn);
    }
    for (int l = 0; l < NL && !rc && !m->use_persist; l++) {
        const layer_t *L = &m->L[l];
        qh_gemv_pro_t pro = {m->x0, NULL, NULL, 0, m->dn, L->in_norm, m->x1, eps};
        if (l == 0) { pro.x = NULL; pro.r = NULL; pro.emb = m->embed; pro.tok = m->state; pro.emb_rows = V; }
        rc = qh_gemv_pro(m->qkv, &pro, L->wqkv, NULL, H, QKV_N, 0);
        /* attention as split-softmax partials, merged in the o GEMV's prologue */
        if (!rc) rc = qm_attention_decode_part(m->qkv, m->apart, m->kc + l * kv_layer_floats(m),
                                               m->vc + l * kv_layer_floats(m), L->qn, L->kn, m->rcos,
                                               m->rsin, m->state + 1, m->max_seq, eps);
        if (!rc) rc = qh_gemv_merge(m->ob, m->apart, L->wo, QW3M_Q_DIM, H);
        const qh_gemv_pro_t pro2 = {m->x1, NULL, NULL, 0, m->ob, L->post_norm, m->x0, eps};
        if (!rc) rc = qh_gemv_pro(m->hb, &pro2, L->wg, L->wu, H, QW3M_INTER, 1);
        if (!rc) rc = qh_gemm(m->dn, m->hb, L->wd, 1, QW3M_INTER, H);
    }
    const qh_gemv_pro_t fin = {m->x0, NULL, NULL, 0, m->dn, m->final_norm, NULL, eps};
    if (!rc) rc = qh_gemv_pro(m->logits, &fin, m->embed, NULL, H, V, 0);
    if (!rc) rc = qh_argmax_step(m->state, m->out_tok, m->state + 2, m->max_seq + 1, m->state + 1, 1,
                                 m->logits, V);
    return rc;
}

static int check_tokens(const int *t, int n) {
    for (int i = 0; i < n; i++)
        if (t[i] < 0 || t[i] >= V) return QWEN3_HIP_EINVAL;
    return QWEN3_HIP_OK;
}

/* tokens -> tok_in and pos0 -> state[1] (synchronous on the host buffer) */
static int load_chunk(qwen3_hip_model *m, const int *tokens, int nt, int pos0) {
    int rc = qh_h2d(m->tok_in, tokens, (size_t)nt * sizeof(int));
    if (!rc) rc = qm_set_i32(m->state + 1, pos0);
    if (!rc) rc = qh_sync();   /* tokens may live in pageable caller memory */
    return rc;
}

int qwen3_hip_model_forward(qwen3_hip_model *m, const int *tokens, int n_token, int pos0) {
    if (!m || !tokens) return QWEN3_HIP_EINVAL;
    if (n_token < 1 || n_token > QM_MAX_CHUNK || pos0 < 0 || pos0 + n_token > m->max_seq)
        return QWEN3_HIP_EINVAL;
    int rc = check_tokens(tokens, n_token);
    const kv_t kv = model_kv(m);
    if (!rc) rc = load_chunk(m, tokens, n_token, pos0);
    if (!rc) rc = run_chunk(m, &kv, n_token, pos0, 1);
    m->have_logits = rc == 0;
    return rc;
}

int qwen3_hip_model_logits(qwen3_hip_model *m, float *out) {
    if (!m || !out || !m->have_logits) return QWEN3_HIP_EINVAL;
    int rc = qh_d2h(out, m->logits, (size_t)V * sizeof(float));
    if (!rc) rc = qh_sync();
    return rc;
}

int qwen3_hip_model_argmax(qwen3_hip_model *m, int *token) {
    if (!m || !token || !m->have_logits) return QWEN3_HIP_EINVAL;
    int rc = qh_argmax(m->state + 3, m->logits, V);
    if (!rc) rc = qh_d2h(token, m->state + 3, sizeof(int));
    if (!rc) rc = qh_sync();
    return rc;
}

int qwen3_hip_model_generate(qwen3_hip_model *m, const int *prompt, int n_prompt, int n_decode,
                             int stop_at_eos, int *out, int *n_out) {
    if (!m || !prompt || !out || !n_out) return QWEN3_HIP_EINVAL;
    *n_out = 0;
    if (n_prompt < 1 || n_decode < 0 || (long)n_prompt + n_decode > m->max_seq) return QWEN3_HIP_EINVAL;
    int rc = check_tokens(prompt, n_prompt);
    if (rc) return rc;

    const kv_t kv = model_kv(m);
    const double t0 = now_ms();
    int nt = 0;
    for (int p0 = 0; p0 < n_prompt && !rc; p0 += QM_MAX_CHUNK) {
        nt = n_prompt - p0 < QM_MAX_CHUNK ? n_prompt - p0 : QM_MAX_CHUNK;
        rc = load_chunk(m, prompt + p0, nt, p0);
        if (!rc) rc = run_chunk(m, &kv, nt, p0, p0 + nt == n_prompt);
    }
    /* first token; state[1] = pos0 of the last chunk + nt = n_prompt */
    if (!rc) rc = qm_set_i32(m->state + 2, 0);
    if (!rc) rc = qh_argmax_step(m->state, m->out_tok, m->state + 2, m->max_seq + 1, m->state + 1, nt,
                                 m->logits, V);
    if (!rc) rc = qh_sync();
    const double t1 = now_ms();
    if (rc) return rc;

    if (n_decode > 0 && m->use_graph && m->graph_id < 0) {
        rc = qh_capture_begin();
        if (!rc) {
            int rc2 = decode_step(m);
            int gid = -1;
            rc = qh_capture_end(&gid);
            if (!rc) rc = rc2;
            if (!rc) m->graph_id = gid;
            else if (gid >= 0) (void)qh_graph_destroy(gid);
        }
        if (rc) return rc;
    }
    for (int s = 0; s < n_decode && !rc; s++)
        rc = m->use_graph ? qh_graph_launch(m->graph_id) : decode_step(m);
    if (!rc) rc = qh_sync();
    const double t2 = now_ms();
    if (rc) return rc;
    m->have_logits = 1;

    rc = qh_d2h(out, m->out_tok, ((size_t)n_decode + 1) * sizeof(int));
    if (!rc) rc = qh_sync();
    if (rc) return rc;
    int n = n_decode + 1;
    if (stop_at_eos)
        for (int i = 0; i < n; i++)
            if (out[i] == QW3M_EOS0 || out[i] == QW3M_EOS1) { n = i + 1; break; }
    *n_out = n;
    m->t_prefill_ms = t1 - t0;
    m->t_decode_ms = t2 - t1;
    return QWEN3_HIP_OK;
}

int qwen3_hip_model_timing(const qwen3_hip_model *m, double *prefill_ms, double *decode_ms) {
    if (!m) return QWEN3_HIP_EINVAL;
    if (prefill_ms) *prefill_ms = m->t_prefill_ms;
    if (decode_ms) *decode_ms = m->t_decode_ms;
    return QWEN3_HIP_OK;
}

/* ---- multi-sequence batched decode ------------------------------------------ */

struct qwen3_hip_batch {
    qwen3_hip_model *m;
    int n_seq, max_ctx, out_ld;
    size_t kv_seq;                     /* floats of one sequence's cache in one layer */
    float *kc, *vc;                    /* [NL][n_seq][kv_seq] */
    float *logits;                     /* [n_seq][V] of the last decode step */
    float *part;                       /* [n_seq][QM_BATCH_PART_FLOATS] */
    int *tok, *pos, *plen;             /* [n_seq]: next token fed, its position, prompt length */
    int *out;                          /* [n_seq][out_ld]: token i of a sequence at i = pos - plen + 1 */
    int *h_next;                       /* host: position of each sequence's next fed token (-1: empty) */
    int *h_plen;                       /* host: prompt length of each sequence */
    int *h_out;                        /* host staging of out */
    int use_graph;
    int graph_id;
    int have_logits;
    double t_decode_ms;
    qwen3_hip_batch *next;             /* the model's list of open batches */
};

/* A batch's graph holds the model's device addresses: when the model closes
 * first, its batches lose the graph and the model, and later calls on them
 * return QWEN3_HIP_ESTATE instead of touching freed memory. */
static void detach_batches(qwen3_hip_model *m) {
    for (qwen3_hip_batch *b = m->batches; b; b = b->next) {
        if (b->graph_id >= 0) (void)qh_graph_destroy(b->graph_id);
        b->graph_id = -1;
        b->m = NULL;
    }
    m->batches = NULL;
}

void qwen3_hip_batch_close(qwen3_hip_batch *b) {
    if (!b) return;
    (void)qh_sync();
    if (b->m) {
        qwen3_hip_batch **pp = &b->m->batches;
        while (*pp && *pp != b) pp = &(*pp)->next;
        if (*pp) *pp = b->next;
    }
    if (b->graph_id >= 0) (void)qh_graph_destroy(b->graph_id);
    void *bufs[] = {b->kc, b->vc, b->logits, b->part, b->tok, b->pos, b->plen, b->out};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++) (void)qh_free(bufs[i]);
    free(b->h_next);
    free(b->h_plen);
    free(b->h_out);
    free(b);
}

int qwen3_hip_batch_open(qwen3_hip_batch **out, qwen3_hip_model *m, int n_seq, int max_ctx) {
    if (!out) return QWEN3_HIP_EINVAL;
    *out = NULL;
    if (!m || n_seq < 1 || n_seq > QM_MAX_CHUNK || max_ctx < 2 || max_ctx > m->max_seq) return QWEN3_HIP_EINVAL;
    qwen3_hip_batch *b = (qwen3_hip_batch *)calloc(1, sizeof *b);
    if (!b) return QWEN3_HIP_ENOMEM;
    b->m = m;
    b->n_seq = n_seq;
    b->max_ctx = max_ctx;
    b->out_ld = max_ctx + 1;
    b->kv_seq = (size_t)QW3M_N_KV_HEADS * max_ctx * QW3M_HEAD_DIM;
    b->use_graph = 1;
    b->graph_id = -1;
    int rc = QWEN3_HIP_ENOMEM;
    b->h_next = (int *)malloc((size_t)n_seq * sizeof(int));
    b->h_plen = (int *)calloc((size_t)n_seq, sizeof(int));
    b->h_out = (int *)malloc((size_t)n_seq * b->out_ld * sizeof(int));
    if (!b->h_next || !b->h_plen || !b->h_out) goto fail;
    for (int s = 0; s < n_seq; s++) b->h_next[s] = -1;
#define DEV(ptr, bytes)                                                   \
    do {                                                                  \
        if ((rc = qh_malloc((void **)&(ptr), (bytes))) != 0) goto fail;   \
    } while (0)
    const size_t kv_bytes = (size_t)NL * n_seq * b->kv_seq * sizeof(float);
    DEV(b->kc, kv_bytes);
    DEV(b->vc, kv_bytes);
    DEV(b->logits, (size_t)n_seq * V * sizeof(float));
    DEV(b->part, (size_t)n_seq * QM_BATCH_PART_FLOATS * sizeof(float));
    DEV(b->tok, (size_t)n_seq * sizeof(int));
    DEV(b->pos, (size_t)n_seq * sizeof(int));
    DEV(b->plen, (size_t)n_seq * sizeof(int));
    DEV(b->out, (size_t)n_seq * b->out_ld * sizeof(int));
#undef DEV
    rc = qm_zero_i32(b->tok, n_seq);
    if (!rc) rc = qm_zero_i32(b->pos, n_seq);
    if (!rc) rc = qm_zero_i32(b->plen, n_seq);
    if (!rc) rc = qh_sync();
    if (rc) goto fail;
    b->next = m->batches;
    m->batches = b;
    *out = b;
    return QWEN3_HIP_OK;
fail:
    qwen3_hip_batch_close(b);
    return rc;
}

int qwen3_hip_batch_set_graph(qwen3_hip_batch *b, int on) {
    if (!b) return QWEN3_HIP_EINVAL;
    if (!b->m) return QWEN3_HIP_ESTATE;
    b->use_graph = on ? 1 : 0;
    return QWEN3_HIP_OK;
}

int qwen3_hip_batch_prefill(qwen3_hip_batch *b, int seq, const int *prompt, int n_prompt) {
    if (!b || !prompt || seq < 0 || seq >= b->n_seq || n_prompt < 1 || n_prompt >= b->max_ctx)
        return QWEN3_HIP_EINVAL;
    if (!b->m) return QWEN3_HIP_ESTATE;
    int rc = check_tokens(prompt, n_prompt);
    if (rc) return rc;
    qwen3_hip_model *m = b->m;
    const kv_t kv = {b->kc + (size_t)seq * b->kv_seq, b->vc + (size_t)seq * b->kv_seq,
                     (size_t)b->n_seq * b->kv_seq, b->max_ctx};
    b->h_next[seq] = -1;
    m->have_logits = 0;             /* the model's logits buffer is reused below */
    for (int p0 = 0; p0 < n_prompt && !rc; p0 += QM_MAX_CHUNK) {
        const int nt = n_prompt - p0 < QM_MAX_CHUNK ? n_prompt - p0 : QM_MAX_CHUNK;
        rc = load_chunk(m, prompt + p0, nt, p0);
        if (!rc) rc = run_chunk(m, &kv, nt, p0, p0 + nt == n_prompt);
    }
    /* first token: out[seq][0] at pos - plen + 1 = 0, then pos = n_prompt */
    if (!rc) rc = qm_set_i32(b->pos + seq, n_prompt - 1);
    if (!rc) rc = qm_set_i32(b->plen + seq, n_prompt);
    if (!rc) rc = qm_argmax_rows(m->logits, V, 1, b->tok + seq, b->pos + seq, b->plen + seq,
                                 b->out + (size_t)seq * b->out_ld, b->out_ld);
    if (!rc) rc = qh_sync();
    if (!rc) {
        b->h_next[seq] = n_prompt;
        b->h_plen[seq] = n_prompt;
    }
    return rc;
}

/* one decode step of every sequence: token tok[s] at position pos[s].  When
 * the o and down projections split K (the skinny kernel at small n), their
 * slice sums are added by the residual + RMSNorm kernel that consumes them
 * (the sums a reduction launch would form), one launch fewer each. */
static int batch_step(qwen3_hip_batch *b) {
    qwen3_hip_model *m = b->m;
    const int n = b->n_seq;
    const float eps = QW3M_RMS_EPS;
    const size_t lstride = (size_t)n * b->kv_seq;
    int rc = QWEN3_HIP_OK;
    const float *dpart = NULL, *opart = NULL;
    int dks = 0, oks = 0;
    for (int l = 0; l < NL && !rc; l++) {
        const layer_t *L = &m->L[l];
        if (l == 0) rc = qm_rows_norm(m->x, NULL, m->embed, b->tok, V, L->in_norm, m->xb, n, H, eps);
        else rc = qm_rows_norm_split(m->x, dks ? NULL : m->dn, NULL, NULL, 0, L->in_norm, m->xb, n, H, eps, dpart, dks);
        if (!rc) rc = qh_gemm(m->qkv, m->xb, L->wqkv, n, H, QKV_N);
        if (!rc) rc = qm_attention_decode_batch(m->qkv, m->att, b->part, b->kc + l * lstride, b->vc + l * lstride,
                                                b->kv_seq, L->qn, L->kn, m->rcos, m->rsin, b->pos, n,
                                                b->max_ctx, eps);
        if (!rc) rc = qh_gemm_split(m->ob, m->att, L->wo, n, QW3M_Q_DIM, H, &opart, &oks);
        if (!rc) rc = qm_rows_norm_split(m->x, oks ? NULL : m->ob, NULL, NULL, 0, L->post_norm, m->xb, n, H, eps,
                                         opart, oks);
        if (!rc) rc = qh_gemm_gate_up_silu(m->hb, m->xb, L->wg, L->wu, n, H, QW3M_INTER);
        if (!rc) rc = qh_gemm_split(m->dn, m->hb, L->wd, n, QW3M_INTER, H, &dpart, &dks);
    }
    if (!rc) rc = qm_rows_norm_split(m->x, dks ? NULL : m->dn, NULL, NULL, 0, m->final_norm, m->xb, n, H, eps,
                                     dpart, dks);
    if (!rc) rc = qh_gemm(b->logits, m->xb, m->embed, n, H, V);
    if (!rc) rc = qm_argmax_rows(b->logits, V, n, b->tok, b->pos, b->plen, b->out, b->out_ld);
    return rc;
}

int qwen3_hip_batch_decode(qwen3_hip_batch *b, int n_decode, int *out) {
    if (!b || !out || n_decode < 0) return QWEN3_HIP_EINVAL;
    if (!b->m) return QWEN3_HIP_ESTATE;
    for (int s = 0; s < b->n_seq; s++)
        if (b->h_next[s] < 0 || (long)b->h_next[s] + n_decode > b->max_ctx) return QWEN3_HIP_EINVAL;
    int rc = QWEN3_HIP_OK;
    const double t0 = now_ms();
    for (int i = 0; i < n_decode && !rc; i++) {
        /* with graphs on, a first step runs eagerly (any workspace its GEMM
           plans need is allocated then, outside capture); later steps replay
           the one captured step */
        if (!b->use_graph || (b->graph_id < 0 && i == 0)) {
            rc = batch_step(b);
            continue;
        }
        if (b->graph_id < 0) {
            rc = qh_capture_begin();
            if (rc) break;
            const int rc2 = batch_step(b);
            int gid = -1;
            rc = qh_capture_end(&gid);
            if (!rc) rc = rc2;
            if (rc) {
                if (gid >= 0) (void)qh_graph_destroy(gid);
                break;
            }
            b->graph_id = gid;
        }
        rc = qh_graph_launch(b->graph_id);
    }
    if (!rc) rc = qh_sync();
    b->t_decode_ms = now_ms() - t0;
    if (rc) return rc;
    if (n_decode > 0) b->have_logits = 1;
    rc = qh_d2h(b->h_out, b->out, (size_t)b->n_seq * b->out_ld * sizeof(int));
    if (!rc) rc = qh_sync();
    if (rc) return rc;
    for (int s = 0; s < b->n_seq; s++) {
        /* the token fed at position h_next sits at out index h_next - plen */
        const int *row = b->h_out + (size_t)s * b->out_ld + (b->h_next[s] - b->h_plen[s]);
        memcpy(out + (size_t)s * (n_decode + 1), row, ((size_t)n_decode + 1) * sizeof(int));
        b->h_next[s] += n_decode;
    }
    return QWEN3_HIP_OK;
}

int qwen3_hip_batch_logits(qwen3_hip_batch *b, float *out) {
    if (!b || !out || !b->have_logits) return QWEN3_HIP_EINVAL;
    if (!b->m) return QWEN3_HIP_ESTATE;
    int rc = qh_d2h(out, b->logits, (size_t)b->n_seq * V * sizeof(float));
    if (!rc) rc = qh_sync();
    return rc;
}

int qwen3_hip_batch_timing(const qwen3_hip_batch *b, double *decode_ms) {
    if (!b) return QWEN3_HIP_EINVAL;
    if (decode_ms) *decode_ms = b->t_decode_ms;
    return QWEN3_HIP_OK;
}
