/* QW3M weight blob: random-init writer and header/tensor-table parser.
 *
 * Format (fpga_bringup/src/src/qwen3_config.h:33-81, parser
 * fpga_bringup/src/src/qwen3.c:87-146):
 *   256-byte little-endian header: "QW3M", version 1, model shapes, dtype 1
 *   (bf16), rope theta, rms eps, special tokens, data_start @68, align @72,
 *   layout @76 (0 = row-major, 1 = tile-major), tile_n @80, tile_k @84;
 *   then 310 bf16 tensors in a fixed order, each starting on an `align`
 *   boundary, with the file ending exactly at the end of the last tensor.
 *   Tile-major files keep embed_tokens and the norm vectors row-major and
 *   store every projection matrix as contiguous tile_n x tile_k blocks at
 *   element offset ((n/tn)*(K/tk) + k/tk)*tn*tk + (n%tn)*tk + k%tk
 *   (fpga_bringup/src/src/kernels_ame.c:212-215).  With align 128 (row) and
 *   4096 (tile) the sizes are 1,192,100,096 and 1,192,433,664 bytes, the
 *   sizes of the reference's exported files (fpga_bringup/L4_demo/README.md:39).
 *
 * Random init (no real weights offline): every projection and embed_tokens
 * ~ N(0, 0.02) rounded to bf16, every norm weight = 1.0.  Tensor t (blob order,
 * 0 = embed_tokens ... 309 = final norm) uses seed base + t.  Values come in
 * blocks of 256: block i of a tensor is seeded with output i of a SplitMix64
 * stream started at the tensor seed, and filled by Box-Muller on 53-bit
 * uniforms from a SplitMix64 stream started at that block seed (both outputs
 * of each pair used), then rounded to bf16 with round-to-nearest-even.  A
 * block depends only on (seed, block index), so the fill runs in parallel.
 */
#include "qw3m.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define GAMMA 0x9E3779B97F4A7C15ull

static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static uint16_t to_bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

/* block `blk` of a N(0, sigma) tensor with seed `seed`: m <= 256 values */
static void normal_block(uint16_t *dst, size_t m, uint64_t seed, uint64_t blk, float sigma) {
    uint64_t st = mix64(seed + (blk + 1) * GAMMA);   /* block seed: output blk of the tensor stream */
    const double two_pi = 6.283185307179586476925286766559;
    size_t i = 0;
    while (i < m) {
        st += GAMMA;
        const double u1 = ((double)(mix64(st) >> 11) + 1.0) * 0x1p-53;   /* (0, 1] */
        st += GAMMA;
        const double u2 = (double)(mix64(st) >> 11) * 0x1p-53;           /* [0, 1) */
        const double r = sqrt(-2.0 * log(u1));
        dst[i++] = to_bf16_rne((float)(r * cos(two_pi * u2) * (double)sigma));
        if (i < m) dst[i++] = to_bf16_rne((float)(r * sin(two_pi * u2) * (double)sigma));
    }
}

/* ---- tensor table --------------------------------------------------------- */

static void tensor_shape(int t, int *rows, int *cols, int *is_matrix) {
    /* blob order, qwen3_config.h:63-78 */
    if (t == 0) { *rows = QW3M_VOCAB; *cols = QW3M_HIDDEN; *is_matrix = 0; return; }
    if (t == QW3M_N_TENSORS - 1) { *rows = 1; *cols = QW3M_HIDDEN; *is_matrix = 0; return; }
    static const int r[11] = {1, QW3M_Q_DIM, QW3M_KV_DIM, QW3M_KV_DIM, 1, 1,
                              QW3M_HIDDEN, 1, QW3M_INTER, QW3M_INTER, QW3M_HIDDEN};
    static const int c[11] = {QW3M_HIDDEN, QW3M_HIDDEN, QW3M_HIDDEN, QW3M_HIDDEN, QW3M_HEAD_DIM,
                              QW3M_HEAD_DIM, QW3M_Q_DIM, QW3M_HIDDEN, QW3M_HIDDEN, QW3M_HIDDEN,
                              QW3M_INTER};
    const int j = (t - 1) % 11;
    *rows = r[j];
    *cols = c[j];
    *is_matrix = r[j] > 1;
}

static size_t align_up(size_t x, size_t a) { return (x + a - 1) & ~(a - 1); }

int qw3m_table(int layout, size_t *offsets, size_t *total) {
    if (layout != QW3M_LAYOUT_ROW && layout != QW3M_LAYOUT_TILE) return -1;
    const size_t al = layout == QW3M_LAYOUT_ROW ? QW3M_ALIGN_ROW : QW3M_ALIGN_TILE;
    size_t pos = align_up(QW3M_HEADER_BYTES, al);
    for (int t = 0; t < QW3M_N_TENSORS; t++) {
        int rows, cols, mat;
        tensor_shape(t, &rows, &cols, &mat);
        pos = align_up(pos, al);
        if (offsets) offsets[t] = pos;
        pos += (size_t)rows * cols * 2;
    }
    if (total) *total = pos;
    return 0;
}

size_t qw3m_size(int layout) {
    size_t total = 0;
    return qw3m_table(layout, NULL, &total) == 0 ? total : 0;
}

void qw3m_tensor_shape(int t, int *rows, int *cols, int *is_matrix) {
    tensor_shape(t, rows, cols, is_matrix);
}

/* ---- writer ------------------------------------------------------------ */

static void put_i32(uint8_t *p, int32_t v) {
    const uint32_t u = (uint32_t)v;
    p[0] = (uint8_t)u; p[1] = (uint8_t)(u >> 8); p[2] = (uint8_t)(u >> 16); p[3] = (uint8_t)(u >> 24);
}
static void put_f32(uint8_t *p, float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    put_i32(p, (int32_t)u);
}

typedef struct {
    uint8_t *blob;
    const size_t *off;
    int layout;
    uint64_t seed;
    size_t first, last;      /* global 256-element block range [first, last) */
    const size_t *tblock;    /* first global block of each tensor, [311] */
} job_t;

static void *fill_worker(void *arg) {
    const job_t *j = (const job_t *)arg;
    uint16_t tmp[256];
    int t = 0;
    for (size_t g = j->first; g < j->last; g++) {
        while (g >= j->tblock[t + 1]) t++;
        int rows, cols, mat;
        tensor_shape(t, &rows, &cols, &mat);
        const size_t n = (size_t)rows * cols;
        const size_t blk = g - j->tblock[t];
        const size_t e0 = blk * 256;
        const size_t m = n - e0 < 256 ? n - e0 : 256;
        uint16_t *base = (uint16_t *)(j->blob + j->off[t]);
        if (!mat && rows == 1) {                      /* norm weights: 1.0 */
            for (size_t i = 0; i < m; i++) base[e0 + i] = 0x3F80u;
            continue;
        }
        normal_block(tmp, m, j->seed + (uint64_t)t, blk, 0.02f);
        if (j->layout == QW3M_LAYOUT_ROW || !mat) {
            memcpy(base + e0, tmp, m * 2);
        } else {
            const size_t ktiles = (size_t)cols / QW3M_TILE_K;
            for (size_t i = 0; i < m; i++) {
                const size_t e = e0 + i;
                const size_t n_ = e / (size_t)cols, k = e % (size_t)cols;
                const size_t tile = (n_ / QW3M_TILE_N) * ktiles + k / QW3M_TILE_K;
                base[tile * QW3M_TILE_N * QW3M_TILE_K + (n_ % QW3M_TILE_N) * QW3M_TILE_K +
                     k % QW3M_TILE_K] = tmp[i];
            }
        }
    }
    return NULL;
}

int qw3m_write_random(void *blob, size_t size, uint64_t seed, int layout, int threads) {
    size_t off[QW3M_N_TENSORS], total = 0;
    if (!blob || qw3m_table(layout, off, &total) != 0) return -1;
    if (size != total) return -1;
    uint8_t *b = (uint8_t *)blob;
    memset(b, 0, QW3M_HEADER_BYTES);
    b[0] = 'Q'; b[1] = 'W'; b[2] = '3'; b[3] = 'M';
    put_i32(b + 4, 1);
    put_i32(b + 8, QW3M_HIDDEN);
    put_i32(b + 12, QW3M_INTER);
    put_i32(b + 16, QW3M_N_LAYERS);
    put_i32(b + 20, QW3M_N_HEADS);
    put_i32(b + 24, QW3M_N_KV_HEADS);
    put_i32(b + 28, QW3M_HEAD_DIM);
    put_i32(b + 32, QW3M_VOCAB);
    put_i32(b + 36, QW3M_MAX_POS);
    put_i32(b + 40, 1);                       /* tie_embeddings */
    put_i32(b + 44, QW3M_DTYPE_BF16);
    put_f32(b + 48, QW3M_ROPE_THETA);
    put_f32(b + 52, QW3M_RMS_EPS);
    put_i32(b + 56, QW3M_BOS);
    put_i32(b + 60, QW3M_EOS0);
    put_i32(b + 64, QW3M_EOS1);
    put_i32(b + 68, (int32_t)off[0]);
    put_i32(b + 72, layout == QW3M_LAYOUT_ROW ? QW3M_ALIGN_ROW : QW3M_ALIGN_TILE);
    put_i32(b + 76, layout);
    put_i32(b + 80, layout == QW3M_LAYOUT_TILE ? QW3M_TILE_N : 0);
    put_i32(b + 84, layout == QW3M_LAYOUT_TILE ? QW3M_TILE_K : 0);
    /* padding between tensors is zero */
    for (int t = 0; t < QW3M_N_TENSORS; t++) {
        int rows, cols, mat;
        tensor_shape(t, &rows, &cols, &mat);
        const size_t end = off[t] + (size_t)rows * cols * 2;
        const size_t next = t + 1 < QW3M_N_TENSORS ? off[t + 1] : total;
        if (next > end) memset(b + end, 0, next - end);
    }
    if (off[0] > QW3M_HEADER_BYTES) memset(b + QW3M_HEADER_BYTES, 0, off[0] - QW3M_HEADER_BYTES);

    size_t tblock[QW3M_N_TENSORS + 1];
    tblock[0] = 0;
    for (int t = 0; t < QW3M_N_TENSORS; t++) {
        int rows, cols, mat;
        tensor_shape(t, &rows, &cols, &mat);
        tblock[t + 1] = tblock[t] + ((size_t)rows * cols + 255) / 256;
    }
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t th[64];
    job_t jobs[64];
    const size_t nb = tblock[QW3M_N_TENSORS];
    int started = 0, rc = 0;
    for (int i = 0; i < threads; i++) {
        jobs[i] = (job_t){b, off, layout, seed, nb * i / threads, nb * (i + 1) / threads, tblock};
        if (i == threads - 1) break;
        if (pthread_create(&th[i], NULL, fill_worker, &jobs[i]) != 0) { rc = -1; break; }
        started++;
    }
    if (rc == 0) {
        fill_worker(&jobs[threads - 1]);
    } else {
        /* run the unstarted ranges on this thread */
        for (int i = started; i < threads; i++) fill_worker(&jobs[i]);
    }
    for (int i = 0; i < started; i++) pthread_join(th[i], NULL);
    return 0;
}

/* ---- parser ------------------------------------------------------------ */

static int32_t get_i32(const uint8_t *p) {
    return (int32_t)((uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
                     ((uint32_t)p[3] << 24));
}
static float get_f32(const uint8_t *p) {
    const uint32_t u = (uint32_t)get_i32(p);
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* checks in the order of qwen3.c:92-143, with the same error codes */
int qw3m_parse(const void *blob, size_t size, qw3m_info_t *info) {
    const uint8_t *b = (const uint8_t *)blob;
    if (!b || size < QW3M_HEADER_BYTES) return QW3M_ERR_SIZE;
    if (b[0] != 'Q' || b[1] != 'W' || b[2] != '3' || b[3] != 'M') return QW3M_ERR_MAGIC;
    if (get_i32(b + 4) != 1) return QW3M_ERR_VERSION;
    if (get_i32(b + 44) != QW3M_DTYPE_BF16) return QW3M_ERR_DTYPE;
    if (get_i32(b + 8) != QW3M_HIDDEN || get_i32(b + 12) != QW3M_INTER ||
        get_i32(b + 16) != QW3M_N_LAYERS || get_i32(b + 20) != QW3M_N_HEADS ||
        get_i32(b + 24) != QW3M_N_KV_HEADS || get_i32(b + 28) != QW3M_HEAD_DIM ||
        get_i32(b + 32) != QW3M_VOCAB)
        return QW3M_ERR_SHAPE;
    const int32_t align = get_i32(b + 72);
    if (align < QW3M_ALIGN_ROW || (align & (align - 1)) != 0) return QW3M_ERR_SHAPE;
    const int layout = get_i32(b + 76), tn = get_i32(b + 80), tk = get_i32(b + 84);
    if (layout == QW3M_LAYOUT_ROW) {
        /* accepted */
    } else if (layout == QW3M_LAYOUT_TILE) {
        /* tiles must divide every matrix dimension (N in {1024, 2048, 3072},
           K in {1024, 2048, 3072}) */
        if (tn <= 0 || tk <= 0 || 1024 % tn || 1024 % tk) return QW3M_ERR_LAYOUT;
    } else {
        return QW3M_ERR_LAYOUT;
    }
    if (get_f32(b + 48) != QW3M_ROPE_THETA || get_f32(b + 52) != QW3M_RMS_EPS) return QW3M_ERR_SHAPE;
    const int32_t ds = get_i32(b + 68);
    if (ds < 0) return QW3M_ERR_SIZE;
    size_t pos = (size_t)ds;
    for (int t = 0; t < QW3M_N_TENSORS; t++) {
        int rows, cols, mat;
        tensor_shape(t, &rows, &cols, &mat);
        pos = align_up(pos, (size_t)align);
        const size_t nbytes = (size_t)rows * cols * 2;
        if (pos + nbytes > size) return QW3M_ERR_SIZE;
        if (info) info->offset[t] = pos;
        pos += nbytes;
    }
    if (pos != size) return QW3M_ERR_SIZE;
    if (info) {
        info->layout = layout;
        info->tile_n = layout == QW3M_LAYOUT_TILE ? tn : 0;
        info->tile_k = layout == QW3M_LAYOUT_TILE ? tk : 0;
        info->align = align;
        info->data_start = ds;
    }
    return 0;
}
