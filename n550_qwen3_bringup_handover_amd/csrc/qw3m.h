/* QW3M weight blob (fpga_bringup/src/src/qwen3_config.h:33-81): constants,
 * tensor table, random-init writer and header parser.  Internal header. */
#ifndef QWEN3_HIP_QW3M_H
#define QWEN3_HIP_QW3M_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Qwen3-0.6B (qwen3_config.h:9-35) */
#define QW3M_HIDDEN      1024
#define QW3M_INTER       3072
#define QW3M_N_LAYERS    28
#define QW3M_N_HEADS     16
#define QW3M_N_KV_HEADS  8
#define QW3M_HEAD_DIM    128
#define QW3M_VOCAB       151936
#define QW3M_MAX_POS     40960
#define QW3M_Q_DIM       2048
#define QW3M_KV_DIM      1024
#define QW3M_ROPE_THETA  1000000.0f
#define QW3M_RMS_EPS     1e-06f
#define QW3M_BOS         151643
#define QW3M_EOS0        151645
#define QW3M_EOS1        151643

#define QW3M_HEADER_BYTES 256
#define QW3M_DTYPE_BF16   1
#define QW3M_LAYOUT_ROW   0          /* kernels.h:67-68 */
#define QW3M_LAYOUT_TILE  1
#define QW3M_ALIGN_ROW    128
#define QW3M_ALIGN_TILE   4096
#define QW3M_TILE_N       128        /* kernels.h:21-22 */
#define QW3M_TILE_K       32
#define QW3M_N_TENSORS    (1 + QW3M_N_LAYERS * 11 + 1)

/* qwen3.h:188-200 */
enum {
    QW3M_OK = 0,
    QW3M_ERR_MAGIC = -1,
    QW3M_ERR_VERSION = -2,
    QW3M_ERR_DTYPE = -3,
    QW3M_ERR_SHAPE = -4,
    QW3M_ERR_SIZE = -5,
    QW3M_ERR_OOM = -6,
    QW3M_ERR_LAYOUT = -7
};

/* per-layer tensor index j = (t - 1) % 11 */
enum {
    QW3M_T_IN_NORM = 0, QW3M_T_WQ, QW3M_T_WK, QW3M_T_WV, QW3M_T_QNORM, QW3M_T_KNORM,
    QW3M_T_WO, QW3M_T_POST_NORM, QW3M_T_WGATE, QW3M_T_WUP, QW3M_T_WDOWN
};

typedef struct {
    size_t offset[QW3M_N_TENSORS];   /* byte offset of each tensor in the blob */
    int layout, tile_n, tile_k, align, data_start;
} qw3m_info_t;

size_t qw3m_size(int layout);                              /* 0 for an unknown layout */
int qw3m_table(int layout, size_t *offsets, size_t *total);
void qw3m_tensor_shape(int t, int *rows, int *cols, int *is_matrix);
int qw3m_write_random(void *blob, size_t size, uint64_t seed, int layout, int threads);
int qw3m_parse(const void *blob, size_t size, qw3m_info_t *info);

#ifdef __cplusplus
}
#endif
#endif
