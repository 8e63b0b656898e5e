/* Host side of the MI355X GEMM plug-in, in C11: the reference's GEMM entry
 * points (fpga_bringup/src/src/kernels.h:44-92) implemented over the HIP shim
 * (hip_shim.h).  This file owns the policy that the reference leaves to the
 * caller: which device copy of a weight to use, where activations are
 * staged, and what happens on an error.  It contains no GPU code and no HIP
 * calls of its own.
 */
#define _POSIX_C_SOURCE 199309L   /* clock_gettime */
#include "qwen3_hip.h"
#include "hip_shim.h"

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* Model dimensions that a TILE layout must divide (the same list the AME
 * kernel checks, fpga_bringup/src/src/kernels_ame.c:196-205). */
static const int k_model_n[] = { 2048, 1024, 1024, 3072 };   /* Q, KV, HIDDEN, INTER */
static const int k_model_k[] = { 1024, 2048, 3072 };         /* HIDDEN, Q, INTER */

/* ---- state ---------------------------------------------------------------- */
static int g_ready;
static int g_abort = 1;
static int g_abort_env_checked;
static int g_err;                       /* sticky: first error since last read */
static int g_layout;                    /* 0 ROW, 1 TILE */
static int g_tile_n = 128, g_tile_k = 32;

static void  *g_a_d;  static size_t g_a_cap;     /* device staging for A */
/* device staging for unmapped B, uploaded on every call: [0] B (or Wg),
 * [1] Wu, [2] a TILE buffer before it is re-laid out row-major */
static void  *g_b_d[3]; static size_t g_b_cap[3];
static int g_wcache = -1;               /* address cache of unmapped B: -1 = not yet read from env */
static void  *g_a_h;  static size_t g_a_hcap;    /* pinned host staging for A */
static void  *g_c_h;  static size_t g_c_hcap;    /* pinned host staging for C */

typedef struct {
    const unsigned char *host;
    size_t bytes;
    unsigned char *dev;
} wmap_t;
#define MAX_MAPS 16
static wmap_t g_maps[MAX_MAPS];
static int g_nmaps;

typedef struct {
    const uint16_t *host;
    int N, K;
    int layout, tn, tk;
    int from_map;           /* device copy derived from a mapped range */
    uint64_t fp;            /* content fingerprint (unmapped buffers only) */
    void *dev;
} wcache_t;
static wcache_t *g_wc;
static int g_nwc, g_capwc;

/* ---- errors ----------------------------------------------------------------- */
static const char *k_err_names[] = {
    "ok", "invalid argument", "no usable gfx950 device", "out of memory",
    "kernel launch failed", "HIP runtime error", "weight layout does not fit the shape",
    "called in the wrong state", "size beyond a supported maximum"
};

const char *qwen3_hip_strerror(int err) {
    if (err < 0 || err > QWEN3_HIP_ETOOBIG) return "unknown error";
    return k_err_names[err];
}

static void check_abort_env(void) {
    if (g_abort_env_checked) return;
    g_abort_env_checked = 1;
    const char *e = getenv("QWEN3_HIP_ABORT");
    if (e && e[0] == '0') g_abort = 0;
}

/* Record an error from a void entry point; abort unless disabled. */
static void fail(int code, const char *where) {
    if (!g_err) g_err = code;
    check_abort_env();
    if (g_abort) {
        fprintf(stderr, "qwen3_hip: %s: %s (hip: %s)\n", where,
                qwen3_hip_strerror(code), qh_last_hip_error_string());
        fflush(stderr);
        abort();
    }
}

static int note(int code) {
    if (code && !g_err) g_err = code;
    return code;
}

int qwen3_hip_last_error(void) {
    int e = g_err;
    g_err = 0;
    return e;
}

void qwen3_hip_set_abort(int on) {
    g_abort_env_checked = 1;
    g_abort = on ? 1 : 0;
}

/* ---- init / release ------------------------------------------------------------ */
int qwen3_hip_init(int device) {
    if (g_ready) return QWEN3_HIP_OK;
    check_abort_env();
    if (device < 0) {
        const char *e = getenv("QWEN3_HIP_DEVICE");
        device = e ? atoi(e) : 0;
    }
    int rc = qh_init(device);
    if (rc) return note(rc);
    g_ready = 1;
    return QWEN3_HIP_OK;
}

static int ensure_ready(void) {
    return g_ready ? QWEN3_HIP_OK : qwen3_hip_init(-1);
}

void qwen3_hip_release(void) {
    if (!g_ready) return;
    (void)qh_sync();
    for (int i = 0; i < g_nwc; i++) (void)qh_free(g_wc[i].dev);
    free(g_wc);
    g_wc = NULL;
    g_nwc = g_capwc = 0;
    for (int i = 0; i < g_nmaps; i++) (void)qh_free(g_maps[i].dev);
    g_nmaps = 0;
    (void)qh_free(g_a_d);
    g_a_d = NULL;
    g_a_cap = 0;
    for (int i = 0; i < 3; i++) {
        (void)qh_free(g_b_d[i]);
        g_b_d[i] = NULL;
        g_b_cap[i] = 0;
    }
    (void)qh_host_free(g_a_h);
    (void)qh_host_free(g_c_h);
    g_a_h = g_c_h = NULL;
    g_a_hcap = g_c_hcap = 0;
    qh_shutdown();
    g_ready = 0;
}

const char *qwen3_kernel_name(void) { return "hip-gfx950"; }

const char *qwen3_hip_device_name(void) { return qh_device_name(); }

/* ---- weight layout (kernels.h:59-89) --------------------------------------------- */
int qwen3_set_weight_layout(int layout, int tile_n, int tile_k) {
    if (layout == 0) {
        g_layout = 0;
        return 0;
    }
    if (layout != 1 || tile_n <= 0 || tile_k <= 0) return -1;
    for (unsigned i = 0; i < sizeof k_model_n / sizeof k_model_n[0]; i++)
        if (k_model_n[i] % tile_n) return -1;
    for (unsigned i = 0; i < sizeof k_model_k / sizeof k_model_k[0]; i++)
        if (k_model_k[i] % tile_k) return -1;
    g_layout = 1;
    g_tile_n = tile_n;
    g_tile_k = tile_k;
    return 0;
}

/* ---- weight copies on the device -------------------------------------------------- */
static uint64_t mix64(uint64_t h, uint64_t v) {
    h ^= v + 0x9E3779B97F4A7C15ull + (h << 6) + (h >> 2);
    h *= 0xBF58476D1CE4E5B9ull;
    return h ^ (h >> 31);
}

/* shape + first/last 256 bytes + 512 sampled 8-byte words */
static uint64_t fingerprint(const uint16_t *b, int N, int K) {
    const unsigned char *p = (const unsigned char *)b;
    const size_t bytes = (size_t)N * (size_t)K * 2u;
    uint64_t h = mix64((uint64_t)N, (uint64_t)K);
    uint64_t w;
    size_t edge = bytes < 256 ? bytes : 256;
    for (size_t i = 0; i + 8 <= edge; i += 8) { memcpy(&w, p + i, 8); h = mix64(h, w); }
    for (size_t i = bytes - edge; i + 8 <= bytes; i += 8) { memcpy(&w, p + i, 8); h = mix64(h, w); }
    if (bytes >= 8) {
        const size_t words = bytes / 8;
        for (size_t s = 0; s < 512; s++) {
            size_t idx = (size_t)((s * 2654435761ull) % words);
            memcpy(&w, p + idx * 8, 8);
            h = mix64(h, w);
        }
    }
    for (size_t i = bytes & ~(size_t)7; i < bytes; i++) h = mix64(h, p[i]);
    return h;
}

static const wmap_t *find_map(const void *b, size_t bytes) {
    const unsigned char *q = (const unsigned char *)b;
    for (int i = 0; i < g_nmaps; i++) {
        const wmap_t *m = &g_maps[i];
        if (q >= m->host && q + bytes <= m->host + m->bytes && q + bytes >= q) return m;
    }
    return NULL;
}

int qwen3_hip_map_weights(const void *blob, size_t size) {
    int rc = ensure_ready();
    if (rc) return rc;
    if (!blob || size == 0) return note(QWEN3_HIP_EINVAL);
    if (find_map(blob, size)) return QWEN3_HIP_OK;
    if (g_nmaps == MAX_MAPS) return note(QWEN3_HIP_ETOOBIG);
    void *d = NULL;
    if ((rc = qh_malloc(&d, size))) return note(rc);
    if ((rc = qh_h2d(d, blob, size)) || (rc = qh_sync())) {
        (void)qh_free(d);
        return note(rc);
    }
    g_maps[g_nmaps].host = (const unsigned char *)blob;
    g_maps[g_nmaps].bytes = size;
    g_maps[g_nmaps].dev = (unsigned char *)d;
    g_nmaps++;
    return QWEN3_HIP_OK;
}

int qwen3_hip_unmap_weights(const void *blob) {
    int idx = -1;
    for (int i = 0; i < g_nmaps; i++)
        if (g_maps[i].host == (const unsigned char *)blob) idx = i;
    if (idx < 0) return note(QWEN3_HIP_EINVAL);
    const wmap_t m = g_maps[idx];
    (void)qh_sync();
    /* copies re-laid out from this range go with it */
    int j = 0;
    for (int i = 0; i < g_nwc; i++) {
        const unsigned char *h = (const unsigned char *)g_wc[i].host;
        if (g_wc[i].from_map && h >= m.host && h < m.host + m.bytes) (void)qh_free(g_wc[i].dev);
        else g_wc[j++] = g_wc[i];
    }
    g_nwc = j;
    (void)qh_free(m.dev);
    g_maps[idx] = g_maps[--g_nmaps];
    return QWEN3_HIP_OK;
}

void qwen3_hip_forget_weights(const void *b) {
    int j = 0;
    for (int i = 0; i < g_nwc; i++) {
        wcache_t *e = &g_wc[i];
        int drop = b ? (e->host == (const uint16_t *)b) : !e->from_map;
        if (drop) {
            (void)qh_sync();
            (void)qh_free(e->dev);
        } else {
            g_wc[j++] = *e;
        }
    }
    g_nwc = j;
}

size_t qwen3_hip_weight_bytes(void) {
    size_t t = 0;
    for (int i = 0; i < g_nmaps; i++) t += g_maps[i].bytes;
    for (int i = 0; i < g_nwc; i++) t += (size_t)g_wc[i].N * (size_t)g_wc[i].K * 2u;
    for (int i = 0; i < 3; i++) t += g_b_cap[i];
    return t;
}

static wcache_t *cache_find(const uint16_t *b, int N, int K, int layout, int tn, int tk) {
    for (int i = 0; i < g_nwc; i++) {
        wcache_t *e = &g_wc[i];
        if (e->host == b && e->N == N && e->K == K && e->layout == layout &&
            (layout == 0 || (e->tn == tn && e->tk == tk)))
            return e;
    }
    return NULL;
}

static wcache_t *cache_add(void) {
    if (g_nwc == g_capwc) {
        int cap = g_capwc ? 2 * g_capwc : 64;
        wcache_t *n = (wcache_t *)realloc(g_wc, (size_t)cap * sizeof *n);
        if (!n) return NULL;
        g_wc = n;
        g_capwc = cap;
    }
    wcache_t *e = &g_wc[g_nwc++];
    memset(e, 0, sizeof *e);
    return e;
}

static int grow(void **p, size_t *cap, size_t need);

static int weight_cache_on(void) {
    if (g_wcache < 0) {
        const char *e = getenv("QWEN3_HIP_WEIGHT_CACHE");
        g_wcache = (e && e[0] == '1') ? 1 : 0;
    }
    return g_wcache;
}

void qwen3_hip_set_weight_cache(int on) {
    if (!on && g_wcache == 1) qwen3_hip_forget_weights(NULL);
    g_wcache = on ? 1 : 0;
}

/* Unmapped B without the address cache: copied to device staging on every
 * call, as the reference reads B on every call (SRC/kernels_scalar.c:9-21),
 * so a caller may change B between calls.  slot 0 holds B (or Wg), slot 1 Wu;
 * a TILE buffer goes through slot 2 and is re-laid out row-major into its
 * slot. */
static const uint16_t *weight_upload(const uint16_t *b, int N, int K, int layout, int slot, int *rc) {
    const size_t bytes = (size_t)N * (size_t)K * 2u;
    if ((*rc = grow(&g_b_d[slot], &g_b_cap[slot], bytes))) return NULL;
    if (layout == 0) {
        if ((*rc = qh_h2d(g_b_d[slot], b, bytes))) return NULL;
        return (const uint16_t *)g_b_d[slot];
    }
    if ((*rc = grow(&g_b_d[2], &g_b_cap[2], bytes))) return NULL;
    if ((*rc = qh_h2d(g_b_d[2], b, bytes))) return NULL;
    if ((*rc = qh_tile_to_row((uint16_t *)g_b_d[slot], (const uint16_t *)g_b_d[2], N, K,
                              g_tile_n, g_tile_k)))
        return NULL;
    return (const uint16_t *)g_b_d[slot];
}

/* Device pointer of B[N,K] in row-major form, for a host pointer b stored in
 * `layout`.  Returns NULL and sets *rc on failure. */
static const uint16_t *weight_dev(const uint16_t *b, int N, int K, int layout, int slot, int *rc) {
    const size_t bytes = (size_t)N * (size_t)K * 2u;
    const int tn = g_tile_n, tk = g_tile_k;
    const wmap_t *m = find_map(b, bytes);
    *rc = 0;

    if (m && layout == 0)       /* zero-cost: an offset into the mapped blob */
        return (const uint16_t *)(m->dev + ((const unsigned char *)b - m->host));

    if (layout == 1 && (N % tn || K % tk)) { *rc = QWEN3_HIP_ELAYOUT; return NULL; }

    if (!m && !weight_cache_on())
        return weight_upload(b, N, K, layout, slot, rc);

    wcache_t *e = cache_find(b, N, K, layout, tn, tk);
    uint64_t fp = 0;
    if (e) {
        if (e->from_map) return (const uint16_t *)e->dev;
        fp = fingerprint(b, N, K);
        if (fp == e->fp) return (const uint16_t *)e->dev;
        /* contents changed under the same address: upload again */
        (void)qh_sync();
        (void)qh_free(e->dev);
        e->dev = NULL;
    } else {
        e = cache_add();
        if (!e) { *rc = QWEN3_HIP_ENOMEM; return NULL; }
        e->host = b; e->N = N; e->K = K; e->layout = layout; e->tn = tn; e->tk = tk;
        if (!m) fp = fingerprint(b, N, K);
    }
    e->from_map = m != NULL;
    e->fp = fp;

    void *dst = NULL;
    if ((*rc = qh_malloc(&dst, bytes))) goto drop;
    if (layout == 0) {
        if ((*rc = qh_h2d(dst, b, bytes))) goto drop_dst;
    } else {
        const void *src_d;
        void *tmp = NULL;
        if (m) {
            src_d = m->dev + ((const unsigned char *)b - m->host);
        } else {
            if ((*rc = qh_malloc(&tmp, bytes))) goto drop_dst;
            if ((*rc = qh_h2d(tmp, b, bytes))) { (void)qh_free(tmp); goto drop_dst; }
            src_d = tmp;
        }
        *rc = qh_tile_to_row((uint16_t *)dst, (const uint16_t *)src_d, N, K, tn, tk);
        if (!*rc) *rc = qh_sync();
        if (tmp) (void)qh_free(tmp);
        if (*rc) goto drop_dst;
    }
    e->dev = dst;
    return (const uint16_t *)dst;

drop_dst:
    (void)qh_free(dst);
drop:
    /* remove the entry so a later call retries cleanly */
    *e = g_wc[g_nwc - 1];
    g_nwc--;
    return NULL;
}

/* ---- staging ------------------------------------------------------------------------ */
static int grow_host(void **p, size_t *cap, size_t need) {
    if (need <= *cap) return 0;
    size_t n = *cap ? *cap : (1u << 20);
    while (n < need) n *= 2;
    (void)qh_sync();
    (void)qh_host_free(*p);
    *p = NULL;
    *cap = 0;
    int rc = qh_host_alloc(p, n);
    if (rc) return rc;
    *cap = n;
    return 0;
}

static int grow(void **p, size_t *cap, size_t need) {
    if (need <= *cap) return 0;
    size_t n = *cap ? *cap : (1u << 20);
    while (n < need) n *= 2;
    (void)qh_sync();
    (void)qh_free(*p);
    *p = NULL;
    *cap = 0;
    int rc = qh_malloc(p, n);
    if (rc) return rc;
    *cap = n;
    return 0;
}

/* ---- the host-pointer GEMM path ------------------------------------------------------ */
/* the longest activation row that travels in a GEMV's kernel arguments */
#define KA_MAX_K 3072
/* bf16 of an fp32 value, round to nearest even -- the device's conversion
 * (v_cvt_pk_bf16_f32) for every non-NaN input, which is the reference's
 * recipe (fpga_bringup/src/src/qwen3.h:31-37); a NaN stays a (quiet) NaN */
/* the row of an M = 1 call, K values (branch-free, so the loop vectorises) */
__attribute__((optimize("tree-vectorize")))
static void bf16_rne_row(uint16_t *dst, const float *src, int K) {
    for (int k = 0; k < K; k++) {
        uint32_t u;
        memcpy(&u, &src[k], sizeof u);
        const uint32_t nan = (u & 0x7fffffffu) > 0x7f800000u;
        const uint32_t rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
        dst[k] = (uint16_t)(nan ? ((u >> 16) | 0x0040u) : rne);
    }
}

/* Completion of an M = 1 GEMV seen in its output: C is written into pinned
 * host memory exactly once per element, so the host fills it with a
 * signalling NaN that arithmetic never produces and waits until no element
 * holds it -- the values arrive over PCIe about 2 us before the runtime's
 * stream synchronisation would return.  After WAIT_US without all values the
 * stream is synchronised (which reports a failed launch). */
#define C_SENTINEL 0x7fa5a5a5u
#define POLL_MAX_ELEMS 65536u
#define WAIT_US 2000.0
static double now_us(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec * 1e6 + (double)t.tv_nsec * 1e-3;
}
static void arm_output(void *c, size_t n) {
    uint32_t *w = (uint32_t *)c;
    for (size_t i = 0; i < n; i++) w[i] = C_SENTINEL;
}
static int wait_output(const void *c, size_t n) {
    const volatile uint32_t *w = (const volatile uint32_t *)c;
    size_t i = 0;
    const double t0 = now_us();
    while (i < n) {
        if (w[i] != C_SENTINEL) { i++; continue; }
        if (now_us() - t0 > WAIT_US) {
            const int rc = qh_sync();
            if (rc) return rc;
            for (; i < n; i++)
                if (w[i] == C_SENTINEL) return QWEN3_HIP_ERUNTIME;
            return 0;
        }
    }
    return 0;
}

static int gemm_host(float *c, const float *a, const uint16_t *b, const uint16_t *b2,
                     int M, int K, int N, int layout, int gated) {
    if (M < 0 || K < 0 || N < 0) return QWEN3_HIP_EINVAL;
    if (M == 0 || N == 0) return 0;
    if (!c || (K > 0 && (!a || !b || (gated && !b2)))) return QWEN3_HIP_EINVAL;
    int rc = ensure_ready();
    if (rc) return rc;
    if (K == 0) {                       /* empty sums: 0, and silu(0) * 0 = 0 */
        memset(c, 0, (size_t)M * (size_t)N * sizeof(float));
        return 0;
    }
    const uint16_t *bd = weight_dev(b, N, K, layout, 0, &rc);
    if (!bd) return rc;
    const uint16_t *bd2 = NULL;
    if (gated && !(bd2 = weight_dev(b2, N, K, layout, 1, &rc))) return rc;

    /* The GEMM writes C straight into pinned staging, which the host copies
     * out once the values are there.  A reaches the GEMM one of two ways:
     *  - M = 1, K <= 3072 (every GEMV of a decode step): the host rounds
     *    the row to bf16 and it travels in the GEMV launch's kernel
     *    arguments (up to 6 KB) -- one launch per call;
     *  - otherwise host -> pinned staging (memcpy) -> device by the
     *    library's copy kernel, on the same stream as the GEMM (a runtime
     *    copy from host memory adds a cross-engine wait to every call).
     * An M = 1 GEMV with at most POLL_MAX_ELEMS outputs is waited for by
     * watching C (wait_output), everything else by a stream synchronisation.
     * Per M = 1 call, measured: 26 us with runtime copies both ways, 17 us
     * with the copy kernel and a synchronisation. */
    const size_t abytes = (size_t)M * (size_t)K * sizeof(float);
    const size_t cbytes = (size_t)M * (size_t)N * sizeof(float);
    if ((rc = grow_host(&g_c_h, &g_c_hcap, cbytes))) return rc;
    const int poll = M == 1 && (size_t)N <= POLL_MAX_ELEMS;
    if (poll) arm_output(g_c_h, (size_t)N);
    if (M == 1 && K <= KA_MAX_K && K % 8 == 0 && ((uintptr_t)bd & 15) == 0 &&
        (!gated || ((uintptr_t)bd2 & 15) == 0) && (size_t)N * (size_t)K * 2 < ((size_t)1 << 31) &&
        strcmp(qh_gemm_plan(M, K, N, gated), "gemv") == 0) {
        uint16_t row[KA_MAX_K];                           /* what qh_gemv_ka reads: zero past K */
        bf16_rne_row(row, a, K);
        memset(row + K, 0, (size_t)(KA_MAX_K - K) * sizeof(uint16_t));
        rc = qh_gemv_ka((float *)g_c_h, row, bd, gated ? bd2 : NULL, K, N);
    } else {
        const size_t a16 = (abytes + 15) & ~(size_t)15;     /* the copy kernel moves 16-byte units */
        if ((rc = grow(&g_a_d, &g_a_cap, a16))) return rc;
        if ((rc = grow_host(&g_a_h, &g_a_hcap, a16))) return rc;
        memcpy(g_a_h, a, abytes);
        if ((rc = qh_copy(g_a_d, g_a_h, a16))) return rc;
        rc = gated ? qh_gemm_gate_up_silu((float *)g_c_h, (const float *)g_a_d, bd, bd2, M, K, N)
                   : qh_gemm((float *)g_c_h, (const float *)g_a_d, bd, M, K, N);
    }
    if (rc) return rc;
    /* only the GEMV plans write each element of C exactly once */
    if (poll && strcmp(qh_last_plan(), "gemv") == 0) rc = wait_output(g_c_h, (size_t)N);
    else rc = qh_sync();
    if (rc) return rc;
    memcpy(c, g_c_h, cbytes);
    return 0;
}

void qwen3_gemm(float *c, const float *a, const uint16_t *b, int M, int K, int N) {
    int rc = gemm_host(c, a, b, NULL, M, K, N, g_layout, 0);
    if (rc) fail(rc, "qwen3_gemm");
}

void qwen3_gemm_row(float *c, const float *a, const uint16_t *b, int M, int K, int N) {
    int rc = gemm_host(c, a, b, NULL, M, K, N, 0, 0);
    if (rc) fail(rc, "qwen3_gemm_row");
}

void qwen3_gemm_gate_up_silu(float *h, const float *x, const uint16_t *wg,
                             const uint16_t *wu, int M, int K, int N) {
    int rc = gemm_host(h, x, wg, wu, M, K, N, g_layout, 1);
    if (rc) fail(rc, "qwen3_gemm_gate_up_silu");
}

/* ---- device-pointer API ------------------------------------------------------------ */
#define READY_OR_RETURN()                    \
    do {                                     \
        int _rc = ensure_ready();            \
        if (_rc) return _rc;                 \
    } while (0)

int qwen3_hip_gemm_dev(float *c, const float *a, const uint16_t *b, int M, int K, int N) {
    READY_OR_RETURN();
    return note(qh_gemm(c, a, b, M, K, N));
}

int qwen3_hip_gemm_noalloc_dev(float *c, const float *a, const uint16_t *b, int M, int K, int N) {
    if (!g_ready) return note(QWEN3_HIP_ESTATE);     /* set-up may allocate: not here */
    return note(qh_gemm_noalloc(c, a, b, M, K, N));
}

size_t qwen3_hip_scratch_bytes(void) { return qh_scratch_bytes(); }

int qwen3_hip_gemm_gate_up_silu_dev(float *h, const float *x, const uint16_t *wg,
                                    const uint16_t *wu, int M, int K, int N) {
    READY_OR_RETURN();
    return note(qh_gemm_gate_up_silu(h, x, wg, wu, M, K, N));
}

int qwen3_hip_gemm_bf16a_dev(float *c, const uint16_t *a, const uint16_t *b, int M, int K, int N) {
    READY_OR_RETURN();
    return note(qh_gemm_bf16a(c, a, b, M, K, N));
}

int qwen3_hip_gemm_gate_up_silu_bf16a_dev(float *h, const uint16_t *x, const uint16_t *wg,
                                          const uint16_t *wu, int M, int K, int N) {
    READY_OR_RETURN();
    return note(qh_gemm_gate_up_silu_bf16a(h, x, wg, wu, M, K, N));
}

int qwen3_hip_decode_set_dev(const uint16_t *const *w, const float *x0, float *out, int layers) {
    READY_OR_RETURN();
    return note(qh_decode_persist(w, x0, out, layers));
}

int qwen3_hip_decode_set_supported(void) { return ensure_ready() == 0 && qh_persist_supported(); }
int qwen3_hip_decode_set_out_ld(void) { return qh_persist_out_ld(); }

int qwen3_hip_decode_set_errors(unsigned *flags) {
    READY_OR_RETURN();
    return note(qh_persist_errors(flags));
}

int qwen3_hip_argmax_dev(int *out, const float *v, int n) {
    READY_OR_RETURN();
    return note(qh_argmax(out, v, n));
}

int qwen3_hip_tile_to_row_dev(uint16_t *dst, const uint16_t *src, int N, int K, int tn, int tk) {
    READY_OR_RETURN();
    return note(qh_tile_to_row(dst, src, N, K, tn, tk));
}

int qwen3_hip_copy_dev(void *dst, const void *src, size_t bytes) {
    READY_OR_RETURN();
    return note(qh_copy(dst, src, bytes));
}

int qwen3_hip_read_dev(const void *src, size_t bytes) {
    READY_OR_RETURN();
    return note(qh_read(src, bytes));
}

int qwen3_hip_capture_begin(void) { READY_OR_RETURN(); return note(qh_capture_begin()); }
int qwen3_hip_capture_end(int *graph_id) { READY_OR_RETURN(); return note(qh_capture_end(graph_id)); }
int qwen3_hip_graph_launch(int graph_id) { READY_OR_RETURN(); return note(qh_graph_launch(graph_id)); }
int qwen3_hip_graph_destroy(int graph_id) { READY_OR_RETURN(); return note(qh_graph_destroy(graph_id)); }

int qwen3_hip_malloc(void **p, size_t bytes) { READY_OR_RETURN(); return note(qh_malloc(p, bytes)); }
int qwen3_hip_free(void *p) { READY_OR_RETURN(); return note(qh_free(p)); }
int qwen3_hip_memcpy_h2d(void *d, const void *s, size_t n) { READY_OR_RETURN(); return note(qh_h2d(d, s, n)); }
int qwen3_hip_memcpy_d2h(void *d, const void *s, size_t n) { READY_OR_RETURN(); return note(qh_d2h(d, s, n)); }
int qwen3_hip_sync(void) { READY_OR_RETURN(); return note(qh_sync()); }
int qwen3_hip_timer_record(int slot) { READY_OR_RETURN(); return note(qh_timer_record(slot)); }
int qwen3_hip_timer_elapsed_ms(int a, int b, float *ms) {
    READY_OR_RETURN();
    return note(qh_timer_elapsed_ms(a, b, ms));
}
const char *qwen3_hip_plan(int M, int K, int N, int gated) { return qh_gemm_plan(M, K, N, gated); }
const char *qwen3_hip_last_plan(void) { return qh_last_plan(); }
int qwen3_hip_force_plan(int plan_id) { return note(qh_force_plan(plan_id)); }
