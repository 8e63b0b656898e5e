// CDNA4 (gfx950) kernels of the device-resident Qwen3-0.6B forward besides
// the projection GEMMs: row-wise residual + RMSNorm (with the embedding
// gather folded in) and the fused attention step.  The arithmetic follows the
// reference's scalar ops (fpga_bringup/src/src/ops_scalar.c) and forward
// (fpga_bringup/src/src/qwen3.c:276-576); sums are reduced in parallel, so
// results agree to rounding, not bit for bit.
//
// Device layouts (all fp32 unless noted):
//   activations   [nt][dim] row-major (the GEMM A/C layout)
//   qkv           [nt][4096] = q (16 heads x 128) | k (8 x 128) | v (8 x 128)
//   K cache       [layer][kv_head][128/4][max_seq][4]   (d-chunk major: one
//                 thread per position reads 16 contiguous bytes per chunk, so
//                 a wave's score loads are one 1 KB contiguous run)
//   V cache       [layer][kv_head][max_seq][128]        (as qwen3.h:62-76)
//   rope tables   [max_seq][64] cos and sin, built on the host with the
//                 reference formula (ops_scalar.c:21-35)
// The attention kernels keep 2 x max_seq scores in LDS (up to 69 KB at
// QM_MAX_SEQ), above the default 64 KB limit that they raise once.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hip_shim.h"
#include "model_shim.h"

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

#define WAVE 64
#define NTH 256
#define HD 128                 // head_dim
#define NKV 8                  // kv heads
#define GRP 2                  // q heads per kv head (qwen3_config.h:22)
#define QKV_LD 4096            // q 2048 | k 1024 | v 1024
#define KOFF 2048
#define VOFF 3072

__device__ __forceinline__ float bf16f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
    return v;
}

// ---------------------------------------------------------------------------
// rows: x[row] = emb[tok[row]] (bf16 -> fp32)   when emb is set, else
//       x[row] = x[row] + r[row]                 when r is set;
//       xb[row] = rmsnorm(x[row]) * nw           (ops_scalar.c:11-16)
// grid = nt blocks of 256 threads; K % 4 == 0, K <= 4096.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(NTH) void k_rows_norm(float *__restrict__ x, const float *__restrict__ r,
                                                   const uint16_t *__restrict__ emb,
                                                   const int *__restrict__ tok, int emb_rows,
                                                   const uint16_t *__restrict__ nw,
                                                   float *__restrict__ xb, int K, float eps) {
    const int row = blockIdx.x, tid = threadIdx.x;
    const int n4 = K >> 2;
    f32x4 v[4];
    float ss = 0.0f;
    int t = 0;
    if (emb) {
        t = tok[row];
        t = t < 0 ? 0 : (t >= emb_rows ? emb_rows - 1 : t);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int c = tid + NTH * j;
        v[j] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (c < n4) {
            if (emb) {
                const uint16_t *e = emb + (size_t)t * K + c * 4;
                v[j] = f32x4{bf16f(e[0]), bf16f(e[1]), bf16f(e[2]), bf16f(e[3])};
            } else {
                v[j] = reinterpret_cast<const f32x4 *>(x + (size_t)row * K)[c];
                if (r) v[j] += reinterpret_cast<const f32x4 *>(r + (size_t)row * K)[c];
            }
            if (emb || r) reinterpret_cast<f32x4 *>(x + (size_t)row * K)[c] = v[j];
            ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
        }
    }
    __shared__ float red[NTH / WAVE];
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    ss = red[0] + red[1] + red[2] + red[3];
    const float scale = 1.0f / sqrtf(ss / (float)K + eps);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int c = tid + NTH * j;
        if (c < n4) {
            const uint16_t *w = nw + c * 4;
            f32x4 o;
            o.x = (v[j].x * scale) * bf16f(w[0]);
            o.y = (v[j].y * scale) * bf16f(w[1]);
            o.z = (v[j].z * scale) * bf16f(w[2]);
            o.w = (v[j].w * scale) * bf16f(w[3]);
            reinterpret_cast<f32x4 *>(xb + (size_t)row * K)[c] = o;
        }
    }
}

// ---------------------------------------------------------------------------
// Chunk of nt tokens at positions pos0 .. pos0+nt-1 (pos0 = *pos_d), step 1:
// QK-norm (qwen3.c:298-305) then RoPE (ops_scalar.c:21-35) of every q and k
// head; q is written back in place, k and v go to the KV cache entry of
// their position (qwen3.c:497-512).  grid = (nt, 6): block (i, b), wave w
// handles row 4b + w of token i (rows 0-15 q heads, 16-23 k heads + v copy).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(NTH) void k_qk_rope_cache(float *__restrict__ qkv, float *__restrict__ kc,
                                                       float *__restrict__ vc,
                                                       const uint16_t *__restrict__ qn,
                                                       const uint16_t *__restrict__ kn,
                                                       const float *__restrict__ rcos,
                                                       const float *__restrict__ rsin,
                                                       const int *__restrict__ pos_d, int max_seq,
                                                       float eps) {
    const int i = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rr = blockIdx.y * 4 + wave;      // 0 .. 23
    const int pos = *pos_d + i;
    if (*pos_d < 0 || pos >= max_seq) return;
    float *row = qkv + (size_t)i * QKV_LD;
    const bool isq = rr < NKV * GRP;
    const int hd = isq ? rr : rr - NKV * GRP;
    float *src = isq ? row + (size_t)hd * HD : row + KOFF + (size_t)hd * HD;
    const uint16_t *w = isq ? qn : kn;
    const float x0 = src[lane], x1 = src[lane + 64];
    const float w0 = bf16f(w[lane]), w1 = bf16f(w[lane + 64]);
    const float c = rcos[(size_t)pos * (HD / 2) + lane], sn = rsin[(size_t)pos * (HD / 2) + lane];
    const float ss = wave_sum(x0 * x0 + x1 * x1);
    const float sc = 1.0f / sqrtf(ss / (float)HD + eps);
    const float y0 = (x0 * sc) * w0, y1 = (x1 * sc) * w1;
    const float o0 = __fsub_rn(__fmul_rn(y0, c), __fmul_rn(y1, sn));
    const float o1 = __fadd_rn(__fmul_rn(y1, c), __fmul_rn(y0, sn));
    if (isq) {
        src[lane] = o0;
        src[lane + 64] = o1;
    } else {
        float *kb = kc + (size_t)hd * (HD / 4) * max_seq * 4;
        kb[((size_t)(lane >> 2) * max_seq + pos) * 4 + (lane & 3)] = o0;
        kb[((size_t)((lane + 64) >> 2) * max_seq + pos) * 4 + (lane & 3)] = o1;
        float *vb = vc + ((size_t)hd * max_seq + pos) * HD;
        const float *vs = row + VOFF + (size_t)hd * HD;
        vb[lane] = vs[lane];
        vb[lane + 64] = vs[lane + 64];
    }
}

// ---------------------------------------------------------------------------
// Chunk step 2: causal GQA attention (qwen3.c:377-436) for token i of the
// chunk and kv head g (block (i, g), its GRP query heads), with roped q in
// qkv and every key/value t <= pos0 + i in the cache (written by step 1).
//   scores s[h][t] = q_h . k_t / sqrt(128); softmax over t (ops_scalar.c:
//   37-44), normalised as there; out_h = sum_t p[h][t] v_t.
// grid = (nt, NKV), 256 threads, dynamic LDS = qm_attention_lds_bytes().
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(NTH) void k_attention(const float *__restrict__ qkv,
                                                   float *__restrict__ out,
                                                   const float *__restrict__ kc,
                                                   const float *__restrict__ vc,
                                                   const int *__restrict__ pos_d, int max_seq,
                                                   float scale) {
    const int i = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int pos0 = *pos_d;
    const int pos = pos0 + i;
    if (pos0 < 0 || pos >= max_seq) return;   // uniform per block, before any barrier
    const int ctx = pos + 1;

    extern __shared__ float sm[];
    float *sq = sm;                            // [GRP][HD]
    float *red = sq + GRP * HD;                // [4][GRP][HD] partial outputs
    float *sred = red + 4 * GRP * HD;          // [2][4] block reductions
    float *p = sred + 8;                       // [GRP][max_seq]

    sq[tid] = qkv[(size_t)i * QKV_LD + (size_t)g * GRP * HD + tid];   // 256 threads = GRP x HD
    __syncthreads();

    // scores
    const f32x4 *kbase = reinterpret_cast<const f32x4 *>(kc) + (size_t)g * (HD / 4) * max_seq;
    for (int t = tid; t < ctx; t += NTH) {
        f32x4 kv[HD / 4];
#pragma unroll
        for (int d4 = 0; d4 < HD / 4; d4++) kv[d4] = kbase[(size_t)d4 * max_seq + t];
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int d4 = 0; d4 < HD / 4; d4++) {
            const f32x4 q0 = reinterpret_cast<const f32x4 *>(sq)[d4];
            const f32x4 q1 = reinterpret_cast<const f32x4 *>(sq + HD)[d4];
            s0 = fmaf(q0.x, kv[d4].x, s0); s0 = fmaf(q0.y, kv[d4].y, s0);
            s0 = fmaf(q0.z, kv[d4].z, s0); s0 = fmaf(q0.w, kv[d4].w, s0);
            s1 = fmaf(q1.x, kv[d4].x, s1); s1 = fmaf(q1.y, kv[d4].y, s1);
            s1 = fmaf(q1.z, kv[d4].z, s1); s1 = fmaf(q1.w, kv[d4].w, s1);
        }
        p[t] = s0 * scale;
        p[max_seq + t] = s1 * scale;
    }
    __syncthreads();

    // softmax per query head
    float m0 = -INFINITY, m1 = -INFINITY;
    for (int t = tid; t < ctx; t += NTH) {
        m0 = fmaxf(m0, p[t]);
        m1 = fmaxf(m1, p[max_seq + t]);
    }
    m0 = wave_max(m0);
    m1 = wave_max(m1);
    if (lane == 0) { sred[wave] = m0; sred[4 + wave] = m1; }
    __syncthreads();
    m0 = fmaxf(fmaxf(sred[0], sred[1]), fmaxf(sred[2], sred[3]));
    m1 = fmaxf(fmaxf(sred[4], sred[5]), fmaxf(sred[6], sred[7]));
    __syncthreads();
    float e0 = 0.0f, e1 = 0.0f;
    for (int t = tid; t < ctx; t += NTH) {
        const float a0 = expf(p[t] - m0), a1 = expf(p[max_seq + t] - m1);
        p[t] = a0;
        p[max_seq + t] = a1;
        e0 += a0;
        e1 += a1;
    }
    e0 = wave_sum(e0);
    e1 = wave_sum(e1);
    if (lane == 0) { sred[wave] = e0; sred[4 + wave] = e1; }
    __syncthreads();
    e0 = (sred[0] + sred[1]) + (sred[2] + sred[3]);
    e1 = (sred[4] + sred[5]) + (sred[6] + sred[7]);
    for (int t = tid; t < ctx; t += NTH) {
        p[t] = p[t] / e0;
        p[max_seq + t] = p[max_seq + t] / e1;
    }
    __syncthreads();

    // out_h[d] = sum_t p[h][t] v_t[d]: wave w takes t = w, w+4, ...; lane l
    // owns d = 2l, 2l+1 of both heads
    f32x2 o0 = {0.f, 0.f}, o1 = {0.f, 0.f};
    const f32x2 *vcache = reinterpret_cast<const f32x2 *>(vc + (size_t)g * max_seq * HD) + lane;
    int t = wave;
    for (; t + 4 * 7 < ctx; t += 4 * 8) {      // 8 loads in flight per lane
        f32x2 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = vcache[(size_t)(t + 4 * u) * (HD / 2)];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float p0 = p[t + 4 * u], p1 = p[max_seq + t + 4 * u];
            o0.x = __fadd_rn(o0.x, __fmul_rn(p0, v[u].x));
            o0.y = __fadd_rn(o0.y, __fmul_rn(p0, v[u].y));
            o1.x = __fadd_rn(o1.x, __fmul_rn(p1, v[u].x));
            o1.y = __fadd_rn(o1.y, __fmul_rn(p1, v[u].y));
        }
    }
    for (; t < ctx; t += 4) {
        const f32x2 v = vcache[(size_t)t * (HD / 2)];
        const float p0 = p[t], p1 = p[max_seq + t];
        o0.x = __fadd_rn(o0.x, __fmul_rn(p0, v.x));
        o0.y = __fadd_rn(o0.y, __fmul_rn(p0, v.y));
        o1.x = __fadd_rn(o1.x, __fmul_rn(p1, v.x));
        o1.y = __fadd_rn(o1.y, __fmul_rn(p1, v.y));
    }
    red[(wave * GRP + 0) * HD + 2 * lane] = o0.x;
    red[(wave * GRP + 0) * HD + 2 * lane + 1] = o0.y;
    red[(wave * GRP + 1) * HD + 2 * lane] = o1.x;
    red[(wave * GRP + 1) * HD + 2 * lane + 1] = o1.y;
    __syncthreads();
    {
        const int h = tid >> 7, d = tid & (HD - 1);   // 256 threads = GRP x HD
        const float sacc = (red[(0 * GRP + h) * HD + d] + red[(1 * GRP + h) * HD + d]) +
                           (red[(2 * GRP + h) * HD + d] + red[(3 * GRP + h) * HD + d]);
        out[(size_t)i * (NKV * GRP * HD) + (size_t)(g * GRP + h) * HD + d] = sacc;
    }
}

// ---------------------------------------------------------------------------
// Decode attention: one token at position pos = *pos_d.  Block b = g + 8*q
// handles kv head g (its GRP query heads) and quarter q of the head
// dimension: it computes the full scores of both query heads (K is read
// once for the pair), the softmax, and out[h][32q .. 32q+32) from a quarter
// of every V row, so no block needs another's result.  The 4 blocks of a kv
// head share XCD g (block b runs on XCD b % 8) and so its L2 for the K rows.
// Built for latency: every thread issues its K loads (32 x 16 B of one
// position, a contiguous 1 KB run per wave in the d-chunk-major cache) and
// its V loads at entry, before QK-norm and RoPE start.  Positions are taken
// 256 at a time; scores live in LDS.  Block (g, 0) writes the new token's
// cache entry.  grid = 4 * NKV blocks of 256 threads; dynamic LDS =
// qm_attention_decode_lds_bytes(max_seq).
// ---------------------------------------------------------------------------
#define DQ 4                      // head-dimension quarters
#define DQW (HD / DQ)             // 32 dims per block

__global__ __launch_bounds__(NTH) void k_attn_decode(const float *__restrict__ qkv,
                                                     float *__restrict__ out,
                                                     float *__restrict__ kc, float *__restrict__ vc,
                                                     const uint16_t *__restrict__ qn,
                                                     const uint16_t *__restrict__ kn,
                                                     const float *__restrict__ rcos,
                                                     const float *__restrict__ rsin,
                                                     const int *__restrict__ pos_d, int max_seq,
                                                     float eps, float scale) {
    const int g = blockIdx.x % NKV, q = blockIdx.x / NKV;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int pos = *pos_d;
    if (pos < 0 || pos >= max_seq) return;      // uniform per launch
    const int ctx = pos + 1;

    extern __shared__ float sm[];
    float *sq = sm;                              // [GRP][HD]
    float *sk = sq + GRP * HD;                   // [HD] k of the new token
    float *red = sk + HD;                        // [32 groups][GRP][DQW]
    float *sred = red + 32 * GRP * DQW;          // [16]
    float *p = sred + 16;                        // [GRP][max_seq]

    const f32x4 *kbase = reinterpret_cast<const f32x4 *>(kc) + (size_t)g * (HD / 4) * max_seq;
    // V: thread (tg = tid / 8, c = tid % 8) owns dims 32q + 4c .. +4 of positions tg, tg + 32, ...
    const int tg = tid >> 3, c4 = tid & 7;
    const f32x4 *vbase = reinterpret_cast<const f32x4 *>(vc + (size_t)g * max_seq * HD + q * DQW) + c4;
    const f32x4 vnew = reinterpret_cast<const f32x4 *>(qkv + VOFF + (size_t)g * HD + q * DQW)[c4];
    constexpr int VB = NTH / 32;                 // positions per thread and pass of 256

    // loads of the first pass go out before anything else
    f32x4 kv[HD / 4];
    if (tid < pos) {
#pragma unroll
        for (int d4 = 0; d4 < HD / 4; d4++) kv[d4] = kbase[(size_t)d4 * max_seq + tid];
    }
    f32x4 vv[VB];
#pragma unroll
    for (int u = 0; u < VB; u++) {
        const int t = tg + 32 * u;
        vv[u] = t < pos ? vbase[(size_t)t * (HD / 4)] : vnew;
    }

    // QK-norm + RoPE: waves 0/1 the two query heads, wave 2 the new k
    if (wave < GRP + 1) {
        const float *src = wave < GRP ? qkv + (size_t)(g * GRP + wave) * HD : qkv + KOFF + (size_t)g * HD;
        const uint16_t *w = wave < GRP ? qn : kn;
        float *dst = wave < GRP ? sq + wave * HD : sk;
        const float x0 = src[lane], x1 = src[lane + 64];
        const float w0 = bf16f(w[lane]), w1 = bf16f(w[lane + 64]);
        const float c = rcos[(size_t)pos * (HD / 2) + lane], sn = rsin[(size_t)pos * (HD / 2) + lane];
        const float ss = wave_sum(x0 * x0 + x1 * x1);
        const float sc = 1.0f / sqrtf(ss / (float)HD + eps);
        const float y0 = (x0 * sc) * w0, y1 = (x1 * sc) * w1;
        dst[lane] = __fsub_rn(__fmul_rn(y0, c), __fmul_rn(y1, sn));
        dst[lane + 64] = __fadd_rn(__fmul_rn(y1, c), __fmul_rn(y0, sn));
    }
    __syncthreads();
    if (q == 0 && tid < HD) {                    // one block per kv head writes the new entry
        kc[(((size_t)g * (HD / 4) + (tid >> 2)) * max_seq + pos) * 4 + (tid & 3)] = sk[tid];
        vc[((size_t)g * max_seq + pos) * HD + tid] = qkv[VOFF + (size_t)g * HD + tid];
    }

    // scores of both query heads: the first 256 positions from the registers
    // loaded at entry, later ones (ctx > 256) in further passes
    auto dot2 = [&](const f32x4 *k, float &s0, float &s1) {
#pragma unroll
        for (int d4 = 0; d4 < HD / 4; d4++) {
            const f32x4 q0 = reinterpret_cast<const f32x4 *>(sq)[d4];
            const f32x4 q1 = reinterpret_cast<const f32x4 *>(sq + HD)[d4];
            s0 = fmaf(q0.x, k[d4].x, s0); s0 = fmaf(q0.y, k[d4].y, s0);
            s0 = fmaf(q0.z, k[d4].z, s0); s0 = fmaf(q0.w, k[d4].w, s0);
            s1 = fmaf(q1.x, k[d4].x, s1); s1 = fmaf(q1.y, k[d4].y, s1);
            s1 = fmaf(q1.z, k[d4].z, s1); s1 = fmaf(q1.w, k[d4].w, s1);
        }
    };
    if (tid < ctx) {
        float s0 = 0.0f, s1 = 0.0f;
        if (tid < pos) dot2(kv, s0, s1);
        else dot2(reinterpret_cast<const f32x4 *>(sk), s0, s1);   // the new token
        p[tid] = s0 * scale;
        p[max_seq + tid] = s1 * scale;
    }
    for (int t = NTH + tid; t < ctx; t += NTH) {
        float s0 = 0.0f, s1 = 0.0f;
        if (t < pos) {
            f32x4 k2[HD / 4];
#pragma unroll
            for (int d4 = 0; d4 < HD / 4; d4++) k2[d4] = kbase[(size_t)d4 * max_seq + t];
            dot2(k2, s0, s1);
        } else {
            dot2(reinterpret_cast<const f32x4 *>(sk), s0, s1);
        }
        p[t] = s0 * scale;
        p[max_seq + t] = s1 * scale;
    }
    __syncthreads();

    // softmax of both heads (ops_scalar.c:37-44)
    float m0 = -INFINITY, m1 = -INFINITY;
    for (int t = tid; t < ctx; t += NTH) {
        m0 = fmaxf(m0, p[t]);
        m1 = fmaxf(m1, p[max_seq + t]);
    }
    m0 = wave_max(m0);
    m1 = wave_max(m1);
    if (lane == 0) { sred[wave] = m0; sred[4 + wave] = m1; }
    __syncthreads();
    m0 = fmaxf(fmaxf(sred[0], sred[1]), fmaxf(sred[2], sred[3]));
    m1 = fmaxf(fmaxf(sred[4], sred[5]), fmaxf(sred[6], sred[7]));
    float e0 = 0.0f, e1 = 0.0f;
    for (int t = tid; t < ctx; t += NTH) {
        const float a0 = expf(p[t] - m0), a1 = expf(p[max_seq + t] - m1);
        p[t] = a0;
        p[max_seq + t] = a1;
        e0 += a0;
        e1 += a1;
    }
    e0 = wave_sum(e0);
    e1 = wave_sum(e1);
    if (lane == 0) { sred[8 + wave] = e0; sred[12 + wave] = e1; }
    __syncthreads();
    const float inv0 = 1.0f / ((sred[8] + sred[9]) + (sred[10] + sred[11]));
    const float inv1 = 1.0f / ((sred[12] + sred[13]) + (sred[14] + sred[15]));

    // out[h][32q + d] = sum_t p[h][t] v_t[32q + d] / e_h
    f32x4 o0 = {0.f, 0.f, 0.f, 0.f}, o1 = {0.f, 0.f, 0.f, 0.f};
    for (int base = 0; base < ctx; base += NTH) {
        if (base > 0) {
#pragma unroll
            for (int u = 0; u < VB; u++) {
                const int t = base + tg + 32 * u;
                vv[u] = t < pos ? vbase[(size_t)t * (HD / 4)] : vnew;
            }
        }
#pragma unroll
        for (int u = 0; u < VB; u++) {
            const int t = base + tg + 32 * u;
            if (t < ctx) {
                const float w0 = p[t], w1 = p[max_seq + t];
                o0.x = fmaf(w0, vv[u].x, o0.x); o0.y = fmaf(w0, vv[u].y, o0.y);
                o0.z = fmaf(w0, vv[u].z, o0.z); o0.w = fmaf(w0, vv[u].w, o0.w);
                o1.x = fmaf(w1, vv[u].x, o1.x); o1.y = fmaf(w1, vv[u].y, o1.y);
                o1.z = fmaf(w1, vv[u].z, o1.z); o1.w = fmaf(w1, vv[u].w, o1.w);
            }
        }
    }
    reinterpret_cast<f32x4 *>(red + (tg * GRP + 0) * DQW)[c4] = o0;
    reinterpret_cast<f32x4 *>(red + (tg * GRP + 1) * DQW)[c4] = o1;
    __syncthreads();
    if (tid < GRP * DQW) {
        const int h = tid / DQW, d = tid % DQW;
        float sacc = 0.0f;
#pragma unroll 8
        for (int k = 0; k < 32; k++) sacc += red[(k * GRP + h) * DQW + d];
        out[(size_t)(g * GRP + h) * HD + q * DQW + d] = sacc * (h ? inv1 : inv0);
    }
}

__global__ void k_set_i32(int *p, int v) {
    if (threadIdx.x == 0 && blockIdx.x == 0) p[0] = v;
}

__global__ void k_zero_i32(int *p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
static inline hipStream_t stream() { return (hipStream_t)qh_stream(); }

extern "C" size_t qm_attention_lds_bytes(int max_seq) {
    return sizeof(float) * ((size_t)GRP * HD + 4 * GRP * HD + 8 + (size_t)GRP * max_seq);
}

extern "C" int qm_rows_norm(float *x, const float *r, const uint16_t *emb, const int *tok, int emb_rows,
                            const uint16_t *nw, float *xb, int nt, int K, float eps) {
    if (!stream()) return QH_ESTATE;
    if (!x || !nw || !xb || nt <= 0 || K <= 0 || K % 4 || K > 4 * 4 * NTH) return QH_EINVAL;
    if (emb && (!tok || emb_rows <= 0)) return QH_EINVAL;
    hipLaunchKernelGGL(k_rows_norm, dim3(nt), dim3(NTH), 0, stream(), x, emb ? nullptr : r, emb, tok,
                       emb_rows, nw, xb, K, eps);
    return hipGetLastError() == hipSuccess ? QH_OK : QH_ELAUNCH;
}

extern "C" int qm_attention(float *qkv, float *out, float *kc, float *vc, const uint16_t *qn,
                            const uint16_t *kn, const float *rcos, const float *rsin, const int *pos_d,
                            int nt, int max_seq, float eps) {
    if (!stream()) return QH_ESTATE;
    if (!qkv || !out || !kc || !vc || !qn || !kn || !rcos || !rsin || !pos_d) return QH_EINVAL;
    if (nt <= 0 || max_seq <= 0 || nt > QM_MAX_CHUNK || max_seq > QM_MAX_SEQ) return QH_EINVAL;
    const size_t lds = qm_attention_lds_bytes(max_seq);
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute((const void *)k_attention, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)qm_attention_lds_bytes(QM_MAX_SEQ)) != hipSuccess)
            return QH_ELAUNCH;
        attr_set = true;
    }
    // 1 / sqrt(head_dim), the constant of qwen3.c:311
    const float scale = 0.08838834764831845f;
    hipLaunchKernelGGL(k_qk_rope_cache, dim3(nt, (NKV * GRP + NKV) / 4), dim3(NTH), 0, stream(), qkv, kc, vc,
                       qn, kn, rcos, rsin, pos_d, max_seq, eps);
    if (hipGetLastError() != hipSuccess) return QH_ELAUNCH;
    hipLaunchKernelGGL(k_attention, dim3(nt, NKV), dim3(NTH), lds, stream(), qkv, out, kc, vc, pos_d, max_seq,
                       scale);
    return hipGetLastError() == hipSuccess ? QH_OK : QH_ELAUNCH;
}

extern "C" size_t qm_attention_decode_lds_bytes(int max_seq) {
    return sizeof(float) * ((size_t)GRP * HD + HD + 32 * GRP * DQW + 16 + (size_t)GRP * max_seq);
}

extern "C" int qm_attention_decode(const float *qkv, float *out, float *kc, float *vc, const uint16_t *qn,
                                   const uint16_t *kn, const float *rcos, const float *rsin,
                                   const int *pos_d, int max_seq, float eps) {
    if (!stream()) return QH_ESTATE;
    if (!qkv || !out || !kc || !vc || !qn || !kn || !rcos || !rsin || !pos_d) return QH_EINVAL;
    if (max_seq <= 0 || max_seq > QM_MAX_SEQ) return QH_EINVAL;
    const size_t lds = qm_attention_decode_lds_bytes(max_seq);
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute((const void *)k_attn_decode, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)qm_attention_decode_lds_bytes(QM_MAX_SEQ)) != hipSuccess)
            return QH_ELAUNCH;
        attr_set = true;
    }
    const float scale = 0.08838834764831845f;   // 1 / sqrt(head_dim), qwen3.c:311
    hipLaunchKernelGGL(k_attn_decode, dim3(DQ * NKV), dim3(NTH), lds, stream(), qkv, out, kc, vc, qn, kn,
                       rcos, rsin, pos_d, max_seq, eps, scale);
    return hipGetLastError() == hipSuccess ? QH_OK : QH_ELAUNCH;
}

extern "C" int qm_zero_i32(int *p, int n) {
    if (!stream()) return QH_ESTATE;
    if (!p || n < 0) return QH_EINVAL;
    if (n == 0) return QH_OK;
    hipLaunchKernelGGL(k_zero_i32, dim3((n + NTH - 1) / NTH < 1024 ? (n + NTH - 1) / NTH : 1024), dim3(NTH), 0,
                       stream(), p, n);
    return hipGetLastError() == hipSuccess ? QH_OK : QH_ELAUNCH;
}

extern "C" int qm_set_i32(int *p, int v) {
    if (!stream()) return QH_ESTATE;
    if (!p) return QH_EINVAL;
    hipLaunchKernelGGL(k_set_i32, dim3(1), dim3(WAVE), 0, stream(), p, v);
    return hipGetLastError() == hipSuccess ? QH_OK : QH_ELAUNCH;
}
