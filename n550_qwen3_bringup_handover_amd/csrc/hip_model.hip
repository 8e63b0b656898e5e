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
// The chunk attention keeps its tokens' scores in LDS, sized by the chunk's
// context: up to 69 KB at QM_MAX_SEQ with one token per block, above the
// default 64 KB limit, which it raises once.
#include <type_traits>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hip_shim.h"
#include "model_shim.h"
#include "fp_pinned.h"

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

// Cross-lane reductions without LDS round trips: DPP within rows of 16 lanes
// (quad permutes for xor 1 / xor 2, the half-row and row mirrors, or a
// rotation by 8), then the gfx950 permlane swaps across rows (xor 16, xor
// 32).  Each step combines a lane with its partner, so partners end with the
// same bits: the results are identical in every lane of the group.
template <int CTRL>
__device__ __forceinline__ float dpp_partner(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ f32x2 swap16(float x) {     // {lanes l and l ^ 16}, in lane order
    const auto p = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, x), __builtin_bit_cast(int, x), false, false);
    return f32x2{__builtin_bit_cast(float, (int)p[0]), __builtin_bit_cast(float, (int)p[1])};
}
__device__ __forceinline__ f32x2 swap32(float x) {     // {lanes l and l ^ 32}, in lane order
    const auto p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, x), __builtin_bit_cast(int, x), false, false);
    return f32x2{__builtin_bit_cast(float, (int)p[0]), __builtin_bit_cast(float, (int)p[1])};
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_partner<0xB1>(v);      // quad_perm [1,0,3,2]
    v += dpp_partner<0x4E>(v);      // quad_perm [2,3,0,1]
    v += dpp_partner<0x141>(v);     // row_half_mirror
    v += dpp_partner<0x140>(v);     // row_mirror
    f32x2 p = swap16(v);
    v = p.x + p.y;
    p = swap32(v);
    return p.x + p.y;
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_partner<0xB1>(v));
    v = fmaxf(v, dpp_partner<0x4E>(v));
    v = fmaxf(v, dpp_partner<0x141>(v));
    v = fmaxf(v, dpp_partner<0x140>(v));
    f32x2 p = swap16(v);
    v = fmaxf(p.x, p.y);
    p = swap32(v);
    return fmaxf(p.x, p.y);
}
// sum over lanes l, l ^ 8, l ^ 16, ..., l ^ 56 (the 8 lanes holding one value
// column): rotation by 8 within each row of 16, then the two permlane swaps
__device__ __forceinline__ float sum_stride8(float v) {
    v += dpp_partner<0x128>(v);     // row_ror:8
    f32x2 p = swap16(v);
    v = p.x + p.y;
    p = swap32(v);
    return p.x + p.y;
}

// raw buffer resource over [p, p + bytes); loads past num_records return
// zeros and read no memory
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *p, size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)(uint32_t)bytes, 0x00020000);
}
#define BUF_OOB 0x80000000u            // an offset past every buffer below 2 GiB

// ---------------------------------------------------------------------------
// rows: x[row] = emb[tok[row]] (bf16 -> fp32)   when emb is set, else
//       x[row] = x[row] + r[row]                 when r is set, else
//       x[row] = x[row] + sum_s part[s][row]     when ks > 0 (split-K slice
//                sums added in slice order: the reduction pass's sums);
//       xb[row] = rmsnorm(x[row]) * nw           (ops_scalar.c:11-16)
// grid = nt blocks of 256 threads; K % 4 == 0, K <= 4096, ks <= KS_MAX.
// ---------------------------------------------------------------------------
#define KS_MAX 16
__global__ __launch_bounds__(NTH) void k_rows_norm(float *__restrict__ x, const float *__restrict__ r,
                                                   const uint16_t *__restrict__ emb,
                                                   const int *__restrict__ tok, int emb_rows,
                                                   const uint16_t *__restrict__ nw,
                                                   float *__restrict__ xb, int K, float eps,
                                                   const float *__restrict__ part, int ks, size_t pstride) {
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
                if (ks > 0) {
                    // every slice's load first, then the sum in slice order
                    const __amdgpu_buffer_rsrc_t rp = buf_rsrc(part, pstride * (size_t)ks * 4);
                    f32x4 p[KS_MAX];
#pragma unroll
                    for (int s = 0; s < KS_MAX; s++)
                        p[s] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                   rp, s < ks ? (uint32_t)(((size_t)s * pstride + (size_t)row * K + 4 * c) * 4) : BUF_OOB,
                                   0, 0));
                    f32x4 sum = p[0];
#pragma unroll
                    for (int s = 1; s < KS_MAX; s++)
                        if (s < ks) sum += p[s];
                    v[j] += sum;
                }
            }
            if (emb || r || ks > 0) reinterpret_cast<f32x4 *>(x + (size_t)row * K)[c] = v[j];
            ss += sumsq4(v[j].x, v[j].y, v[j].z, v[j].w);
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
    const float ss = wave_sum(sumsq2(x0, x1));
    const float sc = 1.0f / sqrtf(ss / (float)HD + eps);
    const float y0 = (x0 * sc) * w0, y1 = (x1 * sc) * w1;
    float o0, o1;
    rope_pair(y0, y1, c, sn, o0, o1);
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
// Chunk step 2: causal GQA attention (qwen3.c:377-436) for QT consecutive
// tokens of the chunk and kv head g: block (b, g) takes tokens QT b ..
// QT b + QT - 1 (those below nt) with their GRP query heads, R = QT GRP rows
// (row r = token r / GRP, head r % GRP), roped q in qkv and every key/value
// t <= pos0 + i in the cache (written by step 1).
//   scores s[r][t] = q_r . k_t / sqrt(128); softmax over t (ops_scalar.c:
//   37-44), normalised as there; out_r = sum_t p[r][t] v_t.
// Every K and V row a block loads serves all R rows, so the cache traffic
// of a chunk falls by QT.  Positions past a row's own context score -inf
// and weigh 0: its max, sums and weighted V are those of a one-token block
// bit for bit (only exact zeros are added, after its own positions).
// grid = ceil(nt / QT) * NKV blocks, block b taking kv head b % NKV and tokens
// QT (b / NKV) ..: blocks run on XCD b mod 8, so each XCD serves one head's K
// and V from its own L2 (measured on MI355X against a (tokens, head) grid:
// 128-token prefill 1.65 -> 1.62 ms, 2,014 tokens 39.7 -> 39.1 ms); 256 threads,
// dynamic LDS =
// qm_attention_lds_bytes(QT, ldp); ldp >= pos0 + nt is the score row stride.
// ---------------------------------------------------------------------------
template <int QT>
__global__ __launch_bounds__(NTH) void k_attention(const float *__restrict__ qkv,
                                                   float *__restrict__ out,
                                                   const float *__restrict__ kc,
                                                   const float *__restrict__ vc,
                                                   const int *__restrict__ pos_d, int nt, int max_seq,
                                                   int ldp, float scale) {
    constexpr int R = QT * GRP;
    const int g = blockIdx.x % NKV, i0 = (int)(blockIdx.x / NKV) * QT, tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int pos0 = *pos_d;
    const int nq = min(QT, nt - i0);           // tokens of this block
    const int ctxmax = pos0 + i0 + nq;         // context of its last token
    // uniform per block, before any barrier
    if (pos0 < 0 || nq <= 0 || ctxmax > max_seq || ctxmax > ldp) return;

    extern __shared__ float sm[];
    float *sq = sm;                            // [R][HD]
    float *red = sq + R * HD;                  // [4][R][HD] partial outputs
    float *sred = red + 4 * R * HD;            // [R][4] block reductions
    float *p = sred + 4 * R;                   // [R][ldp]

    for (int e = tid; e < R * HD; e += NTH) {
        const int r = e / HD, ti = i0 + r / GRP;
        sq[e] = ti < nt ? qkv[(size_t)ti * QKV_LD + (size_t)(g * GRP + r % GRP) * HD + e % HD] : 0.0f;
    }
    __syncthreads();

    // scores: thread t loads key t once for all R rows
    const f32x4 *kbase = reinterpret_cast<const f32x4 *>(kc) + (size_t)g * (HD / 4) * max_seq;
    for (int t = tid; t < ctxmax; t += NTH) {
        f32x4 kv[HD / 4];
#pragma unroll
        for (int d4 = 0; d4 < HD / 4; d4++) kv[d4] = kbase[(size_t)d4 * max_seq + t];
#pragma unroll
        for (int r = 0; r < R; r++) {
            float sr = 0.0f;
#pragma unroll
            for (int d4 = 0; d4 < HD / 4; d4++) {
                const f32x4 q = reinterpret_cast<const f32x4 *>(sq + r * HD)[d4];
                sr = fmaf(q.x, kv[d4].x, sr); sr = fmaf(q.y, kv[d4].y, sr);
                sr = fmaf(q.z, kv[d4].z, sr); sr = fmaf(q.w, kv[d4].w, sr);
            }
            p[r * ldp + t] = t <= pos0 + i0 + r / GRP ? sr * scale : -INFINITY;
        }
    }
    __syncthreads();

    // softmax per row
    float mr[R];
#pragma unroll
    for (int r = 0; r < R; r++) mr[r] = -INFINITY;
    for (int t = tid; t < ctxmax; t += NTH)
#pragma unroll
        for (int r = 0; r < R; r++) mr[r] = fmaxf(mr[r], p[r * ldp + t]);
#pragma unroll
    for (int r = 0; r < R; r++) {
        mr[r] = wave_max(mr[r]);
        if (lane == 0) sred[r * 4 + wave] = mr[r];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; r++)
        mr[r] = fmaxf(fmaxf(sred[r * 4 + 0], sred[r * 4 + 1]), fmaxf(sred[r * 4 + 2], sred[r * 4 + 3]));
    __syncthreads();
    float er[R];
#pragma unroll
    for (int r = 0; r < R; r++) er[r] = 0.0f;
    for (int t = tid; t < ctxmax; t += NTH)
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float av = expf(p[r * ldp + t] - mr[r]);
            p[r * ldp + t] = av;
            er[r] += av;
        }
#pragma unroll
    for (int r = 0; r < R; r++) {
        er[r] = wave_sum(er[r]);
        if (lane == 0) sred[r * 4 + wave] = er[r];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; r++) er[r] = (sred[r * 4 + 0] + sred[r * 4 + 1]) + (sred[r * 4 + 2] + sred[r * 4 + 3]);
    for (int t = tid; t < ctxmax; t += NTH)
#pragma unroll
        for (int r = 0; r < R; r++) p[r * ldp + t] = p[r * ldp + t] / er[r];
    __syncthreads();

    // out_r[d] = sum_t p[r][t] v_t[d]: wave w takes t = w, w+4, ...; lane l
    // owns d = 2l, 2l+1 of every row; each V row serves all R rows.  Passes
    // of 16, then 8, 4 and 1 rows in flight per lane (each pass one L2 round
    // trip; measured on MI355X against one 8-row pass and the 1-row tail:
    // 64 x 2014-token batch prefill 2.71 -> 2.60 s), always adding in
    // ascending t
    f32x2 o[R];
#pragma unroll
    for (int r = 0; r < R; r++) o[r] = f32x2{0.f, 0.f};
    const f32x2 *vcache = reinterpret_cast<const f32x2 *>(vc + (size_t)g * max_seq * HD) + lane;
    int t = wave;
    auto vpass = [&](auto UC) {
        constexpr int U = decltype(UC)::value;
        for (; t + 4 * (U - 1) < ctxmax; t += 4 * U) {
            f32x2 v[U];
#pragma unroll
            for (int u = 0; u < U; u++) v[u] = vcache[(size_t)(t + 4 * u) * (HD / 2)];
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const float pw = p[r * ldp + t + 4 * u];
                    o[r].x = mul_add(pw, v[u].x, o[r].x);
                    o[r].y = mul_add(pw, v[u].y, o[r].y);
                }
        }
    };
    vpass(std::integral_constant<int, 16>{});
    vpass(std::integral_constant<int, 8>{});
    vpass(std::integral_constant<int, 4>{});
    vpass(std::integral_constant<int, 1>{});
#pragma unroll
    for (int r = 0; r < R; r++) {
        red[(wave * R + r) * HD + 2 * lane] = o[r].x;
        red[(wave * R + r) * HD + 2 * lane + 1] = o[r].y;
    }
    __syncthreads();
    for (int e = tid; e < nq * GRP * HD; e += NTH) {
        const int r = e / HD, d = e % HD;
        const float sacc = (red[(0 * R + r) * HD + d] + red[(1 * R + r) * HD + d]) +
                           (red[(2 * R + r) * HD + d] + red[(3 * R + r) * HD + d]);
        out[(size_t)(i0 + r / GRP) * (NKV * GRP * HD) + (size_t)(g * GRP + r % GRP) * HD + d] = sacc;
    }
}

// ---------------------------------------------------------------------------
// Decode attention split over positions: partials, merged by the o GEMV
// ---------------------------------------------------------------------------
// grid = (NKV * S, n_seq): block (g, s) takes positions
// [s*chunk, min(ctx, (s+1)*chunk)) of kv head g, chunk = ceil(ctx / splits)
// rounded up to a multiple of 8 (see attn_chunk), for both query heads of the
// group.  Every block normalises and ropes the
// group's two q heads itself (and the new k); block s = 0 writes the new k/v
// to the cache; the new position's k/v come from registers, never from the
// cache, so no block reads an entry written in this launch.  Each block
// writes, per head, the softmax partial of its range:
//   part[((g*S + s)*GRP + h) * QM_ATT_PART + 0] = m   (max score, -inf if empty)
//   part[... + 1] = l                                  (sum of exp(score - m))
//   part[... + 4 .. + 4 + HD) = o                      (sum exp(score - m) * v)
// The o-projection GEMV merges the splits (k_gemv1 with the merge prologue):
// out = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s with M = max_s m_s, the
// reference softmax (ops_scalar.c:37-44) regrouped over position ranges.
// A pass covers 64 positions (one pass up to ctx = 512): wave w owns head
// dims 32w .. 32w+31.  Scores: lane l takes position l (8 K loads of 16 B,
// each instruction 64 consecutive positions of the d-chunk-major cache).
// Weighted V: lane l takes chunk 8w + l%8 of positions l/8 + 8j (each
// instruction 8 positions x 128 contiguous bytes), then a 3-step shuffle
// sums the 8 lanes of a chunk.  Every K and V load of the first pass goes
// out at entry, before the q prologue: one memory round trip per launch.
// Batched decode: blockIdx.y is the sequence, with its own qkv row, position
// pos_d[seq], cache (kv_seq floats after the previous sequence's) and
// partials (8 * S * 2 * QM_ATT_PART floats after the previous sequence's).
// Positions per range: ceil(ctx / S) rounded up to a multiple of 8.  The K
// cache holds 16 bytes per position in each d-chunk row, so ranges that start
// on a multiple of 8 positions start their 1 KB load runs on a 128-byte line;
// unaligned starts fetched a ninth line per run (batched decode at context
// ~2040: 172 -> 163 us per layer launch).
__device__ __forceinline__ int attn_chunk(int ctx, int S) { return ((ctx + S - 1) / S + 7) & ~7; }

template <int S>
__global__ __launch_bounds__(NTH) void k_attn_part(const float *__restrict__ qkv,
                                                   float *__restrict__ part,
                                                   float *__restrict__ kc, float *__restrict__ vc,
                                                   const uint16_t *__restrict__ qn,
                                                   const uint16_t *__restrict__ kn,
                                                   const float *__restrict__ rcos,
                                                   const float *__restrict__ rsin,
                                                   const int *__restrict__ pos_d, int max_seq,
                                                   size_t kv_seq, float eps, float scale) {
    constexpr int P = 64;                        // positions per pass
    const int g = blockIdx.x % NKV, sp = blockIdx.x / NKV;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // sequence blockIdx.y of a batch: its qkv row, position, cache and partials
    const int seq = blockIdx.y;
    qkv += (size_t)seq * QKV_LD;
    kc += (size_t)seq * kv_seq;
    vc += (size_t)seq * kv_seq;
    part += (size_t)seq * (8 * S * GRP * QM_ATT_PART);
    const int pos = pos_d[seq];
    if (pos < 0 || pos >= max_seq) return;      // uniform per launch
    const int ctx = pos + 1;
    const int chunk = attn_chunk(ctx, S);
    const int t0 = min(ctx, sp * chunk), t1 = min(ctx, t0 + chunk);
    const int n = t1 - t0;                       // positions of this block (may be 0)

    __shared__ float sq[GRP * HD];               // normalised, roped q of both heads
    __shared__ float sk[HD];                     // the new k
    __shared__ float sc[4][GRP][P];              // per-wave partial scores
    __shared__ float pe[GRP][P];                 // softmax weights of the pass

    const f32x4 *vnew4 = reinterpret_cast<const f32x4 *>(qkv + VOFF + (size_t)g * HD);
    const int vch = 8 * wave + (lane & 7);       // V chunk (16 bytes) of this lane
    const int vp = lane >> 3;                    // V positions vp + 8j of the pass

    // 1. prologue sources first: waves 0/1 the rows of the two query heads,
    //    wave 2 the new k (wave 3 repeats wave 2's loads), norm weights, the
    //    rope angles of this position and the new v chunk -- all
    //    unconditional, so a wave later waits for these alone
    const int hw = wave < GRP + 1 ? wave : GRP;
    const float *src = hw < GRP ? qkv + (size_t)(g * GRP + hw) * HD : qkv + KOFF + (size_t)g * HD;
    const uint16_t *nwp = hw < GRP ? qn : kn;
    const float x0 = src[lane], x1 = src[lane + 64];
    const float w0 = bf16f(nwp[lane]), w1 = bf16f(nwp[lane + 64]);
    const float c = rcos[(size_t)pos * (HD / 2) + lane], sn = rsin[(size_t)pos * (HD / 2) + lane];
    const f32x4 vnew = vnew4[vch];
    __builtin_amdgcn_sched_barrier(0);

    // 2. the K and V cache reads of a pass: buffer loads whose offset is out
    //    of range (returns zeros, reads nothing) past this block's positions
    //    and at the new position, which comes from sk / vnew instead
    const __amdgpu_buffer_rsrc_t rk = buf_rsrc(kc + (size_t)g * HD * max_seq, (size_t)HD * max_seq * 4);
    const __amdgpu_buffer_rsrc_t rv = buf_rsrc(vc + (size_t)g * max_seq * HD, (size_t)max_seq * HD * 4);
    // non-temporal (aux 2): each cache entry is read once per step; measured
    // +5% batched decode at context 2048 and +4% single-sequence decode
    auto load_pass = [&](int base, f32x4 (&kk)[8], f32x4 (&vv)[8]) {
        const int tk = t0 + base + lane;
        const bool kin = base + lane < n && tk < pos;
#pragma unroll
        for (int j = 0; j < 8; j++)
            kk[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                        rk, kin ? (uint32_t)(((8 * wave + j) * max_seq + tk) * 16) : BUF_OOB, 0, 2));
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int i = base + vp + 8 * j;
            const int tv = t0 + i;
            vv[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                        rv, (i < n && tv < pos) ? (uint32_t)((tv * (HD / 4) + vch) * 16) : BUF_OOB, 0, 2));
        }
    };
    f32x4 kk[8], vv[8];
    load_pass(0, kk, vv);
    __builtin_amdgcn_sched_barrier(0);

    // 3. QK-norm + RoPE: waves 0/1 the two query heads, wave 2 the new k
    if (wave < GRP + 1) {
        float *dst = wave < GRP ? sq + wave * HD : sk;
        const float ss = wave_sum(sumsq2(x0, x1));
        const float sc_ = 1.0f / sqrtf(ss / (float)HD + eps);
        const float y0 = (x0 * sc_) * w0, y1 = (x1 * sc_) * w1;
        rope_pair(y0, y1, c, sn, dst[lane], dst[lane + 64]);
    }
    __syncthreads();
    if (sp == 0) {                               // one block per kv head writes the new entry
        if (tid < HD) kc[(((size_t)g * (HD / 4) + (tid >> 2)) * max_seq + pos) * 4 + (tid & 3)] = sk[tid];
        if (vp == 0) reinterpret_cast<f32x4 *>(vc + ((size_t)g * max_seq + pos) * HD)[vch] = vnew;
    }

    // partial score of the new position over this wave's 32 dims (its cache
    // loads read zeros): the same chain as below, computed once
    float an0 = 0.0f, an1 = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const f32x4 q0 = reinterpret_cast<const f32x4 *>(sq)[8 * wave + j];
        const f32x4 q1 = reinterpret_cast<const f32x4 *>(sq + HD)[8 * wave + j];
        const f32x4 kj = reinterpret_cast<const f32x4 *>(sk)[8 * wave + j];
        an0 = fmaf(q0.x, kj.x, an0); an0 = fmaf(q0.y, kj.y, an0);
        an0 = fmaf(q0.z, kj.z, an0); an0 = fmaf(q0.w, kj.w, an0);
        an1 = fmaf(q1.x, kj.x, an1); an1 = fmaf(q1.y, kj.y, an1);
        an1 = fmaf(q1.z, kj.z, an1); an1 = fmaf(q1.w, kj.w, an1);
    }

    float m0 = -INFINITY, m1 = -INFINITY, l0 = 0.0f, l1 = 0.0f;
    f32x4 o0 = {0.f, 0.f, 0.f, 0.f}, o1 = {0.f, 0.f, 0.f, 0.f};
    for (int base = 0; base < n; base += P) {
        if (base > 0) load_pass(base, kk, vv);
        // partial scores over this wave's 32 dims; positions past n read
        // zeros and are masked below, the new position takes an0 / an1
        {
            float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const f32x4 q0 = reinterpret_cast<const f32x4 *>(sq)[8 * wave + j];
                const f32x4 q1 = reinterpret_cast<const f32x4 *>(sq + HD)[8 * wave + j];
                a0 = fmaf(q0.x, kk[j].x, a0); a0 = fmaf(q0.y, kk[j].y, a0);
                a0 = fmaf(q0.z, kk[j].z, a0); a0 = fmaf(q0.w, kk[j].w, a0);
                a1 = fmaf(q1.x, kk[j].x, a1); a1 = fmaf(q1.y, kk[j].y, a1);
                a1 = fmaf(q1.z, kk[j].z, a1); a1 = fmaf(q1.w, kk[j].w, a1);
            }
            const bool isnew = t0 + base + lane == pos;
            sc[wave][0][lane] = isnew ? an0 : a0;
            sc[wave][1][lane] = isnew ? an1 : a1;
        }
        __syncthreads();
        // every wave sums the four partials of position `lane` and keeps the
        // pass's softmax statistics (identical in all waves)
        const bool valid = base + lane < n;
        const float s0 = valid ? ((sc[0][0][lane] + sc[1][0][lane]) + (sc[2][0][lane] + sc[3][0][lane])) * scale
                               : -INFINITY;
        const float s1 = valid ? ((sc[0][1][lane] + sc[1][1][lane]) + (sc[2][1][lane] + sc[3][1][lane])) * scale
                               : -INFINITY;
        const float nm0 = fmaxf(m0, wave_max(s0)), nm1 = fmaxf(m1, wave_max(s1));
        const float e0 = valid ? expf(s0 - nm0) : 0.0f, e1 = valid ? expf(s1 - nm1) : 0.0f;
        const float r0 = m0 == -INFINITY ? 0.0f : expf(m0 - nm0);
        const float r1 = m1 == -INFINITY ? 0.0f : expf(m1 - nm1);
        l0 = mul_add(l0, r0, wave_sum(e0));
        l1 = mul_add(l1, r1, wave_sum(e1));
        m0 = nm0;
        m1 = nm1;
        if (wave == 0) { pe[0][lane] = e0; pe[1][lane] = e1; }
        __syncthreads();
        o0 *= r0;
        o1 *= r1;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float pw0 = pe[0][vp + 8 * j], pw1 = pe[1][vp + 8 * j];   // 0 beyond n
            o0.x = fmaf(pw0, vv[j].x, o0.x); o0.y = fmaf(pw0, vv[j].y, o0.y);
            o0.z = fmaf(pw0, vv[j].z, o0.z); o0.w = fmaf(pw0, vv[j].w, o0.w);
            o1.x = fmaf(pw1, vv[j].x, o1.x); o1.y = fmaf(pw1, vv[j].y, o1.y);
            o1.z = fmaf(pw1, vv[j].z, o1.z); o1.w = fmaf(pw1, vv[j].w, o1.w);
        }
        // the new position (its cache loads read zeros): v from vnew, once,
        // in the lanes that own its row of the pass
        {
            const int inew = pos - t0 - base;
            const bool own = inew >= 0 && inew < P && (inew & 7) == vp;
            const float pn0 = own ? pe[0][inew & (P - 1)] : 0.0f, pn1 = own ? pe[1][inew & (P - 1)] : 0.0f;
            o0.x = fmaf(pn0, vnew.x, o0.x); o0.y = fmaf(pn0, vnew.y, o0.y);
            o0.z = fmaf(pn0, vnew.z, o0.z); o0.w = fmaf(pn0, vnew.w, o0.w);
            o1.x = fmaf(pn1, vnew.x, o1.x); o1.y = fmaf(pn1, vnew.y, o1.y);
            o1.z = fmaf(pn1, vnew.z, o1.z); o1.w = fmaf(pn1, vnew.w, o1.w);
        }
        __syncthreads();                          // sc / pe reused by the next pass
    }

    // sum the 8 lanes of each chunk (lanes c, c+8, ..., c+56) and write
    o0 = f32x4{sum_stride8(o0.x), sum_stride8(o0.y), sum_stride8(o0.z), sum_stride8(o0.w)};
    o1 = f32x4{sum_stride8(o1.x), sum_stride8(o1.y), sum_stride8(o1.z), sum_stride8(o1.w)};
    float *pp = part + (size_t)(g * S + sp) * GRP * QM_ATT_PART;
    if (lane < 8) {
        reinterpret_cast<f32x4 *>(pp + 4)[vch] = o0;
        reinterpret_cast<f32x4 *>(pp + QM_ATT_PART + 4)[vch] = o1;
    }
    if (tid == 0) {
        pp[0] = m0;
        pp[1] = l0;
        pp[QM_ATT_PART] = m1;
        pp[QM_ATT_PART + 1] = l1;
    }
}

// ---------------------------------------------------------------------------
// Batched decode: the split partials of k_attn_part merged into the attention
// output att[seq][16 heads x 128], the same softmax merge as the o GEMV's
// prologue: out = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s, M = max_s m_s.
// grid = (NKV, n_seq), 256 threads = 2 query heads x 128 dims.
// ---------------------------------------------------------------------------
template <int S>
__global__ __launch_bounds__(NTH) void k_attn_merge(float *__restrict__ att, const float *__restrict__ part) {
    const int g = blockIdx.x, seq = blockIdx.y, tid = threadIdx.x;
    const int h = tid >> 7, d = tid & (HD - 1);
    const float *pp = part + (size_t)seq * (8 * S * GRP * QM_ATT_PART) + (size_t)(g * S * GRP + h) * QM_ATT_PART;
    float m[S], l[S], o[S];
#pragma unroll
    for (int s = 0; s < S; s++) {
        const float *ps = pp + (size_t)s * GRP * QM_ATT_PART;
        m[s] = ps[0];
        l[s] = ps[1];
        o[s] = ps[4 + d];
    }
    float mx = m[0];
#pragma unroll
    for (int s = 1; s < S; s++) mx = fmaxf(mx, m[s]);
    float den = 0.0f, num = 0.0f;
#pragma unroll
    for (int s = 0; s < S; s++) {
        const float w = m[s] == -INFINITY ? 0.0f : expf(m[s] - mx);
        den = fmaf(w, l[s], den);
        num = fmaf(w, o[s], num);
    }
    att[(size_t)seq * (NKV * GRP * HD) + (size_t)(g * GRP + h) * HD + d] = num * (1.0f / den);
}

// (value, index) argmax step: larger value wins, ties -> lower index, an
// ordered value beats NaN (the strict ">" scan of ops_scalar.c:57-62, whose
// only other case, a NaN at index 0, the caller resolves)
__device__ __forceinline__ void am_take(float &v, int &i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i) || (v != v && v2 == v2)) { v = v2; i = i2; }
}

// ---------------------------------------------------------------------------
// Batched greedy step bookkeeping: block r scans logits row r (n floats),
// tok[r] = first index of its maximum (ops_scalar.c:57-62), then
// out[r * out_ld + pos[r] - plen[r] + 1] = tok[r] when that index lies in
// [0, out_ld), and pos[r] += 1.  grid = n_rows blocks of AM_ROW_THREADS.
// ---------------------------------------------------------------------------
#define AM_ROW_THREADS 1024
__global__ __launch_bounds__(AM_ROW_THREADS) void k_argmax_rows(const float *__restrict__ logits, int n,
                                                               int *__restrict__ tok, int *__restrict__ pos,
                                                               const int *__restrict__ plen,
                                                               int *__restrict__ out, int out_ld) {
    const int r = blockIdx.x, tid = threadIdx.x;
    const float *v = logits + (size_t)r * n;
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(v, (size_t)n * 4);
    const int n4 = n >> 2;
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    // four 16-byte loads in flight per thread; groups past n4 read nothing
    for (int i0 = tid; i0 < n4; i0 += 4 * AM_ROW_THREADS) {
        f32x4 x[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = i0 + u * AM_ROW_THREADS;
            x[u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       rs, i < n4 ? (uint32_t)i * 16u : BUF_OOB, 0, 0));
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = i0 + u * AM_ROW_THREADS;
            if (i < n4) {
                am_take(bv, bi, x[u].x, 4 * i);
                am_take(bv, bi, x[u].y, 4 * i + 1);
                am_take(bv, bi, x[u].z, 4 * i + 2);
                am_take(bv, bi, x[u].w, 4 * i + 3);
            }
        }
    }
    for (int i = 4 * n4 + tid; i < n; i += AM_ROW_THREADS) am_take(bv, bi, v[i], i);
#pragma unroll
    for (int msk = 32; msk >= 1; msk >>= 1) {
        const float ov = __shfl_xor(bv, msk);
        const int oi = __shfl_xor(bi, msk);
        am_take(bv, bi, ov, oi);
    }
    __shared__ float sv[AM_ROW_THREADS / WAVE];
    __shared__ int si[AM_ROW_THREADS / WAVE];
    if ((tid & 63) == 0) { sv[tid >> 6] = bv; si[tid >> 6] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < AM_ROW_THREADS / WAVE; w++) am_take(bv, bi, sv[w], si[w]);
        // the reference's scan starts from v[0]: a NaN there is never beaten
        const int t = (bi == 0x7FFFFFFF || v[0] != v[0]) ? 0 : bi;
        tok[r] = t;
        const int p = pos[r];
        const int idx = p - plen[r] + 1;
        if (idx >= 0 && idx < out_ld) out[(size_t)r * out_ld + idx] = t;
        pos[r] = p + 1;
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

extern "C" size_t qm_attention_lds_bytes(int qt, int ldp) {
    const size_t r = (size_t)qt * GRP;
    return sizeof(float) * (r * HD + 4 * r * HD + 4 * r + r * (size_t)ldp);
}

extern "C" int qm_rows_norm(float *x, const float *r, const uint16_t *emb, const int *tok, int emb_rows,
                            const uint16_t *nw, float *xb, int nt, int K, float eps) {
    return qm_rows_norm_split(x, r, emb, tok, emb_rows, nw, xb, nt, K, eps, nullptr, 0);
}

extern "C" int qm_rows_norm_split(float *x, const float *r, const uint16_t *emb, const int *tok, int emb_rows,
                                  const uint16_t *nw, float *xb, int nt, int K, float eps, const float *part,
                                  int ks) {
    if (!stream()) return QH_ESTATE;
    if (!x || !nw || !xb || nt <= 0 || K <= 0 || K % 4 || K > 4 * 4 * NTH) return QH_EINVAL;
    if (emb && (!tok || emb_rows <= 0)) return QH_EINVAL;
    if (ks < 0 || ks > KS_MAX || (ks > 0 && (!part || emb || r))) return QH_EINVAL;
    const size_t pstride = (size_t)nt * K;                  // one slice: [nt][K]
    if (ks > 0 && pstride * ks * 4 >= ((size_t)1 << 31)) return QH_EINVAL;
    hipLaunchKernelGGL(k_rows_norm, dim3(nt), dim3(NTH), 0, stream(), x, emb ? nullptr : r, emb, tok,
                       emb_rows, nw, xb, K, eps, part, ks, pstride);
    return hipGetLastError() == hipSuccess ? QH_OK : QH_ELAUNCH;
}

// tokens per block of the chunk attention: two while their scores fit in
// 64 KB (contexts up to ~3,440), else one.  Measured prefill of 128 / 512 /
// 1024 / 2048 tokens: 1.92 / 8.2 / 18.5 / 45.1 ms with two, 2.00 / 9.0 /
// 21.4 / 56.3 with one, 2.15 / 9.7 / 23.3 / 52.2 with four (fewer blocks
// than CUs at short contexts)
static int attention_qt(int ldp) {
    return qm_attention_lds_bytes(2, ldp) <= 65536 ? 2 : 1;
}

extern "C" int qm_attention(float *qkv, float *out, float *kc, float *vc, const uint16_t *qn,
                            const uint16_t *kn, const float *rcos, const float *rsin, const int *pos_d,
                            int nt, int max_seq, int ctx_bound, float eps) {
    if (!stream()) return QH_ESTATE;
    if (!qkv || !out || !kc || !vc || !qn || !kn || !rcos || !rsin || !pos_d) return QH_EINVAL;
    if (nt <= 0 || max_seq <= 0 || nt > QM_MAX_CHUNK || max_seq > QM_MAX_SEQ) return QH_EINVAL;
    if (ctx_bound < nt || ctx_bound > max_seq) return QH_EINVAL;
    static int attr_dev = -1;                  // the attribute is held per device
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) return QH_ELAUNCH;
    if (attr_dev != dev) {
        // one token per block at the longest context needs more than the default 64 KB
        if (hipFuncSetAttribute((const void *)k_attention<1>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)qm_attention_lds_bytes(1, QM_MAX_SEQ)) != hipSuccess)
            return QH_ELAUNCH;
        attr_dev = dev;
    }
    // 1 / sqrt(head_dim), the constant of qwen3.c:311
    const float scale = 0.08838834764831845f;
    hipLaunchKernelGGL(k_qk_rope_cache, dim3(nt, (NKV * GRP + NKV) / 4), dim3(NTH), 0, stream(), qkv, kc, vc,
                       qn, kn, rcos, rsin, pos_d, max_seq, eps);
    if (hipGetLastError() != hipSuccess) return QH_ELAUNCH;
    const int qt = attention_qt(ctx_bound);
    const size_t lds = qm_attention_lds_bytes(qt, ctx_bound);
    const dim3 grid((unsigned)(((nt + qt - 1) / qt) * NKV));
    if (qt == 2)
        hipLaunchKernelGGL(k_attention<2>, grid, dim3(NTH), lds, stream(), qkv, out, kc, vc, pos_d, nt, max_seq,
                           ctx_bound, scale);
    else
        hipLaunchKernelGGL(k_attention<1>, grid, dim3(NTH), lds, stream(), qkv, out, kc, vc, pos_d, nt, max_seq,
                           ctx_bound, scale);
    return hipGetLastError() == hipSuccess ? QH_OK : QH_ELAUNCH;
}

extern "C" int qm_attention_decode_part(const float *qkv, float *part, float *kc, float *vc, const uint16_t *qn,
                                        const uint16_t *kn, const float *rcos, const float *rsin,
                                        const int *pos_d, int max_seq, float eps) {
    if (!stream()) return QH_ESTATE;
    if (!qkv || !part || !kc || !vc || !qn || !kn || !rcos || !rsin || !pos_d) return QH_EINVAL;
    if (max_seq <= 0 || max_seq > QM_MAX_SEQ) return QH_EINVAL;
    const float scale = 0.08838834764831845f;   // 1 / sqrt(head_dim), qwen3.c:311
    hipLaunchKernelGGL(k_attn_part<QM_ATT_SPLITS>, dim3(NKV * QM_ATT_SPLITS), dim3(NTH), 0, stream(), qkv, part, kc, vc,
                       qn, kn, rcos, rsin, pos_d, max_seq, (size_t)0, eps, scale);
    return hipGetLastError() == hipSuccess ? QH_OK : QH_ELAUNCH;
}

extern "C" int qm_attention_decode_batch(const float *qkv, float *att, float *part, float *kc, float *vc,
                                         size_t kv_seq, const uint16_t *qn, const uint16_t *kn,
                                         const float *rcos, const float *rsin, const int *pos_d, int n_seq,
                                         int max_seq, float eps) {
    if (!stream()) return QH_ESTATE;
    if (!qkv || !att || !part || !kc || !vc || !qn || !kn || !rcos || !rsin || !pos_d) return QH_EINVAL;
    if (n_seq <= 0 || n_seq > QM_MAX_CHUNK || max_seq <= 0 || max_seq > QM_MAX_SEQ) return QH_EINVAL;
    if (kv_seq < (size_t)NKV * HD * max_seq) return QH_EINVAL;     // sequences' caches must not overlap
    const float scale = 0.08838834764831845f;   // 1 / sqrt(head_dim), qwen3.c:311
    hipLaunchKernelGGL(k_attn_part<QM_BATCH_SPLITS>, dim3(NKV * QM_BATCH_SPLITS, n_seq), dim3(NTH), 0, stream(),
                       qkv, part, kc, vc, qn, kn, rcos, rsin, pos_d, max_seq, kv_seq, eps, scale);
    if (hipGetLastError() != hipSuccess) return QH_ELAUNCH;
    hipLaunchKernelGGL(k_attn_merge<QM_BATCH_SPLITS>, dim3(NKV, n_seq), dim3(NTH), 0, stream(), att, part);
    return hipGetLastError() == hipSuccess ? QH_OK : QH_ELAUNCH;
}

extern "C" int qm_argmax_rows(const float *logits, int n, int n_rows, int *tok, int *pos, const int *plen,
                              int *out, int out_ld) {
    if (!stream()) return QH_ESTATE;
    if (!logits || !tok || !pos || !plen || !out || n <= 0 || n_rows <= 0 || out_ld < 0) return QH_EINVAL;
    if ((size_t)n * 4 >= ((size_t)1 << 31)) return QH_EINVAL;      // one buffer resource per row
    hipLaunchKernelGGL(k_argmax_rows, dim3(n_rows), dim3(AM_ROW_THREADS), 0, stream(), logits, n, tok, pos,
                       plen, out, out_ld);
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
