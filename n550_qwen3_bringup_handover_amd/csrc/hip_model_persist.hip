// Persistent decode step of the Qwen3-0.6B decoder stack on CDNA4 (gfx950):
// the 28 layers of one greedy decode token -- RMSNorm + q|k|v GEMV, QK-norm +
// RoPE + KV-cache write + split attention, softmax merge + o GEMV, residual
// + RMSNorm + gate|up GEMV + silu(gate) * up, down GEMV + residual
// (fpga_bringup/src/src/qwen3.c:455-576 for one token) -- in one launch
// instead of 5 per layer.  The final RMSNorm + lm_head GEMV and the argmax
// stay separate launches (qh_gemv_pro, qh_argmax_step).
//
// Every value is the per-call step's to the bit (model_hip.c decode_step):
// each stage repeats the arithmetic of the per-call kernel it replaces --
// the GEMV prologue's residual add, sum of squares, per-wave sums combined in
// the same order and bf16 rounding (k_gemv1 PRO), the attention partials of
// k_attn_part with the same 8 position ranges per kv head and the same
// block-internal wave layout, the merge of the o GEMV's MERGE prologue, and
// the GEMV rows' packed-bf16 sums in the same order (persist_common.h).
//
// Layout: 256 workgroups (one per CU) of 4 compute waves + 1 poller wave, as
// the GEMV-set kernel (hip_persist.hip).  Per layer, five exchanges of
// tagged words {fp32, epoch}:
//   q|k|v (4,096)   -> the 64 attention workgroups (blocks 0-63: kv head
//                      b % 8, range b / 8), each polling its group's 512
//                      words directly
//   partials        -> the relays, which merge them: relay r takes kv head
//                      r's 8 ranges and forwards its two query heads' merged
//                      attention output (256 floats) to its XCD
//   o (1,024)       -> every workgroup (residual + RMSNorm + gate|up)
//   h (3,072)       -> every workgroup (down)
//   down (1,024)    -> every workgroup (residual + RMSNorm + next q|k|v)
// The relays (PS_RELAYS per XCD, taken from blocks 64-255 by ticket) copy
// each part as fp32 into their XCD's copy and raise a flag.  Each poller
// keeps the residual stream (1,024 floats) in registers and hands the
// prologue's input to the compute waves through LDS; the compute waves hold
// the next stage's weights in registers while they wait (paced loads).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "hip_shim.h"
#include "persist_common.h"
#include "fp_pinned.h"

#define MP_H 1024
#define MP_QKV 4096
#define MP_I 3072
#define MP_HD 128
#define MP_NKV 8
#define MP_GRP 2
#define MP_S QH_ATT_SPLITS                              // position ranges per kv head
#define MP_PART QH_ATT_PART                             // floats per (range, query head)
#define MP_PARTS (MP_NKV * MP_S * MP_GRP * MP_PART)     // 16,896
#define MP_ATT_WG (MP_NKV * MP_S)                       // attention workgroups
#define MP_MAX_LAYERS 32
#define MP_KOFF 2048
#define MP_VOFF 3072

// per-layer exchange words (tagged), offsets in words
#define XW_QKV 0
#define XW_PART MP_QKV
#define XW_O (XW_PART + MP_PARTS)
#define XW_H (XW_O + MP_H)
#define XW_DN (XW_H + MP_I)
#define XW_LD (XW_DN + MP_H)
// per-layer XCD copy (fp32) and flag slots
#define XC_ATT 0                                         // the merged attention output (2,048)
#define XC_O (XC_ATT + MP_GRP * MP_NKV * MP_HD)
#define XC_H (XC_O + MP_H)
#define XC_DN (XC_H + MP_I)
#define XC_LD (XC_DN + MP_H)
#define FS_ATT 0
#define FS_O 1
#define FS_H 2
#define FS_DN 3

static_assert(MP_S == 8 && MP_PART == 132, "the partial layout of k_attn_part");
static_assert(MP_PARTS % PS_RELAYS == 0 && MP_H % PS_RELAYS == 0 && MP_I % PS_RELAYS == 0, "relay parts");
static_assert(PS_RELAYS == MP_NKV, "relay r merges kv head r's partials");
// s_sleep(32) rounds a relay waits after the stage's barrier before polling
// the partials: they come a q|k|v exchange and an attention after it, and
// polls that reach words before their producers' stores slow the exchange
#ifndef MP_PART_PRE
#define MP_PART_PRE 2
#endif

enum { LW_IN_NORM, LW_QKV, LW_QN, LW_KN, LW_O, LW_POST_NORM, LW_G, LW_U, LW_D, LW_N };

struct ModelPersistArgs {
    // per layer: the weights in LW_* order (scalar loads from the kernel
    // arguments, as in hip_persist.hip)
    const uint16_t *w[MP_MAX_LAYERS][LW_N];
    const uint16_t *embed;      // [vocab][1024]
    const int *state;           // [0] token, [1] position
    float *kc, *vc;             // caches of layer 0; layer l at + l * kv_layer
    size_t kv_layer;
    const float *rcos, *rsin;   // [max_seq][64]
    float *x_out;               // the residual after the last layer's o add
    float *dn_out;              // the last layer's down output
    uint64_t *xch;              // [layers][XW_LD] exchange words
    unsigned *st;               // [0] epoch, [1] error flags, [2] arrivals, [4 + x] relay tickets
    float *copy;                // [8 XCDs][MP_MAX_LAYERS][XC_LD]
    unsigned *flags;            // [8 XCDs][MP_MAX_LAYERS][4][PS_RELAYS]
    int vocab, max_seq, layers;
    float eps;
};

__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ void err(unsigned *st, int lane) {
    if (lane == 0) atomicOr(st + 1, 1u);
}
__device__ __forceinline__ void put_word(uint64_t *xch, int i, float v, unsigned tag) {
    __hip_atomic_store(xch + i, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
// the same reductions as k_attn_part (hip_model.hip)
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_partner<0xB1>(v));
    v = fmaxf(v, dpp_partner<0x4E>(v));
    v = fmaxf(v, dpp_partner<0x141>(v));
    v = fmaxf(v, dpp_partner<0x140>(v));
    auto p = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), false, false);
    v = fmaxf(__builtin_bit_cast(float, (int)p[0]), __builtin_bit_cast(float, (int)p[1]));
    p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), false, false);
    return fmaxf(__builtin_bit_cast(float, (int)p[0]), __builtin_bit_cast(float, (int)p[1]));
}
__device__ __forceinline__ float sum_stride8(float v) {
    v += dpp_partner<0x128>(v);
    auto p = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), false, false);
    v = __builtin_bit_cast(float, (int)p[0]) + __builtin_bit_cast(float, (int)p[1]);
    p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), false, false);
    return __builtin_bit_cast(float, (int)p[0]) + __builtin_bit_cast(float, (int)p[1]);
}

// ---- compute waves: the GEMV prologue -------------------------------------------
// The activation chunks of lane `lane` (chunks lane, lane + 64) of
// rmsnorm(x) * nw for the 1,024-vector x in LDS, as k_gemv1's PRO prologue
// computes them: the sum of squares of group i (4 values) by thread i of 256,
// summed per wave of 64 groups, the four wave sums added pairwise; every wave
// here computes the four wave sums itself.  nwc: the lane's chunks of nw.
__device__ __forceinline__ void prologue_chunks(const float *xin, const u32x4 (&nwc)[2], float eps, u32x4 (&xc)[2],
                                                int lane) {
    float p[4];
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const f32x4 xa = reinterpret_cast<const f32x4 *>(xin)[64 * w + lane];
        float ss = 0.0f;
        ss += sumsq4(xa.x, xa.y, xa.z, xa.w);
        p[w] = wave_sum(ss);
    }
    const float ss = (p[0] + p[1]) + (p[2] + p[3]);
    const float scale = 1.0f / sqrtf(ss / (float)MP_H + eps);
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int c = lane + WAVE * j;           // chunk c = groups 2c, 2c + 1
        const f32x4 a = reinterpret_cast<const f32x4 *>(xin)[2 * c];
        const f32x4 b = reinterpret_cast<const f32x4 *>(xin)[2 * c + 1];
        const u32x4 w = nwc[j];
        xc[j] = u32x4{pack_bf16x2((a.x * scale) * bf16lo(w.x), (a.y * scale) * bf16hi(w.x)),
                      pack_bf16x2((a.z * scale) * bf16lo(w.y), (a.w * scale) * bf16hi(w.y)),
                      pack_bf16x2((b.x * scale) * bf16lo(w.z), (b.y * scale) * bf16hi(w.z)),
                      pack_bf16x2((b.z * scale) * bf16lo(w.w), (b.w * scale) * bf16hi(w.w))};
    }
}
__device__ __forceinline__ void load_norm(u32x4 (&nwc)[2], const uint16_t *nw, int lane) {
    const __amdgpu_buffer_rsrc_t r = rsrc(nw, MP_H * 2);
#pragma unroll
    for (int j = 0; j < 2; j++) nwc[j] = __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)(lane + WAVE * j) * 16u, 0, 0);
}
// rows of a GEMV against activation chunks already in registers (K = 1024)
template <int ROWS, bool GATED>
__device__ __forceinline__ float gemv_rows_x(const Wts<ROWS, 2, GATED> &w, const u32x4 (&xc)[2], int lane) {
    constexpr int NB = GATED ? 2 * ROWS : ROWS;
    float acc[NB];
#pragma unroll
    for (int r = 0; r < NB; r++) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) s = bf16_dot2(w.v[r][j][e], xc[j][e], s);
        acc[r] = s;
    }
    float tot = 0.0f, up = 0.0f;
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
        const float t = wave_sum(acc[r]);
        tot = lane == r ? t : tot;
        if constexpr (GATED) {
            const float u = wave_sum(acc[ROWS + r]);
            up = lane == r ? u : up;
        }
    }
    return GATED ? silu_mul(tot, up) : tot;
}

// ---- compute waves: attention (k_attn_part for one (kv head, range)) ----------
struct AttnRange {
    int g, sp, pos, t0, n;
};
__device__ __forceinline__ AttnRange attn_range(int b, int pos) {
    AttnRange a;
    a.g = b % MP_NKV;
    a.sp = b / MP_NKV;
    a.pos = pos;
    const int ctx = pos + 1;
    const int chunk = ((ctx + MP_S - 1) / MP_S + 7) & ~7;   // k_attn_part's ranges
    a.t0 = min(ctx, a.sp * chunk);
    const int t1 = min(ctx, a.t0 + chunk);
    a.n = t1 - a.t0;
    return a;
}
// the attention prologue's sources that do not depend on this step's q|k|v
// (norm weights, rope angles), loaded before the q|k|v exchange
struct AttnPro {
    float w0, w1, c, sn;
};
__device__ __forceinline__ AttnPro attn_pro(const AttnRange &a, const uint16_t *qn, const uint16_t *kn,
                                            const float *rcos, const float *rsin, int wave, int lane) {
    const uint16_t *nwp = (wave < MP_GRP ? wave : MP_GRP) < MP_GRP ? qn : kn;
    AttnPro r;
    r.w0 = __uint_as_float((uint32_t)nwp[lane] << 16);
    r.w1 = __uint_as_float((uint32_t)nwp[lane + 64] << 16);
    r.c = rcos[(size_t)a.pos * (MP_HD / 2) + lane];
    r.sn = rsin[(size_t)a.pos * (MP_HD / 2) + lane];
    return r;
}
struct AttnLds {
    float sq[MP_GRP * MP_HD];   // normalised, roped q of both heads
    float sk[MP_HD];            // the new k
    float sc[4][MP_GRP][64];    // per-wave partial scores
    float pe[MP_GRP][64];       // softmax weights of the pass
};
// the K and V cache loads of one pass (zeros past the range and at the new
// position, whose k and v come from LDS)
__device__ __forceinline__ void attn_load_pass(const AttnRange &a, int base, const float *kc, const float *vc,
                                               int max_seq, int wave, int lane, f32x4 (&kk)[8], f32x4 (&vv)[8]) {
    const __amdgpu_buffer_rsrc_t rk = rsrc(kc + (size_t)a.g * MP_HD * max_seq, (size_t)MP_HD * max_seq * 4);
    const __amdgpu_buffer_rsrc_t rv = rsrc(vc + (size_t)a.g * max_seq * MP_HD, (size_t)max_seq * MP_HD * 4);
    // computed here on each call: hoisted out of the layer loop, these
    // offsets would stay live in registers through every stage
    asm volatile("" : "+v"(lane));
    const int vch = 8 * wave + (lane & 7), vp = lane >> 3;
    const int tk = a.t0 + base + lane;
    const bool kin = base + lane < a.n && tk < a.pos;
#pragma unroll
    for (int j = 0; j < 8; j++)
        kk[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                    rk, kin ? (uint32_t)(((8 * wave + j) * max_seq + tk) * 16) : 0x80000000u, 0, AUX_NT));
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int i = base + vp + 8 * j;
        const int tv = a.t0 + i;
        vv[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                    rv, (i < a.n && tv < a.pos) ? (uint32_t)((tv * (MP_HD / 4) + vch) * 16) : 0x80000000u, 0, AUX_NT));
    }
}
// the attention of k_attn_part from the group's q|k|v rows in LDS (qg: q of
// heads 2g, 2g+1, k, v; 128 floats each); pass 0's cache loads are in kk/vv.
// Writes the partials as tagged words and, for range 0, the new cache entry.
// Barriers: 1 + 3 per pass of 64 positions (the poller takes as many).
__device__ __forceinline__ void attn_body(const AttnRange &a, const float *qg, AttnLds &L, f32x4 (&kk)[8],
                                          f32x4 (&vv)[8], const AttnPro &pr, float *kc, float *vc, int max_seq,
                                          float eps, uint64_t *xpart, unsigned tag, int wave, int lane) {
    constexpr int P = 64;
    const float scale = 0.08838834764831845f;   // 1 / sqrt(head_dim), qwen3.c:311
    const int tid = wave * WAVE + lane;
    const int vch = 8 * wave + (lane & 7), vp = lane >> 3;
    const int hw = wave < MP_GRP + 1 ? wave : MP_GRP;
    const float *src = qg + hw * MP_HD;
    const float x0 = src[lane], x1 = src[lane + 64];
    const float w0 = pr.w0, w1 = pr.w1, c = pr.c, sn = pr.sn;
    const f32x4 vnew = reinterpret_cast<const f32x4 *>(qg + 3 * MP_HD)[vch];

    if (wave < MP_GRP + 1) {
        float *dst = wave < MP_GRP ? L.sq + wave * MP_HD : L.sk;
        const float ss = wave_sum(sumsq2(x0, x1));
        const float sc_ = 1.0f / sqrtf(ss / (float)MP_HD + eps);
        const float y0 = (x0 * sc_) * w0, y1 = (x1 * sc_) * w1;
        rope_pair(y0, y1, c, sn, dst[lane], dst[lane + 64]);
    }
    __syncthreads();
    if (a.sp == 0) {                                 // range 0 writes the new entry
        if (tid < MP_HD) kc[(((size_t)a.g * (MP_HD / 4) + (tid >> 2)) * max_seq + a.pos) * 4 + (tid & 3)] = L.sk[tid];
        if (vp == 0) reinterpret_cast<f32x4 *>(vc + ((size_t)a.g * max_seq + a.pos) * MP_HD)[vch] = vnew;
    }
    float an0 = 0.0f, an1 = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const f32x4 q0 = reinterpret_cast<const f32x4 *>(L.sq)[8 * wave + j];
        const f32x4 q1 = reinterpret_cast<const f32x4 *>(L.sq + MP_HD)[8 * wave + j];
        const f32x4 kj = reinterpret_cast<const f32x4 *>(L.sk)[8 * wave + j];
        an0 = fmaf(q0.x, kj.x, an0); an0 = fmaf(q0.y, kj.y, an0);
        an0 = fmaf(q0.z, kj.z, an0); an0 = fmaf(q0.w, kj.w, an0);
        an1 = fmaf(q1.x, kj.x, an1); an1 = fmaf(q1.y, kj.y, an1);
        an1 = fmaf(q1.z, kj.z, an1); an1 = fmaf(q1.w, kj.w, an1);
    }
    float m0 = -INFINITY, m1 = -INFINITY, l0 = 0.0f, l1 = 0.0f;
    f32x4 o0 = {0.f, 0.f, 0.f, 0.f}, o1 = {0.f, 0.f, 0.f, 0.f};
    for (int base = 0; base < a.n; base += P) {
        if (base > 0) attn_load_pass(a, base, kc, vc, max_seq, wave, lane, kk, vv);
        {
            float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const f32x4 q0 = reinterpret_cast<const f32x4 *>(L.sq)[8 * wave + j];
                const f32x4 q1 = reinterpret_cast<const f32x4 *>(L.sq + MP_HD)[8 * wave + j];
                a0 = fmaf(q0.x, kk[j].x, a0); a0 = fmaf(q0.y, kk[j].y, a0);
                a0 = fmaf(q0.z, kk[j].z, a0); a0 = fmaf(q0.w, kk[j].w, a0);
                a1 = fmaf(q1.x, kk[j].x, a1); a1 = fmaf(q1.y, kk[j].y, a1);
                a1 = fmaf(q1.z, kk[j].z, a1); a1 = fmaf(q1.w, kk[j].w, a1);
            }
            const bool isnew = a.t0 + base + lane == a.pos;
            L.sc[wave][0][lane] = isnew ? an0 : a0;
            L.sc[wave][1][lane] = isnew ? an1 : a1;
        }
        __syncthreads();
        const bool valid = base + lane < a.n;
        const float s0 = valid ? ((L.sc[0][0][lane] + L.sc[1][0][lane]) + (L.sc[2][0][lane] + L.sc[3][0][lane])) * scale
                               : -INFINITY;
        const float s1 = valid ? ((L.sc[0][1][lane] + L.sc[1][1][lane]) + (L.sc[2][1][lane] + L.sc[3][1][lane])) * scale
                               : -INFINITY;
        const float nm0 = fmaxf(m0, wave_max(s0)), nm1 = fmaxf(m1, wave_max(s1));
        const float e0 = valid ? expf(s0 - nm0) : 0.0f, e1 = valid ? expf(s1 - nm1) : 0.0f;
        const float r0 = m0 == -INFINITY ? 0.0f : expf(m0 - nm0);
        const float r1 = m1 == -INFINITY ? 0.0f : expf(m1 - nm1);
        l0 = mul_add(l0, r0, wave_sum(e0));
        l1 = mul_add(l1, r1, wave_sum(e1));
        m0 = nm0;
        m1 = nm1;
        if (wave == 0) { L.pe[0][lane] = e0; L.pe[1][lane] = e1; }
        __syncthreads();
        o0 *= r0;
        o1 *= r1;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float pw0 = L.pe[0][vp + 8 * j], pw1 = L.pe[1][vp + 8 * j];
            o0.x = fmaf(pw0, vv[j].x, o0.x); o0.y = fmaf(pw0, vv[j].y, o0.y);
            o0.z = fmaf(pw0, vv[j].z, o0.z); o0.w = fmaf(pw0, vv[j].w, o0.w);
            o1.x = fmaf(pw1, vv[j].x, o1.x); o1.y = fmaf(pw1, vv[j].y, o1.y);
            o1.z = fmaf(pw1, vv[j].z, o1.z); o1.w = fmaf(pw1, vv[j].w, o1.w);
        }
        {
            const int inew = a.pos - a.t0 - base;
            const bool own = inew >= 0 && inew < P && (inew & 7) == vp;
            const float pn0 = own ? L.pe[0][inew & (P - 1)] : 0.0f, pn1 = own ? L.pe[1][inew & (P - 1)] : 0.0f;
            o0.x = fmaf(pn0, vnew.x, o0.x); o0.y = fmaf(pn0, vnew.y, o0.y);
            o0.z = fmaf(pn0, vnew.z, o0.z); o0.w = fmaf(pn0, vnew.w, o0.w);
            o1.x = fmaf(pn1, vnew.x, o1.x); o1.y = fmaf(pn1, vnew.y, o1.y);
            o1.z = fmaf(pn1, vnew.z, o1.z); o1.w = fmaf(pn1, vnew.w, o1.w);
        }
        __syncthreads();
    }
    o0 = f32x4{sum_stride8(o0.x), sum_stride8(o0.y), sum_stride8(o0.z), sum_stride8(o0.w)};
    o1 = f32x4{sum_stride8(o1.x), sum_stride8(o1.y), sum_stride8(o1.z), sum_stride8(o1.w)};
    // partials as tagged words, the k_attn_part layout: [m, l, 0, 0, o[128]] per query head
    const int pb = (a.g * MP_S + a.sp) * MP_GRP * MP_PART;
    if (lane < 8) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            put_word(xpart, pb + 4 + 4 * vch + e, o0[e], tag);
            put_word(xpart, pb + MP_PART + 4 + 4 * vch + e, o1[e], tag);
        }
    }
    if (tid == 0) {
        put_word(xpart, pb, m0, tag);
        put_word(xpart, pb + 1, l0, tag);
        put_word(xpart, pb + 2, 0.0f, tag);
        put_word(xpart, pb + 3, 0.0f, tag);
        put_word(xpart, pb + MP_PART, m1, tag);
        put_word(xpart, pb + MP_PART + 1, l1, tag);
        put_word(xpart, pb + MP_PART + 2, 0.0f, tag);
        put_word(xpart, pb + MP_PART + 3, 0.0f, tag);
    }
}

// ---- relay: the o GEMV's merge prologue, for one kv head ---------------------
// Relay r polls kv head r's partials (8 ranges x 2 query heads x MP_PART
// words), puts them in LDS (scr, MP_S * MP_GRP * MP_PART floats) and merges
// them as k_gemv1's MERGE prologue does -- lane i takes group i of the two
// heads' 256 outputs (head i / 32, dims 4 (i % 32) .. + 3) -- into dims
// 256 r .. 256 r + 255 of the XCD's copy of the attention output; then,
// once the stores are acknowledged, its flag.
__device__ __forceinline__ void relay_merge(const uint64_t *xpart, int r, float *scr, float *catt, unsigned *flag,
                                            unsigned tag, unsigned *st, int lane, bool &gave_up) {
    constexpr int VP = MP_S * MP_GRP * MP_PART, NL = (VP + 127) / 128;     // 2,112 words
    static_assert(VP == MP_PARTS / PS_RELAYS, "a relay part is one kv head's partials");
    u32x4 d[NL];
#pragma unroll
    for (int k = 0; k < MP_PART_PRE; k++) __builtin_amdgcn_s_sleep(32);
    relay_wait<VP>(xpart + (size_t)r * VP, tag, d, st, lane, gave_up);
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int q = lane + WAVE * i;                    // words 2q, 2q + 1 of the part
        if (2 * q < VP) {
            scr[2 * q] = __uint_as_float(d[i].x);
            scr[2 * q + 1] = __uint_as_float(d[i].z);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);                        // wave-private LDS: written before read
    const int h = lane >> 5, d4 = lane & 31;
    float mml[MP_S][2];
    f32x4 mo[MP_S];
#pragma unroll
    for (int sp = 0; sp < MP_S; sp++) {
        const float *pp = scr + (sp * MP_GRP + h) * MP_PART;
        mml[sp][0] = pp[0];
        mml[sp][1] = pp[1];
        mo[sp] = reinterpret_cast<const f32x4 *>(pp + 4)[d4];
    }
    float mx = mml[0][0];
#pragma unroll
    for (int sp = 1; sp < MP_S; sp++) mx = fmaxf(mx, mml[sp][0]);
    float den = 0.0f;
    f32x4 num = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sp = 0; sp < MP_S; sp++) {
        const float w = mml[sp][0] == -INFINITY ? 0.0f : expf(mml[sp][0] - mx);
        den = fmaf(w, mml[sp][1], den);
        num.x = fmaf(w, mo[sp].x, num.x);
        num.y = fmaf(w, mo[sp].y, num.y);
        num.z = fmaf(w, mo[sp].z, num.z);
        num.w = fmaf(w, mo[sp].w, num.w);
    }
    const float inv = 1.0f / den;
    const f32x4 xa = num * inv;
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, xa), rsrc(catt + (size_t)r * 256, 256 * 4),
                                           (uint32_t)lane * 16u, 0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    if (lane == 0) __builtin_amdgcn_raw_buffer_store_b32(tag, rsrc(flag, PS_RELAYS * 4), (uint32_t)r * 4u, 0, 0);
}

// ---- poller wave ----------------------------------------------------------------
// wait for the group's 512 q|k|v words (q of heads 2g, 2g+1; k and v of kv
// head g) and put them into qg as fp32 (bounded)
__device__ __forceinline__ void poll_group_qkv(const uint64_t *xq, int g, unsigned tag, float *qg, unsigned *st,
                                               int lane, bool &gave_up) {
    const __amdgpu_buffer_rsrc_t rs = rsrc(xq, MP_QKV * 8);
    uint32_t off[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int w = 2 * (lane + WAVE * i);         // first word of piece i, 0 .. 510
        const int row = w < 256 ? 256 * g + w : (w < 384 ? MP_KOFF + 128 * g + (w - 256) : MP_VOFF + 128 * g + (w - 384));
        off[i] = (uint32_t)row * 8u;
    }
    u32x4 d[4];
    uint32_t ready = 0;
    __builtin_amdgcn_s_sleep(PS_PRE);
    for (int spin = 0;; spin++) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (!(ready >> i & 1u)) d[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, off[i], 0, AUX_SC1);
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (d[i].y == tag && d[i].w == tag) ready |= 1u << i;
        if (__all(ready == 15u)) break;
        if (gave_up || spin >= PS_SPIN) {
            err(st, lane);
            gave_up = true;
            break;
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int w = 2 * (lane + WAVE * i);
        qg[w] = __uint_as_float(d[i].x);
        qg[w + 1] = __uint_as_float(d[i].z);
    }
}
// relay: part r of the V words at src into the XCD copy dst (fp32), flag
template <int V>
__device__ __forceinline__ void relay_f32(const uint64_t *src, float *dst, unsigned *flag, int r, unsigned tag,
                                          unsigned *st, int lane, bool &gave_up) {
    constexpr int VP = V / PS_RELAYS, NL = (VP + 127) / 128;
    u32x4 d[NL];
    relay_wait<VP>(src + (size_t)r * VP, tag, d, st, lane, gave_up);
    relay_put_f32<VP>(d, dst + (size_t)r * VP, flag, r, tag, lane);
}
// the residual update x = 0 + (x + r) (k_gemv1's prologue sum with no
// embedding row) from the XCD copy of r; x into xin for the compute waves.
// Lane l holds groups l, l + 64, l + 128, l + 192.
__device__ __forceinline__ void residual_add(f32x4 (&x)[4], const float *r, float *xin) {
    const int lane = threadIdx.x & 63;
    const __amdgpu_buffer_rsrc_t rr = rsrc(r, MP_H * 4);
    f32x4 rv[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
        rv[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rr, (uint32_t)(lane + WAVE * i) * 16u, 0, AUX_SC1));
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        x[i] = zero + (x[i] + rv[i]);
        reinterpret_cast<f32x4 *>(xin)[lane + WAVE * i] = x[i];
    }
}

__global__ __launch_bounds__(PS_THREADS, 1) void k_model_persist(ModelPersistArgs p) {
    __shared__ __align__(16) float xin[MP_H];                  // prologue input (fp32)
    __shared__ __align__(16) uint32_t act[2][PS_LDS_U32];      // bf16 activations: [0] o, [1] down
    __shared__ __align__(16) float qg[4 * MP_HD];              // attention: the group's q|k|v rows
    __shared__ __align__(16) AttnLds alds;
    __shared__ int s_xcd, s_part;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const unsigned tag = __hip_atomic_load(p.st, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    const int pos = p.state[1];
    const bool att = blockIdx.x < MP_ATT_WG;
    if (tid == 0) {
        unsigned xr;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xr));
        const int xcd = (int)(xr & (PS_XCDS - 1));
        s_xcd = xcd;
        s_part = -1;
        if (!att) {
            const unsigned t = __hip_atomic_fetch_add(p.st + 4 + xcd, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_part = t < PS_RELAYS ? (int)t : -1;
        }
    }
    __syncthreads();
    const bool pos_ok = pos >= 0 && pos < p.max_seq;     // uniform: every workgroup reads the same state
    float *const copy = p.copy + (size_t)s_xcd * MP_MAX_LAYERS * XC_LD;
    unsigned *const flags = p.flags + (size_t)s_xcd * MP_MAX_LAYERS * 4 * PS_RELAYS;
    auto cpy = [&](int l) { return copy + (size_t)l * XC_LD; };
    auto flg = [&](int l, int slot) { return flags + ((size_t)l * 4 + slot) * PS_RELAYS; };
    const AttnRange ar = attn_range(blockIdx.x, pos);
    const int npass = (ar.n + 63) / 64;

    if (!pos_ok) {
        if (tid == 0) atomicOr(p.st + 1, 1u);
    } else if (wave == PS_CWAVES) {
        // ---- poller ------------------------------------------------------
        bool gave_up = false;
        const int part = s_part;
        f32x4 x[4];                                           // the residual stream
        for (int l = 0; l < p.layers; l++) {
            const uint64_t *xw = p.xch + (size_t)l * XW_LD;
            // A: x + down of layer l - 1 (layer 0: the embedding row) -> xin
            if (l == 0) {
                int t = p.state[0];
                t = t < 0 ? 0 : (t >= p.vocab ? p.vocab - 1 : t);
                const __amdgpu_buffer_rsrc_t re = rsrc(p.embed + (size_t)t * MP_H, MP_H * 2);
                const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint2 e = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                                                  re, (uint32_t)(lane + WAVE * i) * 8u, 0, 0));
                    x[i] = f32x4{bf16lo(e.x), bf16hi(e.x), bf16lo(e.y), bf16hi(e.y)} + (zero + zero);
                    reinterpret_cast<f32x4 *>(xin)[lane + WAVE * i] = x[i];
                }
            } else {
                if (part >= 0)
                    relay_f32<MP_H>(xw - XW_LD + XW_DN, cpy(l - 1) + XC_DN, flg(l - 1, FS_DN), part, tag, p.st, lane,
                                    gave_up);
                wait_flags(flg(l - 1, FS_DN), tag, p.st, lane, gave_up);
                residual_add(x, cpy(l - 1) + XC_DN, xin);
            }
            __syncthreads();                                  // A
            // B: the attention workgroups' q|k|v, and the barriers of their attention
            if (att) {
                poll_group_qkv(xw + XW_QKV, ar.g, tag, qg, p.st, lane, gave_up);
                __syncthreads();                              // B
                __syncthreads();                              // attention: after the QK-norm
                for (int i = 0; i < npass; i++) {
                    __syncthreads();
                    __syncthreads();
                    __syncthreads();
                }
            }
            // C: the merged attention output (the relays merge the partials) -> act[0] as bf16
            if (part >= 0)
                relay_merge(xw + XW_PART, part, reinterpret_cast<float *>(&act[0][0]), cpy(l) + XC_ATT,
                            flg(l, FS_ATT), tag, p.st, lane, gave_up);
            wait_flags(flg(l, FS_ATT), tag, p.st, lane, gave_up);
            {
                const __amdgpu_buffer_rsrc_t ra = rsrc(cpy(l) + XC_ATT, 2048 * 4);
#pragma unroll
                for (int i = 0; i < 2048 / (4 * WAVE); i++) {
                    const int q = lane + WAVE * i;
                    const f32x4 v = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                  ra, (uint32_t)q * 16u, 0, AUX_SC1));
                    reinterpret_cast<uint2 *>(act[0])[q] = uint2{pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w)};
                }
            }
            __syncthreads();                                  // C
            // D: x + o -> xin
            if (part >= 0) relay_f32<MP_H>(xw + XW_O, cpy(l) + XC_O, flg(l, FS_O), part, tag, p.st, lane, gave_up);
            wait_flags(flg(l, FS_O), tag, p.st, lane, gave_up);
            residual_add(x, cpy(l) + XC_O, xin);
            __syncthreads();                                  // D
            // E: h -> act[1] as bf16 pairs
            if (part >= 0) relay_f32<MP_I>(xw + XW_H, cpy(l) + XC_H, flg(l, FS_H), part, tag, p.st, lane, gave_up);
            wait_flags(flg(l, FS_H), tag, p.st, lane, gave_up);
            {
                const __amdgpu_buffer_rsrc_t rh = rsrc(cpy(l) + XC_H, MP_I * 4);
#pragma unroll
                for (int i = 0; i < MP_I / (4 * WAVE); i++) {
                    const int q = lane + WAVE * i;
                    const f32x4 v = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                  rh, (uint32_t)q * 16u, 0, AUX_SC1));
                    reinterpret_cast<uint2 *>(act[1])[q] = uint2{pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w)};
                }
            }
            __syncthreads();                                  // E
        }
        if (blockIdx.x == 0) {                                // the final prologue's x
#pragma unroll
            for (int i = 0; i < 4; i++) reinterpret_cast<f32x4 *>(p.x_out)[lane + WAVE * i] = x[i];
        }
    } else {
        // ---- compute waves ----------------------------------------------
        const int gw = blockIdx.x * PS_CWAVES + wave;        // 0 .. 1023
        Wts<4, 2, false> wa;    // q|k|v: rows 4gw .. 4gw+3 of 4096, K 1024
        Wts<1, 4, false> wb;    // o: row gw of 1024, K 2048
        Wts<3, 2, true> wc;     // gate|up: rows 3gw .. 3gw+2 of 3072, K 1024
        Wts<1, 6, false> wd;    // down: row gw of 1024, K 3072
        u32x4 nwc[2], xc[2];
        f32x4 kk[8], vv[8];
        load_wts<4, 2, false, 0>(wa, p.w[0][LW_QKV], nullptr, 4 * gw, MP_QKV, lane);
        for (int l = 0; l < p.layers; l++) {
            const uint16_t *const *wl = p.w[l];
            uint64_t *xw = p.xch + (size_t)l * XW_LD;
            float *kc = p.kc + (size_t)l * p.kv_layer, *vc = p.vc + (size_t)l * p.kv_layer;
            load_norm(nwc, wl[LW_IN_NORM], lane);
            __syncthreads();                                  // A
            prologue_chunks(xin, nwc, p.eps, xc, lane);
            float v = gemv_rows_x<4, false>(wa, xc, lane);
            if (lane < 4) put_word(xw + XW_QKV, 4 * gw + lane, v, tag);
            // the attention's cache reads go out before the o weights, so they
            // do not queue behind them
            AttnPro pr;
            if (att) {
                pr = attn_pro(ar, wl[LW_QN], wl[LW_KN], p.rcos, p.rsin, wave, lane);
                attn_load_pass(ar, 0, kc, vc, p.max_seq, wave, lane, kk, vv);
            }
            load_wts<1, 4, false, PACE_O>(wb, wl[LW_O], nullptr, gw, MP_H, lane);
            if (att) {
                __syncthreads();                              // B
                attn_body(ar, qg, alds, kk, vv, pr, kc, vc, p.max_seq, p.eps, xw + XW_PART, tag, wave, lane);
            }
            __syncthreads();                                  // C
            v = gemv_rows(wb, act[0], lane);
            if (lane < 1) put_word(xw + XW_O, gw, v, tag);
            load_wts<3, 2, true, PACE_GU>(wc, wl[LW_G], wl[LW_U], 3 * gw, MP_I, lane);
            load_norm(nwc, wl[LW_POST_NORM], lane);
            __syncthreads();                                  // D
            prologue_chunks(xin, nwc, p.eps, xc, lane);
            v = gemv_rows_x<3, true>(wc, xc, lane);
            if (lane < 3) put_word(xw + XW_H, 3 * gw + lane, v, tag);
            load_wts<1, 6, false, PACE_D>(wd, wl[LW_D], nullptr, gw, MP_H, lane);
            __syncthreads();                                  // E
            v = gemv_rows(wd, act[1], lane);
            if (lane < 1) {
                put_word(xw + XW_DN, gw, v, tag);
                if (l + 1 == p.layers) p.dn_out[gw] = v;
            }
            // the next layer's q|k|v, unconditionally (an empty resource after
            // the last layer: its loads read zeros and touch no memory)
            const bool more = l + 1 < p.layers;
            load_wts<4, 2, false, PACE_QKV>(wa, p.w[more ? l + 1 : l][LW_QKV], nullptr, 4 * gw, more ? MP_QKV : 0, lane);
        }
    }
    // the next launch's epoch, published by the last workgroup to finish
    if (tid == 0) {
        const unsigned arrived = __hip_atomic_fetch_add(p.st + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (arrived == gridDim.x - 1) {
            for (int xd = 0; xd < PS_XCDS; xd++)
                __hip_atomic_store(p.st + 4 + xd, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(p.st + 2, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(p.st, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ---- host side ------------------------------------------------------------------
static uint64_t *g_mx = nullptr;       // [MP_MAX_LAYERS][XW_LD] exchange words
static unsigned *g_mst = nullptr;      // epoch, error flags, arrivals, relay tickets
static float *g_mcopy = nullptr;       // [PS_XCDS][MP_MAX_LAYERS][XC_LD]
static unsigned *g_mflags = nullptr;   // [PS_XCDS][MP_MAX_LAYERS][4][PS_RELAYS]
static int g_mp_ok = 0;

extern "C" void qm_persist_shutdown(void) {
    (void)hipFree(g_mx);
    (void)hipFree(g_mst);
    (void)hipFree(g_mcopy);
    (void)hipFree(g_mflags);
    g_mx = nullptr;
    g_mst = nullptr;
    g_mcopy = nullptr;
    g_mflags = nullptr;
    g_mp_ok = 0;
}

// once, device current: the buffers (the exchange words start at epoch 0,
// which no launch uses) and whether the device keeps the grid resident
extern "C" int qm_persist_init(void) {
    if (g_mx) return QH_OK;
    int dev = 0, cus = 0, nb = 0;
    g_mp_ok = hipGetDevice(&dev) == hipSuccess &&
              hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
              hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_model_persist, PS_THREADS, 0) == hipSuccess &&
              cus == PS_BLOCKS && nb >= 1;
    (void)hipGetLastError();
    const size_t xb = (size_t)MP_MAX_LAYERS * XW_LD * 8;
    const size_t cb = (size_t)PS_XCDS * MP_MAX_LAYERS * XC_LD * 4;
    const size_t fb = (size_t)PS_XCDS * MP_MAX_LAYERS * 4 * PS_RELAYS * 4;
    if (hipMalloc((void **)&g_mx, xb) != hipSuccess || hipMalloc((void **)&g_mst, 64) != hipSuccess ||
        hipMalloc((void **)&g_mcopy, cb) != hipSuccess || hipMalloc((void **)&g_mflags, fb) != hipSuccess ||
        hipMemset(g_mx, 0, xb) != hipSuccess || hipMemset(g_mst, 0, 64) != hipSuccess ||
        hipMemset(g_mcopy, 0, cb) != hipSuccess || hipMemset(g_mflags, 0, fb) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
        (void)hipGetLastError();
        qm_persist_shutdown();
        return QH_ENOMEM;
    }
    return QH_OK;
}

extern "C" int qm_persist_supported(void) { return g_mp_ok; }

extern "C" int qm_decode_layers_persist(const uint16_t *const *w, int layers, const uint16_t *embed, int vocab,
                                        const int *state, float *kc, float *vc, size_t kv_layer, const float *rcos,
                                        const float *rsin, int max_seq, float eps, float *x_out, float *dn_out) {
    if (!w || !embed || !state || !kc || !vc || !rcos || !rsin || !x_out || !dn_out) return QH_EINVAL;
    if (layers < 1 || vocab < 1 || max_seq < 1) return QH_EINVAL;
    if (layers > MP_MAX_LAYERS) return QH_ETOOBIG;
    if (!g_mx || !g_mp_ok) return QH_ENODEV;
    ModelPersistArgs a;
    memset(&a, 0, sizeof a);          // no stray stack bytes in the kernel arguments' padding
    for (int l = 0; l < MP_MAX_LAYERS; l++)
        for (int k = 0; k < LW_N; k++) {
            a.w[l][k] = l < layers ? w[LW_N * l + k] : nullptr;
            if (l < layers && !a.w[l][k]) return QH_EINVAL;
        }
    a.embed = embed;
    a.state = state;
    a.kc = kc;
    a.vc = vc;
    a.kv_layer = kv_layer;
    a.rcos = rcos;
    a.rsin = rsin;
    a.x_out = x_out;
    a.dn_out = dn_out;
    a.xch = g_mx;
    a.st = g_mst;
    a.copy = g_mcopy;
    a.flags = g_mflags;
    a.vocab = vocab;
    a.max_seq = max_seq;
    a.layers = layers;
    a.eps = eps;
    hipLaunchKernelGGL(k_model_persist, dim3(PS_BLOCKS), dim3(PS_THREADS), 0, (hipStream_t)qh_stream(), a);
    return hipGetLastError() == hipSuccess ? QH_OK : QH_ELAUNCH;
}

// error flags raised by launches since the last call (synchronises the stream)
extern "C" int qm_persist_errors(unsigned *flags) {
    if (!g_mst || !flags) return QH_ESTATE;
    unsigned h[2] = {0u, 0u};
    if (hipStreamSynchronize((hipStream_t)qh_stream()) != hipSuccess ||
        hipMemcpy(h, g_mst, sizeof h, hipMemcpyDeviceToHost) != hipSuccess) {
        (void)hipGetLastError();
        return QH_ERUNTIME;
    }
    *flags = h[1];
    if (h[1] && hipMemset(g_mst + 1, 0, sizeof(unsigned)) != hipSuccess) {
        (void)hipGetLastError();
        return QH_ERUNTIME;
    }
    return QH_OK;
}
