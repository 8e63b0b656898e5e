// Types, launch constants and the bf16 / reduction / epilogue helpers that
// every GEMM and GEMV kernel of the library uses (CDNA4, gfx950).
#ifndef QH_GEMM_COMMON_H
#define QH_GEMM_COMMON_H

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "hip_shim.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

#define WAVE 64
#define NTHREADS 256

// ---------------------------------------------------------------------------
// bf16 helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// two fp32 -> packed bf16 pair (low half = first), RNE: one v_cvt_pk_bf16_f32
__device__ __forceinline__ uint32_t pack_bf16x2(float x, float y) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const f32x2_t f = {x, y};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}
__device__ __forceinline__ float round_bf16(float x) {
    return __uint_as_float((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x) << 16);
}

// raw buffer resource over [p, p + bytes): stride 0, num_records = bytes.  A
// load at an offset past num_records returns zeros and reads no memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *p, size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)(uint32_t)bytes, 0x00020000);
}
#define BUF_OOB 0x80000000u      // an offset past every buffer below 2 GiB
#define AUX_SC1 16               // buffer-op cache policy: agent scope, coherent across the XCDs' L2s

// w.lo * x.lo + w.hi * x.hi + acc for two packed bf16 pairs (v_dot2_f32_bf16)
__device__ __forceinline__ float bf16_dot2(uint32_t w, uint32_t x, float acc) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w), __builtin_bit_cast(bf16x2_t, x), acc,
                                           false);
}

// Sum over the 64 lanes of a wave, the same bits in every lane.  Each step
// adds a lane's value and its partner's, so both partners hold the same sum:
// DPP within rows of 16 lanes (quad permutes for xor 1 and xor 2, then the
// half-row mirror and the row mirror, which pair groups that already hold
// equal sums), then the gfx950 permlane swaps across rows (xor 16, xor 32).
// All VALU: no LDS round trip.
template <int CTRL>
__device__ __forceinline__ float dpp_partner(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_sum(float x) {
    x += dpp_partner<0xB1>(x);      // quad_perm [1,0,3,2]
    x += dpp_partner<0x4E>(x);      // quad_perm [2,3,0,1]
    x += dpp_partner<0x141>(x);     // row_half_mirror
    x += dpp_partner<0x140>(x);     // row_mirror
    const auto p16 = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, x), __builtin_bit_cast(int, x), false, false);
    x = __builtin_bit_cast(float, (int)p16[0]) + __builtin_bit_cast(float, (int)p16[1]);
    const auto p32 = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, x), __builtin_bit_cast(int, x), false, false);
    return __builtin_bit_cast(float, (int)p32[0]) + __builtin_bit_cast(float, (int)p32[1]);
}

__device__ __forceinline__ float silu_mul(float g, float u) {
    // reference: (g / (1 + expf(-g))) * u  (ops_scalar.c:46-51)
    return (g / (1.0f + expf(-g))) * u;
}

#endif  // QH_GEMM_COMMON_H
