// Floating-point expressions whose rounding must not depend on the code
// around them.  hipcc contracts a product and a sum into one fused
// multiply-add wherever the backend sees fit (-ffp-contract=fast-honor-
// pragmas), so the same source line -- a*a + b*b, say -- can round
// differently in two kernels, depending on which product the backend fuses
// there.  Each helper below turns contraction off: every product and every
// sum is rounded on its own, as the reference's scalar C computes them
// (fpga_bringup/src/src/ops_scalar.c), and every kernel that uses a helper
// gets the same bits.  The decode kernels share these, so the per-layer
// launches and the persistent decode step agree to the bit.
#ifndef QH_FP_PINNED_H
#define QH_FP_PINNED_H

// a*a + b*b
__device__ __forceinline__ float sumsq2(float a, float b) {
#pragma clang fp contract(off)
    return a * a + b * b;
}
// ((a*a + b*b) + c*c) + d*d
__device__ __forceinline__ float sumsq4(float a, float b, float c, float d) {
#pragma clang fp contract(off)
    return a * a + b * b + c * c + d * d;
}
// a*b + c, the product rounded before the sum
__device__ __forceinline__ float mul_add(float a, float b, float c) {
#pragma clang fp contract(off)
    return a * b + c;
}
// RoPE of one (x0, x1) pair of a head (ops_scalar.c:21-35):
//   o0 = y0 cos - y1 sin,  o1 = y1 cos + y0 sin
__device__ __forceinline__ void rope_pair(float y0, float y1, float c, float sn, float &o0, float &o1) {
#pragma clang fp contract(off)
    o0 = y0 * c - y1 * sn;
    o1 = y1 * c + y0 * sn;
}

#endif
