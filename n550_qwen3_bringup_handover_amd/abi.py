"""Python mirror of the C plug-in ABI (include/qwen3_hip.h), over ctypes.

Names, argument meaning and error behaviour follow the reference plug-in
(fpga_bringup/src/src/kernels.h:44-92): `gemm(c, a, b, M, K, N)` overwrites
c = a . b^T with a fp32 [M,K], b bf16 bits [N,K], c fp32 [M,N].  The helpers
here only adapt numpy arrays to pointers; all arithmetic happens in
libqwen3_hip.so on the GPU.
"""
import ctypes

import numpy as np

from . import runtime
from .runtime import F32P, U16P, VP, check


def _f32(x, name):
    if not (isinstance(x, np.ndarray) and x.dtype == np.float32 and x.flags.c_contiguous):
        raise TypeError(f"{name} must be a C-contiguous float32 array")
    return x


def _u16(x, name):
    if not (isinstance(x, np.ndarray) and x.dtype == np.uint16 and x.flags.c_contiguous):
        raise TypeError(f"{name} must be a C-contiguous uint16 (bf16 bits) array")
    return x


def _need(arr, n, name):
    if arr.size < n:
        raise ValueError(f"{name} holds {arr.size} elements, needs {n}")


def kernel_name():
    return runtime.lib().qwen3_kernel_name().decode()


def set_weight_layout(layout, tile_n=128, tile_k=32):
    return int(runtime.lib().qwen3_set_weight_layout(layout, tile_n, tile_k))


def last_error():
    return int(runtime.lib().qwen3_hip_last_error())


def _host_call(fn, c, a, bs, M, K, N):
    _need(c, M * N, "c")
    _need(a, M * K, "a")
    for i, b in enumerate(bs):
        _need(b, N * K, f"b{i}")
    L = runtime.lib()
    L.qwen3_hip_set_abort(0)
    L.qwen3_hip_last_error()
    fn(c.ctypes.data_as(F32P), a.ctypes.data_as(F32P),
       *[b.ctypes.data_as(U16P) for b in bs], M, K, N)
    check(L.qwen3_hip_last_error(), fn.__name__)
    return c


def gemm(c, a, b, M, K, N):
    """qwen3_gemm: c[M,N] = a[M,K] . b[N,K]^T in the current weight layout."""
    L = runtime.lib()
    return _host_call(L.qwen3_gemm, _f32(c, "c"), _f32(a, "a"), [_u16(b, "b")], M, K, N)


def gemm_row(c, a, b, M, K, N):
    """qwen3_gemm_row: as gemm, with b always row-major."""
    L = runtime.lib()
    return _host_call(L.qwen3_gemm_row, _f32(c, "c"), _f32(a, "a"), [_u16(b, "b")], M, K, N)


def gemm_gate_up_silu(h, x, wg, wu, M, K, N):
    """h = silu(x . wg^T) * (x . wu^T)."""
    L = runtime.lib()
    return _host_call(L.qwen3_gemm_gate_up_silu, _f32(h, "h"), _f32(x, "x"),
                      [_u16(wg, "wg"), _u16(wu, "wu")], M, K, N)


def map_weights(blob):
    """Upload a whole weight blob once (a numpy array kept alive by the caller)."""
    L = runtime.init()
    check(L.qwen3_hip_map_weights(ctypes.c_void_p(blob.ctypes.data), blob.nbytes),
          "qwen3_hip_map_weights")


def unmap_weights(blob):
    check(runtime.lib().qwen3_hip_unmap_weights(ctypes.c_void_p(blob.ctypes.data)),
          "qwen3_hip_unmap_weights")


class DeviceBuffer:
    """A block of device memory owned by Python (freed on close/GC)."""

    def __init__(self, nbytes):
        L = runtime.init()
        p = VP()
        check(L.qwen3_hip_malloc(ctypes.byref(p), int(nbytes)), "qwen3_hip_malloc")
        self.ptr = p.value
        self.nbytes = int(nbytes)

    @classmethod
    def from_array(cls, arr):
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr)
        return buf

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        if arr.nbytes > self.nbytes:
            raise ValueError("array larger than the device buffer")
        L = runtime.lib()
        check(L.qwen3_hip_memcpy_h2d(VP(self.ptr), VP(arr.ctypes.data), arr.nbytes), "h2d")
        check(L.qwen3_hip_sync(), "sync")

    def download(self, dtype, count):
        out = np.empty(int(count), dtype=dtype)
        if out.nbytes > self.nbytes:
            raise ValueError("download larger than the device buffer")
        L = runtime.lib()
        check(L.qwen3_hip_memcpy_d2h(VP(out.ctypes.data), VP(self.ptr), out.nbytes), "d2h")
        check(L.qwen3_hip_sync(), "sync")
        return out

    def close(self):
        if self.ptr:
            runtime.lib().qwen3_hip_free(VP(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def gemm_dev(c_d, a_d, b_d, M, K, N):
    check(runtime.lib().qwen3_hip_gemm_dev(VP(c_d), VP(a_d), VP(b_d), M, K, N), "qwen3_hip_gemm_dev")


def gemm_gate_up_silu_dev(h_d, x_d, wg_d, wu_d, M, K, N):
    check(runtime.lib().qwen3_hip_gemm_gate_up_silu_dev(VP(h_d), VP(x_d), VP(wg_d), VP(wu_d), M, K, N),
          "qwen3_hip_gemm_gate_up_silu_dev")


def gemm_bf16a_dev(c_d, a_d, b_d, M, K, N):
    """C = A.B^T with A already bf16 bits on the device (K % 64 == 0)."""
    check(runtime.lib().qwen3_hip_gemm_bf16a_dev(VP(c_d), VP(a_d), VP(b_d), M, K, N),
          "qwen3_hip_gemm_bf16a_dev")


def gemm_gate_up_silu_bf16a_dev(h_d, x_d, wg_d, wu_d, M, K, N):
    check(runtime.lib().qwen3_hip_gemm_gate_up_silu_bf16a_dev(VP(h_d), VP(x_d), VP(wg_d), VP(wu_d),
                                                              M, K, N),
          "qwen3_hip_gemm_gate_up_silu_bf16a_dev")


def argmax_dev(out_d, v_d, n):
    check(runtime.lib().qwen3_hip_argmax_dev(VP(out_d), VP(v_d), n), "qwen3_hip_argmax_dev")


def sync():
    check(runtime.lib().qwen3_hip_sync(), "qwen3_hip_sync")


def plan(M, K, N, gated=False):
    return runtime.lib().qwen3_hip_plan(M, K, N, int(gated)).decode()


def force_plan(plan_id):
    check(runtime.lib().qwen3_hip_force_plan(plan_id), "qwen3_hip_force_plan")


# plan ids of csrc/hip_gemm.hip (qwen3_hip_force_plan); checked against the
# library's own names by tests/test_abi_cpu.py
PLANS = {"auto": 0, "gemv": 1, "mfma128x128": 2, "mfma64x128": 3, "mfma64x64": 4,
         "mfma32x128": 5, "mfma16x64": 6, "mfma64x64-scalar": 7,
         "pipe32x64k128s4": 8, "pipe32x64k64s4": 9, "pipe64x64k64s3": 10,
         "xl128x128": 11, "xl256x256": 12, "xl64x128": 13,
         "xb256x256k32": 14, "xb128x128": 15, "xb256x256s1": 16,
         "stream": 17, "stream-ks1": 18, "stream-ks2": 19, "stream-ks4": 20, "stream-ks8": 21,
         "skinny": 22, "narrow": 23, "wide": 24, "gemv16": 25, "xl64x64s3": 26, "m16": 27}


def last_plan():
    """the plan the last GEMM call launched (after any fall-back)"""
    return runtime.lib().qwen3_hip_last_plan().decode()
