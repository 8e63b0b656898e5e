"""ctypes binding of the CPU oracle (oracle/liboracle.so) — TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker.  The product library never loads it.

`ref()` additionally opens the reference's own portable C compiled into
oracle/_ref/ (the "ref" target of oracle/Makefile), when that was built.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_DIR = os.path.join(HERE, "_ref")

F32P = ctypes.POINTER(ctypes.c_float)
F64P = ctypes.POINTER(ctypes.c_double)
U16P = ctypes.POINTER(ctypes.c_uint16)
I32P = ctypes.POINTER(ctypes.c_int)

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.orc_bf16_to_f32.restype = ctypes.c_float
        L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        for fn in ("orc_f32_to_bf16", "orc_f32_to_bf16_hw", "orc_f32_to_bf16_fpu"):
            getattr(L, fn).restype = ctypes.c_uint16
            getattr(L, fn).argtypes = [ctypes.c_float]
        L.orc_bf16_rne_selfcheck.restype = ctypes.c_uint64
        L.orc_bf16_rne_selfcheck.argtypes = [U16P, ctypes.c_int]
        L.orc_argmax.restype = ctypes.c_int
        L.orc_tile_offset.restype = ctypes.c_size_t
        L.orc_tile_offset.argtypes = [ctypes.c_int] * 5
        L.orc_splitmix64.restype = ctypes.c_uint64
        L.orc_splitmix64.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        L.orc_now_seconds.restype = ctypes.c_double
        _lib = L
    return _lib


def _p(arr, typ):
    return arr.ctypes.data_as(typ)


def _f32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def _u16(x):
    return np.ascontiguousarray(x, dtype=np.uint16)


# ---- inputs -----------------------------------------------------------------

def bf16_normal(n, seed, sigma):
    """bf16 bit patterns of sigma*N(0,1) (SplitMix64 + Box-Muller, RNE)."""
    out = np.empty(int(n), np.uint16)
    lib().orc_fill_bf16_normal(_p(out, U16P), ctypes.c_size_t(out.size),
                               ctypes.c_uint64(seed), ctypes.c_float(sigma))
    return out


def f32_bf16_normal(n, seed, sigma=1.0):
    """sigma*N(0,1) rounded to bf16, widened back: exactly bf16-representable fp32."""
    out = np.empty(int(n), np.float32)
    lib().orc_fill_f32_bf16_normal(_p(out, F32P), ctypes.c_size_t(out.size),
                                   ctypes.c_uint64(seed), ctypes.c_float(sigma))
    return out


def test_lcg(n, state):
    """The reference unit test's LCG (fpga_bringup/src/src/test_kernels.c:31-35)."""
    out = np.empty(int(n), np.float32)
    st = ctypes.c_uint32(state)
    lib().orc_test_lcg_fill(_p(out, F32P), ctypes.c_size_t(out.size), ctypes.byref(st))
    return out, st.value


# ---- conversions --------------------------------------------------------------

def f32_to_bf16(x):
    x = _f32(x).ravel()
    out = np.empty(x.size, np.uint16)
    lib().orc_f32_to_bf16_array(_p(out, U16P), _p(x, F32P), ctypes.c_size_t(x.size))
    return out


def bf16_to_f32(h):
    h = _u16(h).ravel()
    out = np.empty(h.size, np.float32)
    lib().orc_bf16_to_f32_array(_p(out, F32P), _p(h, U16P), ctypes.c_size_t(h.size))
    return out


def round_bf16(x):
    x = _f32(x)
    out = np.empty_like(x)
    lib().orc_round_bf16_f32(_p(out, F32P), _p(x, F32P), ctypes.c_size_t(x.size))
    return out


# ---- GEMM semantics ----------------------------------------------------------

def gemm_scalar(a, b, M, K, N, cols=None):
    """Reference scalar GEMM (kernels_scalar.c:9-21); a fp32 [M,K], b bf16 [N,K]."""
    a, b = _f32(a), _u16(b)
    c = np.zeros(M * N, np.float32)
    n0, n1 = (0, N) if cols is None else cols
    lib().orc_gemm_scalar_cols(_p(c, F32P), _p(a, F32P), _p(b, U16P), M, K, N, n0, n1)
    return c.reshape(M, N)


def gemm_hw16(a, b, M, K, N):
    a, b = _f32(a), _u16(b)
    c = np.empty(M * N, np.float32)
    lib().orc_gemm_hw16(_p(c, F32P), _p(a, F32P), _p(b, U16P), M, K, N)
    return c.reshape(M, N)


def gemm_exact(a, b, M, K, N):
    """(fp64 C, sum_k |a*b|) for the normalised error metric."""
    a, b = _f32(a), _u16(b)
    c = np.empty(M * N, np.float64)
    s = np.empty(M * N, np.float64)
    lib().orc_gemm_exact(_p(c, F64P), _p(s, F64P), _p(a, F32P), _p(b, U16P), M, K, N)
    return c.reshape(M, N), s.reshape(M, N)


def silu_mul(gate, up):
    g = _f32(gate).copy()
    u = _f32(up)
    lib().orc_silu_mul(_p(g, F32P), _p(u, F32P), g.size)
    return g


def argmax(v):
    v = _f32(v)
    return int(lib().orc_argmax(_p(v, F32P), v.size))


def gate_up_silu(x, wg, wu, M, K, N):
    x, wg, wu = _f32(x), _u16(wg), _u16(wu)
    h = np.empty(M * N, np.float32)
    lib().orc_gate_up_silu(_p(h, F32P), _p(x, F32P), _p(wg, U16P), _p(wu, U16P), M, K, N)
    return h.reshape(M, N)


def tile_offset(n, k, K, tile_n=128, tile_k=32):
    return int(lib().orc_tile_offset(n, k, K, tile_n, tile_k))


def row_to_tile(b, N, K, tile_n=128, tile_k=32):
    b = _u16(b)
    out = np.zeros(N * K, np.uint16)
    lib().orc_row_to_tile(_p(out, U16P), _p(b, U16P), N, K, tile_n, tile_k)
    return out


def now():
    return float(lib().orc_now_seconds())


# ---- the reference's own compiled C (oracle/_ref), when present --------------

def hw16mt():
    """ctypes handle of oracle/libhw16mt.so: this directory's threaded
    restatement of kernels_hwsim.c (symbol qwen3_gemm), built on demand"""
    path = os.path.join(HERE, "libhw16mt.so")
    if not os.path.exists(path):
        subprocess.run(["make", "-s", "-C", HERE, "libhw16mt.so"], check=True)
    return ctypes.CDLL(path)


def ref(name):
    """ctypes handle of oracle/_ref/lib<name>.so, or None if it was not built."""
    path = os.path.join(REF_DIR, f"lib{name}.so")
    if not os.path.exists(path):
        return None
    L = ctypes.CDLL(path)
    return L


def ref_gemm(L, a, b, M, K, N):
    a, b = _f32(a), _u16(b)
    c = np.empty(M * N, np.float32)
    L.qwen3_gemm(_p(c, F32P), _p(a, F32P), _p(b, U16P), M, K, N)
    return c.reshape(M, N)
