#!/usr/bin/env python3
"""Write the small golden fixtures under tests/golden/ (run in the build
container, where the reference tree and oracle/_ref exist).

Two kinds of data are written, both plain arrays (.npz, no pickles):

1. rtl_<case>.npz — the reference's shipped AME golden vectors
   (rtl_verification/cases/<case>/{a,b,a_src,c_ref,c_peak,xor_ref}.bin),
   unpacked from their row-strided memory images into dense [M,K] / [N,K]
   arrays, plus the shape, strides and acceptance tolerance from meta.json.
2. scalar_ref.npz / ops_ref.npz — outputs of the reference's own portable C
   (fpga_bringup/src/src/kernels_scalar.c, kernels_hwsim.c, ops_scalar.c),
   compiled from its sources by `make -C oracle ref`, on seeded inputs made
   by the oracle's RNG.

Nothing here is imported by the product or by GPU runs; tests read only the
.npz files.
"""
import ctypes
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF_RTL = "/root/reference/rtl_verification/cases"
REF_LIB = os.path.join(ROOT, "oracle", "_ref")
ORACLE = os.path.join(ROOT, "oracle", "liboracle.so")

# cases 001-008 carry bf16 A; 009a-011 carry fp32 a_src (A = RNE-bf16 of it)
RTL_CASES = ["001_bf16_full_tile", "002_m1_gemv", "003_partial_m",
             "004_k_multiblock", "005_partial_n", "006_partial_k",
             "007_stride_gap", "008_massive_act", "009a_rvv_ame_handoff_cbo",
             "010_sync_sensitivity", "011_fence_ordering"]

F32P = ctypes.POINTER(ctypes.c_float)
U16P = ctypes.POINTER(ctypes.c_uint16)


def _p(arr, typ):
    return arr.ctypes.data_as(typ)


def write_rtl():
    for name in RTL_CASES:
        d = os.path.join(REF_RTL, name)
        meta = json.load(open(os.path.join(d, "meta.json"), encoding="utf-8"))
        M, N, K = meta["shape"]["M"], meta["shape"]["N"], meta["shape"]["K"]
        out = {"M": M, "N": N, "K": K, "norm_tol": meta["norm_tol"]}
        if os.path.exists(os.path.join(d, "a.bin")):
            sa = meta["stride_elems"]["a"]
            sb = meta["stride_elems"]["b"]
            a = np.fromfile(os.path.join(d, "a.bin"), dtype="<u2")
            b = np.fromfile(os.path.join(d, "b.bin"), dtype="<u2")
            out["a_bf16"] = a.reshape(M, sa)[:, :K].copy()
            out["b_bf16"] = b.reshape(N, sb)[:, :K].copy()
        else:
            a_src = np.fromfile(os.path.join(d, "a_src.bin"), dtype="<f4")
            b = np.fromfile(os.path.join(d, "b.bin"), dtype="<u2")
            out["a_src"] = a_src.reshape(M, K).copy()
            out["b_bf16"] = b.reshape(N, K).copy()
            out["xor_ref"] = np.uint32(int(meta["xor_ref"], 16))
        c_ref = np.fromfile(os.path.join(d, "c_ref.bin"), dtype="<u4")
        c_peak = np.fromfile(os.path.join(d, "c_peak.bin"), dtype="<f4")
        out["c_ref_bits"] = c_ref.reshape(M, N)
        out["c_peak"] = c_peak.reshape(M, N)
        np.savez_compressed(os.path.join(HERE, f"rtl_{name.split('_')[0]}.npz"), **out)
        print("wrote rtl", name, M, N, K)


def write_scalar_and_ops():
    orc = ctypes.CDLL(ORACLE)
    scal = ctypes.CDLL(os.path.join(REF_LIB, "libref_scalar.so"))
    hw = ctypes.CDLL(os.path.join(REF_LIB, "libref_hwsim.so"))
    ops = ctypes.CDLL(os.path.join(REF_LIB, "libref_ops.so"))
    ops.qwen3_op_argmax.restype = ctypes.c_int

    shapes = [(1, 1024, 64), (4, 1024, 48), (16, 1024, 32), (8, 33, 128),
              (3, 17, 13), (2, 3072, 16), (7, 64, 129)]
    store = {}
    for i, (M, K, N) in enumerate(shapes):
        seed_a = 0x03550000 + 16 * 90 + 2 * i
        a = np.empty(M * K, np.float32)
        b = np.empty(N * K, np.uint16)
        orc.orc_fill_f32_bf16_normal(_p(a, F32P), ctypes.c_size_t(a.size),
                                     ctypes.c_uint64(seed_a), ctypes.c_float(1.0))
        orc.orc_fill_bf16_normal(_p(b, U16P), ctypes.c_size_t(b.size),
                                 ctypes.c_uint64(seed_a + 1), ctypes.c_float(0.02))
        # fp32 activations that are NOT bf16-representable, to pin the
        # scalar kernel's use of A as given and hwsim's rounding of it
        a_raw = (a + np.float32(1e-3) * np.sin(np.arange(a.size, dtype=np.float32))).astype(np.float32)
        c_s = np.empty(M * N, np.float32)
        c_h = np.empty(M * N, np.float32)
        c_sr = np.empty(M * N, np.float32)
        c_hr = np.empty(M * N, np.float32)
        scal.qwen3_gemm(_p(c_s, F32P), _p(a, F32P), _p(b, U16P), M, K, N)
        hw.qwen3_gemm(_p(c_h, F32P), _p(a, F32P), _p(b, U16P), M, K, N)
        scal.qwen3_gemm(_p(c_sr, F32P), _p(a_raw, F32P), _p(b, U16P), M, K, N)
        hw.qwen3_gemm(_p(c_hr, F32P), _p(a_raw, F32P), _p(b, U16P), M, K, N)
        key = f"{M}x{K}x{N}"
        store[f"{key}_a"] = a.reshape(M, K)
        store[f"{key}_araw"] = a_raw.reshape(M, K)
        store[f"{key}_b"] = b.reshape(N, K)
        store[f"{key}_c_scalar"] = c_s.reshape(M, N)
        store[f"{key}_c_hwsim"] = c_h.reshape(M, N)
        store[f"{key}_craw_scalar"] = c_sr.reshape(M, N)
        store[f"{key}_craw_hwsim"] = c_hr.reshape(M, N)
    store["shapes"] = np.array(shapes, dtype=np.int32)
    np.savez_compressed(os.path.join(HERE, "scalar_ref.npz"), **store)
    print("wrote scalar_ref.npz")

    # silu_mul and argmax on values covering the special cases
    rng = np.random.default_rng(1234)
    g = np.concatenate([rng.standard_normal(4000).astype(np.float32) * 4,
                        np.array([0.0, -0.0, 1e-30, -1e-30, 20.0, -20.0, 88.0,
                                  -88.0, 100.0, -100.0, 1e4, -1e4], np.float32)])
    u = rng.standard_normal(g.size).astype(np.float32)
    h = g.copy()
    ops.qwen3_op_silu_mul(_p(h, F32P), _p(u, F32P), g.size)
    v = rng.standard_normal(20000).astype(np.float32)
    v[777] = 9.0
    v[19000] = 9.0          # tie: the lower index must win
    am = ops.qwen3_op_argmax(_p(v, F32P), v.size)
    np.savez_compressed(os.path.join(HERE, "ops_ref.npz"), gate=g, up=u,
                        silu_mul=h, argmax_in=v, argmax=np.int64(am))
    print("wrote ops_ref.npz, argmax =", am)


if __name__ == "__main__":
    if not os.path.isdir(REF_RTL):
        sys.exit("reference tree not present: fixtures are generated in the build container only")
    write_rtl()
    write_scalar_and_ops()
