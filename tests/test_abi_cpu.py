"""The C-ABI library on a machine without a GPU: it builds, loads, exports
every symbol include/qwen3_hip.h declares, and its host-only logic (layout
negotiation, argument checks, error reporting) behaves like the reference
plug-in.  No call here reaches a GPU kernel."""
import ctypes
import os
import subprocess
import sys
import textwrap

import numpy as np
import pytest

from n550_qwen3_bringup_handover_amd import abi, runtime

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_header_symbol():
    L = runtime.lib()
    names = runtime.header_symbols()
    # the four reference plug-in symbols (fpga_bringup/src/src/kernels.h:56-92)
    for ref in ("qwen3_gemm", "qwen3_gemm_row", "qwen3_set_weight_layout", "qwen3_kernel_name"):
        assert ref in names
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # and every declared function has a ctypes prototype in runtime.py
    assert set(names) <= set(runtime._PROTOS), set(names) - set(runtime._PROTOS)


def test_library_links_only_the_hip_runtime():
    out = subprocess.run(["ldd", runtime.LIB_PATH], capture_output=True, text=True).stdout
    assert "libamdhip64" in out
    for bad in ("libtorch", "libcuda", "liboracle", "libref_"):
        assert bad not in out


def test_kernel_name():
    assert abi.kernel_name() == "hip-gfx950"


H, Q, KV, I, V = 1024, 2048, 1024, 3072, 151936


@pytest.mark.parametrize("M,K,N,gated,plan", [
    (1, H, Q + 2 * KV, False, "gemv"), (1, Q, H, False, "gemv"), (1, H, V, False, "gemv"),
    (16, H, I, False, "m16"),                                     # gate_proj at M = 16
    (64, H, V, False, "wide"),                                    # lm_head of a 64-sequence batch
    (32, H, V, False, "wide"), (8, H, V, False, "wide"), (64, 2048, V, False, "stream"),
    (4096, H, Q + 2 * KV, False, "xl256x256"), (8192, H, Q + 2 * KV, False, "xb256x256s1"),
    (64, Q, H, False, "narrow"), (64, I, H, False, "narrow"),     # o, down at M = 64
    (16, I, H, False, "m16"), (32, H, Q, False, "narrow"),
    (8, H, I, False, "m16"), (16, H, H, False, "m16"), (4, H, I, False, "m16"), (2, H, Q, False, "m16"),
    (8, Q, H, False, "m16"), (8, I, H, False, "m16"), (12, I, H, False, "m16"), (16, H, 16384, False, "m16"),
    (4, Q, H, False, "m16"), (2, Q, H, False, "gemv"), (8, H, I, True, "m16"), (2, H, 2048, True, "gemv"),
    (16, H, 8192, True, "pipe32x64k128s4"), (1, H, I, True, "gemv"), (4, Q, Q, True, "gemv"), (5, Q, Q, True, "m16"), (16, I, H, True, "pipe32x64k128s4"), (2, Q, I, False, "m16"), (2, I, 8192, False, "gemv"),
    (16, Q, 16384, False, "stream"), (8, I, I, False, "m16"), (16, 3072 + 64, H, False, "skinny"), (16, H, 32768, False, "wide"), (16, H, I, True, "m16"),
    (128, H, KV, False, "narrow"), (128, H, Q, False, "narrow"), (128, Q, H, False, "narrow"),   # M = 128 prefill
    (128, I, H, False, "narrow"), (256, H, KV, False, "narrow"), (256, Q, H, False, "pipe32x64k128s4"),
    (128, H, I, True, "pipe32x64k64s4"), (160, H, Q, False, "pipe32x64k128s4"),
    (256, H, I, True, "xl64x128"), (256, H, Q + 2 * KV, False, "xl64x64s3"), (1024, H, Q, False, "xl64x128"),
    (2048, I, H, False, "xl64x128"), (384, H, Q + 2 * KV, False, "xl64x128"),
    (768, H, Q + 2 * KV, False, "xl128x128"), (2048, H, I, True, "xl256x256"), (4096, H, I, True, "xb128x128"),
    (64, H, Q + 2 * KV, False, "narrow"), (64, H, I, True, "pipe32x64k128s4"),   # q|k|v, gate|up
    (64, H, Q, False, "narrow"), (128, H, Q + 2 * KV, False, "pipe32x64k128s4"),
    (512, H, Q + 2 * KV, False, "xl64x128"), (512, H, I, True, "xl128x128"),
    (512, H, Q, False, "xl64x64s3"), (512, I, H, False, "pipe32x64k128s4"), (512, H, KV, False, "pipe32x64k128s4"),
    (1024, H, KV, False, "xl64x64s3"), (2048, H, KV, False, "xl64x128"),
    (1024, I, H, False, "xl64x64s3"), (2048, Q, H, False, "xl64x128"), (4096, I, H, False, "xl128x128"),
    (8, 33, 128, False, "mfma64x64-scalar"),                      # K % 8 != 0: element-wise loads
])
def test_automatic_plan_table(M, K, N, gated, plan):
    """The automatic kernel choice for the Qwen3-0.6B shapes is host logic
    (measured on MI355X and fixed in the library); it needs no device."""
    assert abi.plan(M, K, N, gated) == plan


def test_plan_ids_match_the_library():
    """abi.PLANS (the ids tests force) names the library's own plans: a
    forced plan is what qwen3_hip_plan reports, with no device needed."""
    try:
        for name, pid in abi.PLANS.items():
            abi.force_plan(pid)
            assert abi.plan(64, 1024, 1024) == (name if pid else abi.plan(64, 1024, 1024))
        with pytest.raises(runtime.Qwen3HipError):
            abi.force_plan(len(abi.PLANS))
    finally:
        abi.force_plan(0)


@pytest.mark.parametrize("layout,tn,tk,ok", [
    (0, 0, 0, True), (0, 128, 32, True),          # ROW ignores tile sizes (qwen3.c:67-73)
    (1, 128, 32, True),                           # the AME tile (kernels.h:20-23)
    (1, 64, 16, True), (1, 1024, 1024, True),     # any tile dividing all model dims
    (1, 100, 32, False), (1, 128, 33, False),     # 2048 % 100, 1024 % 33
    (1, 0, 32, False), (1, 128, -32, False),
    (2, 128, 32, False), (-1, 0, 0, False),       # unknown layout codes
])
def test_set_weight_layout(layout, tn, tk, ok):
    L = runtime.lib()
    try:
        assert (L.qwen3_set_weight_layout(layout, tn, tk) == 0) == ok
    finally:
        L.qwen3_set_weight_layout(0, 0, 0)


def test_strerror_table():
    L = runtime.lib()
    for code in range(9):
        assert L.qwen3_hip_strerror(code)
    assert L.qwen3_hip_strerror(99) == b"unknown error"


def test_invalid_arguments_are_reported_not_computed():
    """M < 0 is rejected before any device work; C is left untouched."""
    L = runtime.lib()
    L.qwen3_hip_set_abort(0)
    L.qwen3_hip_last_error()
    c = np.full(4, 7.0, np.float32)
    a = np.zeros(4, np.float32)
    b = np.zeros(4, np.uint16)
    L.qwen3_gemm(c.ctypes.data_as(runtime.F32P), a.ctypes.data_as(runtime.F32P),
                 b.ctypes.data_as(runtime.U16P), -1, 2, 2)
    assert L.qwen3_hip_last_error() == 1       # QWEN3_HIP_EINVAL
    assert np.all(c == 7.0)
    assert L.qwen3_hip_last_error() == 0       # cleared on read


def test_empty_shapes_are_no_ops_without_a_device():
    L = runtime.lib()
    L.qwen3_hip_set_abort(0)
    L.qwen3_hip_last_error()
    c = np.full(4, 7.0, np.float32)
    L.qwen3_gemm(c.ctypes.data_as(runtime.F32P), None, None, 0, 16, 4)
    L.qwen3_gemm(c.ctypes.data_as(runtime.F32P), None, None, 4, 16, 0)
    assert L.qwen3_hip_last_error() == 0
    assert np.all(c == 7.0)


def test_python_mirror_rejects_wrong_dtypes():
    with pytest.raises(TypeError):
        abi.gemm(np.zeros(4, np.float64), np.zeros(4, np.float32), np.zeros(4, np.uint16), 2, 2, 2)
    with pytest.raises(ValueError):
        abi.gemm(np.zeros(3, np.float32), np.zeros(4, np.float32), np.zeros(4, np.uint16), 2, 2, 2)


@pytest.mark.skipif(runtime.gpu_visible(), reason="checks the no-device path")
def test_no_device_is_a_clear_error():
    L = runtime.lib()
    L.qwen3_hip_set_abort(0)
    L.qwen3_hip_last_error()
    assert L.qwen3_hip_init(-1) == 2            # QWEN3_HIP_ENODEV
    with pytest.raises(runtime.Qwen3HipError):
        runtime.init()


def test_void_entry_points_abort_by_default():
    """The reference ABI cannot return an error, so by default a failure
    prints one line and aborts (checked in a child process)."""
    code = textwrap.dedent(f"""
        import ctypes, sys
        L = ctypes.CDLL({runtime.LIB_PATH!r})
        c = (ctypes.c_float * 4)()
        L.qwen3_gemm(c, c, None, -1, 2, 2)
        print("not reached")
    """)
    env = dict(os.environ)
    env.pop("QWEN3_HIP_ABORT", None)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env)
    assert r.returncode != 0
    assert "not reached" not in r.stdout
    assert "qwen3_gemm: invalid argument" in r.stderr
    env["QWEN3_HIP_ABORT"] = "0"
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env)
    assert r.returncode == 0 and "not reached" in r.stdout


def test_header_compiles_as_c_and_cpp(tmp_path):
    src = tmp_path / "t.c"
    src.write_text('#include "qwen3_hip.h"\nint main(void){return qwen3_kernel_name()[0]==\'h\'?0:1;}\n')
    inc = os.path.join(ROOT, "include")
    for cc, std in (("gcc", "-std=c11"), ("g++", "-std=c++17")):
        exe = tmp_path / f"t_{cc}"
        r = subprocess.run([cc, std, "-Wall", "-Werror", "-x", "c" if cc == "gcc" else "c++",
                            str(src), "-I", inc, "-x", "none", runtime.LIB_PATH, "-o", str(exe),
                            f"-Wl,-rpath,{os.path.dirname(runtime.LIB_PATH)}"],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr
        assert subprocess.run([str(exe)]).returncode == 0
