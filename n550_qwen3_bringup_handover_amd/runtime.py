"""Loader for libqwen3_hip.so — the MI355X GEMM plug-in and device-resident
forward (C ABI in include/qwen3_hip.h and include/qwen3_hip_model.h).

The library is built in-tree (`build()`, or `make -C <pkg>/csrc`) and loaded
from this directory only.  There is no CPU fallback: if the library is
missing or no gfx950 device is visible, the calls fail with an exception.
"""
import ctypes
import os
import subprocess

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_PATH = os.path.join(PKG_DIR, "libqwen3_hip.so")
HEADER = os.path.join(os.path.dirname(PKG_DIR), "include", "qwen3_hip.h")
MODEL_HEADER = os.path.join(os.path.dirname(PKG_DIR), "include", "qwen3_hip_model.h")
HEADERS = (HEADER, MODEL_HEADER)

F32P = ctypes.POINTER(ctypes.c_float)
U16P = ctypes.POINTER(ctypes.c_uint16)
I32P = ctypes.POINTER(ctypes.c_int)
VP = ctypes.c_void_p

_lib = None


class Qwen3HipError(RuntimeError):
    pass


def gpu_visible():
    """True when a GPU device node is present (does not initialise HIP)."""
    return os.path.exists("/dev/kfd")


def build(jobs=4):
    """Compile libqwen3_hip.so for gfx950 (hipcc cross-compiles without a GPU)."""
    subprocess.run(["make", "-s", f"-j{jobs}", "-C", CSRC], check=True)


# name -> (restype, argtypes), mirroring include/qwen3_hip.h
_PROTOS = {
    "qwen3_gemm": (None, [F32P, F32P, U16P, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "qwen3_gemm_row": (None, [F32P, F32P, U16P, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "qwen3_set_weight_layout": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "qwen3_kernel_name": (ctypes.c_char_p, []),
    "qwen3_gemm_gate_up_silu": (None, [F32P, F32P, U16P, U16P, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "qwen3_hip_init": (ctypes.c_int, [ctypes.c_int]),
    "qwen3_hip_release": (None, []),
    "qwen3_hip_last_error": (ctypes.c_int, []),
    "qwen3_hip_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "qwen3_hip_set_abort": (None, [ctypes.c_int]),
    "qwen3_hip_map_weights": (ctypes.c_int, [VP, ctypes.c_size_t]),
    "qwen3_hip_unmap_weights": (ctypes.c_int, [VP]),
    "qwen3_hip_forget_weights": (None, [VP]),
    "qwen3_hip_set_weight_cache": (None, [ctypes.c_int]),
    "qwen3_hip_weight_bytes": (ctypes.c_size_t, []),
    "qwen3_hip_gemm_dev": (ctypes.c_int, [VP, VP, VP, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "qwen3_hip_gemm_gate_up_silu_dev": (ctypes.c_int, [VP, VP, VP, VP, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "qwen3_hip_gemm_noalloc_dev": (ctypes.c_int, [VP, VP, VP, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "qwen3_hip_scratch_bytes": (ctypes.c_size_t, []),
    "qwen3_hip_gemm_bf16a_dev": (ctypes.c_int, [VP, VP, VP, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "qwen3_hip_gemm_gate_up_silu_bf16a_dev": (ctypes.c_int, [VP, VP, VP, VP, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "qwen3_hip_decode_set_dev": (ctypes.c_int, [ctypes.POINTER(VP), VP, VP, ctypes.c_int]),
    "qwen3_hip_decode_set_supported": (ctypes.c_int, []),
    "qwen3_hip_decode_set_out_ld": (ctypes.c_int, []),
    "qwen3_hip_decode_set_errors": (ctypes.c_int, [ctypes.POINTER(ctypes.c_uint)]),
    "qwen3_hip_argmax_dev": (ctypes.c_int, [VP, VP, ctypes.c_int]),
    "qwen3_hip_tile_to_row_dev": (ctypes.c_int, [VP, VP, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "qwen3_hip_copy_dev": (ctypes.c_int, [VP, VP, ctypes.c_size_t]),
    "qwen3_hip_read_dev": (ctypes.c_int, [VP, ctypes.c_size_t]),
    "qwen3_hip_capture_begin": (ctypes.c_int, []),
    "qwen3_hip_capture_end": (ctypes.c_int, [I32P]),
    "qwen3_hip_graph_launch": (ctypes.c_int, [ctypes.c_int]),
    "qwen3_hip_graph_destroy": (ctypes.c_int, [ctypes.c_int]),
    "qwen3_hip_malloc": (ctypes.c_int, [ctypes.POINTER(VP), ctypes.c_size_t]),
    "qwen3_hip_free": (ctypes.c_int, [VP]),
    "qwen3_hip_memcpy_h2d": (ctypes.c_int, [VP, VP, ctypes.c_size_t]),
    "qwen3_hip_memcpy_d2h": (ctypes.c_int, [VP, VP, ctypes.c_size_t]),
    "qwen3_hip_sync": (ctypes.c_int, []),
    "qwen3_hip_timer_record": (ctypes.c_int, [ctypes.c_int]),
    "qwen3_hip_timer_elapsed_ms": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, F32P]),
    "qwen3_hip_plan": (ctypes.c_char_p, [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "qwen3_hip_force_plan": (ctypes.c_int, [ctypes.c_int]),
    "qwen3_hip_last_plan": (ctypes.c_char_p, []),
    "qwen3_hip_device_name": (ctypes.c_char_p, []),
    # include/qwen3_hip_model.h
    "qwen3_hip_qw3m_size": (ctypes.c_size_t, [ctypes.c_int]),
    "qwen3_hip_qw3m_write_random": (ctypes.c_int, [VP, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_int, ctypes.c_int]),
    "qwen3_hip_qw3m_check": (ctypes.c_int, [VP, ctypes.c_size_t]),
    "qwen3_hip_model_open": (ctypes.c_int, [ctypes.POINTER(VP), VP, ctypes.c_size_t, ctypes.c_int]),
    "qwen3_hip_model_close": (None, [VP]),
    "qwen3_hip_model_max_seq": (ctypes.c_int, [VP]),
    "qwen3_hip_model_forward": (ctypes.c_int, [VP, I32P, ctypes.c_int, ctypes.c_int]),
    "qwen3_hip_model_logits": (ctypes.c_int, [VP, F32P]),
    "qwen3_hip_model_argmax": (ctypes.c_int, [VP, I32P]),
    "qwen3_hip_model_generate": (ctypes.c_int, [VP, I32P, ctypes.c_int, ctypes.c_int, ctypes.c_int, I32P, I32P]),
    "qwen3_hip_model_timing": (ctypes.c_int, [VP, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]),
    "qwen3_hip_model_set_graph": (ctypes.c_int, [VP, ctypes.c_int]),
    "qwen3_hip_model_set_persistent": (ctypes.c_int, [VP, ctypes.c_int]),
    "qwen3_hip_model_persistent": (ctypes.c_int, [VP]),
    "qwen3_hip_model_persist_errors": (ctypes.c_int, [VP, ctypes.POINTER(ctypes.c_uint)]),
    "qwen3_hip_model_set_dump": (ctypes.c_int, [VP, VP, VP]),
    "qwen3_hip_batch_open": (ctypes.c_int, [ctypes.POINTER(VP), VP, ctypes.c_int, ctypes.c_int]),
    "qwen3_hip_batch_close": (None, [VP]),
    "qwen3_hip_batch_prefill": (ctypes.c_int, [VP, ctypes.c_int, I32P, ctypes.c_int]),
    "qwen3_hip_batch_decode": (ctypes.c_int, [VP, ctypes.c_int, I32P]),
    "qwen3_hip_batch_logits": (ctypes.c_int, [VP, F32P]),
    "qwen3_hip_batch_set_graph": (ctypes.c_int, [VP, ctypes.c_int]),
    "qwen3_hip_batch_timing": (ctypes.c_int, [VP, ctypes.POINTER(ctypes.c_double)]),
}

# qwen3_hip_dump_fn
DUMP_FN = ctypes.CFUNCTYPE(None, VP, ctypes.c_int, ctypes.c_char_p, F32P, ctypes.c_size_t)


def header_symbols():
    """Function names declared in include/qwen3_hip.h and qwen3_hip_model.h."""
    import re
    names = set()
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
        names.update(re.findall(r"\b(qwen3_\w+)\s*\(", text))
    return sorted(names)


def lib():
    """The loaded library (built first if it is not there yet)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _PROTOS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc, what="qwen3_hip"):
    if rc:
        L = lib()
        raise Qwen3HipError(f"{what}: {L.qwen3_hip_strerror(rc).decode()} (code {rc})")
    return rc


def init(device=-1):
    """Initialise the library on a device (raises without a gfx950 GPU)."""
    L = lib()
    L.qwen3_hip_set_abort(0)
    check(L.qwen3_hip_init(device), "qwen3_hip_init")
    return L
