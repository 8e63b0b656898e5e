"""The persistent decode-set launch (qwen3_hip_decode_set_dev) on the GPU.

It runs the M = 1 GEMV set of L decoder layers (q|k|v, o on the q part,
gate|up with silu(gate) * up, down; the calls of
fpga_bringup/src/src/qwen3.c:477-540) as one launch whose workgroups exchange
activations through tagged memory words.  Its outputs must equal, bit for
bit, the same chain of per-call GEMV entry points (qwen3_hip_gemm_dev,
qwen3_hip_gemm_gate_up_silu_dev), which tests/test_gemm_gpu.py holds to the
CPU oracle; layer 0 is also compared with the oracle here directly.
Repeated launches (the tag advances) and graph replays must give the same
bits, with no exchange error flagged.
"""
import ctypes

import numpy as np
import pytest

import oracle
from n550_qwen3_bringup_handover_amd import abi, runtime
from tests import numerics

pytestmark = pytest.mark.gpu
VP = ctypes.c_void_p
H, QKV, Q, I = 1024, 4096, 2048, 3072
SHAPES = [(QKV, H), (H, Q), (I, H), (I, H), (H, I)]       # (rows, K) of q|k|v, o, gate, up, down


@pytest.fixture(scope="module")
def lib():
    L = runtime.init()
    if not L.qwen3_hip_decode_set_supported():
        pytest.skip("device cannot keep the persistent grid resident")
    return L


def bf16_weights(n, seed):
    """sigma 0.02 normal weights as bf16 bits (numpy RNG, RNE)"""
    x = np.random.default_rng(seed).standard_normal(n, dtype=np.float32) * np.float32(0.02)
    u = x.view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


class Layers:
    """device weights of `n` layers (distinct per layer), host copies kept for
    the first `keep` layers"""

    def __init__(self, n, seed, keep=1):
        self.bufs, self.host = [], []
        for l in range(n):
            row = []
            for k, (rows, K) in enumerate(SHAPES):
                w = bf16_weights(rows * K, seed + 10 * l + k)
                row.append(abi.DeviceBuffer.from_array(w))
                if l < keep:
                    self.host.append(w)
            self.bufs.append(row)
        self.table = (VP * (5 * n))(*[b.ptr for row in self.bufs for b in row])


def per_call_chain(L, layers, x0d, n):
    """the reference chain through the per-call entry points: per layer
    device buffers qkv, o, h, x"""
    outs = []
    x = x0d
    for l in range(n):
        wq, wo, wg, wu, wd = (b.ptr for b in layers.bufs[l])
        qkv, o, h, xn = (abi.DeviceBuffer(4 * v) for v in (QKV, H, I, H))
        runtime.check(L.qwen3_hip_gemm_dev(VP(qkv.ptr), VP(x.ptr), VP(wq), 1, H, QKV), "qkv")
        runtime.check(L.qwen3_hip_gemm_dev(VP(o.ptr), VP(qkv.ptr), VP(wo), 1, Q, H), "o")
        runtime.check(L.qwen3_hip_gemm_gate_up_silu_dev(VP(h.ptr), VP(o.ptr), VP(wg), VP(wu), 1, H, I), "gate_up")
        runtime.check(L.qwen3_hip_gemm_dev(VP(xn.ptr), VP(h.ptr), VP(wd), 1, I, H), "down")
        outs.append((qkv, o, h, xn))
        x = xn
    abi.sync()
    return [tuple(b.download(np.float32, v) for b, v in zip(t, (QKV, H, I, H))) for t in outs]


def run_persist(L, layers, x0d, n, outd):
    runtime.check(L.qwen3_hip_decode_set_dev(layers.table, VP(x0d.ptr), VP(outd.ptr), n), "decode_set")
    abi.sync()
    ld = L.qwen3_hip_decode_set_out_ld()
    return outd.download(np.float32, n * ld).reshape(n, ld)


def errors(L):
    f = ctypes.c_uint(0)
    runtime.check(L.qwen3_hip_decode_set_errors(ctypes.byref(f)), "decode_set_errors")
    return f.value


def split(row):
    return row[0:QKV], row[4096:4096 + H], row[5120:5120 + I], row[8192:8192 + H]


@pytest.mark.parametrize("n", [1, 3])
def test_decode_set_matches_per_call_chain(lib, n):
    print(f"decode set, {n} layers", flush=True)
    layers = Layers(n, 100 * n, keep=1)
    x0 = oracle.f32_bf16_normal(H, 31 + n, 1.0)
    x0d = abi.DeviceBuffer.from_array(x0)
    ld = lib.qwen3_hip_decode_set_out_ld()
    outd = abi.DeviceBuffer.from_array(np.full(n * ld, np.nan, np.float32))
    got = run_persist(lib, layers, x0d, n, outd)
    assert errors(lib) == 0
    want = per_call_chain(lib, layers, x0d, n)
    for l in range(n):
        for name, g, w in zip(("qkv", "o", "h", "down"), split(got[l]), want[l]):
            assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), (l, name)
    # layer 0 against the oracle directly, each GEMV on its device input
    wq, wo, wg, wu, wd = layers.host[:5]
    qkv, o, h, xd = split(got[0])
    numerics.compare(qkv, x0, wq, 1, H, QKV)
    numerics.compare(o, qkv[:Q].copy(), wo, 1, Q, H)
    numerics.compare_gated(h, o.copy(), wg, wu, 1, H, I)
    numerics.compare(xd, h.copy(), wd, 1, I, H)


def test_decode_set_28_layers_repeated_and_graph(lib):
    """the bench's depth: 28 layers, three eager launches and three graph
    replays, every one bit-identical to the per-call chain"""
    n = 28
    layers = Layers(n, 7000, keep=0)
    x0d = abi.DeviceBuffer.from_array(oracle.f32_bf16_normal(H, 77, 1.0))
    ld = lib.qwen3_hip_decode_set_out_ld()
    outd = abi.DeviceBuffer(n * ld * 4)
    want = per_call_chain(lib, layers, x0d, n)
    want_rows = [np.concatenate([w[0], w[1], w[2], w[3]]) for w in want]

    def check(got, what):
        for l in range(n):
            g = np.concatenate(split(got[l]))
            assert np.array_equal(g.view(np.uint32), want_rows[l].view(np.uint32)), (what, l)

    for rep in range(3):
        outd.upload(np.full(n * ld, np.nan, np.float32))
        check(run_persist(lib, layers, x0d, n, outd), f"eager {rep}")
    runtime.check(lib.qwen3_hip_capture_begin(), "capture_begin")
    rc = lib.qwen3_hip_decode_set_dev(layers.table, VP(x0d.ptr), VP(outd.ptr), n)
    gid = ctypes.c_int(-1)
    runtime.check(lib.qwen3_hip_capture_end(ctypes.byref(gid)), "capture_end")
    assert rc == 0
    try:
        for rep in range(3):
            outd.upload(np.full(n * ld, np.nan, np.float32))
            runtime.check(lib.qwen3_hip_graph_launch(gid.value), "graph_launch")
            abi.sync()
            check(outd.download(np.float32, n * ld).reshape(n, ld), f"graph {rep}")
            per_call_chain(lib, layers, x0d, 1)           # other work between replays
    finally:
        runtime.check(lib.qwen3_hip_graph_destroy(gid.value), "graph_destroy")
    assert errors(lib) == 0


def test_decode_set_argument_errors(lib):
    layers = Layers(1, 5, keep=0)
    x0d = abi.DeviceBuffer(4 * H)
    outd = abi.DeviceBuffer(4 * lib.qwen3_hip_decode_set_out_ld())
    assert lib.qwen3_hip_decode_set_dev(layers.table, VP(x0d.ptr), VP(outd.ptr), 0) == 1      # EINVAL
    assert lib.qwen3_hip_decode_set_dev(layers.table, VP(x0d.ptr), VP(outd.ptr), 33) == 8     # ETOOBIG
    assert lib.qwen3_hip_decode_set_dev(layers.table, VP(x0d.ptr), None, 1) == 1
    bad = (VP * 5)(layers.table[0], None, layers.table[2], layers.table[3], layers.table[4])
    assert lib.qwen3_hip_decode_set_dev(bad, VP(x0d.ptr), VP(outd.ptr), 1) == 1
    lib.qwen3_hip_last_error()
