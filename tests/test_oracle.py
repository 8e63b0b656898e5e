"""Pin the CPU oracle (CPU only; no GPU).

Each oracle function is checked against something that is not a retyping of
its own formula: the reference's shipped golden vectors, the reference's own
C compiled from its sources (oracle/_ref, when built), fixtures that compiled
C wrote (tests/golden/*.npz), closed forms, brute force and an independent
FPU formulation of the rounding.
"""
import glob
import os
from fractions import Fraction

import numpy as np
import pytest

import oracle

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def rtl_cases():
    return sorted(glob.glob(os.path.join(GOLD, "rtl_*.npz")))


@pytest.mark.parametrize("path", rtl_cases(), ids=lambda p: os.path.basename(p)[4:-4])
def test_hw16_matches_rtl_golden_vectors_bit_exact(path):
    """rtl_verification/cases/*/c_ref.bin: 16-element exact blocks with fp32
    rounding between blocks reproduces every shipped output word."""
    z = np.load(path)
    M, N, K = int(z["M"]), int(z["N"]), int(z["K"])
    a = oracle.bf16_to_f32(z["a_bf16"]) if "a_bf16" in z else z["a_src"].ravel()
    c = oracle.gemm_hw16(a, z["b_bf16"], M, K, N)
    bits = c.view(np.uint32)
    assert np.array_equal(bits, z["c_ref_bits"])
    if "xor_ref" in z:   # check.py's XOR reduction of the C words
        assert int(np.bitwise_xor.reduce(bits.ravel())) == int(z["xor_ref"])


def test_hw16_model_is_the_16_block_one_not_32():
    """The shipped generator text says K-blocks of 32; the data say 16.  A
    32-block model must NOT reproduce case 004, or the test above would not
    distinguish the two."""
    z = np.load(os.path.join(GOLD, "rtl_004.npz"))
    M, N, K = int(z["M"]), int(z["N"]), int(z["K"])
    a = oracle.bf16_to_f32(z["a_bf16"]).reshape(M, K).astype(np.float64)
    b = oracle.bf16_to_f32(z["b_bf16"]).reshape(N, K).astype(np.float64)
    acc = np.zeros((M, N), np.float32)
    for k0 in range(0, K, 32):
        blk = a[:, k0:k0 + 32] @ b[:, k0:k0 + 32].T
        acc = (acc.astype(np.float64) + blk).astype(np.float32)
    assert not np.array_equal(acc.view(np.uint32), z["c_ref_bits"])


def test_scalar_and_hwsim_match_compiled_reference_fixtures():
    """tests/golden/scalar_ref.npz was written by the reference's
    kernels_scalar.c / kernels_hwsim.c compiled from source."""
    z = np.load(os.path.join(GOLD, "scalar_ref.npz"))
    for M, K, N in z["shapes"]:
        M, K, N = int(M), int(K), int(N)
        key = f"{M}x{K}x{N}"
        for akey, suffix in (("a", "c"), ("araw", "craw")):
            a, b = z[f"{key}_{akey}"], z[f"{key}_b"]
            cs = oracle.gemm_scalar(a, b, M, K, N)
            ch = oracle.gemm_hw16(a, b, M, K, N)
            assert np.array_equal(cs.view(np.uint32), z[f"{key}_{suffix}_scalar"].view(np.uint32)), key
            assert np.array_equal(ch.view(np.uint32), z[f"{key}_{suffix}_hwsim"].view(np.uint32)), key


@pytest.mark.parametrize("M,K,N", [(1, 1024, 2048), (4, 1024, 256), (8, 33, 128),
                                   (129, 64, 130), (1, 3072, 1024)])
def test_scalar_matches_compiled_reference_live(M, K, N):
    """Same comparison against oracle/_ref, on fresh seeded inputs (only where
    the reference's C was compiled)."""
    L = oracle.ref("ref_scalar")
    if L is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    a = oracle.f32_bf16_normal(M * K, 7 + M, 1.0) + np.float32(1e-4)
    b = oracle.bf16_normal(N * K, 8 + N, 0.02)
    assert np.array_equal(oracle.gemm_scalar(a, b, M, K, N).view(np.uint32),
                          oracle.ref_gemm(L, a, b, M, K, N).view(np.uint32))
    H = oracle.ref("ref_hwsim")
    assert np.array_equal(oracle.gemm_hw16(a, b, M, K, N).view(np.uint32),
                          oracle.ref_gemm(H, a, b, M, K, N).view(np.uint32))


@pytest.mark.parametrize("M,K,N", [(1, 1024, 2048), (4, 1024, 256), (8, 33, 128), (129, 64, 130),
                                   (1, 3072, 1024), (7, 17, 5)])
def test_threaded_hw16_is_bit_exact(M, K, N, monkeypatch):
    """oracle/hw16_mt.c (the GEMM the long-context reference build links):
    bit-exact to orc_gemm_hw16 (itself pinned to the RTL golden vectors) for
    any thread count, and to the compiled kernels_hwsim.c where it was built;
    inputs not bf16-representable and K not a multiple of 16 included."""
    T = oracle.hw16mt()
    a = oracle.f32_bf16_normal(M * K, 17 + M, 1.0) + np.float32(3e-5)
    b = oracle.bf16_normal(N * K, 18 + N, 0.02)
    want = oracle.gemm_hw16(a, b, M, K, N)
    for threads in ("1", "3", "8"):
        monkeypatch.setenv("ORC_THREADS", threads)
        got = oracle.ref_gemm(T, a, b, M, K, N)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), threads
    H = oracle.ref("ref_hwsim")
    if H is not None:
        assert np.array_equal(oracle.ref_gemm(H, a, b, M, K, N).view(np.uint32), want.view(np.uint32))


def test_threaded_hw16_on_the_rtl_golden_vectors():
    """the shipped AME vectors through the threaded GEMM: every output bit-exact"""
    T = oracle.hw16mt()
    for path in rtl_cases():
        z = np.load(path)
        M, N, K = int(z["M"]), int(z["N"]), int(z["K"])
        a = oracle.bf16_to_f32(z["a_bf16"]) if "a_bf16" in z else z["a_src"].ravel()
        got = oracle.ref_gemm(T, a, z["b_bf16"], M, K, N)
        assert np.array_equal(got.reshape(-1).view(np.uint32), z["c_ref_bits"].reshape(-1)), path


def test_bf16_rne_against_independent_fpu_rounding():
    """Every high half (all signs, exponents, mantissas) with low halves that
    cover zero, +-1 around the halfway point and the all-ones carry case."""
    lo = np.array([0x0000, 0x0001, 0x3FFF, 0x7FFF, 0x8000, 0x8001, 0xBFFF,
                   0xC000, 0xFFFE, 0xFFFF, 0x1234, 0x9ABC], np.uint16)
    bad = oracle.lib().orc_bf16_rne_selfcheck(lo.ctypes.data_as(oracle.U16P), len(lo))
    assert bad == 0


def test_bf16_rne_known_values():
    f = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -8 + 2 ** -20,
                  -2.5, 3.4028235e38, 1e-45, 0.0], np.float32)
    got = oracle.f32_to_bf16(f)
    # 1+2^-8 is a tie between 1.0 (even) and 1+2^-7 -> 1.0; 1+3*2^-8 ties to
    # 1+2^-6 (even); just above the tie rounds up; FLT_MAX rounds to +Inf
    assert list(got) == [0x3F80, 0x3F80, 0x3F82, 0x3F81, 0xC020, 0x7F80, 0x0000, 0x0000]
    assert oracle.lib().orc_f32_to_bf16_hw(np.float32(np.inf)) == 0x7F80
    # the reference recipe turns this NaN payload into -0 (carry into the
    # sign); the hwsim variant passes NaN through
    nan = np.array([0x7FFFFFFF], np.uint32).view(np.float32)[0]
    assert oracle.lib().orc_f32_to_bf16(nan) == 0x8000
    assert oracle.lib().orc_f32_to_bf16_hw(nan) == 0x7FFF


def test_exact_gemm_closed_forms_and_fraction_brute_force():
    # fpga_bringup/src/tests/bringup.c:218-270: 1x1x32 of ones = 32.0f
    c, s = oracle.gemm_exact(np.ones(32, np.float32), oracle.f32_to_bf16(np.ones(32)), 1, 32, 1)
    assert c[0, 0] == 32.0 and s[0, 0] == 32.0
    rng = np.random.default_rng(5)
    M, K, N = 3, 7, 4
    a = oracle.round_bf16(rng.standard_normal(M * K).astype(np.float32))
    b = oracle.f32_to_bf16(rng.standard_normal(N * K).astype(np.float32))
    bf = oracle.bf16_to_f32(b)
    c, s = oracle.gemm_exact(a, b, M, K, N)
    for m in range(M):
        for n in range(N):
            ex = sum(Fraction(float(a[m * K + k])) * Fraction(float(bf[n * K + k])) for k in range(K))
            ab = sum(abs(Fraction(float(a[m * K + k])) * Fraction(float(bf[n * K + k]))) for k in range(K))
            assert c[m, n] == float(ex)
            assert s[m, n] == float(ab)


def test_scalar_gemm_is_sequential_fp32():
    """A case where the order matters: 2^24 followed by ones.  Sequential fp32
    (k ascending) drops every 1.0; an exact sum keeps them."""
    K = 33
    a = np.ones(K, np.float32)
    a[0] = 2.0 ** 24
    b = oracle.f32_to_bf16(np.ones(K, np.float32))
    assert oracle.gemm_scalar(a, b, 1, K, 1)[0, 0] == np.float32(2.0 ** 24)
    c, _ = oracle.gemm_exact(a, b, 1, K, 1)
    assert c[0, 0] == 2.0 ** 24 + 32
    # and 16-block rounding keeps the ones inside each block: block 0 holds
    # 2^24 + 15 (rounds to 2^24+16 in fp32), the next blocks add 16 and 1
    assert oracle.gemm_hw16(a, b, 1, K, 1)[0, 0] == np.float32(2.0 ** 24 + 32)


def test_reference_unit_test_metric_holds_for_scalar_oracle():
    """fpga_bringup/src/src/test_kernels.c:37-90 — LCG seed 12345, fp32 A,
    bf16 B, max|err|/max|ref| < 1e-5 against fp64, over its 12 shapes."""
    state = 12345
    shapes = [(1, 1024, 2048), (1, 1024, 1024), (1, 2048, 1024), (1, 1024, 3072),
              (1, 3072, 1024), (4, 1024, 2048), (127, 1024, 1024), (128, 1024, 1024),
              (129, 1024, 1024), (8, 32, 128), (8, 64, 128), (8, 33, 128)]
    for M, K, N in shapes:
        a, state = oracle.test_lcg(M * K, state)
        bw, state = oracle.test_lcg(N * K, state)
        b = oracle.f32_to_bf16(bw)
        if M * N * K > 2 ** 27:     # keep the CPU suite fast: sample columns
            cols = (0, 64)
        else:
            cols = (0, N)
        c = oracle.gemm_scalar(a, b, M, K, N, cols=cols)[:, cols[0]:cols[1]]
        bsub = b.reshape(N, K)[cols[0]:cols[1]].ravel()
        ref, _ = oracle.gemm_exact(a, bsub, M, K, cols[1] - cols[0])
        rel = np.max(np.abs(ref - c)) / (np.max(np.abs(ref)) + 1e-30)
        assert rel < 1e-5, (M, K, N, rel)


def test_silu_mul_matches_compiled_reference_and_limits():
    z = np.load(os.path.join(GOLD, "ops_ref.npz"))
    h = oracle.silu_mul(z["gate"], z["up"])
    assert np.array_equal(h.view(np.uint32), z["silu_mul"].view(np.uint32))
    g = np.array([0.0, 50.0, -200.0], np.float32)
    u = np.array([3.0, 2.0, 5.0], np.float32)
    out = oracle.silu_mul(g, u)
    assert out[0] == 0.0
    assert out[1] == np.float32(100.0)       # silu(g) -> g for large g
    assert out[2] == 0.0                     # silu(g) -> 0 for very negative g


def test_argmax_first_max_wins():
    z = np.load(os.path.join(GOLD, "ops_ref.npz"))
    assert oracle.argmax(z["argmax_in"]) == int(z["argmax"]) == 777
    v = np.random.default_rng(3).standard_normal(5000).astype(np.float32)
    assert oracle.argmax(v) == int(np.argmax(v))
    v[10] = v[4000] = 100.0
    assert oracle.argmax(v) == 10


def test_gate_up_silu_is_gemm_gemm_silu():
    M, K, N = 3, 64, 40
    x = oracle.f32_bf16_normal(M * K, 11)
    wg = oracle.bf16_normal(N * K, 12, 0.02)
    wu = oracle.bf16_normal(N * K, 13, 0.02)
    g = oracle.gemm_scalar(x, wg, M, K, N).ravel()
    u = oracle.gemm_scalar(x, wu, M, K, N).ravel()
    L = oracle.ref("ref_ops")
    expect = oracle.silu_mul(g, u)
    if L is not None:   # the reference's compiled silu_mul on the same operands
        gg = g.copy()
        L.qwen3_op_silu_mul(gg.ctypes.data_as(oracle.F32P), u.ctypes.data_as(oracle.F32P), gg.size)
        assert np.array_equal(gg.view(np.uint32), expect.view(np.uint32))
    got = oracle.gate_up_silu(x, wg, wu, M, K, N).ravel()
    assert np.array_equal(got.view(np.uint32), expect.view(np.uint32))


def test_tile_layout_offsets_are_a_permutation():
    N, K = 256, 96
    offs = np.array([oracle.tile_offset(n, k, K) for n in range(N) for k in range(K)])
    assert np.array_equal(np.sort(offs), np.arange(N * K))
    # tile (0,0) is the first 4096 elements, rows 32 elements apart
    assert oracle.tile_offset(0, 31, K) == 31
    assert oracle.tile_offset(1, 0, K) == 32
    assert oracle.tile_offset(0, 32, K) == 4096
    assert oracle.tile_offset(128, 0, K) == 3 * 4096
    b = np.arange(N * K, dtype=np.uint16)
    t = oracle.row_to_tile(b, N, K)
    assert t[oracle.tile_offset(200, 70, K)] == b[200 * K + 70]


def test_splitmix64_published_vector():
    """First outputs of SplitMix64 from seed 1234567 (the reference vector
    published with the algorithm)."""
    import ctypes
    st = ctypes.c_uint64(1234567)
    got = [oracle.lib().orc_splitmix64(ctypes.byref(st)) for _ in range(3)]
    assert got == [6457827717110365317, 3203168211198807973, 9817491932198370423]


def test_inputs_are_bf16_representable_and_deterministic():
    a = oracle.f32_bf16_normal(10000, 99)
    assert np.array_equal(oracle.round_bf16(a), a)
    assert np.array_equal(a, oracle.f32_bf16_normal(10000, 99))
    assert 0.95 < float(np.std(a)) < 1.05
    w = oracle.bf16_to_f32(oracle.bf16_normal(10000, 98, 0.02))
    assert 0.019 < float(np.std(w)) < 0.021
