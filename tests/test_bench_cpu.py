"""bench.py's contract on the CPU: the one-GPU refusal, the algorithmic byte
and flop counts behind `roofline.achieved`, the choice of the headline step
and the CPU-baseline leg (the reference's compiled scalar GEMM, timed on a
tiny budget)."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def _run(args, env=None):
    e = dict(os.environ)
    e.update(env or {})
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")] + args, capture_output=True,
                          text=True, env=e, timeout=120)


@pytest.mark.parametrize("args,env", [(["--gpus", "2"], None), (["--gpus", "8"], None),
                                      ([], {"WORLD_SIZE": "2"})])
def test_more_than_one_gpu_is_refused(args, env):
    r = _run(args + ["--steps", "1"], env)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


def test_algorithmic_bytes_per_launch():
    # bf16 weights + fp32 activation in + fp32 output, per decode GEMV class
    assert bench.gemv_bytes(1024, 2048) == 4_206_592            # q
    assert bench.gemv_bytes(1024, 1024) == 2_105_344            # k, v
    assert bench.gemv_bytes(2048, 1024) == 4_206_592            # o
    assert bench.gemv_bytes(1024, 3072) == 6_307_840            # gate, up
    assert bench.gemv_bytes(3072, 1024) == 6_307_840            # down
    assert bench.gemv_bytes(1024, 151936) == 311_776_768        # lm_head
    # 28 layers of the seven projections plus lm_head: the 197 calls of a decode token
    assert bench.STEP_BYTES == 28 * (4_206_592 + 2 * 2_105_344 + 4_206_592 + 3 * 6_307_840) + 311_776_768
    assert bench.STEP_BYTES == 1_195_103_744
    # the dense bf16 peak the GEMM fractions are quoted against
    assert bench.MFMA_BF16_PEAK_TFLOPS == pytest.approx(256 * 2.4e9 * 4096 / 1e12, rel=1e-4)


def test_cpu_baseline_leg():
    out = bench.run_cpu_baseline(0.5)
    if out.get("value") is None and "not built" in str(out.get("error", "")):
        pytest.skip("oracle/_ref not built")
    assert out["value"] and out["value"] > 0
    assert out["cores"] == 1
    assert out["kind"] in ("reference", "port")
    assert out["unit"] == "tok/s"


@pytest.mark.parametrize("pers,per_call,want", [
    ({"ms_per_step": 0.33, "exchange_errors": 0}, False, True),
    ({"ms_per_step": 0.33, "exchange_errors": 0}, True, False),     # --per-call
    ({"ms_per_step": 0.33, "exchange_errors": 1}, False, False),    # a launch gave up: outputs invalid
    ({"ms_per_step": 0.33}, False, False),                          # no error count: not trusted
    (None, False, False),                                           # grid not resident: not measured
])
def test_headline_step_choice(pers, per_call, want):
    assert bench.use_persistent(pers, per_call) is want


def test_committed_profiles_match_kernel_sources():
    """every rocprofv3 summary under profiles/ was made from the kernel
    sources in the tree: its '# sources:' digest is the one bench.py
    computes, so the roofline figures it quotes describe these kernels"""
    pdir = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "profiles")
    want = bench.kernel_sources_digest()
    stale = {}
    for name in sorted(os.listdir(pdir)):
        if not name.endswith(".txt"):
            continue
        digests = [ln.split(":", 1)[1].split()[0] for ln in open(os.path.join(pdir, name))
                   if ln.startswith("# sources:")]
        if digests != [want]:
            stale[name] = digests
    assert not stale, stale
