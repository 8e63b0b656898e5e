"""The library's host bookkeeping -- graph capture, instantiation, launch and
destruction, workspace growth while graphs hold the old buffers, events,
streams -- checked on the CPU against a recording stand-in for the HIP
runtime, under AddressSanitizer (tests/hostcheck/).  Host-only objects of the
library (no device code) are linked against the stand-in; nothing runs on a
GPU.  The stand-in reports, among others, a launch of a destroyed graph exec,
a graph exec destroyed while its last launch may still run, a buffer freed
while a live graph exec references it, and a kernel pointer argument in freed
memory or in no allocation.

Scenarios (tests/hostcheck/drive.py):
  * selftest: a buffer freed while a live graph uses it, then the graph
    launched -- must be reported (2 violations), so the checks have teeth;
  * bench: the call sequence of `bench.py --no-cpu-baseline --no-model`
    (decode set per-call and persistent, per-kernel timing, GEMM tables with
    workspace growth and rotating weight copies) -- must be clean;
  * model: the device-resident forward and batched decode with graph replay
    and re-prefill -- must be clean.
"""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
HC = os.path.join(HERE, "hostcheck")
OUT = os.path.join(ROOT, "_build", "hostcheck")


def _asan_runtime():
    if not shutil.which("gcc"):
        return None
    p = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    return p if os.path.isabs(p) and os.path.exists(p) else None


@pytest.fixture(scope="module")
def harness():
    if not os.path.exists("/opt/rocm/bin/hipcc") or not os.path.isdir(HC):
        pytest.skip("hipcc or tests/hostcheck not present")
    if not os.path.exists(os.path.join(ROOT, "_build", "hip_gemm.o")):
        pytest.skip("the library is not built (its code objects give the kernel argument table)")
    asan = _asan_runtime()
    if not asan:
        pytest.skip("no AddressSanitizer runtime")
    subprocess.run(["make", "-s", "-j4", "-C", HC], check=True)
    env = dict(os.environ, LD_PRELOAD=asan, ASAN_OPTIONS="detect_leaks=0",
               HIPSTUB_KERNEL_ARGS=os.path.join(OUT, "kernel_args.tsv"))
    return env


def _drive(env, *args):
    p = subprocess.run(["python3", os.path.join(HC, "drive.py"), *args], env=env, capture_output=True,
                       text=True, timeout=900)
    print(p.stdout[-2000:])
    print(p.stderr[-4000:])
    return p


def test_checks_report_a_planted_misuse(harness):
    p = _drive(harness, "selftest")
    assert p.returncode == 2, p.returncode
    assert "is used by live graph exec" in p.stderr
    assert "is in freed allocation" in p.stderr


def test_bench_call_sequence_is_clean(harness):
    p = _drive(harness, "bench", "5")
    assert p.returncode == 0, p.stderr[-4000:]
    assert "0 violations" in p.stderr and "ERROR: AddressSanitizer" not in p.stderr


def test_model_call_sequence_is_clean(harness):
    p = _drive(harness, "model")
    assert p.returncode == 0, p.stderr[-4000:]
    assert "0 violations" in p.stderr and "ERROR: AddressSanitizer" not in p.stderr
