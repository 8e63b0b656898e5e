#!/usr/bin/env python3
"""Benchmark of the Qwen3-0.6B GEMM/GEMV hot path on one MI355X.

Workload (one "step" = one decode token's projections at M = 1):
    28 layers x [ fused q|k|v GEMV 1024 -> 4096,  o GEMV 2048 -> 1024,
                  fused gate|up GEMV 1024 -> 2x3072 with SiLU*mul epilogue,
                  down GEMV 3072 -> 1024 ]
    + tied lm_head GEMV 1024 -> 151936
with distinct random-init bf16 weights per layer (N(0, 0.02); 1.19 GB, more
than the 256 MB last-level cache) and activations already resident in HBM.
Algorithmic bytes per step = 1,195,103,744 (bf16 weights + fp32 inputs +
fp32 outputs of the 197 reference GEMV calls).  value = steps per second =
decode tokens/s of the GEMV set.

Also reported: per-kernel launch times (HIP events on the library stream),
the roofline fraction of the dominant kernel, the GEMM tables of the other
configurations (M = 16 gate_proj; M = 512 projections warm and cold, fused
gate/up included; M = 1024 .. 4096; M = 64 batched decode incl. the
64 x 1024 x 151936 lm_head), a CPU baseline: the reference's portable
scalar GEMM (fpga_bringup/src/src/kernels_scalar.c, compiled from its source
into oracle/_ref) running the same step on 1 host core, and the full
device-resident Qwen3-0.6B forward (128-token prefill + 128 greedy decode
steps) beside the reference forward timed on 1 host core.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import ctypes
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "bf16 GEMM TFLOP/s (% MFMA peak); Qwen3-0.6B decode tok/s, 1 GPU"
HBM_PEAK_GBS = 8000.0               # MI355X HBM3E, published
MFMA_BF16_PEAK_TFLOPS = 2516.6      # 256 CU x 2.4 GHz x 4096 dense bf16 flop/clk

H, Q, KV, I, V, LAYERS = 1024, 2048, 1024, 3072, 151936, 28


def gemv_bytes(K, N, nb=1):
    """algorithmic bytes of an M=1 GEMV: bf16 weights + fp32 in + fp32 out"""
    return 2 * N * K * nb + 4 * K + 4 * N


# the 197 reference GEMV calls of one decode token (M = 1)
STEP_BYTES = LAYERS * (gemv_bytes(H, Q) + 2 * gemv_bytes(H, KV) + gemv_bytes(Q, H)
                       + 2 * gemv_bytes(H, I) + gemv_bytes(I, H)) + gemv_bytes(H, V)
assert STEP_BYTES == 1195103744


# ---------------------------------------------------------------------------
# CPU baseline (child process, pinned to one core, no GPU)
# ---------------------------------------------------------------------------
def cpu_baseline_child(budget_s):
    import numpy as np
    import oracle
    os.sched_setaffinity(0, {sorted(os.sched_getaffinity(0))[0]})
    L = oracle.ref("ref_scalar")
    kind = "reference"
    if L is None:
        L = oracle.lib()
        kind = "port"
        fn = L.orc_gemm_scalar
    else:
        fn = L.qwen3_gemm
    F32P, U16P = oracle.F32P, oracle.U16P
    rng = np.random.default_rng(1)
    # content does not change scalar timing; addresses do (distinct per layer)
    pat = oracle.f32_to_bf16((rng.standard_normal(1 << 22) * 0.02).astype(np.float32))

    def weights(n):
        reps = -(-n // pat.size)
        return np.tile(pat, reps)[:n].copy()

    layers = []
    for _ in range(LAYERS):
        layers.append({"qkv": weights((Q + 2 * KV) * H), "o": weights(H * Q),
                       "g": weights(I * H), "u": weights(I * H), "d": weights(H * I)})
    emb = weights(V * H)
    x = oracle.f32_bf16_normal(I, 5)
    out = np.empty(V, np.float32)
    xp, op = x.ctypes.data_as(F32P), out.ctypes.data_as(F32P)

    def step():
        for w in layers:
            # the reference forward calls q, k, v, o, gate, up, down separately
            q = w["qkv"]
            fn(op, xp, q.ctypes.data_as(U16P), 1, H, Q)
            fn(op, xp, q[Q * H:].ctypes.data_as(U16P), 1, H, KV)
            fn(op, xp, q[(Q + KV) * H:].ctypes.data_as(U16P), 1, H, KV)
            fn(op, xp, w["o"].ctypes.data_as(U16P), 1, Q, H)
            fn(op, xp, w["g"].ctypes.data_as(U16P), 1, H, I)
            fn(op, xp, w["u"].ctypes.data_as(U16P), 1, H, I)
            fn(op, xp, w["d"].ctypes.data_as(U16P), 1, I, H)
        fn(op, xp, emb.ctypes.data_as(U16P), 1, H, V)

    t0 = time.perf_counter()
    step()                                  # warm caches / page in; sizes the runs
    per = time.perf_counter() - t0
    n = max(1, int(budget_s / 3 / per))
    rates = []
    for _ in range(3):                      # median of 3 runs of n steps
        t0 = time.perf_counter()
        for _ in range(n):
            step()
        rates.append(n / (time.perf_counter() - t0))
    cpu = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    print(json.dumps({"value": sorted(rates)[1], "unit": "tok/s", "cores": 1, "kind": kind,
                      "runs_tok_s": [round(r, 3) for r in rates],
                      "sample": f"median of 3 runs of {n} full decode steps (197 GEMV calls each, "
                                f"distinct weights per layer) on 1 core of {cpu} "
                                f"(nproc={os.cpu_count()}); "
                                + ("reference kernels_scalar.c compiled from source"
                                   if kind == "reference" else "oracle restatement")}))


def run_cpu_baseline(budget_s):
    r = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-baseline-child",
                        str(budget_s)], capture_output=True, text=True)
    if r.returncode != 0:
        return {"value": None, "error": r.stderr.strip()[-400:]}
    return json.loads(r.stdout.strip().splitlines()[-1])


MODEL_SEED = 0x03550040      # random-init weights of the full-forward workload


def cpu_model_child(n_prompt=128, n_decode=128):
    """The reference forward (qwen3.c + kernels_scalar.c + ops_scalar.c,
    compiled from source into oracle/_ref) on 1 core on the full-forward
    workload itself: the 128-token prompt prefilled, then 128 greedy decode
    steps; the driver times the prefill and the decode loop separately."""
    import numpy as np
    import oracle
    from n550_qwen3_bringup_handover_amd import model as M
    L = oracle.ref("ref_model_scalar")
    if L is None:
        print(json.dumps({"value": None, "error": "oracle/_ref/libref_model_scalar.so not built"}))
        return
    blob = M.qw3m_random(MODEL_SEED, M.LAYOUT_ROW, threads=4)    # before pinning to one core
    core = sorted(os.sched_getaffinity(0))[-1]
    os.sched_setaffinity(0, {core})
    L.refdrv_generate.restype = ctypes.c_int
    L.refdrv_generate.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_int),
                                  ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_int),
                                  ctypes.c_void_p, ctypes.c_void_p]
    L.refdrv_last_times.restype = None
    L.refdrv_last_times.argtypes = [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]
    prompt = np.random.default_rng(4).integers(0, V, n_prompt).astype(np.int32)
    out = np.zeros(n_decode + 1, np.int32)
    n = L.refdrv_generate(blob.ctypes.data_as(ctypes.c_void_p), blob.nbytes,
                          prompt.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), n_prompt, n_decode, 0,
                          out.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), None, None)
    t_pre, t_dec = ctypes.c_double(), ctypes.c_double()
    L.refdrv_last_times(ctypes.byref(t_pre), ctypes.byref(t_dec))
    ok = n == n_decode + 1 and t_dec.value > 0
    print(json.dumps({"value": n_decode / t_dec.value if ok else None, "unit": "tok/s", "cores": 1,
                      "kind": "reference", "prefill_tok_s": n_prompt / t_pre.value if ok else None,
                      "prefill_s": round(t_pre.value, 2), "decode_s": round(t_dec.value, 2),
                      "first_tokens": [int(t) for t in out[:8]],
                      "sample": f"the whole workload: reference forward qwen3.c + kernels_scalar.c + "
                                f"ops_scalar.c on 1 core (core {core}, run beside the GPU measurements), "
                                f"the {n_prompt}-token prompt prefilled in {t_pre.value:.1f} s, then "
                                f"{n_decode} greedy decode steps in {t_dec.value:.1f} s"}))


def start_cpu_model():
    """the full-forward CPU baseline as a child process on its own core,
    started before the GPU measurements and collected after them"""
    return subprocess.Popen([sys.executable, os.path.abspath(__file__), "--cpu-model-child"],
                            stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)


def finish_cpu_model(proc):
    try:
        out, err = proc.communicate(timeout=900)
    except subprocess.TimeoutExpired:
        proc.kill()
        return {"value": None, "error": "timed out"}
    if proc.returncode != 0:
        return {"value": None, "error": err.strip()[-400:]}
    return json.loads(out.strip().splitlines()[-1])


def host_path(steps=10, warmup=5, runs=3):
    """The decode GEMV set through the host-pointer plug-in ABI, as the
    reference forward calls it (fpga_bringup/src/src/qwen3.c:477-573): 197
    synchronous qwen3_gemm / qwen3_gemm_row calls per token with host A and C
    (copied over PCIe on every call), weights mapped once with
    qwen3_hip_map_weights.  PCIe-inclusive; never the headline value."""
    import numpy as np
    from n550_qwen3_bringup_handover_amd import model as M, runtime
    L = runtime.lib()
    blob = M.qw3m_random(MODEL_SEED, M.LAYOUT_ROW, threads=16)
    runtime.check(L.qwen3_hip_map_weights(blob.ctypes.data_as(ctypes.c_void_p), blob.nbytes), "map_weights")
    tens = M.qw3m_tensors(blob)
    base = blob.ctypes.data
    U16P = ctypes.POINTER(ctypes.c_uint16)
    F32P = ctypes.POINTER(ctypes.c_float)
    x = np.random.default_rng(5).standard_normal(I).astype(np.float32)
    out = np.empty(V, np.float32)
    xp, op = x.ctypes.data_as(F32P), out.ctypes.data_as(F32P)
    calls = []
    for l in range(LAYERS):
        t0 = 1 + 11 * l
        for j in (1, 2, 3, 6, 8, 9, 10):          # q, k, v, o, gate, up, down
            off, rows, cols = tens[t0 + j]
            calls.append((L.qwen3_gemm, ctypes.cast(base + off, U16P), cols, rows))
    calls.append((L.qwen3_gemm_row, ctypes.cast(base + tens[0][0], U16P), H, V))
    L.qwen3_hip_set_abort(0)

    def step():
        for fn, b, K, N in calls:
            fn(op, xp, b, 1, K, N)

    for _ in range(warmup):
        step()
    rates = []
    for _ in range(runs):
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        rates.append(steps / (time.perf_counter() - t0))
    err = L.qwen3_hip_last_error()
    runtime.check(L.qwen3_hip_unmap_weights(blob.ctypes.data_as(ctypes.c_void_p)), "unmap_weights")
    med = sorted(rates)[len(rates) // 2]
    return {"workload": "decode GEMV set through the host-pointer ABI: 197 synchronous qwen3_gemm/"
                        "qwen3_gemm_row calls per token, host A and C copied per call, weights mapped once; "
                        f"median of {runs} runs of {steps} tokens after {warmup} warm-up tokens",
            "tok_s": round(med, 2) if err == 0 else None, "ms_per_token": round(1e3 / med, 3),
            "runs_tok_s": [round(r, 1) for r in rates], "error": err}


def model_forward_p128_d128(n_prompt=128, n_decode=128):
    """Full Qwen3-0.6B forward on the device (include/qwen3_hip_model.h):
    random-init weights, a 128-token random prompt in one prefill chunk, then
    128 greedy decode steps (one graph replay each)."""
    import numpy as np
    from n550_qwen3_bringup_handover_amd import model as M
    blob = M.qw3m_random(MODEL_SEED, M.LAYOUT_ROW, threads=16)
    prompt = np.random.default_rng(4).integers(0, V, n_prompt).astype(np.int32)
    with M.Model(blob, max_seq=n_prompt + n_decode) as m:
        del blob
        m.generate(prompt, 8)                       # warm-up: graph capture, caches
        best = None
        for _ in range(3):
            toks = m.generate(prompt, n_decode)
            pre, dec = m.timing()
            if best is None or dec < best[1]:
                best = (pre, dec, toks)
    pre, dec, toks = best
    return {"workload": f"Qwen3-0.6B full forward, random-init bf16 weights, batch 1: {n_prompt}-token "
                        f"prompt (one prefill chunk) + {n_decode} greedy decode steps (graph replay each); "
                        "best of 3",
            "prefill_ms": round(pre, 3), "prefill_tok_s": round(n_prompt / pre * 1e3, 1),
            "decode_ms": round(dec, 3), "decode_tok_s": round(n_decode / dec * 1e3, 2),
            "ms_per_decode_token": round(dec / n_decode, 4), "first_tokens": [int(t) for t in toks[:8]]}


def model_batch_decode(n_seq=64, ctx=2048, n_decode=32, warm=2):
    """Batched greedy decode (qwen3_hip_batch_*): n_seq sequences, each
    prefilled with its own random prompt of ctx - n_decode - warm tokens;
    `warm` untimed steps (the first eager, then the captured graph), then
    n_decode timed steps of all sequences at once, the last at position
    ctx - 1.  Each step reads every weight once (M = n_seq GEMMs) and every
    sequence's K/V cache up to its position (fp32, 229,376 B per position)."""
    import numpy as np
    from n550_qwen3_bringup_handover_amd import model as M
    n_prompt = ctx - n_decode - warm
    rng = np.random.default_rng(5)
    blob = M.qw3m_random(MODEL_SEED, M.LAYOUT_ROW, threads=16)
    with M.Model(blob, max_seq=ctx) as m:
        del blob
        with M.Batch(m, n_seq, ctx) as b:
            t0 = time.time()
            for s in range(n_seq):
                b.prefill(s, rng.integers(0, V, n_prompt).astype(np.int32))
                if s % 16 == 15:
                    print(f"batched decode: {s + 1} of {n_seq} sequences prefilled, {time.time() - t0:.1f} s",
                          file=sys.stderr, flush=True)
            prefill_s = time.time() - t0
            b.decode(warm)
            out = b.decode(n_decode)
            dec = b.timing()
    kv_pos_bytes = LAYERS * 8 * 128 * 4 * 2
    # positions read by the timed steps: step i of each sequence attends over n_prompt + warm + i + 1
    kv_bytes = n_seq * kv_pos_bytes * sum(n_prompt + warm + i + 1 for i in range(n_decode))
    w_bytes = n_decode * STEP_BYTES
    return {"workload": f"Qwen3-0.6B batched greedy decode, random-init bf16 weights: {n_seq} sequences, "
                        f"each prefilled with its own {n_prompt}-token random prompt, then {n_decode} timed "
                        f"steps of all sequences at once (graph replay each) at positions "
                        f"{n_prompt + warm}..{ctx - 1}; fp32 KV cache",
            "n_seq": n_seq, "ctx": ctx, "prefill_s": round(prefill_s, 2),
            "decode_ms": round(dec, 3), "ms_per_step": round(dec / n_decode, 4),
            "decode_tok_s": round(n_seq * n_decode / dec * 1e3, 1),
            "hbm_bytes_per_step": int((kv_bytes + w_bytes) / n_decode),
            "hbm_GBps": round((kv_bytes + w_bytes) / (dec * 1e-3) / 1e9, 1),
            "first_tokens_seq0": [int(t) for t in out[0, :8]]}


# ---------------------------------------------------------------------------
# GPU side
# ---------------------------------------------------------------------------
class Gpu:
    def __init__(self):
        from n550_qwen3_bringup_handover_amd import runtime
        self.rt = runtime
        self.L = runtime.init()
        self.VP = ctypes.c_void_p
        self.bufs = []

    def alloc(self, nbytes):
        p = ctypes.c_void_p()
        self.rt.check(self.L.qwen3_hip_malloc(ctypes.byref(p), int(nbytes)), "malloc")
        self.bufs.append(p.value)
        return p.value

    def fill_bf16(self, ptr, n, seed):
        """fill n bf16 weights with a 32 MB random N(0,0.02) block, repeated"""
        import numpy as np
        rng = np.random.default_rng(seed)
        blk = min(n, 1 << 24)
        pat = ((rng.standard_normal(blk, dtype=np.float32) * np.float32(0.02)).view(np.uint32)
               + np.uint32(0x8000)) >> np.uint32(16)
        pat = pat.astype(np.uint16)
        done = 0
        while done < n:
            m = min(blk, n - done)
            self.rt.check(self.L.qwen3_hip_memcpy_h2d(self.VP(ptr + 2 * done),
                                                      self.VP(pat.ctypes.data), 2 * m), "h2d")
            done += m
        self.rt.check(self.L.qwen3_hip_sync(), "sync")

    def fill_f32(self, ptr, n, seed):
        import numpy as np
        rng = np.random.default_rng(seed)
        x = rng.standard_normal(n, dtype=np.float32)
        x = ((x.view(np.uint32) + np.uint32(0x8000)) & np.uint32(0xFFFF0000)).view(np.float32)
        self.rt.check(self.L.qwen3_hip_memcpy_h2d(self.VP(ptr), self.VP(x.ctypes.data), x.nbytes), "h2d")
        self.rt.check(self.L.qwen3_hip_sync(), "sync")

    def gemm(self, c, a, b, M, K, N):
        rc = self.L.qwen3_hip_gemm_dev(self.VP(c), self.VP(a), self.VP(b), M, K, N)
        if rc:
            self.rt.check(rc, "qwen3_hip_gemm_dev")

    def gated(self, h, x, wg, wu, M, K, N):
        rc = self.L.qwen3_hip_gemm_gate_up_silu_dev(self.VP(h), self.VP(x), self.VP(wg), self.VP(wu), M, K, N)
        if rc:
            self.rt.check(rc, "qwen3_hip_gemm_gate_up_silu_dev")

    def record(self, slot):
        self.rt.check(self.L.qwen3_hip_timer_record(slot), "timer")

    def elapsed(self, a, b):
        ms = ctypes.c_float()
        self.rt.check(self.L.qwen3_hip_timer_elapsed_ms(a, b, ctypes.byref(ms)), "timer")
        return ms.value

    def sync(self):
        self.rt.check(self.L.qwen3_hip_sync(), "sync")

    def plan(self, M, K, N, gated=False):
        return self.L.qwen3_hip_plan(M, K, N, int(gated)).decode()

    def last_plan(self):
        """the plan the last GEMM call launched (after any fall-back)"""
        return self.L.qwen3_hip_last_plan().decode()


def build_decode_model(g):
    """device weights in the QW3M tensor order: q|k|v and gate|up contiguous"""
    layers = []
    per_layer = (Q + 2 * KV) * H + H * Q + 2 * I * H + H * I
    base = g.alloc(2 * per_layer * LAYERS)
    g.fill_bf16(base, per_layer * LAYERS, 11)
    off = base
    for _ in range(LAYERS):
        w = {"qkv": off}
        off += 2 * (Q + 2 * KV) * H
        w["o"] = off
        off += 2 * H * Q
        w["g"] = off
        w["u"] = off + 2 * I * H
        off += 4 * I * H
        w["d"] = off
        off += 2 * H * I
        layers.append(w)
    emb = g.alloc(2 * V * H)
    g.fill_bf16(emb, V * H, 12)
    act = {}
    for name, n in (("x", H), ("attn", Q), ("h", I), ("qkv", Q + 2 * KV), ("o", H), ("d", H),
                    ("logits", V)):
        act[name] = g.alloc(4 * n)
        g.fill_f32(act[name], n, 13 + len(name))
    return layers, emb, act


def decode_step(g, layers, emb, act):
    """Each GEMV consumes the previous one's output, so launches form the same
    dependency chain as the model forward (attention and norms, which sit
    between them in the model, are outside this hot path): x -> q|k|v; the q
    part stands in for the attention output -> o -> gate|up -> down -> x of
    the next layer; the last x -> lm_head."""
    for w in layers:
        g.gemm(act["qkv"], act["x"], w["qkv"], 1, H, Q + 2 * KV)
        g.gemm(act["o"], act["qkv"], w["o"], 1, Q, H)
        g.gated(act["h"], act["o"], w["g"], w["u"], 1, H, I)
        g.gemm(act["x"], act["h"], w["d"], 1, I, H)
    g.gemm(act["logits"], act["x"], emb, 1, H, V)


def time_step(g, launch_step, graph, warmup, steps):
    """decode steps back to back: `warmup` untimed, then `steps` timed with
    HIP events on the library stream (each step one graph replay if graph)"""
    gid = None
    if graph:
        g.rt.check(g.L.qwen3_hip_capture_begin(), "capture_begin")
        launch_step()
        gid = ctypes.c_int(-1)
        g.rt.check(g.L.qwen3_hip_capture_end(ctypes.byref(gid)), "capture_end")

        def step():
            g.rt.check(g.L.qwen3_hip_graph_launch(gid.value), "graph_launch")
    else:
        step = launch_step
    try:
        for _ in range(warmup):
            step()
        g.sync()
        t0 = time.perf_counter()
        g.record(60)
        for _ in range(steps):
            step()
        g.record(61)
        g.sync()
        wall = time.perf_counter() - t0
        return {"ms_per_step": g.elapsed(60, 61) / steps, "wall_s": round(wall, 3)}
    finally:
        if gid is not None:
            # no graph outlives its section: a workspace grown later is then freed at once
            g.rt.check(g.L.qwen3_hip_graph_destroy(gid.value), "graph_destroy")


def persistent_step(g, layers, emb, act):
    """One decode step on the persistent path: the 28 layers' 112 GEMVs in
    one qwen3_hip_decode_set_dev launch, then the lm_head GEMV.  Step t's
    layer 0 reads the x that step t-1's last down GEMV wrote (as the per-call
    step does); the first step starts from the same x."""
    VP = ctypes.c_void_p
    table = (VP * (5 * LAYERS))(*[w[k] for w in layers for k in ("qkv", "o", "g", "u", "d")])
    ld = g.L.qwen3_hip_decode_set_out_ld()
    out = g.alloc(4 * LAYERS * ld)
    xfin = out + 4 * ((LAYERS - 1) * ld + 8192)
    g.rt.check(g.L.qwen3_hip_copy_dev(VP(xfin), VP(act["x"]), 4 * H), "copy")

    def layers_only():
        rc = g.L.qwen3_hip_decode_set_dev(table, VP(xfin), VP(out), LAYERS)
        if rc:
            g.rt.check(rc, "qwen3_hip_decode_set_dev")

    def launch():
        layers_only()
        g.gemm(act["logits"], xfin, emb, 1, H, V)
    launch.layers_only = layers_only
    launch.keep = table
    return launch


def use_persistent(pers, per_call_flag):
    """whether the headline is the persistent step: it was measured (the
    device keeps its grid resident), no launch gave up waiting on its
    exchange (whose outputs would then be invalid), and --per-call was not
    given"""
    return bool(pers) and not per_call_flag and pers.get("exchange_errors", 1) == 0


def persistent_class(g, launch_step):
    """the persistent launch alone: its duration (HIP events around each
    launch on the library stream; a launch takes ~0.2 ms, so the events'
    own overhead is small) against the algorithmic bytes of the 112 GEMVs it
    runs"""
    ms = time_launches(g, lambda r: launch_step.layers_only(), 16)
    nbytes = STEP_BYTES - gemv_bytes(H, V)
    us = ms * 1e3
    return {"count_per_step": 1, "bytes_per_launch": nbytes, "us_per_launch": round(us, 3),
            "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
            "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "us_per_step": round(us, 2)}


def time_launches(g, launch, reps):
    """average duration of one launch: HIP events around each launch on the
    library stream (pairs of slots), after a warm-up launch"""
    launch(0)
    g.sync()
    tot = 0.0
    n = 0
    for r in range(reps):
        s = 2 * (r % 16)
        g.record(s)
        launch(r)
        g.record(s + 1)
        if s == 30 or r == reps - 1:
            for k in range(0, s + 2, 2):
                tot += g.elapsed(k, k + 1)
                n += 1
    return tot / n


def time_launches_graph(g, launch, reps):
    """average time per launch of `reps` back-to-back launches replayed from
    one captured graph (events around the replay, on the library stream).
    One eager launch first: a workspace the call needs is grown there, since
    the library grows none during capture."""
    launch(0)
    g.sync()
    g.rt.check(g.L.qwen3_hip_capture_begin(), "capture_begin")
    for r in range(reps):
        launch(r)
    gid = ctypes.c_int(-1)
    g.rt.check(g.L.qwen3_hip_capture_end(ctypes.byref(gid)), "capture_end")
    try:
        g.rt.check(g.L.qwen3_hip_graph_launch(gid.value), "graph_launch")
        g.sync()
        best = None
        for _ in range(3):
            g.record(56)
            g.rt.check(g.L.qwen3_hip_graph_launch(gid.value), "graph_launch")
            g.record(57)
            ms = g.elapsed(56, 57) / reps
            best = ms if best is None else min(best, ms)
        return best
    finally:
        g.rt.check(g.L.qwen3_hip_graph_destroy(gid.value), "graph_destroy")


def kernel_classes(g, layers, emb, act):
    """per-launch timing of each kernel class of the decode step"""
    cls = {
        "qkv_gemv": (LAYERS, gemv_bytes(H, Q + 2 * KV),
                     lambda r: g.gemm(act["qkv"], act["x"], layers[r % LAYERS]["qkv"], 1, H, Q + 2 * KV)),
        "o_gemv": (LAYERS, gemv_bytes(Q, H),
                   lambda r: g.gemm(act["o"], act["attn"], layers[r % LAYERS]["o"], 1, Q, H)),
        "gate_up_silu_gemv": (LAYERS, 2 * I * H * 2 + 4 * H + 4 * I,
                              lambda r: g.gated(act["h"], act["x"], layers[r % LAYERS]["g"],
                                                layers[r % LAYERS]["u"], 1, H, I)),
        "down_gemv": (LAYERS, gemv_bytes(I, H),
                      lambda r: g.gemm(act["d"], act["h"], layers[r % LAYERS]["d"], 1, I, H)),
        "lm_head_gemv": (1, gemv_bytes(H, V),
                         lambda r: g.gemm(act["logits"], act["x"], emb, 1, H, V)),
    }
    out = {}
    for name, (count, nbytes, fn) in cls.items():
        ms_ev = time_launches(g, fn, 64 if count > 1 else 32)
        ms = time_launches_graph(g, fn, 4 * LAYERS if count > 1 else 16)
        out[name] = {"count_per_step": count, "bytes_per_launch": nbytes,
                     "us_per_launch": round(ms * 1e3, 3),
                     "us_per_launch_event_pairs": round(ms_ev * 1e3, 3),
                     "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                     "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "us_per_step": round(ms * 1e3 * count, 2)}
    return out


def gemm_entry(g, M, K, N, gated, a, c, w, wrot=None, reps=32):
    """time one GEMM shape on the automatic plan: graph of back-to-back
    launches (each launch includes its ~1.6 us dependent-launch gap).  With
    wrot, launch r uses weight copy r % len(wrot) (cold: the copies exceed
    the 256 MB last-level cache)."""
    ws = wrot or [w]
    if gated:
        fn = lambda r: g.gated(c, a, ws[r % len(ws)], ws[r % len(ws)] + 2 * N * K, M, K, N)
        flops = 2.0 * M * 2 * N * K
        byts = 2 * 2 * N * K + 4 * M * K + 4 * M * N
    else:
        fn = lambda r: g.gemm(c, a, ws[r % len(ws)], M, K, N)
        flops = 2.0 * M * N * K
        byts = 2 * N * K + 4 * M * K + 4 * M * N
    ms = time_launches_graph(g, fn, reps)
    tf = flops / (ms * 1e-3) / 1e12
    return {"M": M, "K": K, "N": N, "gated": gated, "kernel": g.last_plan(),
            "us": round(ms * 1e3, 2), "TFLOPs": round(tf, 1),
            "mfma_frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
            "GBps": round(byts / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "cold_hbm_cap": round(min(1.0, flops / byts / (MFMA_BF16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9))), 3)}


# projection shapes (K, N, gated); qkv is the fused q|k|v the forward uses
SHAPES = {"q": (H, Q, False), "k_v": (H, KV, False), "o": (Q, H, False),
          "gate_up_silu": (H, I, True), "down": (I, H, False), "qkv_fused": (H, Q + 2 * KV, False)}


def gemm_tables(g):
    """The M = 16 gate_proj GEMM, the M = 512 prefill set, the M = 64 batched-
    decode set and an M sweep, on the automatic plans.  Warm: the same
    operands every launch (resident in L2/MALL); the M = 512 set
    also cold, rotating through weight copies larger than the last-level
    cache."""
    Mmax = 4096
    a = g.alloc(4 * Mmax * I)
    g.fill_f32(a, Mmax * I, 21)
    c = g.alloc(4 * Mmax * (Q + 2 * KV))
    w = g.alloc(2 * 2 * I * H)
    g.fill_bf16(w, 2 * I * H, 22)
    out = {}
    # one gate_proj GEMM at M = 16 (HBM-bound)
    out["m16_gate_proj"] = gemm_entry(g, 16, H, I, False, a, c, w)
    # prefill at M = 512, warm and cold
    ncopy = 48                                   # 48 x 12.6 MB = 604 MB of weights
    wrot = [g.alloc(2 * 2 * I * H) for _ in range(ncopy)]
    for p in wrot:
        g.fill_bf16(p, 2 * I * H, 23)
    m512 = {}
    for name, (K, N, gated) in SHAPES.items():
        m512[name] = gemm_entry(g, 512, K, N, gated, a, c, w)
        m512[name]["cold_us"] = gemm_entry(g, 512, K, N, gated, a, c, w, wrot=wrot, reps=ncopy)["us"]
    out["m512_prefill"] = m512
    # M sweep (warm)
    sweep = {}
    for M in (1024, 2048, 4096):
        sweep[str(M)] = {name: gemm_entry(g, M, K, N, gated, a, c, w) for name, (K, N, gated) in SHAPES.items()}
    out["m_sweep"] = sweep
    # one GPU's share of batched decode of 64 sequences, M = 64, incl. lm_head 64 x 1024 x 151936
    emb = g.alloc(2 * V * H)
    g.fill_bf16(emb, V * H, 24)
    m64 = {name: gemm_entry(g, 64, K, N, gated, a, c, w) for name, (K, N, gated) in SHAPES.items()}
    cl = g.alloc(4 * 64 * V)
    m64["lm_head"] = gemm_entry(g, 64, H, V, False, a, cl, emb, reps=16)
    layer_us = sum(m64[n]["us"] for n in ("qkv_fused", "o", "gate_up_silu", "down"))
    m64["step_us"] = round(LAYERS * layer_us + m64["lm_head"]["us"], 1)
    m64["tok_s_projections"] = round(64 / (m64["step_us"] * 1e-6), 1)
    out["m64_batched_decode"] = m64
    return out


# kernel signature of each decode kernel class in the rocprofv3 summaries
# (k_gemv1<rows per wave, chunks per lane, gated, prologue, merge>)
PROFILE_NAMES = {"qkv_gemv": "k_gemv1<1, 2, false, false, false>", "o_gemv": "k_gemv1<1, 4, false, false, false>",
                 "gate_up_silu_gemv": "k_gemv1<1, 2, true, false, false>",
                 "down_gemv": "k_gemv1<1, 6, false, false, false>",
                 "lm_head_gemv": "k_gemv1<4, 2, false, false, false>",
                 "decode_set_persistent": "k_decode_persist"}
DECODE_PROFILE = "decode_gemv_set_kernel_trace.txt"


# the headers hip_gemm.hip includes (its kernel families)
GEMM_KERNEL_HEADERS = ("gemm_common.h", "gemv_kernels.h", "tile_kernels.h", "misc_kernels.h", "small_m_kernels.h")
# the device headers of the model and persistent kernels
MODEL_KERNEL_HEADERS = ("persist_common.h", "fp_pinned.h", "model_shim.h")


def kernel_sources_digest():
    """sha256 over the library's GPU sources (csrc/*.hip, hip_shim.h and the
    kernel headers the .hip files compile, by name): a committed profile
    records the digest of the sources it was made from, so a profile of
    other kernels is not taken for these"""
    import glob
    import hashlib
    h = hashlib.sha256()
    csrc = os.path.join(ROOT, "n550_qwen3_bringup_handover_amd", "csrc")
    headers = ["hip_shim.h"] + list(GEMM_KERNEL_HEADERS) + list(MODEL_KERNEL_HEADERS)
    for path in sorted(glob.glob(os.path.join(csrc, "*.hip")) + [os.path.join(csrc, n) for n in headers]):
        h.update(os.path.basename(path).encode())
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def read_profile_us(kernel):
    """average duration (us) of a kernel class in the committed rocprofv3
    --kernel-trace --stats summary of the decode set, if there is one and it
    was made from the current kernel sources (its '# sources:' digest)"""
    path = os.path.join(ROOT, "profiles", DECODE_PROFILE)
    sig = PROFILE_NAMES.get(kernel)
    if not sig or not os.path.exists(path):
        return None
    digest = None
    for line in open(path):
        if line.startswith("# sources:"):
            digest = line.split(":", 1)[1].split()[0]
    if digest != kernel_sources_digest():
        return None
    for line in open(path):
        if line.startswith("#"):
            continue
        parts = line.split(None, 4)
        if len(parts) == 5 and sig in parts[4]:
            try:
                return float(parts[1]) / 1e3
            except ValueError:
                return None
    return None


def read_traffic(kernel):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if any"""
    path = os.path.join(ROOT, "profiles", f"{kernel}_traffic.txt")
    if not os.path.exists(path):
        return None
    vals = {}
    for line in open(path):
        if ":" in line and not line.startswith("#"):
            k, v = line.split(":", 1)
            try:
                vals[k.strip()] = float(v.split()[0])
            except (ValueError, IndexError):
                pass
    return vals.get("traffic_bytes_per_launch")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="skip per-kernel and GEMM tables")
    ap.add_argument("--no-gemm-tables", action="store_true",
                    help="skip the GEMM tables (keeps the per-kernel decode timing); the profiled run "
                         "of the decode set uses it, the GEMM shapes are profiled one by one")
    ap.add_argument("--no-graph", action="store_true",
                    help="launch the kernels of a step one by one instead of replaying a graph")
    ap.add_argument("--per-call", action="store_true",
                    help="headline on the per-call GEMV kernels instead of the persistent decode-set "
                         "launch (both are measured either way)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a 512 MiB copy and a 512 MiB read-only stream (traffic-counter calibration)")
    ap.add_argument("--no-model", action="store_true", help="skip the full-forward and batched-decode measurements")
    ap.add_argument("--gemm-shape", default=None, metavar="M,K,N,GATED",
                    help="only time one GEMM shape on its automatic plan (--steps launches, "
                         "graph-replayed) and print one JSON line; for profiling runs")
    ap.add_argument("--cpu-baseline-child", type=float, default=None, help=argparse.SUPPRESS)
    ap.add_argument("--cpu-model-child", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()

    if args.cpu_baseline_child is not None:
        cpu_baseline_child(args.cpu_baseline_child)
        return 0
    if args.cpu_model_child:
        cpu_model_child()
        return 0
    if args.gemm_shape:
        M, K, N, gated = (int(v) for v in args.gemm_shape.split(","))
        g = Gpu()
        a = g.alloc(4 * M * K)
        g.fill_f32(a, M * K, 31)
        w = g.alloc(2 * N * K * (2 if gated else 1))
        g.fill_bf16(w, N * K * (2 if gated else 1), 32)
        c = g.alloc(4 * M * N)
        e = gemm_entry(g, M, K, N, bool(gated), a, c, w, reps=max(1, args.steps))
        print(json.dumps({"gemm_shape": e}))
        return 0
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the hot path is a "
                                   "single-GPU GEMM/GEMV library; sharding is designed, "
                                   "not built", "n_gpus": args.gpus}))
        return 2

    # CPU baselines before this process touches the GPU: the full-forward one
    # runs in the background on the last core until the model measurements
    cpu_model_proc = None if (args.no_cpu_baseline or args.no_model) else start_cpu_model()
    cpu = None if args.no_cpu_baseline else run_cpu_baseline(args.cpu_budget)

    g = Gpu()
    layers, emb, act = build_decode_model(g)
    per_call = time_step(g, lambda: decode_step(g, layers, emb, act), not args.no_graph,
                         args.warmup, args.steps)
    # the same step with the 112 layer GEMVs in one persistent launch: the
    # headline when the device keeps its grid resident and no launch gave up
    # waiting on its exchange (then its outputs would be invalid); the
    # per-call step is measured beside it either way
    pers = None
    if g.L.qwen3_hip_decode_set_supported():
        launch_set = persistent_step(g, layers, emb, act)
        pers = time_step(g, launch_set, not args.no_graph, args.warmup, args.steps)
        flags = ctypes.c_uint(0)
        g.rt.check(g.L.qwen3_hip_decode_set_errors(ctypes.byref(flags)), "decode_set_errors")
        pers["exchange_errors"] = flags.value
    persistent = use_persistent(pers, args.per_call)
    ms_step, wall = (pers if persistent else per_call)["ms_per_step"], (pers if persistent else per_call)["wall_s"]
    value = 1000.0 / ms_step
    kclasses = None if args.no_extras else kernel_classes(g, layers, emb, act)
    if kclasses is not None and pers:
        kclasses["decode_set_persistent"] = persistent_class(g, launch_set)
    roofline = None
    if kclasses:
        # the kernel with the largest share of the headline step's time
        used = ("decode_set_persistent", "lm_head_gemv") if persistent else \
            ("qkv_gemv", "o_gemv", "gate_up_silu_gemv", "down_gemv", "lm_head_gemv")
        dom = max(used, key=lambda k: kclasses[k]["us_per_step"])
        d = kclasses[dom]
        # achieved / frac: algorithmic bytes over the kernel's average duration
        # in the committed rocprofv3 kernel trace (profiles/); the live figure
        # from this run's graph replay (launch period of back-to-back
        # dependent launches, HIP events on the library stream) beside it.
        # For the 3-4 us GEMVs the profiler's per-dispatch time exceeds the
        # replay period: with the profiler attached every dispatch carries
        # its own completion signal and time stamps.
        prof_us = read_profile_us(dom)
        nb = d["bytes_per_launch"]
        roofline = {"bound": "hbm", "kernel": dom,
                    "achieved": round(nb / (prof_us * 1e-6) / 1e9, 1) if prof_us else round(d["GBps"], 1),
                    "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(nb / (prof_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4) if prof_us
                    else round(d["hbm_frac"], 4),
                    "traffic": read_traffic(dom), "bytes_per_launch": nb,
                    "us_per_launch_profile": prof_us,
                    "profile": f"profiles/{DECODE_PROFILE}" if prof_us else None,
                    "profile_sources_sha256": kernel_sources_digest()[:16] if prof_us else None,
                    "us_per_launch_graph_replay": round(d["us_per_launch"], 3),
                    "frac_graph_replay": round(d["hbm_frac"], 4),
                    "method": "frac = bytes_per_launch / rocprofv3 average duration / peak, from the committed "
                              "profile when it was made from these kernel sources (sha256 of the GPU sources), else "
                              "frac = frac_graph_replay = bytes_per_launch / graph-replay launch period / peak"}
    gemms = None if (args.no_extras or args.no_gemm_tables) else gemm_tables(g)
    if args.calibrate_copy:
        # kernels of known traffic for scaling FETCH_SIZE / WRITE_SIZE counters
        # in profiled runs, each over 512 MiB (twice the 256 MB last-level
        # cache, so every byte goes to or from HBM): a copy (512 MiB read +
        # 512 MiB written per launch) and a read-only stream in the decode
        # GEMVs' load form (512 MiB read)
        nb = 512 << 20
        src, dst = g.alloc(nb), g.alloc(nb)
        for _ in range(5):
            g.rt.check(g.L.qwen3_hip_copy_dev(ctypes.c_void_p(dst), ctypes.c_void_p(src), nb), "copy")
        for _ in range(5):
            g.rt.check(g.L.qwen3_hip_read_dev(ctypes.c_void_p(src), nb), "read")
        g.sync()

    model = batch = None
    if not args.no_model:
        model = model_forward_p128_d128()
        model["cpu_baseline"] = None
        if cpu_model_proc is not None:
            print("waiting for the full-forward CPU baseline", file=sys.stderr, flush=True)
            model["cpu_baseline"] = finish_cpu_model(cpu_model_proc)
        batch = model_batch_decode()
    hostp = None if args.no_extras else host_path()

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: random bf16 weights N(0,0.02), fp32 activations N(0,1) rounded to bf16",
        "config": {"workload": "Qwen3-0.6B decode GEMV set at M=1: 28 layers x (q|k|v 1024->4096, "
                               "o 2048->1024, gate|up+SiLU 1024->2x3072, down 3072->1024) + "
                               "lm_head 1024->151936; distinct weights per layer",
                   "M": 1, "layers": LAYERS, "step_bytes": STEP_BYTES,
                   "launches_per_step": 2 if persistent else 4 * LAYERS + 1,
                   "path": ("persistent: the 28 layers' 112 GEMVs in one launch + the lm_head GEMV"
                            if persistent else "per-call GEMV kernels"),
                   "hip_graph": not args.no_graph},
        # the step as 113 dependent per-call GEMV launches, and as one persistent
        # launch of the 112 layer GEMVs + the lm_head GEMV (both graph-replayed)
        "per_call_step": {"tok_s": round(1000.0 / per_call["ms_per_step"], 2),
                          "ms_per_step": round(per_call["ms_per_step"], 4)},
        "persistent_step": None if not pers else {
            "tok_s": round(1000.0 / pers["ms_per_step"], 2), "ms_per_step": round(pers["ms_per_step"], 4),
            "exchange_errors": pers["exchange_errors"]},
        "hbm_GBps_step": round(STEP_BYTES / (ms_step * 1e-3) / 1e9, 1),
        # the full Qwen3-0.6B forward (128-token prompt + 128 greedy steps, batch 1): decode tok/s
        "model_decode_tok_s": model["decode_tok_s"] if model else None,
        "wall_s": round(wall, 3),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": kclasses,
        "gemm": gemms,
        "model_forward_p128_d128": model,
        "model_batch_decode": batch,
        "host_pointer_path": hostp,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
