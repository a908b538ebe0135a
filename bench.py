#!/usr/bin/env python3
"""Benchmark of BybyLang's quantized tile-GEMM path on one MI355X (libbybyhip.so).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs c1,c2,c3,c4]

Prints ONE JSON line. The headline (`value`) is config 1 of BASELINE.json: the decode Q4 GEMV
(M=1, K=4096, N=14336, block-32 Q4 weights with fp16 scales, fp16 x and y, fp32 accumulation) in
GB/s of algorithmic bytes, inputs resident in HBM. A step is one GEMV launch. Each measurement is
one session recording (a HIP graph) of a lead-in (a full rotation of the resident weight copies,
then the W warmup steps) followed by exactly K timed steps, with a timing mark before and after
the K steps: a one-thread kernel storing the GPU's constant-rate realtime counter
(byhip_session_mark). Before it, a settle phase replays the rotation for 200 ms of GPU time so the
clocks have left idle. The GEMV cycles through 17 resident weight copies (562 MB, more than twice
the 256 MB Infinity Cache), and the rotation continues across the phases, so every read comes from
HBM. The other configurations (prefill Q4 GEMM, MXFP4 GEMM, the decoder-layer batch, the fused
decode layer) are reported under "configs" with the same method.

roofline.traffic: HBM bytes per launch of the GEMV, read from profiles/q4_gemv_c1_traffic.json,
which bybylang_amd.profile_summary writes from two rocprofv3 --pmc runs of this script
(FETCH_SIZE, WRITE_SIZE) with --copy-probe, each counter scaled by what it reads for the
library's copy kernel moving a known number of bytes in the same run; null when that file is
absent.

cpu_baseline: the reference's CPU path for this op (nimf_cpu_matmul_q4,
backends/cpu/cpu_kernels_impl.inc:293-319) through its C restatement in oracle/ (kind "port", pinned
bit-exact to the reference's own C on the CPU tests), single threaded as the reference runs, on full
config-1 passes. cpu_baselines: the same path on every configuration (the CPU VM's
OP_TILE_GEMM for the FP4 one), on one core and on all the host's cores (at most 16, the box's
share), splitting rows or columns over threads with bit-identical per-output loops; configs whose
full run would take minutes time a stated row subset and scale linearly in M.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
FP16_PEAK_TFLOPS = 2500.0    # dense fp16 / bf16 MFMA
FP4_PEAK_TFLOPS = 10100.0    # dense fp4 MFMA
ROTATE_BYTES = 512 << 20     # weight copies past the 256 MB Infinity Cache


def q4_bytes(M, K, N):
    """Algorithmic bytes of a Q4 GEMV/GEMM in the benchmark format: nibbles, one fp16 scale per
    32 weights, fp16 x and y."""
    return N * K // 2 + N * (K // 32) * 2 + M * K * 2 + M * N * 2


def mx_bytes(M, K, N):
    return M * K // 2 + M * K // 32 + N * K // 2 + N * K // 32 + M * N * 2


class Recorder:
    """Records `fn(step)` for `count` steps as one session recording (a HIP graph)."""

    @staticmethod
    def gb_module():
        from bybylang_amd import gpubackend as gb
        return gb

    def __init__(self, fn, count):
        gb = self.gb = self.gb_module()
        assert gb.sessionBeginRecording(gb.gbHip), gb.sessionGetLastError(gb.gbHip)
        for i in range(count):
            fn(i)
        assert gb.sessionEnd(gb.gbHip), gb.sessionGetLastError(gb.gbHip)
        self.id = gb.sessionLastRecording(gb.gbHip)
        assert self.id >= 0

    def timed(self, times=1) -> float:
        """Replays and returns the GPU seconds between the events around the launches."""
        gb = self.gb
        assert gb.sessionSetGpuTiming(gb.gbHip, True)
        assert gb.sessionReplay(gb.gbHip, self.id, times), gb.sessionGetLastError(gb.gbHip)
        t = gb.sessionGpuSeconds(gb.gbHip)
        gb.sessionSetGpuTiming(gb.gbHip, False)
        return t

    def close(self):
        self.gb.sessionFreeRecording(self.gb.gbHip, self.id)


SETTLE_MS = 200.0  # GPU time of untimed work before each timing, so the clocks are out of idle
# The timing marks are the library's events recorded inside the recording, around exactly the
# timed steps (byhip_session_mark); without them (BENCH_MARKS=0) the lead-in and the timed steps are
# two recordings queued back to back with events between them (byhip_session_replay_after).
MARKS_IN_RECORDING = os.environ.get("BENCH_MARKS", "1") != "0"
# --eager: every step's kernels are launched directly (no recording, no replay), between the same
# realtime-counter marks. For profiler runs: the host's launch gaps are then inside the timed
# region, so the per-step figures are upper bounds; the kernel durations the profiler reports
# are the kernels' own.
EAGER = False
# --graph: recordings are HIP graphs. By default they keep their launches and replay them directly
# (byhip_session_set_direct_replay), so that a kernel-trace profiler sees exactly the timed launches.
GRAPH = False


def run_steps_eager(fn, steps, warmup, settle_steps=8):
    """run_steps without recordings: the settle rotation is launched directly until SETTLE_MS of
    wall time has passed, then the W warmup steps, then the timed steps between two marks."""
    from bybylang_amd import _abi
    gb = Recorder.gb_module()
    lib = _abi.load()
    end = time.perf_counter() + SETTLE_MS * 1e-3
    while time.perf_counter() < end:
        for i in range(settle_steps):
            fn(i - settle_steps)
        _abi.check(lib.byhip_synchronize(), "synchronize")
    for i in range(warmup):
        fn(i)
    assert gb.sessionSetGpuTiming(gb.gbHip, True)
    wall0 = time.perf_counter()
    _abi.check(lib.byhip_session_mark(0), "mark")
    for i in range(steps):
        fn(warmup + i)
    _abi.check(lib.byhip_session_mark(1), "mark")
    _abi.check(lib.byhip_session_take_marks(), "marks")
    wall = time.perf_counter() - wall0
    gpu_s = gb.sessionGpuSeconds(gb.gbHip)
    gb.sessionSetGpuTiming(gb.gbHip, False)
    return gpu_s, wall


def run_steps(fn, steps, warmup, settle_steps=8):
    """Returns (GPU seconds of exactly `steps` timed steps, wall seconds of that replay).

    Step indices are global and every rotation continues across the phases: the settle recording
    is fn(-settle_steps .. -1), the warmup fn(0 .. W-1), the timed run fn(W .. W+S-1). Recordings
    run once when they are made; the settle recording (one full weight rotation where the caller
    rotates copies) is then replayed until SETTLE_MS of GPU time has passed, which also leaves
    every copy's last read in rotation order. Finally the lead-in recording (the settle rotation,
    then the W warmup steps) and the timed recording are queued back to back and only the latter
    is timed: the lead-in lasts long enough for the host to queue the timed launch behind it, so
    the GPU never waits for the host inside the timed region, and the first timed step reads a copy
    last read a whole rotation earlier."""
    if EAGER:
        return run_steps_eager(fn, steps, warmup, settle_steps)
    from bybylang_amd import _abi
    gb = Recorder.gb_module()
    lib = _abi.load()
    settle = Recorder(lambda i: fn(i - settle_steps), settle_steps)
    marked = MARKS_IN_RECORDING

    def whole(i):
        # lead-in and timed steps in one recording, the timing marks between them
        if marked and i == settle_steps + warmup:
            _abi.check(lib.byhip_session_mark(0), "mark")
        fn(i - settle_steps)
        if marked and i == settle_steps + warmup + steps - 1:
            _abi.check(lib.byhip_session_mark(1), "mark")

    if marked:
        run = Recorder(whole, settle_steps + warmup + steps)
        recs = (settle, run)
    else:
        lead = Recorder(lambda i: fn(i - settle_steps), settle_steps + warmup)
        timed = Recorder(lambda i: fn(i + warmup), steps)
        recs = (settle, lead, timed)
    spent = 0.0
    while spent < SETTLE_MS * 1e-3:
        spent += settle.timed()
    assert gb.sessionSetGpuTiming(gb.gbHip, True)
    wall0 = time.perf_counter()
    if marked:
        _abi.check(lib.byhip_session_replay_marked(run.id), "replay")
    else:
        _abi.check(lib.byhip_session_replay_after(lead.id, 1, timed.id, 1), "replay")
    wall = time.perf_counter() - wall0
    gpu_s = gb.sessionGpuSeconds(gb.gbHip)
    gb.sessionSetGpuTiming(gb.gbHip, False)
    for r in recs:
        r.close()
    return gpu_s, wall


def q4_setup(dev, synth, seed, M, K, N, copies):
    g = synth.rng(seed)
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    ws = [dev.Q4Weights(wq, sc, ze, K, N, 32, K // 32) for _ in range(copies)]
    x = dev.DeviceBuffer.from_array(synth.activations(g, M, K, np.float16).reshape(-1))
    y = dev.DeviceBuffer(M * N * 2)
    return ws, x, y


def bench_c1(dev, synth, steps, warmup):
    M, K, N = 1, 4096, 14336
    nbytes = q4_bytes(M, K, N)
    copies = max(1, -(-ROTATE_BYTES // nbytes))
    ws, x, y = q4_setup(dev, synth, 1, M, K, N, copies)
    fn = lambda i: dev.q4_matmul(x, dev.F16, ws[i % copies], y, dev.F16, M)  # noqa: E731
    gpu_s, wall = run_steps(fn, steps, warmup, settle_steps=copies)
    per = gpu_s / steps
    res = {"M": M, "K": K, "N": N, "bytes_per_step": nbytes, "weight_copies": copies,
           "rotation_bytes": nbytes * copies, "us_per_step": per * 1e6,
           "GBps": nbytes / per / 1e9, "TFLOPs": 2 * M * K * N / per / 1e12,
           "wall_us_per_step": wall / steps * 1e6}
    for w in ws:
        w.close()
    return res


def bench_long_k(dev, synth, steps, warmup):
    """Decode at long rows (the GEMV in K slices): a 70B-class down projection, M = 1, K = 28,672,
    N = 8,192, fp16 x and y, weights rotated past the Infinity Cache as in c1; and the fused
    silu(gate) * up GEMV over two such matrices' shape (K = 28,672, N = 2 x 4,096, fp32 input
    with the norm)."""
    out = {}
    M, K, N = 1, 28672, 8192
    nbytes = q4_bytes(M, K, N)
    copies = max(1, -(-ROTATE_BYTES // nbytes))
    ws, x, y = q4_setup(dev, synth, 5, M, K, N, copies)
    fn = lambda i: dev.q4_matmul(x, dev.F16, ws[i % copies], y, dev.F16, M)  # noqa: E731
    gpu_s, _ = run_steps(fn, steps, warmup, settle_steps=copies)
    per = gpu_s / steps
    out["gemv_M1_K28672_N8192"] = {"us": per * 1e6, "GBps": nbytes / per / 1e9, "bytes": nbytes}
    for w in ws:
        w.close()
    Kf, Nf = 28672, 4096
    fb = fused_bytes(1, Kf, [Nf, Nf], True, False)
    copies = max(1, -(-ROTATE_BYTES // fb))
    g = synth.rng(6)
    mats = []
    for _ in range(2):
        wq, sc, ze, _ = synth.q4_weights(g, Nf, Kf)
        mats.append([dev.Q4Weights(wq, sc, ze, Kf, Nf, 32, Kf // 32) for _ in range(copies)])
    a = dev.DeviceBuffer.from_array(g.standard_normal(Kf).astype(np.float32))
    gamma = dev.DeviceBuffer.from_array((1.0 + 0.1 * g.standard_normal(Kf)).astype(np.float32))
    outs = [dev.DeviceBuffer(Nf * 4) for _ in range(2)]

    def call(i):
        assert dev.q4_matmul_fused(1, a, [m[i % copies] for m in mats], outs, None, gamma, 1e-5) == 0

    gpu_s, _ = run_steps(call, steps, warmup, settle_steps=copies)
    per = gpu_s / steps
    out["fused_gate_up_norm_K28672_N4096x2"] = {"us": per * 1e6, "GBps": fb / per / 1e9, "bytes": fb}
    for m in mats:
        for w in m:
            w.close()
    return out


def bench_c0(dev, synth, steps, warmup):
    """Config 0's shape on the GPU at the reference's session dtype (fp32 activations and outputs,
    M = 16, K = N = 4096), and the same weights at M = 512 (fp32 prefill): weights rotated past
    the Infinity Cache as in c1."""
    K, N = 4096, 4096
    out = {}
    copies = max(1, -(-ROTATE_BYTES // q4_bytes(1, K, N)))
    g = synth.rng(0)
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    ws = [dev.Q4Weights(wq, sc, ze, K, N, 32, K // 32) for _ in range(copies)]
    for M in (16, 512):
        x = dev.DeviceBuffer.from_array(synth.activations(g, M, K, np.float32).reshape(-1))
        y = dev.DeviceBuffer(M * N * 4)
        fn = lambda i, M=M, x=x, y=y: dev.q4_matmul(x, dev.F32, ws[i % copies], y, dev.F32, M)  # noqa: E731
        gpu_s, _ = run_steps(fn, steps, warmup, settle_steps=copies)
        per = gpu_s / steps
        flops, b = 2 * M * K * N, q4_bytes(M, K, N) + M * K * 2 + M * N * 2  # fp32 x and y
        out[f"M{M}"] = {"M": M, "K": K, "N": N, "us_per_step": per * 1e6, "TFLOPs": flops / per / 1e12,
                        "GBps": b / per / 1e9}
    out["weight_copies"] = copies
    for w in ws:
        w.close()
    return out


def bench_c2(dev, synth, steps, warmup):
    M, K, N = 512, 4096, 4096
    ws, x, y = q4_setup(dev, synth, 2, M, K, N, 1)
    fn = lambda i: dev.q4_matmul(x, dev.F16, ws[0], y, dev.F16, M)  # noqa: E731
    gpu_s, wall = run_steps(fn, steps, warmup)
    per = gpu_s / steps
    flops = 2 * M * K * N
    return {"M": M, "K": K, "N": N, "flops_per_step": flops, "bytes_per_step": q4_bytes(M, K, N),
            "us_per_step": per * 1e6, "TFLOPs": flops / per / 1e12,
            "frac_fp16_peak": flops / per / 1e12 / FP16_PEAK_TFLOPS, "GBps": q4_bytes(M, K, N) / per / 1e9}


def bench_c3(dev, synth, steps, warmup):
    M, K, N = 2048, 8192, 8192
    g = synth.rng(3)
    xb, _, _ = synth.mxfp4_operand(g, M, K)
    wb, _, _ = synth.mxfp4_operand(g, N, K)
    x = dev.DeviceBuffer.from_array(xb)
    w = dev.DeviceBuffer.from_array(wb)
    y = dev.DeviceBuffer(M * N * 2)
    fn = lambda i: dev.mxfp4_gemm(x, w, y, dev.BF16, M, K, N)  # noqa: E731
    gpu_s, wall = run_steps(fn, steps, warmup)
    per = gpu_s / steps
    flops = 2 * M * K * N
    return {"M": M, "K": K, "N": N, "flops_per_step": flops, "bytes_per_step": mx_bytes(M, K, N),
            "us_per_step": per * 1e6, "TFLOPs": flops / per / 1e12,
            "frac_fp4_peak": flops / per / 1e12 / FP4_PEAK_TFLOPS}


C4_OPS = [("qkv", 4096, 6144), ("o", 4096, 4096), ("gate_up", 4096, 2 * 14336), ("down", 14336, 4096)]


def bench_c4(dev, synth, steps, warmup, tuned=False):
    out = {}
    layer_bytes = {M: sum(q4_bytes(M, K, N) for _, K, N in C4_OPS) for M in (1, 32, 256)}
    copies = max(1, -(-ROTATE_BYTES // layer_bytes[1]))
    g = synth.rng(4)
    weights = []
    for name, K, N in C4_OPS:
        wq, sc, ze, _ = synth.q4_weights(g, N, K)
        weights.append([dev.Q4Weights(wq, sc, ze, K, N, 32, K // 32) for _ in range(copies)])
    for M in (1, 32, 256):
        xs = [dev.DeviceBuffer.from_array(synth.activations(g, M, K, np.float16).reshape(-1))
              for _, K, _ in C4_OPS]
        ys = [dev.DeviceBuffer(M * N * 2) for _, _, N in C4_OPS]
        per_op = {}
        for j, (name, K, N) in enumerate(C4_OPS):
            fn = lambda i, j=j: dev.q4_matmul(xs[j], dev.F16, weights[j][i % copies], ys[j], dev.F16, M)  # noqa: E731
            gpu_s, _ = run_steps(fn, steps, warmup, settle_steps=copies)
            per = gpu_s / steps
            b, f = q4_bytes(M, K, N), 2 * M * K * N
            per_op[name] = {"us": per * 1e6, "GBps": b / per / 1e9, "TFLOPs": f / per / 1e12}

        def layer(i):
            for j in range(len(C4_OPS)):
                dev.q4_matmul(xs[j], dev.F16, weights[j][i % copies], ys[j], dev.F16, M)

        gpu_s, _ = run_steps(layer, steps, warmup, settle_steps=copies)
        per = gpu_s / steps
        flops = sum(2 * M * K * N for _, K, N in C4_OPS)
        out[f"M{M}"] = {"per_op": per_op, "batch_us": per * 1e6,
                        "batch_GBps": layer_bytes[M] / per / 1e9, "batch_TFLOPs": flops / per / 1e12}
        if tuned and M > 1:
            # residentPrepareQ4 for each projection at this M (plans tuned outside the timed region,
            # into a fresh plan directory), then the same batch again
            import tempfile
            with tempfile.TemporaryDirectory() as d:
                os.environ["BYHIP_CACHE_DIR"] = d
                plans = {}
                for j, (name, K, N) in enumerate(C4_OPS):
                    for w in weights[j]:
                        dev.q4_prepare(w, M, dev.F16)
                    info = dev.q4_plan_info(weights[j][0], M, dev.F16)
                    plans[name] = info[0] if info else None
                gpu_s, _ = run_steps(layer, steps, warmup, settle_steps=copies)
                per = gpu_s / steps
                out[f"M{M}"]["tuned"] = {"batch_us": per * 1e6, "plans": plans}
                dev.q4_plans_reset()
                del os.environ["BYHIP_CACHE_DIR"]
    for ws in weights:
        for w in ws:
            w.close()
    out["weight_copies"] = copies
    out["M1_fused"] = bench_c4_fused(dev, synth, steps, warmup)
    return out


def bench_upload_mapped(synth, mib: int = 512, repeats: int = 3):
    """residentUploadQ4Mapped from a checkpoint file mapped read-only: the nibble rows of a
    K = 4096 matrix of `mib` MiB copied straight from the mapping into HBM (host to device; the
    file is read once beforehand so the pages are resident). Best of `repeats` uploads."""
    import tempfile
    from bybylang_amd import gpubackend as gb
    K = 4096
    N = (mib << 20) // (K // 2)
    g = synth.rng(9)
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    with tempfile.NamedTemporaryFile(suffix=".bin", delete=False) as f:
        f.write(wq.tobytes())
        path = f.name
    del wq
    try:
        m = gb.openReadOnlyMapping(path)
        np.frombuffer(m.backing[0], dtype=np.uint8).sum(dtype=np.uint64)  # touch every page
        best = None
        for _ in range(repeats):
            t0 = time.perf_counter()
            w, zero_copy = gb.residentUploadQ4Mapped(gb.gbHip, m.data, m.size, sc, ze, K, N, 32, K // 32)
            dt = time.perf_counter() - t0
            gb.residentFreeQ4(w)
            best = dt if best is None else min(best, dt)
        size = m.size
        gb.unmapReadOnlyFile(m)
    finally:
        os.unlink(path)
    return {"bytes": size, "ms": best * 1e3, "GBps": size / best / 1e9, "zero_copy": zero_copy,
            "note": "host to device (pageable mapping); includes scale repacking and upload"}


# The same decode layer (M = 1) through the fused entry point (sessionMatmulQ4Fused): attention
# norm + QKV as three matrices sharing the input, O + residual, MLP norm + silu(gate) * up, down +
# residual. fp32 input, outputs, norm weights and residual, as the reference's session ops.
C4_FUSED = [("qkv_norm", 0, 4096, [4096, 1024, 1024], True, False),
            ("o_res", 0, 4096, [4096], False, True),
            ("gate_up_norm_silu", 1, 4096, [14336, 14336], True, False),
            ("down_res", 0, 14336, [4096], False, True)]


def fused_bytes(mode, K, Ns, norm, res):
    """Weights (nibbles, fp16 scales) plus fp32 input, outputs (one in mode 1), norm weights and
    residual."""
    w = sum(N * K // 2 + N * (K // 32) * 2 for N in Ns)
    n_out = Ns[0] if mode == 1 else sum(Ns)
    return w + K * 4 + n_out * 4 + (K * 4 if norm else 0) + (max(Ns) * 4 if res else 0)


def bench_c4_fused(dev, synth, steps, warmup):
    layer_bytes = sum(fused_bytes(md, K, Ns, nm, rs) for _, md, K, Ns, nm, rs in C4_FUSED)
    copies = max(1, -(-ROTATE_BYTES // layer_bytes))
    g = synth.rng(44)
    ops = []
    for name, mode, K, Ns, norm, res in C4_FUSED:
        mats = []
        for N in Ns:
            wq, sc, ze, _ = synth.q4_weights(g, N, K)
            mats.append([dev.Q4Weights(wq, sc, ze, K, N, 32, K // 32) for _ in range(copies)])
        a = dev.DeviceBuffer.from_array(g.standard_normal(K).astype(np.float32))
        outs = [dev.DeviceBuffer(N * 4) for N in Ns]
        gamma = dev.DeviceBuffer.from_array((1.0 + 0.1 * g.standard_normal(K)).astype(np.float32)) if norm else None
        r = dev.DeviceBuffer.from_array(g.standard_normal(max(Ns)).astype(np.float32)) if res else None
        ops.append((name, mode, K, Ns, norm, res, mats, a, outs, gamma, r))

    def call(op, i):
        name, mode, K, Ns, norm, res, mats, a, outs, gamma, r = op
        rc = dev.q4_matmul_fused(mode, a, [m[i % copies] for m in mats], outs, r, gamma, 1e-5)
        assert rc == 0, f"fused {name} unsupported"

    out = {"per_op": {}}
    for op in ops:
        name, mode, K, Ns, norm, res = op[:6]
        gpu_s, _ = run_steps(lambda i, op=op: call(op, i), steps, warmup, settle_steps=copies)
        per = gpu_s / steps
        out["per_op"][name] = {"us": per * 1e6, "GBps": fused_bytes(mode, K, Ns, norm, res) / per / 1e9}

    def layer(i):
        for op in ops:
            call(op, i)

    gpu_s, _ = run_steps(layer, steps, warmup, settle_steps=copies)
    per = gpu_s / steps
    out.update({"batch_us": per * 1e6, "batch_GBps": layer_bytes / per / 1e9, "weight_copies": copies,
                "launches": len(C4_FUSED)})

    # The unfused sequence's GEMVs: the same seven matrices as plain fp32-in, fp32-out GEMVs (one
    # launch each, the input of the norm-free form). Its RMSNorms, silu * up and residual adds (five
    # more launches) are not kernels of this library and are not timed: this is a lower bound of
    # the unfused layer.
    ys = {(op[0], j): dev.DeviceBuffer(N * 4) for op in ops for j, N in enumerate(op[3])}

    def unfused(i):
        for name, mode, K, Ns, norm, res, mats, a, outs, gamma, r in ops:
            for j, N in enumerate(Ns):
                dev.q4_matmul(a, dev.F32, mats[j][i % copies], ys[(name, j)], dev.F32, 1)

    gpu_s, _ = run_steps(unfused, steps, warmup, settle_steps=copies)
    out["unfused_gemvs"] = {"us": gpu_s / steps * 1e6, "launches": sum(len(op[3]) for op in ops),
                            "note": "7 plain fp32 GEMVs only; the unfused layer adds 2 RMSNorms, silu*up and "
                                    "2 residual adds (5 launches) not timed here"}
    for y in ys.values():
        y.close()
    for op in ops:
        for m in op[6]:
            for w in m:
                w.close()
    return out


class CpuPath:
    """The reference's CPU path for this op, timed on the host through its C restatement in
    oracle/ (kind "port"): orc_matmul_q4 (nimf_cpu_matmul_q4, cpu_kernels_impl.inc:293-319) for
    Q4 and orc_tile_gemm (the CPU VM's OP_TILE_GEMM, cpu_vm.c:583-628) for FP4-KM, the same loops
    in the same order, bit-exact to the reference's own C on the CPU tests. The reference runs
    single-threaded; the all-core figures split rows (or, at M = 1, columns) over threads, each
    thread running the same per-output loops, so the outputs are bit-identical to one thread's."""

    def __init__(self):
        port = os.path.join(ROOT, "oracle", "liboracle.so")
        if not os.path.exists(port):
            raise FileNotFoundError("no CPU path built (oracle/liboracle.so)")
        self.lib, self.kind = C.CDLL(port), "port"
        self.lib.orc_matmul_q4.argtypes = [C.c_void_p] * 5 + [C.c_int] * 7
        self.lib.orc_tile_gemm.argtypes = ([C.c_uint32] * 4 + [C.c_uint64] * 2 +
                                           [C.c_void_p, C.c_int64, C.c_void_p, C.c_int64, C.c_void_p,
                                            C.c_int64, C.c_void_p, C.c_int64, C.c_uint32, C.c_uint32,
                                            C.c_char_p, C.c_int])

    def q4(self, a, wq, sc, ze, c, M, K, N):
        """Q4 group 32 on host pointers (a [M, K] fp32, rows of wq, fp32 scales / zeros, c [M, N])."""
        self.lib.orc_matmul_q4(a, wq, sc, ze, c, M, K, N, 32, K // 32, 0, M)

    def fp4(self, x, blob, blob_len, table, out, M, K, N):
        """The FP4-KM tile GEMM (the c3 format) on M rows: the CPU VM's OP_TILE_GEMM."""
        err = C.create_string_buffer(256)
        rc = self.lib.orc_tile_gemm(0, M, K, N, N * (K // 2), 0, blob, blob_len, table, 272, x, M * K,
                                    out, M * N, 0, M, err, 256)
        assert rc == 0, err.value


def cpu_threads() -> int:
    """Threads for the all-core figures: the host's cores, at most the box's CPU share (16, as
    OMP_NUM_THREADS says there)."""
    n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, min(n, 16))


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _timed(fn, min_seconds):
    """Seconds per call of fn, over at least min_seconds (and at least one call)."""
    calls, t0 = 0, time.perf_counter()
    while True:
        fn()
        calls += 1
        el = time.perf_counter() - t0
        if el >= min_seconds:
            return el / calls


def _parallel(jobs, threads):
    """Runs the callables on `threads` threads (ctypes releases the GIL inside the C calls)."""
    import concurrent.futures as cf
    with cf.ThreadPoolExecutor(max_workers=threads) as ex:
        for f in [ex.submit(j) for j in jobs]:
            f.result()


def cpu_q4_case(cpu, M, K, N, rows, threads, min_s, seed):
    """Seconds for all M rows of a Q4 product on 1 and on `threads` cores: `rows` rows timed (all
    of them when rows >= M) and scaled by M / rows; at M = 1 the all-core run splits columns."""
    from bybylang_amd import synth
    g = synth.rng(seed)
    wq, sc, ze, _ = synth.q4_weights(g, N, K)
    R = min(M, rows)
    a = synth.activations(g, R, K, np.float32).reshape(-1)
    c = np.zeros(R * N, np.float32)
    P = lambda arr, off=0: int(arr.ctypes.data + int(off) * arr.itemsize)  # noqa: E731
    one = _timed(lambda: cpu.q4(P(a), P(wq), P(sc), P(ze), P(c), R, K, N), min_s) * M / R
    gpr = K // 32
    if R == 1:  # columns split over the threads
        cuts = np.linspace(0, N, threads + 1).astype(int)
        jobs = [lambda n0=n0, n1=n1: cpu.q4(P(a), P(wq, n0 * (K // 2)), P(sc, n0 * gpr), P(ze, n0 * gpr), P(c, n0),
                                            1, K, n1 - n0) for n0, n1 in zip(cuts[:-1], cuts[1:]) if n1 > n0]
        allc = _timed(lambda: _parallel(jobs, threads), min_s) * M
    else:  # rows over the threads: every thread its own row block
        Ra = min(M, max(R, threads))
        aa = synth.activations(g, Ra, K, np.float32).reshape(-1)
        ca = np.zeros(Ra * N, np.float32)
        cuts = np.linspace(0, Ra, threads + 1).astype(int)
        jobs = [lambda r0=r0, r1=r1: cpu.q4(P(aa, r0 * K), P(wq), P(sc), P(ze), P(ca, r0 * N), r1 - r0, K, N)
                for r0, r1 in zip(cuts[:-1], cuts[1:]) if r1 > r0]
        allc = _timed(lambda: _parallel(jobs, threads), min_s) * M / Ra
    return one, allc, R


def cpu_baselines(threads: int, min_s: float = 0.8):
    """The reference CPU path on every configuration, one core and `threads` cores."""
    from bybylang_amd import synth
    cpu = CpuPath()
    out = {"kind": cpu.kind, "cpu_model": cpu_model(), "threads": threads, "nproc": os.cpu_count()}

    def entry(one, allc, flops, nbytes, sample):
        return {"s_1core": one, "s_all": allc, "GFLOPs_1core": flops / one / 1e9, "GFLOPs_all": flops / allc / 1e9,
                "GBps_1core": nbytes / one / 1e9, "GBps_all": nbytes / allc / 1e9, "sample": sample}

    for name, M, K, N, rows in (("c0", 16, 4096, 4096, 16), ("c1", 1, 4096, 14336, 1), ("c2", 512, 4096, 4096, 8)):
        one, allc, R = cpu_q4_case(cpu, M, K, N, rows, threads, min_s, 60)
        out[name] = entry(one, allc, 2 * M * K * N, q4_bytes(M, K, N),
                          "full" if R >= M else f"{R} of {M} rows timed, scaled linearly in M")
    # c3: the FP4-KM tile GEMM through the CPU VM, rows timed and scaled to M = 2048
    M, K, N = 2048, 8192, 8192
    g = synth.rng(63)
    blob, _, _ = synth.mxfp4_operand(g, N, K)
    table = synth.mx_table()
    table[16 + 255] = 0.0
    xs = synth.mx_decode(*synth.mxfp4_operand(g, threads, K)[1:]).reshape(-1)
    o = np.zeros(threads * N, np.float32)
    P = lambda arr, off=0: int(arr.ctypes.data + int(off) * arr.itemsize)  # noqa: E731
    one = _timed(lambda: cpu.fp4(P(xs), P(blob), blob.size, P(table), P(o), 1, K, N), min_s) * M
    jobs = [lambda r=r: cpu.fp4(P(xs, r * K), P(blob), blob.size, P(table), P(o, r * N), 1, K, N) for r in range(threads)]
    allc = _timed(lambda: _parallel(jobs, threads), min_s) * M / threads
    out["c3"] = entry(one, allc, 2 * M * K * N, mx_bytes(M, K, N),
                      f"1 row (1 core) and {threads} rows ({threads} cores) of {M}, scaled linearly in M")
    # c4: the four projections of the layer at M = 1, 32, 256
    for M in (1, 32, 256):
        one = allc = 0.0
        for j, (_, K, N) in enumerate(C4_OPS):
            o1, oa, _ = cpu_q4_case(cpu, M, K, N, 1, threads, min_s / 4, 70 + j)
            one, allc = one + o1, allc + oa
        flops = sum(2 * M * K * N for _, K, N in C4_OPS)
        nbytes = sum(q4_bytes(M, K, N) for _, K, N in C4_OPS)
        out[f"c4_M{M}"] = entry(one, allc, flops, nbytes,
                                "full" if M == 1 else f"1 row per projection (all-core: {threads} rows), scaled to M = {M}")
    return out


def cpu_baseline(baselines):
    """The headline's CPU figure: config 1 on one core, the reference's own single-threaded loops."""
    c1 = baselines["c1"]
    return {"value": c1["GBps_1core"], "unit": "GB/s", "cores": 1, "kind": baselines["kind"],
            "sample": f"full config-1 passes (M=1 K=4096 N=14336, fp32 x), {c1['s_1core'] * 1e3:.1f} ms each, "
                      f"orc_matmul_q4 (C restatement of nimf_cpu_matmul_q4, bit-exact to the reference build) single "
                      f"thread on {baselines['cpu_model']}; on {baselines['threads']} "
                      f"threads {c1['GBps_all']:.2f} GB/s"}


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "q4_gemv_c1_traffic.json")


def measured_traffic():
    """HBM bytes per GEMV launch from the committed counter summary, or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return int(round(t["traffic_bytes"]))
    except (OSError, KeyError, ValueError):
        return None


def bench_read_probe(dev):
    """byhip_debug_read, the plain streaming read the kernels' reads are compared with: over 1 GiB
    (the steady rate), and over config 1's bytes per launch (33,067,008 B) rotating through 32
    slices of that buffer, timed like config 1 (recorded launches, each reading cold)."""
    from bybylang_amd import _abi
    lib = _abi.load()
    big, sink = dev.DeviceBuffer(1 << 30), dev.DeviceBuffer(1 << 20)
    out = {}
    fn = lambda i: _abi.check(lib.byhip_debug_read(big.ptr, 1 << 30, sink.ptr, 1 << 20))  # noqa: E731
    gpu_s, _ = run_steps(fn, 10, 2)
    out["steady_1GiB_GBps"] = (1 << 30) / (gpu_s / 10) / 1e9
    part = q4_bytes(1, 4096, 14336)
    fn = lambda i: _abi.check(lib.byhip_debug_read(big.ptr + (i % 32) * part, part, sink.ptr, 1 << 20))  # noqa: E731
    gpu_s, _ = run_steps(fn, 200, 32)
    out["per_launch_c1_bytes"] = part
    out["per_launch_us"] = gpu_s / 200 * 1e6
    out["per_launch_GBps"] = part / (gpu_s / 200) / 1e9
    big.close()
    sink.close()
    return out


def copy_probe(mib: int, times: int = 10):
    """Runs the library's copy kernel on `mib` MiB device to device `times` times: the known
    transfer that a counter run scales FETCH_SIZE / WRITE_SIZE by."""
    from bybylang_amd import _abi
    from bybylang_amd import device as dev
    n = mib << 20
    src, dst = dev.DeviceBuffer(n), dev.DeviceBuffer(n)
    lib = _abi.load()
    for _ in range(times):
        _abi.check(lib.byhip_debug_copy(dst.ptr, src.ptr, n))
    dev.synchronize()
    src.close()
    dst.close()
    return n


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--configs", default="c0,c1,c2,c3,c4,lk,up,rp",
                    help="configurations to measure (c1 is the headline and always runs; c0 is config 0's shape at "
                         "fp32 in and out, M = 16 and 512); c4t is c4 "
                         "with the batch timed again after byhip_q4_prepare tunes each projection")
    ap.add_argument("--cpu-seconds", type=float, default=0.8,
                    help="minimum seconds per CPU-baseline measurement (0: no CPU baseline)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="also run the copy kernel on MIB MiB (calibration for counter runs)")
    ap.add_argument("--eager", action="store_true",
                    help="launch every step directly from Python instead of replaying recordings")
    ap.add_argument("--graph", action="store_true",
                    help="replay the recordings as HIP graphs (the default replays their kept launches "
                         "directly; graph replays are never run under a profiler)")
    args = ap.parse_args()
    global EAGER, GRAPH
    EAGER = args.eager
    GRAPH = args.graph
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        sys.stderr.write("bench.py measures one GPU only: this build has no multi-GPU path "
                         "(collectives are out of scope); run with --gpus 1\n")
        return 2
    if args.steps < 1:
        sys.stderr.write("--steps must be >= 1\n")
        return 2

    from bybylang_amd import device as dev
    from bybylang_amd import synth
    dev.init(0)
    from bybylang_amd import _abi
    _abi.check(_abi.load().byhip_session_set_direct_replay(0 if GRAPH else 1), "replay mode")
    info = dev.device_info()
    wanted = {c.strip() for c in args.configs.split(",") if c.strip()}
    probe = copy_probe(args.copy_probe) if args.copy_probe > 0 else 0

    c1 = bench_c1(dev, synth, args.steps, args.warmup)
    configs = {}
    if "c0" in wanted:
        configs["c0_session_fp32"] = bench_c0(dev, synth, args.steps, args.warmup)
    if "c2" in wanted:
        configs["c2_prefill_q4_gemm"] = bench_c2(dev, synth, args.steps, args.warmup)
    if "c3" in wanted:
        configs["c3_mxfp4_gemm"] = bench_c3(dev, synth, args.steps, args.warmup)
    if "c4" in wanted or "c4t" in wanted:
        configs["c4_layer_batch"] = bench_c4(dev, synth, args.steps, args.warmup, tuned="c4t" in wanted)
    if "lk" in wanted:
        configs["long_k_decode"] = bench_long_k(dev, synth, args.steps, args.warmup)
    if "up" in wanted:
        configs["resident_upload_mapped"] = bench_upload_mapped(synth)
    if "rp" in wanted:
        configs["hbm_read_probe"] = bench_read_probe(dev)
    baselines = cpu_baselines(cpu_threads(), args.cpu_seconds) if args.cpu_seconds > 0 else None
    cpu = cpu_baseline(baselines) if baselines else None

    per_s = c1["us_per_step"] * 1e-6
    line = {
        "metric": "Q4 GEMV GB/s (% HBM peak) at M=1; Q4/FP4 GEMM TFLOP/s (% MFMA peak) M>=512",
        "value": round(c1["GBps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": c1["us_per_step"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded PCG64: int4 codes uniform [-8,7], fp16 scales |N(0,0.02)|+1e-4, x ~ N(0,1))",
        "config": {"workload": "c1 decode Q4 GEMV: M=1 K=4096 N=14336, block-32 Q4 + fp16 scales, "
                               "fp16 x/y, fp32 accumulate",
                   "weight_copies": c1["weight_copies"], "rotation_bytes": c1["rotation_bytes"],
                   "timing": ("eager launches (profiler run): 200 ms settle, `warmup` steps, then `steps` "
                              "timed launches between two realtime-counter marks, host launch gaps included"
                              if EAGER else
                              "one recording (%s): rotation lead-in, `warmup` steps, then `steps` timed "
                              "launches between two realtime-counter marks; 200 ms settle before"
                              % ("HIP graph" if GRAPH else "kept launches replayed directly on the stream")),
                   "device": info.get("name", ""), "arch": info.get("arch_name", ""),
                   "compute_units": info.get("compute_units")},
        "roofline": {"bound": "hbm", "achieved": round(c1["GBps"], 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(c1["GBps"] / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(), "kernel": "q4_gemv",
                     "bytes_per_launch": c1["bytes_per_step"], "avg_launch_us": round(c1["us_per_step"], 3)},
        "cpu_baseline": cpu,
        "cpu_baselines": baselines,
        "configs": configs,
    }
    if probe:
        line["copy_probe_bytes"] = probe
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
