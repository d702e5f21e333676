#!/usr/bin/env python3
"""Benchmark of the quantized matrix products on one MI355X.

Step = one 9B-class decode layer's projections at batch 1 (Q8_K activations): quantize the
attention input, GEMV q (4096x4096), k, v (1024x4096); quantize the attention output, GEMV o
(4096x4096); quantize the FFN input, GEMV gate, up (12288x4096, all Q4_K); quantize the FFN
middle, GEMV down (4096x12288 Q6_K).  Weights are seeded N(0, 0.02) quantized by the repo's
quantizer; the layer is resident in HBM in 32 copies at distinct addresses (3.9 GB) and step i
uses copy i % 32, so the 256 MB Infinity Cache cannot serve repeats.  Steps are replayed from
HIP graphs (one graph of 32 steps plus a remainder graph) so host launch overhead is not timed.

value = algorithmic bytes per step (weights + activations read + outputs written, each once)
        / measured time per step, in GB/s.
Also reported: the dominant kernel's roofline fraction (Q4_K GEMV, per-launch HIP events), the
reference CPU path (kc_matvec, fp32 activations) on the host cores, the same step with the three
4096-column inputs quantized inside their GEMV launches (kq_gemv_q8k_x), speculative-verify batched
GEMV (per matrix and through the layer), the fp32-activation drop-in over the same layer, the prefill GEMM, the output heads and the
full decode weight stream.
"""
import argparse
import ctypes as C
import json
import os
import sys
import statistics
import subprocess
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "oxcoder-9b_amd"))

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
METRIC = "Q4_K decode GEMV GB/s (% of HBM peak) + prefill GEMM TOPS at 9B shapes"

LAYER = [  # name, R, C, type, input slot
    ("attn_q", 4096, 4096, 12, 0), ("attn_k", 1024, 4096, 12, 0), ("attn_v", 1024, 4096, 12, 0),
    ("attn_output", 4096, 4096, 12, 1), ("ffn_gate", 12288, 4096, 12, 2), ("ffn_up", 12288, 4096, 12, 2),
    ("ffn_down", 4096, 12288, 14, 3),
]
INPUT_COLS = [4096, 4096, 4096, 12288]
BLOCK = {12: 144, 14: 210}
Q8K = 292


def wbytes(R, C_, ty):
    return R * (C_ // 256) * BLOCK[ty]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Runner:
    """Direct C-ABI launches with precomputed arguments (no per-call Python checks)."""

    def __init__(self, torch):
        from kq import _lib
        self.torch = torch
        self.lib = _lib.kq()
        self.check = _lib.check

    def stream(self):
        return C.c_void_p(self.torch.cuda.current_stream().cuda_stream)

    def quantize(self, x, C_, xq, s, N=1):
        self.check(self.lib.kq_q8k_quantize(C.c_void_p(x.data_ptr()), C_, C_, N, C.c_void_p(xq.data_ptr()), s))

    def gemv(self, w, R, C_, ty, xq, N, y, s):
        self.check(self.lib.kq_gemv_q8k(C.c_void_p(w.data_ptr()), R, C_, ty, C.c_void_p(xq.data_ptr()), N,
                                        C.c_void_p(y.data_ptr()), R, s))

    def gemv_multi(self, mats, xq, ys, s, N=1):
        """mats: [(w, R, C, type)] sharing xq (N tokens; y rows of R floats); one launch per type."""
        n = len(mats)
        W = (C.c_void_p * n)(*[m[0].data_ptr() for m in mats])
        Rs = (C.c_int * n)(*[m[1] for m in mats])
        Ts = (C.c_int * n)(*[m[3] for m in mats])
        Y = (C.c_void_p * n)(*[y.data_ptr() for y in ys])
        L = (C.c_int64 * n)(*[m[1] for m in mats])
        self.check(self.lib.kq_gemv_q8k_multi(n, W, Rs, mats[0][2], Ts, C.c_void_p(xq.data_ptr()), N, Y, L, s))

    def gemv_x(self, mats, x, ys, xq, s):
        """mats: [(w, R, C, type)] sharing fp32 x (one token), quantized to Q8_K inside the launch
        (kq_gemv_q8k_x; xq receives the bytes, needed for C > 4096)."""
        n = len(mats)
        W = (C.c_void_p * n)(*[m[0].data_ptr() for m in mats])
        Rs = (C.c_int * n)(*[m[1] for m in mats])
        Ts = (C.c_int * n)(*[m[3] for m in mats])
        Y = (C.c_void_p * n)(*[y.data_ptr() for y in ys])
        self.check(self.lib.kq_gemv_q8k_x(n, W, Rs, mats[0][2], Ts, C.c_void_p(x.data_ptr()), Y,
                                          C.c_void_p(xq.data_ptr()) if mats[0][2] > 4096 else None, s))

    def rms_q8k(self, h, res, w, D, xq, s):
        """kq_rms_q8k on one row: h += res, xq = Q8_K(RMSNorm(h) * w)."""
        self.check(self.lib.kq_rms_q8k(C.c_void_p(h.data_ptr()), C.c_void_p(res.data_ptr()), 1,
                                       C.c_void_p(w.data_ptr()), D, 1, D, None, C.c_void_p(xq.data_ptr()), s))

    def swiglu_q8k(self, g, u, n, xq, s):
        """kq_swiglu_q8k on one row: xq = Q8_K(silu(g) * u)."""
        self.check(self.lib.kq_swiglu_q8k(C.c_void_p(g.data_ptr()), C.c_void_p(u.data_ptr()), n, 1, n, None,
                                          C.c_void_p(xq.data_ptr()), s))

    def gemm(self, w, R, C_, ty, xq, M, y, ws, s):
        """kq_gemm_q8k_ws with a preallocated workspace (ws: 256-byte aligned device tensor)."""
        self.check(self.lib.kq_gemm_q8k_ws(C.c_void_p(w.data_ptr()), R, C_, ty, C.c_void_p(xq.data_ptr()), M,
                                           C.c_void_p(y.data_ptr()), R, C.c_void_p(ws.data_ptr()), ws.numel(), s))


def make_layer(torch, dev, copies):
    from kq import quantize as kqq
    base = {}
    for i, (name, R, C_, ty, _) in enumerate(LAYER):
        base[name] = torch.from_numpy(kqq.synthetic_matrix(R, C_, ty, seed=i)).to(dev)
    layers = [base]
    for _ in range(copies - 1):
        layers.append({k: v.clone() for k, v in base.items()})
    return layers


def step_bytes():
    """Algorithmic bytes of one decode-layer step."""
    total = 0
    for _, R, C_, ty, _ in LAYER:
        total += wbytes(R, C_, ty) + (C_ // 256) * Q8K + R * 4
    for C_ in INPUT_COLS:
        total += C_ * 4 + (C_ // 256) * Q8K
    return total


def run_step(rn, layer, xs, xqs, ys, s):
    """Quantize each of the 4 inputs once; the matrices sharing it go in one launch."""
    for slot, C_ in enumerate(INPUT_COLS):
        rn.quantize(xs[slot], C_, xqs[slot], s)
        group = [(n, R, C2, ty) for n, R, C2, ty, sl in LAYER if sl == slot]
        rn.gemv_multi([(layer[n], R, C2, ty) for n, R, C2, ty in group], xqs[slot], [ys[n] for n, *_ in group], s)


def run_step_x(rn, layer, xs, xqs, ys, s):
    """The same step with each 4096-column input quantized inside its GEMV launch (kq_gemv_q8k_x:
    q+k+v, o, gate+up; the down projection's 12288 columns keep the quantizer's own launch)."""
    for slot, C_ in enumerate(INPUT_COLS):
        group = [(n, R, C2, ty) for n, R, C2, ty, sl in LAYER if sl == slot]
        rn.gemv_x([(layer[n], R, C2, ty) for n, R, C2, ty in group], xs[slot], [ys[n] for n, *_ in group],
                  xqs[slot], s)


def capture(torch, fn):
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()                      # warm the stream once outside capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def time_graphs(torch, plan):
    """plan: list of graphs to replay in order; returns elapsed seconds between events."""
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for g in plan:
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3


def kernel_roofline(torch, rn, layers, xqs, ys, repeats=5):
    """Dominant kernel: the Q4_K x Q8_K GEMV (launched for q+k+v, o and gate+up each step).
    A graph holds those launches for every resident layer copy back to back; HIP events around
    its replays on the launch stream give the mean launch duration (inter-launch gaps
    included).  Returns (mean algorithmic bytes per launch, mean seconds per launch, launches)."""
    groups = roofline_groups()

    def fn():
        s = rn.stream()
        for layer in layers:
            for slot, g in groups:
                rn.gemv_multi([(layer[n], R, C2, ty) for n, R, C2, ty in g], xqs[slot], [ys[n] for n, *_ in g], s)

    graph = capture(torch, fn)
    time_graphs(torch, [graph])
    el = time_graphs(torch, [graph] * repeats)
    launches = repeats * len(layers) * len(groups)
    nbytes = [sum(wbytes(R, C2, ty) + R * 4 for _, R, C2, ty in g) + (g[0][2] // 256) * Q8K for _, g in groups]
    return float(np.mean(nbytes)), el / launches, launches


def roofline_groups():
    groups = []
    for slot, C_ in enumerate(INPUT_COLS):
        g = [(n, R, C2, ty) for n, R, C2, ty, sl in LAYER if sl == slot]
        if all(ty == 12 for *_, ty in g):
            groups.append((slot, g))
    return groups


def pmc_workload(torch, rn, layers, xs, xqs, ys, dev):
    """The roofline kernel's launches (direct, no graph) over every resident layer copy, then a
    64 MiB device-to-device copy whose FETCH_SIZE / WRITE_SIZE calibrate the counters."""
    s = rn.stream()
    for slot, g in roofline_groups():
        rn.quantize(xs[slot], g[0][2], xqs[slot], s)
    for layer in layers:
        for slot, g in roofline_groups():
            rn.gemv_multi([(layer[n], R, C2, ty) for n, R, C2, ty in g], xqs[slot], [ys[n] for n, *_ in g], s)
    src = torch.ones(1 << 24, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    log("pmc workload: %d GEMV launches, one 64 MiB copy" % (len(layers) * len(roofline_groups())))


def pmc_workload_q6k(torch, rn, dev):
    """Q6_K GEMV launches for counter runs (direct, no graph): the 151936x4096 output head and the
    4096x12288 ffn_down, 4 calls each on alternating resident copies, then the 248320x4096 Q4_K
    head twice for comparison, then a 64 MiB device copy (counter calibration)."""
    from kq import ops, quantize as kqq
    s = rn.stream()
    for R, C_, ty, seed in ((151936, 4096, 14, 999), (4096, 12288, 14, 6)):
        w0 = torch.from_numpy(kqq.synthetic_matrix(R, C_, ty, seed=seed)).to(dev)
        ws = [w0, w0.clone()]
        xq = ops.q8k_quantize(torch.from_numpy(kqq.synthetic_activations(1, C_, seed=0)).to(dev))
        y = torch.empty(R, device=dev)
        torch.cuda.synchronize()
        for i in range(4):
            rn.gemv(ws[i % 2], R, C_, ty, xq, 1, y, s)
        torch.cuda.synchronize()
        del ws, w0
    R4, C4 = 248320, 4096
    raw = np.random.default_rng(5).integers(0, 256, (R4 * 16, 144), dtype=np.uint8)
    raw[:, 0:2] = np.array([4e-4], np.float16).view(np.uint8)
    raw[:, 2:4] = np.array([1e-3], np.float16).view(np.uint8)
    w4 = torch.from_numpy(raw.reshape(-1)).to(dev)
    xq = ops.q8k_quantize(torch.from_numpy(kqq.synthetic_activations(1, C4, seed=0)).to(dev))
    y = torch.empty(R4, device=dev)
    for _ in range(2):
        rn.gemv(w4, R4, C4, 12, xq, 1, y, s)
    src = torch.ones(1 << 24, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    log("pmc workload: Q6_K head x4, Q6_K down x4, Q4_K head x2, one 64 MiB copy")


def traffic_from_profile(path=os.path.join(ROOT, "profiles", "gemv_q4k_decode_layer_traffic.md")):
    """HBM bytes per launch of the roofline kernel as recorded by the committed counter summary
    (line 'traffic_bytes_per_launch = N'), or None when the summary is absent."""
    try:
        for line in open(path):
            if line.strip().startswith("traffic_bytes_per_launch"):
                return int(float(line.split("=")[1]))
    except OSError:
        return None
    return None


def host_cpus():
    """CPUs this process can use, read from the host: the affinity mask (os.sched_getaffinity), the
    cgroup CPU quota (/sys/fs/cgroup/cpu.max, cpu.cfs_quota_us) and lscpu's physical cores of the
    whole machine.  ``usable`` = the affinity count, capped by the quota when there is one."""
    aff = len(os.sched_getaffinity(0))
    quota = None
    for path, fmt in (("/sys/fs/cgroup/cpu.max", "v2"), ("/sys/fs/cgroup/cpu/cpu.cfs_quota_us", "v1")):
        try:
            if fmt == "v2":
                q, period = open(path).read().split()[:2]
                if q != "max":
                    quota = int(q) / int(period)
            else:
                q = int(open(path).read())
                period = int(open(os.path.join(os.path.dirname(path), "cpu.cfs_period_us")).read())
                if q > 0:
                    quota = q / period
            break
        except (OSError, ValueError):
            continue
    phys = None
    try:
        out = subprocess.run(["lscpu", "-p=CORE,SOCKET"], capture_output=True, text=True, timeout=20).stdout
        phys = len({l for l in out.splitlines() if l and not l.startswith("#")}) or None
    except (OSError, ValueError, subprocess.SubprocessError):
        pass
    usable = aff if quota is None else max(1, min(aff, int(quota)))
    return {"affinity": aff, "cgroup_quota": quota, "physical_cores_host": phys, "usable": usable}


def cpu_baseline(budget_s=12.0, budget_2t_s=6.0, runs=5):
    """The reference's CPU path (kc_matvec, fp32 activations) on the same layer shapes: `runs` timed
    runs after one warm-up, median, on every CPU this process can use (host_cpus(): the affinity
    mask capped by the cgroup quota; KQ_CPU_THREADS overrides) and on 2 threads (the reference's
    validated default, scripts/kindi_q4/kindi/cpu4.py:99)."""
    from kq import quantize as kqq
    from oracle import oracle
    hc = host_cpus()
    threads = int(os.environ.get("KQ_CPU_THREADS", hc["usable"]))
    gomp = C.CDLL("libgomp.so.1")
    kind = "reference" if oracle.ref_available() else "port"
    mats = []
    for i, (name, R, C_, ty, slot) in enumerate(LAYER):
        W = kqq.synthetic_matrix(R, C_, ty, seed=i)
        mats.append((W, R, C_, ty, kqq.synthetic_activations(1, C_, seed=slot)[0]))
    copies = [mats] + [[(W.copy(), R, C_, ty, x) for (W, R, C_, ty, x) in mats] for _ in range(3)]
    fn = oracle.ref_matvec if kind == "reference" else oracle.matvec_f32
    per_step = sum(wbytes(R, C_, ty) + C_ * 4 + R * 4 for (_, R, C_, ty, _) in mats)

    def timed(nthreads, seconds):
        # libgomp has already read OMP_NUM_THREADS (the host quantizer uses it); set the team size
        # of this thread's parallel regions through the runtime instead.
        gomp.omp_set_num_threads(nthreads)
        for (W, R, C_, ty, x) in copies[0]:
            fn(W, R, C_, ty, x)           # warm-up
        rates, steps = [], 0
        for _ in range(runs):
            t0 = time.perf_counter()
            n = 0
            while True:
                for (W, R, C_, ty, x) in copies[n % len(copies)]:
                    fn(W, R, C_, ty, x)
                n += 1
                el = time.perf_counter() - t0
                if el >= seconds / runs:
                    break
            rates.append(per_step * n / el / 1e9)
            steps += n
        return statistics.median(rates), steps

    v, n = timed(threads, budget_s)
    v2, n2 = timed(2, budget_2t_s)
    gomp.omp_set_num_threads(threads)
    return {"value": round(v, 3), "unit": "GB/s", "cores": threads, "kind": kind,
            "cores_source": "KQ_CPU_THREADS" if "KQ_CPU_THREADS" in os.environ else
                            "os.sched_getaffinity(0) capped by the cgroup CPU quota",
            "host_cpus": hc,
            "value_2_threads": round(v2, 3),
            "sample": "median of %d runs (%d decode-layer steps in %.0f s) of the 7 matvecs of one decode layer "
                      "(fp32 activations, kc_matvec%s) rotating 4 host copies (486 MB); value_2_threads: the same, "
                      "2 threads, %d steps in %.0f s" % (runs, n, budget_s, "" if kind == "reference" else " restated",
                                                        n2, budget_2t_s)}


def batched_extra(torch, rn, dev, steps):
    """Speculative-verify batched GEMV, N in {2,4,8,16}: 12288x4096 Q4_K and 4096x12288 Q6_K."""
    from kq import ops, quantize as kqq
    out = {}
    for name, R, C_, ty in (("gate_12288x4096_q4k", 12288, 4096, 12), ("down_4096x12288_q6k", 4096, 12288, 14)):
        base = torch.from_numpy(kqq.synthetic_matrix(R, C_, ty, seed=40 + ty)).to(dev)
        ws = [base] + [base.clone() for _ in range(15)]           # 16 copies: > 450 MB
        for N in (1, 2, 4, 8, 16):
            X = torch.from_numpy(kqq.synthetic_activations(N, C_, seed=N)).to(dev)
            xq = torch.empty(N * (C_ // 256) * Q8K, dtype=torch.uint8, device=dev)
            ops.q8k_quantize(X, xq.view(N, -1))
            y = torch.empty((N, R), device=dev)
            g = capture(torch, lambda: [rn.gemv(w, R, C_, ty, xq, N, y, rn.stream()) for w in ws])
            reps = max(1, steps // 16)
            time_graphs(torch, [g])
            el = time_graphs(torch, [g] * reps)
            per = el / (reps * len(ws))
            nbytes = wbytes(R, C_, ty) + N * (C_ // 256) * Q8K + N * R * 4
            out["%s_N%d" % (name, N)] = {"us": round(per * 1e6, 2), "GB/s": round(nbytes / per / 1e9, 1),
                                         "TOPS": round(2 * N * R * C_ / per / 1e12, 2)}
    return out


def step_x_extra(torch, rn, layers, xs, xqs, ys, steps=640):
    """The decode-layer step with the activation quantization inside the GEMV launches (kq_gemv_q8k_x
    for the three 4096-column inputs: 5 launches per step instead of 8), beside the headline step
    (separate quantizer launches) on the same resident layer copies.  Same algorithmic bytes."""
    def fn(step):
        def go():
            s = rn.stream()
            for lay in layers:
                step(rn, lay, xs, xqs, ys, s)
        return go
    out = {}
    for tag, step in (("quantizer_launches", run_step), ("quantize_in_gemv", run_step_x)):
        g = capture(torch, fn(step))
        time_graphs(torch, [g] * 2)
        reps = max(1, steps // len(layers))
        per = time_graphs(torch, [g] * reps) / (reps * len(layers))
        out[tag + "_us"] = round(per * 1e6, 2)
        out[tag + "_GB/s"] = round(step_bytes() / per / 1e9, 1)
    return out


def single_gemv_extra(torch, rn, dev, copies=64, reps=8):
    """One 4096x4096 Q4_K GEMV at batch 1 (seed-0 N(0, 0.02) weights, one N(0, 1) activation row):
    the GEMV alone on a resident Q8_K row, and with the row's quantization in front of it.  64
    resident weight copies (605 MB) rotate so the 256 MB last-level cache cannot serve repeats; each
    graph holds one call per copy."""
    from kq import quantize as kqq
    R = C_ = 4096
    base = torch.from_numpy(kqq.synthetic_matrix(R, C_, 12, seed=0)).to(dev)
    ws = [base] + [base.clone() for _ in range(copies - 1)]
    x = torch.from_numpy(kqq.synthetic_activations(1, C_, seed=0)[0]).to(dev)
    xq = torch.empty((C_ // 256) * Q8K, dtype=torch.uint8, device=dev)
    y = torch.empty(R, device=dev)
    rn.quantize(x, C_, xq, rn.stream())
    out = {}
    gemv_bytes = wbytes(R, C_, 12) + (C_ // 256) * Q8K + R * 4
    for name, fn, nbytes in (
            ("gemv", lambda s, w: rn.gemv(w, R, C_, 12, xq, 1, y, s), gemv_bytes),
            ("quantize_gemv", lambda s, w: (rn.quantize(x, C_, xq, s), rn.gemv(w, R, C_, 12, xq, 1, y, s)),
             gemv_bytes + C_ * 4 + (C_ // 256) * Q8K)):
        g = capture(torch, lambda: [fn(rn.stream(), w) for w in ws])
        time_graphs(torch, [g] * 2)
        per = time_graphs(torch, [g] * reps) / (reps * copies)
        out[name] = {"us": round(per * 1e6, 2), "GB/s": round(nbytes / per / 1e9, 1),
                     "hbm_frac": round(nbytes / per / 1e9 / HBM_PEAK_GBS, 4), "bytes": nbytes}
    return out


def verify_layer_extra(torch, rn, layers, dev, steps=320):
    """Speculative verify of N draft tokens through one decode layer's 7 matrices (the batched form of
    the step: Engine.gemv_batch's path; the ternary engine's spec.verify, spec.py:790): each of the 4
    inputs quantized as N Q8_K rows, the matrices sharing it in one kq_gemv_q8k_multi call with N
    tokens, every row bit-identical to one token.  N = 1 is the decode step itself; vs_one_token is
    what verifying N tokens costs against decoding one."""
    from kq import quantize as kqq
    out = {}
    reps = max(1, steps // len(layers))
    for N in (1, 2, 4, 8):
        xs = [torch.from_numpy(kqq.synthetic_activations(N, c, seed=20 + i)).to(dev) for i, c in enumerate(INPUT_COLS)]
        xqs = [torch.empty(N * (c // 256) * Q8K, dtype=torch.uint8, device=dev) for c in INPUT_COLS]
        ys = {name: torch.empty((N, R), device=dev) for name, R, _, _, _ in LAYER}

        def run():
            s = rn.stream()
            for lay in layers:
                for slot, C_ in enumerate(INPUT_COLS):
                    rn.quantize(xs[slot], C_, xqs[slot], s, N)
                    group = [(n, R, C2, ty) for n, R, C2, ty, sl in LAYER if sl == slot]
                    rn.gemv_multi([(lay[n], R, C2, ty) for n, R, C2, ty in group], xqs[slot],
                                  [ys[n] for n, *_ in group], s, N)
        g = capture(torch, run)
        time_graphs(torch, [g] * 2)
        per = time_graphs(torch, [g] * reps) / (reps * len(layers))
        out["N%d_us" % N] = round(per * 1e6, 2)
    for N in (2, 4, 8):
        out["N%d_vs_one_token" % N] = round(out["N%d_us" % N] / out["N1_us"], 3)
    return out


def producers_extra(torch, rn, layers, dev, steps=320):
    """Decode layer with the fused producers and a real layer's data dependencies: RMSNorm of the
    residual stream (adding the previous block's output) straight to Q8_K -> q/k/v; quantize the
    attention output (attention itself is not part of this path: a fixed synthetic vector) -> o;
    RMSNorm (adding o's output) to Q8_K -> gate/up; SwiGLU of their outputs to Q8_K -> down.  Also
    the same layer with the attention output quantized inside the o launch (kq_gemv_q8k_x: 7
    launches instead of 8), and the latency of one fused producer call (64 back-to-back calls in a
    graph)."""
    from kq import quantize as kqq
    D, F = 4096, 12288
    g = torch.Generator().manual_seed(5)
    h = torch.randn(D, generator=g).to(dev)
    w_attn = (1 + 0.1 * torch.randn(D, generator=g)).to(dev)
    w_ffn = (1 + 0.1 * torch.randn(D, generator=g)).to(dev)
    att = torch.from_numpy(kqq.synthetic_activations(1, D, seed=77)[0]).to(dev)
    xa, xo, xf = [torch.empty((D // 256) * Q8K, dtype=torch.uint8, device=dev) for _ in range(3)]
    xd = torch.empty((F // 256) * Q8K, dtype=torch.uint8, device=dev)
    ys = {name: torch.zeros(R, device=dev) for name, R, _, _, _ in LAYER}

    def step(lay, s, o_in_gemv=False):
        rn.rms_q8k(h, ys["ffn_down"], w_attn, D, xa, s)
        rn.gemv_multi([(lay[n], R, C2, ty) for n, R, C2, ty, sl in LAYER if sl == 0], xa,
                      [ys[n] for n, R, C2, ty, sl in LAYER if sl == 0], s)
        if o_in_gemv:   # the attention output quantized inside the o launch (kq_gemv_q8k_x)
            rn.gemv_x([(lay["attn_output"], 4096, D, 12)], att, [ys["attn_output"]], xo, s)
        else:
            rn.quantize(att, D, xo, s)
            rn.gemv(lay["attn_output"], 4096, D, 12, xo, 1, ys["attn_output"], s)
        rn.rms_q8k(h, ys["attn_output"], w_ffn, D, xf, s)
        rn.gemv_multi([(lay[n], R, C2, ty) for n, R, C2, ty, sl in LAYER if sl == 2], xf,
                      [ys["ffn_gate"], ys["ffn_up"]], s)
        rn.swiglu_q8k(ys["ffn_gate"], ys["ffn_up"], F, xd, s)
        rn.gemv(lay["ffn_down"], 4096, F, 14, xd, 1, ys["ffn_down"], s)

    wbytes_layer = sum(wbytes(R, C_, ty) for _, R, C_, ty, _ in LAYER)
    out = {}
    for tag, o_in_gemv in (("", False), ("o_quantize_in_gemv_", True)):
        def run_all():
            s = rn.stream()
            for lay in layers:
                step(lay, s, o_in_gemv)

        gr = capture(torch, run_all)
        time_graphs(torch, [gr] * 2)
        reps = max(1, steps // len(layers))
        per = time_graphs(torch, [gr] * reps) / (reps * len(layers))
        out.update({tag + "layer_us": round(per * 1e6, 2), tag + "weight_GB/s": round(wbytes_layer / per / 1e9, 1)})

    def single(fn):
        gs = capture(torch, lambda: [fn(rn.stream()) for _ in range(64)])
        time_graphs(torch, [gs] * 2)
        return round(time_graphs(torch, [gs] * 5) / (5 * 64) * 1e6, 2)

    out["rms_q8k_4096_us"] = single(lambda s: rn.rms_q8k(h, ys["attn_output"], w_ffn, D, xf, s))
    out["swiglu_q8k_12288_us"] = single(lambda s: rn.swiglu_q8k(ys["ffn_gate"], ys["ffn_up"], F, xd, s))
    out["q8k_quantize_12288_us"] = single(lambda s: rn.quantize(ys["ffn_gate"], F, xd, s))
    return out


def f32_layer_extra(torch, rn, layers, dev, steps=320):
    """The fp32-activation drop-in for q4_gemv (Kindi's numerics, no activation quantization) over
    one decode layer's 7 matrices, as Engine(mode="f32").gemv runs them: the matrices that share an
    input in one kq_gemv_multi launch (q/k/v, gate/up), o and down alone (4 launches; the
    reference launches q4_gemv once per matrix, gpu4.py:95-99); also one kq_gemv launch per matrix
    (7 launches).  The resident layer copies rotate, replayed from graphs.  Algorithmic bytes:
    weights + fp32 input (C*4) once per launch + fp32 output (R*4) per matrix."""
    from kq import quantize as kqq
    xs = [torch.from_numpy(kqq.synthetic_activations(1, c, seed=s)[0]).to(dev) for s, c in enumerate(INPUT_COLS)]
    ys = {name: torch.empty(R, device=dev) for name, R, _, _, _ in LAYER}
    p = lambda t: C.c_void_p(t.data_ptr())

    def grouped():
        s = rn.stream()
        for lay in layers:
            for slot, C_ in enumerate(INPUT_COLS):
                g = [(n, R, ty) for n, R, C2, ty, sl in LAYER if sl == slot]
                k = len(g)
                W = (C.c_void_p * k)(*[lay[n].data_ptr() for n, _, _ in g])
                Rs = (C.c_int * k)(*[R for _, R, _ in g])
                Ts = (C.c_int * k)(*[ty for _, _, ty in g])
                Y = (C.c_void_p * k)(*[ys[n].data_ptr() for n, _, _ in g])
                rn.check(rn.lib.kq_gemv_multi(k, W, Rs, C_, Ts, p(xs[slot]), Y, s))

    def per_matrix():
        s = rn.stream()
        for lay in layers:
            for name, R, C_, ty, slot in LAYER:
                rn.check(rn.lib.kq_gemv(p(lay[name]), R, C_, ty, p(xs[slot]), p(ys[name]), s))

    out = {}
    reps = max(1, steps // len(layers))
    for tag, fn in (("", grouped), ("per_matrix_", per_matrix)):
        g = capture(torch, fn)
        time_graphs(torch, [g] * 2)
        per = time_graphs(torch, [g] * reps) / (reps * len(layers))
        launches = len(INPUT_COLS) if not tag else len(LAYER)
        nbytes = sum(wbytes(R, C_, ty) + R * 4 for _, R, C_, ty, _ in LAYER)
        nbytes += (sum(INPUT_COLS) if not tag else sum(C_ for _, _, C_, _, _ in LAYER)) * 4
        out.update({tag + "layer_us": round(per * 1e6, 2), tag + "launches": launches, tag + "bytes_per_layer": nbytes,
                    tag + "GB/s": round(nbytes / per / 1e9, 1),
                    tag + "hbm_frac": round(nbytes / per / 1e9 / HBM_PEAK_GBS, 4)})
    return out


def pack_extra(torch, dev, layers=2):
    """Pack loading (the F3 path, gpu4.Weights over a Kindi pack): write a pack with the 9B profile's
    dimensions for `layers` layers plus the 248320-row embedding and head (random block bytes: the
    loader does not look inside blocks), check it with verify_pack (full: sizes, sha256, shapes),
    then bring every quantized tensor to the device through PackWeights twice: with the file in the
    host page cache, and after asking the kernel to drop its pages (POSIX_FADV_DONTNEED; no effect
    where the temporary directory is memory-backed)."""
    import shutil
    import tempfile
    from kq import pack
    shapes = pack.profile_shapes(layers)
    dims = dict(pack.PROFILE_DIMS, layers=layers)
    rng = np.random.default_rng(7)
    tensors = {}
    for name, (R, C_) in shapes.items():
        if pack._float_storage(name, R):
            tensors[name] = (rng.standard_normal(R * C_).astype(np.float32), R, C_, 0)
        else:
            ty = 14 if name.endswith(("output.weight", "ffn_down.weight")) else 12
            nbytes = R * (C_ // 256) * (210 if ty == 14 else 144)
            tensors[name] = (rng.integers(0, 256, nbytes, dtype=np.uint8), R, C_, ty)
    root = tempfile.mkdtemp(prefix="kq_pack_", dir=os.environ.get("TMPDIR", "/tmp"))
    try:
        path = os.path.join(root, "pack")
        t0 = time.perf_counter()
        pack.write_pack(path, tensors, dims=dims)
        t_write = time.perf_counter() - t0
        del tensors
        wbin = os.path.join(path, "weights.bin")
        fd = os.open(wbin, os.O_RDONLY)
        os.fsync(fd)
        t0 = time.perf_counter()
        pack.verify_pack(path, full=True, dims=dims, shapes=shapes)
        t_verify = time.perf_counter() - t0
        qnames = [n for n, (R, _) in shapes.items() if not pack._float_storage(n, R)]
        out = {}
        for label, drop in (("page_cache", False), ("after_fadv_dontneed", True)):
            if drop:
                os.posix_fadvise(fd, 0, 0, os.POSIX_FADV_DONTNEED)
            w = pack.PackWeights(path, device=dev)
            w._staging()                                # pinned staging allocated once, not timed
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            total = 0
            for n in qnames:
                buf = w[n][0]
                total += buf.numel()
            torch.cuda.synchronize()
            el = time.perf_counter() - t0
            out[label] = {"GB/s": round(total / el / 1e9, 2), "s": round(el, 3)}
            w.close()
            del w
            torch.cuda.empty_cache()
        os.close(fd)
        out.update({"bytes": total, "tensors": len(qnames), "layers": layers,
                    "write_s": round(t_write, 2), "verify_full_s": round(t_verify, 2)})
        return out
    finally:
        shutil.rmtree(root, ignore_errors=True)


def warm_then_time(torch, g, launches, warm_s=0.1, reps=4):
    """Replay graph g for at least warm_s seconds (clocks settle under sustained load), then time
    `reps` replays; returns seconds per launch (g holds `launches` launches)."""
    warm = 0.0
    while warm < warm_s:
        warm += time_graphs(torch, [g] * 2)
    return time_graphs(torch, [g] * reps) / (reps * launches)


def head_extra(torch, rn, dev):
    """Output head 151936x4096 Q6_K with the greedy pick: fused (kq_gemv_q8k_argmax) against the GEMV
    followed by kq_argmax; two resident copies (1 GB) alternate so the cache does not serve them.
    Then a 248320x4096 Q4_K head (the real model's output size), GEMV and fused, two copies."""
    from kq import ops, quantize as kqq
    R, C_ = 151936, 4096
    w0 = torch.from_numpy(kqq.synthetic_matrix(R, C_, 14, seed=999)).to(dev)
    ws_w = [w0, w0.clone()]
    x = torch.from_numpy(kqq.synthetic_activations(1, C_, seed=0)).to(dev)
    xq = ops.q8k_quantize(x)
    y = torch.empty(R, device=dev)
    aws = ops.argmax_workspace(dev)
    out = torch.empty(1, dtype=torch.int32, device=dev)
    lib = rn.lib
    p = lambda t: C.c_void_p(t.data_ptr())

    # each graph holds ROUNDS rounds of the two copies: replaying a graph costs several us between
    # replays, which a graph of two launches would charge to the kernel
    ROUNDS = 8

    def fused():
        for w in ws_w * ROUNDS:
            rn.check(lib.kq_gemv_q8k_argmax(p(w), R, C_, 14, p(xq), p(y), p(aws), p(out), rn.stream()))

    def separate():
        for w in ws_w * ROUNDS:
            rn.gemv(w, R, C_, 14, xq, 1, y, rn.stream())
            rn.check(lib.kq_argmax(p(y), R, p(aws), p(out), rn.stream()))

    def gemv_only():
        for w in ws_w * ROUNDS:
            rn.gemv(w, R, C_, 14, xq, 1, y, rn.stream())

    res = {}
    for name, fn in (("gemv_us", gemv_only), ("fused_us", fused), ("gemv_then_argmax_us", separate)):
        g = capture(torch, fn)
        res[name] = round(warm_then_time(torch, g, 2 * ROUNDS) * 1e6, 2)
    res["weight_GB/s_fused"] = round(wbytes(R, C_, 14) / (res["fused_us"] * 1e-6) / 1e9, 1)
    nb6 = wbytes(R, C_, 14) + (C_ // 256) * Q8K + R * 4
    res["gemv_GB/s"] = round(nb6 / (res["gemv_us"] * 1e-6) / 1e9, 1)
    res["gemv_hbm_frac"] = round(nb6 / (res["gemv_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
    del ws_w, w0
    # the real model's output size as Q4_K (output.weight 248320x4096, q4pack.py:22): random block
    # bytes with fp16 scales of a N(0, 0.02) row; the Q4_K GEMV's rate where the launch cost is
    # negligible (572 MB per launch)
    R4 = 248320
    rng = np.random.default_rng(5)
    raw = rng.integers(0, 256, (R4 * 16, 144), dtype=np.uint8)
    raw[:, 0:2] = np.array([4e-4], np.float16).view(np.uint8)
    raw[:, 2:4] = np.array([1e-3], np.float16).view(np.uint8)
    q0 = torch.from_numpy(raw.reshape(-1)).to(dev)
    del raw
    ws4 = [q0, q0.clone()]
    y4 = torch.empty(R4, device=dev)

    def gemv4():
        for w in ws4 * ROUNDS:
            rn.gemv(w, R4, C_, 12, xq, 1, y4, rn.stream())

    def fused4():
        for w in ws4 * ROUNDS:
            rn.check(lib.kq_gemv_q8k_argmax(p(w), R4, C_, 12, p(xq), p(y4), p(aws), p(out), rn.stream()))

    for name, fn in (("q4k_248320_gemv_us", gemv4), ("q4k_248320_fused_us", fused4)):
        g = capture(torch, fn)
        res[name] = round(warm_then_time(torch, g, 2 * ROUNDS) * 1e6, 2)
    nb = wbytes(R4, C_, 12) + (C_ // 256) * Q8K + R4 * 4
    res["q4k_248320_GB/s"] = round(nb / (res["q4k_248320_gemv_us"] * 1e-6) / 1e9, 1)
    res["q4k_248320_hbm_frac"] = round(nb / (res["q4k_248320_gemv_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
    del ws4, q0
    return res


def gemm_extra(torch, rn, dev, timed=True):
    """Prefill GEMM: M in {128, 256, 512, 2048} (256: the Engine's prefill chunk, KINDI_CHUNK; at 128
    and 256 K is split where the tiles are too few); 12288x4096 Q4_K and 4096x12288 Q6_K (timed=False:
    two direct calls per shape at M = 512 and 2048, for counter runs)."""
    from kq import ops, quantize as kqq
    out = {}
    for name, R, C_, ty in (("gate_12288x4096_q4k", 12288, 4096, 12), ("down_4096x12288_q6k", 4096, 12288, 14)):
        w = torch.from_numpy(kqq.synthetic_matrix(R, C_, ty, seed=60 + ty)).to(dev)
        for M in ((128, 256, 512, 2048) if timed else (512, 2048)):
            X = torch.from_numpy(kqq.synthetic_activations(M, C_, seed=M)).to(dev)
            xq = ops.q8k_quantize(X)
            y = torch.empty((M, R), device=dev)
            ws = ops.gemm_workspace(R, C_, M, dev)
            if not timed:
                for _ in range(2):
                    rn.gemm(w, R, C_, ty, xq, M, y, ws, rn.stream())
                torch.cuda.synchronize()
                continue
            # 4 calls per graph: replaying a graph costs several us between replays
            g = capture(torch, lambda: [rn.gemm(w, R, C_, ty, xq, M, y, ws, rn.stream()) for _ in range(4)])
            # warm-up of at least 0.2 s: the clock settles only after some ms of sustained MFMA
            # load (the first 10 calls run ~20 % slower than the steady state)
            warm = 0.0
            while warm < 0.2:
                warm += time_graphs(torch, [g] * 20)
            reps = 10
            el = time_graphs(torch, [g] * reps) / (4 * reps)
            out["%s_M%d" % (name, M)] = {"us": round(el * 1e6, 1), "TOPS": round(2 * M * R * C_ / el / 1e12, 2),
                                         "frac_int8_peak": round(2 * M * R * C_ / el / 1e12 / INT8_PEAK_TOPS, 4)}
    return out


def decode_stream_extra(torch, rn, dev):
    """Full 9B-shaped decode weight stream at batch 1: 32 layers (Q6_K attn_v and ffn_down on
    even layers, Q4_K otherwise) + 151936x4096 Q6_K lm_head; one graph per token.  Also with each
    layer's 4096-column inputs quantized inside their GEMV launches (kq_gemv_q8k_x)."""
    from kq import ops, quantize as kqq
    shapes = {}
    for i, (name, R, C_, ty, slot) in enumerate(LAYER):
        for t in (12, 14) if name in ("attn_v", "ffn_down") else (ty,):
            shapes[(name, t)] = torch.from_numpy(kqq.synthetic_matrix(R, C_, t, seed=100 + 10 * i + t)).to(dev)
    head = torch.from_numpy(kqq.synthetic_matrix(151936, 4096, 14, seed=999)).to(dev)
    layers, total = [], 0
    for l in range(32):
        lay = {}
        for name, R, C_, ty, slot in LAYER:
            t = (14 if l % 2 == 0 else 12) if name in ("attn_v", "ffn_down") else ty
            lay[name] = (shapes[(name, t)].clone(), R, C_, t, slot)
            total += wbytes(R, C_, t)
        layers.append(lay)
    total += wbytes(151936, 4096, 14)
    xs = [torch.from_numpy(kqq.synthetic_activations(1, c, seed=s)[0]).to(dev) for s, c in enumerate(INPUT_COLS)]
    xqs = [torch.empty((c // 256) * Q8K, dtype=torch.uint8, device=dev) for c in INPUT_COLS]
    ys = {name: torch.empty(R, device=dev) for name, R, _, _, _ in LAYER}
    logits = torch.empty(151936, device=dev)

    def token(in_gemv):
        def go():
            s = rn.stream()
            for lay in layers:
                for slot, c in enumerate(INPUT_COLS):
                    group = [(name, v) for name, v in lay.items() if v[4] == slot]
                    mats = [(w, R, C_, t) for _, (w, R, C_, t, _) in group]
                    if in_gemv:
                        rn.gemv_x(mats, xs[slot], [ys[name] for name, _ in group], xqs[slot], s)
                    else:
                        rn.quantize(xs[slot], c, xqs[slot], s)
                        rn.gemv_multi(mats, xqs[slot], [ys[name] for name, _ in group], s)
            rn.quantize(xs[0], 4096, xqs[0], s)
            rn.gemv(head, 151936, 4096, 14, xqs[0], 1, logits, s)
        return go

    out = {"weight_bytes_per_token": total}
    for tag, in_gemv in (("", False), ("quantize_in_gemv_", True)):
        g = capture(torch, token(in_gemv))
        time_graphs(torch, [g])
        reps = 10
        el = time_graphs(torch, [g] * reps) / reps
        out.update({tag + "ms_per_token": round(el * 1e3, 4), tag + "tokens_per_s": round(1 / el, 1),
                    tag + "GB/s": round(total / el / 1e9, 1), tag + "hbm_frac": round(total / el / 1e9 / HBM_PEAK_GBS, 4)})
        del g
    del layers, shapes, head
    return out


def prefill_chunk_extra(torch, rn, dev, layers, M=256):
    """One prefill chunk of M tokens (the Engine's KINDI_CHUNK) through a decode layer's 7 matrices, as
    Engine.gemm runs it: for each of the 4 fp32 inputs one kq_gemm_f32_multi call for the matrices
    sharing it (one launch quantizes the chunk and writes the GEMM's fragment copy, one GEMM launch);
    beside it the same chunk with kq_q8k_quantize and one kq_gemm_q8k_ws call per matrix.  The
    resident layer copies rotate."""
    from kq import ops, quantize as kqq
    xs = [torch.from_numpy(kqq.synthetic_activations(M, c, seed=10 + s)).to(dev) for s, c in enumerate(INPUT_COLS)]
    xqs = [torch.empty(M * (c // 256) * Q8K, dtype=torch.uint8, device=dev) for c in INPUT_COLS]
    ys = {name: torch.empty((M, R), device=dev) for name, R, _, _, _ in LAYER}
    groups = [[(n, R, C2, ty) for n, R, C2, ty, sl in LAYER if sl == slot] for slot in range(len(INPUT_COLS))]
    need = max(ops.gemm_f32_multi_workspace_bytes([R for _, R, _, _ in g], g[0][2], M) for g in groups)
    need = max(need, max(ops.gemm_workspace_bytes(R, C_, M) for _, R, C_, _, _ in LAYER))
    ws = torch.empty(need + 256, dtype=torch.uint8, device=dev)
    wsa = ws[(-ws.data_ptr()) % 256:]
    copies = min(len(layers), 8)

    def run(grouped):
        def fn():
            s = rn.stream()
            for lay in layers[:copies]:
                for slot, c in enumerate(INPUT_COLS):
                    if grouped:
                        ops.gemm_f32_multi([(lay[n], R, C2, ty) for n, R, C2, ty in groups[slot]], xs[slot],
                                           [ys[n] for n, *_ in groups[slot]], ws)
                        continue
                    rn.check(rn.lib.kq_q8k_quantize(C.c_void_p(xs[slot].data_ptr()), c, c, M,
                                                    C.c_void_p(xqs[slot].data_ptr()), s))
                    for n, R, C2, ty in groups[slot]:
                        rn.gemm(lay[n], R, C2, ty, xqs[slot], M, ys[n], wsa, s)

        g = capture(torch, fn)
        warm = 0.0
        while warm < 0.2:
            warm += time_graphs(torch, [g])
        reps = 5
        return time_graphs(torch, [g] * reps) / (reps * copies)

    per = run(True)
    per_single = run(False)
    ops_ = sum(2 * M * R * C_ for _, R, C_, _, _ in LAYER)
    return {"tokens": M, "us_per_layer": round(per * 1e6, 1), "tokens_per_s_per_layer": round(M / per, 1),
            "TOPS": round(ops_ / per / 1e12, 1), "frac_int8_peak": round(ops_ / per / 1e12 / INT8_PEAK_TOPS, 4),
            "one_call_per_matrix_us": round(per_single * 1e6, 1)}


def tp_shard_extra(torch, rn, dev, tp=8, copies=64):
    """One GPU's share of the decode layer under tensor parallelism over `tp` GPUs, at its real
    shapes: column-parallel q, k, v, gate, up keep R/tp rows; row-parallel o and down keep C/tp
    columns (their partial outputs would then be all-reduced, which one GPU cannot show).  Same
    step structure as the headline (4 quantizations, shared-input matrices in one launch), `copies`
    resident shard copies, graph-replayed."""
    from kq import quantize as kqq
    cols = [4096, 4096 // tp, 4096, 12288 // tp]
    shard = []
    for name, R, C_, ty, slot in LAYER:
        if name in ("attn_output", "ffn_down"):
            shard.append((name, R, C_ // tp, ty, slot))
        else:
            shard.append((name, R // tp, C_, ty, slot))
    base = {name: torch.from_numpy(kqq.synthetic_matrix(R, C_, ty, seed=200 + i)).to(dev)
            for i, (name, R, C_, ty, _) in enumerate(shard)}
    lays = [base] + [{k: v.clone() for k, v in base.items()} for _ in range(copies - 1)]
    xs = [torch.from_numpy(kqq.synthetic_activations(1, c, seed=s)[0]).to(dev) for s, c in enumerate(cols)]
    xqs = [torch.empty((c // 256) * Q8K, dtype=torch.uint8, device=dev) for c in cols]
    ys = {name: torch.empty(R, device=dev) for name, R, _, _, _ in shard}

    def fn():
        s = rn.stream()
        for lay in lays:
            for slot, c in enumerate(cols):
                rn.quantize(xs[slot], c, xqs[slot], s)
                group = [(n, R, C2, ty) for n, R, C2, ty, sl in shard if sl == slot]
                rn.gemv_multi([(lay[n], R, C2, ty) for n, R, C2, ty in group], xqs[slot], [ys[n] for n, *_ in group], s)

    g = capture(torch, fn)
    time_graphs(torch, [g])
    reps = 10
    per = time_graphs(torch, [g] * reps) / (reps * copies)
    nbytes = sum(wbytes(R, C_, ty) + (C_ // 256) * Q8K + R * 4 for _, R, C_, ty, _ in shard)
    nbytes += sum(c * 4 + (c // 256) * Q8K for c in cols)
    del lays, base
    return {"tp": tp, "shapes": {n: "%dx%d %s" % (R, C_, "Q4_K" if ty == 12 else "Q6_K") for n, R, C_, ty, _ in shard},
            "bytes_per_step": nbytes, "us_per_step": round(per * 1e6, 2), "GB/s": round(nbytes / per / 1e9, 1),
            "launches_per_step": 8}


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=640)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--copies", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extras", action="store_true", help="skip batched / GEMM / decode-stream extras")
    ap.add_argument("--only", choices=("single", "batched", "verify", "producers", "f32_layer", "gemm", "head",
                                       "decode_stream",
                                       "pack", "tp_shard", "prefill_chunk", "step_x"),
                    help="run only this extra (no headline step, no CPU baseline) and print its JSON; for "
                         "profiling one workload")
    ap.add_argument("--pmc-workload", choices=("gemv", "gemm", "q6k"),
                    help="no timing, for rocprofv3 --pmc runs: 'gemv' launches the roofline kernel's "
                         "workload once per layer copy, then one 64 MiB device copy (the calibration "
                         "kernel); 'gemm' runs each prefill GEMM shape twice; 'q6k' runs the Q6_K head and down "
                         "projection GEMVs (and the Q4_K head) a few times")
    a = ap.parse_args()
    if a.steps < 1 or a.warmup < 0 or a.copies < 1:
        ap.error("--steps and --copies must be positive, --warmup not negative")
    if a.gpus != 1:
        print("bench.py measures one GPU: the library has no multi-GPU path (the products would shard by "
              "output rows, with one all-reduce per token for o and down). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    rn = Runner(torch)
    if a.pmc_workload == "gemm":
        gemm_extra(torch, rn, dev, timed=False)
        return
    if a.pmc_workload == "q6k":
        pmc_workload_q6k(torch, rn, dev)
        return
    if a.only:
        need_layers = a.only in ("verify", "producers", "f32_layer", "prefill_chunk", "step_x")
        lay = make_layer(torch, dev, a.copies) if need_layers else None
        if a.only == "step_x":
            from kq import quantize as kqq
            xs_ = [torch.from_numpy(kqq.synthetic_activations(1, c, seed=s)[0]).to(dev)
                   for s, c in enumerate(INPUT_COLS)]
            xqs_ = [torch.empty((c // 256) * Q8K, dtype=torch.uint8, device=dev) for c in INPUT_COLS]
            ys_ = {name: torch.empty(R, device=dev) for name, R, _, _, _ in LAYER}
        fn = {"single": lambda: single_gemv_extra(torch, rn, dev),
              "step_x": lambda: step_x_extra(torch, rn, lay, xs_, xqs_, ys_),
              "batched": lambda: batched_extra(torch, rn, dev, 160),
              "verify": lambda: verify_layer_extra(torch, rn, lay, dev),
              "producers": lambda: producers_extra(torch, rn, lay, dev),
              "f32_layer": lambda: f32_layer_extra(torch, rn, lay, dev),
              "gemm": lambda: gemm_extra(torch, rn, dev),
              "head": lambda: head_extra(torch, rn, dev),
              "decode_stream": lambda: decode_stream_extra(torch, rn, dev),
              "pack": lambda: pack_extra(torch, dev),
              "tp_shard": lambda: tp_shard_extra(torch, rn, dev),
              "prefill_chunk": lambda: prefill_chunk_extra(torch, rn, dev, lay)}[a.only]
        print(json.dumps({a.only: fn()}), flush=True)
        return
    log("bench: building %d resident layer copies" % a.copies)
    layers = make_layer(torch, dev, a.copies)
    from kq import quantize as kqq
    xs = [torch.from_numpy(kqq.synthetic_activations(1, c, seed=s)[0]).to(dev) for s, c in enumerate(INPUT_COLS)]
    ys = {name: torch.empty(R, device=dev) for name, R, _, _, _ in LAYER}

    xqs = [torch.empty((c // 256) * Q8K, dtype=torch.uint8, device=dev) for c in INPUT_COLS]
    if a.pmc_workload == "gemv":
        pmc_workload(torch, rn, layers, xs, xqs, ys, dev)
        return

    def steps(n, start=0):
        def fn():
            s = rn.stream()
            for i in range(start, start + n):
                run_step(rn, layers[i % a.copies], xs, xqs, ys, s)
        return fn

    full = capture(torch, steps(a.copies))
    graphs = {a.copies: full}

    def plan_of(n):
        # exactly n steps: whole graphs of `copies` steps, then one graph of the remainder
        rem = n % a.copies
        if rem and rem not in graphs:
            graphs[rem] = capture(torch, steps(rem))
        return [full] * (n // a.copies) + ([graphs[rem]] if rem else [])

    plan = plan_of(a.steps)
    log("bench: warmup %d steps" % a.warmup)
    if a.warmup:
        time_graphs(torch, plan_of(a.warmup))
    el = time_graphs(torch, plan)
    per_step = el / a.steps
    nbytes = step_bytes()
    value = nbytes / per_step / 1e9
    log("bench: %.2f us/step  %.1f GB/s" % (per_step * 1e6, value))

    kb, ks, kn = kernel_roofline(torch, rn, layers, xqs, ys)
    achieved = kb / ks / 1e9
    result = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(per_step * 1e3, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded N(0,0.02) weights quantized by the repo quantizer; N(0,1) activations)",
        "config": {"workload": "one 9B-class decode layer's projections at batch 1 with Q8_K activations: "
                               "q/o 4096x4096, k/v 1024x4096, gate/up 12288x4096 Q4_K, down 4096x12288 Q6_K, "
                               "plus 4 activation quantizations",
                   "bytes_per_step": nbytes, "resident_layer_copies": a.copies,
                   "hbm_frac": round(value / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_from_profile(),
                     "traffic_source": "profiles/gemv_q4k_decode_layer_traffic.md: rocprofv3 --pmc FETCH_SIZE and "
                                       "WRITE_SIZE of bench.py --pmc-workload gemv, calibrated on a 64 MiB copy "
                                       "(read from that committed summary, not measured in this run)",
                     "kernel": "k_gemv_q8k_split<12,1,2> (Q4_K x Q8_K GEMV: q+k+v, o, gate+up launches)",
                     "launches": kn,
                     "avg_bytes_per_launch": round(kb), "avg_us_per_launch": round(ks * 1e6, 3)},
    }
    def extra(key, msg, fn):
        # an extra that raises is recorded as such; the headline figures above stand
        log("bench: " + msg)
        try:
            result[key] = fn()
        except Exception as e:      # noqa: BLE001
            log("bench: %s failed: %r" % (key, e))
            result[key] = {"error": repr(e)}

    if not a.no_extras:
        extra("step_quantize_in_gemv", "the step with the quantization inside the GEMV launches",
              lambda: step_x_extra(torch, rn, layers, xs, xqs, ys))
        extra("single_gemv_4096", "single 4096x4096 Q4_K GEMV", lambda: single_gemv_extra(torch, rn, dev))
        extra("batched_gemv", "batched GEMV", lambda: batched_extra(torch, rn, dev, 160))
        extra("verify_layer", "speculative verify through a layer", lambda: verify_layer_extra(torch, rn, layers, dev))
        extra("producers", "fused producers", lambda: producers_extra(torch, rn, layers, dev))
        extra("f32_layer", "fp32-activation layer", lambda: f32_layer_extra(torch, rn, layers, dev))
        extra("prefill_gemm", "prefill GEMM", lambda: gemm_extra(torch, rn, dev))
        extra("prefill_chunk_layer", "prefill chunk through a layer", lambda: prefill_chunk_extra(torch, rn, dev, layers))
        del layers
        torch.cuda.empty_cache()
        extra("head", "output head", lambda: head_extra(torch, rn, dev))
        extra("decode_stream", "full decode stream", lambda: decode_stream_extra(torch, rn, dev))
        extra("pack_load", "pack loading", lambda: pack_extra(torch, dev))
        extra("tp8_shard_layer", "one GPU's share of the layer at TP8", lambda: tp_shard_extra(torch, rn, dev))
    if not a.no_cpu:
        extra("cpu_baseline", "CPU baseline", cpu_baseline)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
