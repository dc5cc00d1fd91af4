#!/usr/bin/env python3
"""Benchmark of the numrs autograd backward hot path on one MI355X.

Headline: matmul_backward on A, B, dC [2048,2048]
fp32 -- dA = dC @ B^T and dB = A^T @ dC in one launch -- reported as GFLOP/s
(4*M*K*N per step) and as a fraction of the fp32 MFMA peak.  A "step" is one
backward pass of that node over one batch of synthetic N(0,1) inputs that are
already resident in HBM.  Secondary lines measure the other BASELINE configs'
kernels (non-square matmul backward, fused ReLU+bias backward, Adam step).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]

Prints ONE JSON line.  Only one GPU is supported: --gpus N > 1 exits.

Every timed region is a run of back-to-back launches that cycle through
several copies of the workload's buffers, enough that each launch's operands
were pushed out of the 256 MB Infinity Cache since that copy's last use: the
figures are HBM-resident rates.  Each entry also reports the same launch
repeated on one set of buffers (`resident_*`), which a cache-sized working
set serves partly from that cache.  Before any measurement an untimed,
time-based device warm-up (--device-warm-ms, default 300 ms of 2048^3
launches) lets the device settle, since the early launches of a run are
slower; its length is reported as `warm_ms` in the JSON line.  The --warmup
launches of each workload follow it, untimed as well.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "backward GFLOP/s & GB/s at 1 MI355X + % of fp32-MFMA/HBM roofline"
PEAK_FP32_MFMA_TFLOPS = 157.3  # MI355X dense fp32 matrix peak
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E peak
SEED = 20261201


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def randn(rng, shape):
    return rng.standard_normal(shape, dtype=np.float32)


class QueueAhead:
    """GPU work queued in front of a timed region: four 2048^3 matmul_backward
    launches (about 1.2 ms) keep the GPU busy while the host enqueues the
    region's launches, so the region measures back-to-back kernels and never
    the host's launch rate."""

    def __init__(self, ctx, rng):
        n = 2048
        self.ctx = ctx
        self.bufs = [ctx.to_device(randn(rng, (n, n))) for _ in range(3)]
        self.outs = [ctx.empty((n, n)) for _ in range(2)]

    def __call__(self) -> None:
        dC, A, B = self.bufs
        for _ in range(4):
            self.ctx.matmul_backward(dC, A, B, self.outs[0], self.outs[1])


_AHEAD = None

# Untimed, time-based warm-up of every timed region (--warm-ms).  The first
# launches after the GPU has idled are slower: a trace of the default run
# shows the 2048^3 launch at 291 us (1st), 308 (10th), 280 (30th), 258 (60th),
# 246 (90th) and 240-243 us after 150 launches, and the ramp starts over after
# the second or so of host work (buffer uploads) between two regions.  So
# each region first runs its own launch for WARM_MS of wall time, after its
# --warmup launches; the counts are reported in the JSON line.
WARM_MS = 50.0
_WARM_LAUNCHES: dict = {}


def host_cpu() -> dict:
    """The host CPU the CPU baselines run on: model name, logical CPUs, and
    the CPUs this process may use."""
    model = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count() or 1
    return {"model": model, "logical_cpus": os.cpu_count(), "usable_cpus": usable}


def cpu_threads() -> int:
    """Threads for an all-cores CPU baseline: the usable CPUs, at most 16
    (one GPU's share of the box)."""
    return max(1, min(16, host_cpu()["usable_cpus"]))

# MI355X's Infinity Cache (MALL) holds 256 MB in front of HBM.  A kernel
# relaunched on the same buffers whose bytes fit in it reads them back from
# that cache, not from HBM (a 201 MB read-2-write-1 stream measured 0.98 of
# 8 TB/s that way, 0.66 with its operands in HBM).  HBM-roofline figures are
# therefore taken with launches that cycle through enough copies of their
# buffers that each launch's operands were evicted since its copy was last
# used: k copies with k x footprint >= ROTATE_BYTES.
MALL_BYTES = 256 << 20
ROTATE_BYTES = 3 * MALL_BYTES


def n_sets(footprint_bytes) -> int:
    """Copies of a workload's buffers for a rotation past the Infinity Cache."""
    return max(2, -(-ROTATE_BYTES // int(footprint_bytes)))


class Rot:
    """k device copies of one array; copy i % k serves launch i."""

    def __init__(self, ctx, k: int, host=None, shape=None, dtype=np.float32):
        if host is not None:
            self.copies = [ctx.to_device(host) for _ in range(k)]
        else:
            self.copies = [ctx.empty(shape, dtype) for _ in range(k)]

    def __getitem__(self, i: int):
        return self.copies[i % len(self.copies)]


def warm_for(ctx, launch, first: int, ms: float) -> int:
    """Untimed launches launch(first), launch(first + 1), ... in batches of 32,
    each batch waited for, until `ms` of wall time have passed; returns how
    many were made."""
    n = 0
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(32):
            launch(first + n)
            n += 1
        ctx.sync()
    return n


def time_launches(ctx, launch, steps: int, warmup: int, tag: str = ""):
    """Calls launch(i) for i = 0, 1, ... : warmup times, then for WARM_MS of
    wall time (untimed; the count is kept under `tag` for the JSON line), then
    `steps` times back to back inside one timed region (HIP events in slots
    0/1 on the context's stream, the stream the kernels run on), queued behind
    QueueAhead's work.  Returns (total ms of the region, mean ms per
    launch)."""
    for i in range(warmup):
        launch(i)
    nw = warm_for(ctx, launch, warmup, WARM_MS)
    if tag:
        _WARM_LAUNCHES.setdefault(tag, []).append(warmup + nw)
    first = warmup + nw
    ctx.sync()
    if _AHEAD is not None:
        _AHEAD()
    ctx.timer_record(0)
    for i in range(first, first + steps):
        launch(i)
    ctx.timer_record(1)
    ctx.sync()
    total = ctx.timer_elapsed_ms(0, 1)
    return total, total / steps


def traffic_from_profile(name: str):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, calibrated against a copy kernel), if a committed summary
    exists under profiles/."""
    path = os.path.join(ROOT, "profiles", f"{name}_traffic.json")
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            return json.load(f).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


# The kernel matmul_backward launches for aligned shapes with a 256 x 128 tile
# per CU (2048^3 and the non-square C2 case): dA and dB tiles in one grid.
HEAD_KERNEL = "matmul_backward_stream"
COPY_PROBE_BYTES = 256 << 20  # calibration copy: reads and writes this many bytes


def traffic_probe(ctx, rng, reps: int = 3) -> None:
    """The launches the two counter runs (FETCH_SIZE, then WRITE_SIZE) measure:
    `reps` device copies of COPY_PROBE_BYTES -- the calibration kernel, whose
    true HBM traffic is known -- then `reps` launches each of the 2048^3
    matmul_backward, the C3 fused ReLU + bias backward (4096^2) and the C3
    Adam step (2^24 params), each launch on its own copy of the operands."""
    n = COPY_PROBE_BYTES // 4
    src, dst = ctx.to_device(randn(rng, n)), ctx.empty(n)
    for _ in range(reps):
        ctx.copy(dst, src)
    ctx.sync()
    # The non-temporal calibration pair (arrays of 2^23 floats and more are
    # streamed with non-temporal accesses): a fill that writes exactly n
    # floats (fill_grad_kernel) and a full sum that reads exactly n floats
    # (reduce_pass1; its partials are a few KiB).
    from numrs_amd import _lib as L
    g0, s = ctx.to_device(np.ones(1, np.float32)), ctx.empty((1,))
    for _ in range(reps):
        ctx.fill_grad(g0, dst)
        ctx._check(L.load().numrs_hip_sum(ctx.handle, src.ptr, n, 0, s.ptr))
    ctx.sync()
    # The same pair below the streaming threshold (2^22 floats, cached float4
    # accesses): a second cached calibration beside copy_kernel.
    nc = 1 << 22
    sc, dc = src.view(0, (nc,)), dst.view(0, (nc,))
    for _ in range(reps):
        ctx.fill_grad(g0, dc)
        ctx._check(L.load().numrs_hip_sum(ctx.handle, sc.ptr, nc, 0, s.ptr))
    ctx.sync()
    del src, dst, sc, dc
    M = K = N = 2048
    A_, B_, dC_ = (ctx.to_device(randn(rng, s)) for s in ((M, K), (K, N), (M, N)))
    dA_, dB_ = ctx.empty((M, K)), ctx.empty((K, N))
    for _ in range(reps):
        ctx.matmul_backward(dC_, A_, B_, dA_, dB_)
    ctx.sync()
    del A_, B_, dC_, dA_, dB_
    R = C = 4096
    for _ in range(reps):
        g, z = ctx.to_device(randn(rng, (R, C))), ctx.to_device(randn(rng, (R, C)))
        dx, db = ctx.empty((R, C)), ctx.empty((C,))
        ctx.relu_bias_backward(g, z, dx, db)
        ctx.sync()
        del g, z, dx, db
    na = 1 << 24
    for t in range(reps):
        p, g = ctx.to_device(randn(rng, na)), ctx.to_device(randn(rng, na))
        m, v = ctx.zeros(na), ctx.zeros(na)
        ctx.adam_step(p, g, m, v, t + 1, lr=1e-3)
        ctx.sync()
        del p, g, m, v
    # The HBM rows of bench.py --rows below 0.70 of the HBM peak, each at its
    # row's shape on fresh operands: a25 full sum and a5 bias unbroadcast of
    # a 4096^2 gradient, a11 transpose 4096^2, N2 LayerNorm backward
    # [32768, 512], N5 row argmax [16384, 1024], a18 MSE backward [4096, 512].
    lib = L.load()
    for _ in range(reps):
        g = ctx.to_device(randn(rng, (R, C)))
        ctx._check(lib.numrs_hip_sum(ctx.handle, g.ptr, R * C, 0, s.ptr))
        ctx.sync()
        del g
    for _ in range(reps):
        g, b = ctx.to_device(randn(rng, (R, C))), ctx.empty((C,))
        ctx.sum_to_shape(g, b)
        ctx.sync()
        del g, b
    for _ in range(reps):
        g, tr = ctx.to_device(randn(rng, (R, C))), ctx.empty((C, R))
        ctx._check(lib.numrs_hip_transpose(ctx.handle, g.ptr, tr.ptr, R, C))
        ctx.sync()
        del g, tr
    RL, CL = 32768, 512
    gam = ctx.to_device(np.ones(CL, np.float32))
    dgm, dbt = ctx.empty((CL,)), ctx.empty((CL,))
    for _ in range(reps):
        gl, xl = ctx.to_device(randn(rng, (RL, CL))), ctx.to_device(randn(rng, (RL, CL)))
        mean, rstd = ctx.to_device(randn(rng, RL)), ctx.to_device(np.ones(RL, np.float32))
        dxl = ctx.empty((RL, CL))
        ctx._check(lib.numrs_hip_layernorm_backward(ctx.handle, gl.ptr, xl.ptr, gam.ptr, mean.ptr,
                                                    rstd.ptr, dxl.ptr, dgm.ptr, dbt.ptr, RL, CL, 0,
                                                    0, 0))
        ctx.sync()
        del gl, xl, mean, rstd, dxl
    for _ in range(reps):
        am, idx = ctx.to_device(randn(rng, (16384, 1024))), ctx.empty((16384,), np.int32)
        ctx.argmax_rows(am, idx)
        ctx.sync()
        del am, idx
    g1 = ctx.to_device(np.array([0.75], np.float32))
    for _ in range(reps):
        pm, tm, dp = (ctx.to_device(randn(rng, (4096, 512))), ctx.to_device(randn(rng, (4096, 512))),
                      ctx.empty((4096, 512)))
        ctx.mse_backward(g1, pm, tm, dp)
        ctx.sync()
        del pm, tm, dp
    log(f"traffic probe: {reps} copies of {COPY_PROBE_BYTES} B, {reps} matmul_backward 2048^3, "
        f"{reps} relu+bias 4096^2, {reps} Adam 2^24, {reps} each of the a25, a5, a11, N2, N5 "
        f"and a18 rows")


def _pmc_per_dispatch(directory: str, counter: str) -> dict:
    """The values of `counter`, one per dispatch in dispatch order, by
    kernel name, from a rocprofv3 --pmc -f csv output directory."""
    import csv
    import glob
    files = glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise FileNotFoundError(f"no counter_collection.csv under {directory}")
    per = {}
    for path in files:
        with open(path) as f:
            for row in csv.DictReader(f):
                if row.get("Counter_Name") != counter:
                    continue
                key = (row["Kernel_Name"], row["Dispatch_Id"])
                if key in per:
                    raise ValueError(f"{counter}: two records for dispatch {key}")
                per[key] = float(row["Counter_Value"])
    out = {}
    for (name, did), v in sorted(per.items(), key=lambda kv: int(kv[0][1])):
        out.setdefault(name, []).append(v)
    return out  # kernel name -> values in dispatch order


# Kernels of the traffic probe: (profile name, workload, [(kernel-name part,
# access mode, group)] whose dispatches make up one launch of the workload,
# algorithmic bytes).  Mode "nt": the kernel streams with non-temporal
# accesses, and its counters are scaled by the non-temporal calibration pair.
# Group g: the probe's (g+1)-th run of `reps` dispatches of that kernel (the
# probe launches its workloads in a fixed order, and some kernels serve
# several of them: reduce_pass1<0, 2> the calibration sum and the a25 row,
# reduce_final the three sums, colreduce_finalize the C3 relu+bias, a5 and
# N2 rows).
TRAFFIC_KERNELS = [
    ("matmul_backward_2048", "C2 2048^3", [(HEAD_KERNEL, "cached", 0)],
     5 * 2048 * 2048 * 4),                          # read A, B, dC; write dA, dB
    ("relu_bias_4096", "C3 relu(X+b) backward 4096^2",
     [("colreduce_pass1<true", "nt", 0), ("colreduce_finalize", "cached", 0)],
     12 * 4096 * 4096 + 4 * 4096),                  # read g, z; write dx; write db
    ("adam_16m", "C3 Adam step 2^24 params", [("adam_kernel", "nt", 0)],
     28 * (1 << 24)),                               # read p, g, m, v; write p, m, v
    ("sum_full_4096", "a25 ops::sum of 4096^2", [("::reduce_pass1<0, 2>", "nt", 1),
                                                 ("::reduce_final", "cached", 2)],
     4 * 4096 * 4096),                              # read g
    ("unbroadcast_bias_4096", "a5 unbroadcast [4096,4096] -> [4096]",
     [("colreduce_pass1<false, 2>", "nt", 0), ("colreduce_finalize", "cached", 1)],
     4 * 4096 * 4096 + 4 * 4096),                   # read g; write db
    ("transpose_4096", "a11 transpose 4096^2", [("transpose_reg_kernel<2>", "nt", 0)],
     8 * 4096 * 4096),                              # read x; write x^T
    ("layernorm_backward_32768x512", "N2 LayerNorm backward [32768,512]",
     [("layernorm_bwd_vec<2, 2>", "nt", 0), ("colreduce_finalize", "cached", 2)],
     12 * 32768 * 512 + 8 * 32768),                 # read g, x; write dx; read mean, rstd
    ("argmax_16384x1024", "N5 argmax rows [16384,1024]", [("argmax_vec<4, false, 2>", "nt", 0)],
     4 * 16384 * 1024 + 4 * 16384),                 # read x; write idx
    ("mse_backward_4096x512", "a18 mse_backward [4096,512]", [("mse_bwd_kernel<1>", "cached", 0)],
     12 * 4096 * 512),                              # read p, t; write dp
]


def traffic_summary(fetch_dir: str, write_dir: str) -> list:
    """HBM bytes per launch of each probed workload: FETCH_SIZE and
    WRITE_SIZE (KiB per dispatch), each scaled by the factor that maps a
    calibration kernel's reading of the same counter onto its known bytes --
    copy_kernel (COPY_PROBE_BYTES read and written, cached accesses) for
    cached kernels, reduce_pass1 (reads) and fill_grad_kernel (writes) over
    the same bytes for non-temporal ones -- summed over the workload's
    kernels."""
    fetch = _pmc_per_dispatch(fetch_dir, "FETCH_SIZE")
    write = _pmc_per_dispatch(write_dir, "WRITE_SIZE")

    def pick(d, part, group=0, reps=3):
        # The probe makes `reps` dispatches of a kernel per workload that
        # uses it; a record set that is not a whole number of such runs, or
        # lacks the asked-for run, is refused.
        keys = [k for k in d if part in k]
        if len(keys) != 1:
            raise KeyError(f"{part}: {keys}")
        vals = d[keys[0]]
        if len(vals) % reps or len(vals) < (group + 1) * reps:
            raise ValueError(f"{part}: {len(vals)} dispatch records, expected a multiple of "
                             f"{reps} covering run {group}: the counter output is incomplete")
        return float(np.mean(vals[group * reps:(group + 1) * reps]))

    known_kib = COPY_PROBE_BYTES / 1024.0
    small_kib = 4.0 * (1 << 22) / 1024.0
    # Access mode 2 (non-temporal) and 1 (cached float4) of the calibration
    # pair; copy_kernel is a second cached calibration.
    cal = {"cached": (pick(fetch, "copy_kernel"), pick(write, "copy_kernel")),
           "nt": (pick(fetch, "::reduce_pass1<0, 2>"), pick(write, "fill_grad_kernel<2>"))}
    fac = {m: (known_kib / f, known_kib / w) for m, (f, w) in cal.items()}
    cached2 = (small_kib / pick(fetch, "::reduce_pass1<0, 1>"),
               small_kib / pick(write, "fill_grad_kernel<1>"))
    out = []
    for name, workload, parts, algorithmic in TRAFFIC_KERNELS:
        f_raw = w_raw = traffic = 0.0
        for part, mode, group in parts:
            f, w = pick(fetch, part, group), pick(write, part, group)
            f_raw, w_raw = f_raw + f, w_raw + w
            traffic += (f * fac[mode][0] + w * fac[mode][1]) * 1024.0
        out.append({"name": name, "kernel": "+".join(p for p, _, _ in parts),
                    "workload": workload, "modes": [m for _, m, _ in parts],
                    "fetch_kib_raw": f_raw, "write_kib_raw": w_raw,
                    "calibration_kib_raw": {m: list(v) for m, v in cal.items()},
                    "calibration_bytes": COPY_PROBE_BYTES,
                    "factors": {m: list(v) for m, v in fac.items()},
                    "cached_factors_second_pair": list(cached2),
                    "bytes_per_launch": traffic, "algorithmic_bytes": algorithmic,
                    "traffic_over_algorithmic": traffic / algorithmic})
    return out


def trace_summary(trace_csv: str, bench_out: str) -> str:
    """Markdown summary of a rocprofv3 --kernel-trace of the default bench
    run: the timed dispatches of each workload, picked out of the trace by
    the launch order bench.py follows (counts from the run's JSON line), so
    the kernel's own durations can be set beside the line's figures."""
    import csv

    with open(bench_out) as f:
        line = [json.loads(s) for s in f if s.startswith("{")][-1]
    K = line["steps"]
    K2 = max(5, K // 2)
    warm = line["warm_launches"]  # per tag: untimed launches before [timed, resident]
    with open(trace_csv) as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))

    def seq(part, grid=None):
        return [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in rows
                if part in r["Kernel_Name"] and (grid is None or int(r["Grid_Size_X"]) == grid)]

    c2, c2p = seq(HEAD_KERNEL, 256 * 512), seq(HEAD_KERNEL, 512 * 512)
    relu, fin, adam = seq("colreduce_pass1<true"), seq("colreduce_finalize"), seq("adam_kernel")
    # 2048^3 dispatches in launch order: per region its untimed launches, 4
    # queue-ahead, K timed; the same for the resident region; one check
    # launch; then 4 queue-ahead before each later timed region.  The other
    # kernels: untimed launches, K timed, untimed, K resident.
    a, b = warm["C2"]
    t0 = a + 4
    r0 = t0 + K + b + 4
    c, _ = warm["C2'"]
    e, _ = warm["C3 relu"]
    g, _ = warm["C3 Adam"]
    both = [x + y for x, y in zip(relu[e:e + K], fin[e:e + K])]
    sec = {s["workload"][:7]: s for s in line.get("secondary", [])}
    spec = [
        ("C2 2048^3, timed", HEAD_KERNEL, c2[t0:t0 + K], 4.0 * 2048 ** 3, "flop",
         line["roofline"]["kernel_ms"]),
        ("C2 2048^3, resident", HEAD_KERNEL, c2[r0:r0 + K], 4.0 * 2048 ** 3, "flop",
         line["roofline"]["resident_kernel_ms"]),
        ("C2' 4096x1024x4096, timed", HEAD_KERNEL, c2p[c:c + K2], 4.0 * 4096 * 1024 * 4096,
         "flop", sec.get("C2' mat", {}).get("kernel_ms")),
        ("C3 relu+bias, pass 1, timed", "colreduce_pass1<true, 2>", relu[e:e + K], None, None,
         None),
        ("C3 relu+bias, finalize, timed", "colreduce_finalize", fin[e:e + K], None, None, None),
        ("C3 relu+bias, both kernels", "pass 1 + finalize", both, 12.0 * 4096 * 4096 + 4 * 4096,
         "byte", sec.get("C3 relu", {}).get("kernel_ms")),
        ("C3 Adam 2^24, timed", "adam_kernel<false, 2>", adam[g:g + K], 28.0 * (1 << 24), "byte",
         sec.get("C3 Adam", {}).get("kernel_ms")),
    ]
    out = ["| Workload | Kernel | Dispatches | Mean (us) | Min (us) | Max (us) | Work per launch "
           "| Achieved (trace mean) | Fraction | bench.py line (ms) |",
           "|---|---|---|---|---|---|---|---|---|---|"]
    for label, kern, d, work, kind, bench_ms in spec:
        if not d:
            continue
        mean = float(np.mean(d))
        ach = frac = ""
        if kind == "flop":
            tf = work / (mean * 1e-6) / 1e12
            ach, frac = f"{tf:.1f} TFLOP/s", f"{tf / PEAK_FP32_MFMA_TFLOPS:.3f}"
            wk = f"{work / 1e9:.2f} GFLOP"
        elif kind == "byte":
            gb = work / (mean * 1e-6) / 1e9
            ach, frac = f"{gb:.0f} GB/s", f"{gb / PEAK_HBM_GBS:.3f}"
            wk = f"{work / 1e6:.1f} MB"
        else:
            wk = ""
        out.append(f"| {label} | {kern} | {len(d)} | {mean:.1f} | {min(d):.1f} | {max(d):.1f} | "
                   f"{wk} | {ach} | {frac} | {bench_ms if bench_ms is not None else ''} |")
    ramp = c2[:a]
    if ramp:
        pts = [i for i in (0, 9, 29, 59, 89, 149) if i < len(ramp)]
        out.append("")
        out.append(f"C2's untimed launches before its timed region ({a}: {line['warmup']} "
                   f"--warmup + {line['warm_ms']} ms time-based): launch " +
                   ", ".join(f"{i + 1}: {ramp[i]:.1f} us" for i in pts) +
                   f"; mean of the last 8: {np.mean(ramp[-8:]):.1f} us.")
    return "\n".join(out)


def bench_matmul_backward(ctx, rng, M, K, N, steps, warmup, tag="C2"):
    """Timed over launches that cycle through n_sets copies of A, B, dC, dA,
    dB (operands streamed from HBM); `resident_ms` repeats the launch on one
    set, whose 80 MB stay in the Infinity Cache."""
    A, B, dC = randn(rng, (M, K)), randn(rng, (K, N)), randn(rng, (M, N))
    k = n_sets(4.0 * (2 * M * K + 2 * K * N + M * N))
    A_, B_, dC_ = Rot(ctx, k, A), Rot(ctx, k, B), Rot(ctx, k, dC)
    dA_, dB_ = Rot(ctx, k, shape=(M, K)), Rot(ctx, k, shape=(K, N))

    def launch(i):
        ctx.matmul_backward(dC_[i], A_[i], B_[i], dA_[i], dB_[i])

    total, per = time_launches(ctx, launch, steps, warmup, tag)
    _, resident = time_launches(ctx, lambda i: launch(0), steps, warmup, tag)
    launch(0)
    flops = 4.0 * M * K * N
    # Sanity: one sampled row of each gradient against float64 numpy.
    ga, gb = dA_[0].numpy()[M // 3], dB_[0].numpy()[K // 5]
    ra = dC[M // 3].astype(np.float64) @ B.astype(np.float64).T
    rb = A[:, K // 5].astype(np.float64) @ dC.astype(np.float64)
    # Tolerance of the parity tests: 1e-5 + 1e-4|r| plus the fp32 rounding
    # allowance 4 * 2^-24 * K of a length-K contraction.
    ok = bool(np.all(np.abs(ga - ra) <= 1e-5 + 4 * 2.0**-24 * N + 1e-4 * np.abs(ra)) and
              np.all(np.abs(gb - rb) <= 1e-5 + 4 * 2.0**-24 * M + 1e-4 * np.abs(rb)))
    return {"ms_per_step": total / steps, "kernel_ms": per, "resident_ms": resident,
            "sets": k, "flops": flops, "sample_ok": ok, "inputs": (A, B, dC)}


def bench_relu_bias(ctx, rng, rows, cols, steps, warmup):
    g, z = randn(rng, (rows, cols)), randn(rng, (rows, cols))
    nbytes = 12.0 * rows * cols + 4.0 * cols  # read g, z; write dx; write db
    k = n_sets(nbytes)
    g_, z_ = Rot(ctx, k, g), Rot(ctx, k, z)
    dx_, db_ = Rot(ctx, k, shape=(rows, cols)), Rot(ctx, k, shape=(cols,))

    def launch(i):
        ctx.relu_bias_backward(g_[i], z_[i], dx_[i], db_[i])

    total, per = time_launches(ctx, launch, steps, warmup, "C3 relu")
    _, resident = time_launches(ctx, lambda i: launch(0), steps, warmup, "C3 relu")
    return {"ms_per_step": total / steps, "kernel_ms": per, "resident_ms": resident,
            "sets": k, "bytes": nbytes, "inputs": (g, z)}


def bench_adam(ctx, rng, n, steps, warmup):
    k = n_sets(16.0 * n)  # p, g, m, v (p, m, v updated in place)
    p_, g_ = Rot(ctx, k, randn(rng, n)), Rot(ctx, k, randn(rng, n))
    m_, v_ = Rot(ctx, k, np.zeros(n, np.float32)), Rot(ctx, k, np.zeros(n, np.float32))
    state = {"t": 0}

    def launch(i):
        state["t"] += 1
        ctx.adam_step(p_[i], g_[i], m_[i], v_[i], state["t"], lr=1e-3)

    total, per = time_launches(ctx, launch, steps, warmup, "C3 Adam")
    _, resident = time_launches(ctx, lambda i: launch(0), steps, warmup, "C3 Adam")
    return {"ms_per_step": total / steps, "kernel_ms": per, "resident_ms": resident,
            "sets": k, "bytes": 28.0 * n}


# Kernels of one C1 step: layer 1 forward (split-K reduced in the same
# launch), layer 2 forward, the cross-entropy loss, layer 2's backward pair,
# layer 1's weight gradient, SGD.
C1_KERNELS = 6


def bench_c1(ctx, steps, warmup, graphs=True):
    """2-layer MLP (64x784 -> 128 -> ReLU -> 10, softmax CE,
    SGD lr 0.01) -- forward, backward and SGD step through the device
    autograd engine.  n steps are launched back to back and the loss is read
    back once at the end, so the figure is the step rate a training loop that
    reads its loss occasionally sees: GPU-bound on a fast host, host-bound
    (six kernel launches and the Python calls per step) on a slow one.  The
    graph replay below queues each step with one launch."""
    import numrs_amd as nr
    from numrs_amd import Tensor, nn, optim
    from workloads import make_c1

    nr.set_default_context(ctx)
    p = make_c1(seed=1)
    l1 = nn.Linear.with_weights(784, 128, p["W1"], p["b1"])
    l2 = nn.Linear.with_weights(128, 10, p["W2"], p["b2"])
    model = nn.Sequential([l1, nn.ReLU(), l2])
    opt = optim.SGD.simple(model.parameters(), 0.01)
    x = Tensor.new(p["x"], False)
    onehot = Tensor.new(np.eye(10, dtype=np.float32)[p["labels"]], False)

    def step():
        loss = model.forward(x).cross_entropy_loss(onehot)
        loss.backward()
        opt.step()
        opt.zero_grad()
        return loss

    for _ in range(warmup):
        step().item()
    _WARM_LAUNCHES["C1"] = [warmup + warm_for(ctx, lambda i: step(), 0, WARM_MS)]
    # a step is tens of microseconds: time enough of them for a stable mean
    n = max(steps, 200)
    t0 = time.perf_counter()
    for _ in range(n):
        loss = step()
    loss.item()
    per = (time.perf_counter() - t0) / n
    out = {"us_per_step": per * 1e6, "loss": loss.item(), "steps": n}
    if not graphs:
        return out
    # The same step recorded once into a HIP graph and replayed: every kernel
    # of every step still runs, queued by one launch per step.
    g = nr.StepGraph(ctx, step)
    try:
        for _ in range(warmup):
            g.replay()
        ctx.sync()
        t0 = time.perf_counter()
        for _ in range(n):
            g.replay()
        gloss = g.outputs.item()
        out["graph_us_per_step"] = (time.perf_counter() - t0) / n * 1e6
        out["graph_loss"] = gloss
    finally:
        g.close()
    # The floor a chain of dependent launches sits on: as many of the smallest
    # kernel the library has (numrs_hip_stream_probe writing four floats) as
    # the step launches, on the same stream, recorded into a graph like the
    # step above and replayed, so that the host's launch rate does not enter.
    from numrs_amd import _lib as L
    lib = L.load()
    tiny = ctx.empty((4,))

    def chain():
        for _ in range(C1_KERNELS):
            ctx._check(lib.numrs_hip_stream_probe(ctx.handle, None, None, None, tiny.ptr, None,
                                                  4, 0, 1))
        return tiny
    chain()
    g7 = nr.StepGraph(ctx, chain)
    try:
        for _ in range(warmup):
            g7.replay()
        ctx.sync()
        t0 = time.perf_counter()
        for _ in range(n):
            g7.replay()
        ctx.sync()
        out["launch_floor_us"] = (time.perf_counter() - t0) / n / C1_KERNELS * 1e6
    finally:
        g7.close()
    return out


def c4_flops(B=16, S=256, D=512, H=8, F=2048):
    """Forward GEMM flops of the pre-LN block (QKV/O projections, FFN,
    QK^T and PV); backward is twice that (dX and dW per product)."""
    T = B * S
    fwd = 2 * T * D * D * 4 + 2 * T * D * F * 2 + 2 * 2 * B * H * S * S * (D // H)
    return fwd, 2 * fwd


def bench_c4(ctx, steps, warmup):
    """pre-LN transformer encoder block train step
    (B 16, S 256, d 512, 8 heads, FFN 2048 GELU, MSE): forward + backward +
    SGD step through the device autograd engine."""
    import numrs_amd as nr
    from numrs_amd import Tensor, nn, optim
    from workloads import make_c4

    nr.set_default_context(ctx)
    w, x, t, (B, S, H) = make_c4(seed=4)
    blk = nn.TransformerEncoderBlock(w, H)
    opt = optim.SGD.simple(blk.parameters(), 1e-3)
    xt, tt = Tensor.new(x, False), Tensor.new(t, False)

    def step():
        loss = blk.forward_seq(xt, B, S).mse_loss(tt)
        loss.backward()
        opt.step()
        opt.zero_grad()
        return loss

    for _ in range(warmup):
        step().item()
    _WARM_LAUNCHES["C4"] = [warmup + warm_for(ctx, lambda i: step(), 0, WARM_MS)]
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        loss = step()
    loss.item()
    per = (time.perf_counter() - t0) / steps
    fwd, bwd = c4_flops()
    return {"ms_per_step": per * 1e3, "tflops": (fwd + bwd) / per / 1e12, "loss": loss.item()}


def c5_flops(B=64, T=128, I=64, H=256):
    """Forward GEMM flops of the 2-layer LSTM (input and recurrent products;
    the 256->1 head is negligible); BPTT is twice that."""
    fwd = 2 * B * T * 4 * H * (I + H) + 2 * B * T * 4 * H * (H + H)
    return fwd, 2 * fwd


def bench_c5(ctx, steps, warmup):
    """2-layer LSTM forecaster (in 64, hidden 256, seq 128,
    batch 64, Linear 256->1 head on the last step, MSE) -- forward, BPTT and
    SGD step through the device autograd engine."""
    import numrs_amd as nr
    from numrs_amd import Tensor, nn, optim
    from workloads import make_c5

    nr.set_default_context(ctx)
    layers, hw, hb, x, target = make_c5(seed=5)
    model = nn.LSTMForecaster(layers, hw, hb)
    opt = optim.SGD.simple(model.parameters(), 1e-3)
    xt, tt = Tensor.new(x, False), Tensor.new(target, False)

    def step():
        loss = model.forward(xt).mse_loss(tt)
        loss.backward()
        opt.step()
        opt.zero_grad()
        return loss

    for _ in range(warmup):
        step().item()
    _WARM_LAUNCHES["C5"] = [warmup + warm_for(ctx, lambda i: step(), 0, WARM_MS)]
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        loss = step()
    loss.item()
    per = (time.perf_counter() - t0) / steps
    fwd, bwd = c5_flops()
    return {"ms_per_step": per * 1e3, "tflops": (fwd + bwd) / per / 1e12, "loss": loss.item()}


def cpu_baseline(A, B, dC, rows_a: int, rows_b: int):
    """numrs's matmul_backward restated in C (single thread, fp32 triple
    loops of backward.rs:123-146), timed on this host over a bounded sample
    of output rows and scaled to the whole step."""
    from oracle import oracle as O

    M, K = A.shape
    N = B.shape[1]
    t0 = time.perf_counter()
    O.matmul_backward(dC, A, B, need_b=False, rows_a=(0, rows_a))
    ta = time.perf_counter() - t0
    t0 = time.perf_counter()
    O.matmul_backward(dC, A, B, need_a=False, rows_b=(0, rows_b))
    tb = time.perf_counter() - t0
    full_s = ta / rows_a * M + tb / rows_b * K
    cpu = host_cpu()
    return {
        "value": round(4.0 * M * K * N / full_s / 1e9, 4),
        "unit": "GFLOP/s",
        "cores": 1,
        "kind": "port",
        "cpu_model": cpu["model"],
        "sample": (f"C restatement of numrs matmul_backward (oracle/numrs_oracle.c, fp32 triple "
                   f"loops of backward.rs:123-146, single-threaded as there), {rows_a} of {M} dA "
                   f"rows ({ta:.2f} s) + {rows_b} of {K} dB rows ({tb:.2f} s), scaled to the "
                   f"full {M}x{K}x{N} step ({full_s:.1f} s); {cpu['logical_cpus']} logical CPUs, "
                   f"{cpu['usable_cpus']} usable, 1 thread used"),
    }


def cpu_baseline_c1(reps: int = 5) -> dict:
    """numrs's C1 train step on the host, in the reference's node order
    (autograd/train.rs:159-183 over backward.rs): the forward products in host
    BLAS sgemm (numrs runs them through MKL, blas/mod.rs), everything after
    the forward in the oracle's C restatement on one thread -- CE backward,
    the bias unbroadcast, matmul_backward's fp32 triple loops for dA and dB
    (backward.rs:123-146; the reference computes dA of the input too,
    tensor.rs:206), transposes, ReLU backward and SGD (sgd.rs:87-124).
    Median of `reps` whole steps."""
    from oracle import oracle as O
    from workloads import make_c1

    p = make_c1(seed=1)
    x, onehot = p["x"], np.eye(10, dtype=np.float32)[p["labels"]]
    W1, b1, W2, b2 = (p[k].copy() for k in ("W1", "b1", "W2", "b2"))

    def step():
        W1t, W2t = O.transpose(W1), O.transpose(W2)
        z1 = x @ W1t + b1
        h = O.relu(z1)
        z2 = h @ W2t + b2
        O.cross_entropy_loss(z2, onehot)
        dz2 = O.cross_entropy_backward(1.0, z2, onehot)
        db2 = O.sum_to_shape(dz2, (10,))
        dh, dW2t = O.matmul_backward(dz2, h, W2t)
        dz1 = O.relu_backward(dh, z1)
        db1 = O.sum_to_shape(dz1, (128,))
        _, dW1t = O.matmul_backward(dz1, x, W1t)
        for prm, g in ((W1, O.transpose(dW1t)), (b1, db1), (W2, O.transpose(dW2t)), (b2, db2)):
            O.sgd_step(prm, g, None, 0.01)

    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    us = float(np.median(times)) * 1e6
    cpu = host_cpu()
    return {"value": round(us, 1), "unit": "us/step", "cores": 1, "kind": "port",
            "cpu_model": cpu["model"],
            "sample": f"whole step, median of {reps}; forward products in host BLAS sgemm "
                      f"(numrs: MKL), backward and SGD in the oracle's C loops on 1 thread"}


def cpu_baseline_adam(n: int, sample: int = 1 << 22) -> dict:
    """numrs's Adam::step loop (optim/adam.rs:124-167, one thread, scalar)
    restated in C, on the first `sample` of n parameters, scaled to n."""
    from oracle import oracle as O

    rng = np.random.default_rng(SEED + 7)
    p, g = randn(rng, sample), randn(rng, sample)
    m, v = np.zeros(sample, np.float32), np.zeros(sample, np.float32)
    O.adam_step(p, g, m, v, 1)  # page in
    t0 = time.perf_counter()
    O.adam_step(p, g, m, v, 2)
    dt = (time.perf_counter() - t0) * n / sample
    return {"value": round(28.0 * n / dt / 1e9, 3), "unit": "GB/s", "ms": round(dt * 1e3, 2),
            "cores": 1, "kind": "port", "cpu_model": host_cpu()["model"],
            "sample": f"first {sample:,} of {n:,} params ({dt * sample / n * 1e3:.1f} ms), "
                      f"scaled x{n / sample:g}"}


def cpu_baseline_relu_bias(g, z, sample: int = 1 << 22) -> dict:
    """numrs's backward of y = relu(X + b) on the host: relu_backward
    (backward.rs:152-163, one thread, scalar) over the first `sample`
    elements scaled to the whole [R, C], then add_backward's unbroadcast of
    the bias, which numrs forms as ops::sum of everything (backward.rs:12-39)
    added into db[0] (tensor.rs:120-132), timed on the whole array on all
    usable cores (at most 16) in the AVX2 8-lane chunk order of
    simd.rs:247-283.  GB/s over the GPU row's algorithmic bytes."""
    from oracle import oracle as O

    R, C = g.shape
    n = R * C
    gs, zs = g.ravel()[:sample], z.ravel()[:sample]
    O.relu_backward(gs, zs)  # page in
    t0 = time.perf_counter()
    O.relu_backward(gs, zs)
    t_relu = (time.perf_counter() - t0) * n / sample
    dz = O.relu_backward(g, z).ravel()
    nt = cpu_threads()
    O.sum_avx2_order_mt(dz, nt)
    t0 = time.perf_counter()
    O.sum_avx2_order_mt(dz, nt)
    t_sum = time.perf_counter() - t0
    tot = t_relu + t_sum
    return {"value": round((12.0 * n + 4.0 * C) / tot / 1e9, 3), "unit": "GB/s",
            "ms": round(tot * 1e3, 2), "cores": nt, "kind": "port", "cpu_model": host_cpu()["model"],
            "sample": f"relu_backward on the first {sample:,} of {n:,} elements on 1 thread "
                      f"({t_relu * sample / n * 1e3:.1f} ms, scaled x{n / sample:g}); the bias "
                      f"unbroadcast as numrs forms it, ops::sum of all {n:,} elements on {nt} "
                      f"threads x 8-lane AVX2 order ({t_sum * 1e3:.1f} ms)"}


def _blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info
        return max([int(d.get("num_threads", 1)) for d in threadpool_info()
                    if d.get("user_api") == "blas"] or [1])
    except Exception:  # noqa: BLE001  (the count is a label only)
        return 0


def cpu_baseline_c4() -> dict:
    """No numrs CPU path exists for C4 (the reference has no attention,
    LayerNorm or GELU).  A clearly non-numrs CPU point instead: the same
    block's forward and backward in fp32 numpy (oracle/transformer_oracle.py,
    host BLAS for the products), one step."""
    from oracle import transformer_oracle as TO
    from workloads import make_c4

    w, x, t, dims = make_c4(seed=4)
    TO.block(w, x[:256], t[:256], (1,) + dims[1:], dtype=np.float32)  # warm the BLAS
    t0 = time.perf_counter()
    TO.block(w, x, t, dims, dtype=np.float32)
    dt = time.perf_counter() - t0
    fwd, bwd = c4_flops()
    return {"value": round(dt * 1e3, 1), "unit": "ms/step", "tflops": round((fwd + bwd) / dt / 1e12, 3),
            "cores": _blas_threads(), "kind": "port", "cpu_model": host_cpu()["model"],
            "sample": "not numrs (the reference has no attention, LayerNorm or GELU): the block's "
                      "forward + backward in fp32 numpy with host BLAS (oracle/transformer_oracle.py), "
                      "one whole step; cores = BLAS threads"}


def cpu_baseline_c5() -> dict:
    """No numrs CPU path exists for C5 (the reference has no recurrent
    layer).  A clearly non-numrs CPU point instead: the forecaster's forward
    and BPTT in fp32 numpy (oracle/lstm_oracle.py, host BLAS for the per-step
    products), one step."""
    from oracle import lstm_oracle as LO
    from workloads import make_c5

    layers, hw, hb, x, target = make_c5(seed=5)
    LO.forecaster(layers, hw, hb, x[:, :4], target, dtype=np.float32)  # warm the BLAS
    t0 = time.perf_counter()
    LO.forecaster(layers, hw, hb, x, target, dtype=np.float32)
    dt = time.perf_counter() - t0
    fwd, bwd = c5_flops()
    return {"value": round(dt * 1e3, 1), "unit": "ms/step", "tflops": round((fwd + bwd) / dt / 1e12, 3),
            "cores": _blas_threads(), "kind": "port", "cpu_model": host_cpu()["model"],
            "sample": "not numrs (the reference has no recurrent layer): the forecaster's forward + "
                      "BPTT in fp32 numpy with host BLAS (oracle/lstm_oracle.py), one whole step; "
                      "cores = BLAS threads"}


ROW_ELEMS = (4096, 4096)  # BASELINE configs[2] (C3), the elementwise/broadcast config


def _cpu_time(fn, reps: int = 1) -> float:
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    return (time.perf_counter() - t0) / reps


def bench_rows(ctx, rng, steps: int, warmup: int, cpu: bool = True) -> list:
    """One measurement per hot-path row: the kernel behind each backward
    function at a BASELINE-config shape, timed as back-to-back launches between
    HIP events on the library's stream, against the roofline that bounds it;
    beside it the
    numrs CPU algorithm (the oracle's C restatement, one thread) on a bounded
    sample of the same input, scaled to the full size, and a check of the GPU
    output against that same oracle output on the sample."""
    from numrs_amd import _lib as L
    from oracle import oracle as O

    out = []

    def f32(shape, scale=1.0):
        return (rng.standard_normal(shape) * scale).astype(np.float32)

    cpu_model = host_cpu()["model"]

    probe_y_ = ctx.empty((1 << 16,))  # the probe's store target when it writes nothing

    def stream_ceiling(reads, writes, ne, rd, wr):
        """Mean time of numrs_hip_stream_probe moving the row's traffic (reads and
        writes of ne floats, one launch) on the row's own buffer copies, cycled
        like the row, so from HBM."""
        lib = L.load()

        def probe(i):
            a = [r[i].ptr for r in rd] + [None] * (3 - len(rd))
            y = wr[0][i].ptr if writes > 0 else probe_y_.ptr
            z = wr[1][i].ptr if writes > 1 else None
            ctx._check(lib.numrs_hip_stream_probe(ctx.handle, a[0], a[1], a[2], y, z, ne,
                                                  reads, writes))
        return time_launches(ctx, probe, steps, warmup)[1]

    def record(row, fn_name, kernel, shape, bytes_=None, flops=None, launch=None,
               cpu_fn=None, cpu_scale=1.0, cpu_sample="", check=None, note="", cpu_cores=1,
               ceil=None):
        total, per = time_launches(ctx, launch, steps, warmup)
        _, resident = time_launches(ctx, lambda i: launch(0), steps, warmup)
        cper = stream_ceiling(*ceil) if ceil is not None else None
        launch(0)  # the checks read copy 0
        ent = {"row": row, "function": fn_name, "kernel": kernel, "shape": shape,
               "kernel_us": round(per * 1e3, 2), "resident_us": round(resident * 1e3, 2)}
        if bytes_ is not None:
            gbs = bytes_ / (per * 1e-3) / 1e9
            ent.update({"bound": "hbm", "algorithmic_bytes": int(bytes_),
                        "achieved": round(gbs, 1), "unit": "GB/s",
                        "frac": round(gbs / PEAK_HBM_GBS, 4),
                        "resident_frac": round(bytes_ / (resident * 1e-3) / 1e9 / PEAK_HBM_GBS,
                                               4)})
            if cper is not None:
                reads, writes, ne = ceil[0], ceil[1], ceil[2]
                pb = 4.0 * (reads + writes) * ne
                pgbs = pb / (cper * 1e-3) / 1e9
                ent["ceiling"] = {
                    "kernel": f"stream_probe ({reads} reads, {writes} writes of {ne:,} floats, "
                              f"one launch)",
                    "us": round(cper * 1e3, 2), "achieved": round(pgbs, 1), "unit": "GB/s",
                    "frac": round(pgbs / PEAK_HBM_GBS, 4),
                    "row_frac_of_ceiling": round(gbs / pgbs, 4)}
        else:
            tf = flops / (per * 1e-3) / 1e12
            ent.update({"bound": "mfma", "algorithmic_flops": int(flops),
                        "achieved": round(tf, 2), "unit": "TFLOP/s",
                        "frac": round(tf / PEAK_FP32_MFMA_TFLOPS, 4)})
        if cpu and cpu_fn is not None:
            cpu_fn()  # page the sample in
            t = _cpu_time(cpu_fn) * cpu_scale
            ent["cpu_baseline"] = {"us": round(t * 1e6, 1), "kind": "port", "cores": cpu_cores,
                                   "cpu_model": cpu_model, "sample": cpu_sample}
            ent["gpu_vs_cpu"] = round(t / (per * 1e-3), 1)
        elif cpu:
            ent["cpu_baseline"] = None
        if check is not None:
            ent["sample_ok"] = bool(check())
        if note:
            ent["note"] = note
        out.append(ent)
        log(f"  {row:4s} {fn_name:28s} {ent['kernel_us']:9.2f} us  {ent['achieved']:9.1f} "
            f"{ent['unit']}  frac {ent['frac']:.3f}  (resident {ent['resident_us']:.2f} us)"
            + (f"  ceiling {ent['ceiling']['us']:.2f} us = {ent['ceiling']['frac']:.3f}, row at "
               f"{ent['ceiling']['row_frac_of_ceiling']:.3f} of it" if "ceiling" in ent else ""))

    def same_bits(a, b):
        return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))

    def close(a, b, rtol=1e-5, atol=1e-6):
        return np.allclose(np.asarray(a, np.float64), np.asarray(b, np.float64), rtol=rtol,
                           atol=atol)

    R, C = ROW_ELEMS
    n = R * C
    ns = 1 << 20  # CPU sample: the first 1,048,576 elements
    scale = n / ns
    samp = f"first {ns:,} of {n:,} elements, scaled x{scale:g}"
    g, x, y = f32((R, C)), f32((R, C)), f32((R, C))
    k = n_sets(4.0 * n)  # the smallest C3-shaped row (fill, sums) moves 4 B/elem
    g_, x_, y_ = Rot(ctx, k, g), Rot(ctx, k, x), Rot(ctx, k, y)
    dx_, dy_ = Rot(ctx, k, shape=(R, C)), Rot(ctx, k, shape=(R, C))
    shape = f"[{R},{C}] (C3)"

    # a3 accumulate_gradient: g += incoming (tensor.rs:120-132)
    acc_ = Rot(ctx, k, y)
    record("a3", "accumulate_gradient", "binary_backward(ADD, acc)", shape, bytes_=12.0 * n,
           launch=lambda i: ctx.binary_backward(L.ADD, g_[i], None, None, acc_[i], None,
                                                accumulate=True),
           ceil=(2, 1, n, [g_, acc_], [dx_]),
           cpu_fn=lambda: O.accumulate(y.ravel()[:ns].copy(), g.ravel()[:ns]), cpu_scale=scale,
           cpu_sample=samp)
    # a7 sub_backward: dx = g, dy = -g
    record("a7", "sub_backward", "binary_backward(SUB)", shape, bytes_=12.0 * n,
           launch=lambda i: ctx.binary_backward(L.SUB, g_[i], None, None, dx_[i], dy_[i]),
           ceil=(1, 2, n, [g_], [dx_, dy_]),
           cpu_fn=lambda: O.sub_backward(g.ravel()[:ns]), cpu_scale=scale, cpu_sample=samp,
           check=lambda: same_bits(dy_[0].numpy().ravel()[:ns], O.sub_backward(g.ravel()[:ns])[1]))
    # a8 mul_backward: dx = g*y, dy = g*x
    record("a8", "mul_backward", "binary_backward(MUL)", shape, bytes_=20.0 * n,
           launch=lambda i: ctx.binary_backward(L.MUL, g_[i], x_[i], y_[i], dx_[i], dy_[i]),
           ceil=(3, 2, n, [g_, x_, y_], [dx_, dy_]),
           cpu_fn=lambda: O.mul_backward(g.ravel()[:ns], x.ravel()[:ns], y.ravel()[:ns]),
           cpu_scale=scale, cpu_sample=samp,
           check=lambda: same_bits(dx_[0].numpy().ravel()[:ns],
                                   O.mul_backward(g.ravel()[:ns], x.ravel()[:ns],
                                                  y.ravel()[:ns])[0]))
    # a9 div_backward: dx = g/y, dy = -g*x/y^2
    record("a9", "div_backward", "binary_backward(DIV)", shape, bytes_=20.0 * n,
           launch=lambda i: ctx.binary_backward(L.DIV, g_[i], x_[i], y_[i], dx_[i], dy_[i]),
           ceil=(3, 2, n, [g_, x_, y_], [dx_, dy_]),
           cpu_fn=lambda: O.div_backward(g.ravel()[:ns], x.ravel()[:ns], y.ravel()[:ns]),
           cpu_scale=scale, cpu_sample=samp,
           check=lambda: same_bits(dy_[0].numpy().ravel()[:ns],
                                   O.div_backward(g.ravel()[:ns], x.ravel()[:ns],
                                                  y.ravel()[:ns])[1]))
    # a13-a15, a21, N1 unary grads: read g and the saved value, write dx
    pos = np.abs(x) + np.float32(0.5)
    pos_ = Rot(ctx, k, pos)
    sig = (1.0 / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)
    sig_ = Rot(ctx, k, sig)
    th = np.tanh(x).astype(np.float32)
    th_ = Rot(ctx, k, th)
    for row, name, kind, v, v_, ofn, exact in [
            ("a13", "sigmoid_backward", L.SIGMOID, sig, sig_, O.sigmoid_backward, True),
            ("a14", "tanh_backward", L.TANH, th, th_, O.tanh_backward, True),
            ("a15", "exp_backward", L.EXP, pos, pos_, O.exp_backward, True),
            ("a15", "log_backward", L.LOG, pos, pos_, O.log_backward, True),
            ("a21", "sqrt_backward", L.SQRT, pos, pos_, O.sqrt_backward, False),
            ("N1", "gelu_backward (new op)", L.GELU, x, x_, None, False)]:
        vs = v.ravel()[:ns]
        if ofn is not None:
            cfn = (lambda ofn=ofn, vs=vs: ofn(g.ravel()[:ns], vs))
            chk = (lambda ofn=ofn, vs=vs, exact=exact:
                   (same_bits if exact else close)(dx_[0].numpy().ravel()[:ns],
                                                   ofn(g.ravel()[:ns], vs)))
        else:
            cfn = None
            chk = (lambda vs=vs: close(dx_[0].numpy().ravel()[:ns],
                                       O.gelu_backward(g.ravel()[:ns], vs), 1e-5, 1e-6))
        record(row, name, f"unary_backward({name.split('_')[0].upper()})", shape,
               bytes_=12.0 * n,
               launch=(lambda i, kind=kind, v_=v_: ctx.unary_backward(kind, g_[i], v_[i],
                                                                      dx_[i])),
               ceil=(2, 1, n, [g_, v_], [dx_]),
               cpu_fn=cfn, cpu_scale=scale, cpu_sample=samp, check=chk,
               note="" if ofn is not None else "no numrs CPU path: the reference has no GELU")
    record("a21", "pow_backward (n=3)", "unary_backward(POW)", shape, bytes_=12.0 * n,
           launch=lambda i: ctx.unary_backward(L.POW, g_[i], x_[i], dx_[i], 3.0),
           ceil=(2, 1, n, [g_, x_], [dx_]),
           cpu_fn=lambda: O.pow_backward(g.ravel()[:ns], x.ravel()[:ns], 3.0), cpu_scale=scale,
           cpu_sample=samp,
           check=lambda: close(dx_[0].numpy().ravel()[:ns],
                               O.pow_backward(g.ravel()[:ns], x.ravel()[:ns], 3.0), 1e-5, 1e-5))
    # a11 transpose_backward: dX = dY^T (8 B/elem)
    tr_ = Rot(ctx, k, shape=(C, R))
    rs = ns // C
    record("a11", "transpose_backward", "transpose_reg_kernel", shape, bytes_=8.0 * n,
           launch=lambda i: ctx._check(L.load().numrs_hip_transpose(ctx.handle, g_[i].ptr,
                                                                      tr_[i].ptr, R, C)),
           ceil=(1, 1, n, [g_], [tr_]),
           cpu_fn=lambda: O.transpose(g[:rs]), cpu_scale=R / rs,
           cpu_sample=f"first {rs} of {R} rows, scaled x{R / rs:g}",
           check=lambda: same_bits(tr_[0].numpy()[:, :rs], O.transpose(g[:rs])))
    del tr_
    # a16/a17 sum/mean backward: fill with g[0] (or g[0]/n), 4 B/elem
    g1_ = ctx.to_device(np.array([0.75], np.float32))
    record("a17", "mean_backward", "fill_grad", shape, bytes_=4.0 * n,
           launch=lambda i: ctx.fill_grad(g1_, dx_[i], divide_by_n=True),
           ceil=(0, 1, n, [], [dx_]),
           cpu_fn=lambda: O.mean_backward(0.75, (ns,)), cpu_scale=scale, cpu_sample=samp,
           check=lambda: same_bits(dx_[0].numpy().ravel()[:16],
                                   O.mean_backward(0.75, (n,))[:16]))
    # a25 ops::sum over all elements (4 B/elem).  CPU: the whole array on all
    # usable cores (at most 16), each thread's chunk in the AVX2 8-lane order
    # of simd.rs:247-283 -- Rayon's par_iter split (scalar.rs:500) over the
    # reference's SIMD loop.
    s_ = ctx.empty((1,))
    nt = cpu_threads()
    gflat = g.ravel()
    mt_samp = f"whole {n:,}-element array, {nt} threads x 8-lane AVX2 order"
    record("a25", "ops::sum (full)", "reduce_pass1+final", shape, bytes_=4.0 * n,
           launch=lambda i: ctx._check(L.load().numrs_hip_sum(ctx.handle, g_[i].ptr, n, 0,
                                                                s_.ptr)),
           ceil=(1, 0, n, [g_], []),
           cpu_fn=lambda: O.sum_avx2_order_mt(gflat, nt), cpu_cores=nt, cpu_sample=mt_samp,
           check=lambda: abs(float(s_.numpy()[0]) - float(g.astype(np.float64).sum()))
           <= 1e-3 * np.sqrt(n))
    # a5 unbroadcast to a bias: [R, C] -> [C] column reduce (4 B/elem).  numrs
    # reduces a broadcast grad with ops::sum over everything (backward.rs:12-39),
    # so its CPU cost is the full sum above.
    b_ = ctx.empty((C,))
    record("a5", "unbroadcast (bias, CORRECT)", "colreduce_pass1+finalize", shape,
           bytes_=4.0 * n + 4.0 * C,
           launch=lambda i: ctx.sum_to_shape(g_[i], b_),
           ceil=(1, 0, n, [g_], []),
           cpu_fn=lambda: O.sum_avx2_order_mt(gflat, nt), cpu_cores=nt,
           cpu_sample=mt_samp + " (numrs reduces with ops::sum, backward.rs:12-39)",
           check=lambda: close(b_.numpy(), g.astype(np.float64).sum(0), 1e-4, 1e-3))
    del acc_, pos_, sig_, th_, g_, x_, y_, dx_, dy_
    # a18 mse_backward at C4's output [4096, 512] (dp only: 12 B/elem)
    p, t = f32((4096, 512)), f32((4096, 512))
    k = n_sets(12.0 * p.size)
    p_, t_, dp_ = Rot(ctx, k, p), Rot(ctx, k, t), Rot(ctx, k, shape=(4096, 512))
    record("a18", "mse_backward", "mse_backward_kernel", "[4096,512] (C4 output)",
           bytes_=12.0 * p.size,
           launch=lambda i: ctx.mse_backward(g1_, p_[i], t_[i], dp_[i]),
           ceil=(2, 1, p.size, [p_, t_], [dp_]),
           cpu_fn=lambda: O.mse_backward(0.75, p, t), cpu_sample="whole input",
           check=lambda: same_bits(dp_[0].numpy(), O.mse_backward(0.75, p, t)[0]))
    del p_, t_, dp_
    # a19 cross_entropy_backward, one-hot target (12 B/elem)
    B_, C_ = 16384, 1024
    logits = f32((B_, C_), 2.0)
    lab = rng.integers(0, C_, B_)
    onehot = np.zeros((B_, C_), np.float32)
    onehot[np.arange(B_), lab] = 1.0
    k = n_sets(12.0 * B_ * C_)
    lg_, oh_, dl_ = Rot(ctx, k, logits), Rot(ctx, k, onehot), Rot(ctx, k, shape=(B_, C_))
    record("a19", "cross_entropy_backward", "softmax_ce_backward", f"[{B_},{C_}] one-hot",
           bytes_=12.0 * B_ * C_,
           launch=lambda i: ctx.softmax_ce_backward(g1_, lg_[i], dl_[i], onehot=oh_[i]),
           ceil=(2, 1, B_ * C_, [lg_, oh_], [dl_]),
           cpu_fn=lambda: O.cross_entropy_backward(0.75, logits[:512], onehot[:512]),
           cpu_scale=B_ / 512, cpu_sample=f"first 512 of {B_} rows, scaled x{B_ / 512:g}",
           check=lambda: close(dl_[0].numpy()[:512],
                               O.cross_entropy_backward(0.75, logits[:512], onehot[:512]) *
                               np.float32(512 / B_), 1e-5, 1e-7),
           note="C1's [64,10] is latency-bound; C3's element count shows the roofline")
    del lg_, oh_, dl_
    # a20 softmax_backward over C4's attention probabilities [128*256, 256]
    rows_s = 16 * 8 * 256
    sm = O.softmax_rows(f32((rows_s, 256)))
    gs = f32((rows_s, 256))
    k = n_sets(12.0 * sm.size)
    sm_, gs_, ds_ = Rot(ctx, k, sm), Rot(ctx, k, gs), Rot(ctx, k, shape=(rows_s, 256))
    record("a20", "softmax_backward", "softmax_backward_kernel", "[32768,256] (C4 attention)",
           bytes_=12.0 * sm.size,
           launch=lambda i: ctx.softmax_backward(sm_[i], gs_[i], ds_[i]),
           ceil=(2, 1, sm.size, [sm_, gs_], [ds_]),
           cpu_fn=lambda: O.softmax_backward(sm[:4096], gs[:4096]), cpu_scale=rows_s / 4096,
           cpu_sample=f"first 4096 of {rows_s} rows, scaled x{rows_s / 4096:g}",
           check=lambda: close(ds_[0].numpy()[:4096], O.softmax_backward(sm[:4096], gs[:4096]),
                               1e-5, 1e-6))
    del sm_, gs_, ds_
    # N2 layernorm backward: C4's row width 512, C3's element count
    RL = 32768
    xl, gl = f32((RL, 512)), f32((RL, 512))
    gam = (1.0 + 0.1 * rng.standard_normal(512)).astype(np.float32)
    _, mean, rstd = O.layernorm_fwd(xl, gam, np.zeros(512, np.float32))
    k = n_sets(12.0 * xl.size)
    xl_, gl_, gam_ = Rot(ctx, k, xl), Rot(ctx, k, gl), ctx.to_device(gam)
    mean_, rstd_ = Rot(ctx, k, mean), Rot(ctx, k, rstd)
    dxl_, dgm_, dbt_ = Rot(ctx, k, shape=(RL, 512)), ctx.empty((512,)), ctx.empty((512,))
    record("N2", "layernorm_backward (new op)", "layernorm_bwd_vec+finalize",
           f"[{RL},512] (C4 rows of 512; C3 element count)", bytes_=12.0 * xl.size + 8.0 * RL,
           launch=lambda i: ctx._check(L.load().numrs_hip_layernorm_backward(
               ctx.handle, gl_[i].ptr, xl_[i].ptr, gam_.ptr, mean_[i].ptr, rstd_[i].ptr,
               dxl_[i].ptr, dgm_.ptr, dbt_.ptr, RL, 512, 0, 0, 0)),
           ceil=(2, 1, xl.size, [xl_, gl_], [dxl_]),
           check=lambda: close(dxl_[0].numpy()[:4096],
                               O.layernorm_backward(gl[:4096], xl[:4096], gam)[0], 1e-4, 1e-5),
           note="no numrs CPU path: the reference has no LayerNorm; C4's own [4096,512] "
                "is 8 MB per operand and latency-bound")
    del xl_, gl_, gam_, mean_, rstd_, dxl_, dgm_, dbt_
    # N5 argmax over rows (int result; 4 B/elem + 4 B/row)
    am = f32((16384, 1024))
    k = n_sets(4.0 * am.size)
    am_, idx_ = Rot(ctx, k, am), Rot(ctx, k, shape=(16384,), dtype=np.int32)
    record("N5", "argmax (rows, first max)", "argmax_vec", "[16384,1024]",
           bytes_=4.0 * am.size + 4.0 * 16384,
           launch=lambda i: ctx.argmax_rows(am_[i], idx_[i]),
           ceil=(1, 0, am.size, [am_], []),
           cpu_fn=lambda: O.argmax_rows(am[:512]), cpu_scale=32.0,
           cpu_sample="first 512 of 16384 rows, scaled x32",
           check=lambda: np.array_equal(idx_[0].numpy(), O.argmax_rows(am)),
           note="C1's [64,10] is latency-bound; C3's element count shows the roofline")
    del am_, idx_
    # a23 SGD step (mu = 0): read p, g, write p (12 B/elem)
    nsgd = 1 << 24
    ps, gsg = f32(nsgd), f32(nsgd)
    k = n_sets(12.0 * nsgd)
    ps_, gsg_ = Rot(ctx, k, ps), Rot(ctx, k, gsg)
    record("a23", "SGD::step (mu=0)", "sgd_kernel", "16,777,216 params", bytes_=12.0 * nsgd,
           launch=lambda i: ctx.sgd_step(ps_[i], gsg_[i], lr=0.01),
           cpu_fn=lambda: O.sgd_step(ps[:ns].copy(), gsg[:ns], None, 0.01), cpu_scale=nsgd / ns,
           cpu_sample=f"first {ns:,} of {nsgd:,} params, scaled x{nsgd / ns:g}")
    del ps_, gsg_
    # a26 Linear::forward at C4's FFN up-projection: y[4096,2048] = x[4096,512] W^T + b
    T_, In, Out = 4096, 512, 2048
    xw, W, bb = f32((T_, In)), f32((Out, In), 0.05), f32(Out)
    k = n_sets(4.0 * (T_ * In + Out * In + 2 * T_ * Out))
    xw_, W_, bb_ = Rot(ctx, k, xw), Rot(ctx, k, W), Rot(ctx, k, bb)
    yw_ = Rot(ctx, k, shape=(T_, Out))
    record("a26", "Linear::forward (fused)", "gemm_stream_kernel (bias epilogue)",
           "[4096,512]x[512,2048]",
           flops=2.0 * T_ * In * Out,
           launch=lambda i: ctx._check(L.load().numrs_hip_linear_forward(
               ctx.handle, xw_[i].ptr, W_[i].ptr, bb_[i].ptr, yw_[i].ptr, T_, In, Out)),
           check=lambda: close(yw_[0].numpy()[:64], xw[:64].astype(np.float64) @
                               W.T.astype(np.float64) + bb, 1e-4, 1e-4),
           note="numrs runs this forward through MKL sgemm; no CPU port here")
    # a26 backward of the same layer: dx = g W, dW = g^T x, db = colsum(g)
    gw = f32((T_, Out))
    gw_, dxw_ = Rot(ctx, k, gw), Rot(ctx, k, shape=(T_, In))
    dW_, db_ = Rot(ctx, k, shape=(Out, In)), Rot(ctx, k, shape=(Out,))
    record("a10+a11+a5", "Linear backward (fused)",
           "linear_backward_stream_small (split reduction and bias sums in the launch)",
           "[4096,512]x[512,2048]", flops=4.0 * T_ * In * Out,
           launch=lambda i: ctx._check(L.load().numrs_hip_linear_backward(
               ctx.handle, gw_[i].ptr, xw_[i].ptr, W_[i].ptr, dxw_[i].ptr, dW_[i].ptr, db_[i].ptr,
               T_, In, Out, 0, 0, 0, L.UNBROADCAST_CORRECT)),
           check=lambda: close(dxw_[0].numpy()[:64], gw[:64].astype(np.float64) @ W, 1e-4, 1e-4))
    del xw_, W_, bb_, yw_, gw_, dxw_, dW_, db_
    # N3 attention backward at C4: 128 heads of 256x256x64
    Bq, Sq, Hq, Dq = 16, 256, 8, 512
    q, k, v, do = (f32((Bq * Sq, Dq), 0.5) for _ in range(4))
    ks = n_sets(4.0 * (7 * Bq * Sq * Dq + Bq * Hq * Sq * Sq))
    q_, k_, v_, do_ = (Rot(ctx, ks, a) for a in (q, k, v, do))
    P_ = Rot(ctx, ks, shape=(Bq * Hq, Sq, Sq))
    o_ = Rot(ctx, ks, shape=(Bq * Sq, Dq))
    for i in range(ks):
        ctx._check(L.load().numrs_hip_attention_forward(ctx.handle, q_[i].ptr, k_[i].ptr,
                                                        v_[i].ptr, P_[i].ptr, o_[i].ptr, Bq, Sq,
                                                        Hq, Dq))
    dh = Dq // Hq
    # the forward at C4: P = softmax(alpha Q K^T) stored, O = P V
    record("N3f", "attention forward (new op)", "attn_fwd_wave_rows_kernel (eight waves of whole query rows)",
           "16x256, 8 heads of 64", flops=2 * 2.0 * Bq * Hq * Sq * Sq * dh,
           launch=lambda i: ctx._check(L.load().numrs_hip_attention_forward(
               ctx.handle, q_[i].ptr, k_[i].ptr, v_[i].ptr, P_[i].ptr, o_[i].ptr, Bq, Sq, Hq, Dq)),
           note="two products per head, P stored (33.5 MB); no numrs CPU path")
    dq_, dk_, dv_ = (Rot(ctx, ks, shape=(Bq * Sq, Dq)) for _ in range(3))
    # the engine's call: the backward given the forward's output (row totals dO . O)
    record("N3", "attention backward (new op)", "attn_bwd_wave_rows (dS, dQ) + attn_bwd_wave_keys (dV, dK)",
           "16x256, 8 heads of 64", flops=4 * 2.0 * Bq * Hq * Sq * Sq * dh,
           launch=lambda i: ctx._check(L.load().numrs_hip_attention_backward_out_strided(
               ctx.handle, q_[i].ptr, k_[i].ptr, v_[i].ptr, Dq, P_[i].ptr, o_[i].ptr, do_[i].ptr,
               Dq, dq_[i].ptr, dk_[i].ptr, dv_[i].ptr, Bq, Sq, Hq, Dq, 0)),
           note="four products per head, dS through a [B H, S, S] buffer; no numrs CPU path")
    del q_, k_, v_, do_, P_, o_, dq_, dk_, dv_
    # N4 two stacked LSTM layers at C5 (batch 64, seq 128, in 64, hidden 256):
    # the forward entry point (input projection of layer 1 + the persistent
    # recurrence of both layers) and the backward one (persistent recurrence
    # + the weight gradients and dx batched over time).  Latency-bound: 128
    # dependent steps per direction; the fraction is of the fp32 MFMA peak.
    from workloads import make_c5
    layers5, _, _, x5, _ = make_c5(seed=5)
    B5, T5, I5 = x5.shape
    H5 = layers5[0]["w_hh"].shape[1]
    lw = [{kk: ctx.to_device(vv) for kk, vv in l.items()} for l in layers5]
    x5_ = ctx.to_device(x5)
    seq = [ctx.empty((B5, T5, H5)) for _ in range(4)]       # h1, c1, h2, c2
    acts = [ctx.empty((B5, T5, 4 * H5)) for _ in range(2)]  # acts1, acts2
    dh2_ = ctx.to_device(f32((B5, T5, H5)))
    dx5_ = ctx.empty((B5, T5, I5))
    dws = [ctx.empty(l[kk].shape) for l in layers5 for kk in ("w_ih", "w_hh", "b")]
    lib = L.load()

    def lstm_fwd(i):
        ctx._check(lib.numrs_hip_lstm2_forward(
            ctx.handle, x5_.ptr, lw[0]["w_ih"].ptr, lw[0]["w_hh"].ptr, lw[0]["b"].ptr,
            lw[1]["w_ih"].ptr, lw[1]["w_hh"].ptr, lw[1]["b"].ptr, seq[0].ptr, seq[1].ptr,
            acts[0].ptr, seq[2].ptr, seq[3].ptr, acts[1].ptr, B5, T5, I5, H5, H5))

    def lstm_bwd(i):
        ctx._check(lib.numrs_hip_lstm2_backward(
            ctx.handle, x5_.ptr, lw[0]["w_ih"].ptr, lw[0]["w_hh"].ptr, lw[1]["w_ih"].ptr,
            lw[1]["w_hh"].ptr, seq[0].ptr, seq[1].ptr, acts[0].ptr, seq[2].ptr, seq[3].ptr,
            acts[1].ptr, dh2_.ptr, dx5_.ptr, dws[0].ptr, dws[1].ptr, dws[2].ptr, dws[3].ptr,
            dws[4].ptr, dws[5].ptr, B5, T5, I5, H5, H5, 0, 0, 0, 0, 0, 0, 0))

    prod = 2.0 * B5 * T5 * 4 * H5  # flops per unit of reduction length, all steps
    fwd_flops = prod * I5 + 3 * prod * H5          # x W_ih1^T, then h1 W_hh1^T, h1 W_ih2^T, h2 W_hh2^T
    bwd_flops = 3 * prod * H5 + 3 * prod * H5 + 2 * prod * I5  # recurrences; dW_ih2, dW_hh2, dW_hh1; dW_ih1, dx
    lstm_fwd(0)
    record("N4", "LSTM x2 forward (new op)", "fill_bits + lstm2_fwd_persist",
           f"B {B5}, T {T5}, in {I5}, hidden {H5} (C5)", flops=fwd_flops, launch=lstm_fwd,
           note="one persistent launch for all 128 steps of both layers, the first layer's "
                "input projection inside the steps; no numrs CPU path")
    record("N4", "LSTM x2 backward (new op)",
           "lstm2_bwd_prep + lstm2_bwd_persist + 2 x (tn_pair_stream_small + splitk_reduce)",
           f"B {B5}, T {T5}, in {I5}, hidden {H5} (C5)", flops=bwd_flops, launch=lstm_bwd,
           note="one persistent launch for all 128 steps of both layers (bias partials formed "
                "in the steps), then each layer's dW_ih and dW_hh over all steps as one paired "
                "launch; no numrs CPU path")
    del lw, x5_, seq, acts, dh2_, dx5_, dws
    return out


def main() -> int:
    global WARM_MS, _AHEAD
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--warm-ms", type=float, default=WARM_MS,
                    help="untimed, time-based warm-up of each timed region on its own launches, "
                         "after its --warmup launches (reported in the JSON line)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--cpu-rows-a", type=int, default=512)
    ap.add_argument("--cpu-rows-b", type=int, default=192)
    ap.add_argument("--rows", action="store_true",
                    help="measure every hot-path row's kernel instead (one JSON line per row)")
    ap.add_argument("--split-reduction", choices=["fused", "separate"], default="fused",
                    help="where split-K partials are added (numrs_hip_set_split_reduction): "
                         "inside the products' own launch (fused, the default) or by one more "
                         "launch (separate); the same bits either way")
    ap.add_argument("--recurrence", choices=["auto", "per_step", "plain_launch", "cooperative"],
                    default="auto",
                    help="how the LSTM recurrences run (numrs_hip_set_recurrence_mode): auto "
                         "and plain_launch start the persistent kernels with an ordinary "
                         "launch, cooperative with a cooperative one (rocprofv3's teardown "
                         "faults after those)")
    ap.add_argument("--eager-only", action="store_true",
                    help="with --only c1: the eager steps only, no graph recording or replay "
                         "(for kernel traces: rocprofv3's kernel trace ended in a host "
                         "segmentation fault inside hipGraphLaunch on one run)")
    ap.add_argument("--only", choices=["c1", "c4", "c5"], default=None,
                    help="run only this secondary workload (for profiling); prints its entry")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only launch the calibration copy, the 2048^3 matmul_backward, the C3 "
                         "relu+bias backward and the C3 Adam step (run under rocprofv3 --pmc "
                         "FETCH_SIZE, then WRITE_SIZE)")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="turn the two --pmc outputs of --traffic-probe into "
                         "profiles/<kernel>_traffic.json files (no GPU needed)")
    ap.add_argument("--trace-summary", nargs=2, metavar=("KERNEL_TRACE_CSV", "BENCH_OUT"),
                    help="markdown table of the timed dispatches in a rocprofv3 kernel trace of "
                         "the default run, beside that run's JSON line (no GPU needed)")
    args = ap.parse_args()

    if args.traffic_summary:
        for res in traffic_summary(*args.traffic_summary):
            with open(os.path.join(ROOT, "profiles", f"{res['name']}_traffic.json"), "w") as f:
                json.dump(res, f, indent=1)
                f.write("\n")
            print(json.dumps(res), flush=True)
        return 0
    if args.trace_summary:
        print(trace_summary(*args.trace_summary), flush=True)
        return 0

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); this build has "
              f"no multi-GPU path: run with --gpus 1", file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print("--steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2

    from numrs_amd import Context

    ctx = Context(0)
    ctx.set_recurrence_mode(args.recurrence)
    ctx.set_split_reduction(args.split_reduction)
    n_cus, arch = ctx.info()
    log(f"device {arch}, {n_cus} CUs")
    rng = np.random.default_rng(SEED)
    if not args.traffic_probe:
        _AHEAD = QueueAhead(ctx, np.random.default_rng(SEED + 1))

    if args.traffic_probe:
        traffic_probe(ctx, rng)
        ctx.close()
        return 0

    WARM_MS = max(0.0, args.warm_ms)

    if args.rows:
        for ent in bench_rows(ctx, rng, args.steps, args.warmup, cpu=not args.no_cpu_baseline):
            print(json.dumps(ent), flush=True)
        ctx.close()
        return 0

    if args.only is not None:
        fn = {"c1": lambda: bench_c1(ctx, args.steps, args.warmup, graphs=not args.eager_only),
              "c4": lambda: bench_c4(ctx, args.steps, args.warmup),
              "c5": lambda: bench_c5(ctx, args.steps, args.warmup)}[args.only]
        res = fn()
        print(json.dumps({"workload": args.only, **res}), flush=True)
        ctx.close()
        return 0

    M = K = N = 2048
    log(f"matmul_backward {M}x{K}x{N}: {args.warmup} warmup + {args.steps} timed steps")
    head = bench_matmul_backward(ctx, rng, M, K, N, args.steps, args.warmup)
    gflops = head["flops"] / (head["ms_per_step"] * 1e-3) / 1e9
    achieved_tf = head["flops"] / (head["kernel_ms"] * 1e-3) / 1e12
    resident_tf = head["flops"] / (head["resident_ms"] * 1e-3) / 1e12
    log(f"  {head['ms_per_step']:.4f} ms/step, kernel {head['kernel_ms']:.4f} ms, "
        f"{achieved_tf:.2f} TFLOP/s over {head['sets']} rotating operand sets "
        f"(one set, cache-resident: {head['resident_ms']:.4f} ms, {resident_tf:.2f} TFLOP/s), "
        f"sample_ok={head['sample_ok']}")

    secondary = []
    if not args.no_secondary:
        sq = bench_matmul_backward(ctx, rng, 4096, 1024, 4096, max(5, args.steps // 2),
                                   args.warmup, "C2'")
        tf = sq["flops"] / (sq["kernel_ms"] * 1e-3) / 1e12
        ent = {"workload": "C2' matmul_backward A[4096,1024] B[1024,4096]",
               "kernel": HEAD_KERNEL, "kernel_ms": round(sq["kernel_ms"], 5),
               "value": round(tf * 1e3, 1), "unit": "GFLOP/s",
               "frac": round(tf / PEAK_FP32_MFMA_TFLOPS, 4), "bound": "mfma",
               "resident_kernel_ms": round(sq["resident_ms"], 5), "sample_ok": sq["sample_ok"]}
        if not args.no_cpu_baseline:
            ent["cpu_baseline"] = cpu_baseline(*sq["inputs"], 256, 48)
        secondary.append(ent)
        log(f"  C2' {sq['kernel_ms']:.4f} ms {tf:.2f} TFLOP/s (resident {sq['resident_ms']:.4f} ms)")
        del sq
        rb = bench_relu_bias(ctx, rng, 4096, 4096, args.steps, args.warmup)
        gbs = rb["bytes"] / (rb["kernel_ms"] * 1e-3) / 1e9
        ent = {"workload": "C3 relu(X+b) backward: dX masked + db column sum, 4096x4096",
               "kernel": "colreduce_pass1+colreduce_finalize",
               "kernel_ms": round(rb["kernel_ms"], 5), "value": round(gbs, 1),
               "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4), "bound": "hbm",
               "algorithmic_bytes": rb["bytes"], "operand_sets": rb["sets"],
               "traffic": traffic_from_profile("relu_bias_4096"),
               "resident_kernel_ms": round(rb["resident_ms"], 5)}
        if not args.no_cpu_baseline:
            ent["cpu_baseline"] = cpu_baseline_relu_bias(*rb["inputs"])
        secondary.append(ent)
        log(f"  C3 relu+bias {rb['kernel_ms']:.4f} ms {gbs:.1f} GB/s "
            f"(resident {rb['resident_ms']:.4f} ms)")
        del rb
        ad = bench_adam(ctx, rng, 1 << 24, args.steps, args.warmup)
        gbs = ad["bytes"] / (ad["kernel_ms"] * 1e-3) / 1e9
        ent = {"workload": "C3 Adam step, 16,777,216 params", "kernel": "adam_kernel",
               "kernel_ms": round(ad["kernel_ms"], 5), "value": round(gbs, 1),
               "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4), "bound": "hbm",
               "algorithmic_bytes": ad["bytes"], "operand_sets": ad["sets"],
               "traffic": traffic_from_profile("adam_16m"),
               "resident_kernel_ms": round(ad["resident_ms"], 5)}
        if not args.no_cpu_baseline:
            ent["cpu_baseline"] = cpu_baseline_adam(1 << 24)
        secondary.append(ent)
        log(f"  C3 adam {ad['kernel_ms']:.4f} ms {gbs:.1f} GB/s "
            f"(resident {ad['resident_ms']:.4f} ms)")
        c1 = bench_c1(ctx, args.steps, args.warmup)
        ent = {"workload": "C1 MLP train step 64x784->128->10, CE, SGD 0.01 "
                           "(forward+backward+step via the device autograd engine)",
               "value": round(c1["us_per_step"], 1), "unit": "us/step",
               "bound": "latency", "kernels_per_step": C1_KERNELS,
               "launch_floor_us": round(c1["launch_floor_us"], 2),
               "final_loss": round(c1["loss"], 6)}
        if not args.no_cpu_baseline:
            ent["cpu_baseline"] = cpu_baseline_c1()
        secondary.append(ent)
        secondary.append({"workload": "C1 MLP train step as above, recorded once into a HIP graph "
                                      "and replayed per step (numrs_hip_graph_*; every kernel runs "
                                      "every step)",
                          "value": round(c1["graph_us_per_step"], 1), "unit": "us/step",
                          "steps": c1["steps"], "bound": "latency",
                          "final_loss": round(c1["graph_loss"], 6)})
        log(f"  C1 MLP step {c1['us_per_step']:.1f} us, graph replay "
            f"{c1['graph_us_per_step']:.1f} us, dependent-launch floor "
            f"{c1['launch_floor_us']:.2f} us ({C1_KERNELS} tiny kernels, graph-replayed)")
        c4 = bench_c4(ctx, max(10, args.steps), 3)
        ent = {"workload": "C4 pre-LN transformer block train step (16x256, d512, 8 "
                           "heads, FFN 2048 GELU, MSE, SGD) via the device engine",
               "value": round(c4["ms_per_step"], 3), "unit": "ms/step",
               "tflops_over_step": round(c4["tflops"], 2),
               "frac_of_fp32_mfma": round(c4["tflops"] / PEAK_FP32_MFMA_TFLOPS, 4),
               "bound": "mfma (GEMMs) + hbm (LN/GELU/softmax)",
               "final_loss": round(c4["loss"], 6)}
        if not args.no_cpu_baseline:
            ent["cpu_baseline"] = cpu_baseline_c4()
        secondary.append(ent)
        log(f"  C4 block step {c4['ms_per_step']:.3f} ms {c4['tflops']:.1f} TFLOP/s")
        c5 = bench_c5(ctx, max(5, args.steps // 4), 2)
        ent = {"workload": "C5 2-layer LSTM forecaster train step (in 64, hidden 256, "
                           "seq 128, batch 64, head 256->1, MSE, SGD) via the device engine",
               "value": round(c5["ms_per_step"], 3), "unit": "ms/step",
               "tflops_over_step": round(c5["tflops"], 2),
               "frac_of_fp32_mfma": round(c5["tflops"] / PEAK_FP32_MFMA_TFLOPS, 4),
               "bound": "latency (128 dependent steps per direction, one persistent launch each)",
               "final_loss": round(c5["loss"], 6)}
        if not args.no_cpu_baseline:
            ent["cpu_baseline"] = cpu_baseline_c5()
        secondary.append(ent)
        log(f"  C5 LSTM step {c5['ms_per_step']:.3f} ms {c5['tflops']:.2f} TFLOP/s")

    cpu = None
    if not args.no_cpu_baseline:
        log(f"cpu baseline: {args.cpu_rows_a} dA rows + {args.cpu_rows_b} dB rows, 1 thread")
        A, B, dC = head["inputs"]
        cpu = cpu_baseline(A, B, dC, args.cpu_rows_a, args.cpu_rows_b)
        log(f"  cpu {cpu['value']} GFLOP/s")

    line = {
        "metric": METRIC,
        "value": round(gflops, 1),
        "unit": "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warm_ms": WARM_MS,
        "warm_launches": _WARM_LAUNCHES,
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic N(0,1) inputs resident in HBM (seeded numpy PCG64); timed launches "
                "cycle through operand sets so that each launch reads HBM, not the 256 MB "
                "Infinity Cache",
        "config": {"workload": "C2 matmul_backward: dA = dC @ B^T, dB = A^T @ dC, fp32",
                   "M": M, "K": K, "N": N, "flops_per_step": head["flops"],
                   "operand_sets": head["sets"], "sample_ok": head["sample_ok"],
                   "device": arch, "cus": n_cus},
        "roofline": {"bound": "mfma", "kernel": HEAD_KERNEL,
                     "achieved": round(achieved_tf, 3), "peak": PEAK_FP32_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved_tf / PEAK_FP32_MFMA_TFLOPS, 4),
                     "kernel_ms": round(head["kernel_ms"], 5),
                     "traffic": traffic_from_profile("matmul_backward_2048"),
                     "resident_kernel_ms": round(head["resident_ms"], 5),
                     "resident_frac": round(resident_tf / PEAK_FP32_MFMA_TFLOPS, 4)},
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
