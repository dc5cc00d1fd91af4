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


def time_launches(ctx, launch, steps: int, warmup: int):
    """Runs `launch` warmup times, then `steps` times inside one timed region
    (event slots 0/1) on the context's stream -- the stream the kernels run
    on.  The first min(steps, 127) launches also get their own event pair
    (slots 2.., read only after the region, so the host never stalls the
    stream).  Returns (total ms of the region, mean per-launch ms)."""
    for _ in range(warmup):
        launch()
    ctx.sync()
    paired = min(steps, 127)
    ctx.timer_record(0)
    for i in range(steps):
        if i < paired:
            ctx.timer_record(2 + 2 * i)
        launch()
        if i < paired:
            ctx.timer_record(3 + 2 * i)
    ctx.timer_record(1)
    ctx.sync()
    total = ctx.timer_elapsed_ms(0, 1)
    per = [ctx.timer_elapsed_ms(2 + 2 * i, 3 + 2 * i) for i in range(paired)]
    return total, float(np.mean(per))


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
    true HBM traffic is known -- then `reps` 2048^3 matmul_backward launches."""
    n = COPY_PROBE_BYTES // 4
    src, dst = ctx.to_device(randn(rng, n)), ctx.empty(n)
    for _ in range(reps):
        ctx.copy(dst, src)
    ctx.sync()
    M = K = N = 2048
    A_, B_, dC_ = (ctx.to_device(randn(rng, s)) for s in ((M, K), (K, N), (M, N)))
    dA_, dB_ = ctx.empty((M, K)), ctx.empty((K, N))
    for _ in range(reps):
        ctx.matmul_backward(dC_, A_, B_, dA_, dB_)
    ctx.sync()
    log(f"traffic probe: {reps} copies of {COPY_PROBE_BYTES} B, {reps} matmul_backward 2048^3")


def _pmc_per_dispatch(directory: str, counter: str) -> dict:
    """Mean value of `counter` per dispatch, by kernel name, from a rocprofv3
    --pmc -f csv output directory."""
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
                per[key] = per.get(key, 0.0) + float(row["Counter_Value"])
    out = {}
    for (name, _), v in per.items():
        out.setdefault(name, []).append(v)
    return {k: float(np.mean(v)) for k, v in out.items()}


def traffic_summary(fetch_dir: str, write_dir: str) -> dict:
    """HBM bytes per matmul_backward launch: FETCH_SIZE and WRITE_SIZE (KiB
    per dispatch), each scaled by the factor that maps the copy kernel's
    reading of the same counter onto its known COPY_PROBE_BYTES."""
    fetch = _pmc_per_dispatch(fetch_dir, "FETCH_SIZE")
    write = _pmc_per_dispatch(write_dir, "WRITE_SIZE")

    def pick(d, part):
        keys = [k for k in d if part in k]
        if len(keys) != 1:
            raise KeyError(f"{part}: {keys}")
        return d[keys[0]]

    known_kib = COPY_PROBE_BYTES / 1024.0
    f_copy, w_copy = pick(fetch, "copy_kernel"), pick(write, "copy_kernel")
    f_mm, w_mm = pick(fetch, HEAD_KERNEL), pick(write, HEAD_KERNEL)
    ff, fw = known_kib / f_copy, known_kib / w_copy
    traffic = (f_mm * ff + w_mm * fw) * 1024.0
    algorithmic = 5 * 2048 * 2048 * 4  # read A, B, dC; write dA, dB
    res = {"kernel": HEAD_KERNEL, "workload": "C2 2048^3",
           "fetch_kib_raw": f_mm, "write_kib_raw": w_mm,
           "copy_fetch_kib_raw": f_copy, "copy_write_kib_raw": w_copy,
           "copy_bytes": COPY_PROBE_BYTES, "fetch_factor": ff, "write_factor": fw,
           "bytes_per_launch": traffic, "algorithmic_bytes": algorithmic,
           "traffic_over_algorithmic": traffic / algorithmic}
    return res


def bench_matmul_backward(ctx, rng, M, K, N, steps, warmup):
    A, B, dC = randn(rng, (M, K)), randn(rng, (K, N)), randn(rng, (M, N))
    dA_, B_, dC_ = ctx.empty((M, K)), ctx.to_device(B), ctx.to_device(dC)
    A_, dB_ = ctx.to_device(A), ctx.empty((K, N))
    total, per = time_launches(ctx, lambda: ctx.matmul_backward(dC_, A_, B_, dA_, dB_), steps,
                               warmup)
    flops = 4.0 * M * K * N
    # Sanity: one sampled row of each gradient against float64 numpy.
    ga, gb = dA_.numpy()[M // 3], dB_.numpy()[K // 5]
    ra = dC[M // 3].astype(np.float64) @ B.astype(np.float64).T
    rb = A[:, K // 5].astype(np.float64) @ dC.astype(np.float64)
    # Tolerance of the parity tests: 1e-5 + 1e-4|r| plus the fp32 rounding
    # allowance 4 * 2^-24 * K of a length-K contraction.
    ok = bool(np.all(np.abs(ga - ra) <= 1e-5 + 4 * 2.0**-24 * N + 1e-4 * np.abs(ra)) and
              np.all(np.abs(gb - rb) <= 1e-5 + 4 * 2.0**-24 * M + 1e-4 * np.abs(rb)))
    return {"ms_per_step": total / steps, "kernel_ms": per, "flops": flops, "sample_ok": ok,
            "inputs": (A, B, dC)}


def bench_relu_bias(ctx, rng, rows, cols, steps, warmup):
    g, z = randn(rng, (rows, cols)), randn(rng, (rows, cols))
    g_, z_ = ctx.to_device(g), ctx.to_device(z)
    dx_, db_ = ctx.empty((rows, cols)), ctx.empty((cols,))
    total, per = time_launches(ctx, lambda: ctx.relu_bias_backward(g_, z_, dx_, db_), steps, warmup)
    nbytes = 12.0 * rows * cols + 4.0 * cols  # read g, z; write dx; write db
    return {"ms_per_step": total / steps, "kernel_ms": per, "bytes": nbytes}


def bench_adam(ctx, rng, n, steps, warmup):
    p_, g_ = ctx.to_device(randn(rng, n)), ctx.to_device(randn(rng, n))
    m_, v_ = ctx.zeros(n), ctx.zeros(n)
    state = {"t": 0}

    def launch():
        state["t"] += 1
        ctx.adam_step(p_, g_, m_, v_, state["t"], lr=1e-3)

    total, per = time_launches(ctx, launch, steps, warmup)
    return {"ms_per_step": total / steps, "kernel_ms": per, "bytes": 28.0 * n}


def bench_c1(ctx, steps, warmup):
    """2-layer MLP (64x784 -> 128 -> ReLU -> 10, softmax CE,
    SGD lr 0.01) -- forward, backward and SGD step through the device
    autograd engine, timed per step with a device sync at the end of each
    step (a loss read-back is what a training loop does)."""
    import numrs_amd as nr
    from numrs_amd import Tensor, nn, optim
    from tests.mlp_oracle import make_c1

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
    t0 = time.perf_counter()
    for _ in range(steps):
        loss = step()
    loss.item()
    per = (time.perf_counter() - t0) / steps
    return {"us_per_step": per * 1e6, "loss": loss.item()}


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
    from tests.transformer_oracle import make_c4

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
    from tests.lstm_oracle import make_c5

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
    return {
        "value": round(4.0 * M * K * N / full_s / 1e9, 4),
        "unit": "GFLOP/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"C restatement of numrs matmul_backward (oracle/numrs_oracle.c, fp32 triple "
                   f"loops of backward.rs:123-146), {rows_a} of {M} dA rows ({ta:.2f} s) + "
                   f"{rows_b} of {K} dB rows ({tb:.2f} s), scaled to the full 2048^3 step "
                   f"({full_s:.1f} s); host {platform.processor() or platform.machine()}, "
                   f"{os.cpu_count()} logical CPUs visible, 1 thread used"),
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--cpu-rows-a", type=int, default=512)
    ap.add_argument("--cpu-rows-b", type=int, default=192)
    ap.add_argument("--only", choices=["c1", "c4", "c5"], default=None,
                    help="run only this secondary workload (for profiling); prints its entry")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only launch the calibration copy and the 2048^3 matmul_backward "
                         "(run under rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE)")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="turn the two --pmc outputs of --traffic-probe into "
                         "profiles/matmul_backward_2048_traffic.json (no GPU needed)")
    args = ap.parse_args()

    if args.traffic_summary:
        res = traffic_summary(*args.traffic_summary)
        with open(os.path.join(ROOT, "profiles", "matmul_backward_2048_traffic.json"), "w") as f:
            json.dump(res, f, indent=1)
            f.write("\n")
        print(json.dumps(res), flush=True)
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
    n_cus, arch = ctx.info()
    log(f"device {arch}, {n_cus} CUs")
    rng = np.random.default_rng(SEED)

    if args.traffic_probe:
        traffic_probe(ctx, rng)
        ctx.close()
        return 0

    if args.only is not None:
        fn = {"c1": lambda: bench_c1(ctx, args.steps, args.warmup),
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
    log(f"  {head['ms_per_step']:.4f} ms/step, kernel {head['kernel_ms']:.4f} ms, "
        f"{achieved_tf:.2f} TFLOP/s, sample_ok={head['sample_ok']}")

    secondary = []
    if not args.no_secondary:
        sq = bench_matmul_backward(ctx, rng, 4096, 1024, 4096, max(5, args.steps // 2),
                                   args.warmup)
        tf = sq["flops"] / (sq["kernel_ms"] * 1e-3) / 1e12
        secondary.append({"workload": "C2' matmul_backward A[4096,1024] B[1024,4096]",
                          "kernel": HEAD_KERNEL, "kernel_ms": round(sq["kernel_ms"], 5),
                          "value": round(tf * 1e3, 1), "unit": "GFLOP/s",
                          "frac": round(tf / PEAK_FP32_MFMA_TFLOPS, 4), "bound": "mfma",
                          "sample_ok": sq["sample_ok"]})
        log(f"  C2' {sq['kernel_ms']:.4f} ms {tf:.2f} TFLOP/s")
        rb = bench_relu_bias(ctx, rng, 4096, 4096, args.steps, args.warmup)
        gbs = rb["bytes"] / (rb["kernel_ms"] * 1e-3) / 1e9
        secondary.append({"workload": "C3 relu(X+b) backward: dX masked + db column sum, 4096x4096",
                          "kernel": "colreduce_pass1+colreduce_finalize",
                          "kernel_ms": round(rb["kernel_ms"], 5), "value": round(gbs, 1),
                          "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4), "bound": "hbm",
                          "algorithmic_bytes": rb["bytes"]})
        log(f"  C3 relu+bias {rb['kernel_ms']:.4f} ms {gbs:.1f} GB/s")
        ad = bench_adam(ctx, rng, 1 << 24, args.steps, args.warmup)
        gbs = ad["bytes"] / (ad["kernel_ms"] * 1e-3) / 1e9
        secondary.append({"workload": "C3 Adam step, 16,777,216 params", "kernel": "adam_kernel",
                          "kernel_ms": round(ad["kernel_ms"], 5), "value": round(gbs, 1),
                          "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4), "bound": "hbm",
                          "algorithmic_bytes": ad["bytes"]})
        log(f"  C3 adam {ad['kernel_ms']:.4f} ms {gbs:.1f} GB/s")
        c1 = bench_c1(ctx, args.steps, args.warmup)
        secondary.append({"workload": "C1 MLP train step 64x784->128->10, CE, SGD 0.01 "
                                      "(forward+backward+step via the device autograd engine)",
                          "value": round(c1["us_per_step"], 1), "unit": "us/step",
                          "bound": "latency", "final_loss": round(c1["loss"], 6)})
        log(f"  C1 MLP step {c1['us_per_step']:.1f} us")
        c4 = bench_c4(ctx, max(3, args.steps // 5), 2)
        secondary.append({"workload": "C4 pre-LN transformer block train step (16x256, d512, 8 "
                                      "heads, FFN 2048 GELU, MSE, SGD) via the device engine",
                          "value": round(c4["ms_per_step"], 3), "unit": "ms/step",
                          "tflops_over_step": round(c4["tflops"], 2),
                          "frac_of_fp32_mfma": round(c4["tflops"] / PEAK_FP32_MFMA_TFLOPS, 4),
                          "bound": "mfma (GEMMs) + hbm (LN/GELU/softmax)",
                          "final_loss": round(c4["loss"], 6)})
        log(f"  C4 block step {c4['ms_per_step']:.3f} ms {c4['tflops']:.1f} TFLOP/s")
        c5 = bench_c5(ctx, max(3, args.steps // 10), 1)
        secondary.append({"workload": "C5 2-layer LSTM forecaster train step (in 64, hidden 256, "
                                      "seq 128, batch 64, head 256->1, MSE, SGD) via the device "
                                      "engine",
                          "value": round(c5["ms_per_step"], 3), "unit": "ms/step",
                          "tflops_over_step": round(c5["tflops"], 2),
                          "bound": "latency (256 sequential step kernels per direction)",
                          "final_loss": round(c5["loss"], 6)})
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
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic N(0,1) inputs resident in HBM (seeded numpy PCG64)",
        "config": {"workload": "C2 matmul_backward: dA = dC @ B^T, dB = A^T @ dC, fp32",
                   "M": M, "K": K, "N": N, "flops_per_step": head["flops"],
                   "sample_ok": head["sample_ok"], "device": arch, "cus": n_cus},
        "roofline": {"bound": "mfma", "kernel": HEAD_KERNEL,
                     "achieved": round(achieved_tf, 3), "peak": PEAK_FP32_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved_tf / PEAK_FP32_MFMA_TFLOPS, 4),
                     "kernel_ms": round(head["kernel_ms"], 5),
                     "traffic": traffic_from_profile("matmul_backward_2048")},
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
