#!/usr/bin/env python3
"""INT8 InferenceSession throughput on one MI355X.

Default workload: the 4096^2 Linear stack (4 x Linear 4096->4096 + GELU,
input f32 [8192, 4096], seeded xavier weights), on which the metric's
"% of i8 MFMA peak" is quoted.  A step is one InferenceSession run over the
whole batch with the input already resident in HBM: per layer the absmax /
quantize kernels, the i8 MFMA GEMM with its fused dequant+bias+GELU
epilogue, all on the session's HIP stream.  The timed region is K runs back
to back bracketed by HIP events (rgnpu_program_benchmark); inside it every
kernel records the completion timestamp of its own dispatch, so the dominant
kernel's mean duration comes from the same region without perturbing it.

Prints one JSON line (driver contract): value = samples/s of the whole job,
roofline = the dominant kernel against the MI355X peak, cpu_baseline = the
C restatement of the reference's rayon CPU path timed on a bounded sample on
this host.  --workload gemv selects the batch-1 GEMV decode shape (HBM
roofline) for measurement runs.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "INT8 InferenceSession samples/s; achieved TOPS as % of i8 MFMA peak"
METRIC_FP16 = "FP16 InferenceSession samples/s; achieved TFLOP/s as % of f16 MFMA peak"
METRIC_FP32 = "FP32 (ExecutionProvider::Gpu) InferenceSession samples/s; achieved TFLOP/s as % of f32 MFMA peak"
PEAK_I8_TOPS = 5000.0     # MI355X dense i8 MFMA, 5.0 POP/s
PEAK_F16_TFLOPS = 2500.0  # MI355X dense f16 MFMA, 2.5 PFLOP/s
PEAK_F32_TFLOPS = 157.3   # MI355X dense f32 MFMA
PEAK_HBM_GBS = 8000.0     # MI355X HBM3E, 8 TB/s


def build_workload(name: str, batch: int, stack_act: str = "gelu", gemv_act: str = "silu"):
    from rustgears_amd import configs
    from rustgears_amd.inference import Activation, LayerSpec
    if name == "linear_stack":
        model, x = configs.linear_stack()
        layers = model.export()
        if stack_act != "gelu":  # measurement aid: same GEMMs with a cheap epilogue
            act = {"relu": Activation.RELU, "none": Activation.NONE}[stack_act]
            layers = [LayerSpec.Activation(act) if isinstance(l, LayerSpec.Activation) else l for l in layers]
        return layers, x, {"workload": f"linear_stack_4x4096_{stack_act}", "rows": 8192, "width": 4096,
                           "depth": 4, "activation": stack_act.upper(), "global_batch": 8192}
    if name == "gemv":
        # SiLU is the build's extension (nn/layers.rs:341-343 has no export);
        # the ReLU twin is a model the reference itself can express
        act = {"silu": Activation.SILU, "relu": Activation.RELU}[gemv_act]
        layers, x = configs.gemv(batch=batch, act=act)
        return layers, x, {"workload": f"gemv_8192x28672_{gemv_act}_b{batch}", "batch": batch, "d": 8192, "h": 28672,
                           "activation": gemv_act.upper(), "global_batch": batch}
    if name == "deep_mlp":
        model, x = configs.deep_mlp()
        return model.export(), x, {"workload": "deep_mlp_784_1024_1024_10", "rows": 4096, "global_batch": 4096}
    if name == "cnn":
        model, x = configs.cnn()
        return model.export(), x, {"workload": "cnn_3x32x32", "images": 256, "global_batch": 256}
    if name == "quickstart":
        model, x = configs.quickstart()
        return model.export(), x, {"workload": "quickstart_mlp", "rows": 64, "global_batch": 64}
    if name == "copy":
        # calibration: one standalone Activation(None) = a plain f32 copy of
        # 8192 x 4096 (128 MiB read, 128 MiB written) through the product's
        # elementwise kernel; used to scale the FETCH_SIZE / WRITE_SIZE counters
        from rustgears_amd import rng
        rng.manual_seed(11)
        x = rng.randn([8192, 4096])
        return [LayerSpec.Activation(Activation.NONE)], x, {"workload": "copy_8192x4096_f32", "rows": 8192,
                                                            "global_batch": 8192}
    raise SystemExit(f"unknown workload {name}")


def measured_traffic(workload: str, kernel: str, prec: str = "int8", occurrence: int = 0):
    """HBM bytes per launch of the `occurrence`-th op labelled `kernel` in
    `workload` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
    (profiles/hbm_traffic.txt: lines `workload<TAB>op label<TAB>bytes` in op
    order, already scaled by the copy calibration; the workload carries an
    `@fp16` / `@fp32` suffix for the other precisions, whose op labels can
    equal the INT8 ones); None when that op was not profiled."""
    if prec != "int8":
        workload = f"{workload}@{prec}"
    path = os.path.join(ROOT, "profiles", "hbm_traffic.txt")
    if not os.path.exists(path):
        return None
    seen = 0
    with open(path) as f:
        for line in f:
            parts = line.rstrip("\n").split("\t")
            if len(parts) == 3 and parts[0] == workload and parts[1] == kernel:
                if seen == occurrence:
                    return int(parts[2])
                seen += 1
    return None


# per precision: (metric, MFMA peak, dtype, bytes per weight/activation element, oracle precision)
PRECISIONS = {
    "int8": (METRIC, PEAK_I8_TOPS, "i8", 1, 0),
    "fp16": (METRIC_FP16, PEAK_F16_TFLOPS, "f16", 2, 1),
    "fp32": (METRIC_FP32, PEAK_F32_TFLOPS, "f32", 4, 2),
}


def dominant_roofline(name, records, layers, x, workload, prec="int8"):
    """Roofline of the dominant kernel (largest total kernel time per step)."""
    _, peak, _, eb, _ = PRECISIONS[prec]
    best = max(range(len(records)), key=lambda i: records[i].kernel_ns)
    r = records[best]
    if r.kernel_ns <= 0:
        return None, best
    occ = sum(1 for rr in records[:best] if rr.op == r.op)  # ops sharing the label before it
    secs = r.kernel_ns / 1e9
    if name == "gemv":
        # algorithmic bytes of one GEMV launch: weights N*K + f32 bias N +
        # activations B*K (i8, or binary16 for FP16) + f32 output B*N
        lin = [l for l in layers if type(l).__name__ == "Linear"]
        idx = [i for i, rr in enumerate(records) if "Gemm" in rr.op or "Linear" in rr.op][: len(lin)]
        li = lin[idx.index(best)] if best in idx else lin[0]
        b = x.shape[0]
        byts = eb * li.in_features * li.out_features + 4 * li.out_features + eb * b * li.in_features + 4 * b * li.out_features
        ach = byts / secs / 1e9
        return {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(ach / PEAK_HBM_GBS, 4), "traffic": measured_traffic(workload, r.op, prec, occ),
                "kernel": r.op, "kernel_us": round(r.kernel_ns / 1e3, 2), "algorithmic_bytes": byts}, best
    if r.macs == 0:
        # elementwise op (copy calibration): f32 in + f32 out
        byts = 8 * int(np.prod(x.shape))
        ach = byts / secs / 1e9
        return {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(ach / PEAK_HBM_GBS, 4), "traffic": measured_traffic(workload, r.op, prec, occ), "kernel": r.op,
                "kernel_us": round(r.kernel_ns / 1e3, 2), "algorithmic_bytes": byts}, best
    # ops that launch nothing after it ran inside its kernel (the second conv
    # of a conv pair, the later Linears of a whole-program kernel)
    macs, fused = r.macs, []
    for rr in records[best + 1:]:
        if rr.kernel_ns > 0:
            break
        if rr.macs > 0:
            macs += rr.macs
            fused.append(rr.op)
    ops = 2 * macs
    ach = ops / secs / 1e12
    out = {"bound": "mfma", "achieved": round(ach, 1), "peak": peak, "unit": "TFLOP/s",
           "frac": round(ach / peak, 4), "traffic": measured_traffic(workload, r.op, prec, occ), "kernel": r.op,
           "kernel_us": round(r.kernel_ns / 1e3, 2), "algorithmic_ops": ops}
    if fused:
        out["fused_ops"] = fused
    return out, best


def host_description() -> dict:
    """CPU model and glibc version of the host the baseline ran on (the
    oracle's GELU, Sigmoid and Tanh follow the host libm)."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        libc = os.confstr("CS_GNU_LIBC_VERSION")
    except (ValueError, OSError):
        libc = ""
    return {"cpu": model, "logical_cpus": os.cpu_count(), "libc": libc}


def cpu_baseline(name, layers, x, target_s: float, prec="int8"):
    """The oracle (C restatement of the reference's rayon INT8 path, or of
    its FP16 path) on a bounded sample of the same workload, all host
    threads: a probe pass over a row sample, then as many passes as fill
    about target_s seconds."""
    import oracle
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
    oracle.set_threads(threads)
    prog = oracle.RefProgram(layers, precision=PRECISIONS[prec][4])
    fp16 = prec == "fp16"
    n = x.shape[0]
    rows = n if name in ("gemv", "copy") else max(1, min(n, 64))
    t0 = time.perf_counter()
    prog.run(x[:rows], parallel=True)
    dt = time.perf_counter() - t0
    if rows < n and dt < target_s / 8:
        rows = int(min(n, max(rows, rows * target_s / 4 / max(dt, 1e-6))))
        t0 = time.perf_counter()
        prog.run(x[:rows], parallel=True)
        dt = time.perf_counter() - t0
    passes = int(max(1, min(1000, round(target_s / max(dt, 1e-6)))))
    t0 = time.perf_counter()
    for _ in range(passes):
        prog.run(x[:rows], parallel=True)
    dt = time.perf_counter() - t0
    eff = min(rows, threads)
    if fp16:
        # the reference's FP16 Linear is serial (npu.rs:433-445); only conv
        # images run in parallel (npu.rs:331)
        cores = threads if name == "cnn" else 1
        return {"value": round(passes * rows / dt, 3), "unit": "samples/s", "cores": cores, "kind": "port",
                "sample": f"{passes} pass(es) over {rows} of {n} samples of the same workload ({dt:.1f} s); FP16 "
                          f"path: Linear serial as in the reference, conv image-parallel"}
    if prec == "fp32":
        return {"value": round(passes * rows / dt, 3), "unit": "samples/s", "cores": threads, "kind": "port",
                "sample": f"{passes} pass(es) over {rows} of {n} samples of the same workload ({dt:.1f} s); the "
                          f"standard path with a serial-k f32 matmul (no FMA), parallel over rows and 256-column "
                          f"blocks (the reference's CPU backend blocks its matmul with AVX2/FMA, cpu.rs:43-160)"}
    return {"value": round(passes * rows / dt, 3), "unit": "samples/s", "cores": threads, "kind": "port",
            "sample": f"{passes} pass(es) over {rows} of {n} samples of the same workload ({dt:.1f} s); row-parallel "
                      f"like rayon (quantize.rs:104), effective parallelism min(rows, threads) = {eff}"}


def mfma_peak(rg, args):
    """The sustained i8 MFMA rate the GEMMs are measured against: the
    register-only probe kernel (kernels.hip mfma_peak_kernel, 8 waves per CU,
    32 independent v_mfma_i32_16x16x64_i8 per round, the large GEMM's inner
    loop without its memory traffic) on random and on all-zero operand bytes,
    for launches of about 1, 5 and 20 ms; `steps` launches each, the
    median reported.  The rate under random data is what bounds the S
    GEMM's K loop; the zero-operand rate shows the data-dependent power
    limit."""
    import ctypes
    from rustgears_amd import _native as N
    peak = 5000.0
    res = {}
    for mode, rnd in (("random", 1), ("zero", 0)):
        res[mode] = {}
        for iters in (500, 2_500, 10_000):
            rates, mss = [], []
            for k in range(args.warmup + args.steps):
                ms, tops = ctypes.c_double(), ctypes.c_double()
                N.check(N.lib().rgnpu_probe_mfma_rate(0, iters, rnd, ctypes.byref(ms), ctypes.byref(tops)))
                if k >= args.warmup:
                    rates.append(tops.value)
                    mss.append(ms.value)
            res[mode][iters] = (float(np.median(rates)), float(np.median(mss)))
            print(f"# mfma probe {mode:6s} iters {iters:6d}: {res[mode][iters][1]:7.3f} ms "
                  f"{res[mode][iters][0]:8.1f} TOPS ({100 * res[mode][iters][0] / peak:.1f}% of {peak:.0f})",
                  file=sys.stderr, flush=True)
    long_iters = 10_000
    v = res["random"][long_iters][0]
    line = {"metric": "sustained i8 MFMA rate (register-only probe, random operands)", "value": round(v, 1),
            "unit": "TOPS", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(res["random"][long_iters][1], 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "i8", "data": "synthetic: SplitMix64 operand bytes / all-zero bytes",
            "config": {"workload": "mfma_peak", "kernel": "mfma_peak_kernel", "waves_per_cu": 8,
                       "mfma": "v_mfma_i32_16x16x64_i8"},
            "frac_of_peak": round(v / peak, 4), "peak": peak,
            "by_launch": {mode: {str(it): {"tops": round(r[0], 1), "ms": round(r[1], 4)} for it, r in d.items()}
                          for mode, d in res.items()}}
    print(json.dumps(line))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="linear_stack",
                    choices=["linear_stack", "gemv", "deep_mlp", "cnn", "quickstart", "copy", "mfma_peak"])
    ap.add_argument("--batch", type=int, default=1, help="gemv batch (1 or 8)")
    ap.add_argument("--gemv-act", default="silu", choices=["silu", "relu"],
                    help="activation after the first gemv layer (relu: the twin the reference can express)")
    ap.add_argument("--stack-act", default="gelu", choices=["gelu", "relu", "none"],
                    help="activation of the linear_stack workload (gelu is the benchmark config)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--prewarm-ms", type=float, default=200.0,
                    help="before the W warmup steps, run the step untimed for at least this long, so the GPU's "
                         "clocks have ramped up when the timed region starts (0: off)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--device-only", action="store_true",
                    help="skip the host-pointer rates (pcie_inclusive*): profiler runs of the device-resident "
                         "region")
    ap.add_argument("--precision", default="int8", choices=["int8", "fp16", "fp32"],
                    help="NpuPrecision of the session (the headline metric is INT8)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus must be 1 (multi-GPU sharding is "
                                   "designed, not built or run)"}))
        sys.exit(2)

    import rustgears_amd as rg

    if args.workload == "mfma_peak":
        mfma_peak(rg, args)
        return

    t_setup = time.perf_counter()
    layers, x, config = build_workload(args.workload, args.batch, args.stack_act, args.gemv_act)
    fp16 = args.precision == "fp16"
    fp32 = args.precision == "fp32"
    provider = (rg.ExecutionProvider.mi355x_fp16() if fp16 else
                rg.ExecutionProvider.Gpu(0) if fp32 else rg.ExecutionProvider.mi355x_int8())
    sess = rg.InferenceSession.from_layers(layers, provider)
    out_shape = sess.output_shape(x.shape)
    dx = rg.DeviceBuffer.from_array(x)
    dy = rg.DeviceBuffer(int(np.prod(out_shape)) * 4)
    print(f"# setup {time.perf_counter() - t_setup:.1f}s; {sess.compilation_report().splitlines()[-1].strip()}",
          file=sys.stderr, flush=True)

    # Clock ramp: a few warmup steps of a sub-millisecond step are over
    # before the GPU leaves its idle clocks, and the timed region then ran
    # ~5% slower than the same runs measured right after it.
    prewarm_runs, t_pw = 0, time.perf_counter()
    while args.prewarm_ms > 0 and (time.perf_counter() - t_pw) * 1e3 < args.prewarm_ms:
        sess.benchmark(dx, x.shape, dy, 10, per_kernel_events=False)
        prewarm_runs += 10
    if args.warmup > 0:
        sess.benchmark(dx, x.shape, dy, args.warmup, per_kernel_events=False)
    rg.lib().rgnpu_device_synchronize()
    # Timed region: K runs back to back between two HIP events, no other
    # events recorded.
    w0 = time.perf_counter()
    dev_ms, _ = sess.benchmark(dx, x.shape, dy, args.steps, per_kernel_events=False)
    rg.lib().rgnpu_device_synchronize()
    wall = time.perf_counter() - w0
    ms_per_step = dev_ms / args.steps
    # The same K runs again with every kernel recording the completion
    # timestamp of its own dispatch (no marker packet per kernel): each op's
    # mean kernel duration, for the roofline, comes from this region.
    dev_ms_ev, recs = sess.benchmark(dx, x.shape, dy, args.steps, per_kernel_events=True)

    batch = x.shape[0]
    value = batch / (ms_per_step / 1e3)
    total_macs = sum(r.macs for r in recs)
    tops = 2 * total_macs / (ms_per_step / 1e3) / 1e12
    roof, dom = dominant_roofline(args.workload, recs, layers, x, config["workload"], args.precision)
    if roof is not None and roof["bound"] == "hbm":
        # The same kernel with the 256 MB memory-side cache displaced before
        # every run (512 MiB of other data read outside the op intervals): a
        # duration equal to kernel_us shows that the cache does not serve the
        # weights between back-to-back runs.
        _, recs_ev = sess.benchmark(dx, x.shape, dy, min(args.steps, 20), per_kernel_events=True, evict_cache=True)
        k_ev = recs_ev[dom].kernel_ns / 1e3
        if k_ev > 0:
            roof["kernel_us_cache_evicted"] = round(k_ev, 2)
            roof["achieved_cache_evicted"] = round(roof["achieved"] * roof["kernel_us"] / k_ev, 1)
    metric, peak, dtype, _, _ = PRECISIONS[args.precision]
    for r in recs:
        print(f"#   {r.op:<44} {r.macs:>14} MACs  op {r.duration_ns / 1e3:9.2f} us  kernel {r.kernel_ns / 1e3:9.2f} us",
              file=sys.stderr)
    line = {
        "metric": metric, "value": round(value, 2), "unit": "samples/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "prewarm_runs": prewarm_runs,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": dtype,
        "data": "synthetic: RustGears SplitMix64 seeded weights and inputs (rustgears_amd/configs.py)",
        "config": config,
        "tops": round(tops, 2),
        ("tops_frac_of_i8_peak" if args.precision == "int8" else f"tflops_frac_of_{dtype}_peak"):
            round(tops / peak, 4),
        "ms_per_step_with_kernel_events": round(dev_ms_ev / args.steps, 4),
        "wall_s_timed_region": round(wall, 4),
        "roofline": roof,
    }
    # PCIe-inclusive rate: InferenceSession.run with host buffers (H2D of the
    # input, the run, D2H of the output), wall clock; reported beside value.
    # Each rate runs for at least HOST_S seconds of wall clock.
    HOST_S = 0.5

    def host_runs(deadline):
        n = 0
        while n < 3 or time.perf_counter() < deadline:
            sess.run(x)
            n += 1
        return n

    if args.device_only:
        if not args.no_cpu_baseline:
            line["cpu_baseline"] = cpu_baseline(args.workload, layers, x, args.cpu_seconds, args.precision)
            line["cpu_baseline"]["host"] = host_description()
        print(json.dumps(line), flush=True)
        return
    sess.run(x)
    h0 = time.perf_counter()
    n_host = host_runs(h0 + HOST_S)
    host_s = (time.perf_counter() - h0) / n_host
    line["pcie_inclusive"] = {"value": round(batch / host_s, 2), "unit": "samples/s", "ms_per_step": round(host_s * 1e3, 3),
                              "steps": n_host, "note": "host-pointer run(): H2D input + run + D2H output, wall clock"}
    # The same from several threads on the one session (run(&self) is Sync):
    # each call borrows its own worker stream, so copies overlap kernels.
    threads = 4
    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(threads) as ex:
        list(ex.map(lambda _: sess.run(x), range(threads)))
        h0 = time.perf_counter()
        n_conc = sum(ex.map(host_runs, [h0 + HOST_S] * threads))
        conc_s = time.perf_counter() - h0
    line["pcie_inclusive_concurrent"] = {
        "value": round(n_conc * batch / conc_s, 2), "unit": "samples/s", "threads": threads,
        "runs": n_conc, "note": "host-pointer run() from several threads on one session, wall clock",
        # cumulative over the session (all runs above): workgroups of the
        # persistent grids that gave up waiting at the barrier and deferred
        # their quantization, and finished barrier launches
        "barrier": sess.barrier_stats()}
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args.workload, layers, x, args.cpu_seconds, args.precision)
        line["cpu_baseline"]["host"] = host_description()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
