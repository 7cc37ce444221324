"""Benchmark: the BASELINE StableHLO graphs through the MI355X PJRT plugin (client.compile → resident input
buffers → execute → await), reported as whole-job TFLOP/s (GB/s for the memory-bound calibrations) plus each
graph's dominant kernel against its roofline.

A step is one execution of a graph's StableHLO module on inputs already resident in HBM. Steps are enqueued back to
back (async dispatch, like a JAX-style caller) and the timed region ends when the last step's done event is ready;
the per-step latency with an await after every execute is reported alongside. Kernel durations come from HIP events
recorded on the plugin's stream by each step's first and last kernel launch (the plugin's timing extension), in a
separate pass; the roofline uses their median.

With no --config every graph runs: C5 (the largest, by FLOPs) is the headline line's `value`, and `per_graph`
holds C1–C5 plus the two HBM calibrations (copy, rmsnorm), each with its own value, kernels, roofline and CPU
baseline. HBM traffic and MFMA utilisation come from rocprofv3 counter runs committed under profiles/
(counters_<workload>.json): MFMA busy = (SQ_VALU_MFMA_BUSY_CYCLES / 1024 SIMDs) / (SQ_BUSY_CU_CYCLES / 256 CUs).

`--config argmax` runs an extra workload that is not a BASELINE graph: greedy decoding's argmax over f32 logits
[64, 128256] (a value-and-position reduce), priced in bytes like the calibrations.

The cyclic garbage collector is paused during the timed region (as `timeit` does); the plugin's own work is
unchanged.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config all|c1|c2|c3|c4|c5|c5x|copy|rmsnorm|argmax]
                       [--cpu-seconds S] [--no-cpu-baseline]
"""
import argparse
import gc
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "TFLOP/s and % of MFMA/HBM roofline per StableHLO graph on 1 MI355X vs XLA CPU"
HEADLINE = "c5"
ALL = ["c5", "c1", "c2", "c3", "c4", "copy", "rmsnorm"]
CHOICES = ["all", "c1", "c2", "c3", "c4", "c5", "c5x", "copy", "rmsnorm", "argmax"]


def _workload(name):
    from ryft_amd import configs
    return configs.CONFIGS[name]()


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _blas_threads():
    try:
        from threadpoolctl import threadpool_info
        n = [p["num_threads"] for p in threadpool_info() if p.get("user_api") == "blas"]
        if n:
            return max(n)
    except Exception:
        pass
    return int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)


def _cpu_baseline(name, seconds, w=None, gpu_outputs=None):
    """CPU baseline of graph `name`: the C++ / OpenMP executor of the graph (oracle/cpu_exec.cc, built -O3
    -march=native for this host, OpenMP over its cores) on the full workload `w` — the same input bytes the GPU
    ran — for at least 5 evaluations and `seconds`; its outputs are compared with the GPU's (`gpu_outputs`, raw
    arrays). Graphs it does not implement (the fp8-activation C5 extra) time the numpy oracle on a bounded sample."""
    from oracle import cpu_exec
    from oracle import stablehlo as sh
    from ryft_amd import configs
    from tests.helpers import MLIR_DT

    if name in ("c1", "c2", "c3", "c4", "c5", "copy", "rmsnorm"):
        w = w or configs.CONFIGS[name]()
        fn, outs = cpu_exec.prepare(name, w)
        _, arch = cpu_exec.library()
        threads = cpu_exec.threads()
        fn()  # first touch of the output pages and the packed panels
        t0 = time.perf_counter()
        reps = 0
        while True:
            fn()
            reps += 1
            el = time.perf_counter() - t0
            if (reps >= 5 and el >= seconds) or reps >= 500:
                break
        agree = None
        if gpu_outputs:
            errs = []
            for got, ref in zip(outs, gpu_outputs):
                if got.dtype.kind in "iu" and ref.dtype.kind in "iu" and got.dtype == ref.dtype and \
                        got.dtype.itemsize == 4:
                    errs.append(float(np.count_nonzero(got != ref)))  # integer accumulators: mismatch count
                else:
                    dt = {2: "bf16", 1: "f8E4M3FN"}.get(got.dtype.itemsize, "f32") if got.dtype.kind in "iu" else "f32"
                    errs.append(sh.rel_error(sh.from_raw(got, dt), sh.from_raw(ref, dt)))
            agree = errs
        what = (f"the full {w.name} workload (same input bytes as the GPU run), {reps} evaluation(s) in {el:.2f} s; "
                f"C++ executor oracle/cpu_exec.cc (-O3 -march={arch}, OpenMP, {threads} threads; register-tiled "
                f"GEMMs over packed panels, bf16 / f8 widened to f32 while packing, int8 exactly in int32); host "
                f"{_cpu_model()}, {os.cpu_count()} logical CPUs visible")
        res = {"unit": "GB/s" if not w.flops else "TFLOP/s", "cores": threads, "kind": "port", "sample": what,
               "evaluations": reps, "seconds": round(el, 3)}
        res["value"] = round(w.bytes * reps / el / 1e9, 4) if not w.flops else round(w.flops * reps / el / 1e12, 6)
        if agree is not None:
            res["rel_error_vs_gpu"] = agree
        return res

    if name == "argmax":
        # numpy's argmax of the same logits (first occurrence, as the comparator body picks): the oracle folds the
        # body element by element, too slow to be a fair CPU figure
        w = w or configs.CONFIGS[name]()
        x = w.inputs[0].data
        t0 = time.perf_counter()
        reps = 0
        while True:
            np.argmax(x, axis=1)
            np.max(x, axis=1)
            reps += 1
            el = time.perf_counter() - t0
            if (reps >= 5 and el >= seconds) or reps >= 10000:
                break
        what = (f"the full {w.name} workload, {reps} evaluation(s) in {el:.2f} s (numpy argmax + max over the rows, "
                f"one thread; host {_cpu_model()}, {os.cpu_count()} logical CPUs visible)")
        return {"value": round(w.bytes * reps / el / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": what, "evaluations": reps, "seconds": round(el, 3)}

    samples = {"c5x": (configs.c5x_swiglu_fp8_activations, {"m": 64}, "64 of the 512 tokens of C5 (fp8 activations)")}
    fn, kw, desc = samples[name]
    w = fn(**kw)
    vals = [sh.from_raw(x.data, MLIR_DT[x.type]) for x in w.inputs]
    t0 = time.perf_counter()
    reps = 0
    while True:
        sh.evaluate(w.program, vals, dot_precision="f32")
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds or reps >= 1000:
            break
    threads = _blas_threads()
    what = (f"{desc}, {reps} evaluation(s) in {el:.1f} s (numpy oracle: f32 dots on {threads} BLAS threads, "
            f"other ops single-threaded; host {_cpu_model()}, {os.cpu_count()} logical CPUs visible)")
    return {"value": round(w.flops * reps / el / 1e12, 6), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": what}


def _counters(workload_name, kernel):
    """HBM bytes per launch, MFMA busy fraction and shader clock of `kernel` from the committed counter runs."""
    path = os.path.join(ROOT, "profiles", f"counters_{workload_name}.json")
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        return json.load(f).get(kernel, {})


def measure(name, steps, warmup, cpu_seconds, client, dev):
    from ryft_amd import configs, pjrt

    w = _workload(name)
    exe = client.compile(pjrt.Program.mlir(w.program))
    bufs = [client.buffer(x.data, x.type, x.dims, device=dev) for x in w.inputs]
    for b in bufs:
        b.ready_event().await_()

    def step():
        return exe.execute([bufs])[0]

    # warm-up in the timed pattern (back to back), so the allocator already caches the output blocks that
    # overlapping steps hold
    last = None
    for _ in range(warmup):
        last = step()
    if last is not None:
        last.done.await_()

    # timed region: K steps enqueued back to back, ending when the last one is done. Python's cyclic garbage
    # collector is paused while the steps are timed (as timeit does): one full collection stalls the enqueueing
    # thread for about a millisecond, which would be billed to the steps, not to the plugin or its kernels.
    gc.collect()
    gc.disable()
    t0 = time.perf_counter()
    last = None
    for _ in range(steps):
        last = step()
    t_enqueued = time.perf_counter()
    last.done.await_()
    elapsed = time.perf_counter() - t0
    gc.enable()
    ms_per_step = elapsed / steps * 1e3

    # per-step latency with an await after each execute (the README's call pattern)
    t1 = time.perf_counter()
    for _ in range(steps):
        step().done.await_()
    ms_sync = (time.perf_counter() - t1) / steps * 1e3

    # PCIe-inclusive rate (not the headline): host inputs → device buffers → execute → results back to host
    pcie_steps = max(1, min(steps, 3))
    t2 = time.perf_counter()
    for _ in range(pcie_steps):
        hb = [client.buffer(x.data, x.type, x.dims, device=dev) for x in w.inputs]
        res = exe.execute([hb])[0]
        res.done.await_()
        gpu_outputs = [o.to_numpy() for o in res.outputs]
    ms_pcie = (time.perf_counter() - t2) / pcie_steps * 1e3

    # kernel timing pass (HIP events on the plugin stream, carried by the launches themselves)
    client.set_kernel_timing(True)
    for _ in range(steps):
        last = step()
    last.done.await_()
    kernels = client.kernel_timing()
    client.set_kernel_timing(False)

    dom_name, dom = max(kernels.items(), key=lambda kv: kv[1]["total_ms"])
    mfma = dom["flops"] > 0
    med_s = dom["median_us"] * 1e-6
    if mfma:
        achieved = dom["flops"] / med_s / 1e12
        peak = configs.PEAK_TFLOPS[w.compute_dtype]
        unit = "TFLOP/s"
    else:
        achieved = dom["bytes"] / med_s / 1e9
        peak = configs.PEAK_HBM_GBS
        unit = "GB/s"
    ctr = _counters(w.name, dom_name)
    roofline = {"bound": "mfma" if mfma else "hbm", "achieved": round(achieved, 2), "peak": peak, "unit": unit,
                "frac": round(achieved / peak, 4), "traffic": ctr.get("hbm_bytes"), "kernel": dom_name,
                "kernel_median_us": round(dom["median_us"], 2), "kernel_avg_us": round(dom["avg_us"], 2),
                "work_per_launch": dom["flops"] if mfma else dom["bytes"]}
    mdt = w.info.get("mfma_dtype")
    if mfma and mdt and mdt != w.compute_dtype:  # C5: fp8 weights on the bf16 MFMA (exact widening)
        roofline["frac_vs_" + mdt + "_peak"] = round(achieved / configs.PEAK_TFLOPS[mdt], 4)
        roofline["mfma_dtype"] = mdt
    if "mfma_busy" in ctr:
        roofline["mfma_busy"] = ctr["mfma_busy"]
    if "shader_mhz" in ctr:
        roofline["shader_mhz"] = ctr["shader_mhz"]
    if ctr:  # traffic / MFMA busy / clock are read from committed counter runs, not measured by this run
        roofline["counters_source"] = f"profiles/counters_{w.name}.json (rocprofv3 --pmc runs of bench.py, committed)"

    if w.flops:
        value, vunit = w.flops / (ms_per_step * 1e-3) / 1e12, "TFLOP/s"
    else:  # the calibration workloads are priced in bytes
        value, vunit = w.bytes / (ms_per_step * 1e-3) / 1e9, "GB/s"
    dtype = {"f32": "f32", "bf16": "bf16", "int8": "int8", "fp8": "fp8"}[mdt or w.compute_dtype]
    result = {
        "value": round(value, 2), "unit": vunit, "ms_per_step": round(ms_per_step, 4), "dtype": dtype,
        "workload": w.name, "input_shapes": {i: list(x.dims) for i, x in enumerate(w.inputs)},
        "flops_per_step": w.flops, "bytes_per_step": w.bytes, "ms_per_step_await_each": round(ms_sync, 4),
        "host_enqueue_us_per_step": round((t_enqueued - t0) / steps * 1e6, 2),
        "pcie_inclusive": {"ms_per_step": round(ms_pcie, 3),
                           "value": round((w.flops or w.bytes) / (ms_pcie * 1e-3) / (1e12 if w.flops else 1e9), 3),
                           "steps": pcie_steps,
                           "what": "host buffers uploaded, executed, outputs copied back to host memory"},
        "kernels": {k: {"median_us": round(v["median_us"], 2), "avg_us": round(v["avg_us"], 2),
                        "count_per_step": v["count"] / steps} for k, v in kernels.items()},
        "roofline": roofline,
        "cpu_baseline": None if cpu_seconds <= 0 else _cpu_baseline(name, cpu_seconds, w, gpu_outputs),
    }
    if w.info.get("baseline_config") is False or name in ("copy", "rmsnorm"):
        result["note"] = "calibration / extra workload, not a BASELINE config"
    del exe, bufs
    return result


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="all", choices=CHOICES,
                    help="all (default): every BASELINE graph plus the HBM calibrations, C5 as the headline; "
                         "or one workload, which then is the headline")
    ap.add_argument("--cpu-seconds", type=float, default=2.0,
                    help="CPU baseline: time each graph's CPU executor for at least 5 evaluations and this long")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported in this build "
              "(no multi-GPU path; see the sharding notes in DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1:
        print("--steps must be at least 1", file=sys.stderr)
        sys.exit(2)

    from ryft_amd import pjrt

    names = ALL if args.config == "all" else [args.config]
    head = HEADLINE if args.config == "all" else args.config
    plugin = pjrt.load_plugin()
    client = plugin.client({"visible_devices": [0]})
    dev = client.addressable_devices()[0]
    cpu_s = 0.0 if args.no_cpu_baseline else args.cpu_seconds
    per = {}
    for n in names:
        t = time.perf_counter()
        per[n] = measure(n, args.steps, args.warmup, cpu_s, client, dev)
        print(f"[bench] {n}: {per[n]['value']} {per[n]['unit']}, kernel {per[n]['roofline']['kernel']} "
              f"frac {per[n]['roofline']['frac']} ({time.perf_counter() - t:.1f} s)", file=sys.stderr, flush=True)

    h = per[head]
    config = {k: h[k] for k in ("workload", "input_shapes", "flops_per_step", "bytes_per_step",
                                "ms_per_step_await_each", "host_enqueue_us_per_step", "pcie_inclusive", "kernels")}
    if head == "c5":
        config["weights_dtype"] = "f8E4M3FN (widened exactly to bf16 for the bf16 MFMA)"
    line = {
        "metric": METRIC, "value": h["value"], "unit": h["unit"], "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": h["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": h["dtype"],
        "data": "synthetic (seeded splitmix64 inputs with the BASELINE.json distributions)",
        "config": config,
        "roofline": h["roofline"],
        "cpu_baseline": h["cpu_baseline"],
    }
    if len(names) > 1:
        line["per_graph"] = {n: {k: v for k, v in r.items() if k != "input_shapes"} for n, r in per.items()}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
