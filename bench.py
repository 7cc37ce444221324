"""Benchmark: one StableHLO workload through the MI355X PJRT plugin (client.compile → resident input buffers →
execute → await), reported as whole-job TFLOP/s plus the dominant kernel's roofline fraction.

A step is one execution of the config's StableHLO module on inputs already resident in HBM. Steps are enqueued
back to back (async dispatch, like a JAX-style caller) and the timed region ends when the last step's done event is
ready; the per-step latency with an await after every execute is reported alongside. Kernel durations come from
HIP events recorded on the plugin's stream around each launch (the plugin's timing extension), in a separate pass.

The cyclic garbage collector is paused during the timed region (as `timeit` does); the plugin's own work is
unchanged.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2] [--cpu-seconds 10]
"""
import argparse
import gc
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "TFLOP/s and % of MFMA/HBM roofline per StableHLO graph on 1 MI355X vs XLA CPU"


def _workload(name):
    from ryft_amd import configs
    return configs.CONFIGS[name]()


def _cpu_baseline(name, seconds):
    """The oracle (a numpy port of the StableHLO semantics, dots as f32 GEMMs the way XLA's CPU backend upcasts
    bf16) timed on a bounded sample of the same workload on this host's cores."""
    import numpy as np
    from oracle import stablehlo as sh
    from ryft_amd import configs
    from tests.helpers import MLIR_DT

    samples = {
        "c1": (configs.c1_f32_dot, {}, "full C1"),
        "c2": (configs.c2_bf16_batched_dot, {"batch": 2}, "2 of the 16 batches of C2"),
        "c3": (configs.c3_int8_gemm, {"m": 512}, "512 of the 4096 rows of C3"),
        "c4": (configs.c4_causal_attention, {"b": 1, "h": 2}, "2 of the 128 heads of C4"),
        "c5": (configs.c5_swiglu_fp8, {"m": 64}, "64 of the 512 tokens of C5"),
        "c5x": (configs.c5x_swiglu_fp8_activations, {"m": 64}, "64 of the 512 tokens of C5 (fp8 activations)"),
        "copy": (configs.hbm_copy_f32, {}, "the full copy calibration vector"),
        "rmsnorm": (configs.rmsnorm_fp8_rows, {"m": 1024}, "1024 of the 16384 rows"),
    }
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
    cores = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    if not w.flops:
        return {"value": w.bytes * reps / el / 1e9, "unit": "GB/s", "cores": cores, "kind": "port",
                "sample": f"{desc}, {reps} evaluation(s) in {el:.1f} s (numpy oracle)"}
    return {"value": w.flops * reps / el / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"{desc}, {reps} evaluation(s) in {el:.1f} s (numpy oracle, f32 dots)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5", "c5x", "copy", "rmsnorm"],
                    help="c1..c5: the BASELINE configs (c2 is the headline); copy: the HBM calibration kernel")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported in this build "
              "(no multi-GPU path; see the sharding notes in DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    from ryft_amd import configs, pjrt

    w = _workload(args.config)
    plugin = pjrt.load_plugin()
    client = plugin.client()
    dev = client.addressable_devices()[0]
    exe = client.compile(pjrt.Program.mlir(w.program))
    bufs = [client.buffer(x.data, x.type, x.dims, device=dev) for x in w.inputs]
    for b in bufs:
        b.ready_event().await_()

    def step():
        return exe.execute([bufs])[0]

    # warm-up in the timed pattern (back to back), so the allocator already caches the output blocks that
    # overlapping steps hold
    last = None
    for _ in range(args.warmup):
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
    for _ in range(args.steps):
        last = step()
    t_enqueued = time.perf_counter()
    last.done.await_()
    elapsed = time.perf_counter() - t0
    gc.enable()
    ms_per_step = elapsed / args.steps * 1e3

    # per-step latency with an await after each execute (the README's call pattern)
    t1 = time.perf_counter()
    for _ in range(args.steps):
        step().done.await_()
    ms_sync = (time.perf_counter() - t1) / args.steps * 1e3

    # PCIe-inclusive rate (not the headline): host inputs → device buffers → execute → results back to host
    pcie_steps = max(1, min(args.steps, 5))
    t2 = time.perf_counter()
    for _ in range(pcie_steps):
        hb = [client.buffer(x.data, x.type, x.dims, device=dev) for x in w.inputs]
        res = exe.execute([hb])[0]
        res.done.await_()
        for o in res.outputs:
            o.to_numpy()
    ms_pcie = (time.perf_counter() - t2) / pcie_steps * 1e3

    # kernel timing pass (HIP events on the plugin stream)
    client.set_kernel_timing(True)
    for _ in range(args.steps):
        last = step()
    last.done.await_()
    kernels = client.kernel_timing()
    client.set_kernel_timing(False)

    dom_name, dom = max(kernels.items(), key=lambda kv: kv[1]["total_ms"])
    mfma = dom["flops"] > 0
    if mfma:
        achieved = dom["flops"] / (dom["avg_us"] * 1e-6) / 1e12
        peak = configs.PEAK_TFLOPS[w.compute_dtype]
        unit = "TFLOP/s"
    else:
        achieved = dom["bytes"] / (dom["avg_us"] * 1e-6) / 1e9
        peak = configs.PEAK_HBM_GBS
        unit = "GB/s"
    traffic = None
    tf = os.path.join(ROOT, "profiles", f"traffic_{w.name}.json")
    if os.path.exists(tf):
        with open(tf) as f:
            traffic = json.load(f).get(dom_name)
    roofline = {"bound": "mfma" if mfma else "hbm", "achieved": round(achieved, 2), "peak": peak, "unit": unit,
                "frac": round(achieved / peak, 4), "traffic": traffic, "kernel": dom_name,
                "kernel_avg_us": round(dom["avg_us"], 2), "work_per_launch": dom["flops"] if mfma else dom["bytes"]}

    cpu = None if args.no_cpu_baseline else _cpu_baseline(args.config, args.cpu_seconds)
    if w.flops:
        value, vunit = w.flops / (ms_per_step * 1e-3) / 1e12, "TFLOP/s"
    else:  # the copy calibration workload is priced in bytes
        value, vunit = w.bytes / (ms_per_step * 1e-3) / 1e9, "GB/s"
    dtype = {"f32": "f32", "bf16": "bf16", "int8": "int8", "fp8": "fp8"}[w.compute_dtype]
    shapes = {x_i: list(x.dims) for x_i, x in enumerate(w.inputs)}
    line = {
        "metric": METRIC, "value": round(value, 2), "unit": vunit, "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": dtype,
        "data": "synthetic (seeded splitmix64 inputs with the BASELINE.json distributions)",
        "config": {"workload": w.name, "input_shapes": shapes, "flops_per_step": w.flops,
                   "bytes_per_step": w.bytes, "ms_per_step_await_each": round(ms_sync, 4),
                   "host_enqueue_us_per_step": round((t_enqueued - t0) / args.steps * 1e6, 2),
                   "pcie_inclusive": {"ms_per_step": round(ms_pcie, 3),
                                      "value": round((w.flops or w.bytes) / (ms_pcie * 1e-3) / (1e12 if w.flops else 1e9), 2),
                                      "steps": pcie_steps,
                                      "what": "host buffers uploaded, executed, outputs copied back to host memory"},
                   "kernels": {k: {"avg_us": round(v["avg_us"], 2), "count_per_step": v["count"] / args.steps}
                               for k, v in kernels.items()}},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
