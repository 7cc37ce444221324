"""ctypes front of oracle/cpu_exec.cc, the C++ / OpenMP CPU executor of the BASELINE graphs and the HBM calibrations
(the timed CPU baseline of bench.py; test infrastructure like the rest of oracle/). `library(native=True)` builds it
with -march=native for the host it runs on (one build per host under oracle/_build/, remade when the source changes),
falling back to the portable x86-64-v3 build; `run(name, w)`
evaluates workload `w` (a ryft_amd.configs.Workload of config `name`) and returns its outputs as raw arrays in the
layout the plugin's buffers use."""
from __future__ import annotations

import ctypes as C
import hashlib
import os
import platform
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIBS = {}

_SIGS = {
    "cpu_exec_threads": ([], C.c_int),
    "cpu_c1": ([C.c_void_p] * 3 + [C.c_int] * 3, None),
    "cpu_c2": ([C.c_void_p] * 3 + [C.c_int] * 4, None),
    "cpu_c3": ([C.c_void_p] * 6 + [C.c_int] * 3, None),
    "cpu_c4": ([C.c_void_p] * 4 + [C.c_int] * 4 + [C.c_float], None),
    "cpu_c5": ([C.c_void_p] * 9 + [C.c_int] * 3 + [C.c_float] * 2, None),
    "cpu_copy_negate": ([C.c_void_p] * 2 + [C.c_int64], None),
    "cpu_rmsnorm_f8": ([C.c_void_p] * 3 + [C.c_int] * 2 + [C.c_float] * 2, None),
}


def _host_tag() -> str:
    model = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith(("model name", "flags")):
                    model += ln
    except OSError:
        pass
    return hashlib.sha1(model.encode()).hexdigest()[:12]


def _build(arch: str, out: str) -> bool:
    r = subprocess.run(["make", "-s", "-C", HERE, f"HOST_ARCH={arch}", f"OUT={out}"], capture_output=True, text=True)
    return r.returncode == 0 and os.path.exists(os.path.join(HERE, out))


def library(native: bool = True):
    """The loaded executor and the -march it was built for."""
    key = "native" if native else "portable"
    if key in _LIBS:
        return _LIBS[key]
    arch, rel = "x86-64-v3", os.path.join("_build", "libcpu_exec.so")
    if native:
        nrel = os.path.join("_build", f"libcpu_exec_native_{_host_tag()}.so")
        if _build("native", nrel):
            arch, rel = "native", nrel
    if arch != "native" and not _build("x86-64-v3", rel):
        raise RuntimeError("cannot build oracle/cpu_exec.cc")
    lib = C.CDLL(os.path.join(HERE, rel))
    for name, (args, res) in _SIGS.items():
        f = getattr(lib, name)
        f.argtypes, f.restype = args, res
    _LIBS[key] = (lib, arch)
    return _LIBS[key]


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def prepare(name: str, w):
    """(run, outputs): a closure evaluating `w` once into preallocated output arrays, and those arrays."""
    lib, _ = library()
    x = [np.ascontiguousarray(i.data) for i in w.inputs]
    if name == "c1":
        m, k = w.inputs[0].dims
        n = w.inputs[1].dims[1]
        out = [np.empty((m, n), np.float32)]
        return (lambda: lib.cpu_c1(_p(x[0]), _p(x[1]), _p(out[0]), m, k, n)), out
    if name == "c2":
        b, m, k = w.inputs[0].dims
        n = w.inputs[1].dims[2]
        out = [np.empty((b, m, n), np.uint16)]
        return (lambda: lib.cpu_c2(_p(x[0]), _p(x[1]), _p(out[0]), b, m, k, n)), out
    if name == "c3":
        m, k = w.inputs[0].dims
        n = w.inputs[1].dims[1]
        out = [np.empty((m, n), np.int32), np.empty((m, n), np.float32)]
        return (lambda: lib.cpu_c3(_p(x[0]), _p(x[1]), _p(x[2]), _p(x[3]), _p(out[0]), _p(out[1]), m, k, n)), out
    if name == "c4":
        b, h, s, d = w.inputs[0].dims
        if w.inputs[1].dims[2] != s or "compare" not in w.program:
            raise ValueError("the CPU executor runs the causal attention graph with equal query and key lengths")
        out = [np.empty((b, h, s, d), np.uint16)]
        scale = float(np.float32(1.0 / np.sqrt(d)))
        return (lambda: lib.cpu_c4(_p(x[0]), _p(x[1]), _p(x[2]), _p(out[0]), b, h, s, d, scale)), out
    if name == "c5":
        m, d = w.inputs[0].dims
        f = w.inputs[2].dims[1]
        out = [np.empty((m, d), np.uint16)]
        inv_d, eps = float(np.float32(1.0 / d)), float(np.float32(1e-6))
        return (lambda: lib.cpu_c5(*[_p(a) for a in x], _p(out[0]), m, d, f, inv_d, eps)), out
    if name == "copy":
        n = w.inputs[0].dims[0]
        out = [np.empty((n,), np.float32)]
        return (lambda: lib.cpu_copy_negate(_p(x[0]), _p(out[0]), n)), out
    if name == "rmsnorm":
        m, d = w.inputs[0].dims
        out = [np.empty((m, d), np.uint8)]
        inv_d, eps = float(np.float32(1.0 / d)), float(np.float32(1e-6))
        return (lambda: lib.cpu_rmsnorm_f8(_p(x[0]), _p(x[1]), _p(out[0]), m, d, inv_d, eps)), out
    raise KeyError(name)


def run(name: str, w):
    fn, out = prepare(name, w)
    fn()
    return out


def threads() -> int:
    return library()[0].cpu_exec_threads()
