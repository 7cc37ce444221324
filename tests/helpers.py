"""Helpers shared by the parity tests: run a workload through the PJRT C API, evaluate it with the oracle."""
from __future__ import annotations

import numpy as np

from oracle import stablehlo as sh
from ryft_amd import pjrt

MLIR_DT = {pjrt.BufferType.F32: "f32", pjrt.BufferType.BF16: "bf16", pjrt.BufferType.S8: "i8",
           pjrt.BufferType.S32: "i32", pjrt.BufferType.F8E4M3FN: "f8E4M3FN", pjrt.BufferType.F16: "f16",
           pjrt.BufferType.PRED: "i1", pjrt.BufferType.S64: "i64", pjrt.BufferType.U8: "ui8",
           pjrt.BufferType.S16: "i16", pjrt.BufferType.F64: "f64", pjrt.BufferType.U32: "ui32",
           pjrt.BufferType.U16: "ui16"}


def run_pjrt(client, program: str, host_inputs, executable=None):
    """client.compile → client.buffer per input → execute → done.await → copy_to_host per output (raw arrays)."""
    exe = executable or client.compile(pjrt.Program.mlir(program))
    device = exe.addressable_devices()[0]
    bufs = [client.buffer(x.data, x.type, x.dims, device=device) for x in host_inputs]
    out = exe.execute([bufs])[0]
    out.done.await_()
    return [b.to_numpy() for b in out.outputs], exe


def oracle_outputs(program: str, host_inputs, dot_precision="f64"):
    vals = [sh.from_raw(x.data, MLIR_DT[x.type]) for x in host_inputs]
    return sh.evaluate(program, vals, dot_precision=dot_precision)


def check(got_raw, want, tol: float, name: str = ""):
    """Compare one plugin output (raw PJRT bits) with an oracle result: bit-exact for integers, normwise relative
    error <= tol for floats. Returns the error."""
    vals, dt = want
    got = sh.from_raw(got_raw, dt)
    assert got.shape == vals.shape, f"{name}: shape {got.shape} != {vals.shape}"
    if dt in sh.FLOAT:
        assert np.all(np.isfinite(got)) == np.all(np.isfinite(vals)), f"{name}: non-finite mismatch"
        err = sh.rel_error(got, vals)
        assert err <= tol, f"{name}: relative error {err:.3e} > {tol:.1e}"
        return err
    mism = np.count_nonzero(got != vals)
    assert mism == 0, f"{name}: {mism} integer mismatches"
    return 0.0
