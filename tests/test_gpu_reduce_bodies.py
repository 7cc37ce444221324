"""reduce with several inputs and general bodies on the GPU (functional.rs:109-230), against the oracle: argmax /
argmin in JAX's comparator form over the innermost, middle and outermost dims, rows short (a wavefront per output)
and long (a workgroup per output, vocabulary-sized), more outputs than the grid has workgroups, f32 / bf16 / i32
values with ties and NaN; two inputs with independent bodies; one-input bodies outside the fast set; init values
that are device scalars; an empty reduced dimension. Indices and selected values bit-exact; sums to a tolerance
(the fold order differs from the oracle's)."""
import numpy as np
import pytest

from ryft_amd import configs, hostdata as hd, pjrt
from tests.helpers import check, oracle_outputs, run_pjrt
from tests.test_reduce_bodies import argmax_program, one_input_program, sum_max_program

pytestmark = pytest.mark.gpu

_BT = {"f32": pjrt.BufferType.F32, "bf16": pjrt.BufferType.BF16, "i32": pjrt.BufferType.S32}


def _values(seed, shape, dim, dt, nan=False):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(shape).astype(np.float32)
    moved = np.moveaxis(x, dim, -1)
    flat = moved.reshape(-1, shape[dim])
    n = shape[dim]
    for r in range(0, flat.shape[0], 3):  # equal extremes: the lower index must win
        flat[r, [n // 3, n - 1]] = 9.0
        flat[r, [0, n // 2]] = -9.0
    if nan:
        flat[1::5, n // 4] = np.nan
    x = np.moveaxis(flat.reshape(moved.shape), -1, dim).copy()
    if dt == "bf16":
        return configs.HostInput(hd.f32_to_bf16_bits(x), pjrt.BufferType.BF16, shape)
    if dt == "i32":
        return configs.HostInput(np.nan_to_num(x * 100).astype(np.int32), pjrt.BufferType.S32, shape)
    return configs.HostInput(x, pjrt.BufferType.F32, shape)


def _exact(client, prog, ins, name):
    print(f"[reduce] {name}", flush=True)
    outs, exe = run_pjrt(client, prog, ins)
    for o, w in zip(outs, oracle_outputs(prog, ins)):
        vals, dt = w
        if dt in ("f32", "bf16"):
            from oracle import stablehlo as sh
            got = sh.from_raw(o, dt)
            assert np.array_equal(np.isnan(got), np.isnan(vals)), name
            ok = ~np.isnan(vals)
            assert np.array_equal(got[ok], vals[ok]), name
        else:
            check(o, w, 0, name)
    return exe


@pytest.mark.parametrize("kind", ["argmax", "argmin"])
@pytest.mark.parametrize("dt", ["f32", "bf16", "i32"])
@pytest.mark.parametrize("shape,dim", [((8, 1000), 1), ((8, 32000), 1), ((2, 100000), 1), ((4100, 40), 1),
                                       ((300, 7, 3), 0), ((5, 129, 6), 1)])
def test_argmax_argmin(gpu_client, kind, dt, shape, dim):
    """The argmax / argmin rule (one wavefront or workgroup per row, or segments folded by a second launch for long
    rows of few outputs), against the oracle's fold of the body in index order."""
    prog = argmax_program(shape, dim, dt=dt, kind=kind)
    _exact(gpu_client, prog, [_values(11, shape, dim, dt, nan=dt != "i32")], f"{kind} {dt} {shape} dim {dim}")


def test_argmax_i64_positions_and_several_nans(gpu_client):
    # i64 positions; rows with several NaNs (the first one wins, as in a fold in index order)
    shape = (40, 6000)
    x = _values(17, shape, 1, "f32")
    x.data[3, [10, 20, 4000]] = np.nan
    x.data[7, [5999, 1]] = np.nan
    for kind in ("argmax", "argmin"):
        _exact(gpu_client, argmax_program(shape, 1, it="i64", kind=kind), [x], f"{kind} i64 positions")


def test_body_program_in_segments(gpu_client):
    # a body the rule does not cover (xor) over long rows of few outputs: segments folded by a second launch
    shape = (3, 50000)
    x = np.random.default_rng(18).integers(-2 ** 31, 2 ** 31, size=shape).astype(np.int32)
    prog = one_input_program(shape, 1, "xor", "i32")
    assert "segments=" in gpu_client.compile(pjrt.Program.mlir(prog)).describe_plan()
    _exact(gpu_client, prog, [configs.HostInput(x, pjrt.BufferType.S32, shape)], "xor in segments")


def test_argmax_generic_form_and_bytecode(gpu_client):
    from tests import mlir_bytecode as mb
    shape = (16, 2048)
    ins = [_values(12, shape, 1, "f32", nan=True)]
    for form in ("generic",):
        _exact(gpu_client, argmax_program(shape, 1, form=form), ins, f"argmax {form}")
    prog = argmax_program(shape, 1)
    print("[reduce] argmax bytecode", flush=True)
    outs, _ = run_pjrt(gpu_client, mb.to_bytecode(prog), ins)
    want = oracle_outputs(prog, ins)
    check(outs[1], want[1], 0, "argmax bytecode indices")


@pytest.mark.parametrize("shape,dims", [((64, 3000), [1]), ((6, 50, 40), [0, 2]), ((2000, 16), [1])])
def test_two_inputs_independent_bodies(gpu_client, shape, dims):
    prog = sum_max_program(shape, dims)
    ins = [_values(13, shape, dims[-1], "f32"), _values(14, shape, dims[-1], "f32")]
    print(f"[reduce] sum+max {shape} {dims}", flush=True)
    outs, _ = run_pjrt(gpu_client, prog, ins)
    want = oracle_outputs(prog, ins)
    check(outs[0], want[0], 1e-5, "sum")
    check(outs[1], want[1], 0, "max")


@pytest.mark.parametrize("body,dt", [("select_max", "f32"), ("xor", "i32")])
@pytest.mark.parametrize("shape,dim", [((32, 5000), 1), ((1000, 33), 1), ((17, 9, 11), 1)])
def test_one_input_general_bodies(gpu_client, body, dt, shape, dim):
    prog = one_input_program(shape, dim, body, dt)
    if dt == "i32":
        x = np.random.default_rng(15).integers(-2 ** 31, 2 ** 31, size=shape).astype(np.int32)
        ins = [configs.HostInput(x, pjrt.BufferType.S32, shape)]
    else:
        ins = [_values(15, shape, dim, dt)]
    _exact(gpu_client, prog, ins, f"{body} {shape}")


def test_device_scalar_inits_and_empty_rows(gpu_client):
    # init values passed as arguments (read on the device), and a reduced dimension of extent 0 (results = inits)
    prog = argmax_program((6, 77), 1).replace("%cst = stablehlo.constant dense<0xFF800000> : tensor<f32>", "") \
        .replace("%c = stablehlo.constant dense<0> : tensor<i32>", "") \
        .replace("%arg0 init: %cst", "%arg0 init: %arg1").replace("(%0 init: %c)", "(%0 init: %arg2)") \
        .replace("func.func @main(%arg0: tensor<6x77xf32>)",
                 "func.func @main(%arg0: tensor<6x77xf32>, %arg1: tensor<f32>, %arg2: tensor<i32>)")
    ins = [_values(16, (6, 77), 1, "f32"), configs.HostInput(np.array(5.0, np.float32), pjrt.BufferType.F32, ()),
           configs.HostInput(np.array(-1, np.int32), pjrt.BufferType.S32, ())]
    _exact(gpu_client, prog, ins, "device scalar inits")
    empty = argmax_program((4, 0), 1)
    outs, _ = run_pjrt(gpu_client, empty, [configs.HostInput(np.zeros((4, 0), np.float32), pjrt.BufferType.F32, (4, 0))])
    assert np.all(np.isneginf(outs[0])) and outs[1].tolist() == [0, 0, 0, 0]
