"""scatter (crates/ryft-mlir/src/dialects/stable_hlo/operations/manipulation.rs:1614-1690) on the CPU:

  * oracle      the reference's worked example (batching dims, an out-of-range index whose window is skipped, an
                add update computation), and numpy: row replacement with repeated rows (numpy's fancy assignment:
                the last write of a repeated row wins, as in the sequential semantics), np.add.at / np.maximum.at /
                np.multiply.at for the combining bodies, and windows past the operand's end skipped whole;
  * front-ends  the generic text form and bytecode (binary and textual #stablehlo.scatter attributes, both property
                orders) plan alike; unique_indices selects the parallel kernel, otherwise the windows are applied
                in order by one workgroup;
  * checks      mismatched update shapes, wrong dimension lists, several inputs and unsupported update
                computations are refused.
GPU parity: tests/test_gpu_scatter.py."""
import numpy as np
import pytest

from oracle import stablehlo as sh
from ryft_amd import pjrt
from tests import mlir_bytecode as mb


def _t(shape, dt):
    return "tensor<" + "".join(f"{d}x" for d in shape) + dt + ">"


def scatter_program(xs, idx_shape, us, dims, body="add", dt="f32", it="i32", unique=False, sorted_=False):
    """One scatter of an operand `xs`, indices `idx_shape` and updates `us`; `dims` maps the dimension-number field
    names to lists (index_vector_dim to an int); `body` is "set" (return the update) or a binary op name."""
    X, I, U, S = _t(xs, dt), _t(idx_shape, it), _t(us, dt), f"tensor<{dt}>"
    order = ["update_window_dims", "inserted_window_dims", "input_batching_dims", "scatter_indices_batching_dims",
             "scatter_dims_to_operand_dims"]
    fields = [f"{k} = {list(dims[k])}" for k in order if dims.get(k)] + [f"index_vector_dim = {dims['index_vector_dim']}"]
    if body == "set":
        ops = f"      stablehlo.return %arg4 : {S}"
    else:
        ops = f"      %5 = stablehlo.{body} %arg3, %arg4 : {S}\n      stablehlo.return %5 : {S}"
    return f"""module {{
  func.func @main(%arg0: {X}, %arg1: {I}, %arg2: {U}) -> {X} {{
    %0 = "stablehlo.scatter"(%arg0, %arg1, %arg2) <{{indices_are_sorted = {str(sorted_).lower()}, scatter_dimension_numbers = #stablehlo.scatter<{", ".join(fields)}>, unique_indices = {str(unique).lower()}}}> ({{
    ^bb0(%arg3: {S}, %arg4: {S}):
{ops}
    }}) : ({X}, {I}, {U}) -> {X}
    return %0 : {X}
  }}
}}
"""


# rows of an [n, d] table replaced / combined at indices [k, 1] (JAX's x.at[i].set / .add on the leading dim)
ROWS = {"update_window_dims": [1], "inserted_window_dims": [0], "scatter_dims_to_operand_dims": [0],
        "index_vector_dim": 1}


def _rows_program(n, d, k, body, dt="f32", unique=False):
    return scatter_program((n, d), (k, 1), (k, d), ROWS, body=body, dt=dt, unique=unique)


def _plan(client, program):
    return client.compile(pjrt.Program.mlir(program)).describe_plan()


# ------------------------------------------------------------------------------------------------ oracle
def reference_example():
    x = np.arange(1, 49).reshape(2, 3, 4, 2)
    idx = np.array([[[[0, 0], [1, 0], [2, 1]], [[0, 1], [1, 1], [0, 9]]],
                    [[[0, 0], [2, 1], [2, 2]], [[1, 2], [0, 1], [1, 0]]]])
    upd = np.ones((2, 2, 3, 2, 2), np.int64)
    dims = {"update_window_dims": [3, 4], "inserted_window_dims": [1], "input_batching_dims": [0],
            "scatter_indices_batching_dims": [1], "scatter_dims_to_operand_dims": [2, 1], "index_vector_dim": 3}
    want = np.array([[[[3, 4], [6, 7], [6, 7], [7, 8]], [[9, 10], [11, 12], [15, 16], [17, 18]],
                      [[17, 18], [19, 20], [22, 23], [24, 25]]],
                     [[[25, 26], [28, 29], [30, 31], [31, 32]], [[35, 36], [38, 39], [38, 39], [39, 40]],
                      [[41, 42], [44, 45], [46, 47], [47, 48]]]])
    return x, idx, upd, dims, want


def test_reference_example():
    # manipulation.rs:1620-1682
    x, idx, upd, dims, want = reference_example()
    prog = scatter_program(x.shape, idx.shape, upd.shape, dims, body="add", dt="i64", it="i64")
    (r, dt), = sh.evaluate(prog, [x, idx, upd])
    assert dt == "i64" and np.array_equal(r, want)


def test_row_set_last_write_wins():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((10, 6)).astype(np.float32).astype(np.float64)
    idx = np.array([[3], [7], [3], [0], [7], [3]])
    upd = rng.standard_normal((6, 6)).astype(np.float32).astype(np.float64)
    (r, _), = sh.evaluate(_rows_program(10, 6, 6, "set"), [x, idx, upd])
    want = x.copy()
    want[idx[:, 0]] = upd  # numpy assigns repeated rows in order: the last one stays
    assert np.array_equal(r, want) and np.array_equal(r[3], upd[5]) and np.array_equal(r[7], upd[4])


@pytest.mark.parametrize("body,ufunc", [("add", np.add), ("maximum", np.maximum), ("multiply", np.multiply),
                                        ("minimum", np.minimum)])
def test_row_combines_are_numpys_at(body, ufunc):
    rng = np.random.default_rng(2)
    x = rng.integers(-50, 50, size=(12, 5))
    idx = rng.integers(0, 12, size=(40, 1))
    upd = rng.integers(-3, 4, size=(40, 5))
    (r, _), = sh.evaluate(_rows_program(12, 5, 40, body, dt="i32"), [x, idx, upd])
    want = x.copy()
    ufunc.at(want, idx[:, 0], upd)
    assert np.array_equal(r, want)


def test_windows_past_the_end_are_skipped():
    # [8, 6] operand, 2×3 windows at (row, col) starts; a window that does not fit is dropped whole
    dims = {"update_window_dims": [1, 2], "scatter_dims_to_operand_dims": [0, 1], "index_vector_dim": 1}
    x = np.zeros((8, 6), np.int64)
    starts = np.array([[0, 0], [6, 3], [7, 0], [-1, 2], [2, 4], [3, 1]])
    upd = np.arange(1, 6 * 6 + 1).reshape(6, 2, 3)
    (r, _), = sh.evaluate(scatter_program((8, 6), (6, 2), (6, 2, 3), dims, body="add", dt="i32"), [x, starts, upd])
    want = x.copy()
    for (a, b), w in zip(starts, upd):
        if 0 <= a <= 8 - 2 and 0 <= b <= 6 - 3:
            want[a:a + 2, b:b + 3] += w
    assert np.array_equal(r, want)
    assert np.count_nonzero(want) == 3 * 6  # three of the six windows landed


def test_scalar_updates_with_implicit_index_vector():
    # indices [k] with index_vector_dim = 1 = rank: each index a 1-vector; scalar windows (x.at[i].add(v) on a vector)
    dims = {"inserted_window_dims": [0], "scatter_dims_to_operand_dims": [0], "index_vector_dim": 1}
    x = np.zeros(16)
    idx = np.array([1, 5, 1, 15, 16, 5, 5])
    upd = np.array([1.0, 2.0, 3.0, 4.0, 5.0, 6.0, 7.0])
    (r, _), = sh.evaluate(scatter_program((16,), (7,), (7,), dims, body="add"), [x, idx, upd])
    want = x.copy()
    ok = idx < 16
    np.add.at(want, idx[ok], upd[ok])
    assert np.array_equal(r, want)


# ------------------------------------------------------------------------------------------------ front-ends
def test_forms_plan_alike(compile_client):
    x, idx, upd, dims, _ = reference_example()
    progs = [scatter_program(x.shape, idx.shape, upd.shape, dims, body="add", dt="i32", it="i32"),
             _rows_program(64, 128, 32, "set"), _rows_program(64, 128, 32, "maximum", unique=True)]
    for prog in progs:
        plans = [_plan(compile_client, p) for p in
                 (prog, mb.to_bytecode(prog), mb.to_bytecode(prog, stablehlo_attrs="text"),
                  mb.to_bytecode(prog, order="declared"))]
        assert len(set(plans)) == 1, plans
    plan = _plan(compile_client, progs[1]).strip().split("\n")
    assert len(plan) == 2 and "copy" in plan[0] and "scatter" in plan[1] and "serial" in plan[1], plan
    assert "windows=32 window_elems=128 kind=0" in plan[1]
    plan = _plan(compile_client, progs[2])
    assert "parallel" in plan and "kind=4" in plan, plan


def test_input_is_copied_into_the_result(compile_client):
    # an intermediate input is materialized and copied into the result, and a donated input gets a result buffer of
    # its own (neither is done in place for scatter)
    T = _t((64, 128), "f32")
    prog = _rows_program(64, 128, 8, "add").replace(
        '%0 = "stablehlo.scatter"(%arg0,', f'%9 = stablehlo.exponential %arg0 : {T}\n    %0 = "stablehlo.scatter"(%9,')
    plan = _plan(compile_client, prog).strip().split("\n")
    assert len(plan) == 3 and "elementwise" in plan[0] and "copy" in plan[1] and "scatter" in plan[2], plan
    donated = _rows_program(64, 128, 1, "set").replace("%arg0: tensor<64x128xf32>",
                                                       "%arg0: tensor<64x128xf32> {tf.aliasing_output = 0 : i32}")
    assert "(own buffer)" in _plan(compile_client, donated)


@pytest.mark.parametrize("prog,code", [
    (scatter_program((8, 6), (3, 1), (3, 7), ROWS), "INVALID_ARGUMENT"),       # window wider than the operand
    (scatter_program((8, 6), (3, 1), (4, 6), ROWS), "INVALID_ARGUMENT"),       # scatter dim ≠ the indices'
    (scatter_program((8, 6), (3, 1), (3, 6), dict(ROWS, update_window_dims=[0])), "INVALID_ARGUMENT"),
    (scatter_program((8, 6), (3, 1), (3, 6), dict(ROWS, scatter_dims_to_operand_dims=[0, 1])), "INVALID_ARGUMENT"),
    (scatter_program((8, 6), (3, 1), (3, 6), dict(ROWS, index_vector_dim=3)), "INVALID_ARGUMENT"),
    (scatter_program((8, 6), (3, 1), (3, 6), ROWS, body="subtract"), "UNIMPLEMENTED"),
    (scatter_program((8, 6), (3, 1), (3, 6), ROWS, body="add", dt="f64"), "UNIMPLEMENTED"),
    (scatter_program((8, 6), (3, 1), (3, 6), ROWS, body="and"), "UNIMPLEMENTED"),  # and of floats
])
def test_malformed(compile_client, prog, code):
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.compile(pjrt.Program.mlir(prog))
    assert e.value.code == getattr(pjrt.ErrorCode, code), e.value.message
