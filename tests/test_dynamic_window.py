"""dynamic_slice / dynamic_update_slice and gather on the CPU: the oracle pinned to the reference's worked examples
(crates/ryft-mlir/src/dialects/stable_hlo/operations/manipulation.rs:955-976, 1045-1071, 1240-1300), to the
clamping formula by brute force and to numpy's indexing for gather's special cases (row lookup, take_along_axis), and
the plugin's front-ends and planner — the printed forms of the reference's builder tests (manipulation.rs:2447-2580,
2690-2710) compile, text and bytecode plan alike, malformed windows and gathers are rejected, and a donated operand
is updated in place."""
import itertools

import numpy as np
import pytest

from oracle import stablehlo as sh
from ryft_amd import pjrt
from tests import mlir_bytecode as mb


def _mod(args, ret, body):
    sig = ", ".join(f"%arg{i}: {t}" for i, t in enumerate(args))
    return f"module {{\n  func.func @main({sig}) -> {ret} {{\n{body}\n  }}\n}}\n"


def ds_program(shape, sizes, dt="i32", it="i64"):
    t = "tensor<" + "".join(f"{d}x" for d in shape) + dt + ">"
    o = "tensor<" + "".join(f"{d}x" for d in sizes) + dt + ">"
    idx = [f"tensor<{it}>"] * len(shape)
    args = ", ".join(f"%arg{i + 1}" for i in range(len(shape)))
    sizes_s = ", ".join(map(str, sizes))
    return _mod([t] + idx, o, f"    %0 = stablehlo.dynamic_slice %arg0, {args}, sizes = [{sizes_s}] : "
                              f"({', '.join([t] + idx)}) -> {o}\n    return %0 : {o}")


def dus_program(shape, ushape, dt="i32", it="i64", donate=False):
    t = "tensor<" + "".join(f"{d}x" for d in shape) + dt + ">"
    u = "tensor<" + "".join(f"{d}x" for d in ushape) + dt + ">"
    idx = [f"tensor<{it}>"] * len(shape)
    args = ", ".join(f"%arg{i + 2}" for i in range(len(shape)))
    prog = _mod([t, u] + idx, t, f"    %0 = stablehlo.dynamic_update_slice %arg0, %arg1, {args} : "
                                 f"({', '.join([t, u] + idx)}) -> {t}\n    return %0 : {t}")
    if donate:
        prog = prog.replace(f"%arg0: {t}", f"%arg0: {t} {{tf.aliasing_output = 0 : i32}}", 1)
    return prog


def test_reference_examples():
    # manipulation.rs:955-976: starts (-1, 3) clamp to (0, 2)
    x = np.array([[0, 0, 1, 1], [0, 0, 1, 1], [0, 0, 0, 0], [0, 0, 0, 0]])
    (out, _), = sh.evaluate(ds_program((4, 4), (2, 2)), [x, np.array(-1), np.array(3)])
    assert out.tolist() == [[1, 1], [1, 1]]
    # manipulation.rs:1045-1071: the update lands at the clamped start (0, 2)
    x = np.array([[1, 1, 0, 0], [1, 1, 0, 0], [1, 1, 1, 1], [1, 1, 1, 1]])
    (out, _), = sh.evaluate(dus_program((4, 4), (2, 2)), [x, np.array([[1, 1], [1, 1]]), np.array(-1), np.array(3)])
    assert out.tolist() == [[1] * 4] * 4


@pytest.mark.parametrize("it", ["i8", "i32", "i64", "ui8", "ui32"])
def test_clamping_matches_the_index_formula(it):
    # result[i] = operand[clamp(0, start, shape - sizes) + i] (manipulation.rs:950-953), element by element, for
    # starts below zero, inside and past the end; update: the window elements take the update's values, the rest the
    # operand's
    shape, sizes = (5, 3, 6), (2, 3, 4)
    x = np.arange(np.prod(shape)).reshape(shape)
    u = -1 - np.arange(np.prod(sizes)).reshape(sizes)
    unsigned = it.startswith("ui")
    cand = [0, 1, 2, 5, 9, 200] if unsigned else [-7, -1, 0, 1, 2, 9, 100]
    for starts in itertools.islice(itertools.product(cand, repeat=3), 0, None, 7):
        clamped = [min(max(s, 0), n - k) for s, n, k in zip(starts, shape, sizes)]
        idx = [np.array(s) for s in starts]
        (got, _), = sh.evaluate(ds_program(shape, sizes, it=it), [x] + idx)
        want = np.empty(sizes, dtype=x.dtype)
        for i in np.ndindex(*sizes):
            want[i] = x[tuple(c + k for c, k in zip(clamped, i))]
        assert np.array_equal(got, want), starts
        (got, _), = sh.evaluate(dus_program(shape, sizes, it=it), [x, u] + idx)
        want = x.copy()
        for i in np.ndindex(*sizes):
            want[tuple(c + k for c, k in zip(clamped, i))] = u[i]
        assert np.array_equal(got, want), starts


# the printed forms of the reference's builder tests (manipulation.rs:2497-2507, 2566-2579; entry renamed @main)
PRINTED = {
    "dynamic_slice": """module {
  func.func @main(%arg0: tensor<3x4x5xi32>, %arg1: tensor<i64>, %arg2: tensor<i64>, %arg3: tensor<i64>) -> tensor<1x2x3xi32> {
    %0 = stablehlo.dynamic_slice %arg0, %arg1, %arg2, %arg3, sizes = [1, 2, 3] : (tensor<3x4x5xi32>, tensor<i64>, tensor<i64>, tensor<i64>) -> tensor<1x2x3xi32>
    return %0 : tensor<1x2x3xi32>
  }
}""",
    "dynamic_update_slice": """module {
  func.func @main(%arg0: tensor<3x4x5xi32>, %arg1: tensor<1x2x3xi32>, %arg2: tensor<i64>, %arg3: tensor<i64>, %arg4: tensor<i64>) -> tensor<3x4x5xi32> {
    %0 = stablehlo.dynamic_update_slice %arg0, %arg1, %arg2, %arg3, %arg4 : (tensor<3x4x5xi32>, tensor<1x2x3xi32>, tensor<i64>, tensor<i64>, tensor<i64>) -> tensor<3x4x5xi32>
    return %0 : tensor<3x4x5xi32>
  }
}""",
}

GENERIC = {
    "dynamic_slice": """module {
  func.func @main(%arg0: tensor<3x4x5xi32>, %arg1: tensor<i64>, %arg2: tensor<i64>, %arg3: tensor<i64>) -> tensor<1x2x3xi32> {
    %0 = "stablehlo.dynamic_slice"(%arg0, %arg1, %arg2, %arg3) <{slice_sizes = array<i64: 1, 2, 3>}> : (tensor<3x4x5xi32>, tensor<i64>, tensor<i64>, tensor<i64>) -> tensor<1x2x3xi32>
    return %0 : tensor<1x2x3xi32>
  }
}""",
    "dynamic_update_slice": """module {
  func.func @main(%arg0: tensor<3x4x5xi32>, %arg1: tensor<1x2x3xi32>, %arg2: tensor<i64>, %arg3: tensor<i64>, %arg4: tensor<i64>) -> tensor<3x4x5xi32> {
    %0 = "stablehlo.dynamic_update_slice"(%arg0, %arg1, %arg2, %arg3, %arg4) : (tensor<3x4x5xi32>, tensor<1x2x3xi32>, tensor<i64>, tensor<i64>, tensor<i64>) -> tensor<3x4x5xi32>
    return %0 : tensor<3x4x5xi32>
  }
}""",
}


def _plan(client, program):
    exe = client.compile(pjrt.Program.mlir(program))
    return exe, exe.describe_plan()


@pytest.mark.parametrize("name", ["dynamic_slice", "dynamic_update_slice"])
def test_printed_generic_and_bytecode_forms_plan_alike(compile_client, name):
    _, text = _plan(compile_client, PRINTED[name])
    _, generic = _plan(compile_client, GENERIC[name])
    _, code = _plan(compile_client, mb.to_bytecode(PRINTED[name]))
    assert name in text and text == generic == code
    if name == "dynamic_update_slice":  # the operand is copied into the result, then the window is written
        assert text.split("\n")[0].split()[1] == "copy"


@pytest.mark.parametrize("bad", [
    # a start index missing, a start index that is not a scalar, mixed index types, a float index
    ("tensor<4x4xi32>", ["tensor<i64>"], "sizes = [2, 2]", "tensor<2x2xi32>"),
    ("tensor<4x4xi32>", ["tensor<i64>", "tensor<1xi64>"], "sizes = [2, 2]", "tensor<2x2xi32>"),
    ("tensor<4x4xi32>", ["tensor<i64>", "tensor<i32>"], "sizes = [2, 2]", "tensor<2x2xi32>"),
    ("tensor<4x4xi32>", ["tensor<f32>", "tensor<f32>"], "sizes = [2, 2]", "tensor<2x2xi32>"),
    # a window larger than the operand, a result that is not the window
    ("tensor<4x4xi32>", ["tensor<i64>", "tensor<i64>"], "sizes = [5, 2]", "tensor<5x2xi32>"),
    ("tensor<4x4xi32>", ["tensor<i64>", "tensor<i64>"], "sizes = [2, 2]", "tensor<2x3xi32>"),
])
def test_malformed_dynamic_slices_are_invalid(compile_client, bad):
    t, idx, sizes, out = bad
    args = ", ".join(f"%arg{i + 1}" for i in range(len(idx)))
    prog = _mod([t] + idx, out, f"    %0 = stablehlo.dynamic_slice %arg0, {args}, {sizes} : "
                                f"({', '.join([t] + idx)}) -> {out}\n    return %0 : {out}")
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.compile(pjrt.Program.mlir(prog))
    assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT, e.value.message


def test_malformed_dynamic_update_slices_are_invalid(compile_client):
    for shape, ushape, ut in [((4, 4), (5, 1), "i32"), ((4, 4), (2, 2), "f32"), ((4, 4), (2,), "i32")]:
        t = "tensor<" + "".join(f"{d}x" for d in shape) + "i32>"
        u = "tensor<" + "".join(f"{d}x" for d in ushape) + ut + ">"
        prog = _mod([t, u, "tensor<i32>", "tensor<i32>"], t,
                    f"    %0 = stablehlo.dynamic_update_slice %arg0, %arg1, %arg2, %arg3 : "
                    f"({t}, {u}, tensor<i32>, tensor<i32>) -> {t}\n    return %0 : {t}")
        with pytest.raises(pjrt.PjrtError) as e:
            compile_client.compile(pjrt.Program.mlir(prog))
        assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT, (shape, ushape, ut, e.value.message)


def test_donated_operand_is_updated_in_place(compile_client):
    # a KV-cache style update: only the window is written into the donated buffer (the copy into the result is a
    # no-op at execute time)
    _, plan = _plan(compile_client, dus_program((2, 8, 256, 64), (2, 8, 1, 64), dt="bf16", it="i32", donate=True))
    assert "alias: result 0 <- parameter 0 (in place)" in plan
    assert "dynamic_update_slice" in plan


def test_operand_read_elsewhere_keeps_its_own_buffer(compile_client):
    # the operand is also a result: it is computed into a slot of its own and copied, so the window write cannot
    # change the other result
    t, u = "tensor<8x8xf32>", "tensor<2x8xf32>"
    prog = _mod([t, u, "tensor<i32>", "tensor<i32>"], f"({t}, {t})", f"""    %0 = stablehlo.negate %arg0 : {t}
    %1 = stablehlo.dynamic_update_slice %0, %arg1, %arg2, %arg3 : ({t}, {u}, tensor<i32>, tensor<i32>) -> {t}
    return %0, %1 : {t}, {t}""")
    _, plan = _plan(compile_client, prog)
    lines = [ln.split()[1] for ln in plan.strip().splitlines()]
    assert lines == ["elementwise", "copy", "dynamic_update_slice"], lines


# ------------------------------------------------------------------------------------------------ gather
def gather_program(x_t, i_t, out_t, offset_dims, collapsed, start_map, ivd, sizes, op_batch=(), idx_batch=()):
    fields = [f"offset_dims = {list(offset_dims)}", f"collapsed_slice_dims = {list(collapsed)}"]
    if op_batch:
        fields += [f"operand_batching_dims = {list(op_batch)}", f"start_indices_batching_dims = {list(idx_batch)}"]
    fields += [f"start_index_map = {list(start_map)}", f"index_vector_dim = {ivd}"]
    sz = ", ".join(map(str, sizes))
    return _mod([x_t, i_t], out_t, f'    %0 = "stablehlo.gather"(%arg0, %arg1) <{{dimension_numbers = '
                                   f'#stablehlo.gather<{", ".join(fields)}>, indices_are_sorted = false, '
                                   f'slice_sizes = array<i64: {sz}>}}> : ({x_t}, {i_t}) -> {out_t}\n'
                                   f'    return %0 : {out_t}')


# manipulation.rs:1240-1300: batching dims, a collapsed dim, an index vector of two, and one out-of-range start
# ([0, 9] clamps to [0, 2]) — the documented result
GATHER_EXAMPLE = dict(
    x=np.arange(1, 49).reshape(2, 3, 4, 2),
    idx=np.array([[[[0, 0], [1, 0], [2, 1]], [[0, 1], [1, 1], [0, 9]]],
                  [[[0, 0], [2, 1], [2, 2]], [[1, 2], [0, 1], [1, 0]]]]),
    want=[[[[[1, 2], [3, 4]], [[3, 4], [5, 6]], [[13, 14], [15, 16]]],
           [[[33, 34], [35, 36]], [[35, 36], [37, 38]], [[41, 42], [43, 44]]]],
          [[[[1, 2], [3, 4]], [[13, 14], [15, 16]], [[21, 22], [23, 24]]],
           [[[43, 44], [45, 46]], [[33, 34], [35, 36]], [[27, 28], [29, 30]]]]])


def gather_example_program():
    return gather_program("tensor<2x3x4x2xi32>", "tensor<2x2x3x2xi64>", "tensor<2x2x3x2x2xi32>", [3, 4], [1], [2, 1],
                          3, [1, 1, 2, 2], op_batch=[0], idx_batch=[1])


def test_gather_reference_example():
    (out, _), = sh.evaluate(gather_example_program(), [GATHER_EXAMPLE["x"], GATHER_EXAMPLE["idx"]])
    assert out.tolist() == GATHER_EXAMPLE["want"]


def test_gather_embedding_lookup_and_take_along_axis():
    # two textbook special cases, against numpy: rows of a table by index (clamped at the end), and a gather of one
    # element per row along the last axis (index vector dim = rank of the indices: an implicit trailing 1)
    table = np.arange(50).reshape(10, 5)
    ids = np.array([3, 0, 9, 12, -2])
    prog = gather_program("tensor<10x5xi32>", "tensor<5xi32>", "tensor<5x5xi32>", [1], [0], [0], 1, [1, 5])
    (out, _), = sh.evaluate(prog, [table, ids])
    assert np.array_equal(out, table[np.clip(ids, 0, 9)])
    x = np.arange(24).reshape(4, 6)
    cols = np.array([[5], [0], [2], [3]])
    prog = gather_program("tensor<4x6xi32>", "tensor<4x1xi32>", "tensor<4xi32>", [], [1], [1], 1, [1, 1],
                          op_batch=[0], idx_batch=[0])
    (out, _), = sh.evaluate(prog, [x, cols])
    assert np.array_equal(out, np.take_along_axis(x, cols, axis=1)[:, 0])


GATHER_PRINTED = """module {
  func.func @main(%arg0: tensor<3x4x2xi64>, %arg1: tensor<2x3x2xi64>) -> tensor<2x3x2x2xi64> {
    %0 = "stablehlo.gather"(%arg0, %arg1) <{dimension_numbers = #stablehlo.gather<offset_dims = [2, 3], collapsed_slice_dims = [0], start_index_map = [1, 0], index_vector_dim = 2>, indices_are_sorted = false, slice_sizes = array<i64: 1, 2, 2>}> : (tensor<3x4x2xi64>, tensor<2x3x2xi64>) -> tensor<2x3x2x2xi64>
    return %0 : tensor<2x3x2x2xi64>
  }
}"""


def test_gather_plans(compile_client):
    # the printed form of the reference's builder test (manipulation.rs:2690-2710), the documented example, a row
    # lookup and a take_along_axis (collapsed and batching dims kept apart, as StableHLO requires)
    rows = gather_program("tensor<10x5xi32>", "tensor<5xi32>", "tensor<5x5xi32>", [1], [0], [0], 1, [1, 5])
    along = gather_program("tensor<4x6xi32>", "tensor<4x1xi32>", "tensor<4xi32>", [], [1], [1], 1, [1, 1],
                           op_batch=[0], idx_batch=[0])
    for prog in (GATHER_PRINTED, gather_example_program(), rows, along):
        _, plan = _plan(compile_client, prog)
        assert plan.split("\n")[0].split()[1] == "gather", plan


@pytest.mark.parametrize("bad", [
    dict(ivd=3),                                  # index vector dim past the indices' rank
    dict(start_map=[0]),                          # one start index map entry for index vectors of two
    dict(sizes=[1, 4, 2]),                        # a slice larger than the operand
    dict(collapsed=[1]),                          # a collapsed dim whose slice is 2
    dict(offset_dims=[3, 2]),                     # offset dims not sorted
    dict(op_batch=[0], idx_batch=[0]),           # dim 0 both collapsed and a batching dim
    dict(out_t="tensor<2x3x2x3xi64>"),            # result not the gathered shape
])
def test_malformed_gathers_are_invalid(compile_client, bad):
    kw = dict(x_t="tensor<3x4x2xi64>", i_t="tensor<2x3x2xi64>", out_t="tensor<2x3x2x2xi64>", offset_dims=[2, 3],
              collapsed=[0], start_map=[1, 0], ivd=2, sizes=[1, 2, 2])
    kw.update(bad)
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.compile(pjrt.Program.mlir(gather_program(**kw)))
    assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT, e.value.message


def test_gather_bytecode_plans_like_text(compile_client):
    # every writer variant (dialect-encoded or assembly-text dimension numbers, sorted or declared property order)
    from tests.test_bytecode import VARIANTS
    for prog in (GATHER_PRINTED, gather_example_program()):
        _, text = _plan(compile_client, prog)
        for vname, opts in VARIANTS.items():
            _, code = _plan(compile_client, mb.to_bytecode(prog, **opts))
            assert code == text, vname
