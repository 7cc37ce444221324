"""reverse, optimization_barrier, map and same-width bitcast_convert (crates/ryft-mlir/src/dialects/stable_hlo/
operations/miscellaneous.rs:309-450, functional.rs:13-104, casting.rs:8-73), on the CPU:

  * oracle      the reference's worked examples (reverse [[1, 2], [3, 4], [5, 6]] along dim 1, map's multiply of
                [[0, 1], [2, 3]] and [[4, 5], [6, 7]], optimization_barrier's identity), numpy's flip for more
                reversals, and bitcast_convert against numpy's views of the same bytes;
  * front-ends  printed, generic and bytecode forms plan alike (map as its generic form: it has no printed one);
                reverse is a backwards read (one elementwise step, no copy), optimization_barrier and map leave no
                step of their own;
  * checks      repeated or out-of-range reverse dims, map dimensions other than 0..rank-1, a map body of the wrong
                arity and a bitcast_convert that changes the element width are refused.
GPU parity: tests/test_gpu_misc_ops.py."""
import numpy as np
import pytest

from oracle import stablehlo as sh
from ryft_amd import pjrt
from tests import mlir_bytecode as mb


def _t(shape, dt):
    return "tensor<" + "".join(f"{d}x" for d in shape) + dt + ">"


def reverse_program(shape, dims, dt="i32", consumer=False):
    T = _t(shape, dt)
    ds = ", ".join(map(str, dims))
    extra = f"\n    %1 = stablehlo.add %0, %arg0 : {T}" if consumer else ""
    ret = "%1" if consumer else "%0"
    return f"""module {{
  func.func @main(%arg0: {T}) -> {T} {{
    %0 = stablehlo.reverse %arg0, dims = [{ds}] : {T}{extra}
    return {ret} : {T}
  }}
}}
"""


def map_program(shape, dt="i32"):
    """The reference's example body (multiply), plus a compare / select and a constant to inline."""
    T, S = _t(shape, dt), f"tensor<{dt}>"
    P = _t(shape, "i1")
    return f"""module {{
  func.func @main(%arg0: {T}, %arg1: {T}) -> ({T}, {T}) {{
    %0 = "stablehlo.map"(%arg0, %arg1) <{{dimensions = array<i64: {", ".join(str(d) for d in range(len(shape)))}>}}> ({{
    ^bb0(%arg2: {S}, %arg3: {S}):
      %1 = stablehlo.multiply %arg2, %arg3 : {S}
      stablehlo.return %1 : {S}
    }}) : ({T}, {T}) -> {T}
    %2 = "stablehlo.map"(%arg0, %arg1) <{{dimensions = array<i64: {", ".join(str(d) for d in range(len(shape)))}>}}> ({{
    ^bb0(%a: {S}, %b: {S}):
      %c = stablehlo.constant dense<3> : {S}
      %d = stablehlo.add %a, %c : {S}
      %e = stablehlo.compare  GT, %d, %b : ({S}, {S}) -> tensor<i1>
      %f = stablehlo.select %e, %d, %b : tensor<i1>, {S}
      stablehlo.return %f : {S}
    }}) : ({T}, {T}) -> {T}
    return %0, %2 : {T}, {T}
  }}
}}
"""


def barrier_program(shape):
    T = _t(shape, "f32")
    return f"""module {{
  func.func @main(%arg0: {T}, %arg1: {T}) -> ({T}, {T}) {{
    %0:2 = stablehlo.optimization_barrier %arg0, %arg1 : {T}, {T}
    %1 = stablehlo.multiply %0#0, %0#1 : {T}
    return %1, %0#1 : {T}, {T}
  }}
}}
"""


def bitcast_program(shape, src, dst, generic=False):
    A, B = _t(shape, src), _t(shape, dst)
    op = (f'%0 = "stablehlo.bitcast_convert"(%arg0) : ({A}) -> {B}' if generic
          else f"%0 = stablehlo.bitcast_convert %arg0 : ({A}) -> {B}")
    return f"""module {{
  func.func @main(%arg0: {A}) -> {B} {{
    {op}
    return %0 : {B}
  }}
}}
"""


def _plan(client, program):
    return client.compile(pjrt.Program.mlir(program)).describe_plan()


# ------------------------------------------------------------------------------------------------ oracle
def test_reference_examples():
    # miscellaneous.rs:320-327
    (r, _), = sh.evaluate(reverse_program((3, 2), [1]), [np.array([[1, 2], [3, 4], [5, 6]])])
    assert r.tolist() == [[2, 1], [4, 3], [6, 5]]
    # functional.rs:29-37 (documented for i64: the same values in i32)
    (m, _), (s, _) = sh.evaluate(map_program((2, 2)), [np.array([[0, 1], [2, 3]]), np.array([[4, 5], [6, 7]])])
    assert m.tolist() == [[0, 5], [12, 21]]
    assert s.tolist() == [[4, 5], [6, 7]]  # max(a + 3, b)
    # miscellaneous.rs:418-424: the identity
    a, b = np.array([1.0]), np.array([2.0])
    (p, _), (q, _) = sh.evaluate(barrier_program((1,)), [a, b])
    assert p.tolist() == [2.0] and q.tolist() == [2.0]


@pytest.mark.parametrize("shape,dims", [((4, 5, 6), [0, 2]), ((7,), [0]), ((3, 4), []), ((2, 3, 4, 5), [1, 2, 3])])
def test_reverse_is_numpys_flip(shape, dims):
    x = np.arange(np.prod(shape)).reshape(shape)
    (r, _), = sh.evaluate(reverse_program(shape, dims), [x])
    assert np.array_equal(r, np.flip(x, axis=tuple(dims)))


@pytest.mark.parametrize("src,dst,npsrc,npdst", [("f32", "i32", np.float32, np.int32), ("i32", "f32", np.int32, np.float32),
                                                 ("ui32", "i32", np.uint32, np.int32), ("i16", "ui16", np.int16, np.uint16),
                                                 ("i8", "ui8", np.int8, np.uint8)])
def test_bitcast_is_numpys_view(src, dst, npsrc, npdst):
    rng = np.random.default_rng(3)
    if npsrc == np.float32:
        x = rng.standard_normal(64).astype(np.float32)
    else:
        info = np.iinfo(npsrc)
        x = rng.integers(info.min, info.max, size=64, endpoint=True).astype(npsrc)
        if npdst == np.float32:  # bit patterns of finite floats (NaN payloads are not carried by the oracle's values)
            x = np.where(np.isfinite(x.view(np.float32)), x, 0).astype(npsrc)
    (r, dt), = sh.evaluate(bitcast_program((64,), src, dst), [x.astype(np.float64 if npsrc == np.float32 else np.int64)])
    want = x.view(npdst)
    assert dt == dst and np.array_equal(np.asarray(r), want.astype(np.float64 if npdst == np.float32 else np.int64))


def test_bitcast_of_narrow_floats_round_trips():
    # bf16 / f16 / f8 bits through an integer of the same width and back
    x = np.array([1.0, -2.5, 0.15625, 3.0e4, -0.0])
    for ft, it in (("bf16", "i16"), ("f16", "ui16"), ("f8E4M3FN", "ui8")):
        xs = sh.normalize(x, ft)
        (bits, _), = sh.evaluate(bitcast_program((5,), ft, it), [xs])
        (back, _), = sh.evaluate(bitcast_program((5,), it, ft), [bits])
        assert np.array_equal(np.asarray(back), xs, equal_nan=True) and np.array_equal(np.signbit(back), np.signbit(xs))
        raw = sh.to_raw(xs, ft)
        assert np.array_equal(np.asarray(bits).astype(np.int64) & (0xFFFF if it.endswith("16") else 0xFF),
                              raw.astype(np.int64))


# ------------------------------------------------------------------------------------------------ front-ends
def test_forms_plan_alike(compile_client):
    for prog in (reverse_program((8, 64), [1], consumer=True), barrier_program((8, 64)),
                 bitcast_program((8, 64), "f32", "i32")):
        generic = prog.replace("stablehlo.reverse %arg0, dims = [1] : tensor<8x64xi32>",
                               '"stablehlo.reverse"(%arg0) <{dimensions = array<i64: 1>}> : (tensor<8x64xi32>) -> '
                               'tensor<8x64xi32>')
        plans = [_plan(compile_client, p) for p in (prog, generic, mb.to_bytecode(prog))]
        assert plans[0] == plans[1] == plans[2], plans
    # a reverse feeding an add is one elementwise step reading backwards; the barrier adds no step of its own (its
    # second result is the parameter itself, returned by a copy)
    plan = _plan(compile_client, reverse_program((8, 64), [1], consumer=True)).strip().split("\n")
    assert len(plan) == 1 and plan[0].startswith("0: elementwise") and "leaves=2" in plan[0], plan
    plan = _plan(compile_client, barrier_program((8, 64))).strip().split("\n")
    assert len(plan) == 2 and "elementwise" in plan[0] and "copy" in plan[1], plan
    # each map's body inlined into one elementwise step over the inputs
    plan = _plan(compile_client, map_program((8, 64))).strip().split("\n")
    assert len(plan) == 2 and all("elementwise" in ln and "leaves=2" in ln for ln in plan), plan


@pytest.mark.parametrize("prog,code", [
    (reverse_program((4, 5), [1, 1]), "INVALID_ARGUMENT"),
    (reverse_program((4, 5), [2]), "INVALID_ARGUMENT"),
    (map_program((2, 2)).replace("array<i64: 0, 1>", "array<i64: 1, 0>", 1), "INVALID_ARGUMENT"),
    (map_program((2, 2)).replace("^bb0(%arg2: tensor<i32>, %arg3: tensor<i32>):",
                                 "^bb0(%arg2: tensor<i32>, %arg3: tensor<i32>, %arg9: tensor<i32>):"), "INVALID_ARGUMENT"),
    (bitcast_program((4,), "f32", "i16"), "UNIMPLEMENTED"),
    (bitcast_program((4,), "f64", "i64"), "UNIMPLEMENTED"),
])
def test_malformed(compile_client, prog, code):
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.compile(pjrt.Program.mlir(prog))
    assert e.value.code == getattr(pjrt.ErrorCode, code), e.value.message


# ------------------------------------------------------------------------------------------------ reduce_precision
def reduce_precision_program(shape, e, m, dt="f32", generic=False):
    T = _t(shape, dt)
    op = (f'%0 = "stablehlo.reduce_precision"(%arg0) <{{exponent_bits = {e} : i32, mantissa_bits = {m} : i32}}> : '
          f'({T}) -> {T}' if generic else f"%0 = stablehlo.reduce_precision %arg0, format = e{e}m{m} : {T}")
    return f"""module {{
  func.func @main(%arg0: {T}) -> {T} {{
    {op}
    return %0 : {T}
  }}
}}
"""


def _rp(x, e, m, dt="f32"):
    (r, _), = sh.evaluate(reduce_precision_program(np.shape(x), e, m, dt), [x])
    return np.asarray(r)


def test_reduce_precision_reference_example_and_identity():
    # casting.rs:293-300: [1, 2, 3] at e5m10 stay as they are; a format as wide as the type is the identity
    assert _rp(np.array([1.0, 2.0, 3.0]), 5, 10).tolist() == [1.0, 2.0, 3.0]
    x = np.random.default_rng(4).standard_normal(256).astype(np.float32).astype(np.float64)
    assert np.array_equal(_rp(x, 8, 23), x)


def test_reduce_precision_e8m7_is_bf16_rounding():
    # the bf16 format: round to nearest even at 7 mantissa bits, f32's exponent range (bf16 conversion is pinned
    # exhaustively against torch in test_oracle)
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(4096) * np.exp2(rng.integers(-60, 60, 4096))).astype(np.float32).astype(np.float64)
    x[:4] = [1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -(1.0 + 2.0 ** -8), 3.4e38]  # ties to even, overflow by rounding
    assert np.array_equal(_rp(x, 8, 7), sh.normalize(x, "bf16"))


def test_reduce_precision_e5m10_is_float16_in_its_normal_range():
    rng = np.random.default_rng(6)
    x = (rng.standard_normal(4096) * np.exp2(rng.integers(-13, 15, 4096))).astype(np.float32).astype(np.float64)
    r = _rp(x, 5, 10)
    ok = np.abs(x.astype(np.float16).astype(np.float64)) >= 2.0 ** -14  # numpy's f16 (RNE), outside its subnormals
    assert np.array_equal(r[ok], x[ok].astype(np.float16).astype(np.float64))
    # past the largest f16 (65504, rounding up from 65520) ±inf; below the smallest normal (2^-14) ±0, subnormals
    # of the reduced format included
    big = _rp(np.array([65519.0, 65520.0, -1e6, 2.0 ** -14, 2.0 ** -15, -3e-6]), 5, 10)
    assert big.tolist()[:3] == [65504.0, np.inf, -np.inf] and big[3] == 2.0 ** -14
    assert big[4] == 0.0 and big[5] == 0.0 and np.signbit(big[5])


def test_reduce_precision_of_f16_subnormals_rounds_their_own_field():
    # an f16 subnormal keeps exponent field 0: m mantissa bits leave it a multiple of 2^(-24 + 10 - m), rounded to
    # nearest with ties to the even multiple (closed form against the bit algorithm)
    v = np.arange(1, 1024) * 2.0 ** -24  # every positive f16 subnormal
    for m in (0, 3, 7):
        q = 2.0 ** (-24 + 10 - m)
        want = np.round(v / q) * q  # numpy rounds half to even
        got = _rp(v, 5, m, "f16")
        assert np.array_equal(got, want), m


def test_reduce_precision_nan_and_forms(compile_client):
    r = _rp(np.array([np.nan, np.inf, -np.inf]), 3, 2)
    assert np.isnan(r[0]) and r[1] == np.inf and r[2] == -np.inf
    progs = [reduce_precision_program((8, 64), 4, 3), reduce_precision_program((8, 64), 4, 3, generic=True)]
    plans = [_plan(compile_client, p) for p in progs + [mb.to_bytecode(progs[0])]]
    assert plans[0] == plans[1] == plans[2] and plans[0].count("elementwise") == 1, plans
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.compile(pjrt.Program.mlir(reduce_precision_program((4,), 0, 3)))
    assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.compile(pjrt.Program.mlir(reduce_precision_program((4,), 5, 10, dt="f64")))
    assert e.value.code == pjrt.ErrorCode.UNIMPLEMENTED


def test_replica_and_partition_ids(compile_client):
    # communication.rs:110-190: with one replica and one partition both ids are 0
    prog = """module {
  func.func @main(%arg0: tensor<4xui32>) -> (tensor<4xui32>, tensor<ui32>) {
    %0 = stablehlo.replica_id : tensor<ui32>
    %1 = "stablehlo.partition_id"() : () -> tensor<ui32>
    %2 = stablehlo.add %0, %1 : tensor<ui32>
    %3 = stablehlo.broadcast_in_dim %2, dims = [] : (tensor<ui32>) -> tensor<4xui32>
    %4 = stablehlo.add %arg0, %3 : tensor<4xui32>
    return %4, %0 : tensor<4xui32>, tensor<ui32>
  }
}
"""
    (a, _), (b, _) = sh.evaluate(prog, [np.arange(4)])
    assert a.tolist() == [0, 1, 2, 3] and int(b) == 0
    pretty = prog.replace('"stablehlo.partition_id"() : () -> tensor<ui32>', "stablehlo.partition_id : tensor<ui32>")
    assert _plan(compile_client, prog) == _plan(compile_client, pretty) == _plan(compile_client, mb.to_bytecode(pretty))


# ------------------------------------------------------------------------------------------------ if / case
CASE_EXAMPLE = """module {
  func.func @main(%arg0: tensor<i32>) -> tensor<2xi64> {
    %result = "stablehlo.case"(%arg0) ({
      %c = stablehlo.constant dense<0> : tensor<2xi64>
      stablehlo.return %c : tensor<2xi64>
    }, {
      %c = stablehlo.constant dense<1> : tensor<2xi64>
      stablehlo.return %c : tensor<2xi64>
    }) : (tensor<i32>) -> tensor<2xi64>
    return %result : tensor<2xi64>
  }
}
"""
IF_EXAMPLE = CASE_EXAMPLE.replace('"stablehlo.case"', '"stablehlo.if"').replace("tensor<i32>", "tensor<i1>")


def if_program(shape):
    """Two results; the branches use the function's arguments (values of the enclosing scope) and return one of them."""
    T = _t(shape, "f32")
    return f"""module {{
  func.func @main(%arg0: tensor<i1>, %arg1: {T}, %arg2: {T}) -> ({T}, {T}) {{
    %s = stablehlo.subtract %arg1, %arg2 : {T}
    %0:2 = "stablehlo.if"(%arg0) ({{
      %1 = stablehlo.add %s, %arg2 : {T}
      stablehlo.return %1, %arg1 : {T}, {T}
    }}, {{
      %1 = stablehlo.multiply %arg1, %arg2 : {T}
      stablehlo.return %1, %s : {T}, {T}
    }}) : (tensor<i1>) -> ({T}, {T})
    %2 = stablehlo.add %0#0, %0#1 : {T}
    return %2, %0#1 : {T}, {T}
  }}
}}
"""


def case_program(n_branches, shape):
    """Branch k returns arg1 · (k + 1) + arg2 (as a product with a constant and a sum)."""
    T = _t(shape, "f32")
    branches = []
    for k in range(n_branches):
        branches.append(f"""      %c = stablehlo.constant dense<{k + 1}.0> : {T}
      %m = stablehlo.multiply %arg1, %c : {T}
      %a = stablehlo.add %m, %arg2 : {T}
      stablehlo.return %a : {T}""")
    body = "\n    }, {\n".join(branches)
    return f"""module {{
  func.func @main(%arg0: tensor<i32>, %arg1: {T}, %arg2: {T}) -> {T} {{
    %0 = "stablehlo.case"(%arg0) ({{
{body}
    }}) : (tensor<i32>) -> {T}
    return %0 : {T}
  }}
}}
"""


def test_if_and_case_reference_examples():
    # control_flow.rs:19-33 (case, index 1 → [1, 1]) and :77-91 (if, true → [0, 0]); out-of-range indices take the
    # last branch (control_flow.rs:13-15)
    for idx, want in ((1, [1, 1]), (0, [0, 0]), (7, [1, 1]), (-1, [1, 1])):
        (r, _), = sh.evaluate(CASE_EXAMPLE, [np.array(idx)])
        assert r.tolist() == want, idx
    for p, want in ((True, [0, 0]), (False, [1, 1])):
        (r, _), = sh.evaluate(IF_EXAMPLE, [np.array(p)])
        assert r.tolist() == want


def test_if_with_captures_and_two_results():
    rng = np.random.default_rng(11)
    a, b = rng.standard_normal((2, 4, 8))
    for p in (True, False):
        (r0, _), (r1, _) = sh.evaluate(if_program((4, 8)), [np.array(p), a, b])
        s = sh.normalize(a - b, "f32")
        first, second = (sh.normalize(s + b, "f32"), a) if p else (sh.normalize(a * b, "f32"), s)
        assert np.array_equal(r0, sh.normalize(first + second, "f32")) and np.array_equal(r1, second)


def test_if_and_case_forms_plan_alike(compile_client):
    for prog in (CASE_EXAMPLE, IF_EXAMPLE, if_program((8, 64)), case_program(3, (8, 64))):
        plans = [_plan(compile_client, p) for p in (prog, mb.to_bytecode(prog))]
        assert plans[0] == plans[1], plans
    # every branch computed, the results selected: one fused elementwise step per result
    plan = _plan(compile_client, case_program(3, (8, 64))).strip().split("\n")
    assert len(plan) == 1 and "elementwise" in plan[0], plan


GET_DIM_EXAMPLE = """module {
  func.func @main(%arg0: tensor<2x3xi64>) -> (tensor<i32>, tensor<i32>) {
    %0 = stablehlo.get_dimension_size %arg0, dim = 1 : (tensor<2x3xi64>) -> tensor<i32>
    %1 = "stablehlo.get_dimension_size"(%arg0) <{dimension = 0 : i64}> : (tensor<2x3xi64>) -> tensor<i32>
    return %0, %1 : tensor<i32>, tensor<i32>
  }
}
"""


def test_get_dimension_size(compile_client):
    # manipulation.rs:22-26: [[1, 2, 3], [4, 5, 6]], dim = 1 → 3
    (a, dt), (b, _) = sh.evaluate(GET_DIM_EXAMPLE, [np.array([[1, 2, 3], [4, 5, 6]])])
    assert dt == "i32" and int(a) == 3 and int(b) == 2
    pretty = GET_DIM_EXAMPLE.replace('"stablehlo.get_dimension_size"(%arg0) <{dimension = 0 : i64}> :',
                                     "stablehlo.get_dimension_size %arg0, dim = 0 :")
    assert _plan(compile_client, GET_DIM_EXAMPLE) == _plan(compile_client, pretty) == \
        _plan(compile_client, mb.to_bytecode(pretty))
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.compile(pjrt.Program.mlir(GET_DIM_EXAMPLE.replace("dim = 1", "dim = 2")))
    assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT
