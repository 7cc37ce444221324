"""reduce with several inputs and with bodies other than one binary op (crates/ryft-mlir/src/dialects/stable_hlo/
operations/functional.rs:109-230: `reduce(inputs, initial_values, dimensions, computation)`), on the CPU:

  * oracle     argmax / argmin in the comparator form JAX lowers them to (values with an iota of indices, the larger
               (smaller) value winning, NaN winning, the lower index winning ties) against numpy's argmax / argmin
               (first occurrence); a two-input reduce with independent bodies (sum, max) against numpy; a one-input
               body that is not a single op (max written as compare + select) and one outside the fast set (xor);
  * front-ends the pretty form (`reduce(%x init: %i), (%y init: %j) ... reducer(%a: T, %c: T) (%b: U, %d: U)`), the
               generic form (`"stablehlo.reduce"(...) ({ ^bb0(...): ... })`) and bytecode plan alike;
  * checks     a body whose arguments or results do not match the inputs, an odd operand count, inputs of different
               shapes and more than two inputs are refused with the error each deserves.
GPU parity of the same programs: tests/test_gpu_reduce_bodies.py."""
import numpy as np
import pytest

from oracle import stablehlo as sh
from ryft_amd import pjrt
from tests import mlir_bytecode as mb


def _t(shape, dt):
    return "tensor<" + "".join(f"{d}x" for d in shape) + dt + ">"


def _neg_limit(dt):
    return {"f32": "0xFF800000", "bf16": "0xFF80", "f16": "0xFC00"}.get(dt, "-2147483648")


def _pos_limit(dt):
    return {"f32": "0x7F800000", "bf16": "0x7F80", "f16": "0x7C00"}.get(dt, "2147483647")


def argmax_program(shape, dim, dt="f32", it="i32", kind="argmax", form="pretty"):
    """JAX's lowering of argmax / argmin along `dim`: values paired with an iota of their indices, the body keeping
    the larger (smaller) value — a NaN wins, and of equal values the lower index — returning both results."""
    fl = dt in ("f32", "bf16", "f16")
    out = [d for i, d in enumerate(shape) if i != dim]
    X, I, S, SI = _t(shape, dt), _t(shape, it), f"tensor<{dt}>", f"tensor<{it}>"
    RX, RI = _t(out, dt), _t(out, it)
    init = _neg_limit(dt) if kind == "argmax" else _pos_limit(dt)
    cmp = "GT" if kind == "argmax" else "LT"
    ctype = "FLOAT" if fl else "SIGNED"
    a, b, ai, bi = "%a", "%b", "%ai", "%bi"
    if form == "pretty":
        body = f"""      %2 = stablehlo.compare  {cmp}, {a}, {b},  {ctype} : ({S}, {S}) -> tensor<i1>
      %3 = stablehlo.compare  NE, {a}, {a},  {ctype} : ({S}, {S}) -> tensor<i1>
      %4 = stablehlo.or %2, %3 : tensor<i1>
      %5 = stablehlo.compare  EQ, {a}, {b},  {ctype} : ({S}, {S}) -> tensor<i1>
      %6 = stablehlo.compare  LT, {ai}, {bi},  SIGNED : ({SI}, {SI}) -> tensor<i1>
      %7 = stablehlo.and %5, %6 : tensor<i1>
      %8 = stablehlo.or %4, %7 : tensor<i1>
      %9 = stablehlo.select %4, {a}, {b} : tensor<i1>, {S}
      %10 = stablehlo.select %8, {ai}, {bi} : tensor<i1>, {SI}
      stablehlo.return %9, %10 : {S}, {SI}"""
        op = (f"""    %1:2 = stablehlo.reduce(%arg0 init: %cst), (%0 init: %c) across dimensions = [{dim}] : """
              f"""({X}, {I}, {S}, {SI}) -> ({RX}, {RI})
     reducer({a}: {S}, {b}: {S}) ({ai}: {SI}, {bi}: {SI})  {{
{body}
    }}""")
    else:
        def c(d, x, y, t, st):
            return (f'      %{d} = "stablehlo.compare"({x}, {y}) <{{comparison_direction = #stablehlo<comparison_direction '
                    f'{t}>, compare_type = #stablehlo<comparison_type {st}>}}> : ({S if x in (a, b) else SI}, '
                    f'{S if x in (a, b) else SI}) -> tensor<i1>')
        body = "\n".join([
            c(2, a, b, cmp, ctype), c(3, a, a, "NE", ctype),
            '      %4 = "stablehlo.or"(%2, %3) : (tensor<i1>, tensor<i1>) -> tensor<i1>',
            c(5, a, b, "EQ", ctype), c(6, ai, bi, "LT", "SIGNED"),
            '      %7 = "stablehlo.and"(%5, %6) : (tensor<i1>, tensor<i1>) -> tensor<i1>',
            '      %8 = "stablehlo.or"(%4, %7) : (tensor<i1>, tensor<i1>) -> tensor<i1>',
            f'      %9 = "stablehlo.select"(%4, {a}, {b}) : (tensor<i1>, {S}, {S}) -> {S}',
            f'      %10 = "stablehlo.select"(%8, {ai}, {bi}) : (tensor<i1>, {SI}, {SI}) -> {SI}',
            f'      "stablehlo.return"(%9, %10) : ({S}, {SI}) -> ()'])
        op = (f'    %1:2 = "stablehlo.reduce"(%arg0, %0, %cst, %c) <{{dimensions = array<i64: {dim}>}}> ({{\n'
              f"    ^bb0({a}: {S}, {ai}: {SI}, {b}: {S}, {bi}: {SI}):\n{body}\n"
              f"    }}) : ({X}, {I}, {S}, {SI}) -> ({RX}, {RI})")
    return f"""module {{
  func.func @main(%arg0: {X}) -> ({RX}, {RI}) {{
    %0 = stablehlo.iota dim = {dim} : {I}
    %cst = stablehlo.constant dense<{init}> : {S}
    %c = stablehlo.constant dense<0> : {SI}
{op}
    return %1#0, %1#1 : {RX}, {RI}
  }}
}}
"""


def sum_max_program(shape, dims, dt="f32"):
    """Two inputs reduced together with independent bodies: the sum of the first and the maximum of the second."""
    out = [d for i, d in enumerate(shape) if i not in dims]
    X, S, R = _t(shape, dt), f"tensor<{dt}>", _t(out, dt)
    ds = ", ".join(map(str, dims))
    return f"""module {{
  func.func @main(%arg0: {X}, %arg1: {X}) -> ({R}, {R}) {{
    %z = stablehlo.constant dense<0.000000e+00> : {S}
    %m = stablehlo.constant dense<{_neg_limit(dt)}> : {S}
    %1:2 = stablehlo.reduce(%arg0 init: %z), (%arg1 init: %m) across dimensions = [{ds}] : ({X}, {X}, {S}, {S}) -> ({R}, {R})
     reducer(%a: {S}, %b: {S}) (%c: {S}, %d: {S})  {{
      %2 = stablehlo.add %a, %b : {S}
      %3 = stablehlo.maximum %c, %d : {S}
      stablehlo.return %2, %3 : {S}, {S}
    }}
    return %1#0, %1#1 : {R}, {R}
  }}
}}
"""


def one_input_program(shape, dim, body, dt):
    """One input whose body is not one recognised binary op: "select_max" (max as compare GT + select) or "xor"."""
    out = [d for i, d in enumerate(shape) if i != dim]
    X, S, R = _t(shape, dt), f"tensor<{dt}>", _t(out, dt)
    if body == "select_max":
        init = _neg_limit(dt)
        ops = f"""      %2 = stablehlo.compare  GT, %a, %b : ({S}, {S}) -> tensor<i1>
      %3 = stablehlo.select %2, %a, %b : tensor<i1>, {S}
      stablehlo.return %3 : {S}"""
    else:
        init = "0"
        ops = f"""      %3 = stablehlo.xor %a, %b : {S}
      stablehlo.return %3 : {S}"""
    return f"""module {{
  func.func @main(%arg0: {X}) -> {R} {{
    %i = stablehlo.constant dense<{init}> : {S}
    %1 = stablehlo.reduce(%arg0 init: %i) across dimensions = [{dim}] : ({X}, {S}) -> {R}
     reducer(%a: {S}, %b: {S})  {{
{ops}
    }}
    return %1 : {R}
  }}
}}
"""


# ------------------------------------------------------------------------------------------------ oracle pins
def _with_ties(seed, shape, dim):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(shape).astype(np.float32).astype(np.float64)
    # plant equal maxima (the first must win) and equal minima
    flat = np.moveaxis(x, dim, -1).reshape(-1, shape[dim])
    for r in range(0, flat.shape[0], 3):
        flat[r, [1, shape[dim] - 2]] = 9.0
        flat[r, [0, shape[dim] - 1]] = -9.0
    return np.moveaxis(flat.reshape(np.moveaxis(x, dim, -1).shape), -1, dim).copy()


@pytest.mark.parametrize("form", ["pretty", "generic"])
@pytest.mark.parametrize("kind", ["argmax", "argmin"])
@pytest.mark.parametrize("shape,dim", [((6, 50), 1), ((7, 5, 9), 0), ((3, 4, 17), 2)])
def test_oracle_argmax_argmin_are_numpys(form, kind, shape, dim):
    x = _with_ties(1, shape, dim)
    (v, vdt), (i, idt) = sh.evaluate(argmax_program(shape, dim, kind=kind, form=form), [x])
    want_i = np.argmax(x, axis=dim) if kind == "argmax" else np.argmin(x, axis=dim)
    want_v = np.max(x, axis=dim) if kind == "argmax" else np.min(x, axis=dim)
    assert (vdt, idt) == ("f32", "i32")
    assert np.array_equal(i, want_i) and np.array_equal(v, want_v)


def test_oracle_argmax_nan_wins_and_integer_values():
    x = np.array([[1.0, np.nan, 5.0, np.nan], [2.0, 7.0, 7.0, 1.0]])
    (v, _), (i, _) = sh.evaluate(argmax_program((2, 4), 1), [x])
    assert i.tolist() == [1, 1] and np.isnan(v[0]) and v[1] == 7.0
    xi = np.array([[3, -5, 3, 8, 8], [-1, -1, -7, -7, 0]], np.int64)
    (v, _), (i, _) = sh.evaluate(argmax_program((2, 5), 1, dt="i32"), [xi])
    assert i.tolist() == [3, 4] and v.tolist() == [8, 0]
    (v, _), (i, _) = sh.evaluate(argmax_program((2, 5), 1, dt="i32", kind="argmin"), [xi])
    assert i.tolist() == [1, 2] and v.tolist() == [-5, -7]


def test_oracle_two_bodies_and_one_input_bodies():
    rng = np.random.default_rng(2)
    a = rng.standard_normal((5, 6, 7)).astype(np.float32).astype(np.float64)
    b = rng.standard_normal((5, 6, 7)).astype(np.float32).astype(np.float64)
    (s, _), (m, _) = sh.evaluate(sum_max_program((5, 6, 7), [0, 2]), [a, b])
    assert np.allclose(s, a.sum(axis=(0, 2)), rtol=1e-5) and np.array_equal(m, b.max(axis=(0, 2)))
    (r, _), = sh.evaluate(one_input_program((5, 6, 7), 1, "select_max", "f32"), [a])
    assert np.array_equal(r, a.max(axis=1))
    xi = rng.integers(-2 ** 31, 2 ** 31, size=(4, 33)).astype(np.int64)
    (r, _), = sh.evaluate(one_input_program((4, 33), 1, "xor", "i32"), [xi])
    want = np.bitwise_xor.reduce(xi.astype(np.int32), axis=1).astype(np.int64)
    assert np.array_equal(r, want)


# ------------------------------------------------------------------------------------------------ front-ends
def _plan(client, program):
    return client.compile(pjrt.Program.mlir(program)).describe_plan()


@pytest.mark.parametrize("kind", ["argmax", "argmin"])
def test_forms_plan_alike(compile_client, kind):
    printed = argmax_program((8, 1000), 1, kind=kind)
    plans = [_plan(compile_client, printed), _plan(compile_client, argmax_program((8, 1000), 1, kind=kind,
                                                                                   form="generic"))]
    plans += [_plan(compile_client, mb.to_bytecode(printed, **o)) for o in ({}, {"isolated_reduce": True})]
    assert all(p == plans[0] for p in plans), plans
    # one step computes both results, each written straight into its output buffer; the body is recognised as the
    # argmax / argmin rule (no body program)
    assert plans[0].startswith(f"0: {kind} ") and "inputs=2" in plans[0] and "copy" not in plans[0], plans[0]
    assert "out=f32,i32" in plans[0] and "body_instrs=0" in plans[0], plans[0]


def test_argmax_recognition(compile_client):
    # integer and bf16 values, the reduced dim outermost, an i64 position
    for prog in (argmax_program((6, 40), 1, dt="i32"), argmax_program((40, 6), 0, dt="bf16", it="i64"),
                 argmax_program((3, 4, 50), 2, kind="argmin", form="generic")):
        plan = _plan(compile_client, prog)
        assert plan.split()[1] in ("argmax", "argmin") and "body_instrs=0" in plan, plan
    # long rows of few outputs: segments folded by a second launch
    plan = _plan(compile_client, argmax_program((8, 32000), 1))
    assert "segments=3" in plan, plan
    # bodies that are not the rule run the body program: the later position winning ties, or a value compared
    # with a constant
    later = argmax_program((6, 40), 1).replace("LT, %ai, %bi", "GT, %ai, %bi")
    capped = argmax_program((6, 40), 1).replace(
        "%3 = stablehlo.compare  NE, %a, %a,  FLOAT", "%k = stablehlo.constant dense<1.000000e+00> : tensor<f32>\n"
        "      %3 = stablehlo.compare  NE, %a, %k,  FLOAT")
    for prog in (later, capped):
        plan = _plan(compile_client, prog)
        assert plan.startswith("0: reduce ") and "body_instrs=0" not in plan, plan
    # the index input must be an iota along the reduced dim
    other_dim = argmax_program((6, 40), 1).replace("stablehlo.iota dim = 1", "stablehlo.iota dim = 0")
    assert _plan(compile_client, other_dim).startswith("0: reduce ")


def test_one_input_general_bodies_plan(compile_client):
    for body, dt in (("select_max", "f32"), ("xor", "i32")):
        plan = _plan(compile_client, one_input_program((16, 300), 1, body, dt))
        assert "inputs=1" in plan and "body_instrs=" in plan, plan
    # a region applying one recognised op to its two arguments is the fast reduction
    text = one_input_program((16, 300), 1, "select_max", "f32").replace(
        """      %2 = stablehlo.compare  GT, %a, %b : (tensor<f32>, tensor<f32>) -> tensor<i1>
      %3 = stablehlo.select %2, %a, %b : tensor<i1>, tensor<f32>""", "      %3 = stablehlo.maximum %b, %a : tensor<f32>")
    plan = _plan(compile_client, text)
    assert "reduce" in plan and "inputs=" not in plan, plan


@pytest.mark.parametrize("edit,code", [
    # the body returns one value for two inputs
    (lambda t: t.replace("stablehlo.return %9, %10 : tensor<f32>, tensor<i32>", "stablehlo.return %9 : tensor<f32>"),
     "INVALID_ARGUMENT"),
    # a body result of the wrong type
    (lambda t: t.replace("stablehlo.return %9, %10 : tensor<f32>, tensor<i32>",
                         "stablehlo.return %10, %9 : tensor<i32>, tensor<f32>"), "INVALID_ARGUMENT"),
    # body arguments of another type than the inputs (promotion)
    (lambda t: t.replace("(%ai: tensor<i32>, %bi: tensor<i32>)", "(%ai: tensor<i64>, %bi: tensor<i64>)"),
     "UNIMPLEMENTED"),
])
def test_malformed_bodies(compile_client, edit, code):
    text = edit(argmax_program((4, 64), 1))
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.compile(pjrt.Program.mlir(text))
    assert e.value.code == getattr(pjrt.ErrorCode, code), e.value.message


def test_inputs_of_different_shapes_and_three_inputs(compile_client):
    text = sum_max_program((4, 6), [1]).replace("%arg1: tensor<4x6xf32>", "%arg1: tensor<4x7xf32>").replace(
        "(tensor<4x6xf32>, tensor<4x6xf32>, tensor<f32>", "(tensor<4x6xf32>, tensor<4x7xf32>, tensor<f32>")
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.compile(pjrt.Program.mlir(text))
    assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT and "shape" in e.value.message
    S = "tensor<f32>"
    three = f"""module {{
  func.func @main(%a0: tensor<4x6xf32>, %a1: tensor<4x6xf32>, %a2: tensor<4x6xf32>) -> tensor<4xf32> {{
    %z = stablehlo.constant dense<0.000000e+00> : {S}
    %1:3 = stablehlo.reduce(%a0 init: %z), (%a1 init: %z), (%a2 init: %z) across dimensions = [1] : (tensor<4x6xf32>, tensor<4x6xf32>, tensor<4x6xf32>, {S}, {S}, {S}) -> (tensor<4xf32>, tensor<4xf32>, tensor<4xf32>)
     reducer(%a: {S}, %b: {S}) (%c: {S}, %d: {S}) (%e: {S}, %f: {S})  {{
      %2 = stablehlo.add %a, %b : {S}
      %3 = stablehlo.add %c, %d : {S}
      %4 = stablehlo.add %e, %f : {S}
      stablehlo.return %2, %3, %4 : {S}, {S}, {S}
    }}
    return %1#2 : tensor<4xf32>
  }}
}}
"""
    (r, _), = sh.evaluate(three, [np.ones((4, 6))] * 3)
    assert r.tolist() == [6.0] * 4
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.compile(pjrt.Program.mlir(three))
    assert e.value.code == pjrt.ErrorCode.UNIMPLEMENTED and "inputs" in e.value.message


def test_argmax_workload(compile_client):
    """bench.py's argmax workload (ryft_amd/configs.py) is the argmax rule: its plan, and its oracle against numpy's
    argmax on a small instance."""
    from ryft_amd import configs
    w = configs.CONFIGS["argmax"](m=4, v=4096)
    plan = _plan(compile_client, w.program)
    assert plan.startswith("0: argmax ") and "out=f32,i32" in plan, plan
    x = sh.from_raw(w.inputs[0].data, "f32")
    (v, _), (i, _) = sh.evaluate(w.program, [x])
    assert np.array_equal(i, np.argmax(x, axis=1)) and np.array_equal(v, np.max(x, axis=1))
    full = configs.CONFIGS["argmax"]()
    assert _plan(compile_client, full.program).startswith("0: argmax ") and full.bytes == 4.0 * 64 * 128256 + 8 * 64
