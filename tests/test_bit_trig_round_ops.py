"""The trigonometric, cube-root, rounding, is_finite and bit-manipulation ops on the CPU: the oracle pinned by
methods of its own, and the plugin's front-ends and node checks.

  * bit ops      shift_left / shift_right_arithmetic / shift_right_logical / popcnt / count_leading_zeros
                 (crates/ryft-mlir/src/dialects/stable_hlo/operations/bit_manipulation.rs:5-280) over every pair of
                 8-bit values, signed and unsigned, against a restatement on binary digit strings, and against
                 numpy's own shifts at 16 and 32 bits for amounts inside the width;
  * rounding     round_nearest_even / round_nearest_afz (rounding.rs:91-180) against Python's round() (ties to
                 even) and decimal's ROUND_HALF_UP on f32 values, halves and signed zeros included;
  * float maps   sine / cosine / tan / atan2 / cbrt / is_finite (trigonometric.rs:7-262, exponential.rs:166-210,
                 arithmetic.rs:470-515) against the math module and identities (sin^2 + cos^2 = 1, the quadrants
                 of atan2, cbrt(x)^3 = x);
  * front-ends   the printed, generic and bytecode forms plan alike; operand / result types the ops do not take are
                 INVALID_ARGUMENT; bit ops on 64-bit integers are UNIMPLEMENTED (64-bit integer elements live in
                 32-bit registers in elementwise programs).
The reference's worked examples of these ops are in tests/ref_examples.py (oracle: tests/test_oracle.py, GPU:
tests/test_gpu_ops.py)."""
import decimal
import math

import numpy as np
import pytest

from oracle import stablehlo as sh
from ryft_amd import pjrt
from tests import mlir_bytecode as mb


def _prog(op, in_types, out_type, shape, generic=False):
    dims = "".join(f"{d}x" for d in shape)
    ts = [f"tensor<{dims}{t}>" for t in in_types]
    to = f"tensor<{dims}{out_type}>"
    sig = ", ".join(f"%arg{i}: {t}" for i, t in enumerate(ts))
    args = ", ".join(f"%arg{i}" for i in range(len(ts)))
    if generic:
        body = f'%0 = "stablehlo.{op}"({args}) : ({", ".join(ts)}) -> {to}'
    elif len(set(ts)) != 1 or ts[0] != to:
        body = f"%0 = stablehlo.{op} {args} : ({', '.join(ts)}) -> {to}"
    else:
        body = f"%0 = stablehlo.{op} {args} : {to}"
    return f"module {{\n  func.func @main({sig}) -> {to} {{\n    {body}\n    return %0 : {to}\n  }}\n}}\n"


def _eval(op, dt, *vals, out_type=None):
    vals = [np.asarray(v) for v in vals]
    (out, odt), = sh.evaluate(_prog(op, [dt] * len(vals), out_type or dt, vals[0].shape), vals)
    return np.asarray(out), odt


# ------------------------------------------------------------------------------------------------ bit operations
def _digits(v, w):
    return format(v & ((1 << w) - 1), f"0{w}b")


def _value(bits, signed):
    v = int(bits, 2)
    return v - (1 << len(bits)) if signed and bits[0] == "1" else v


def _by_digits(op, a, b, w, signed):
    """One element on its binary digits (most significant first)."""
    s = _digits(a, w)
    if op == "popcnt":
        return s.count("1")
    if op == "count_leading_zeros":
        return len(s) - len(s.lstrip("0"))
    k = b & ((1 << w) - 1)  # the amount as a w-bit unsigned integer
    if op == "shift_left":
        out = (s[k:] + "0" * k) if k < w else "0" * w
    elif op == "shift_right_logical":
        out = ("0" * k + s[:w - k]) if k < w else "0" * w
    else:
        out = (s[0] * k + s[:w - k]) if k < w else s[0] * w
    return _value(out, signed)


@pytest.mark.parametrize("dt", ["i8", "ui8"])
@pytest.mark.parametrize("op", ["shift_left", "shift_right_arithmetic", "shift_right_logical", "popcnt",
                                "count_leading_zeros"])
def test_bit_ops_every_8bit_pair(op, dt):
    signed = dt == "i8"
    vals = np.arange(-128, 128) if signed else np.arange(256)
    a, b = np.meshgrid(vals, vals, indexing="ij")
    a, b = a.astype(np.int64), b.astype(np.int64)
    binary = op.startswith("shift")
    got, odt = _eval(op, dt, a, b) if binary else _eval(op, dt, a[:, :1])
    assert odt == dt
    if binary:
        want = np.array([[_by_digits(op, int(x), int(y), 8, signed) for x, y in zip(ra, rb)] for ra, rb in zip(a, b)])
    else:
        want = np.array([[_by_digits(op, int(x), 0, 8, signed)] for x in a[:, 0]])
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dt,npt", [("i16", np.int16), ("ui16", np.uint16), ("i32", np.int32), ("ui32", np.uint32)])
def test_shifts_match_numpy_inside_the_width(dt, npt):
    w = np.iinfo(npt).bits
    rng = np.random.default_rng(w + (dt[0] == "u"))
    info = np.iinfo(npt)
    a = rng.integers(info.min, info.max, size=4096, endpoint=True).astype(npt)
    a[:6] = [info.min, info.max, 0, 1, info.max // 2, info.min + 1]
    k = rng.integers(0, w, size=4096).astype(npt)
    for op, fn in (("shift_left", np.left_shift), ("shift_right_logical", None),
                   ("shift_right_arithmetic", np.right_shift)):
        got, _ = _eval(op, dt, a.astype(np.int64), k.astype(np.int64))
        if op == "shift_right_logical":
            u = a.view({16: np.uint16, 32: np.uint32}[w])
            want = np.right_shift(u, k.astype(u.dtype)).view(npt)
        elif op == "shift_right_arithmetic":
            s = a.view({16: np.int16, 32: np.int32}[w])
            want = np.right_shift(s, k.astype(s.dtype)).view(npt)
        else:
            want = fn(a, k)
        assert np.array_equal(got, want.astype(np.int64)), op
    # popcnt / count_leading_zeros against Python's own bit counts
    u = [int(x) & ((1 << w) - 1) for x in a.astype(np.int64)]
    got, _ = _eval("popcnt", dt, a.astype(np.int64))
    assert got.tolist() == [bin(x).count("1") for x in u]
    got, _ = _eval("count_leading_zeros", dt, a.astype(np.int64))
    assert got.tolist() == [w - x.bit_length() for x in u]


def test_shift_amounts_outside_the_width():
    # amounts of the width or more (and negative ones, which read as large unsigned amounts) shift everything out:
    # 0 for left and logical shifts, the sign for arithmetic ones
    a = np.array([-7, -7, -7, 7, 7, 7], np.int64)
    k = np.array([32, 33, -1, 32, 100, -32], np.int64)
    assert _eval("shift_left", "i32", a, k)[0].tolist() == [0] * 6
    assert _eval("shift_right_logical", "i32", a, k)[0].tolist() == [0] * 6
    assert _eval("shift_right_arithmetic", "i32", a, k)[0].tolist() == [-1, -1, -1, 0, 0, 0]


# ------------------------------------------------------------------------------------------------ rounding
def _f32_samples():
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(2000) * 10, rng.standard_normal(500) * 1e6,
                        np.arange(-40, 41) / 2.0,  # every half in [-20, 20]
                        np.array([2.0 ** 23 - 0.5, 2.0 ** 23 + 1, 2.0 ** 24 + 2, 0.49999997, -0.49999997, 1.5,
                                  -1.5, 0.4, -0.4, 0.0, -0.0, 3.0e38, -3.0e38, 1e-40])])
    return x.astype(np.float32).astype(np.float64)


def test_round_nearest_even_is_pythons_round():
    x = _f32_samples()
    got, _ = _eval("round_nearest_even", "f32", x)
    want = np.array([math.copysign(float(round(v)), v) for v in x])  # a zero result keeps the operand's sign
    assert np.array_equal(got, want) and np.array_equal(np.signbit(got), np.signbit(want))
    inf = _eval("round_nearest_even", "f32", np.array([np.inf, -np.inf, np.nan]))[0]
    assert inf[0] == np.inf and inf[1] == -np.inf and np.isnan(inf[2])


def test_round_nearest_afz_is_decimal_half_up():
    x = _f32_samples()
    got, _ = _eval("round_nearest_afz", "f32", x)
    ctx = decimal.Context(prec=80)  # room for every f32 integer (3e38 has 39 digits)
    want = np.array([math.copysign(float(decimal.Decimal(v).quantize(decimal.Decimal(1), decimal.ROUND_HALF_UP,
                                                                     context=ctx)), v) for v in x])
    assert np.array_equal(got, want) and np.array_equal(np.signbit(got), np.signbit(want))


def test_rounding_of_bf16_operands():
    # bf16 operands round to bf16 results without a second rounding step (every integer below the operand's
    # magnitude that the rounding can produce is a bf16 value)
    x = np.array([0.5, 1.5, 2.5, -2.5, 3.5, 255.5, -0.5, 100.0], np.float64)
    assert _eval("round_nearest_even", "bf16", x)[0].tolist() == [0.0, 2.0, 2.0, -2.0, 4.0, 256.0, -0.0, 100.0]
    assert _eval("round_nearest_afz", "bf16", x)[0].tolist() == [1.0, 2.0, 3.0, -3.0, 4.0, 256.0, -1.0, 100.0]


# ------------------------------------------------------------------------------------------------ float maps
def test_trig_and_cbrt_match_the_math_module():
    x = np.linspace(-20, 20, 401).astype(np.float32).astype(np.float64)
    for op, fn in (("sine", math.sin), ("cosine", math.cos), ("tan", math.tan), ("cbrt", None)):
        got, _ = _eval(op, "f32", x)
        if op == "cbrt":
            want = np.array([math.copysign(abs(v) ** (1.0 / 3.0), v) for v in x])
            tol = 1e-6  # the power form of the cube root is itself off in the last bits
        else:
            want = np.array([fn(v) for v in x])
            tol = 0.0
        w32 = want.astype(np.float32).astype(np.float64)
        assert np.all(np.abs(got - w32) <= tol * np.maximum(1.0, np.abs(w32))), op
    s, _ = _eval("sine", "f32", x)
    c, _ = _eval("cosine", "f32", x)
    assert np.allclose(s * s + c * c, 1.0, atol=2e-7)
    cube = np.array([-27.0, -8.0, -1.0, 0.0, 1.0, 8.0, 27.0, 64.0, 1e-30, 1e30])
    got, _ = _eval("cbrt", "f32", cube.astype(np.float32).astype(np.float64))
    assert np.allclose(got ** 3, cube.astype(np.float32), rtol=1e-6)
    assert got[:7].tolist() == [-3.0, -2.0, -1.0, 0.0, 1.0, 2.0, 3.0]


def test_atan2_quadrants_and_special_values():
    y = np.array([1.0, 1.0, -1.0, -1.0, 0.0, -0.0, 0.0, -0.0, np.inf, -np.inf, 1.0, np.nan])
    x = np.array([1.0, -1.0, 1.0, -1.0, 1.0, 1.0, -1.0, -1.0, np.inf, 2.0, 0.0, 1.0])
    got, _ = _eval("atan2", "f32", y, x)
    want = [math.atan2(a, b) for a, b in zip(y, x)]
    assert np.array_equal(got[:-1], np.array(want[:-1], np.float32).astype(np.float64))
    assert np.array_equal(np.signbit(got[:-1]), np.signbit(np.array(want[:-1]))) and np.isnan(got[-1])
    # quadrants: atan2(y, -x) = pi - atan2(y, x) for y > 0
    q = np.linspace(0.1, 5, 50)
    a, _ = _eval("atan2", "f32", q, q[::-1])
    b, _ = _eval("atan2", "f32", q, -q[::-1])
    assert np.allclose(a + b, math.pi, atol=4e-7)


def test_is_finite():
    x = np.array([0.0, -0.0, 1.0, -65504.0, 2.0 ** -24, np.inf, -np.inf, np.nan])
    for dt in ("f32", "bf16", "f16"):
        got, odt = _eval("is_finite", dt, x, out_type="i1")
        assert odt == "i1"
        assert got.tolist() == [1, 1, 1, 1, 1, 0, 0, 0]


# ------------------------------------------------------------------------------------------------ front-ends
CASES = [("sine", ["f32"], "f32"), ("cosine", ["bf16"], "bf16"), ("tan", ["f32"], "f32"), ("cbrt", ["f32"], "f32"),
         ("atan2", ["f32", "f32"], "f32"), ("round_nearest_even", ["bf16"], "bf16"),
         ("round_nearest_afz", ["f32"], "f32"), ("is_finite", ["f32"], "i1"), ("popcnt", ["i32"], "i32"),
         ("count_leading_zeros", ["ui16"], "ui16"), ("shift_left", ["i8", "i8"], "i8"),
         ("shift_right_arithmetic", ["ui32", "ui32"], "ui32"), ("shift_right_logical", ["i32", "i32"], "i32")]


@pytest.mark.parametrize("op,ins,out", CASES, ids=[c[0] for c in CASES])
def test_forms_plan_alike(compile_client, op, ins, out):
    printed = _prog(op, ins, out, (4, 33))
    plans = [compile_client.compile(pjrt.Program.mlir(p)).describe_plan()
             for p in (printed, _prog(op, ins, out, (4, 33), generic=True), mb.to_bytecode(printed))]
    assert plans[0] == plans[1] == plans[2]
    assert "elementwise" in plans[0] or "map" in plans[0], plans[0]


@pytest.mark.parametrize("op,ins,out", [
    ("sine", ["i32"], "i32"), ("atan2", ["f32", "bf16"], "f32"), ("cbrt", ["f32"], "bf16"),
    ("is_finite", ["f32"], "f32"), ("is_finite", ["i32"], "i1"), ("popcnt", ["f32"], "f32"),
    ("popcnt", ["i1"], "i1"), ("shift_left", ["i32", "i8"], "i32"), ("shift_right_logical", ["f32", "f32"], "f32"),
    ("count_leading_zeros", ["i32"], "i8"), ("round_nearest_even", ["i32"], "i32")])
def test_types_the_ops_do_not_take_are_invalid(compile_client, op, ins, out):
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.compile(pjrt.Program.mlir(_prog(op, ins, out, (8,), generic=True)))
    assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT, e.value.message


@pytest.mark.parametrize("op,n", [("shift_left", 2), ("shift_right_logical", 2), ("popcnt", 1),
                                  ("count_leading_zeros", 1)])
def test_bit_ops_on_64bit_integers_are_unimplemented(compile_client, op, n):
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.compile(pjrt.Program.mlir(_prog(op, ["i64"] * n, "i64", (8,))))
    assert e.value.code == pjrt.ErrorCode.UNIMPLEMENTED and "64-bit" in e.value.message
