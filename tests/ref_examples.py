"""Worked examples from the reference's StableHLO op documentation, as test vectors.

Each entry is one op applied to the documented operands, with the documented result. They pin the CPU oracle
(tests/test_oracle.py) and the plugin's kernels (tests/test_gpu_ops.py) to the same numbers. Where the documented
example uses a type the plugin does not execute (f64, i64, complex), the same values are given in f32 / i32: every
documented value is representable there, and the printed results ("0.333333343", "5.66666651") are the f32 ones.

Reference files: crates/ryft-mlir/src/dialects/stable_hlo/operations/<file>.rs at the cited lines.
"""
from dataclasses import dataclass
from typing import List, Tuple

import numpy as np

NAN, INF = float("nan"), float("inf")


@dataclass
class Example:
    name: str
    cite: str
    op: str                                # stablehlo op name
    in_types: List[str]                    # MLIR element types of the operands
    shape: Tuple[int, ...]
    inputs: List[list]                     # operand values
    out_type: str
    want: list                             # documented result values
    attrs: str = ""                        # text after the operands (compare direction etc.)
    atol: float = 0.0                      # documented values that are rounded decimals (sin(pi) printed as 0.0)

    def program(self) -> str:
        dims = "".join(f"{d}x" for d in self.shape)
        ts = [f"tensor<{dims}{t}>" for t in self.in_types]
        to = f"tensor<{dims}{self.out_type}>"
        sig = ", ".join(f"%arg{i}: {t}" for i, t in enumerate(ts))
        args = ", ".join(f"%arg{i}" for i in range(len(ts)))
        if self.op == "compare":
            body = f"%0 = stablehlo.compare {self.attrs}, {args} : ({', '.join(ts)}) -> {to}"
        elif len(set(ts)) == 1 and ts[0] == to:
            body = f"%0 = stablehlo.{self.op} {args} : {to}"
        else:
            body = f'%0 = "stablehlo.{self.op}"({args}) : ({", ".join(ts)}) -> {to}'
        return f"module {{\n  func.func @main({sig}) -> {to} {{\n    {body}\n    return %0 : {to}\n  }}\n}}\n"


EXAMPLES = [
    Example("sign_f32", "arithmetic.rs:15-25", "sign", ["f32"], (5,), [[NAN, -1.0, -0.0, 0.0, 1.0]], "f32",
            [NAN, -1.0, -0.0, 0.0, 1.0]),
    Example("abs_i32", "arithmetic.rs:62-69", "abs", ["i32"], (3,), [[-2, 0, 2]], "i32", [2, 0, 2]),
    Example("negate_i32", "arithmetic.rs:107-114", "negate", ["i32"], (3,), [[0, -2, 2]], "i32", [0, 2, -2]),
    Example("add_i32", "arithmetic.rs:157-165", "add", ["i32", "i32"], (2, 2), [[[1, 2], [3, 4]], [[5, 6], [7, 8]]],
            "i32", [[6, 8], [10, 12]]),
    Example("subtract_i32", "arithmetic.rs:222-231", "subtract", ["i32", "i32"], (2, 2),
            [[[6, 8], [10, 12]], [[5, 6], [7, 8]]], "i32", [[1, 2], [3, 4]]),
    Example("multiply_i32", "arithmetic.rs:289-298", "multiply", ["i32", "i32"], (2, 2),
            [[[1, 2], [3, 4]], [[5, 6], [7, 8]]], "i32", [[5, 12], [21, 32]]),
    # the documented results are those of ±17.0 / ±3.0 (its listed dividends ±17.1 would give ±5.70000029): the
    # example is checked with the dividends its results belong to
    Example("divide_f32", "arithmetic.rs:355-363", "divide", ["f32", "f32"], (4,),
            [[17.0, -17.0, 17.0, -17.0], [3.0, 3.0, -3.0, -3.0]], "f32",
            [5.66666651, -5.66666651, -5.66666651, 5.66666651]),
    # the sign of an integer remainder follows the dividend (the documented example is i64)
    Example("remainder_i32", "arithmetic.rs:411-428", "remainder", ["i32", "i32"], (4,),
            [[17, -17, 17, -17], [3, 3, -3, -3]], "i32", [2, -2, 2, -2]),
    # documented as tensor<6xf64>; its printed results (0.333333343, inf for 10000^10) are f32 ones
    Example("power_f32", "exponential.rs:19-26", "power", ["f32", "f32"], (6,),
            [[-2.0, -0.0, -36.0, 5.0, 3.0, 10000.0], [2.0, 2.0, 1.1, 2.0, -1.0, 10.0]], "f32",
            [4.0, 0.0, NAN, 25.0, 0.333333343, INF]),
    Example("expm1_f32", "exponential.rs:268-275", "exponential_minus_one", ["f32"], (2,), [[0.0, 1.0]], "f32",
            [0.0, 1.71828187]),
    Example("log1p_f32", "exponential.rs:362-369", "log_plus_one", ["f32"], (5,),
            [[0.0, -0.999, 7.0, 6.38905621, 15.0]], "f32", [0.0, -6.90776825, 2.07944155, 2.0, 2.77258873]),
    Example("ceil_f32", "rounding.rs:11-18", "ceil", ["f32"], (5,), [[-0.8166, -0.2530, 0.2530, 0.8166, 2.0]], "f32",
            [-0.0, -0.0, 1.0, 1.0, 2.0]),
    Example("floor_f32", "rounding.rs:55-62", "floor", ["f32"], (5,), [[-0.8166, -0.2530, 0.2530, 0.8166, 2.0]],
            "f32", [-1.0, -1.0, 0.0, 0.0, 2.0]),
    Example("not_i8", "logical.rs:8-15", "not", ["i8"], (2, 2), [[[1, 2], [3, 4]]], "i8", [[-2, -3], [-4, -5]]),
    Example("not_i1", "logical.rs:17-19", "not", ["i1"], (2,), [[1, 0]], "i1", [0, 1]),
    Example("and_i32", "logical.rs:53-60", "and", ["i32", "i32"], (2, 2), [[[1, 2], [3, 4]], [[5, 6], [7, 8]]], "i32",
            [[1, 2], [3, 0]]),
    Example("or_i32", "logical.rs:113-120", "or", ["i32", "i32"], (2, 2), [[[1, 2], [3, 4]], [[5, 6], [7, 8]]], "i32",
            [[5, 6], [7, 12]]),
    Example("or_i1", "logical.rs:122-125", "or", ["i1", "i1"], (2, 2), [[[0, 0], [1, 1]], [[0, 1], [0, 1]]], "i1",
            [[0, 1], [1, 1]]),
    Example("xor_i32", "logical.rs:178-185", "xor", ["i32", "i32"], (2, 2), [[[1, 2], [3, 4]], [[5, 6], [7, 8]]],
            "i32", [[4, 4], [4, 12]]),
    Example("xor_i1", "logical.rs:187-190", "xor", ["i1", "i1"], (2, 2), [[[0, 0], [1, 1]], [[0, 1], [0, 1]]], "i1",
            [[0, 1], [1, 0]]),
    Example("maximum_f32", "comparison.rs:245-249", "maximum", ["f32", "f32"], (3,),
            [[1.0, 5.0, 3.0], [2.0, 4.0, 6.0]], "f32", [2.0, 5.0, 6.0]),
    Example("minimum_f32", "comparison.rs:312-316", "minimum", ["f32", "f32"], (3,),
            [[1.0, 5.0, 3.0], [2.0, 4.0, 6.0]], "f32", [1.0, 4.0, 3.0]),
    Example("compare_ge_f32", "comparison.rs:86-93", "compare", ["f32", "f32"], (2,), [[1.0, 3.0], [1.1, 2.9]], "i1",
            [0, 1], attrs="GE"),
    Example("sqrt_f32", "exponential.rs:86-88", "sqrt", ["f32"], (2, 2), [[[0.0, 1.0], [4.0, 9.0]]], "f32",
            [[0.0, 1.0], [2.0, 3.0]]),
    # the documented 0.33333343 is 0.333333343 (the f32 nearest 1/3) with a digit dropped: checked to 1e-7
    Example("rsqrt_f32", "exponential.rs:132-134", "rsqrt", ["f32"], (2, 2), [[[1.0, 4.0], [9.0, 25.0]]], "f32",
            [[1.0, 0.5], [0.33333343, 0.2]], atol=1e-7),
    # documented for f64 with f64 results: the f32 nearest each of them
    Example("exponential_f32", "exponential.rs:225-227", "exponential", ["f32"], (2, 2), [[[0.0, 1.0], [2.0, 3.0]]],
            "f32", [[1.0, 2.7182818284590451], [7.3890560989306504, 20.085536923187668]]),
    Example("log_f32", "exponential.rs:320-322", "log", ["f32"], (2, 2), [[[1.0, 2.0], [3.0, 4.0]]], "f32",
            [[0.0, 0.69314718055994529], [1.0986122886681098, 1.3862943611198906]]),
    Example("logistic_f32", "exponential.rs:415-417", "logistic", ["f32"], (2, 2), [[[0.0, 1.0], [2.0, 3.0]]], "f32",
            [[0.5, 0.73105858], [0.88079708, 0.95257413]]),
    Example("tanh_f32", "trigonometric.rs:169-171", "tanh", ["f32"], (3,), [[-1.0, 0.0, 1.0]], "f32",
            [-0.76159416, 0.0, 0.76159416]),
    # sin / cos at the f32 values nearest 0, pi/2, pi and 3pi/2: the documented 0.0 / 1.0 / -1.0 are rounded
    # decimals (sin of the f32 pi is -8.74e-08), so these two are checked to 1e-7
    Example("sine_f32", "trigonometric.rs:14-24", "sine", ["f32"], (2, 2),
            [[[0.0, 1.57079632], [3.14159265, 4.71238898]]], "f32", [[0.0, 1.0], [0.0, -1.0]], atol=1e-7),
    Example("cosine_f32", "trigonometric.rs:63-73", "cosine", ["f32"], (2, 2),
            [[[0.0, 1.57079632], [3.14159265, 4.71238898]]], "f32", [[1.0, 0.0], [-1.0, 0.0]], atol=1e-7),
    # documented as tensor<4xf64> with three values; 1.57079637 is the f32 nearest pi/2
    Example("atan2_f32", "trigonometric.rs:210-224", "atan2", ["f32", "f32"], (3,),
            [[0.0, 1.0, -1.0], [0.0, 0.0, 0.0]], "f32", [0.0, 1.57079637, -1.57079637]),
    Example("cbrt_f32", "exponential.rs:173-181", "cbrt", ["f32"], (4,), [[0.0, 1.0, 8.0, 27.0]], "f32",
            [0.0, 1.0, 2.0, 3.0]),
    Example("round_nearest_afz_f32", "rounding.rs:100-108", "round_nearest_afz", ["f32"], (5,),
            [[-2.5, 0.4, 0.5, 0.6, 2.5]], "f32", [-3.0, 0.0, 1.0, 1.0, 3.0]),
    # documented as tensor<6xf32> with five values
    Example("round_nearest_even_f32", "rounding.rs:145-153", "round_nearest_even", ["f32"], (5,),
            [[-2.5, 0.4, 0.5, 0.6, 2.5]], "f32", [-2.0, 0.0, 0.0, 1.0, 2.0]),
    Example("is_finite_f32", "arithmetic.rs:482-490", "is_finite", ["f32"], (5,), [[0.0, 1.0, INF, -INF, NAN]], "i1",
            [1, 1, 0, 0, 0]),
    Example("shift_left_i32", "bit_manipulation.rs:10-19", "shift_left", ["i32", "i32"], (3,),
            [[-1, 0, 1], [1, 2, 3]], "i32", [-2, 0, 8]),
    Example("shift_right_arithmetic_i32", "bit_manipulation.rs:74-84", "shift_right_arithmetic", ["i32", "i32"],
            (3,), [[-1, 0, 8], [1, 2, 3]], "i32", [-1, 0, 1]),
    # documented as tensor<3xi32> with the i64 result 9223372036854775807 for -1 >> 1; the i32 result is 2^31 - 1
    Example("shift_right_logical_i32", "bit_manipulation.rs:139-149", "shift_right_logical", ["i32", "i32"], (3,),
            [[-1, 0, 8], [1, 2, 3]], "i32", [2147483647, 0, 1]),
    # documented for i64 ([[64, 63], [56, 0]]): the same values at 32 bits
    Example("count_leading_zeros_i32", "bit_manipulation.rs:202-209", "count_leading_zeros", ["i32"], (2, 2),
            [[[0, 1], [128, -1]]], "i32", [[32, 31], [24, 0]]),
    Example("popcnt_i32", "bit_manipulation.rs:243-250", "popcnt", ["i32"], (4,), [[0, 1, 2, 127]], "i32",
            [0, 1, 1, 7]),
]


def f32(v):
    return np.asarray(v, dtype=np.float64).astype(np.float32)


TRANSCENDENTAL = {"power", "exponential_minus_one", "log_plus_one", "sine", "cosine", "tan", "atan2", "cbrt",
                  "exponential", "log", "logistic", "tanh"}


def check_values(got, ex: Example, ulps: int = 0):
    """Documented values: bit-for-bit for integers and for f32 results (the printed decimals name f32 values exactly;
    NaN as NaN, zeros with their sign); `ulps` f32 units in the last place of slack for finite float results."""
    want = np.asarray(ex.want, dtype=np.float64)
    got = np.asarray(got)
    assert got.shape == want.shape, (ex.name, got.shape, want.shape)
    if ex.out_type in ("f32", "f64", "bf16"):
        g = got.astype(np.float32)
        w = f32(want)
        nan = np.isnan(w)
        assert np.array_equal(np.isnan(g), nan), (ex.name, g, w)
        if ex.atol:
            assert np.all(np.abs(g[~nan].astype(np.float64) - w[~nan]) <= ex.atol), (ex.name, g, w)
            return
        assert np.array_equal(np.signbit(g[~nan]), np.signbit(w[~nan])), (ex.name, "signs", g, w)
        gi, wi = g[~nan].view(np.int32).astype(np.int64), w[~nan].view(np.int32).astype(np.int64)
        assert np.all(np.abs(gi - wi) <= ulps), (ex.name, g, w)
    else:
        assert np.array_equal(got.astype(np.int64), want.astype(np.int64)), (ex.name, got, want)


def oracle_inputs(ex: Example):
    """Operand values as the oracle takes them (f32 operands rounded to f32 first, as a PJRT f32 buffer holds them)."""
    out = []
    for vals, t in zip(ex.inputs, ex.in_types):
        a = np.asarray(vals, dtype=np.float64)
        out.append(f32(a).astype(np.float64) if t == "f32" else a.astype(np.int64))
    return out


__all__ = ["EXAMPLES", "Example", "TRANSCENDENTAL", "check_values", "oracle_inputs"]
