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
]


def f32(v):
    return np.asarray(v, dtype=np.float64).astype(np.float32)


TRANSCENDENTAL = {"power", "exponential_minus_one", "log_plus_one"}


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
