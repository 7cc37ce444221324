"""StableHLO programs whose reductions over the innermost dim feed back into an elementwise consumer (RMSNorm,
LayerNorm, softmax, an integer row maximum): the shapes the planner runs as one row-fused launch. Shared by the CPU
plan tests and the GPU parity tests."""
from __future__ import annotations


def _t(shape, dt="f32"):
    return "tensor<" + "".join(f"{s}x" for s in shape) + dt + ">"


def _module(args, ret, body):
    sig = ", ".join(f"%arg{i}: {t}" for i, t in enumerate(args))
    return f"module {{\n  func.func @main({sig}) -> {ret} {{\n{body}\n  }}\n}}\n"


def _lit(x):
    return f"{x:.9e}"


def rmsnorm(shape, dt="f32", eps=1e-6, quant=None):
    """y = x · rsqrt(mean(x²) + eps) · w, computed in f32, result in `dt` (then converted to `quant`, e.g.
    f8E4M3FN, when given: C5's normalise-and-quantise step)."""
    *outer, d = shape
    X, XF, W, WF = _t(shape, dt), _t(shape), _t((d,), dt), _t((d,))
    R = _t(outer)
    od = list(range(len(outer)))
    body = f"""    %0 = stablehlo.convert %arg0 : ({X}) -> {XF}
    %1 = stablehlo.multiply %0, %0 : {XF}
    %cst = stablehlo.constant dense<0.000000e+00> : tensor<f32>
    %2 = stablehlo.reduce(%1 init: %cst) applies stablehlo.add across dimensions = [{len(outer)}] : ({XF}, tensor<f32>) -> {R}
    %cst_0 = stablehlo.constant dense<{_lit(1.0 / d)}> : tensor<f32>
    %3 = stablehlo.broadcast_in_dim %cst_0, dims = [] : (tensor<f32>) -> {R}
    %4 = stablehlo.multiply %2, %3 : {R}
    %cst_1 = stablehlo.constant dense<{_lit(eps)}> : tensor<f32>
    %5 = stablehlo.broadcast_in_dim %cst_1, dims = [] : (tensor<f32>) -> {R}
    %6 = stablehlo.add %4, %5 : {R}
    %7 = stablehlo.rsqrt %6 : {R}
    %8 = stablehlo.broadcast_in_dim %7, dims = {od} : ({R}) -> {XF}
    %9 = stablehlo.multiply %0, %8 : {XF}
    %10 = stablehlo.convert %arg1 : ({W}) -> {WF}
    %11 = stablehlo.broadcast_in_dim %10, dims = [{len(outer)}] : ({WF}) -> {XF}
    %12 = stablehlo.multiply %9, %11 : {XF}
    %13 = stablehlo.convert %12 : ({XF}) -> {X}"""
    if quant is None:
        return _module([X, W], X, body + f"\n    return %13 : {X}")
    Q = _t(shape, quant)
    return _module([X, W], Q, body + f"\n    %14 = stablehlo.convert %13 : ({X}) -> {Q}\n    return %14 : {Q}")


def softmax(shape):
    """Row softmax in f32 written out as reduce-max, subtract, exp, reduce-sum, divide (two chained reductions)."""
    *outer, d = shape
    T, R = _t(shape), _t(outer)
    od = list(range(len(outer)))
    last = len(outer)
    body = f"""    %cst = stablehlo.constant dense<0xFF800000> : tensor<f32>
    %0 = stablehlo.reduce(%arg0 init: %cst) applies stablehlo.maximum across dimensions = [{last}] : ({T}, tensor<f32>) -> {R}
    %1 = stablehlo.broadcast_in_dim %0, dims = {od} : ({R}) -> {T}
    %2 = stablehlo.subtract %arg0, %1 : {T}
    %3 = stablehlo.exponential %2 : {T}
    %cst_0 = stablehlo.constant dense<0.000000e+00> : tensor<f32>
    %4 = stablehlo.reduce(%3 init: %cst_0) applies stablehlo.add across dimensions = [{last}] : ({T}, tensor<f32>) -> {R}
    %5 = stablehlo.broadcast_in_dim %4, dims = {od} : ({R}) -> {T}
    %6 = stablehlo.divide %3, %5 : {T}
    return %6 : {T}"""
    return _module([T], T, body)


def layernorm(shape, eps=1e-5):
    """(x − mean) · rsqrt(var + eps) · γ + β with var = mean((x − mean)²), f32."""
    *outer, d = shape
    T, R, V = _t(shape), _t(outer), _t((d,))
    od = list(range(len(outer)))
    last = len(outer)
    body = f"""    %cst = stablehlo.constant dense<0.000000e+00> : tensor<f32>
    %0 = stablehlo.reduce(%arg0 init: %cst) applies stablehlo.add across dimensions = [{last}] : ({T}, tensor<f32>) -> {R}
    %cst_0 = stablehlo.constant dense<{_lit(1.0 / d)}> : tensor<f32>
    %1 = stablehlo.broadcast_in_dim %cst_0, dims = [] : (tensor<f32>) -> {R}
    %2 = stablehlo.multiply %0, %1 : {R}
    %3 = stablehlo.broadcast_in_dim %2, dims = {od} : ({R}) -> {T}
    %4 = stablehlo.subtract %arg0, %3 : {T}
    %5 = stablehlo.multiply %4, %4 : {T}
    %6 = stablehlo.reduce(%5 init: %cst) applies stablehlo.add across dimensions = [{last}] : ({T}, tensor<f32>) -> {R}
    %7 = stablehlo.multiply %6, %1 : {R}
    %cst_1 = stablehlo.constant dense<{_lit(eps)}> : tensor<f32>
    %8 = stablehlo.broadcast_in_dim %cst_1, dims = [] : (tensor<f32>) -> {R}
    %9 = stablehlo.add %7, %8 : {R}
    %10 = stablehlo.rsqrt %9 : {R}
    %11 = stablehlo.broadcast_in_dim %10, dims = {od} : ({R}) -> {T}
    %12 = stablehlo.multiply %4, %11 : {T}
    %13 = stablehlo.broadcast_in_dim %arg1, dims = [{last}] : ({V}) -> {T}
    %14 = stablehlo.multiply %12, %13 : {T}
    %15 = stablehlo.broadcast_in_dim %arg2, dims = [{last}] : ({V}) -> {T}
    %16 = stablehlo.add %14, %15 : {T}
    return %16 : {T}"""
    return _module([T, V, V], T, body)


def int_row_max_gap(shape):
    """max over each i32 row minus every element (integer class, bit-exact), plus the row maxima as a 2nd result."""
    *outer, d = shape
    T, R = _t(shape, "i32"), _t(outer, "i32")
    od = list(range(len(outer)))
    last = len(outer)
    body = f"""    %cst = stablehlo.constant dense<-2147483648> : tensor<i32>
    %0 = stablehlo.reduce(%arg0 init: %cst) applies stablehlo.maximum across dimensions = [{last}] : ({T}, tensor<i32>) -> {R}
    %1 = stablehlo.broadcast_in_dim %0, dims = {od} : ({R}) -> {T}
    %2 = stablehlo.subtract %1, %arg0 : {T}
    return %2, %0 : {T}, {R}"""
    return _module([T], f"({T}, {R})", body)
