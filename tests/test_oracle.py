"""Pins the CPU oracle before it is trusted as the parity checker.

Each oracle function is checked against something a plausible mistake would fail:
  * dot_general   README KAT [58,64,139,154] (README.md:122-137); brute-force loops over batch / permuted
                  contracting dims; exact int64 for i8→i32.
  * add (i32)     KAT [7,-1]+[35,-41] = [42,-42] (crates/ryft-pjrt/src/programs.rs:2781-2829).
  * narrow floats exhaustive decode of all bf16 / f8E4M3FN codes and random encodes vs torch's CPU dtype casts
                  (third-party, not the reference), plus the f8 overflow edge (448 / 464 / 480).
  * softmax attention  torch scaled_dot_product_attention(is_causal=True) in float64; rows of P sum to one.
  * RMSNorm + SwiGLU   closed form in float64 numpy (independent code path).
  * reduce / broadcast / transpose / iota / compare / select   closed forms on small inputs.
  * op semantics  the reference's documented example of each elementwise op (tests/ref_examples.py: sign of -0.0,
                  remainder signs, power's NaN and overflow, ceil / floor, not / and / or / xor, expm1 / log1p,
                  maximum / minimum, compare); clamp's operand order with all three operands distinct; integer
                  divide / remainder against exact integer arithmetic; float remainder's sign; float → int
                  truncation and int → float rounding; reduce with every body and a non-neutral init; compare in
                  every direction with a NaN operand.
"""
import math

import numpy as np
import pytest
import torch

from oracle import numerics as nm
from oracle import stablehlo as sh
from ryft_amd import configs
from ryft_amd import hostdata as hd


def _mod(args, ret, body):
    sig = ", ".join(f"%arg{i}: {t}" for i, t in enumerate(args))
    return f"module {{\n  func.func @main({sig}) -> {ret} {{\n{body}\n  }}\n}}\n"


def test_readme_dot_kat():
    prog = _mod(["tensor<2x3xf32>", "tensor<3x2xf32>"], "tensor<2x2xf32>",
                "    %0 = stablehlo.dot_general %arg0, %arg1, contracting_dims = [1] x [0] : "
                "(tensor<2x3xf32>, tensor<3x2xf32>) -> tensor<2x2xf32>\n    return %0 : tensor<2x2xf32>")
    (out, dt), = sh.evaluate(prog, [np.array([[1., 2, 3], [4, 5, 6]]), np.array([[7., 8], [9, 10], [11, 12]])])
    assert dt == "f32"
    assert out.ravel().tolist() == [58.0, 64.0, 139.0, 154.0]


def test_add_kat():
    prog = _mod(["tensor<2xi32>", "tensor<2xi32>"], "tensor<2xi32>",
                "    %0 = stablehlo.add %arg0, %arg1 : tensor<2xi32>\n    return %0 : tensor<2xi32>")
    (out, _), = sh.evaluate(prog, [np.array([7, -1]), np.array([35, -41])])
    assert out.tolist() == [42, -42]


def test_dot_general_brute_force_batch_and_permuted_contraction():
    rng = np.random.default_rng(0)
    a = rng.integers(-5, 6, (3, 4, 2, 5)).astype(float)  # [b, k1, m, k2]
    b = rng.integers(-5, 6, (5, 3, 6, 4)).astype(float)  # [k2, b, n, k1]
    prog = _mod(["tensor<3x4x2x5xf32>", "tensor<5x3x6x4xf32>"], "tensor<3x2x6xf32>",
                "    %0 = stablehlo.dot_general %arg0, %arg1, batching_dims = [0] x [1], contracting_dims = [1, 3] x [3, 0]"
                " : (tensor<3x4x2x5xf32>, tensor<5x3x6x4xf32>) -> tensor<3x2x6xf32>\n    return %0 : tensor<3x2x6xf32>")
    (out, _), = sh.evaluate(prog, [a, b])
    want = np.zeros((3, 2, 6))
    for bb in range(3):
        for m in range(2):
            for n in range(6):
                for k1 in range(4):
                    for k2 in range(5):
                        want[bb, m, n] += a[bb, k1, m, k2] * b[k2, bb, n, k1]
    assert np.array_equal(out, want)


def test_int8_dot_exact():
    w = configs.c3_int8_gemm(m=64, k=96, n=32)
    a, b = w.inputs[0].data.astype(np.int64), w.inputs[1].data.astype(np.int64)
    outs = sh.evaluate(w.program, [sh.from_raw(x.data, t) for x, t in zip(w.inputs, ["i8", "i8", "f32", "f32"])])
    assert outs[0][1] == "i32"
    assert np.array_equal(outs[0][0], a @ b)
    scaled = (a @ b).astype(np.float64) * w.inputs[2].data.astype(np.float64) * w.inputs[3].data.astype(np.float64)
    assert sh.rel_error(outs[1][0], scaled) < 1e-6


def test_bf16_decode_exhaustive_vs_torch():
    codes = np.arange(1 << 16, dtype=np.uint16)
    want = torch.from_numpy(codes.view(np.int16)).view(torch.bfloat16).float().numpy().astype(np.float64)
    got = nm.decode_bits(codes, "bf16")
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[~np.isnan(got)], want[~np.isnan(want)])


def test_f8e4m3fn_decode_exhaustive_vs_torch():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    got = nm.decode_bits(codes, "f8E4M3FN")
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[~np.isnan(got)], want[~np.isnan(want)])
    assert np.nanmax(got) == 448.0


@pytest.mark.parametrize("dtype,torch_dtype,scale", [("bf16", torch.bfloat16, 1e3), ("f8E4M3FN", torch.float8_e4m3fn, 30.0),
                                                     ("f16", torch.float16, 1e2)])
def test_encode_random_vs_torch(dtype, torch_dtype, scale):
    x = hd.normal(7, (300000,), 0.0, scale)
    edges = np.array([448, 460, 464, 465, 479, 480, 500, 1e6, -464, -470, 2 ** -10, 1.5 * 2 ** -9, 3 * 2 ** -10, 0.0,
                      -0.0, 65504, 65520, 65536], dtype=np.float32)
    x = np.concatenate([x, edges]).astype(np.float32)
    bits = torch.from_numpy(x).to(torch_dtype)
    want = bits.view(torch.uint8 if torch_dtype == torch.float8_e4m3fn else torch.int16).numpy()
    got = nm.encode_bits(x, dtype)
    assert np.array_equal(got.view(want.dtype), want)


def test_product_encoders_agree_with_oracle():
    x = np.concatenate([hd.normal(9, (200000,), 0.0, 50.0), np.array([464, 470, -1e9, 1e-12], np.float32)])
    assert np.array_equal(hd.f32_to_bf16_bits(x), nm.encode_bits(x, "bf16"))
    assert np.array_equal(hd.f32_to_e4m3fn_bits(x), nm.encode_bits(x, "f8E4M3FN"))
    codes = np.arange(256, dtype=np.uint8)
    a, b = hd.e4m3fn_bits_to_f32(codes), nm.decode_bits(codes, "f8E4M3FN")
    assert np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(a[~np.isnan(a)], b[~np.isnan(b)])


def test_causal_attention_vs_torch_sdpa():
    w = configs.c4_causal_attention(b=1, h=2, s=128, d=64)
    ins = [sh.from_raw(x.data, "bf16") for x in w.inputs]
    (out, dt), = sh.evaluate(w.program, ins)
    assert dt == "bf16"
    q, k, v = (torch.from_numpy(x) for x in ins)
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True).numpy()
    assert sh.rel_error(out, ref) < 1e-2
    # row 0 attends only to key 0: output row 0 = bf16(V[0])
    assert np.array_equal(out[:, :, 0, :], nm.round_to(ins[2][:, :, 0, :], "bf16"))


def test_rmsnorm_swiglu_closed_form():
    m, d, f = 16, 64, 96
    w = configs.c5_swiglu_fp8(m=m, d=d, f=f, activations="bf16")
    ins = [sh.from_raw(x.data, t) for x, t in zip(w.inputs, ["bf16", "bf16", "f8E4M3FN", "f32", "f8E4M3FN", "f32",
                                                               "f8E4M3FN", "f32"])]
    (out, _), = sh.evaluate(w.program, ins)
    x, g, wg, sg, wu, su, wd, sd = ins
    xn = x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + 1e-6) * g[None, :]
    xn = nm.round_to(xn, "bf16")
    gg = (xn @ wg) * sg
    uu = (xn @ wu) * su
    h = nm.round_to(gg / (1 + np.exp(-gg)) * uu, "bf16")
    ref = (h @ wd) * sd
    assert sh.rel_error(out, ref) < 1e-2


def test_reduce_broadcast_transpose_iota_select():
    prog = _mod(["tensor<3x4xf32>"], "(tensor<3xf32>, tensor<4x3xf32>, tensor<3x4xf32>)", """
    %cst = stablehlo.constant dense<0.000000e+00> : tensor<f32>
    %0 = stablehlo.reduce(%arg0 init: %cst) applies stablehlo.add across dimensions = [1] : (tensor<3x4xf32>, tensor<f32>) -> tensor<3xf32>
    %1 = stablehlo.transpose %arg0, dims = [1, 0] : (tensor<3x4xf32>) -> tensor<4x3xf32>
    %2 = stablehlo.iota dim = 0 : tensor<3x4xi32>
    %3 = stablehlo.iota dim = 1 : tensor<3x4xi32>
    %4 = stablehlo.compare  LE, %3, %2,  SIGNED : (tensor<3x4xi32>, tensor<3x4xi32>) -> tensor<3x4xi1>
    %5 = stablehlo.broadcast_in_dim %0, dims = [0] : (tensor<3xf32>) -> tensor<3x4xf32>
    %6 = stablehlo.select %4, %arg0, %5 : tensor<3x4xi1>, tensor<3x4xf32>
    return %0, %1, %6 : tensor<3xf32>, tensor<4x3xf32>, tensor<3x4xf32>""")
    x = np.arange(12, dtype=float).reshape(3, 4)
    (r, _), (t, _), (s, _) = sh.evaluate(prog, [x])
    assert r.tolist() == x.sum(1).tolist()
    assert np.array_equal(t, x.T)
    want = np.where(np.arange(4)[None, :] <= np.arange(3)[:, None], x, x.sum(1)[:, None])
    assert np.array_equal(s, want)


def test_broadcast_in_dim_permuting_dims():
    # manipulation.rs:305 example: [1,3] → [2,3,2] with dims = [2, 1]
    prog = _mod(["tensor<1x3xi32>"], "tensor<2x3x2xi32>", """
    %0 = stablehlo.broadcast_in_dim %arg0, dims = [2, 1] : (tensor<1x3xi32>) -> tensor<2x3x2xi32>
    return %0 : tensor<2x3x2xi32>""")
    (out, _), = sh.evaluate(prog, [np.array([[1, 2, 3]])])
    want = np.array([[[1, 1], [2, 2], [3, 3]], [[1, 1], [2, 2], [3, 3]]])
    assert np.array_equal(out, want)


def test_pad_concatenate_slice_reference_examples():
    # the worked examples in ryft-mlir's documentation of each builder (manipulation.rs:549-570, 772-781, 848-864)
    pad = _mod(["tensor<2x3xi32>", "tensor<i32>"], "tensor<5x9xi32>", """
    %0 = stablehlo.pad %arg0, %arg1, low = [0, 1], high = [2, 1], interior = [1, 2] : (tensor<2x3xi32>, tensor<i32>) -> tensor<5x9xi32>
    return %0 : tensor<5x9xi32>""")
    (out, _), = sh.evaluate(pad, [np.array([[1, 2, 3], [4, 5, 6]]), np.array(0)])
    assert out.tolist() == [[0, 1, 0, 0, 2, 0, 0, 3, 0], [0] * 9, [0, 4, 0, 0, 5, 0, 0, 6, 0], [0] * 9, [0] * 9]
    cat = _mod(["tensor<3x2xi64>", "tensor<1x2xi64>"], "tensor<4x2xi64>", """
    %0 = stablehlo.concatenate %arg0, %arg1, dim = 0 : (tensor<3x2xi64>, tensor<1x2xi64>) -> tensor<4x2xi64>
    return %0 : tensor<4x2xi64>""")
    (out, _), = sh.evaluate(cat, [np.array([[1, 2], [3, 4], [5, 6]]), np.array([[7, 8]])])
    assert out.tolist() == [[1, 2], [3, 4], [5, 6], [7, 8]]
    sl = _mod(["tensor<3x4xi64>"], "tensor<2x2xi64>", """
    %0 = stablehlo.slice %arg0 [1:3, 2:4] : (tensor<3x4xi64>) -> tensor<2x2xi64>
    return %0 : tensor<2x2xi64>""")
    (out, _), = sh.evaluate(sl, [np.array([[0, 0, 0, 0], [0, 0, 1, 1], [0, 0, 1, 1]])])
    assert out.tolist() == [[1, 1], [1, 1]]


@pytest.mark.parametrize("shape,lo,hi,interior", [((3, 4), (2, -1), (-2, 3), (0, 1)), ((5,), (-3,), (-4,), (2,)),
                                                  ((2, 3, 2), (1, 0, -1), (0, 2, -1), (1, 0, 3)),
                                                  ((4, 1), (-4, 0), (1, 0), (0, 0))])
def test_pad_matches_the_index_formula(shape, lo, hi, interior):
    # the builder documentation's definition (manipulation.rs:544-546): result[lo + i·(interior + 1)] = operand[i]
    # where that index lies in the result, the padding value elsewhere; checked element by element against the
    # oracle's interior-then-edges construction, including negative edges that cut interior padding
    out_shape = tuple(l + h + k + (k - 1) * it for k, l, h, it in zip(shape, lo, hi, interior))
    t = "tensor<" + "x".join(map(str, shape)) + "xi32>"
    ot = "tensor<" + "x".join(map(str, out_shape)) + "xi32>"
    prog = _mod([t, "tensor<i32>"], ot, f"""
    %0 = stablehlo.pad %arg0, %arg1, low = {list(lo)}, high = {list(hi)}, interior = {list(interior)} : ({t}, tensor<i32>) -> {ot}
    return %0 : {ot}""")
    x = np.arange(1, 1 + int(np.prod(shape))).reshape(shape)
    (out, _), = sh.evaluate(prog, [x, np.array(-7)])
    want = np.full(out_shape, -7)
    for idx in np.ndindex(*shape):
        pos = tuple(l + i * (it + 1) for l, i, it in zip(lo, idx, interior))
        if all(0 <= p < n for p, n in zip(pos, out_shape)):
            want[pos] = x[idx]
    assert np.array_equal(out, want)


# ----------------------------------------------------------------------------------------------- op semantics
from tests.ref_examples import EXAMPLES, check_values, oracle_inputs  # noqa: E402


@pytest.mark.parametrize("ex", EXAMPLES, ids=[e.name for e in EXAMPLES])
def test_reference_worked_examples(ex):
    """The reference's documented example of each op (tests/ref_examples.py cites file:line) gives the documented
    result: pins sign conventions (remainder, sign of -0.0, ceil of small negatives), operand order of the binary
    ops, NaN production (power of a negative base) and overflow (10000^10 in f32)."""
    (out, dt), = sh.evaluate(ex.program(), oracle_inputs(ex))
    assert dt == ex.out_type
    check_values(out, ex)


def _eval1(prog, *vals):
    (out, dt), = sh.evaluate(prog, [np.asarray(v) for v in vals])
    return out


def test_clamp_operand_order():
    # comparison.rs:166-176: `clamp %min, %operand, %max` bounds the middle operand. With min / operand / max all
    # different, swapping any two of them changes the result.
    T = "tensor<3xi32>"
    prog = _mod([T, T, T], T, f"    %0 = stablehlo.clamp %arg0, %arg1, %arg2 : {T}\n    return %0 : {T}")
    assert _eval1(prog, [5, 10, 15], [3, 13, 23], [10, 15, 20]).tolist() == [5, 13, 20]
    F, S = "tensor<4xf32>", "tensor<f32>"
    prog = _mod([S, F, S], F, f"    %0 = stablehlo.clamp %arg0, %arg1, %arg2 : ({S}, {F}, {S}) -> {F}\n    return %0 : {F}")
    out = _eval1(prog, np.float64(-1.0), [-3.0, -0.5, 0.5, 3.0], np.float64(1.0))
    assert out.tolist() == [-1.0, -0.5, 0.5, 1.0]


def test_integer_divide_and_remainder_truncate_toward_zero():
    # brute force against Python's exact integer arithmetic: q = sign(a)·sign(b)·(|a| // |b|), r = a - q·b
    T = "tensor<451xi32>"
    a, b = np.meshgrid(np.arange(-20, 21), np.array([v for v in range(-6, 7) if v != 0]))
    a, b = a.ravel()[:451], b.ravel()[:451]
    q_prog = _mod([T, T], T, f"    %0 = stablehlo.divide %arg0, %arg1 : {T}\n    return %0 : {T}")
    r_prog = _mod([T, T], T, f"    %0 = stablehlo.remainder %arg0, %arg1 : {T}\n    return %0 : {T}")
    q, r = _eval1(q_prog, a, b), _eval1(r_prog, a, b)
    for x, y, qq, rr in zip(a.tolist(), b.tolist(), q.tolist(), r.tolist()):
        want_q = (1 if (x >= 0) == (y > 0) else -1) * (abs(x) // abs(y))
        assert qq == want_q and rr == x - want_q * y, (x, y, qq, rr)
    # i32 wraparound of the one overflowing quotient, INT_MIN / -1
    T1 = "tensor<1xi32>"
    prog = _mod([T1, T1], T1, f"    %0 = stablehlo.divide %arg0, %arg1 : {T1}\n    return %0 : {T1}")
    assert _eval1(prog, [-2 ** 31], [-1]).tolist() == [-2 ** 31]


def test_float_remainder_sign_follows_dividend():
    # the result has the dividend's sign and a magnitude below the divisor's (fmod), not IEEE round-to-nearest
    # remainder: 17.1 rem 3 is 2.1, never -0.9
    T = "tensor<4xf32>"
    prog = _mod([T, T], T, f"    %0 = stablehlo.remainder %arg0, %arg1 : {T}\n    return %0 : {T}")
    a = np.float32([17.1, -17.1, 17.1, -17.1]).astype(np.float64)
    out = _eval1(prog, a, [3.0, 3.0, -3.0, -3.0])
    want = np.float32(np.float32(17.1) - np.float32(15.0))  # exact: 15 is a multiple of 3 below 17.1
    assert out.tolist() == [want, -want, want, -want]


def test_convert_float_to_int_truncates_toward_zero():
    F, I = "tensor<6xf32>", "tensor<6xi32>"
    prog = _mod([F], I, f"    %0 = stablehlo.convert %arg0 : ({F}) -> {I}\n    return %0 : {I}")
    assert _eval1(prog, [-2.7, -0.5, -0.0, 0.5, 2.7, 100.9]).tolist() == [-2, 0, 0, 0, 2, 100]
    # integer → f32 rounds to nearest even: 2^24 + 1 is halfway between 2^24 and 2^24 + 2
    I1, F1 = "tensor<2xi32>", "tensor<2xf32>"
    prog = _mod([I1], F1, f"    %0 = stablehlo.convert %arg0 : ({I1}) -> {F1}\n    return %0 : {F1}")
    assert _eval1(prog, [2 ** 24 + 1, 2 ** 24 + 3]).tolist() == [2.0 ** 24, 2.0 ** 24 + 4]


def test_reduce_bodies_and_init_values():
    # functional.rs:121-129: [[0, 1, 2, 3, 4, 5]] summed from 0 is [15]
    def red(body, init, vals, dt="i32"):
        T, R, S = f"tensor<1x{len(vals)}x{dt}>", f"tensor<1x{dt}>", f"tensor<{dt}>"
        prog = _mod([T, S], R, f"    %0 = stablehlo.reduce(%arg0 init: %arg1) applies stablehlo.{body} across "
                               f"dimensions = [1] : ({T}, {S}) -> {R}\n    return %0 : {R}")
        return _eval1(prog, np.asarray([vals]), np.asarray(init)).tolist()[0]
    assert red("add", 0, [0, 1, 2, 3, 4, 5]) == 15
    assert red("add", 100, [0, 1, 2, 3, 4, 5]) == 115           # the init value takes part
    assert red("multiply", 1, [1, 2, 3, 4, 5]) == 120
    assert red("multiply", 2, [1, 2, 3, 4, 5]) == 240
    assert red("maximum", 0, [-5, -3, -9]) == 0                  # init above every element
    assert red("maximum", -100, [-5, -3, -9]) == -3
    assert red("minimum", 0, [5, 3, 9]) == 0
    assert red("minimum", 100, [5, 3, 9]) == 3
    assert red("and", -1, [0b1110, 0b0111]) == 0b0110
    assert red("and", 0b0010, [0b1110, 0b0111]) == 0b0010
    assert red("or", 0, [0b1000, 0b0001]) == 0b1001
    assert red("or", 0b0100, [0b1000, 0b0001]) == 0b1101
    assert red("multiply", 1.0, [2.0, -0.5, 3.0], "f32") == -3.0


def test_compare_directions_and_nan():
    T, P = "tensor<4xf32>", "tensor<4xi1>"
    a, b = [1.0, 2.0, 3.0, float("nan")], [2.0, 2.0, 2.0, 2.0]
    want = {"EQ": [0, 1, 0, 0], "NE": [1, 0, 1, 1], "LT": [1, 0, 0, 0], "LE": [1, 1, 0, 0], "GT": [0, 0, 1, 0],
            "GE": [0, 1, 1, 0]}
    for d, w in want.items():
        prog = _mod([T, T], P, f"    %0 = stablehlo.compare  {d}, %arg0, %arg1,  FLOAT : ({T}, {T}) -> {P}\n"
                               f"    return %0 : {P}")
        assert _eval1(prog, a, b).tolist() == w, d


def test_sign_of_integers_and_not_of_bits():
    I = "tensor<5xi32>"
    prog = _mod([I], I, f"    %0 = stablehlo.sign %arg0 : {I}\n    return %0 : {I}")
    assert _eval1(prog, [-7, -1, 0, 1, 9]).tolist() == [-1, -1, 0, 1, 1]
    prog = _mod([I], I, f"    %0 = stablehlo.not %arg0 : {I}\n    return %0 : {I}")
    assert _eval1(prog, [0, -1, 5, 2 ** 31 - 1, -2 ** 31]).tolist() == [-1, 0, -6, -2 ** 31, 2 ** 31 - 1]
