"""GPU coverage of the generic kernels (elementwise programs, reductions, transposes, iota / compare / select,
conversions, the generic GEMM) against the oracle on small shapes.

Shapes with an innermost extent of 33 run the one-element-per-thread kernels; extents that are multiples of 8 run
the 8-wide kernels (vector loads / stores, broadcast and strided leaves), and rows of ≥1024 elements the
workgroup-per-row reduction."""
import numpy as np
import pytest

from oracle import numerics, stablehlo as sh
from ryft_amd import configs, hostdata as hd, pjrt
from tests.helpers import check, oracle_outputs, run_pjrt

pytestmark = pytest.mark.gpu


def _mod(args, rets, body):
    sig = ", ".join(f"%arg{i}: {t}" for i, t in enumerate(args))
    ret = rets[0] if len(rets) == 1 else "(" + ", ".join(rets) + ")"
    return f"module {{\n  func.func @main({sig}) -> {ret} {{\n{body}\n  }}\n}}\n"


F = "tensor<8x33xf32>"
SHAPES = [(8, 33), (6, 64)]


def _t(shape, dt="f32"):
    return "tensor<" + "".join(f"{s}x" for s in shape) + dt + ">"


def _f32_inputs(n, shape=(8, 33), seed=1):
    return [configs.HostInput(hd.normal(seed + i, shape), pjrt.BufferType.F32, shape) for i in range(n)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("op", ["add", "subtract", "multiply", "divide", "maximum", "minimum"])
def test_binary_f32(gpu_client, op, shape):
    T = _t(shape)
    prog = _mod([T, T], [T], f"    %0 = stablehlo.{op} %arg0, %arg1 : {T}\n    return %0 : {T}")
    ins = _f32_inputs(2, shape)
    outs, _ = run_pjrt(gpu_client, prog, ins)
    check(outs[0], oracle_outputs(prog, ins)[0], 1e-6, op)


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("op", ["exponential", "log", "rsqrt", "sqrt", "tanh", "logistic", "negate", "abs", "floor"])
def test_unary_f32(gpu_client, op, shape):
    T = _t(shape)
    prog = _mod([T], [T], f"    %0 = stablehlo.abs %arg0 : {T}\n    %1 = stablehlo.{op} %0 : {T}\n    return %1 : {T}")
    ins = _f32_inputs(1, shape)
    outs, _ = run_pjrt(gpu_client, prog, ins)
    check(outs[0], oracle_outputs(prog, ins)[0], 2e-6, op)


def test_int_ops_and_wraparound(gpu_client):
    T = "tensor<64xi32>"
    body = f"""    %0 = stablehlo.multiply %arg0, %arg1 : {T}
    %1 = stablehlo.add %0, %arg0 : {T}
    %2 = stablehlo.divide %1, %arg1 : {T}
    %3 = stablehlo.remainder %1, %arg1 : {T}
    %4 = stablehlo.maximum %2, %3 : {T}
    %5 = stablehlo.convert %4 : ({T}) -> tensor<64xi8>
    return %1, %5 : {T}, tensor<64xi8>"""
    prog = _mod([T, T], [T, "tensor<64xi8>"], body)
    a = hd.int_uniform(3, (64,), -2 ** 30, 2 ** 30).astype(np.int32)
    b = hd.int_uniform(4, (64,), 1, 1000).astype(np.int32) * np.where(np.arange(64) % 2, 1, -1).astype(np.int32)
    ins = [configs.HostInput(a, pjrt.BufferType.S32, (64,)), configs.HostInput(b, pjrt.BufferType.S32, (64,))]
    outs, _ = run_pjrt(gpu_client, prog, ins)
    for o, w in zip(outs, oracle_outputs(prog, ins)):
        check(o, w, 0, "int")


@pytest.mark.parametrize("shape", SHAPES)
def test_convert_chain_bf16_f8(gpu_client, shape):
    F, B, E, I = _t(shape), _t(shape, "bf16"), _t(shape, "f8E4M3FN"), _t(shape, "i32")
    body = f"""    %0 = stablehlo.convert %arg0 : ({F}) -> {B}
    %1 = stablehlo.convert %0 : ({B}) -> {E}
    %2 = stablehlo.convert %arg0 : ({F}) -> {I}
    %3 = stablehlo.convert %1 : ({E}) -> {F}
    return %0, %1, %2, %3 : {B}, {E}, {I}, {F}"""
    prog = _mod([F], [B, E, I, F], body)
    n = shape[0] * shape[1]
    x = np.concatenate([hd.normal(5, (n - 6,), 0, 100), np.array([464, 470, -500, 1e-3, 2.5, -2.5])])
    ins = [configs.HostInput(x.astype(np.float32).reshape(shape), pjrt.BufferType.F32, shape)]
    outs, _ = run_pjrt(gpu_client, prog, ins)
    for i, (o, w) in enumerate(zip(outs, oracle_outputs(prog, ins))):
        # conversions are exact: compare bits
        assert np.array_equal(np.asarray(o).view(np.uint8), sh.to_raw(w[0], w[1]).view(np.uint8)) or \
            np.array_equal(np.isnan(sh.from_raw(o, w[1])), np.isnan(w[0])), f"convert output {i}"


@pytest.mark.parametrize("shape", [(4, 64), (8, 33)])
def test_convert_f32_to_f8e4m3fn_special_values_bits(gpu_client, shape):
    # every special value in every byte position of a packed 4-byte group (the 8-wide store converts pairs and fixes
    # NaN signs only for groups holding a 0x7f / 0xff byte): NaNs of both signs, infinities, the overflow boundary
    # (464 rounds to 448, anything above is NaN), ±0, subnormals and their ties, mixed with ordinary values
    specials = np.array([0x7fc00000, 0xffc00000, 0x7f800001, 0x7f800000, 0xff800000], np.uint32).view(np.float32)
    specials = np.concatenate([specials, np.array([448, 449, 463.99, 464, 464.01, -464, -465, 0.0, -0.0, 2.0 ** -9,
                                                   2.0 ** -10, 3 * 2.0 ** -10, -2.0 ** -10, 1e-30, 1.5, -2.5],
                                                  np.float32)])
    n = shape[0] * shape[1]
    x = hd.normal(7, (n,), 0, 50).astype(np.float32)
    for i, v in enumerate(specials):  # special i at 13·i + 5·j, j = 0..3: once in each byte position of a 4-group
        for j in range(4):
            pos = (i * 13 + j * 5) % n
            x[pos] = v
    T, E = _t(shape), _t(shape, "f8E4M3FN")
    prog = _mod([T], [E], f"    %0 = stablehlo.convert %arg0 : ({T}) -> {E}\n    return %0 : {E}")
    ins = [configs.HostInput(x.reshape(shape), pjrt.BufferType.F32, shape)]
    outs, _ = run_pjrt(gpu_client, prog, ins)
    got = np.asarray(outs[0]).view(np.uint8).reshape(-1)
    # the oracle's encoder on the f32 inputs (its decoded float64 values would not keep a NaN's sign)
    ref = numerics._encode(x.astype(np.float64), "f8E4M3FN").astype(np.uint8)
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, [(float(x[i]), hex(got[i]), hex(ref[i])) for i in bad[:8]]


@pytest.mark.parametrize("shape", SHAPES + [(5, 2048)])
@pytest.mark.parametrize("dims,body", [([1], "add"), ([0], "add"), ([0, 1], "maximum"), ([1], "minimum")])
def test_reduce(gpu_client, dims, body, shape):
    F = _t(shape)
    out_shape = [s for i, s in enumerate(shape) if i not in dims]
    ot = _t(out_shape)
    init = "0.000000e+00" if body == "add" else ("0xFF800000" if body == "maximum" else "0x7F800000")
    prog = _mod([F], [ot], f"""    %cst = stablehlo.constant dense<{init}> : tensor<f32>
    %0 = stablehlo.reduce(%arg0 init: %cst) applies stablehlo.{body} across dimensions = {dims} : ({F}, tensor<f32>) -> {ot}
    return %0 : {ot}""")
    ins = _f32_inputs(1, shape)
    outs, _ = run_pjrt(gpu_client, prog, ins)
    check(outs[0], oracle_outputs(prog, ins)[0], 1e-6, "reduce")


@pytest.mark.parametrize("cols", [64, 4096])
def test_rmsnorm_rows_bf16(gpu_client, cols):
    # reduce with a fused prologue over bf16 rows (wavefront-per-row and workgroup-per-row reductions), then a
    # broadcast row statistic applied by the elementwise kernel
    X, R, XF = _t((6, cols), "bf16"), _t((6,)), _t((6, cols))
    body = f"""    %0 = stablehlo.convert %arg0 : ({X}) -> {XF}
    %1 = stablehlo.multiply %0, %0 : {XF}
    %cst = stablehlo.constant dense<0.000000e+00> : tensor<f32>
    %2 = stablehlo.reduce(%1 init: %cst) applies stablehlo.add across dimensions = [1] : ({XF}, tensor<f32>) -> {R}
    %c = stablehlo.constant dense<{1.0 / cols:e}> : {R}
    %3 = stablehlo.multiply %2, %c : {R}
    %4 = stablehlo.rsqrt %3 : {R}
    %5 = stablehlo.broadcast_in_dim %4, dims = [0] : ({R}) -> {XF}
    %6 = stablehlo.multiply %0, %5 : {XF}
    %7 = stablehlo.convert %6 : ({XF}) -> {X}
    return %7 : {X}"""
    prog = _mod([X], [X], body)
    ins = [configs.HostInput(hd.f32_to_bf16_bits(hd.normal(21, (6, cols))), pjrt.BufferType.BF16, (6, cols))]
    outs, _ = run_pjrt(gpu_client, prog, ins)
    check(outs[0], oracle_outputs(prog, ins)[0], 1e-2, "rmsnorm")


def test_reduce_with_argument_init(gpu_client):
    prog = _mod(["tensor<3x4xi32>", "tensor<i32>"], ["tensor<3xi32>"], """    %0 = stablehlo.reduce(%arg0 init: %arg1) applies stablehlo.add across dimensions = [1] : (tensor<3x4xi32>, tensor<i32>) -> tensor<3xi32>
    return %0 : tensor<3xi32>""")
    ins = [configs.HostInput(np.arange(12, dtype=np.int32).reshape(3, 4), pjrt.BufferType.S32, (3, 4)),
           configs.HostInput(np.array(100, dtype=np.int32), pjrt.BufferType.S32, ())]
    outs, _ = run_pjrt(gpu_client, prog, ins)
    assert outs[0].tolist() == [106, 122, 138]


def test_transpose_broadcast_iota_select(gpu_client):
    body = """    %0 = stablehlo.transpose %arg0, dims = [1, 0] : (tensor<8x33xf32>) -> tensor<33x8xf32>
    %1 = stablehlo.iota dim = 0 : tensor<33x8xi32>
    %2 = stablehlo.iota dim = 1 : tensor<33x8xi32>
    %3 = stablehlo.compare  LT, %2, %1,  SIGNED : (tensor<33x8xi32>, tensor<33x8xi32>) -> tensor<33x8xi1>
    %4 = stablehlo.broadcast_in_dim %arg1, dims = [1] : (tensor<8xf32>) -> tensor<33x8xf32>
    %5 = stablehlo.select %3, %0, %4 : tensor<33x8xi1>, tensor<33x8xf32>
    %6 = stablehlo.reshape %5 : (tensor<33x8xf32>) -> tensor<264xf32>
    return %6 : tensor<264xf32>"""
    prog = _mod([F, "tensor<8xf32>"], ["tensor<264xf32>"], body)
    ins = _f32_inputs(1) + [configs.HostInput(hd.normal(9, (8,)), pjrt.BufferType.F32, (8,))]
    outs, _ = run_pjrt(gpu_client, prog, ins)
    check(outs[0], oracle_outputs(prog, ins)[0], 0.0, "select")


def test_generic_gemm_transposed_operands(gpu_client):
    # lhs contracting dim first (m-contiguous A) and a rank-3 batch layout: generic GEMM path
    body = """    %0 = stablehlo.dot_general %arg0, %arg1, batching_dims = [2] x [0], contracting_dims = [0] x [2] : (tensor<24x20x3xf32>, tensor<3x18x24xf32>) -> tensor<3x20x18xf32>
    %1 = stablehlo.exponential %0 : tensor<3x20x18xf32>
    return %1 : tensor<3x20x18xf32>"""
    prog = _mod(["tensor<24x20x3xf32>", "tensor<3x18x24xf32>"], ["tensor<3x20x18xf32>"], body)
    ins = [configs.HostInput(hd.normal(11, (24, 20, 3), 0, 0.2), pjrt.BufferType.F32, (24, 20, 3)),
           configs.HostInput(hd.normal(12, (3, 18, 24), 0, 0.2), pjrt.BufferType.F32, (3, 18, 24))]
    outs, exe = run_pjrt(gpu_client, prog, ins)
    check(outs[0], oracle_outputs(prog, ins)[0], 1e-5, "generic gemm")


def test_mfma_bf16_with_generic_epilogue(gpu_client):
    # an epilogue the MFMA kernels do not implement natively (tanh): dot on MFMA, expression as its own kernel
    T, O = "tensor<128x128xbf16>", "tensor<128x128xf32>"
    body = f"""    %0 = stablehlo.dot_general %arg0, %arg1, contracting_dims = [1] x [0] : ({T}, {T}) -> {O}
    %1 = stablehlo.tanh %0 : {O}
    return %1 : {O}"""
    prog = _mod([T, T], [O], body)
    ins = [configs.HostInput(hd.f32_to_bf16_bits(hd.normal(13 + i, (128, 128), 0, 0.1)), pjrt.BufferType.BF16,
                             (128, 128)) for i in range(2)]
    outs, exe = run_pjrt(gpu_client, prog, ins)
    assert "gemm_bf16_mfma" in exe.describe_plan()
    check(outs[0], oracle_outputs(prog, ins)[0], 1e-4, "bf16+tanh")


# slice / concatenate / pad (manipulation.rs:530-917): slices are views read in place, concatenate writes each
# operand's expression into its region, pad fills and then writes the kept operand elements
def _ints_input(seed, shape, dt="i32"):
    x = hd.int_uniform(seed, shape, -1000, 1000).astype(np.int32)
    return configs.HostInput(x, pjrt.BufferType.S32, shape)


@pytest.mark.parametrize("case", ["strided_f32", "outer_rows_bf16", "golden_i32"])
def test_slice_views(gpu_client, case):
    if case == "strided_f32":
        prog = _mod(["tensor<8x33xf32>"], ["tensor<6x11xf32>"], """    %0 = stablehlo.slice %arg0 [1:7, 2:33:3] : (tensor<8x33xf32>) -> tensor<6x11xf32>
    %1 = stablehlo.negate %0 : tensor<6x11xf32>
    return %1 : tensor<6x11xf32>""")
        ins = _f32_inputs(1, (8, 33))
    elif case == "outer_rows_bf16":
        # contiguous rows: the plan copies bytes from an offset into the operand
        prog = _mod(["tensor<4x64xbf16>"], ["tensor<2x64xbf16>"], """    %0 = stablehlo.slice %arg0 [1:3, 0:64] : (tensor<4x64xbf16>) -> tensor<2x64xbf16>
    return %0 : tensor<2x64xbf16>""")
        x = hd.f32_to_bf16_bits(hd.normal(3, (4, 64)))
        ins = [configs.HostInput(x, pjrt.BufferType.BF16, (4, 64))]
    else:
        prog = _mod(["tensor<3x4x5xi32>"], ["tensor<2x2x3xi32>"], """    %0 = stablehlo.slice %arg0 [0:2, 1:3, 0:5:2] : (tensor<3x4x5xi32>) -> tensor<2x2x3xi32>
    return %0 : tensor<2x2x3xi32>""")
        ins = [_ints_input(4, (3, 4, 5))]
    outs, _ = run_pjrt(gpu_client, prog, ins)
    for o, w in zip(outs, oracle_outputs(prog, ins)):
        check(o, w, 0, case)


def test_slice_feeds_gemm_in_place(gpu_client):
    prog = _mod(["tensor<64x256xbf16>", "tensor<128x64xbf16>"], ["tensor<64x64xf32>"], """    %0 = stablehlo.slice %arg0 [0:64, 128:256] : (tensor<64x256xbf16>) -> tensor<64x128xbf16>
    %1 = stablehlo.dot_general %0, %arg1, contracting_dims = [1] x [0] : (tensor<64x128xbf16>, tensor<128x64xbf16>) -> tensor<64x64xf32>
    return %1 : tensor<64x64xf32>""")
    ins = [configs.HostInput(hd.f32_to_bf16_bits(hd.normal(5, (64, 256))), pjrt.BufferType.BF16, (64, 256)),
           configs.HostInput(hd.f32_to_bf16_bits(hd.normal(6, (128, 64))), pjrt.BufferType.BF16, (128, 64))]
    outs, exe = run_pjrt(gpu_client, prog, ins)
    assert exe.describe_plan().split()[1].startswith("gemm")
    check(outs[0], oracle_outputs(prog, ins)[0], 1e-5, "slice·B")  # bf16 products are exact in f32


def test_concatenate_with_fused_producers(gpu_client):
    prog = _mod(["tensor<8x16xf32>", "tensor<8x16xf32>"], ["tensor<8x40xf32>", "tensor<24x16xf32>"], """    %0 = stablehlo.slice %arg0 [0:8, 4:12] : (tensor<8x16xf32>) -> tensor<8x8xf32>
    %1 = stablehlo.slice %arg1 [0:8, 0:16:2] : (tensor<8x16xf32>) -> tensor<8x8xf32>
    %2 = stablehlo.add %0, %1 : tensor<8x8xf32>
    %3 = stablehlo.negate %arg1 : tensor<8x16xf32>
    %4 = stablehlo.concatenate %3, %2, %arg0, dim = 1 : (tensor<8x16xf32>, tensor<8x8xf32>, tensor<8x16xf32>) -> tensor<8x40xf32>
    %5 = stablehlo.concatenate %arg0, %3, %arg1, dim = 0 : (tensor<8x16xf32>, tensor<8x16xf32>, tensor<8x16xf32>) -> tensor<24x16xf32>
    return %4, %5 : tensor<8x40xf32>, tensor<24x16xf32>""")
    ins = _f32_inputs(2, (8, 16))
    outs, _ = run_pjrt(gpu_client, prog, ins)
    for i, (o, w) in enumerate(zip(outs, oracle_outputs(prog, ins))):
        check(o, w, 0, f"concatenate {i}")


@pytest.mark.parametrize("shape,lo,hi,interior", [((2, 3), (0, 1), (2, 1), (1, 2)), ((8, 16), (1, -1), (3, 2), (0, 0)),
                                                  ((5, 7), (-3, 2), (-4, -2), (2, 1)),
                                                  ((3, 4), (-3, 0), (1, 0), (0, 0))])  # last: all operand rows cut
def test_pad(gpu_client, shape, lo, hi, interior):
    out_shape = tuple(l + h + k + (k - 1) * it for k, l, h, it in zip(shape, lo, hi, interior))
    t, ot = _t(shape, "i32"), _t(out_shape, "i32")
    prog = _mod([t, "tensor<i32>"], [ot], f"""    %0 = stablehlo.pad %arg0, %arg1, low = {list(lo)}, high = {list(hi)}, interior = {list(interior)} : ({t}, tensor<i32>) -> {ot}
    return %0 : {ot}""")
    ins = [_ints_input(7, shape), configs.HostInput(np.array(-5, np.int32), pjrt.BufferType.S32, ())]
    outs, _ = run_pjrt(gpu_client, prog, ins)
    check(outs[0], oracle_outputs(prog, ins)[0], 0, "pad")


def test_pad_float_with_computed_value(gpu_client):
    prog = _mod(["tensor<6x8xf32>", "tensor<f32>"], ["tensor<9x10xf32>"], """    %0 = stablehlo.exponential %arg1 : tensor<f32>
    %1 = stablehlo.pad %arg0, %0, low = [2, 1], high = [-1, 1], interior = [0, 0] : (tensor<6x8xf32>, tensor<f32>) -> tensor<7x10xf32>
    %2 = stablehlo.pad %1, %arg1, low = [1, 0], high = [1, 0], interior = [0, 0] : (tensor<7x10xf32>, tensor<f32>) -> tensor<9x10xf32>
    return %2 : tensor<9x10xf32>""")
    ins = _f32_inputs(1, (6, 8)) + [configs.HostInput(np.array(0.5, np.float32), pjrt.BufferType.F32, ())]
    outs, _ = run_pjrt(gpu_client, prog, ins)
    check(outs[0], oracle_outputs(prog, ins)[0], 1e-6, "pad f32")


# ----------------------------------------------------------------------------------------------- op semantics
from tests.ref_examples import EXAMPLES, TRANSCENDENTAL, check_values  # noqa: E402

_BT = {"f32": pjrt.BufferType.F32, "i32": pjrt.BufferType.S32, "i8": pjrt.BufferType.S8, "i1": pjrt.BufferType.PRED}
_NP = {"f32": np.float32, "i32": np.int32, "i8": np.int8, "i1": np.bool_}


@pytest.mark.parametrize("ex", EXAMPLES, ids=[e.name for e in EXAMPLES])
def test_reference_worked_examples(gpu_client, ex):
    """The reference's documented example of each op (tests/ref_examples.py) on the GPU: bit-exact, except 2 ulps of
    slack for the ops computed by device libm (tests/ref_examples.py's TRANSCENDENTAL)."""
    ins = [configs.HostInput(np.asarray(v, dtype=np.float64).astype(_NP[t]), _BT[t], ex.shape)
           for v, t in zip(ex.inputs, ex.in_types)]
    outs, _ = run_pjrt(gpu_client, ex.program(), ins)
    check_values(outs[0], ex, ulps=2 if ex.op in TRANSCENDENTAL else 0)


@pytest.mark.parametrize("shape", SHAPES)
def test_clamp_f32_and_i32(gpu_client, shape):
    """clamp(min, x, max) with per-element bounds (NaN in any operand gives NaN), scalar bounds, and i32."""
    T, I, S = _t(shape), _t(shape, "i32"), "tensor<f32>"
    lo = hd.normal(21, shape) - 0.5
    hi = lo + np.abs(hd.normal(22, shape))
    x = hd.normal(23, shape) * 2
    for arr, idx in ((x, 0), (lo, 7), (hi, 13)):
        arr.reshape(-1)[idx] = np.nan
    body = f"""    %0 = stablehlo.clamp %arg0, %arg1, %arg2 : {T}
    %1 = stablehlo.clamp %arg3, %arg1, %arg4 : ({S}, {T}, {S}) -> {T}
    %2 = stablehlo.convert %arg1 : ({T}) -> {I}
    %3 = stablehlo.constant dense<-1> : {I}
    %4 = stablehlo.constant dense<2> : {I}
    %5 = stablehlo.clamp %3, %2, %4 : {I}
    return %0, %1, %5 : {T}, {T}, {I}"""
    prog = _mod([T, T, T, S, S], [T, T, I], body)
    ins = [configs.HostInput(v.astype(np.float32), pjrt.BufferType.F32, shape) for v in (lo, x, hi)] + [
        configs.HostInput(np.float32(-0.25), pjrt.BufferType.F32, ()), configs.HostInput(np.float32(0.75),
                                                                                       pjrt.BufferType.F32, ())]
    outs, _ = run_pjrt(gpu_client, prog, ins)
    want = oracle_outputs(prog, ins)
    got0 = outs[0].astype(np.float64)
    assert np.isnan(got0.reshape(-1)[[0, 7, 13]]).all()
    for o, w, name in zip(outs, want, ("clamp", "clamp_scalar_bounds", "clamp_i32")):
        g, v = sh.from_raw(o, w[1]), w[0]
        assert np.array_equal(np.isnan(g), np.isnan(v)), name
        ok = ~np.isnan(v)
        assert np.array_equal(g[ok], v[ok]), name


@pytest.mark.parametrize("shape", SHAPES)
def test_power_and_remainder_f32(gpu_client, shape):
    T = _t(shape)
    body = f"""    %0 = stablehlo.abs %arg0 : {T}
    %1 = stablehlo.power %0, %arg1 : {T}
    %2 = stablehlo.remainder %arg0, %arg1 : {T}
    return %1, %2 : {T}, {T}"""
    prog = _mod([T, T], [T, T], body)
    ins = _f32_inputs(2, shape, seed=31)
    outs, _ = run_pjrt(gpu_client, prog, ins)
    want = oracle_outputs(prog, ins)
    check(outs[0], want[0], 1e-5, "power")
    check(outs[1], want[1], 0, "remainder")  # fmod is exact


@pytest.mark.parametrize("dt,bt", [("bf16", pjrt.BufferType.BF16), ("f8E4M3FN", pjrt.BufferType.F8E4M3FN),
                                   ("i8", pjrt.BufferType.S8), ("f32", pjrt.BufferType.F32)])
def test_streaming_maps_by_element_size(gpu_client, dt, bt):
    """Maps over one or two contiguous leaves run the streaming kernel, whose fetches are specialised by element size
    (4, 2 and 1 bytes): a unary map and a binary map of the same type, checked bit-exactly against the oracle."""
    shape = (16, 4096)
    T, F = _t(shape, dt), _t(shape, "f32")
    body = f"""    %0 = stablehlo.convert %arg0 : ({T}) -> {F}
    %1 = stablehlo.negate %0 : {F}
    %2 = stablehlo.add %arg0, %arg1 : {T}
    return %1, %2 : {F}, {T}"""
    prog = _mod([T, T], [F, T], body)
    if dt == "i8":
        raw = [hd.int_uniform(41 + i, shape, -60, 60).astype(np.int8) for i in range(2)]
    elif dt == "f32":
        raw = [hd.normal(41 + i, shape).astype(np.float32) for i in range(2)]
    elif dt == "bf16":
        raw = [hd.f32_to_bf16_bits(hd.normal(41 + i, shape)) for i in range(2)]
    else:
        raw = [hd.f32_to_e4m3fn_bits(hd.normal(41 + i, shape)) for i in range(2)]
    ins = [configs.HostInput(r, bt, shape) for r in raw]
    outs, exe = run_pjrt(gpu_client, prog, ins)
    for o, w, name in zip(outs, oracle_outputs(prog, ins), ("convert-negate", "add")):
        check(o, w, 0.0, f"{dt} {name}")


_MAP_SPECIALS = np.array([np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-40, -3e-39, 3.0e38, -1.5, 2.5, 1.0],
                         np.float32)


def _map_input(seed, shape, dt):
    x = (hd.normal(seed, shape) * 10).astype(np.float32).reshape(-1)
    x[seed % 7::97][:len(_MAP_SPECIALS)] = _MAP_SPECIALS[:len(x[seed % 7::97])]
    x = x.reshape(shape)
    if dt == "bf16":
        return configs.HostInput(hd.f32_to_bf16_bits(x), pjrt.BufferType.BF16, shape)
    return configs.HostInput(x, pjrt.BufferType.F32, shape)


def _same_bits(got_raw, want, name):
    """Exactly the oracle's values: equal numbers with equal signs (zeros included), NaN where it has NaN."""
    vals, dt = want
    got = sh.from_raw(got_raw, dt)
    nan = np.isnan(vals)
    assert np.array_equal(np.isnan(got), nan), f"{name}: NaN positions differ"
    ok = (got[~nan] == vals[~nan]) & (np.signbit(got[~nan]) == np.signbit(vals[~nan]))
    assert np.all(ok), f"{name}: {np.count_nonzero(~ok)} elements differ"


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("form", ["leaves", "const_right", "const_left", "same_leaf"])
@pytest.mark.parametrize("op", ["add", "subtract", "multiply", "divide", "maximum", "minimum"])
def test_direct_binary_maps(gpu_client, dt, form, op):
    """One binary operation over contiguous f32 / bf16 leaves (or a leaf and a splat constant on either side) runs the
    direct map kernel: bit-exact against the oracle, NaN / infinity / signed-zero / subnormal inputs included."""
    shape = (8, 1024)
    T = _t(shape, dt)
    const = f"    %c = stablehlo.constant dense<-2.500000e+00> : {T}\n"
    lhs, rhs, args = {"leaves": ("%arg0", "%arg1", [T, T]), "const_right": ("%arg0", "%c", [T]),
                      "const_left": ("%c", "%arg0", [T]), "same_leaf": ("%arg0", "%arg0", [T])}[form]
    body = (const if "const" in form else "") + f"    %0 = stablehlo.{op} {lhs}, {rhs} : {T}\n    return %0 : {T}"
    prog = _mod(args, [T], body)
    ins = [_map_input(61 + i, shape, dt) for i in range(len(args))]
    outs, _ = run_pjrt(gpu_client, prog, ins)
    _same_bits(outs[0], oracle_outputs(prog, ins)[0], f"{dt} {form} {op}")


@pytest.mark.parametrize("case", ["negate_f32", "abs_bf16", "negate_bf16", "convert_f32_bf16", "convert_bf16_f32"])
def test_direct_unary_maps(gpu_client, case):
    shape = (4, 2048)
    F, B = _t(shape), _t(shape, "bf16")
    if case.startswith("convert"):
        src, dst = (F, B) if case == "convert_f32_bf16" else (B, F)
        body = f"    %0 = stablehlo.convert %arg0 : ({src}) -> {dst}\n    return %0 : {dst}"
        prog, ins = _mod([src], [dst], body), [_map_input(71, shape, "f32" if src == F else "bf16")]
    else:
        op, dt = case.split("_")
        T = _t(shape, dt)
        prog, ins = _mod([T], [T], f"    %0 = stablehlo.{op} %arg0 : {T}\n    return %0 : {T}"), [_map_input(72, shape, dt)]
    outs, _ = run_pjrt(gpu_client, prog, ins)
    _same_bits(outs[0], oracle_outputs(prog, ins)[0], case)


# ------------------------------------------------------------------ trigonometric, rounding and bit operations
def _within_ulps(got_raw, want, ulps, name):
    """Equal NaN positions and infinities; finite values within `ulps` units in the last place of the oracle's value
    at the result type (device libm against float64 rounded once)."""
    vals, dt = want
    got = sh.from_raw(got_raw, dt)
    nan = np.isnan(vals)
    assert np.array_equal(np.isnan(got), nan), f"{name}: NaN positions differ"
    g, w = got[~nan], vals[~nan]
    inf = np.isinf(w)
    assert np.array_equal(g[inf], w[inf]), f"{name}: infinities differ"
    unit = np.spacing(np.abs(w[~inf]).astype(np.float32)).astype(np.float64) * (65536.0 if dt == "bf16" else 1.0)
    err = np.abs(g[~inf] - w[~inf]) / unit
    assert np.all(err <= ulps), f"{name}: {np.count_nonzero(err > ulps)} values beyond {ulps} ulps (max {err.max()})"


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("shape", [(8, 33), (4, 2048)])
def test_trigonometric_cbrt_rounding_is_finite(gpu_client, dt, shape):
    """sine, cosine, tan, cbrt and atan2 within 4 ulps (f32) or 1 ulp (bf16, one rounding of the f32 result) of the
    oracle; round_nearest_even, round_nearest_afz and is_finite bit-exact; NaN, infinities, signed zeros,
    subnormals and 3e38 among the operands."""
    T, P = _t(shape, dt), _t(shape, "i1")
    ops = ["sine", "cosine", "tan", "cbrt", "round_nearest_even", "round_nearest_afz"]
    body = "".join(f"    %{i} = stablehlo.{op} %arg0 : {T}\n" for i, op in enumerate(ops))
    body += f"    %6 = stablehlo.atan2 %arg0, %arg1 : {T}\n"
    body += f"    %7 = stablehlo.is_finite %arg0 : ({T}) -> {P}\n"
    body += "    return " + ", ".join(f"%{i}" for i in range(8)) + " : " + ", ".join([T] * 7 + [P])
    prog = _mod([T, T], [T] * 7 + [P], body)
    ins = [_map_input(81, shape, dt), _map_input(82, shape, dt)]
    print(f"[ops] trig/round {dt} {shape}", flush=True)
    outs, _ = run_pjrt(gpu_client, prog, ins)
    want = oracle_outputs(prog, ins)
    for i, name in enumerate(ops + ["atan2"]):
        if name.startswith("round"):
            _same_bits(outs[i], want[i], f"{dt} {name}")
        else:
            _within_ulps(outs[i], want[i], 4 if dt == "f32" else 1, f"{dt} {name}")
    check(outs[7], want[7], 0, "is_finite")


_INT_TYPES = {"i8": (np.int8, pjrt.BufferType.S8), "ui8": (np.uint8, pjrt.BufferType.U8),
              "i16": (np.int16, pjrt.BufferType.S16), "ui16": (np.uint16, pjrt.BufferType.U16),
              "i32": (np.int32, pjrt.BufferType.S32), "ui32": (np.uint32, pjrt.BufferType.U32)}


@pytest.mark.parametrize("dt", list(_INT_TYPES))
@pytest.mark.parametrize("shape", [(8, 33), (4, 1024)])
def test_bit_operations(gpu_client, dt, shape):
    """shift_left / shift_right_arithmetic / shift_right_logical by amounts inside and outside the width (negative
    ones too), popcnt and count_leading_zeros, bit-exact against the oracle at every integer width."""
    npt, bt = _INT_TYPES[dt]
    info, w = np.iinfo(npt), np.iinfo(npt).bits
    rng = np.random.default_rng(w + 3 * (dt[0] == "u"))
    a = rng.integers(info.min, info.max, size=shape, endpoint=True).astype(npt)
    a.reshape(-1)[:4] = [info.min, info.max, 0, 1]
    k = rng.integers(max(info.min, -3), w + 3, size=shape).astype(npt)
    T = _t(shape, dt)
    ops = ["shift_left", "shift_right_arithmetic", "shift_right_logical"]
    body = "".join(f"    %{i} = stablehlo.{op} %arg0, %arg1 : {T}\n" for i, op in enumerate(ops))
    body += f"    %3 = stablehlo.popcnt %arg0 : {T}\n    %4 = stablehlo.count_leading_zeros %arg0 : {T}\n"
    body += "    return %0, %1, %2, %3, %4 : " + ", ".join([T] * 5)
    prog = _mod([T, T], [T] * 5, body)
    ins = [configs.HostInput(a, bt, shape), configs.HostInput(k, bt, shape)]
    print(f"[ops] bits {dt} {shape}", flush=True)
    outs, _ = run_pjrt(gpu_client, prog, ins)
    for o, want, name in zip(outs, oracle_outputs(prog, ins), ops + ["popcnt", "count_leading_zeros"]):
        check(o, want, 0, f"{dt} {name}")


@pytest.mark.parametrize("dt", ["i8", "ui8"])
def test_shifts_over_every_8bit_pair(gpu_client, dt):
    npt, bt = _INT_TYPES[dt]
    vals = np.arange(np.iinfo(npt).min, np.iinfo(npt).max + 1)
    a, k = (x.astype(npt) for x in np.meshgrid(vals, vals, indexing="ij"))
    T = _t((256, 256), dt)
    ops = ["shift_left", "shift_right_arithmetic", "shift_right_logical"]
    body = "".join(f"    %{i} = stablehlo.{op} %arg0, %arg1 : {T}\n" for i, op in enumerate(ops))
    body += "    return %0, %1, %2 : " + ", ".join([T] * 3)
    prog = _mod([T, T], [T] * 3, body)
    ins = [configs.HostInput(a, bt, (256, 256)), configs.HostInput(k, bt, (256, 256))]
    outs, _ = run_pjrt(gpu_client, prog, ins)
    for o, want, name in zip(outs, oracle_outputs(prog, ins), ops):
        check(o, want, 0, f"{dt} {name}")


def test_counter_hash_rounds_ui32(gpu_client):
    """A counter-based hash in the style of threefry's rounds (add, rotate by shift_left | shift_right_logical, xor)
    over an iota counter and a key, bit-exact against the same rounds in numpy's uint32 arithmetic."""
    n = 1 << 14
    U = f"tensor<{n}xui32>"
    S = "tensor<ui32>"
    lines = [f"    %x0 = stablehlo.iota dim = 0 : {U}",
             f"    %k = stablehlo.broadcast_in_dim %arg0, dims = [] : ({S}) -> {U}",
             f"    %y0 = stablehlo.xor %x0, %k : {U}"]
    x, y = "%x0", "%y0"
    rots = [13, 15, 26, 6]
    for i, r in enumerate(rots):
        lines += [f"    %r{i} = stablehlo.constant dense<{r}> : {U}",
                  f"    %q{i} = stablehlo.constant dense<{32 - r}> : {U}",
                  f"    %s{i} = stablehlo.add {x}, {y} : {U}",
                  f"    %l{i} = stablehlo.shift_left {y}, %r{i} : {U}",
                  f"    %h{i} = stablehlo.shift_right_logical {y}, %q{i} : {U}",
                  f"    %o{i} = stablehlo.or %l{i}, %h{i} : {U}",
                  f"    %t{i} = stablehlo.xor %o{i}, %s{i} : {U}"]
        x, y = f"%s{i}", f"%t{i}"
    lines.append(f"    return {x}, {y} : {U}, {U}")
    prog = _mod([S], [U, U], "\n".join(lines))
    key = np.uint32(0x1BD11BDA)
    outs, _ = run_pjrt(gpu_client, prog, [configs.HostInput(np.array(key), pjrt.BufferType.U32, ())])
    xs = np.arange(n, dtype=np.uint32)
    ys = xs ^ key
    for r in rots:
        xs = xs + ys
        ys = ((ys << np.uint32(r)) | (ys >> np.uint32(32 - r))) ^ xs
    assert np.array_equal(outs[0].view(np.uint32), xs) and np.array_equal(outs[1].view(np.uint32), ys)


def test_rotary_angles_from_positions_bf16(gpu_client):
    """Rotary position angles computed in the program: positions (iota) times per-column frequencies, cosine and
    sine fused with the bf16 products x·cos + y·sin; against the oracle to bf16 rounding."""
    S, D = 512, 128
    X, F, A = f"tensor<{S}x{D}xbf16>", f"tensor<{D}xf32>", f"tensor<{S}x{D}xf32>"
    body = f"""    %p = stablehlo.iota dim = 0 : {A}
    %f = stablehlo.broadcast_in_dim %arg2, dims = [1] : ({F}) -> {A}
    %a = stablehlo.multiply %p, %f : {A}
    %c = stablehlo.cosine %a : {A}
    %s = stablehlo.sine %a : {A}
    %x = stablehlo.convert %arg0 : ({X}) -> {A}
    %y = stablehlo.convert %arg1 : ({X}) -> {A}
    %xc = stablehlo.multiply %x, %c : {A}
    %ys = stablehlo.multiply %y, %s : {A}
    %r = stablehlo.add %xc, %ys : {A}
    %o = stablehlo.convert %r : ({A}) -> {X}
    return %o : {X}"""
    prog = _mod([X, X, F], [X], body)
    freqs = (10000.0 ** (-np.arange(D) / D)).astype(np.float32)
    ins = [configs.HostInput(hd.f32_to_bf16_bits(hd.normal(91 + i, (S, D))), pjrt.BufferType.BF16, (S, D))
           for i in range(2)] + [configs.HostInput(freqs, pjrt.BufferType.F32, (D,))]
    outs, _ = run_pjrt(gpu_client, prog, ins)
    check(outs[0], oracle_outputs(prog, ins)[0], 4e-3, "rotary bf16")
