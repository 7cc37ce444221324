"""reverse, optimization_barrier, map and same-width bitcast_convert on the GPU (crates/ryft-mlir/src/dialects/
stable_hlo/operations/miscellaneous.rs:309-450, functional.rs:13-104, casting.rs:8-73), bit-exact:

  * reverse            against the oracle (numpy's flip) for every element size, one, several and no reversed
                       dimensions, innermost extents that do and do not allow 16-byte vectors, a fused consumer and a
                       reverse of a slice;
  * map                the reference's multiply example and a body with a constant, a compare and a select;
  * optimization_barrier  the identity on each operand;
  * bitcast_convert    against numpy's view of the same bytes (the definition of the op) for 32-, 16- and 8-bit pairs,
                       float ones included (finite values, infinities, signed zeros and subnormals; NaN patterns of
                       the 32-bit float type kept bit for bit);
  * reduce_precision   against the oracle (itself pinned to bf16 / f16 rounding and a closed form for f16
                       subnormals) on every non-NaN 16-bit pattern of bf16 and f16 and on f32 values across the whole
                       exponent range, for several formats;
  * if / case          every branch computed and the taken one selected, against the oracle (which runs only the taken
                       branch) for in-range and out-of-range indices, with the reference's worked example."""
import numpy as np
import pytest

from oracle import stablehlo as sh
from ryft_amd import configs, pjrt
from tests.helpers import oracle_outputs, run_pjrt
from tests.test_misc_ops import barrier_program, bitcast_program, map_program, reverse_program, _t

pytestmark = pytest.mark.gpu

BT = {"f32": (pjrt.BufferType.F32, np.float32), "bf16": (pjrt.BufferType.BF16, np.uint16),
      "f16": (pjrt.BufferType.F16, np.uint16), "f8E4M3FN": (pjrt.BufferType.F8E4M3FN, np.uint8),
      "i8": (pjrt.BufferType.S8, np.int8), "ui8": (pjrt.BufferType.U8, np.uint8),
      "i16": (pjrt.BufferType.S16, np.int16), "ui16": (pjrt.BufferType.U16, np.uint16),
      "i32": (pjrt.BufferType.S32, np.int32), "ui32": (pjrt.BufferType.U32, np.uint32),
      "f64": (pjrt.BufferType.F64, np.float64), "i1": (pjrt.BufferType.PRED, np.bool_)}


def _input(raw: np.ndarray, dt: str) -> configs.HostInput:
    raw = np.asarray(raw)
    raw = np.ascontiguousarray(raw) if raw.ndim else raw  # (ascontiguousarray makes a 0-d array 1-d)
    return configs.HostInput(raw, BT[dt][0], tuple(raw.shape))


def _random(seed, shape, dt):
    rng = np.random.default_rng(seed)
    npt = BT[dt][1]
    if dt == "f32" or dt == "f64":
        return rng.standard_normal(shape).astype(npt)
    if dt == "bf16":
        return rng.integers(0x3C00, 0x4400, size=shape).astype(np.uint16)
    if dt == "i1":
        return rng.integers(0, 2, size=shape).astype(np.bool_)
    info = np.iinfo(npt)
    return rng.integers(info.min, info.max, size=shape, endpoint=True).astype(npt)


def _exact(client, prog, ins, name):
    print(f"[misc] {name}", flush=True)
    outs, _ = run_pjrt(client, prog, ins)
    for k, (got, (vals, dt)) in enumerate(zip(outs, oracle_outputs(prog, ins))):
        want = np.asarray(sh.to_raw(np.asarray(vals), dt)).reshape(np.shape(vals))
        assert got.shape == want.shape, f"{name} #{k}: shape {got.shape} != {want.shape}"
        mism = np.count_nonzero(got.view(want.dtype) != want) if got.dtype.itemsize == want.dtype.itemsize else -1
        assert mism == 0, f"{name} #{k}: {mism} elements differ"


@pytest.mark.parametrize("dt", ["f32", "bf16", "i8", "f64", "i1", "ui16"])
@pytest.mark.parametrize("shape,dims", [((6, 64), [1]), ((6, 64), [0]), ((5, 7, 9), [0, 2]), ((4, 33), [0, 1]),
                                        ((300,), [0]), ((3, 8), [])])
def test_reverse(gpu_client, dt, shape, dims):
    _exact(gpu_client, reverse_program(shape, dims, dt=dt), [_input(_random(1, shape, dt), dt)],
           f"reverse {dt} {shape} {dims}")


def test_reference_reverse_example(gpu_client):
    # miscellaneous.rs:320-327
    outs, _ = run_pjrt(gpu_client, reverse_program((3, 2), [1]),
                       [_input(np.array([[1, 2], [3, 4], [5, 6]], np.int32), "i32")])
    assert outs[0].tolist() == [[2, 1], [4, 3], [6, 5]]


@pytest.mark.parametrize("dt", ["f32", "i32"])
def test_reverse_with_consumer(gpu_client, dt):
    shape = (16, 256)
    _exact(gpu_client, reverse_program(shape, [1], dt=dt, consumer=True), [_input(_random(2, shape, dt), dt)],
           f"reverse + add {dt}")


def test_reverse_of_a_slice_and_of_a_reverse(gpu_client):
    T, S = _t((8, 40), "f32"), _t((4, 13), "f32")
    prog = f"""module {{
  func.func @main(%arg0: {T}) -> ({S}, {T}) {{
    %0 = stablehlo.slice %arg0 [1:8:2, 3:40:3] : ({T}) -> {S}
    %1 = stablehlo.reverse %0, dims = [0, 1] : {S}
    %2 = stablehlo.reverse %arg0, dims = [1] : {T}
    %3 = stablehlo.reverse %2, dims = [0, 1] : {T}
    return %1, %3 : {S}, {T}
  }}
}}
"""
    _exact(gpu_client, prog, [_input(_random(3, (8, 40), "f32"), "f32")], "reverse of a slice / of a reverse")


def test_map(gpu_client):
    # functional.rs:29-37: multiply of [[0, 1], [2, 3]] and [[4, 5], [6, 7]]
    a = _input(np.array([[0, 1], [2, 3]], np.int32), "i32")
    b = _input(np.array([[4, 5], [6, 7]], np.int32), "i32")
    outs, _ = run_pjrt(gpu_client, map_program((2, 2)), [a, b])
    assert outs[0].tolist() == [[0, 5], [12, 21]] and outs[1].tolist() == [[4, 5], [6, 7]]
    shape = (64, 96)
    _exact(gpu_client, map_program(shape), [_input(_random(4, shape, "i32") % 1000, "i32"),
                                            _input(_random(5, shape, "i32") % 1000, "i32")], "map i32")


def test_optimization_barrier(gpu_client):
    shape = (32, 64)
    _exact(gpu_client, barrier_program(shape), [_input(_random(6, shape, "f32"), "f32"),
                                                _input(_random(7, shape, "f32"), "f32")], "optimization_barrier")


def _bit_patterns(n_bits: int, float_dt: str, rng) -> np.ndarray:
    """Random patterns of `n_bits`, with special values of `float_dt` mixed in; NaN patterns of narrow floats left out
    (a narrow float's register form is an f32 value, so a NaN's payload is not kept)."""
    u = {32: np.uint32, 16: np.uint16, 8: np.uint8}[n_bits]
    x = rng.integers(0, 1 << n_bits, size=4096, dtype=np.uint64).astype(u)
    specials = {"f32": [0x7F800000, 0xFF800000, 0x80000000, 0x00000001, 0x807FFFFF, 0x7FC00001, 0xFFC00000],
                "bf16": [0x7F80, 0xFF80, 0x8000, 0x0001, 0x807F],
                "f16": [0x7C00, 0xFC00, 0x8000, 0x0001, 0x83FF],
                "f8E4M3FN": [0x80, 0x01, 0x87, 0x7E, 0xFE]}[float_dt]
    x[:len(specials)] = np.array(specials, dtype=np.uint64).astype(u)
    if float_dt != "f32":
        exp_mask, man_mask = {"bf16": (0x7F80, 0x7F), "f16": (0x7C00, 0x3FF), "f8E4M3FN": (0x78, 0x7)}[float_dt]
        if float_dt == "f8E4M3FN":
            nan = (x & 0x7F) == 0x7F
        else:
            nan = ((x & exp_mask) == exp_mask) & ((x & man_mask) != 0)
        x = np.where(nan, x & ~np.array(exp_mask, dtype=u), x).astype(u)
    return x


@pytest.mark.parametrize("src,dst", [("f32", "i32"), ("i32", "f32"), ("ui32", "f32"), ("f32", "ui32"),
                                     ("ui32", "i32"), ("bf16", "i16"), ("i16", "bf16"), ("f16", "ui16"),
                                     ("ui16", "f16"), ("bf16", "f16"), ("f8E4M3FN", "ui8"), ("ui8", "f8E4M3FN"),
                                     ("i8", "ui8"), ("ui8", "i8"), ("i8", "f8E4M3FN")])
def test_bitcast_convert_is_a_view_of_the_bytes(gpu_client, src, dst):
    rng = np.random.default_rng(8)
    width = np.dtype(BT[src][1]).itemsize * 8
    fl = next((t for t in (src, dst) if t in ("f32", "bf16", "f16", "f8E4M3FN")), "f32" if width == 32 else
              ("bf16" if width == 16 else "f8E4M3FN"))
    bits = _bit_patterns(width, fl, rng)
    if {src, dst} == {"bf16", "f16"}:  # no NaN pattern of either type
        bits = np.where((bits & 0x7C00) == 0x7C00, bits & 0x83FF, bits).astype(np.uint16)
    x = bits.view(BT[src][1])
    print(f"[misc] bitcast_convert {src} -> {dst}", flush=True)
    outs, _ = run_pjrt(gpu_client, bitcast_program((x.size,), src, dst), [_input(x, src)])
    got = np.ascontiguousarray(outs[0]).view(BT[dst][1])
    assert np.array_equal(got.view(bits.dtype), bits), \
        f"{np.count_nonzero(got.view(bits.dtype) != bits)} elements differ, e.g. " \
        f"{[(hex(a), hex(b)) for a, b in zip(bits[got.view(bits.dtype) != bits][:4], got.view(bits.dtype)[got.view(bits.dtype) != bits][:4])]}"


def test_bitcast_round_trip_fused(gpu_client):
    # f32 → i32 → (integer add 1) → f32: the next representable float above each positive value
    T, I = _t((1024,), "f32"), _t((1024,), "i32")
    prog = f"""module {{
  func.func @main(%arg0: {T}) -> {T} {{
    %0 = stablehlo.bitcast_convert %arg0 : ({T}) -> {I}
    %c = stablehlo.constant dense<1> : {I}
    %1 = stablehlo.add %0, %c : {I}
    %2 = stablehlo.bitcast_convert %1 : ({I}) -> {T}
    return %2 : {T}
  }}
}}
"""
    x = np.abs(_random(9, (1024,), "f32")) + np.float32(1e-3)
    outs, _ = run_pjrt(gpu_client, prog, [_input(x, "f32")])
    assert np.array_equal(outs[0].view(np.float32), np.nextafter(x, np.float32(np.inf)))


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("e,m", [(5, 10), (8, 7), (4, 3), (2, 0), (8, 23), (6, 12)])
def test_reduce_precision(gpu_client, dt, e, m):
    from tests.test_misc_ops import reduce_precision_program
    rng = np.random.default_rng(30 + e * 31 + m)
    if dt == "f32":
        x = (rng.standard_normal(4096) * np.exp2(rng.integers(-140, 128, 4096))).astype(np.float32)
        x[:6] = [np.inf, -np.inf, 0.0, -0.0, 1.0 + 2.0 ** -8, 3.0 * 2.0 ** -149]
    else:  # every 16-bit pattern but the NaNs
        x = np.arange(65536, dtype=np.uint32).astype(np.uint16)
        exp_mask, man_mask = (0x7F80, 0x7F) if dt == "bf16" else (0x7C00, 0x3FF)
        x = x[~(((x & exp_mask) == exp_mask) & ((x & man_mask) != 0))]
    _exact(gpu_client, reduce_precision_program(x.shape, e, m, dt), [_input(x, dt)], f"reduce_precision {dt} e{e}m{m}")


def test_replica_and_partition_ids(gpu_client):
    # communication.rs:110-190: one replica, one partition; both ids 0
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
    outs, _ = run_pjrt(gpu_client, prog, [_input(np.arange(4, dtype=np.uint32) + 7, "ui32")])
    assert outs[0].tolist() == [7, 8, 9, 10] and int(outs[1]) == 0


@pytest.mark.parametrize("idx", [0, 1, 2, 5, -3])
def test_case(gpu_client, idx):
    from tests.test_misc_ops import CASE_EXAMPLE, case_program
    shape = (16, 256)
    ins = [_input(np.array(idx, np.int32), "i32"), _input(_random(40, shape, "f32"), "f32"),
           _input(_random(41, shape, "f32"), "f32")]
    _exact(gpu_client, case_program(3, shape), ins, f"case index {idx}")
    outs, _ = run_pjrt(gpu_client, CASE_EXAMPLE, [_input(np.array(idx, np.int32), "i32")])
    assert outs[0].tolist() == ([0, 0] if idx == 0 else [1, 1])  # control_flow.rs:19-33


@pytest.mark.parametrize("pred", [True, False])
def test_if(gpu_client, pred):
    from tests.test_misc_ops import if_program
    shape = (16, 256)
    ins = [_input(np.array(pred), "i1"), _input(_random(42, shape, "f32"), "f32"),
           _input(_random(43, shape, "f32"), "f32")]
    _exact(gpu_client, if_program(shape), ins, f"if {pred}")


def test_get_dimension_size(gpu_client):
    from tests.test_misc_ops import GET_DIM_EXAMPLE
    outs, _ = run_pjrt(gpu_client, GET_DIM_EXAMPLE, [configs.HostInput(np.array([[1, 2, 3], [4, 5, 6]], np.int64),
                                                                       pjrt.BufferType.S64, (2, 3))])
    assert int(outs[0]) == 3 and int(outs[1]) == 2  # manipulation.rs:22-26
