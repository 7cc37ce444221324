"""dynamic_slice / dynamic_update_slice and gather on the GPU (crates/ryft-mlir/src/dialects/stable_hlo/operations/
manipulation.rs:943-1307), bit-exact against the oracle: the reference's worked examples, every element size with
start indices of several integer types inside, below and past the bounds (clamped), windows moved as 16-byte vectors
and element by element, a fused consumer and a read-modify-write of one window, a KV-cache style update of a
donated buffer written in place, and gathers with batching dimensions, embedding rows and unaligned windows."""
import numpy as np
import pytest

from ryft_amd import configs, pjrt
from tests.helpers import check, oracle_outputs, run_pjrt
from tests.test_dynamic_window import ds_program, dus_program, _mod

pytestmark = pytest.mark.gpu

BT = {"f32": (pjrt.BufferType.F32, np.float32), "bf16": (pjrt.BufferType.BF16, np.uint16),
      "i8": (pjrt.BufferType.S8, np.int8), "f64": (pjrt.BufferType.F64, np.float64),
      "i64": (pjrt.BufferType.S64, np.int64), "i32": (pjrt.BufferType.S32, np.int32),
      "ui32": (pjrt.BufferType.U32, np.uint32), "i1": (pjrt.BufferType.PRED, np.bool_)}


def _tensor(seed, shape, dt):
    bt, npt = BT[dt]
    rng = np.random.default_rng(seed)
    if dt == "bf16":
        x = rng.integers(0x3C00, 0x4400, size=shape).astype(np.uint16)  # finite bf16 patterns
    elif dt == "i1":
        x = rng.integers(0, 2, size=shape).astype(np.bool_)
    elif dt in ("f32", "f64"):
        x = rng.standard_normal(shape).astype(npt)
    else:
        x = rng.integers(-100, 100, size=shape).astype(npt)
    return configs.HostInput(x, bt, tuple(shape))


def _index(v, it):
    bt, npt = BT[it]
    return configs.HostInput(np.array(v).astype(npt).reshape(()), bt, ())


def _check_exact(client, prog, ins, name):
    print(f"[window] {name}", flush=True)
    outs, exe = run_pjrt(client, prog, ins)
    for o, w in zip(outs, oracle_outputs(prog, ins)):
        check(o, w, 0.0, name)
    return exe


def test_reference_examples(gpu_client):
    x = configs.HostInput(np.array([[0, 0, 1, 1], [0, 0, 1, 1], [0, 0, 0, 0], [0, 0, 0, 0]], np.int32),
                          pjrt.BufferType.S32, (4, 4))
    outs, _ = run_pjrt(gpu_client, ds_program((4, 4), (2, 2)), [x, _index(-1, "i64"), _index(3, "i64")])
    assert outs[0].tolist() == [[1, 1], [1, 1]]
    x = configs.HostInput(np.array([[1, 1, 0, 0], [1, 1, 0, 0], [1, 1, 1, 1], [1, 1, 1, 1]], np.int32),
                          pjrt.BufferType.S32, (4, 4))
    u = configs.HostInput(np.ones((2, 2), np.int32), pjrt.BufferType.S32, (2, 2))
    outs, _ = run_pjrt(gpu_client, dus_program((4, 4), (2, 2)), [x, u, _index(-1, "i64"), _index(3, "i64")])
    assert outs[0].tolist() == [[1] * 4] * 4


@pytest.mark.parametrize("dt,it", [("f32", "i32"), ("bf16", "i64"), ("i8", "ui32"), ("f64", "i32"), ("i1", "i64")])
@pytest.mark.parametrize("starts", [(0, 0, 0), (1, 2, 3), (-5, 7, 100), (4, -1, 2)])
def test_every_element_size_and_clamping(gpu_client, dt, it, starts):
    shape, sizes = (5, 7, 9), (2, 3, 4)
    if it.startswith("ui"):
        starts = tuple(abs(s) for s in starts)
    x = _tensor(1, shape, dt)
    idx = [_index(s, it) for s in starts]
    _check_exact(gpu_client, ds_program(shape, sizes, dt=dt, it=it), [x] + idx, f"dynamic_slice {dt} {starts}")
    u = _tensor(2, sizes, dt)
    _check_exact(gpu_client, dus_program(shape, sizes, dt=dt, it=it), [x, u] + idx,
                 f"dynamic_update_slice {dt} {starts}")


@pytest.mark.parametrize("col", [0, 32, 3])  # vector-aligned window origins (0, 32) and an unaligned one (3)
def test_vector_and_element_paths(gpu_client, col):
    # f32 rows of 128 with windows 64 wide: whole 16-byte vectors when the origin column is a multiple of 4
    shape, sizes = (6, 16, 128), (3, 5, 64)
    x = _tensor(3, shape, "f32")
    idx = [_index(s, "i32") for s in (2, 9, col)]
    _check_exact(gpu_client, ds_program(shape, sizes, dt="f32", it="i32"), [x] + idx, f"dynamic_slice col {col}")
    u = _tensor(4, sizes, "f32")
    _check_exact(gpu_client, dus_program(shape, sizes, dt="f32", it="i32"), [x, u] + idx,
                 f"dynamic_update_slice col {col}")


def test_fused_consumer_and_read_modify_write(gpu_client):
    # out0 = dynamic_slice(x) + 1 (the slice feeds an elementwise step); out1 = x with that window doubled
    t, w = "tensor<64x96xf32>", "tensor<16x32xf32>"
    prog = _mod([t, "tensor<i32>", "tensor<i32>"], f"({w}, {t})", f"""    %0 = stablehlo.dynamic_slice %arg0, %arg1, %arg2, sizes = [16, 32] : ({t}, tensor<i32>, tensor<i32>) -> {w}
    %c = stablehlo.constant dense<1.000000e+00> : {w}
    %1 = stablehlo.add %0, %c : {w}
    %2 = stablehlo.add %0, %0 : {w}
    %3 = stablehlo.dynamic_update_slice %arg0, %2, %arg1, %arg2 : ({t}, {w}, tensor<i32>, tensor<i32>) -> {t}
    return %1, %3 : {w}, {t}""")
    x = _tensor(5, (64, 96), "f32")
    for r, c in [(10, 40), (60, -3), (0, 95)]:
        _check_exact(gpu_client, prog, [x, _index(r, "i32"), _index(c, "i32")], f"read-modify-write ({r}, {c})")


def test_kv_cache_update_in_place(gpu_client):
    """A decode step's cache write: the donated [B, H, S, D] cache takes the new position's keys in place (only the
    window is written), step after step, each result donated to the next step."""
    shape, ushape = (2, 8, 256, 64), (2, 8, 1, 64)
    prog = dus_program(shape, ushape, dt="bf16", it="i32", donate=True)
    le = gpu_client.compile(pjrt.Program.mlir(prog))
    assert "(in place)" in le.describe_plan()
    dev = le.addressable_devices()[0]
    cache = _tensor(6, shape, "bf16")
    want = cache.data.copy()
    buf = gpu_client.buffer(cache.data, cache.type, shape, device=dev)
    p0 = buf.unsafe_pointer()
    zero = gpu_client.buffer(np.zeros((), np.int32), pjrt.BufferType.S32, (), device=dev)
    for step, pos in enumerate([0, 1, 5, 255, 300]):  # 300 clamps to the last position
        u = _tensor(10 + step, ushape, "bf16")
        ub = gpu_client.buffer(u.data, u.type, ushape, device=dev)
        pb = gpu_client.buffer(np.array(pos, np.int32), pjrt.BufferType.S32, (), device=dev)
        out = le.execute([[pjrt.ExecutionInput(buf, donatable=True), ub, zero, zero, pb, zero]])[0]
        assert buf.is_deleted()
        buf = out.outputs[0]
        want[:, :, min(pos, 255):min(pos, 255) + 1, :] = u.data
    out.done.await_()
    assert buf.unsafe_pointer() == p0
    assert np.array_equal(buf.to_numpy(), want)


# ------------------------------------------------------------------------------------------------ gather
from tests.test_dynamic_window import GATHER_EXAMPLE, gather_example_program, gather_program  # noqa: E402


def test_gather_reference_example(gpu_client):
    ins = [configs.HostInput(GATHER_EXAMPLE["x"].astype(np.int32), pjrt.BufferType.S32, (2, 3, 4, 2)),
           configs.HostInput(GATHER_EXAMPLE["idx"].astype(np.int64), pjrt.BufferType.S64, (2, 2, 3, 2))]
    outs, exe = run_pjrt(gpu_client, gather_example_program(), ins)
    assert "gather" in exe.describe_plan()
    assert outs[0].tolist() == GATHER_EXAMPLE["want"]


@pytest.mark.parametrize("dt", ["bf16", "f32", "i8", "f64"])
def test_gather_embedding_rows(gpu_client, dt):
    # rows of a [1000, 256] table by 4096 ids, some out of range (clamped to the first / last row): 16-byte vectors
    # along the rows; checked against numpy's indexing (the oracle's agreement with it is pinned on the CPU)
    table = _tensor(20, (1000, 256), dt)
    rng = np.random.default_rng(21)
    ids = rng.integers(-20, 1020, size=4096).astype(np.int32)
    t = "tensor<1000x256x" + dt + ">"
    prog = gather_program(t, "tensor<4096xi32>", "tensor<4096x256x" + dt + ">", [1], [0], [0], 1, [1, 256])
    outs, _ = run_pjrt(gpu_client, prog, [table, configs.HostInput(ids, pjrt.BufferType.S32, (4096,))])
    want = table.data[np.clip(ids, 0, 999)]
    assert np.array_equal(outs[0].view(np.uint8), np.ascontiguousarray(want).view(np.uint8))


@pytest.mark.parametrize("case", ["take_along_axis", "unaligned_windows", "reference_printed"])
def test_gather_against_the_oracle(gpu_client, case):
    if case == "take_along_axis":
        # batching dims: one element per row at a per-row column
        x = _tensor(22, (64, 100), "f32")
        cols = configs.HostInput(np.random.default_rng(23).integers(-5, 110, size=(64, 1)).astype(np.int64),
                                 pjrt.BufferType.S64, (64, 1))
        prog = gather_program("tensor<64x100xf32>", "tensor<64x1xi64>", "tensor<64xf32>", [], [1], [1], 1,
                              [1, 1], op_batch=[0], idx_batch=[0])
        ins = [x, cols]
    elif case == "unaligned_windows":
        # 3x8 windows of a [50, 12] f32 table at (row, column) start pairs: rows of whole vectors, origins mostly not
        # on a vector boundary (the kernel's element path inside its vector form)
        x = _tensor(24, (50, 12), "f32")
        starts = np.random.default_rng(25).integers(-3, 60, size=(5, 7, 2)).astype(np.int32)
        prog = gather_program("tensor<50x12xf32>", "tensor<5x7x2xi32>", "tensor<5x7x3x8xf32>", [2, 3], [], [0, 1],
                              2, [3, 8])
        ins = [x, configs.HostInput(starts, pjrt.BufferType.S32, (5, 7, 2))]
    else:
        # the printed form of the reference's builder test with data of its shapes
        from tests.test_dynamic_window import GATHER_PRINTED
        prog = GATHER_PRINTED
        ins = [_tensor(26, (3, 4, 2), "i64"),
               configs.HostInput(np.random.default_rng(27).integers(-1, 5, size=(2, 3, 2)).astype(np.int64),
                                 pjrt.BufferType.S64, (2, 3, 2))]
    _check_exact(gpu_client, prog, ins, f"gather {case}")
