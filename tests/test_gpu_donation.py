"""Input donation on the GPU (ExecutionInput::donatable, crates/ryft-pjrt/src/programs.rs:784-810, 865-893,
1003-1016): a donated argument aliased to a result is consumed by the execution (its buffer reads as deleted, its
memory becomes the result's when the plan computes in place); a non-donatable one is copy-protected (the result gets
a buffer of its own and the argument stays valid). Results are checked against the oracle either way."""
import numpy as np
import pytest

from ryft_amd import configs, hostdata as hd, pjrt
from tests import donation_programs as dp, mlir_bytecode
from tests.helpers import check, oracle_outputs

pytestmark = pytest.mark.gpu


def _inputs(program_name, seed=0):
    rng = np.random.default_rng(seed)
    if program_name == "SGD":
        return [configs.HostInput(rng.standard_normal(dp.N).astype(np.float32), pjrt.BufferType.F32, (dp.N,))
                for _ in range(2)]
    if program_name == "GEMM":
        return [configs.HostInput(hd.f32_to_bf16_bits((rng.standard_normal((256, 256)) / 16).astype(np.float32)),
                                  pjrt.BufferType.BF16, (256, 256)) for _ in range(2)]
    if program_name == "TRANSPOSED":
        return [configs.HostInput(rng.standard_normal((64, 64)).astype(np.float32), pjrt.BufferType.F32, (64, 64))]
    if program_name == "PASSTHROUGH":
        return [configs.HostInput(rng.integers(-1000, 1000, 1024, dtype=np.int32), pjrt.BufferType.S32, (1024,))
                for _ in range(2)]
    return [configs.HostInput(rng.standard_normal(512).astype(np.float32), pjrt.BufferType.F32, (512,)),
            configs.HostInput(rng.integers(-1000, 1000, 512, dtype=np.int32), pjrt.BufferType.S32, (512,))]


def _run(client, program, host_inputs, donate, code=None):
    le = client.compile(pjrt.Program.mlir(code or program))
    dev = le.addressable_devices()[0]
    bufs = [client.buffer(x.data, x.type, x.dims, device=dev) for x in host_inputs]
    ptrs = [b.unsafe_pointer() for b in bufs]
    out = le.execute([[pjrt.ExecutionInput(b, donatable=donate) for b in bufs]])[0]
    out.done.await_()
    return le, bufs, ptrs, out.outputs


@pytest.mark.parametrize("name,param,result,in_place", [("SGD", 0, 0, True), ("GEMM", 0, 0, False),
                                                        ("TRANSPOSED", 0, 0, False), ("PASSTHROUGH", 0, 1, True),
                                                        ("DONOR", 0, 1, True)])
def test_donated_argument_is_consumed(gpu_client, name, param, result, in_place):
    program = getattr(dp, name)
    host = _inputs(name)
    _, bufs, ptrs, outs = _run(gpu_client, program, host, donate=True)
    assert bufs[param].is_deleted()
    assert all(not b.is_deleted() for i, b in enumerate(bufs) if i != param)
    assert (outs[result].unsafe_pointer() == ptrs[param]) == in_place
    want = oracle_outputs(program, host)
    for o, w in zip(outs, want):
        check(o.to_numpy(), w, 2e-2 if name == "GEMM" else 1e-6, name)
    with pytest.raises(pjrt.PjrtError) as e:  # a donated buffer cannot be used again
        bufs[param].to_numpy()
    assert e.value.code == pjrt.ErrorCode.FAILED_PRECONDITION


@pytest.mark.parametrize("name", ["SGD", "GEMM", "PASSTHROUGH"])
def test_non_donatable_argument_is_copy_protected(gpu_client, name):
    program = getattr(dp, name)
    host = _inputs(name, seed=1)
    _, bufs, ptrs, outs = _run(gpu_client, program, host, donate=False)
    assert not any(b.is_deleted() for b in bufs)
    assert all(o.unsafe_pointer() not in ptrs for o in outs)
    for b, x in zip(bufs, host):  # the arguments are unchanged
        assert b.to_numpy().tobytes() == np.ascontiguousarray(x.data).tobytes()
    for o, w in zip(outs, oracle_outputs(program, host)):
        check(o.to_numpy(), w, 2e-2 if name == "GEMM" else 1e-6, name)


def test_donation_through_bytecode(gpu_client):
    host = _inputs("SGD", seed=2)
    _, bufs, ptrs, outs = _run(gpu_client, dp.SGD, host, donate=True, code=mlir_bytecode.to_bytecode(dp.SGD))
    assert bufs[0].is_deleted() and outs[0].unsafe_pointer() == ptrs[0]
    check(outs[0].to_numpy(), oracle_outputs(dp.SGD, host)[0], 1e-6, "SGD bytecode")


def test_repeated_in_place_updates(gpu_client):
    """Ten optimizer steps, each donating the previous step's result: the parameter stays in one allocation."""
    le = gpu_client.compile(pjrt.Program.mlir(dp.SGD))
    dev = le.addressable_devices()[0]
    rng = np.random.default_rng(3)
    w = rng.standard_normal(dp.N).astype(np.float32)
    g = rng.standard_normal(dp.N).astype(np.float32)
    wb = gpu_client.buffer(w, pjrt.BufferType.F32, (dp.N,), device=dev)
    gb = gpu_client.buffer(g, pjrt.BufferType.F32, (dp.N,), device=dev)
    p0 = wb.unsafe_pointer()
    for _ in range(10):
        out = le.execute([[pjrt.ExecutionInput(wb, donatable=True), gb]])[0]
        wb = out.outputs[0]
    out.done.await_()
    assert wb.unsafe_pointer() == p0
    want = w.copy()
    for _ in range(10):
        want = (want - (g * np.float32(0.125)).astype(np.float32)).astype(np.float32)
    assert np.array_equal(wb.to_numpy(), want)


def test_donation_errors(gpu_client):
    le = gpu_client.compile(pjrt.Program.mlir(dp.SGD))
    dev = le.addressable_devices()[0]
    x = gpu_client.buffer(np.ones(dp.N, np.float32), pjrt.BufferType.F32, (dp.N,), device=dev)
    with pytest.raises(pjrt.PjrtError) as e:  # the donated buffer is also the other argument
        le.execute([[pjrt.ExecutionInput(x, donatable=True), x]])
    assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT and "also argument 1" in str(e.value)
    assert not x.is_deleted()
    # an unaliased argument marked donatable is not consumed
    y = gpu_client.buffer(np.ones(dp.N, np.float32), pjrt.BufferType.F32, (dp.N,), device=dev)
    out = le.execute([[x, pjrt.ExecutionInput(y, donatable=True)]])[0]
    out.done.await_()
    assert not x.is_deleted() and not y.is_deleted()
    assert np.array_equal(out.outputs[0].to_numpy(), np.full(dp.N, 0.875, np.float32))
