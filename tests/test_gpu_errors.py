"""Failure propagation through buffers, on the GPU: error buffers (Client::error_buffer, ryft-pjrt's
test_client_error_buffer, crates/ryft-pjrt/src/buffers.rs:4234-4260) and poisoned executions
(Device::poison_execution, test_device_poison_execution, devices.rs:1255-1363). An error buffer holds an error
instead of data: its ready event, copies of it to the host or to a device and executions that take it all fail with
that error, payload included. A poisoned execution still runs its kernels to the end, then completes with the poison's
error, and its results are error buffers from the moment it is poisoned."""
import numpy as np
import pytest

from ryft_amd import configs, pjrt

pytestmark = pytest.mark.gpu

ADD_PROGRAM = """module {
  func.func @main(%arg0: tensor<4xui8>, %arg1: tensor<4xui8>) -> tensor<4xui8> {
    %0 = stablehlo.add %arg0, %arg1 : tensor<4xui8>
    return %0 : tensor<4xui8>
  }
}
"""

DOT_4096 = """module {
  func.func @main(%arg0: tensor<4096x4096xf32>, %arg1: tensor<4096x4096xf32>) -> tensor<4096x4096xf32> {
    %0 = stablehlo.dot_general %arg0, %arg1, batching_dims = [] x [], contracting_dims = [1] x [0] : (tensor<4096x4096xf32>, tensor<4096x4096xf32>) -> tensor<4096x4096xf32>
    return %0 : tensor<4096x4096xf32>
  }
}
"""


def _raises(fn, code, message):
    with pytest.raises(pjrt.PjrtError) as e:
        fn()
    assert e.value.code == code and message in e.value.message, (e.value.code, e.value.message)
    return e.value


def test_client_error_buffer(gpu_client):
    error = pjrt.PjrtError(pjrt.ErrorCode.ABORTED, "test error")
    b = gpu_client.error_buffer(error, pjrt.BufferType.U8, [4])
    assert b.element_type() == pjrt.BufferType.U8 and b.dimensions() == [4]
    _raises(lambda: b.ready_event().await_(), pjrt.ErrorCode.ABORTED, "test error")

    payload = {"launch_id": "17", "reason": "unit-test"}
    b = gpu_client.error_buffer(error, pjrt.BufferType.U8, [4], payload=payload)
    err = _raises(lambda: b.ready_event().await_(), pjrt.ErrorCode.ABORTED, "test error")
    assert dict(err.payload) == payload
    assert dict(err.payload).get("missing") is None


def test_error_buffer_consumers_fail_with_its_error(gpu_client):
    payload = {"reason": "consumer"}
    b = gpu_client.error_buffer(pjrt.PjrtError(pjrt.ErrorCode.DATA_LOSS, "lost bytes"), pjrt.BufferType.U8, [4],
                                payload=payload)
    # copies to the host (ToHostBuffer, CopyRawToHost) and to a device
    for fn in (lambda: b.to_numpy(), lambda: b.copy_to_host().await_(), lambda: b.copy_raw_to_host(2, 1).await_(),
               lambda: b.copy_to_device(gpu_client.addressable_devices()[0]).ready_event().await_()):
        err = _raises(fn, pjrt.ErrorCode.DATA_LOSS, "lost bytes")
        assert dict(err.payload) == payload
    # an execution that takes it fails at once with the same error; nothing runs
    le = gpu_client.compile(pjrt.Program.mlir(ADD_PROGRAM))
    good = gpu_client.buffer(np.array([1, 2, 3, 4], np.uint8), pjrt.BufferType.U8, (4,))
    err = _raises(lambda: le.execute([[good, b]]), pjrt.ErrorCode.DATA_LOSS, "lost bytes")
    assert dict(err.payload) == payload
    # the same executable still runs on good buffers
    out = le.execute([[good, good]])[0]
    out.done.await_()
    assert out.outputs[0].to_numpy().tolist() == [2, 4, 6, 8]


def test_error_buffer_rejects_an_ok_code(gpu_client):
    _raises(lambda: gpu_client.error_buffer(pjrt.PjrtError(pjrt.ErrorCode.OK, "fine"), pjrt.BufferType.F32, [2]),
            pjrt.ErrorCode.INVALID_ARGUMENT, "OK")


def test_device_poison_execution(gpu_client):
    device = gpu_client.addressable_devices()[0]
    le = gpu_client.compile(pjrt.Program.mlir(DOT_4096))
    x = np.zeros((4096, 4096), np.float32)
    bufs = [gpu_client.buffer(x, pjrt.BufferType.F32, (4096, 4096)) for _ in range(2)]
    # three executions queued ahead on the device's one stream keep the poisoned one from finishing before the poison
    ahead = [le.execute([bufs], launch_id=3)[0] for _ in range(3)]
    target = le.execute([bufs], launch_id=17)[0]
    payload = {"launch_id": "17", "reason": "unit-test"}
    assert device.poison_execution(17, pjrt.PjrtError(pjrt.ErrorCode.ABORTED, "test poison error"), payload)
    err = _raises(lambda: target.done.await_(), pjrt.ErrorCode.ABORTED, "test poison error")
    assert err.message == "test poison error"
    assert dict(err.payload) == payload
    # its result is an error buffer; the executions ahead of it are untouched
    _raises(lambda: target.outputs[0].to_numpy(), pjrt.ErrorCode.ABORTED, "test poison error")
    for a in ahead:
        a.done.await_()
        assert not np.any(a.outputs[0].to_numpy())
    # finished executions (and launch ids never used) cannot be poisoned
    assert not device.poison_execution(17, pjrt.PjrtError(pjrt.ErrorCode.ABORTED, "late"))
    assert not device.poison_execution(3, pjrt.PjrtError(pjrt.ErrorCode.ABORTED, "late"))
    assert not device.poison_execution(12345, pjrt.PjrtError(pjrt.ErrorCode.ABORTED, "never"))
    # a result of the poisoned execution fails an execution that takes it
    _raises(lambda: le.execute([[target.outputs[0], bufs[1]]]), pjrt.ErrorCode.ABORTED, "test poison error")


def test_poison_takes_the_earliest_unfinished_execution(gpu_client):
    device = gpu_client.addressable_devices()[0]
    w = configs.c2_bf16_batched_dot()
    le = gpu_client.compile(pjrt.Program.mlir(w.program))
    bufs = [gpu_client.buffer(i.data, i.type, i.dims) for i in w.inputs]
    ref = le.execute([bufs])[0]
    ref.done.await_()
    want = ref.outputs[0].to_numpy()
    # long executions queued ahead keep all four from finishing before the poisons
    big = gpu_client.compile(pjrt.Program.mlir(DOT_4096))
    x = [gpu_client.buffer(np.zeros((4096, 4096), np.float32), pjrt.BufferType.F32, (4096, 4096)) for _ in range(2)]
    ahead = [big.execute([x])[0] for _ in range(3)]
    runs = [le.execute([bufs], launch_id=5)[0] for _ in range(4)]
    assert device.poison_execution(5, pjrt.PjrtError(pjrt.ErrorCode.CANCELLED, "first"))
    assert device.poison_execution(5, pjrt.PjrtError(pjrt.ErrorCode.CANCELLED, "second"))
    _raises(lambda: runs[0].done.await_(), pjrt.ErrorCode.CANCELLED, "first")
    _raises(lambda: runs[1].done.await_(), pjrt.ErrorCode.CANCELLED, "second")
    for r in runs[2:]:
        r.done.await_()
        assert np.array_equal(r.outputs[0].to_numpy(), want)
    for a in ahead:
        a.done.await_()
