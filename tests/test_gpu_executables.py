"""GPU checks of the executable and buffer entry points around the hot path: the sequence of ryft-pjrt's
test_client_compile (programs.rs:2576-2623) against a device client, serialized executables that run like the
original (test_client_deserialize_and_load_executable, programs.rs:2691-2723), and raw byte-range copies to the host
(Buffer::copy_raw_to_host_buffer, buffers.rs:1318-1340)."""
import ctypes

import numpy as np
import pytest

from ryft_amd import configs, hostdata as hd, pjrt, profiler
from tests.helpers import run_pjrt

pytestmark = pytest.mark.gpu

ADD_PROGRAM = """module {
  func.func @main(%arg0: tensor<2x1xi32>, %arg1: tensor<2x1xi32>) -> tensor<2x1xi32> {
    %0 = stablehlo.add %arg0, %arg1 : tensor<2x1xi32>
    return %0 : tensor<2x1xi32>
  }
}
"""


def test_client_compile_sequence(gpu_client):
    opts = pjrt.CompilationOptions()
    le = gpu_client.compile(pjrt.Program.mlir(ADD_PROGRAM), opts)
    assert le.addressable_devices() == gpu_client.addressable_devices()[:1]
    assert le.device_assignment() == pjrt.DeviceAssignment(1, 1, [0])
    e = le.executable()
    assert e.name() == "main"
    assert (e.replica_count(), e.computation_count(), e.output_count()) == (1, 1, 1)
    assert e.output_element_types() == [pjrt.BufferType.S32]
    assert e.output_dimensions() == [[2, 1]]
    assert e.input_memory_kinds() == ["device", "device"]
    assert e.output_memory_kinds() == ["device"]
    assert e.fingerprint()
    assert e.compile_options() == opts.encode()
    assert e.memory_statistics()["argument_size_in_bytes"] == 16
    assert e.serialize()
    # the i32 add known answer (programs.rs:2823-2827)
    ins = [configs.HostInput(np.array([[7], [-50]], np.int32), pjrt.BufferType.S32, (2, 1)),
           configs.HostInput(np.array([[35], [8]], np.int32), pjrt.BufferType.S32, (2, 1))]
    outs, _ = run_pjrt(gpu_client, ADD_PROGRAM, ins)
    assert outs[0].reshape(-1).tolist() == [42, -42]


@pytest.mark.parametrize("cfg,kw", [("c2", {"batch": 2, "m": 256, "k": 256, "n": 256}),
                                    ("c3", {"m": 256, "k": 512, "n": 256}),
                                    ("c4", {"b": 1, "h": 2, "s": 256})])
def test_deserialized_executable_runs_like_the_original(gpu_client, cfg, kw):
    w = {"c2": configs.c2_bf16_batched_dot, "c3": configs.c3_int8_gemm, "c4": configs.c4_causal_attention}[cfg](**kw)
    le = gpu_client.compile(pjrt.Program.mlir(w.program))
    le2 = gpu_client.deserialize_and_load_executable(le.executable().serialize())
    assert le2.device_assignment() == le.device_assignment()
    dev = gpu_client.addressable_devices()[0]
    bufs = [gpu_client.buffer(x.data, x.type, x.dims, device=dev) for x in w.inputs]
    a = le.execute([bufs])[0]
    b = le2.execute([bufs])[0]
    a.done.await_()
    b.done.await_()
    for x, y in zip(a.outputs, b.outputs):
        assert np.array_equal(x.to_numpy(), y.to_numpy())


def test_copy_raw_to_host_ranges(gpu_client):
    dev = gpu_client.addressable_devices()[0]
    x = hd.int_uniform(5, (1000,), -2 ** 31, 2 ** 31 - 1).astype(np.int32)
    b = gpu_client.buffer(x, pjrt.BufferType.S32, (1000,), device=dev)
    b.ready_event().await_()
    raw = x.tobytes()
    assert b.copy_raw_to_host(4000).await_() == raw
    for off, size in [(0, 1), (8, 100), (3, 17), (3999, 1), (4000, 0), (0, 0)]:
        assert b.copy_raw_to_host(size, off).await_() == raw[off:off + size], (off, size)
    # ranges outside the buffer are rejected before anything is copied (the host array is large enough either way)
    dst = (ctypes.c_uint8 * 8192)()
    for off, size in [(0, 4001), (4000, 1), (-1, 4), (10, -2)]:
        with pytest.raises(pjrt.PjrtError) as e:
            b.api.call("PJRT_Buffer_CopyRawToHost", buffer=b.handle, dst=ctypes.cast(dst, ctypes.c_void_p), offset=off,
                       transfer_size=size)
        assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT, (off, size)
    b.delete()
    with pytest.raises(pjrt.PjrtError) as e:
        b.copy_raw_to_host(4)
    assert e.value.code == pjrt.ErrorCode.FAILED_PRECONDITION


def test_buffer_memory_layout(gpu_client):
    # buffers are dense row-major; the layout handed out is the caller's (destroyed when dropped)
    dev = gpu_client.addressable_devices()[0]
    for dims in [(3, 4, 5), (7,), ()]:
        x = np.zeros(dims, np.float32)
        b = gpu_client.buffer(x, pjrt.BufferType.F32, dims, device=dev)
        layout = b.memory_layout()
        assert layout.serialize() == "{" + ",".join(str(len(dims) - 1 - i) for i in range(len(dims))) + "}"
        assert not layout.borrowed
        assert layout == gpu_client.default_layout(pjrt.BufferType.F32, list(dims))


def test_device_memory_descriptions(gpu_client):
    # ryft-pjrt's test_device_memory_descriptions (extensions/memory_descriptions.rs:297-316): non-empty kinds,
    # non-zero kind ids, a default; the one memory is HBM, kind "device", with the kind id XLA's plugins use for it
    # (memories.rs:354), the same one Memory_Kind_Id reports
    device = gpu_client.addressable_devices()[0]
    descs, default = device.memory_descriptions()
    assert descs == [("device", 42097224)] and default == 0
    mem = device.default_memory()
    assert mem.kind() == "device"
    assert mem.kind_id() == 42097224


def test_compile_options_choose_the_device(gpu_client):
    """device_ordinal / a one-device assignment pick the executable's device; a device the client does not have is
    INVALID_ARGUMENT at compile time; an explicit device_ordinal 0 runs like the default."""
    n = len(gpu_client.addressable_devices())
    with pytest.raises(pjrt.PjrtError) as e:
        gpu_client.compile(pjrt.Program.mlir(ADD_PROGRAM), pjrt.CompilationOptions(device_ordinal=n))
    assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT
    le = gpu_client.compile(pjrt.Program.mlir(ADD_PROGRAM), pjrt.CompilationOptions(device_ordinal=0))
    assert le.addressable_devices() == gpu_client.addressable_devices()[:1]
    a = configs.HostInput(np.array([[7], [-1]], np.int32), pjrt.BufferType.S32, (2, 1))
    b = configs.HostInput(np.array([[35], [-41]], np.int32), pjrt.BufferType.S32, (2, 1))
    outs, _ = run_pjrt(gpu_client, "", [a, b], executable=le)
    assert outs[0].ravel().tolist() == [42, -42]


def test_profiler(gpu_client):
    """ryft-pjrt's test_profiler (extensions/profiler.rs:552-628): profile compiling and running the i32 add known
    answer; the results hold no errors, the host plane the compilation and the execution, and the device plane the
    add's kernel step with its algorithmic bytes."""
    opts = profiler.ProfileOptions(version=1, device_type=1, host_tracing_level=2, device_tracing_level=1)
    prof = gpu_client.profiler(opts)
    other = gpu_client.profiler(opts)  # two sessions started together both record
    prof.start()
    other.start()
    ins = [configs.HostInput(np.array([[7], [-1]], np.int32), pjrt.BufferType.S32, (2, 1)),
           configs.HostInput(np.array([[35], [-41]], np.int32), pjrt.BufferType.S32, (2, 1))]
    outs, _ = run_pjrt(gpu_client, ADD_PROGRAM, ins)
    assert outs[0].reshape(-1).tolist() == [42, -42]
    prof.stop()
    other.stop()
    space = prof.results()
    assert space.errors == []
    host = [e.name for e in space.plane("/host:CPU").lines[0].events]
    assert "compile main" in host and "execute main" in host
    dev = space.plane("/device:GPU:0")
    assert dev is not None
    (line,) = dev.lines
    assert len(line.events) >= 1
    for ev in line.events:
        assert ev.duration_ps > 0 and ev.offset_ps >= 0
    assert sum(ev.stats["bytes accessed"] for ev in line.events) == 24  # two 8-byte operands, one 8-byte result
    assert [e.name for e in other.results().plane("/device:GPU:0").lines[0].events] == [e.name for e in line.events]


def test_profiler_device_events_time_the_gemm(gpu_client):
    """A bf16 batched GEMM under the profiler: one device event per plan step, named by its kernel, with the step's
    algorithmic flops, lasting about what the plugin's own kernel timing reports for the same steps."""
    w = configs.c2_bf16_batched_dot(batch=4, m=512, k=512, n=512)
    le = gpu_client.compile(pjrt.Program.mlir(w.program))
    dev = gpu_client.addressable_devices()[0]
    bufs = [gpu_client.buffer(x.data, x.type, x.dims, device=dev) for x in w.inputs]
    le.execute([bufs])[0].done.await_()  # warm
    prof = gpu_client.profiler()
    prof.start()
    for _ in range(3):
        le.execute([bufs])[0].done.await_()
    prof.stop()
    line = prof.results().plane("/device:GPU:0").lines[0]
    gemm = [e for e in line.events if e.name.startswith("gemm_bf16")]
    assert len(gemm) == 3, [e.name for e in line.events]
    for e in gemm:
        assert e.stats["flops"] == 2.0 * 4 * 512 * 512 * 512
        assert 1e6 < e.duration_ps < 5e9  # 1 µs .. 5 ms
    offs = [e.offset_ps for e in gemm]
    assert offs == sorted(offs) and offs[0] >= 0
