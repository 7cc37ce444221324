"""The allocation-free entry point RyftMi355x_ExecuteNoAlloc (include/ryft_mi355x.h), called through the C ABI, gives
the same bits as PJRT_LoadedExecutable_Execute on the same executable and inputs: twice in a row, the second call on
a smaller executable, so the shared scratch array holds the first call's intermediates when the second starts."""
import ctypes as C

import numpy as np
import pytest

from ryft_amd import configs, pjrt

pytestmark = pytest.mark.gpu


def _entry(plugin):
    f = plugin.lib.RyftMi355x_ExecuteNoAlloc
    f.restype = C.c_int
    f.argtypes = [C.c_void_p, C.POINTER(C.c_void_p), C.POINTER(C.c_size_t), C.c_size_t, C.POINTER(C.c_void_p),
                  C.POINTER(C.c_size_t), C.c_size_t, C.c_void_p, C.POINTER(C.c_char_p)]
    return f


def _hip():
    lib = C.CDLL("libamdhip64.so")
    lib.hipDeviceSynchronize.restype = C.c_int
    return lib


def _call(plugin, exe, ins, in_sizes, outs, out_sizes):
    f = _entry(plugin)
    msg = C.c_char_p()
    rc = f(exe.handle, (C.c_void_p * max(len(ins), 1))(*ins), (C.c_size_t * max(len(ins), 1))(*in_sizes), len(ins),
           (C.c_void_p * max(len(outs), 1))(*outs), (C.c_size_t * max(len(outs), 1))(*out_sizes), len(outs), None,
           C.byref(msg))
    return rc, (msg.value or b"").decode()


def _compare(plugin, client, w):
    print(f"[no-alloc] {w.name} {[x.dims for x in w.inputs]}", flush=True)
    exe = client.compile(pjrt.Program.mlir(w.program))
    bufs = [client.buffer(x.data, x.type, x.dims) for x in w.inputs]
    for b in bufs:
        b.ready_event().await_()
    ref = exe.execute([bufs])[0]
    ref.done.await_()
    want = [o.to_numpy() for o in ref.outputs]
    outs = [client.uninitialized_buffer(o.element_type(), o.dimensions()) for o in ref.outputs]
    rc, msg = _call(plugin, exe, [b.unsafe_pointer() for b in bufs], [b.on_device_size_in_bytes() for b in bufs],
                    [o.unsafe_pointer() for o in outs], [o.on_device_size_in_bytes() for o in outs])
    assert rc == 0, msg
    assert _hip().hipDeviceSynchronize() == 0
    for i, (o, r) in enumerate(zip(outs, want)):
        got = o.to_numpy()
        assert got.dtype == r.dtype and got.shape == r.shape
        assert np.array_equal(got.view(np.uint8), r.view(np.uint8)), f"{w.name} output {i} differs from Execute"
    return exe, bufs, outs


def test_no_alloc_matches_execute_twice(plugin, gpu_client):
    # C5 at full size (split-K partial sums, a normalised activation and the SwiGLU product in scratch), then a
    # smaller C5 whose intermediates overwrite a prefix of what the first call left there
    _compare(plugin, gpu_client, configs.c5_swiglu_fp8())
    _compare(plugin, gpu_client, configs.c5_swiglu_fp8(m=128, d=1024, f=2048))


def test_no_alloc_rejects_what_it_cannot_run(plugin, gpu_client):
    # intermediates beyond the 64 MiB scratch: an unfused attention over 4 heads of 2048 keys keeps f32 score
    # matrices of 64 MiB each; nothing is launched
    w = configs.c4_causal_attention(b=1, h=4, s=2048, d=128, mask="GT")
    exe = gpu_client.compile(pjrt.Program.mlir(w.program))
    assert "attention_fwd" not in exe.describe_plan()
    # real, correctly sized buffers: should the plan ever fit the scratch, the call runs on valid memory and the
    # wrong return code is what fails
    ins = [gpu_client.uninitialized_buffer(x.type, x.dims) for x in w.inputs]
    out = gpu_client.uninitialized_buffer(w.inputs[0].type, w.inputs[0].dims)
    sizes = [b.on_device_size_in_bytes() for b in ins]
    rc, msg = _call(plugin, exe, [b.unsafe_pointer() for b in ins], sizes, [out.unsafe_pointer()],
                    [out.on_device_size_in_bytes()])
    assert _hip().hipDeviceSynchronize() == 0
    assert rc == pjrt.ErrorCode.RESOURCE_EXHAUSTED and "scratch" in msg, (rc, msg)
    # a size that is not the program's, and a misaligned pointer: rejected before anything is launched
    w = configs.c2_bf16_batched_dot(batch=1, m=256, k=256, n=256)
    exe = gpu_client.compile(pjrt.Program.mlir(w.program))
    bufs = [gpu_client.buffer(x.data, x.type, x.dims) for x in w.inputs]
    out = gpu_client.uninitialized_buffer(pjrt.BufferType.BF16, (1, 256, 256))
    ptrs = [b.unsafe_pointer() for b in bufs]
    rc, msg = _call(plugin, exe, ptrs, [256 * 256 * 2, 100], [out.unsafe_pointer()], [256 * 256 * 2])
    assert rc == pjrt.ErrorCode.INVALID_ARGUMENT and "input 1" in msg, (rc, msg)
    rc, msg = _call(plugin, exe, [ptrs[0] + 16, ptrs[1]], [256 * 256 * 2] * 2, [out.unsafe_pointer()], [256 * 256 * 2])
    assert rc == pjrt.ErrorCode.INVALID_ARGUMENT and "aligned" in msg, (rc, msg)
    rc, msg = _call(plugin, exe, ptrs, [256 * 256 * 2] * 2, [], [])
    assert rc == pjrt.ErrorCode.INVALID_ARGUMENT and "output" in msg, (rc, msg)
