"""GPU parity: every config through the PJRT C API (client.compile → buffer → execute → await → copy_to_host),
compared with the oracle on the same seeded inputs.

Tolerances (normwise relative error): f32 1e-4; bf16 1e-2; int8→i32 bit-exact and the scaled f32
output 1e-5; causal attention 2e-2; fp8 SwiGLU 3e-2. Full BASELINE sizes run for C1, C2, C3 and C5; C4 at full size
is checked on sampled heads plus size-independent properties (finite output, row 0 equals V[0]).
"""
import time

import numpy as np
import pytest

from oracle import numerics as nm
from oracle import stablehlo as sh
from ryft_amd import configs, pjrt
from tests.helpers import MLIR_DT, check, oracle_outputs, run_pjrt

pytestmark = pytest.mark.gpu


def _run_and_check(client, w, oracle_w=None):
    print(f"[parity] {w.name}", flush=True)
    outs, exe = run_pjrt(client, w.program, w.inputs)
    want = oracle_outputs((oracle_w or w).program, (oracle_w or w).inputs)
    errs = [check(o, r, w.tolerance, f"{w.name}[{i}]") for i, (o, r) in enumerate(zip(outs, want))]
    print(f"[parity] {w.name} errors {errs}", flush=True)
    return outs, exe


def test_client_basics(gpu_client):
    c = gpu_client
    assert c.platform_name() == "rocm"
    devs = c.addressable_devices()
    assert len(devs) >= 1
    d = devs[0]
    assert d.attributes()["gfx_arch"].startswith("gfx950")
    assert d.default_memory().kind() == "device"
    assert c.lookup_device(0) == d
    with pytest.raises(pjrt.PjrtError) as e:
        c.lookup_device(len(devs))
    assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT


@pytest.mark.parametrize("bt,np_t", [(pjrt.BufferType.F32, np.float32), (pjrt.BufferType.BF16, np.uint16),
                                     (pjrt.BufferType.S8, np.int8), (pjrt.BufferType.S32, np.int32),
                                     (pjrt.BufferType.F8E4M3FN, np.uint8), (pjrt.BufferType.PRED, np.bool_),
                                     (pjrt.BufferType.F64, np.float64), (pjrt.BufferType.U8, np.uint8)])
def test_buffer_round_trip(gpu_client, bt, np_t):
    # buffers.rs:3874-3923: bytes in == bytes out
    rng = np.random.default_rng(int(bt))
    raw = rng.integers(0, 256, size=3 * 5 * 7 * np.dtype(np_t).itemsize, dtype=np.uint8)
    if np_t == np.bool_:
        raw = raw & 1
    b = gpu_client.buffer(raw.tobytes(), bt, (3, 5, 7))
    assert b.element_type() == bt and b.dimensions() == [3, 5, 7]
    assert not b.is_on_cpu()
    assert b.on_device_size_in_bytes() == raw.size
    assert b.copy_to_host().await_() == raw.tobytes()


@pytest.mark.parametrize("n,bt,np_t", [((16 << 20) + 1, pjrt.BufferType.U8, np.uint8),
                                       ((24 << 20) + 2, pjrt.BufferType.U8, np.uint8),
                                       (10485761, pjrt.BufferType.F32, np.float32)])
def test_buffer_round_trip_split_copies(gpu_client, n, bt, np_t):
    # sizes whose host staging copy is split over 2, 3 and 5 threads with a remainder the page-rounded pieces must
    # still cover; a stained staging block first, so stale bytes from an earlier transfer cannot pass for the data
    print(f"[round trip] {n} x {np.dtype(np_t).name}", flush=True)
    rng = np.random.default_rng(n)
    stain = np.frombuffer(np.full(n * np.dtype(np_t).itemsize, 0x5A, np.uint8).tobytes(), dtype=np_t)
    gpu_client.buffer(stain, bt, (n,)).to_numpy()
    raw = rng.integers(0, 256, size=n * np.dtype(np_t).itemsize, dtype=np.uint8)
    raw[-64:] = np.arange(1, 65, dtype=np.uint8)          # the tail carries no 0x5A byte
    x = raw.view(np_t)
    b = gpu_client.buffer(x, bt, (n,))
    back = b.to_numpy()
    assert np.array_equal(back.view(np.uint8), raw)
    assert b.copy_to_host().await_() == raw.tobytes()


def test_buffer_strided_upload(gpu_client):
    x = np.arange(12, dtype=np.float32).reshape(3, 4)
    xt = np.asfortranarray(x)
    b = gpu_client.buffer(xt.tobytes(order="A"), pjrt.BufferType.F32, (3, 4), byte_strides=(4, 12))
    assert np.array_equal(b.to_numpy(), x)


def test_readme_kat(gpu_client):
    prog = """module {
  func.func @main(%arg0: tensor<2x3xf32>, %arg1: tensor<3x2xf32>) -> tensor<2x2xf32> {
    %0 = stablehlo.dot_general %arg0, %arg1, contracting_dims = [1] x [0] : (tensor<2x3xf32>, tensor<3x2xf32>) -> tensor<2x2xf32>
    return %0 : tensor<2x2xf32>
  }
}"""
    exe = gpu_client.compile(pjrt.Program.mlir(prog), pjrt.CompilationOptions())
    device = exe.addressable_devices()[0]
    lhs = gpu_client.buffer(np.array([1, 2, 3, 4, 5, 6], np.float32), pjrt.BufferType.F32, (2, 3), device=device)
    rhs = gpu_client.buffer(np.array([7, 8, 9, 10, 11, 12], np.float32), pjrt.BufferType.F32, (3, 2), device=device)
    out = exe.execute([[lhs, rhs]])[0]
    out.done.await_()
    got = np.frombuffer(out.outputs[0].copy_to_host().await_(), np.float32)
    assert got.tolist() == [58.0, 64.0, 139.0, 154.0]


def test_add_kat(gpu_client):
    prog = """module {
  func.func @main(%arg0: tensor<2xi32>, %arg1: tensor<2xi32>) -> tensor<2xi32> {
    %0 = stablehlo.add %arg0, %arg1 : tensor<2xi32>
    return %0 : tensor<2xi32>
  }
}"""
    exe = gpu_client.compile(pjrt.Program.mlir(prog))
    a = gpu_client.buffer(np.array([7, -1], np.int32), pjrt.BufferType.S32, (2,))
    b = gpu_client.buffer(np.array([35, -41], np.int32), pjrt.BufferType.S32, (2,))
    out = exe.execute([[a, b]])[0]
    seen = []
    out.done.on_ready(lambda err: seen.append(err))
    out.done.await_()
    assert out.outputs[0].to_numpy().tolist() == [42, -42]
    assert out.done.is_ready()
    deadline = time.time() + 10
    while not seen and time.time() < deadline:  # the callback may run on the completion worker
        time.sleep(0.001)
    assert seen == [None]


def test_execution_event_callbacks_without_await(gpu_client):
    """Callbacks registered on a pending execution event fire once, with no error, when nothing awaits it
    (events.rs:90-120 `on_ready`); later registrations on the ready event run at once."""
    import threading
    w = configs.c2_bf16_batched_dot(batch=2, m=256, k=256, n=256)
    exe = gpu_client.compile(pjrt.Program.mlir(w.program))
    bufs = [gpu_client.buffer(x.data, x.type, x.dims) for x in w.inputs]
    fired = threading.Event()
    seen = []
    outs = [exe.execute([bufs])[0] for _ in range(4)]
    outs[-1].done.on_ready(lambda err: (seen.append(err), fired.set()))
    assert fired.wait(30), "OnReady callback of an execution event never ran"
    assert seen == [None] and outs[-1].done.is_ready()
    late = []
    outs[-1].done.on_ready(lambda err: late.append(err))
    assert late == [None]
    for o in outs[:-1]:
        o.done.await_()


def test_execute_validates_arguments(gpu_client):
    w = configs.c1_f32_dot(m=64, k=32, n=64)
    exe = gpu_client.compile(pjrt.Program.mlir(w.program))
    a = gpu_client.buffer(w.inputs[0].data, w.inputs[0].type, w.inputs[0].dims)  # [64, 32]; the rhs is [32, 64]
    with pytest.raises(pjrt.PjrtError) as e:
        exe.execute([[a]])
    assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT
    with pytest.raises(pjrt.PjrtError) as e:
        exe.execute([[a, a]])  # wrong shape for the rhs
    assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT


def test_c1_f32_full(gpu_client):
    _run_and_check(gpu_client, configs.c1_f32_dot())


@pytest.mark.parametrize("kw", [dict(m=128, k=1024, n=128), dict(m=256, k=1024, n=128), dict(m=128, k=2048, n=192)])
def test_f32_split_k_ranges(gpu_client, kw):
    # split-K f32 GEMMs over 16 K ranges of 64 (the first two) and 128 (the last) elements, ragged N / M ratios
    w = configs.c1_f32_dot(**kw)
    exe = gpu_client.compile(pjrt.Program.mlir(w.program))
    assert "_splitk" in exe.describe_plan()
    _run_and_check(gpu_client, w)


@pytest.mark.parametrize("kw", [dict(batch=2, m=128, k=128, n=128), dict(batch=1, m=64, k=96, n=80),
                                dict(batch=3, m=256, k=512, n=256)])
def test_c2_bf16_small(gpu_client, kw):
    _run_and_check(gpu_client, configs.c2_bf16_batched_dot(**kw))


def test_c2_bf16_full(gpu_client):
    _run_and_check(gpu_client, configs.c2_bf16_batched_dot())


@pytest.mark.parametrize("kw", [dict(m=128, k=256, n=128), dict(m=256, k=512, n=512), dict(m=96, k=64, n=48)])
def test_c3_int8_small(gpu_client, kw):
    _run_and_check(gpu_client, configs.c3_int8_gemm(**kw))


def test_c3_int8_full(gpu_client):
    _run_and_check(gpu_client, configs.c3_int8_gemm())


@pytest.mark.parametrize("kw", [dict(b=1, h=2, s=256, d=128), dict(b=2, h=1, s=128, d=64), dict(b=1, h=1, s=512, d=128),
                                # unmasked, key blocks of 64 in odd and even counts (the last step computes no next
                                # block's scores; the first is the last when there is one)
                                dict(b=1, h=2, s=128, d=128, mask=None, sk=192),
                                dict(b=1, h=1, s=256, d=64, mask=None, sk=320),
                                dict(b=1, h=2, s=128, d=128, mask=None, sk=64),
                                dict(b=2, h=1, s=256, d=128, mask=None),
                                # causal with an odd number of 256-query tiles (the middle one alone) and a last tile
                                # of 128 queries
                                dict(b=1, h=3, s=640, d=128), dict(b=1, h=2, s=384, d=64)])
def test_c4_attention_small(gpu_client, kw):
    w = configs.c4_causal_attention(**kw)
    outs, exe = _run_and_check(gpu_client, w)
    assert "attention_fwd" in exe.describe_plan()


@pytest.mark.parametrize("kw", [
    # batch·heads a multiple of 8: the workgroups of a head are grouped on one XCD (workgroup x → head slot x mod 8)
    dict(b=1, h=8, s=256, d=128),                 # causal, one query-block pair per head
    dict(b=4, h=2, s=384, d=128),                 # causal, 3 query blocks: a pair and a block alone
    dict(b=2, h=8, s=640, d=64),                  # causal, 5 query blocks, 16 heads over two slot rounds
    dict(b=1, h=8, s=256, d=128, mask=None),      # unmasked: one workgroup per query block
    dict(b=1, h=16, s=128, d=128, mask=None, sk=192)])
def test_c4_attention_heads_grouped_per_xcd(gpu_client, kw):
    w = configs.c4_causal_attention(**kw)
    outs, exe = run_pjrt(gpu_client, w.program, w.inputs)
    assert "attention_fwd" in exe.describe_plan()
    assert (kw["b"] * kw["h"]) % 8 == 0
    (want, dt), = oracle_outputs(w.program, w.inputs)
    got = sh.from_raw(outs[0], dt)
    for bi in range(kw["b"]):
        for hi in range(kw["h"]):
            err = sh.rel_error(got[bi, hi], want[bi, hi])
            assert err <= w.tolerance, f"head ({bi},{hi}): relative error {err:.3e}"
    print(f"[parity] {w.name} {kw}: every head within {w.tolerance}", flush=True)


def test_c4_attention_full_sampled(gpu_client):
    w = configs.c4_causal_attention()
    outs, exe = run_pjrt(gpu_client, w.program, w.inputs)
    assert "attention_fwd" in exe.describe_plan()
    got = sh.from_raw(outs[0], "bf16")
    assert np.all(np.isfinite(got))
    v = sh.from_raw(w.inputs[2].data, "bf16")
    assert np.array_equal(got[:, :, 0, :], nm.round_to(v[:, :, 0, :], "bf16"))  # row 0 attends to key 0 only
    small = configs.c4_causal_attention(b=1, h=1, s=2048, d=128)
    # one head per residue of b·H + h modulo 8 (the head slot its workgroups take on the XCDs), plus the first and
    # last heads
    heads = [(0, 0), (0, 9), (0, 18), (0, 27), (1, 4), (1, 13), (2, 22), (3, 31), (3, 23)]
    assert sorted({(b * 32 + h) % 8 for b, h in heads}) == list(range(8))
    for (bi, hi) in heads:
        sub = [configs.HostInput(x.data[bi:bi + 1, hi:hi + 1].copy(), x.type, (1, 1, 2048, 128)) for x in w.inputs]
        (want, dt), = oracle_outputs(small.program, sub)
        err = sh.rel_error(got[bi:bi + 1, hi:hi + 1], want)
        print(f"[parity] c4 head ({bi},{hi}) error {err:.3e}", flush=True)
        assert err <= w.tolerance


@pytest.mark.parametrize("kw", [dict(s=200), dict(s=96, d=64), dict(fill="-3.40282347E+38"), dict(p_type="f32")])
def test_c4_attention_graphs_the_kernel_declines(gpu_client, kw):
    """Attention graphs outside the fused kernel's preconditions run unfused and match the oracle."""
    base = dict(b=1, h=2, s=256, d=128)
    base.update(kw)
    outs, exe = _run_and_check(gpu_client, configs.c4_causal_attention(**base))
    assert "attention_fwd" not in exe.describe_plan()


def test_c4_strict_mask_first_row_is_nan(gpu_client):
    """A strict causal mask (key < query) leaves query 0 with no visible key: with the -inf fill its reduce-max is
    -inf, exp(-inf - -inf) is NaN, so StableHLO gives a NaN row; every other row matches the oracle."""
    w = configs.c4_causal_attention(b=1, h=2, s=256, d=128, mask="GT")
    outs, exe = run_pjrt(gpu_client, w.program, w.inputs)
    assert "attention_fwd" not in exe.describe_plan()
    (want, dt), = oracle_outputs(w.program, w.inputs)
    got = sh.from_raw(outs[0], dt)
    assert np.all(np.isnan(want[:, :, 0])) and np.all(np.isnan(got[:, :, 0]))
    assert np.all(np.isfinite(got[:, :, 1:]))
    err = sh.rel_error(got[:, :, 1:], want[:, :, 1:])
    print(f"[parity] c4 strict mask rows 1.. error {err:.3e}", flush=True)
    assert err <= w.tolerance


@pytest.mark.parametrize("kw,kernel", [(dict(m=256, d=512, f=1024), "gemm_bf16f8_mfma_dual_256x128"),
                                       (dict(m=128, d=256, f=512), "gemm_bf16f8_mfma_dual_128x128"),
                                       (dict(m=64, d=256, f=384), "gemm_bf16f8_mfma_dual_edge_128x128"),
                                       # f8 weight rows of 360 bytes: copied into 16-byte aligned rows first
                                       (dict(m=64, d=256, f=360), "gemm_bf16f8_mfma_dual_edge_128x128")])
def test_c5_swiglu_small(gpu_client, kw, kernel):
    outs, exe = _run_and_check(gpu_client, configs.c5_swiglu_fp8(**kw))
    assert kernel in exe.describe_plan() and "gemm_generic" not in exe.describe_plan()


def test_c5_swiglu_direct_f8_operands(gpu_client):
    # the dot_generals take the f8E4M3FN weights as operands (mixed operand types) instead of converted copies
    outs, exe = _run_and_check(gpu_client, configs.c5_swiglu_fp8(m=256, d=512, f=1024, weights="direct"))
    assert "gemm_bf16f8_mfma_dual_256x128" in exe.describe_plan()


def test_c5_swiglu_full(gpu_client):
    # C5 as BASELINE.json states it: bf16 activations × f8E4M3FN weights, on the bf16 MFMA (no generic kernel)
    w = configs.c5_swiglu_fp8()
    outs, exe = _run_and_check(gpu_client, w)
    plan = exe.describe_plan()
    assert "gemm_generic" not in plan and "gemm_bf16f8_mfma_dual" in plan, plan


def test_c5x_fp8_activations_full(gpu_client):
    # not a BASELINE config: activations quantized to f8E4M3FN too (fp8 × fp8 MFMA), checked against its own graph
    w = configs.c5x_swiglu_fp8_activations()
    outs, exe = _run_and_check(gpu_client, w)
    assert "gemm_fp8_mfma_dual" in exe.describe_plan()


def _widen_program(k_contiguous):
    if k_contiguous:  # rhs stored [n, k]
        return """module {
  func.func @main(%arg0: tensor<256x256xbf16>, %arg1: tensor<256x256xf8E4M3FN>) -> tensor<256x256xf32> {
    %0 = stablehlo.dot_general %arg0, %arg1, contracting_dims = [1] x [1] : (tensor<256x256xbf16>, tensor<256x256xf8E4M3FN>) -> tensor<256x256xf32>
    return %0 : tensor<256x256xf32>
  }
}"""
    return """module {
  func.func @main(%arg0: tensor<256x256xbf16>, %arg1: tensor<256x256xf8E4M3FN>) -> tensor<256x256xf32> {
    %0 = stablehlo.dot_general %arg0, %arg1, contracting_dims = [1] x [0] : (tensor<256x256xbf16>, tensor<256x256xf8E4M3FN>) -> tensor<256x256xf32>
    return %0 : tensor<256x256xf32>
  }
}"""


@pytest.mark.parametrize("k_contiguous", [False, True])
def test_bf16_f8_widening_every_code(gpu_client, k_contiguous):
    """The bf16 × f8E4M3FN GEMM widens every f8 code exactly: identity lhs, rhs holding all 254 finite codes in
    every row and column (subnormals and signed zeros included), f32 result equal to the decoded codes
    (StableHLO convert f8E4M3FN → bf16 is exact, casting.rs:75-122). A column holding a NaN code is NaN in every
    row (0 · NaN = NaN), the other columns unchanged."""
    eye = nm.encode_bits(np.eye(256), "bf16")
    idx = (np.arange(256)[:, None] + np.arange(256)[None, :]) % 256
    codes = idx.astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x00  # finite codes only
    nan_codes = codes.copy()
    nan_codes[17, 3] = 0x7F
    nan_codes[200, 250] = 0xFF
    exe = gpu_client.compile(pjrt.Program.mlir(_widen_program(k_contiguous)))
    assert "gemm_bf16f8_mfma" in exe.describe_plan(), exe.describe_plan()
    decoded = nm.decode_bits(codes, "f8E4M3FN").astype(np.float32)
    for rhs, nan_cols in ((codes, []), (nan_codes, [3, 250])):
        stored = np.ascontiguousarray(rhs.T) if k_contiguous else rhs  # k-contiguous: the [n, k] layout
        ins = [configs.HostInput(eye, pjrt.BufferType.BF16, (256, 256)),
               configs.HostInput(stored, pjrt.BufferType.F8E4M3FN, (256, 256))]
        outs, _ = run_pjrt(gpu_client, "", ins, executable=exe)
        got = outs[0].view(np.float32).reshape(256, 256)
        want = decoded  # C = I · B = B in both layouts
        ok = np.ones(256, bool)
        ok[nan_cols] = False
        # values, not bits: the diagonal's -0 product summed with +0 products is +0
        assert np.array_equal(got[:, ok], want[:, ok])
        for c in nan_cols:
            assert np.all(np.isnan(got[:, c]))


def test_repeated_execution_is_deterministic(gpu_client):
    w = configs.c2_bf16_batched_dot(batch=2, m=256, k=256, n=256)
    exe = gpu_client.compile(pjrt.Program.mlir(w.program))
    bufs = [gpu_client.buffer(x.data, x.type, x.dims) for x in w.inputs]
    first = None
    for _ in range(5):
        out = exe.execute([bufs])[0]
        out.done.await_()
        r = out.outputs[0].copy_to_host().await_()
        first = first or r
        assert r == first
