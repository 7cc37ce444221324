"""Split-K GEMMs on the GPU (few output tiles over a long K: per-range partial sums in a workspace, which the range
that finishes each tile last sums in range order and takes through the epilogue, inside the GEMM launch) against
the oracle: int8 → i32 stays bit-exact (integer sums do not depend on their order), bf16 / fp8 / f32 within the
configs' tolerances, repeated executions reuse the workspace and the arrival counters, and executions with other
inputs in between never see a previous execution's partial sums."""
import numpy as np
import pytest

from ryft_amd import configs
from tests.helpers import check, oracle_outputs, run_pjrt

pytestmark = pytest.mark.gpu


def _run(client, w, kernel_prefix):
    print(f"[splitk] {w.name}", flush=True)
    outs, exe = run_pjrt(client, w.program, w.inputs)
    plan = exe.describe_plan()
    assert kernel_prefix in plan and "_splitk" in plan, plan
    for i, (o, r) in enumerate(zip(outs, oracle_outputs(w.program, w.inputs))):
        check(o, r, w.tolerance, f"{w.name}[{i}]")
    return outs, exe


def test_int8_split_k_is_bit_exact(gpu_client):
    w = configs.c3_int8_gemm(m=256, k=8192, n=256)
    outs, exe = _run(gpu_client, w, "gemm_i8_mfma_128x128")
    # a second execution (same workspace, now holding the first one's partials) gives the same bits
    again, _ = run_pjrt(gpu_client, w.program, w.inputs, executable=exe)
    for a, b in zip(outs, again):
        assert np.array_equal(a, b)


def test_bf16_split_k(gpu_client):
    _run(gpu_client, configs.c2_bf16_batched_dot(batch=1, m=256, k=4096, n=256), "gemm_bf16_mfma_128x128")


def test_fp8_split_k_scaled_epilogue(gpu_client):
    # C5 with fp8 activations at 128 tokens: the down projection (M=128, N=1024, K=2048) runs split-K with the
    # per-column scale epilogue
    _run(gpu_client, configs.c5x_swiglu_fp8_activations(m=128, d=1024, f=2048), "gemm_fp8_mfma_128x128")


def test_bf16_f8_split_k_scaled_epilogue(gpu_client):
    # C5 as stated (bf16 activations, f8 weights) at 128 tokens: the same split on the widening bf16 kernel
    _run(gpu_client, configs.c5_swiglu_fp8(m=128, d=1024, f=2048), "gemm_bf16f8_mfma_128x256")


def test_f32_split_k(gpu_client):
    _run(gpu_client, configs.c1_f32_dot(), "gemm_f32_mfma_64x64")


@pytest.mark.parametrize("make,kernel", [
    (lambda seed: configs.c1_f32_dot(seed=seed), "gemm_f32_mfma_64x64"),
    (lambda seed: configs.c5_swiglu_fp8(m=128, d=1024, f=2048, seed=seed), "gemm_bf16f8_mfma_128x256"),
    (lambda seed: configs.c3_int8_gemm(m=256, k=8192, n=256, seed=seed), "gemm_i8_mfma_128x128")])
def test_split_k_alternating_inputs(gpu_client, make, kernel):
    # one executable, inputs A, B, A, B, A back to back without waiting in between: every result matches the oracle
    # for its own inputs (a stale partial sum of the other execution, read by the finishing range, would not)
    from ryft_amd import pjrt
    wa, wb = make(0x51), make(0x52)
    exe = gpu_client.compile(pjrt.Program.mlir(wa.program))
    plan = exe.describe_plan()
    assert kernel in plan and "_splitk" in plan, plan
    dev = exe.addressable_devices()[0]
    bufs = {w.name + str(i): [gpu_client.buffer(x.data, x.type, x.dims, device=dev) for x in w.inputs]
            for i, w in enumerate((wa, wb))}
    runs = [exe.execute([bufs[(wa if k % 2 == 0 else wb).name + str(k % 2)]])[0] for k in range(5)]
    want = [oracle_outputs(w.program, w.inputs) for w in (wa, wb)]
    for k, r in enumerate(runs):
        r.done.await_()
        for i, (o, ref) in enumerate(zip(r.outputs, want[k % 2])):
            check(o.to_numpy(), ref, wa.tolerance, f"execution {k} output {i}")
    print(f"[splitk] alternating inputs {wa.name}: 5 executions match", flush=True)
