"""GPU parity of the edge instantiations of the MFMA GEMMs (tests/edge_programs.py): shapes that are not tile
multiples (partial tiles, a K that ends inside a k-tile), m-contiguous and k-contiguous operand layouts, every MFMA
element type. Integer results bit-exact; floats within the stated normwise bound of the oracle."""
import numpy as np
import pytest

from tests.edge_programs import CASES
from tests.helpers import check, oracle_outputs, run_pjrt

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("case", CASES, ids=[c[0][0] for c in CASES])
def test_edge_tiles(gpu_client, case):
    (name, prog, ins), kernel, tol = case
    print(f"[edge] {name}", flush=True)
    outs, exe = run_pjrt(gpu_client, prog, ins)
    assert kernel in exe.describe_plan(), exe.describe_plan()
    err = check(outs[0], oracle_outputs(prog, ins)[0], tol, name)
    print(f"[edge] {name} error {err:.3e}", flush=True)


def test_c3_scale_epilogue_on_partial_tiles(gpu_client):
    # the two-output scale epilogue (raw i32 and scaled f32) with per-row / per-column scales on partial tiles
    from ryft_amd import configs
    w = configs.c3_int8_gemm(m=300, k=528, n=272)
    outs, exe = run_pjrt(gpu_client, w.program, w.inputs)
    assert "gemm_i8_mfma_edge_128x128" in exe.describe_plan(), exe.describe_plan()
    for i, (o, r) in enumerate(zip(outs, oracle_outputs(w.program, w.inputs))):
        check(o, r, w.tolerance, f"c3 edge [{i}]")


@pytest.mark.parametrize("kw", [dict(m=64, d=128, f=100), dict(m=100, d=200, f=136)])
def test_c5_ragged_unaligned_weights(gpu_client, kw):
    # f8 weight rows of 100 / 136 / 200 bytes (not 16-byte aligned): padded copies feed the dual SwiGLU GEMM and the
    # down projection on the MFMA edge kernels, whose epilogues store the partial output chunks element by element
    from ryft_amd import configs
    w = configs.c5_swiglu_fp8(**kw)
    print(f"[edge] c5 {kw}", flush=True)
    outs, exe = run_pjrt(gpu_client, w.program, w.inputs)
    plan = exe.describe_plan()
    assert "gemm_bf16f8_mfma_dual_edge_128x128" in plan and "gemm_generic" not in plan, plan
    err = check(outs[0], oracle_outputs(w.program, w.inputs)[0], w.tolerance, f"c5 {kw}")
    print(f"[edge] c5 {kw} error {err:.3e}", flush=True)


def test_c5_on_partial_tiles(gpu_client):
    # C5's graph at sizes that are not tile multiples: dual SwiGLU GEMM and down projection on the edge kernels
    from ryft_amd import configs
    w = configs.c5_swiglu_fp8(m=100, d=272, f=400)
    outs, exe = run_pjrt(gpu_client, w.program, w.inputs)
    plan = exe.describe_plan()
    assert "gemm_bf16f8_mfma_dual_edge_128x128" in plan and "gemm_generic" not in plan, plan
    check(outs[0], oracle_outputs(w.program, w.inputs)[0], w.tolerance, "c5 edge")
