"""GPU parity of the row-fused kernel (reductions over the innermost dim consumed by an elementwise expression in the
same launch) against the oracle: RMSNorm, LayerNorm, softmax and an integer row maximum.

Row lengths cover each launch shape: multiples of 8 with ≥ 2048 elements (a workgroup per row, 8 elements per thread),
shorter multiples of 8 (a wavefront per row), and ragged lengths (one element per thread; a workgroup per row from 1024
elements on). Tolerances: f32 results 1e-5 normwise relative (the kernel sums in f32 in its own order, the oracle in
f64; BASELINE allows 1e-4 for f32), bf16 results 1e-2, integers bit-exact."""
import numpy as np
import pytest

from ryft_amd import configs, hostdata as hd, pjrt
from tests import row_programs
from oracle import stablehlo as sh
from tests.helpers import check, oracle_outputs, run_pjrt

pytestmark = pytest.mark.gpu


def _f32(seed, shape, mean=0.0, std=1.0):
    return configs.HostInput(hd.normal(seed, shape, mean, std), pjrt.BufferType.F32, shape)


def _bf16(seed, shape, mean=0.0, std=1.0):
    return configs.HostInput(hd.f32_to_bf16_bits(hd.normal(seed, shape, mean, std)), pjrt.BufferType.BF16, shape)


@pytest.fixture(scope="module")
def interp_client(plugin):
    """A client whose plans keep every row-fused step on the interpreted row kernel (no specialised kernels)."""
    return plugin.client({"fast_paths": False, "visible_devices": [0]})


def _run(client, prog, ins, tol, name):
    outs, exe = run_pjrt(client, prog, ins)
    plan = exe.describe_plan()
    assert "row_fused" in plan or "row_norm" in plan, plan
    for o, w in zip(outs, oracle_outputs(prog, ins)):
        check(o, w, tol, name)
    return outs


@pytest.mark.parametrize("shape,dt", [((16, 4096), "f32"), ((8, 256), "bf16"), ((8, 33), "f32"), ((4, 1100), "f32"),
                                      ((2, 3, 4096), "bf16")])
def test_rmsnorm(gpu_client, shape, dt):
    d = shape[-1]
    mk = _f32 if dt == "f32" else _bf16
    ins = [mk(11, shape), mk(12, (d,), 1.0, 0.02)]
    _run(gpu_client, row_programs.rmsnorm(shape, dt), ins, 1e-5 if dt == "f32" else 1e-2, f"rmsnorm{shape}")


@pytest.mark.parametrize("shape,dt,quant", [((512, 4096), "bf16", "f8E4M3FN"), ((16, 4096), "f32", None),
                                            ((8, 256), "bf16", None), ((2, 3, 4096), "bf16", "f8E4M3FN"),
                                            ((4, 8192), "f32", None), ((3, 16400), "bf16", None),
                                            ((2048, 4096), "bf16", "f8E4M3FN"), ((2048, 4096), "f32", None),
                                            ((2048, 8192), "f32", None), ((2049, 1016), "f32", None),
                                            ((6000, 2048), "bf16", None), ((16384, 4096), "bf16", "f8E4M3FN"),
                                            ((8192, 520), "bf16", "f8E4M3FN")])
def test_rmsnorm_fast_path_matches_interpreter(gpu_client, interp_client, shape, dt, quant):
    # the row-norm kernels and the interpreted row kernel fold in the same order: identical bits, and both match the
    # oracle. C5's normalise-and-quantise step at its full size is the first case. With few rows a workgroup takes a
    # row: rows of ≤ 2048, ≤ 4096, ≤ 8192 and longer elements cover the one-, two-, four-chunk register-resident and
    # the re-reading variants. Short rows, and rows of ≤ 8192 elements when there are ≥ 2048 of them, take a
    # wavefront each (8 and 16 chunks per lane, 16- and 32-bit inputs, a ragged last chunk column); with 16-bit
    # inputs and more rows than the chip holds wavefronts, a wavefront takes several rows (the last three cases: a
    # ragged number of rows per wavefront, the calibration workload's shape, a ragged last chunk column).
    d = shape[-1]
    mk = _f32 if dt == "f32" else _bf16
    ins = [mk(51, shape), mk(52, (d,), 1.0, 0.02)]
    prog = row_programs.rmsnorm(shape, dt, quant=quant)
    fast, exe = run_pjrt(gpu_client, prog, ins)
    assert exe.describe_plan().split()[1] == "row_norm"
    slow, exe2 = run_pjrt(interp_client, prog, ins)
    assert exe2.describe_plan().split()[1] == "row_fused"
    assert np.array_equal(fast[0], slow[0]), f"{np.count_nonzero(fast[0] != slow[0])} differing elements"
    want = oracle_outputs(prog, ins)[0]
    # f8 outputs: one quantisation step (2^-3 relative) where the f32 sums round differently, so a looser bound
    check(fast[0], want, 1e-5 if dt == "f32" else (3e-2 if quant else 1e-2), f"rmsnorm{shape}")


@pytest.mark.parametrize("weights", ["finite", "special"])
def test_rmsnorm_f8_rows_with_special_values(gpu_client, interp_client, weights):
    # many bf16 rows (a wavefront takes several): rows holding +NaN, -NaN, ±inf, an all-zero row (s = rsqrt(eps)),
    # a row whose x·s overflows f32, and ordinary rows; the f8E4M3FN conversion must keep each NaN's sign wherever a
    # NaN arises. With "special" weights (a +NaN, a -NaN and an inf column) every row takes the NaN sign repair.
    m, d = 4096, 4096
    rng = np.random.default_rng(61)
    x = hd.f32_to_bf16_bits(rng.standard_normal((m, d)).astype(np.float32))
    w = hd.f32_to_bf16_bits(rng.normal(1.0, 0.02, d).astype(np.float32))
    x[7, 5], x[9, 100], x[11, 3], x[13, 4000] = 0x7FC0, 0xFFC0, 0x7F80, 0xFF80
    x[15] = 0
    x[17, :] = 0
    x[17, 0] = 0x7F7F  # the largest finite bf16: its square overflows f32, so s = 0
    x[19, :] = 0x0001  # the smallest bf16 subnormal in every column: Σx² is tiny, s = rsqrt(eps)
    if weights == "special":
        w[1], w[2], w[3] = 0x7FC0, 0xFFC0, 0x7F80
    ins = [configs.HostInput(x, pjrt.BufferType.BF16, (m, d)), configs.HostInput(w, pjrt.BufferType.BF16, (d,))]
    prog = row_programs.rmsnorm((m, d), "bf16", quant="f8E4M3FN")
    fast, exe = run_pjrt(gpu_client, prog, ins)
    assert exe.describe_plan().split()[1] == "row_norm"
    slow, _ = run_pjrt(interp_client, prog, ins)
    assert np.array_equal(fast[0], slow[0]), f"{np.count_nonzero(fast[0] != slow[0])} differing elements"
    # NaN bytes (0x7f / 0xff) where the oracle has NaNs; the sign each NaN keeps is the interpreter's (above)
    vals, dt = oracle_outputs(prog, ins)[0]
    assert np.array_equal((fast[0] & 0x7F) == 0x7F, np.isnan(vals))
    if weights == "finite":
        # elementwise: at most one f8E4M3FN step apart (where the f32 sums round differently from the oracle's),
        # and rarely so
        rows = [r for r in range(m) if r not in (7, 9, 11, 13)]
        got, want = sh.from_raw(fast[0][rows], dt), vals[rows]
        with np.errstate(divide="ignore"):
            step = np.maximum(2.0 ** (np.floor(np.log2(np.abs(want))) - 3), 2.0 ** -9)
        assert np.all(np.abs(got - want) <= step)
        assert np.count_nonzero(got != want) < 1e-3 * got.size


@pytest.mark.parametrize("shape", [(4, 8, 200), (6, 2048), (5, 37)])
def test_softmax_rows(gpu_client, shape):
    ins = [_f32(21, shape, 0.0, 4.0)]
    _run(gpu_client, row_programs.softmax(shape), ins, 1e-5, f"softmax{shape}")


@pytest.mark.parametrize("shape", [(8, 33), (32, 4096), (3, 5, 128)])
def test_layernorm(gpu_client, shape):
    d = shape[-1]
    ins = [_f32(31, shape, 3.0, 2.0), _f32(32, (d,), 1.0, 0.1), _f32(33, (d,), 0.0, 0.1)]
    _run(gpu_client, row_programs.layernorm(shape), ins, 1e-5, f"layernorm{shape}")


@pytest.mark.parametrize("shape", [(8, 64), (3, 2050)])
def test_int_row_max(gpu_client, shape):
    x = hd.int_uniform(41, shape, -2 ** 30, 2 ** 30).astype(np.int32)
    ins = [configs.HostInput(x, pjrt.BufferType.S32, shape)]
    _run(gpu_client, row_programs.int_row_max_gap(shape), ins, 0, f"int_row_max{shape}")

