"""The README path on the GPU: each config (at test sizes) handed to the plugin as MLIR bytecode executes to the same
bits as its text form, and matches the oracle within the config's tolerance."""
import numpy as np
import pytest

from ryft_amd import configs, pjrt
from tests import mlir_bytecode as mb
from tests.helpers import check, oracle_outputs, run_pjrt

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,kw", [
    ("c1", {}),
    ("c2", {"batch": 2, "m": 256, "k": 256, "n": 256}),
    ("c3", {"m": 256, "k": 256, "n": 256}),
    ("c4", {"b": 1, "h": 2, "s": 256, "d": 128}),
    ("c5", {"m": 64, "d": 256, "f": 512}),
])
def test_bytecode_executes_like_text(gpu_client, name, kw):
    w = configs.CONFIGS[name](**kw)
    text_outs, _ = run_pjrt(gpu_client, w.program, w.inputs)
    exe = gpu_client.compile(pjrt.Program.mlir(mb.to_bytecode(w.program)))
    bc_outs, _ = run_pjrt(gpu_client, w.program, w.inputs, executable=exe)
    assert len(bc_outs) == len(text_outs)
    for a, b in zip(bc_outs, text_outs):
        assert np.array_equal(a, b)
    for got, want in zip(bc_outs, oracle_outputs(w.program, w.inputs)):
        check(got, want, w.tolerance, name)  # integer outputs (C3's i32 accumulator) are compared bit-exactly
