"""The CPU executor behind bench.py's cpu_baseline (oracle/cpu_exec.cc) against the numpy oracle on the same seeded
inputs, at sizes that take every blocking edge (M, N, K not multiples of its register tiles or cache blocks): it must
compute the graphs it is timed on. Tolerances are the configs' own (int8 accumulator bit-exact)."""
import numpy as np
import pytest

from oracle import cpu_exec
from ryft_amd import configs
from tests.helpers import check, oracle_outputs


@pytest.mark.parametrize("name,kw", [
    ("c1", dict(m=100, k=300, n=70)),
    ("c1", dict(m=256, k=512, n=256)),
    ("c2", dict(batch=2, m=130, k=260, n=100)),
    ("c3", dict(m=97, k=515, n=301)),
    ("c4", dict(b=1, h=2, s=200, d=64)),
    ("c4", dict(b=2, h=1, s=96, d=128)),
    ("c5", dict(m=37, d=96, f=200)),
    ("c5", dict(m=64, d=256, f=512)),
    ("copy", dict(n=1000003)),
    ("rmsnorm", dict(m=33, d=4096)),
])
def test_cpu_executor_matches_the_oracle(name, kw):
    w = configs.CONFIGS[name](**kw)
    got = cpu_exec.run(name, w)
    want = oracle_outputs(w.program, w.inputs)
    assert len(got) == len(want)
    for i, (g, r) in enumerate(zip(got, want)):
        check(g, r, w.tolerance, f"{name}{kw}[{i}]")


def test_cpu_executor_threads():
    assert cpu_exec.threads() >= 1
