"""bench.py's command-line contract that holds without a GPU: more than one GPU is refused with a message before
anything touches a device, and the workload list names the BASELINE configs."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)


def test_more_than_one_gpu_exits_with_a_message():
    r = _bench("--gpus", "2")
    assert r.returncode == 2
    assert "--gpus 2 is not supported" in r.stderr and r.stdout == ""


def test_help_lists_the_configs():
    r = _bench("--help")
    assert r.returncode == 0
    for c in ("c1", "c2", "c3", "c4", "c5", "copy", "rmsnorm", "argmax"):
        assert c in r.stdout
    assert "--steps" in r.stdout and "--warmup" in r.stdout
