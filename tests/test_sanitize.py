"""The plugin's host path under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU: the MLIR text and
bytecode front-ends, the planner and the CompileOptionsProto decoder (the bytes ryft-pjrt hands to
PJRT_Client_Compile, crates/ryft-pjrt/src/programs.rs:1245-1263) built with -fsanitize=address,undefined
(tests/sanitize/Makefile) and fed the test corpus — every config, edge, row, donation, manipulation, reduce-body and
elementwise-op program as text and as bytecode in each writer variant, and CompileOptions encodings — plus truncated
and bit-flipped copies of every file (tests/sanitize/frontend_check.cc). Rejections are expected; a sanitizer report fails the test. The whole
host side of the plugin (runtime, C API, profiler included) is also built with -fsanitize=thread and driven from several
threads at once (tests/sanitize/tsan_check.cc)."""
import os
import subprocess

import pytest

from ryft_amd import configs, pjrt
from tests import donation_programs, edge_programs, mlir_bytecode as mb, row_programs
from tests import test_bit_trig_round_ops as bt, test_dynamic_window as dw, test_reduce_bodies as rb
from tests.test_bytecode import SLICE_CONCAT_PAD, VARIANTS

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sanitize")


def _programs():
    progs = {
        "c1": configs.c1_f32_dot(m=64, k=32, n=64).program,
        "c2": configs.c2_bf16_batched_dot(batch=2, m=128, k=64, n=128).program,
        "c3": configs.c3_int8_gemm(m=128, k=128, n=128).program,
        "c4": configs.c4_causal_attention(b=1, h=2, s=128, d=64).program,
        "c4_strict_mask": configs.c4_causal_attention(b=1, h=1, s=128, d=64, mask="GT").program,
        "c4_unmasked": configs.c4_causal_attention(b=1, h=1, s=128, d=64, mask=None, sk=192).program,
        "c4_f32_p": configs.c4_causal_attention(b=1, h=1, s=128, d=64, p_type="f32").program,
        "c5": configs.c5_swiglu_fp8(m=64, d=128, f=256).program,
        "c5_ragged": configs.c5_swiglu_fp8(m=64, d=128, f=100).program,
        "rmsnorm": row_programs.rmsnorm((16, 256), "bf16"),
        "softmax": row_programs.softmax((4, 8, 200)),
        "layernorm": row_programs.layernorm((8, 33)),
        "int_row_max": row_programs.int_row_max_gap((8, 64)),
        "slice_concatenate_pad": SLICE_CONCAT_PAD,
        "dynamic_slice": dw.ds_program((5, 7, 9), (2, 3, 4), dt="bf16", it="i32"),
        "dynamic_update_slice": dw.dus_program((2, 8, 256, 64), (2, 8, 1, 64), dt="bf16", it="i32", donate=True),
        "gather": dw.gather_example_program(),
        "gather_printed": dw.GATHER_PRINTED,
        "argmax": rb.argmax_program((8, 100), 1),
        "argmin_generic": rb.argmax_program((6, 7, 9), 0, kind="argmin", form="generic"),
        "sum_max": rb.sum_max_program((6, 50, 40), [0, 2]),
        "xor_reduce": rb.one_input_program((4, 33), 1, "xor", "i32"),
        "shift_left": bt._prog("shift_left", ["i8", "i8"], "i8", (4, 33)),
        "is_finite": bt._prog("is_finite", ["bf16"], "i1", (4, 33)),
        "atan2": bt._prog("atan2", ["f32", "f32"], "f32", (4, 33), generic=True),
    }
    for (name, prog, _), _, _ in edge_programs.CASES:
        progs["edge_" + name] = prog
    for name in ("SGD", "GEMM", "TRANSPOSED"):
        if hasattr(donation_programs, name):
            progs["donation_" + name.lower()] = getattr(donation_programs, name)
    return progs


def _options():
    C = pjrt.CompilationOptions
    return {"default": C(), "device0": C(device_ordinal=0), "replicas2": C(replica_count=2),
            "partitions3": C(partition_count=3), "precision": C(matrix_unit_operand_precision=1)}


def test_host_path_under_sanitizers(tmp_path):
    build = subprocess.run(["make", "-C", HERE, "-j8"], capture_output=True, text=True, timeout=1200)
    assert build.returncode == 0, build.stdout[-3000:] + build.stderr[-3000:]
    files = []
    for name, text in _programs().items():
        p = tmp_path / f"{name}.mlir"
        p.write_text(text)
        files.append(str(p))
        for vname, opts in VARIANTS.items():
            try:
                code = mb.to_bytecode(text, **opts)
            except Exception:  # a writer variant that does not cover this program
                continue
            q = tmp_path / f"{name}.{vname}.mlirbc"
            q.write_bytes(code)
            files.append(str(q))
    for name, o in _options().items():
        q = tmp_path / f"options_{name}.pb"
        q.write_bytes(o.encode())
        files.append(str(q))
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:halt_on_error=1",
               LSAN_OPTIONS=f"suppressions={os.path.join(HERE, 'lsan.supp')}",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    run = subprocess.run([os.path.join(HERE, "_build", "frontend_check")] + files, capture_output=True, text=True,
                         timeout=1500, env=env)
    print(run.stdout[-2000:], run.stderr[-2000:])
    assert run.returncode == 0, run.stdout[-3000:] + run.stderr[-6000:]
    assert "frontend_check:" in run.stdout and "AddressSanitizer" not in run.stderr and "runtime error" not in run.stderr


def test_c_api_from_several_threads_under_tsan(tmp_path):
    """tests/sanitize/tsan_check.cc under ThreadSanitizer: compiles on four threads of one compile-only client beside
    profiler sessions, and user events whose OnReady callbacks are registered from three threads while another
    thread sets them and two more await them (each callback exactly once, with its event's outcome)."""
    build = subprocess.run(["make", "-C", HERE, "-j8", "_build/tsan_check"], capture_output=True, text=True,
                           timeout=1200)
    assert build.returncode == 0, build.stdout[-3000:] + build.stderr[-3000:]
    files = []
    for name, text in _programs().items():
        p = tmp_path / f"{name}.mlir"
        p.write_text(text)
        files.append(str(p))
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1:second_deadlock_stack=1")
    run = subprocess.run([os.path.join(HERE, "_build", "tsan_check")] + files, capture_output=True, text=True,
                         timeout=900, env=env)
    print(run.stdout[-2000:], run.stderr[-2000:])
    assert run.returncode == 0, run.stdout[-3000:] + run.stderr[-6000:]
    assert "tsan_check:" in run.stdout and "ThreadSanitizer" not in run.stderr
