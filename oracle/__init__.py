"""CPU oracle for the MI355X PJRT plugin — TEST INFRASTRUCTURE ONLY.

A restatement, in numpy, of the StableHLO semantics that the reference's hot path delegates to XLA's CPU PJRT
plugin (crates/ryft-xla-sys/BUILD.bazel:108-110; XLA is not vendored in the reference, commit pinned at
crates/ryft-xla-sys/WORKSPACE:9-11). Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may use it, and only as the checker / the timed CPU baseline — never as a product code path.

Modules:
  numerics   — narrow float types (bf16, f16, f8E4M3FN, f8E5M2) by nearest-representable search over the
               format's value table (ties to the even code), independent of the product's bit manipulations.
  stablehlo  — a small StableHLO text parser and a numpy interpreter for the op set the plugin supports.

Parity pinning (what each function is checked against) is listed in tests/test_oracle.py; the reference's worked
op examples it is checked against are in tests/ref_examples.py.

Parity unpinned (no reference test, fixture or documented example fixes them; the oracle follows XLA's conventions,
which the plugin implements too): integer division by zero (quotient -1, all bits set for unsigned; remainder = the
dividend); float → integer conversion of NaN (0) and of values outside the target range (saturated to its bounds),
which the StableHLO specification leaves implementation-defined; the exact bits of transcendental functions (exp,
log, tanh, logistic, power, sine, cosine, tan, atan2, cbrt), which parity tests cover with tolerances (their
values are pinned to the math module and to identities in tests/test_bit_trig_round_ops.py). The XLA CPU plugin itself
is unavailable offline (no Bazel, no network), so semantics rest on the ryft-mlir op documentation cited per
function, the reference's known-answer tests (README.md:122-137, programs.rs:2781-2829), closed forms, brute force
on small cases, and torch's CPU dtype conversions for the narrow float types.
"""
