"""MLIR bytecode front-end (the README path: `Program::Mlir { bytecode: module.bytecode() }`, README.md:88,
crates/ryft-mlir/src/operations/operation.rs:805-819) on the CPU: every config and row program written as bytecode
by tests/mlir_bytecode.py, in each variant a producer may emit, compiles to the same plan as its text; encoding
known-answers; malformed input is rejected with the PJRT error codes ryft-pjrt surfaces.

Parity unpinned against bytes written by MLIR itself (no MLIR build exists here, and ryft-mlir cannot be built):
the writer and the reader share this repository's reading of MLIR's bytecode format."""
import functools

import pytest

from ryft_amd import configs, pjrt
from tests import mlir_bytecode as mb, row_programs

VARIANTS = {
    "v6-properties-sorted": {},
    "v6-properties-declared": {"order": "declared"},
    "v6-attribute-dicts": {"properties": False},
    "v4-attribute-dicts": {"properties": False, "version": 4},
    "v6-stablehlo-attrs-as-text": {"stablehlo_attrs": "text"},
    "v6-isolated-reduce-body": {"isolated_reduce": True},
}


@functools.lru_cache(maxsize=None)
def _config_program(name):
    return configs.CONFIGS[name]().program  # (generates the inputs too: once per config)


SLICE_CONCAT_PAD = """module {
  func.func @main(%arg0: tensor<6x8xf32>, %arg1: tensor<f32>) -> (tensor<6x12xf32>, tensor<9x8xf32>) {
    %0 = stablehlo.slice %arg0 [0:6, 1:8:2] : (tensor<6x8xf32>) -> tensor<6x4xf32>
    %1 = stablehlo.concatenate %arg0, %0, dim = 1 : (tensor<6x8xf32>, tensor<6x4xf32>) -> tensor<6x12xf32>
    %2 = stablehlo.pad %arg0, %arg1, low = [2, -1], high = [-1, 0], interior = [1, 0] : (tensor<6x8xf32>, tensor<f32>) -> tensor<12x7xf32>
    %3 = stablehlo.slice %2 [3:12, 0:7] : (tensor<12x7xf32>) -> tensor<9x7xf32>
    %4 = stablehlo.concatenate %3, %3, dim = 1 : (tensor<9x7xf32>, tensor<9x7xf32>) -> tensor<9x14xf32>
    %5 = stablehlo.slice %4 [0:9, 3:11] : (tensor<9x14xf32>) -> tensor<9x8xf32>
    return %1, %5 : tensor<6x12xf32>, tensor<9x8xf32>
  }
}
"""

PROGRAMS = {
    "c1": lambda: _config_program("c1"),
    "c2": lambda: _config_program("c2"),
    "c3": lambda: _config_program("c3"),
    "c4": lambda: _config_program("c4"),
    "c5": lambda: _config_program("c5"),
    "layernorm": lambda: row_programs.layernorm((8, 33)),
    "int_row_max": lambda: row_programs.int_row_max_gap((8, 64)),
    "slice_concatenate_pad": lambda: SLICE_CONCAT_PAD,
    # two dot_generals whose dimension numbers differ and whose contracted sizes differ (128 queries, 192 keys): a
    # property blob read in the wrong field order would hand one dot the other's numbers
    "attention_cross_lengths": lambda: configs.c4_causal_attention(b=1, h=1, s=128, d=64, mask=None, sk=192).program,
}


def test_varint_known_answers():
    # prefix varints: the trailing zero bits of the first byte (+1) give the byte count; 0x00 → 8 more bytes
    assert mb.varint(0) == b"\x01"
    assert mb.varint(1) == b"\x03"
    assert mb.varint(127) == b"\xff"
    assert mb.varint(128) == b"\x02\x02"
    assert mb.varint(2 ** 14 - 1) == b"\xfe\xff"
    assert mb.varint(2 ** 14) == b"\x04\x00\x02"
    assert mb.varint(2 ** 56) == b"\x00" + (2 ** 56).to_bytes(8, "little")
    assert mb.svarint(-1) == b"\x03" and mb.svarint(1) == b"\x05" and mb.svarint(-2) == b"\x07"


@pytest.mark.parametrize("variant", list(VARIANTS))
@pytest.mark.parametrize("name", list(PROGRAMS))
def test_bytecode_compiles_to_the_text_plan(compile_client, name, variant):
    text = PROGRAMS[name]()
    code = mb.to_bytecode(text, **VARIANTS[variant])
    assert code[:4] == b"ML\xefR"
    want = compile_client.compile(pjrt.Program.mlir(text))
    got = compile_client.compile(pjrt.Program.mlir(code))
    assert got.describe_plan() == want.describe_plan()
    e1, e2 = want.executable(), got.executable()
    assert e2.output_count() == e1.output_count()
    assert e2.output_element_types() == e1.output_element_types()
    assert e2.output_dimensions() == e1.output_dimensions()


def _error(client, code):
    with pytest.raises(pjrt.PjrtError) as e:
        client.compile(pjrt.Program.mlir(code))
    return e.value


def test_truncated_bytecode_is_invalid_argument(compile_client):
    code = mb.to_bytecode(PROGRAMS["c2"]())
    for cut in (6, len(code) // 2, len(code) - 1):
        err = _error(compile_client, code[:cut])
        assert err.code == pjrt.ErrorCode.INVALID_ARGUMENT, (cut, err.message)


def test_newer_bytecode_version_is_unimplemented(compile_client):
    code = mb.to_bytecode(PROGRAMS["c1"]())
    err = _error(compile_client, code[:4] + mb.varint(7) + code[5:])
    assert err.code == pjrt.ErrorCode.UNIMPLEMENTED and "version 7" in err.message


def test_unsupported_op_in_bytecode_is_unimplemented(compile_client):
    T = "tensor<8xf32>"
    text = f"""module {{
  func.func @main(%arg0: {T}) -> {T} {{
    %0 = stablehlo.real %arg0 : {T}
    return %0 : {T}
  }}
}}
"""
    err = _error(compile_client, mb.to_bytecode(text))
    assert err.code == pjrt.ErrorCode.UNIMPLEMENTED and "stablehlo.real" in err.message


def test_missing_entry_function_is_invalid_argument(compile_client):
    code = mb.to_bytecode(PROGRAMS["c1"]())
    i = code.index(b"main\x00")
    err = _error(compile_client, code[:i] + b"mian" + code[i + 4:])
    assert err.code == pjrt.ErrorCode.INVALID_ARGUMENT and "@main" in err.message
