"""CPU-side checks of the plugin: the C-ABI library, the PJRT table, the StableHLO front-end and the planner.

Runs without a GPU through a compile-only client (programs are parsed and planned; nothing executes).
"""
import ctypes
import os
import re
import subprocess

import pytest

from tests import row_programs
from ryft_amd import configs, pjrt, profiler

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_only_its_entry_points():
    # GetPjrtApi (what load_plugin resolves) and the allocation-free execute entry point; nothing else
    out = subprocess.run(["nm", "-D", "--defined-only", pjrt.DEFAULT_PLUGIN_PATH], capture_output=True, text=True,
                         check=True).stdout
    syms = sorted({ln.split()[-1].split("@")[0] for ln in out.splitlines() if ln.strip()})
    assert syms == ["GetPjrtApi", "RyftMi355x_ExecuteNoAlloc"]


def test_header_declares_what_the_library_exports():
    header = open(os.path.join(ROOT, "include", "ryft_mi355x.h")).read()
    decls = re.findall(r"^(?:const\s+)?\w+\*?\s+(\w+)\(", header, re.M)
    lib = ctypes.CDLL(pjrt.DEFAULT_PLUGIN_PATH)
    assert decls == ["GetPjrtApi", "RyftMi355x_ExecuteNoAlloc"]
    for d in decls:
        assert hasattr(lib, d)


def test_api_table(plugin):
    api = plugin.api()
    assert api.version == pjrt.VERSION == (0, 104)
    assert api.struct_size == 40 + 135 * 8
    assert len(pjrt.SLOTS) == 135
    # slots ryft-pjrt calls on the hot path are populated
    for name in ["PJRT_Client_Create", "PJRT_Client_Compile", "PJRT_Client_BufferFromHostBuffer",
                 "PJRT_LoadedExecutable_Execute", "PJRT_LoadedExecutable_GetExecutable", "PJRT_Executable_NumOutputs",
                 "PJRT_Executable_Destroy", "PJRT_Buffer_ToHostBuffer", "PJRT_Event_Await", "PJRT_Event_OnReady",
                 "PJRT_Device_DefaultMemory", "PJRT_Error_Destroy",
                 # the rest of what ryft-pjrt's test_client_compile calls (programs.rs:2576-2623), executable
                 # serialization, raw copies and execution contexts
                 "PJRT_LoadedExecutable_GetDeviceAssignment", "PJRT_Executable_GetCompiledMemoryStats",
                 "PJRT_Executable_ParameterMemoryKinds", "PJRT_Executable_OutputMemoryKinds",
                 "PJRT_Executable_Serialize", "PJRT_Executable_DeserializeAndLoad", "PJRT_Buffer_CopyRawToHost",
                 "PJRT_ExecuteContext_Create", "PJRT_ExecuteContext_Destroy"]:
        assert api.fn(name) is not None
    with pytest.raises(pjrt.PjrtError) as e:
        api.fn("PJRT_Compile")
    assert e.value.code == pjrt.ErrorCode.UNIMPLEMENTED


def test_failure_propagation_slots(plugin, compile_client):
    # error buffers and poisoned executions (buffers.rs:2321-2430, devices.rs:257-300): both slots are filled, the
    # args structs the Python mirror declares have the sizes the header asserts, and a compile-only client (no
    # memory to place the buffer in) rejects an error buffer without a memory
    api = plugin.api()
    assert api.fn("PJRT_Client_CreateErrorBuffer") is not None
    assert api.fn("PJRT_Device_PoisonExecution") is not None
    assert ctypes.sizeof(pjrt.A["PJRT_Client_CreateErrorBuffer"]) == 112
    assert ctypes.sizeof(pjrt.A["PJRT_Device_PoisonExecution"]) == 72
    dims = (ctypes.c_int64 * 1)(4)
    msg = b"boom"
    with pytest.raises(pjrt.PjrtError) as e:
        api.call("PJRT_Client_CreateErrorBuffer", client=compile_client.handle, error_code=int(pjrt.ErrorCode.ABORTED),
                 error_message=ctypes.cast(ctypes.c_char_p(msg), ctypes.c_void_p), error_message_size=len(msg),
                 shape_dims=dims, shape_num_dims=1, shape_element_type=int(pjrt.BufferType.U8), memory=None)
    assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT and "memory" in e.value.message


def test_plugin_attributes(plugin):
    attrs = plugin.attributes()
    assert attrs["stablehlo_current_version"] == [1, 16, 0]
    assert attrs["stablehlo_minimum_version"] == [0, 9, 0]
    assert attrs["xla_version"] == 2
    with pytest.raises(pjrt.PjrtError) as e:
        plugin.attribute("__missing__")
    assert e.value.code == pjrt.ErrorCode.NOT_FOUND


def test_extension_chain(plugin):
    assert plugin.api().extension(pjrt.RYFT_MI355X_EXTENSION_TYPE) is not None
    assert plugin.api().extension(pjrt.PJRT_EXTENSION_TYPE_LAYOUTS) is not None
    assert plugin.api().extension(pjrt.PJRT_EXTENSION_TYPE_MEMORY_DESCRIPTIONS) is not None
    assert plugin.api().extension(profiler.PJRT_EXTENSION_TYPE_PROFILER) is not None


def test_profiler_extension(plugin, compile_client):
    # as ryft-pjrt's test_profiler_extension (extensions/profiler.rs:536-550) for the GPU plugins
    assert plugin.profiler_extension().trace_me_context_id == 0
    assert compile_client.profiler_extension().table == plugin.profiler_extension().table


def test_profiler_session_records_compilation(compile_client):
    """Create → start → compile → stop → results on a compile-only client: a host plane with the compilation's span,
    no device plane (nothing ran) and no errors."""
    prof = compile_client.profiler(profiler.ProfileOptions(version=1, device_type=1, host_tracing_level=2,
                                                           device_tracing_level=1))
    prof.start()
    compile_client.compile(pjrt.Program.mlir(ADD_2X1))
    prof.stop()
    space = prof.results()
    assert space.errors == []
    host = space.plane("/host:CPU")
    assert host is not None and [p.name for p in space.planes] == ["/host:CPU"]
    (line,) = host.lines
    assert [e.name for e in line.events] == ["compile main"]
    assert line.events[0].duration_ps > 0 and line.timestamp_ns > 0
    assert prof.results_bytes() == prof.results_bytes()  # serialization is deterministic


def test_profiler_session_errors_and_levels(compile_client, plugin):
    prof = plugin.profiler()
    with pytest.raises(pjrt.PjrtError) as e:
        prof.stop()  # never started
    assert e.value.code == pjrt.ErrorCode.FAILED_PRECONDITION
    prof.start()
    with pytest.raises(pjrt.PjrtError) as e:
        prof.start()
    assert e.value.code == pjrt.ErrorCode.FAILED_PRECONDITION
    with pytest.raises(pjrt.PjrtError) as e:
        prof.results()  # still running
    assert e.value.code == pjrt.ErrorCode.FAILED_PRECONDITION
    prof.stop()
    assert prof.results().errors == []
    # host tracing level 0: no host plane; compilations after stop are not recorded by a stopped session
    quiet = compile_client.profiler(profiler.ProfileOptions(host_tracing_level=0))
    quiet.start()
    compile_client.compile(pjrt.Program.mlir(ADD_2X1))
    quiet.stop()
    assert quiet.results().planes == []
    compile_client.compile(pjrt.Program.mlir(ADD_2X1))
    assert [e.name for e in prof.results().plane("/host:CPU").lines[0].events] == []
    # version 0 stands for the default session, whatever the levels say
    default = compile_client.profiler(profiler.ProfileOptions(version=0, host_tracing_level=0))
    default.start()
    compile_client.compile(pjrt.Program.mlir(ADD_2X1))
    default.stop()
    assert [p.name for p in default.results().planes] == ["/host:CPU"]
    ext = plugin.profiler_extension()
    bad = (ctypes.c_ubyte * 2)(0x10, 0x80)  # field 2, varint truncated
    args = profiler._CreateArgs(0, ctypes.cast(bad, ctypes.c_void_p), 2, None)
    with pytest.raises(pjrt.PjrtError) as e:
        ext.call("PLUGIN_Profiler_Create", args)
    assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT and "profile options" in str(e.value)


def test_profile_options_encoding():
    # field numbers of tensorflow.ProfileOptions (protos.rs:3423-3490)
    enc = profiler.ProfileOptions(version=1, device_type=1, host_tracing_level=2, device_tracing_level=1).encode()
    assert enc == bytes([0x10, 2, 0x18, 1, 0x28, 1, 0x30, 1])
    assert profiler.ProfileOptions(version=0, host_tracing_level=0, device_tracing_level=0).encode() == b""


def test_layouts_extension_default_layouts(compile_client):
    # as ryft-pjrt's test_layout (extensions/layouts.rs:829-841): the default layout of an f32 [2, 3, 4] buffer is
    # the dense row-major {2,1,0}, and equal layouts serialize equally
    layout = compile_client.default_layout(pjrt.BufferType.F32, [2, 3, 4])
    assert layout.serialize() == "{2,1,0}"
    assert repr(layout) == "Layout[{2,1,0}]"
    assert layout == compile_client.default_layout(pjrt.BufferType.BF16, [7, 1, 9])
    assert compile_client.default_layout(pjrt.BufferType.S32, []).serialize() == "{}"
    assert compile_client.default_layout(pjrt.BufferType.S8, [5]).serialize() == "{0}"
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.default_layout(pjrt.BufferType.F32, [2, -1])
    assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT


def test_layouts_extension_executable_layouts(compile_client):
    # ryft-pjrt's test_executable_layouts (extensions/layouts.rs:944-1000): two [2, 1] i32 parameters and one result,
    # all {1,0}; the layouts belong to the executable (borrowed, never destroyed by the caller)
    e = compile_client.compile(pjrt.Program.mlir(ADD_2X1)).executable()
    ins, outs = e.input_layouts(), e.output_layouts()
    assert [x.serialize() for x in ins] == ["{1,0}", "{1,0}"]
    assert len(outs) == e.output_count() and [x.serialize() for x in outs] == ["{1,0}"]
    assert all(x.borrowed for x in ins + outs)
    e2 = compile_client.compile(pjrt.Program.mlir(configs.c4_causal_attention(b=1, h=2, s=128).program)).executable()
    assert [x.serialize() for x in e2.input_layouts()] == ["{3,2,1,0}"] * 3


ADD_2X1 = """module {
  func.func @main(%arg0: tensor<2x1xi32>, %arg1: tensor<2x1xi32>) -> tensor<2x1xi32> {
    %0 = stablehlo.add %arg0, %arg1 : tensor<2x1xi32>
    return %0 : tensor<2x1xi32>
  }
}
"""


def test_compile_only_client(compile_client):
    c = compile_client
    assert c.platform_name() == "rocm"
    assert c.process_index() == 0
    assert c.devices() == []


def _plan(client, program):
    exe = client.compile(pjrt.Program.mlir(program))
    return exe, [ln.split(":")[1].split()[0] for ln in exe.describe_plan().strip().splitlines()]


@pytest.mark.parametrize("name,kw,expect", [
    ("c1", {}, ["gemm_f32_mfma_64x64_splitk8"]),
    ("c2", {}, ["gemm_bf16_mfma_256x256"]),
    ("c3", {}, ["gemm_i8_mfma_256x256"]),
    ("c4", {}, ["attention_fwd"]),
    ("c5", {}, ["row_norm", "gemm_bf16f8_mfma_dual_256x128", "gemm_bf16f8_mfma_128x256_splitk4"]),
    ("c5", {"weights": "direct"}, ["row_norm", "gemm_bf16f8_mfma_dual_256x128", "gemm_bf16f8_mfma_128x256_splitk4"]),
    ("c5x", {}, ["row_norm", "gemm_fp8_mfma_dual_128x128", "gemm_fp8_mfma_128x128_splitk2"]),
])
def test_full_size_plans(compile_client, name, kw, expect):
    w = configs.CONFIGS[name](**kw)
    exe, kernels = _plan(compile_client, w.program)
    assert kernels == expect
    e = exe.executable()
    assert e.name() == "main"
    assert e.replica_count() == 1 and e.computation_count() == 1
    cost = e.cost_analysis()
    assert cost["flops"] == pytest.approx(w.flops, rel=1e-3)


def test_int8_epilogue_writes_both_outputs(compile_client):
    w = configs.c3_int8_gemm()
    exe = compile_client.compile(pjrt.Program.mlir(w.program))
    e = exe.executable()
    assert e.output_element_types() == [pjrt.BufferType.S32, pjrt.BufferType.F32]
    assert e.output_dimensions() == [[4096, 4096], [4096, 4096]]
    plan = exe.describe_plan()
    assert "epilogue=1" in plan and len(plan.strip().splitlines()) == 1


# Printer goldens of ryft-mlir, which fix the text the front-end must accept.
GOLDENS = {
    # crates/ryft-mlir/src/dialects/stable_hlo/operations/linear_algebra.rs:2240-2263 (joined lines)
    "dot_general_algorithm": """module {
  func.func @main(%arg0: tensor<2x2x2xi64>, %arg1: tensor<2x2x2xi64>) -> tensor<2x2x2xi64> {
    %0 = stablehlo.dot_general %arg0, %arg1, batching_dims = [0] x [0], contracting_dims = [2] x [1], algorithm = <lhs_precision_type = f8E5M2, rhs_precision_type = f8E5M2, accumulation_type = f32, lhs_component_count = 1, rhs_component_count = 1, num_primitive_operations = 1, allow_imprecise_accumulation = true> : (tensor<2x2x2xi64>, tensor<2x2x2xi64>) -> tensor<2x2x2xi64>
    return %0 : tensor<2x2x2xi64>
  }
}""",
    # functional.rs:529-541
    "reduce": """module {
  func.func @main(%arg0: tensor<3x4xi32>, %arg1: tensor<i32>) -> tensor<3xi32> {
    %0 = stablehlo.reduce(%arg0 init: %arg1) applies stablehlo.add across dimensions = [1] : (tensor<3x4xi32>, tensor<i32>) -> tensor<3xi32>
    return %0 : tensor<3xi32>
  }
}""",
    # manipulation.rs:2022
    "transpose": """module {
  func.func @main(%arg0: tensor<3x4x5xi32>) -> tensor<5x3x4xi32> {
    %0 = stablehlo.transpose %arg0, dims = [2, 0, 1] : (tensor<3x4x5xi32>) -> tensor<5x3x4xi32>
    return %0 : tensor<5x3x4xi32>
  }
}""",
    # manipulation.rs:2154
    "broadcast_in_dim": """module {
  func.func @main(%arg0: tensor<1x3xi32>) -> tensor<2x3x2xi32> {
    %0 = stablehlo.broadcast_in_dim %arg0, dims = [2, 1] : (tensor<1x3xi32>) -> tensor<2x3x2xi32>
    return %0 : tensor<2x3x2xi32>
  }
}""",
    # control_flow.rs:596
    "select": """module {
  func.func @main(%arg0: tensor<3x4xi1>, %arg1: tensor<3x4xi32>, %arg2: tensor<3x4xi32>) -> tensor<3x4xi32> {
    %0 = stablehlo.select %arg0, %arg1, %arg2 : tensor<3x4xi1>, tensor<3x4xi32>
    return %0 : tensor<3x4xi32>
  }
}""",
    # miscellaneous.rs:1181
    "iota": """module {
  func.func @main() -> tensor<4x5xi32> {
    %0 = stablehlo.iota dim = 1 : tensor<4x5xi32>
    return %0 : tensor<4x5xi32>
  }
}""",
    # comparison.rs:500
    "compare": """module {
  func.func @main(%arg0: tensor<3xf32>, %arg1: tensor<3xf32>) -> tensor<3xi1> {
    %0 = stablehlo.compare GE, %arg0, %arg1, TOTALORDER : (tensor<3xf32>, tensor<3xf32>) -> tensor<3xi1>
    return %0 : tensor<3xi1>
  }
}""",
    # manipulation.rs:2257-2265, 2388-2389, 2438 (joined lines, entry renamed @main)
    "pad": """module {
  func.func @main(%arg0: tensor<2x3xi32>, %arg1: tensor<i32>) -> tensor<5x5xi32> {
    %0 = stablehlo.pad %arg0, %arg1, low = [0, 1], high = [2, 1], interior = [1, 0] : (tensor<2x3xi32>, tensor<i32>) -> tensor<5x5xi32>
    return %0 : tensor<5x5xi32>
  }
}""",
    "concatenate": """module {
  func.func @main(%arg0: tensor<3x2xi64>, %arg1: tensor<1x2xi64>) -> tensor<4x2xi64> {
    %0 = stablehlo.concatenate %arg0, %arg1, dim = 0 : (tensor<3x2xi64>, tensor<1x2xi64>) -> tensor<4x2xi64>
    return %0 : tensor<4x2xi64>
  }
}""",
    "slice": """module {
  func.func @main(%arg0: tensor<3x4x5xi32>) -> tensor<2x2x3xi32> {
    %0 = stablehlo.slice %arg0 [0:2, 1:3, 0:5:2] : (tensor<3x4x5xi32>) -> tensor<2x2x3xi32>
    return %0 : tensor<2x2x3xi32>
  }
}""",
    # README.md example (programs.rs test program shape) with the reduce region form and generic syntax
    "generic_forms": """module @jit_f attributes {mhlo.num_partitions = 1 : i32} {
  func.func public @main(%arg0: tensor<4x8xf32> {mhlo.sharding = "{replicated}"}) -> (tensor<4xf32> {jax.result_info = ""}) {
    %cst = stablehlo.constant dense<0xFF800000> : tensor<f32>
    %0 = stablehlo.reduce(%arg0 init: %cst) across dimensions = [1] : (tensor<4x8xf32>, tensor<f32>) -> tensor<4xf32>
     reducer(%arg1: tensor<f32>, %arg2: tensor<f32>)  {
      %2 = stablehlo.maximum %arg1, %arg2 : tensor<f32>
      stablehlo.return %2 : tensor<f32>
    }
    %1 = "stablehlo.exponential"(%0) : (tensor<4xf32>) -> tensor<4xf32>
    return %1 : tensor<4xf32>
  }
}""",
}


@pytest.mark.parametrize("name", sorted(GOLDENS))
def test_printer_golden_forms_compile(compile_client, name):
    exe = compile_client.compile(pjrt.Program.mlir(GOLDENS[name]))
    assert exe.executable().output_count() == 1


def test_malformed_bytecode_is_invalid_argument(compile_client):
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.compile(pjrt.Program.mlir(b"ML\xefR\x0dMLIR\x00\x05rest-of-bytecode"))
    assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT
    assert "bytecode" in e.value.message


def test_hlo_format_is_rejected(compile_client):
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.compile(pjrt.Program(b"HloModule m", "hlo"))
    assert e.value.code == pjrt.ErrorCode.UNIMPLEMENTED


def test_parse_errors_are_invalid_argument(compile_client):
    bad = GOLDENS["transpose"].replace("dims = [2, 0, 1]", "dims = [2, 0")
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.compile(pjrt.Program.mlir(bad))
    assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT


def test_unsupported_op_is_unimplemented(compile_client):
    prog = GOLDENS["transpose"].replace("stablehlo.transpose %arg0, dims = [2, 0, 1]", "stablehlo.fft %arg0")
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.compile(pjrt.Program.mlir(prog))
    assert e.value.code in (pjrt.ErrorCode.UNIMPLEMENTED, pjrt.ErrorCode.INVALID_ARGUMENT)


def test_shape_mismatch_is_invalid_argument(compile_client):
    prog = GOLDENS["transpose"].replace("-> tensor<5x3x4xi32>\n    return", "-> tensor<5x4x3xi32>\n    return")
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.compile(pjrt.Program.mlir(prog))
    assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT


def test_compile_options_round_trip(compile_client):
    opts = pjrt.CompilationOptions(matrix_unit_operand_precision=0)
    exe = compile_client.compile(pjrt.Program.mlir(GOLDENS["iota"]), opts)
    assert exe.executable().compile_options() == opts.encode()
    assert len(exe.executable().fingerprint()) == 16


def _ebo(*fields):
    """CompileOptionsProto bytes whose executable_build_options (field 3) holds `fields` (raw encoded fields)."""
    body = b"".join(fields)
    return b"\x1a" + bytes([len(body)]) + body


@pytest.mark.parametrize("name,opts,code", [
    ("two_replicas", pjrt.CompilationOptions(replica_count=2).encode(), pjrt.ErrorCode.UNIMPLEMENTED),
    ("two_partitions", pjrt.CompilationOptions(partition_count=2).encode(), pjrt.ErrorCode.UNIMPLEMENTED),
    ("tupled_parameters", b"\x10\x01", pjrt.ErrorCode.UNIMPLEMENTED),
    # device assignment {replica_count 2, computation_count 1, ids [0, 1]}
    ("two_device_assignment", _ebo(b"\x4a\x0a\x08\x02\x10\x01\x1a\x04\x0a\x02\x00\x01"), pjrt.ErrorCode.UNIMPLEMENTED),
    ("assignment_size_mismatch", _ebo(b"\x4a\x09\x08\x02\x10\x01\x1a\x03\x0a\x01\x00"), pjrt.ErrorCode.INVALID_ARGUMENT),
    ("truncated_build_options", b"\x1a\x05\x08", pjrt.ErrorCode.INVALID_ARGUMENT),
    ("truncated_varint", b"\x50\x80", pjrt.ErrorCode.INVALID_ARGUMENT),
    ("group_wire_type", b"\x0b", pjrt.ErrorCode.INVALID_ARGUMENT),
    ("unknown_precision", b"\x50\x03", pjrt.ErrorCode.INVALID_ARGUMENT),
    ("negative_device_ordinal", _ebo(b"\x08" + b"\xfe" + b"\xff" * 8 + b"\x01"), pjrt.ErrorCode.INVALID_ARGUMENT),
])
def test_compile_options_rejected(compile_client, name, opts, code):
    """CompileOptionsProto decoding (protos.rs:3298-3346, 2391-2530): what one executable of this plugin cannot be
    (several replicas / partitions / devices, tupled parameters) is UNIMPLEMENTED; malformed bytes are
    INVALID_ARGUMENT."""
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.compile(pjrt.Program.mlir(GOLDENS["iota"]), opts)
    assert e.value.code == code, (name, e.value)


@pytest.mark.parametrize("name,opts", [
    ("empty", b""),
    ("defaults", pjrt.CompilationOptions().encode()),
    ("highest_precision", pjrt.CompilationOptions(matrix_unit_operand_precision=2).encode()),
    ("device_ordinal_0", pjrt.CompilationOptions(device_ordinal=0).encode()),
    # one-device assignment {1, 1, [0]}, packed and unpacked id encodings
    ("one_device_assignment", _ebo(b"\x4a\x08\x08\x01\x10\x01\x1a\x02\x08\x00")),
    ("one_device_assignment_packed", _ebo(b"\x4a\x09\x08\x01\x10\x01\x1a\x03\x0a\x01\x00")),
    # fields the plugin does not act on are skipped by wire type: portable (4), profile_version (5), multi-slice
    # config bytes (6), an unknown fixed64 (15) and fixed32 (16) field, debug options inside the build options
    ("skipped_fields", b"\x20\x01\x28\x07\x32\x02ab\x79" + b"\x00" * 8 + b"\x85\x01" + b"\x00" * 4 +
     _ebo(b"\x1a\x02\x08\x01", b"\x20\x01")),
])
def test_compile_options_accepted(compile_client, name, opts):
    exe = compile_client.compile(pjrt.Program.mlir(GOLDENS["iota"]), opts)
    assert exe.executable().compile_options() == opts


def test_serialize_deserialize_round_trip(compile_client):
    # as ryft-pjrt's test_client_deserialize_and_load_executable (programs.rs:2691-2723): the deserialized executable
    # reports the same name, counts, output types / dims / memory kinds, fingerprint and compile options
    opts = pjrt.CompilationOptions()
    le = compile_client.compile(pjrt.Program.mlir(configs.c3_int8_gemm(m=256, k=256, n=256).program), opts)
    e = le.executable()
    blob = e.serialize()
    le2 = compile_client.deserialize_and_load_executable(blob, opts)
    e2 = le2.executable()
    assert e2.name() == e.name() == "main"
    assert (e2.replica_count(), e2.computation_count()) == (e.replica_count(), e.computation_count()) == (1, 1)
    assert e2.output_count() == e.output_count() == 2
    assert e2.output_element_types() == e.output_element_types() == [pjrt.BufferType.S32, pjrt.BufferType.F32]
    assert e2.output_dimensions() == e.output_dimensions() == [[256, 256], [256, 256]]
    assert e2.output_memory_kinds() == e.output_memory_kinds() == ["device", "device"]
    assert e2.fingerprint() == e.fingerprint()
    assert e2.compile_options() == opts.encode()
    assert e2.cost_analysis() == e.cost_analysis()
    assert le2.describe_plan() == le.describe_plan()
    # serializing the deserialized executable gives the same bytes; without override options the serialized
    # ones are used
    assert e2.serialize() == blob
    assert compile_client.deserialize_and_load_executable(blob).executable().compile_options() == opts.encode()


@pytest.mark.parametrize("mutate", ["magic", "truncate_length", "truncate_payload", "trailing"])
def test_malformed_serialized_executable_is_invalid_argument(compile_client, mutate):
    blob = compile_client.compile(pjrt.Program.mlir(GOLDENS["iota"])).executable().serialize()
    bad = {"magic": b"XXXX" + blob[4:], "truncate_length": blob[:12], "truncate_payload": blob[:-3],
           "trailing": blob + b"\0"}[mutate]
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.deserialize_and_load_executable(bad)
    assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT


def test_memory_statistics_and_memory_kinds(compile_client):
    # C1 plans an 8-range split-K: the f32 partial sums are the executable's only temporary (8 × 256 × 256 × 4 B);
    # its one constant is the zero-initialised arrival counter per 64×64 output tile of the in-kernel finish (16 × 4 B)
    e = compile_client.compile(pjrt.Program.mlir(configs.c1_f32_dot().program)).executable()
    st = e.memory_statistics()
    assert st["argument_size_in_bytes"] == 2 * 256 * 512 * 4
    assert st["output_size_in_bytes"] == 256 * 256 * 4
    assert st["temp_size_in_bytes"] == 8 * 256 * 256 * 4
    assert st["generated_code_size_in_bytes"] == 0 and st["alias_size_in_bytes"] == 0
    assert st["peak_memory_in_bytes"] == (st["argument_size_in_bytes"] + st["output_size_in_bytes"] +
                                          st["temp_size_in_bytes"] + 16 * 4)
    assert e.input_memory_kinds() == ["device", "device"]
    assert e.output_memory_kinds() == ["device"]


def test_execution_context_create_destroy(compile_client):
    ctx = compile_client.execution_context()
    assert ctx.handle
    del ctx


def test_device_assignment_needs_a_device(compile_client):
    le = compile_client.compile(pjrt.Program.mlir(GOLDENS["iota"]))
    with pytest.raises(pjrt.PjrtError) as e:
        le.device_assignment()
    assert e.value.code == pjrt.ErrorCode.FAILED_PRECONDITION


def test_device_assignment_proto_decoding():
    # xla.DeviceAssignmentProto{replica_count: 2, computation_count: 1, computation_devices: [{replica_device_ids:
    # [3, 5]}]} in both the packed and the unpacked repeated encodings, read as devices.rs:674-688 does
    packed = bytes([0x08, 2, 0x10, 1, 0x1a, 4, 0x0a, 2, 3, 5])
    unpacked = bytes([0x08, 2, 0x10, 1, 0x1a, 4, 0x08, 3, 0x08, 5])
    for data in (packed, unpacked):
        assert pjrt.DeviceAssignment.decode(data) == pjrt.DeviceAssignment(2, 1, [3, 5])
    with pytest.raises(pjrt.PjrtError):
        pjrt.DeviceAssignment.decode(bytes([0x08, 2, 0x10, 1, 0x1a, 3, 0x0a, 1, 3]))  # one id for two replicas


def test_slice_concatenate_pad_plans(compile_client):
    # a slice is a view (no step of its own: the slice of a parameter feeding an add is one elementwise step, and a
    # bf16 slice feeding a dot is read by the GEMM in place); concatenate writes each operand's expression into its
    # region (one step per operand); pad is a fill plus one strided write
    prog = """module {
  func.func @main(%arg0: tensor<8x16xf32>, %arg1: tensor<8x16xf32>, %arg2: tensor<f32>) -> (tensor<8x8xf32>, tensor<8x40xf32>, tensor<12x17xf32>) {
    %0 = stablehlo.slice %arg0 [0:8, 4:12] : (tensor<8x16xf32>) -> tensor<8x8xf32>
    %1 = stablehlo.slice %arg1 [0:8, 0:16:2] : (tensor<8x16xf32>) -> tensor<8x8xf32>
    %2 = stablehlo.add %0, %1 : tensor<8x8xf32>
    %3 = stablehlo.negate %arg1 : tensor<8x16xf32>
    %4 = stablehlo.concatenate %3, %2, %arg0, dim = 1 : (tensor<8x16xf32>, tensor<8x8xf32>, tensor<8x16xf32>) -> tensor<8x40xf32>
    %5 = stablehlo.pad %arg0, %arg2, low = [1, -1], high = [3, 2], interior = [0, 0] : (tensor<8x16xf32>, tensor<f32>) -> tensor<12x17xf32>
    return %2, %4, %5 : tensor<8x8xf32>, tensor<8x40xf32>, tensor<12x17xf32>
  }
}"""
    with pytest.raises(pjrt.PjrtError) as e:  # 12x17 is the pad's shape; 11x18 is not
        compile_client.compile(pjrt.Program.mlir(prog.replace("tensor<12x17xf32>", "tensor<11x18xf32>")))
    assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT
    exe, kinds = _plan(compile_client, prog)
    assert kinds.count("elementwise") == 1
    assert kinds.count("concatenate") == 3
    assert kinds.count("pad_fill") == 1 and kinds.count("pad") == 1
    dot = """module {
  func.func @main(%arg0: tensor<64x256xbf16>, %arg1: tensor<128x64xbf16>) -> tensor<64x64xf32> {
    %0 = stablehlo.slice %arg0 [0:64, 128:256] : (tensor<64x256xbf16>) -> tensor<64x128xbf16>
    %1 = stablehlo.dot_general %0, %arg1, contracting_dims = [1] x [0] : (tensor<64x128xbf16>, tensor<128x64xbf16>) -> tensor<64x64xf32>
    return %1 : tensor<64x64xf32>
  }
}"""
    _, kinds = _plan(compile_client, dot)
    assert len(kinds) == 1 and kinds[0].startswith("gemm"), kinds


@pytest.mark.parametrize("bad", [
    ("slice %arg0 [0:2, 1:3, 0:5:2]", "slice %arg0 [0:2, 1:5, 0:5:2]"),      # limit past the dimension
    ("slice %arg0 [0:2, 1:3, 0:5:2]", "slice %arg0 [0:2, 1:3, 0:5:0]"),      # zero stride
    ("slice %arg0 [0:2, 1:3, 0:5:2]", "slice %arg0 [0:2, 1:3]"),             # one entry per dimension
])
def test_slice_validation_errors(compile_client, bad):
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.compile(pjrt.Program.mlir(GOLDENS["slice"].replace(*bad)))
    assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT


def test_attention_not_fused_when_intermediate_escapes(compile_client):
    # returning the probabilities as well forces the unfused path (the [S,S] matrix is a program result)
    w = configs.c4_causal_attention(b=1, h=1, s=128, d=64)
    prog = w.program.replace("return %18 : ", "return %18, %15 : ").replace(
        "-> tensor<1x1x128x64xbf16> {", "-> (tensor<1x1x128x64xbf16>, tensor<1x1x128x128xf32>) {").replace(
        "return %18, %15 : tensor<1x1x128x64xbf16>", "return %18, %15 : tensor<1x1x128x64xbf16>, tensor<1x1x128x128xf32>")
    exe, kernels = _plan(compile_client, prog)
    assert "attention_fwd" not in kernels
    assert exe.executable().output_count() == 2


@pytest.mark.parametrize("name,kw", [
    ("s200", dict(s=200)),                        # not a multiple of the 128-query block
    ("s96", dict(s=96)),
    ("strict_mask", dict(mask="GT")),             # query 0 sees no key: NaN under the -inf fill
    ("finite_fill", dict(fill="-3.40282347E+38")),
    ("f32_probabilities", dict(p_type="f32")),    # P·V asks for f32 P; the kernel rounds P to bf16
])
def test_attention_declined_when_the_kernel_cannot_run_it(compile_client, name, kw):
    """The fused kernel's preconditions are checked when planning: a graph it cannot run (or would compute
    differently) plans to the unfused steps instead of failing or deviating at execute time."""
    base = dict(b=1, h=2, s=256, d=128)
    base.update(kw)
    w = configs.c4_causal_attention(**base)
    exe, kernels = _plan(compile_client, w.program)
    assert "attention_fwd" not in kernels, (name, kernels)
    _, kernels = _plan(compile_client, configs.c4_causal_attention(b=1, h=2, s=256, d=128).program)
    assert "attention_fwd" in kernels


def test_edge_tile_plans(compile_client):
    # shapes that are not tile multiples, and m-contiguous lhs operands, plan to the edge MFMA kernels; operands whose
    # rows are not 16-byte aligned are copied into padded rows first
    from tests.edge_programs import CASES
    for (name, prog, _), kernel, _ in CASES:
        _, kernels = _plan(compile_client, prog)
        assert kernels[-1] == kernel and all(k == "dot_operand_copy" for k in kernels[:-1]), (name, kernels)
        unaligned = "unaligned" in name or "odd" in name or name in ("fp8_n40", "bf16_f8_n72")
        assert ("dot_operand_copy" in kernels) == unaligned, (name, kernels)


@pytest.mark.parametrize("kw", [dict(m=64, d=128, f=100), dict(m=100, d=200, f=136)])
def test_ragged_swiglu_plans_stay_on_mfma(compile_client, kw):
    # weights whose rows are not 16-byte aligned are copied (still f8) into padded rows: the dual SwiGLU GEMM and the
    # down projection run on the bf16 x f8 MFMA edge kernels
    _, kernels = _plan(compile_client, configs.c5_swiglu_fp8(**kw).program)
    assert "gemm_generic" not in kernels and "gemm_bf16f8_mfma_dual_edge_128x128" in kernels, kernels


@pytest.mark.parametrize("name,build,reductions", [
    ("rmsnorm", lambda: row_programs.rmsnorm((16, 4096), "bf16"), 1),
    ("softmax", lambda: row_programs.softmax((4, 8, 200)), 2),
    ("layernorm", lambda: row_programs.layernorm((8, 33)), 2),
    ("int_row_max", lambda: row_programs.int_row_max_gap((8, 64)), 1),
])
def test_row_fusion_plans(compile_client, name, build, reductions):
    # a reduction over the innermost dim broadcast back into its consumer runs in the consumer's launch
    exe, kernels = _plan(compile_client, build())
    fused = "row_norm" if name == "rmsnorm" else "row_fused"  # RMSNorm has a specialised kernel
    assert fused in kernels, kernels
    assert f"reductions={reductions}" in exe.describe_plan()
    if name == "int_row_max":  # the row maxima are also a result: a reduce launch of their own writes them
        assert sorted(kernels) == ["reduce", "row_fused"]
    else:
        assert kernels == [fused]


def test_rmsnorm_fast_path_recognition(plugin):
    # scaled sum-of-squares normalisations run on the row-norm kernel; the fast_paths=false client option keeps them
    # on the interpreted row kernel; near misses (an extra offset) stay interpreted
    fast = plugin.client({"compile_only": True})
    slow = plugin.client({"compile_only": True, "fast_paths": False})
    for prog in (row_programs.rmsnorm((512, 4096), "bf16", quant="f8E4M3FN"), row_programs.rmsnorm((3, 5, 64))):
        assert _plan(fast, prog)[1] == ["row_norm"]
        assert _plan(slow, prog)[1] == ["row_fused"]
    near = row_programs.rmsnorm((8, 64)).replace("%12 = stablehlo.multiply %9, %11", "%12 = stablehlo.add %9, %11")
    assert _plan(fast, near)[1] == ["row_fused"]


def test_row_fusion_skips_non_innermost_reductions(compile_client):
    # a reduction over dim 0 is not a row reduction: it stays a reduce launch feeding an elementwise one
    T, R = "tensor<64x32xf32>", "tensor<32xf32>"
    prog = f"""module {{
  func.func @main(%arg0: {T}) -> {T} {{
    %cst = stablehlo.constant dense<0.000000e+00> : tensor<f32>
    %0 = stablehlo.reduce(%arg0 init: %cst) applies stablehlo.add across dimensions = [0] : ({T}, tensor<f32>) -> {R}
    %1 = stablehlo.broadcast_in_dim %0, dims = [1] : ({R}) -> {T}
    %2 = stablehlo.divide %arg0, %1 : {T}
    return %2 : {T}
  }}
}}
"""
    _, kernels = _plan(compile_client, prog)
    assert kernels == ["reduce", "elementwise"]


@pytest.mark.parametrize("name,kw,kernel", [
    ("c2", {"batch": 1, "m": 256, "k": 4096, "n": 256}, "gemm_bf16_mfma_128x128_splitk16"),
    ("c3", {"m": 256, "k": 8192, "n": 256}, "gemm_i8_mfma_128x128_splitk16"),
    ("c3", {"m": 4096, "k": 4096, "n": 4096}, "gemm_i8_mfma_256x256"),
])
def test_split_k_plans(compile_client, name, kw, kernel):
    # few output tiles over a long K: the K range is split over 128×128 tiles (partial sums in a workspace, then one
    # reduction launch applies the epilogue); tile counts that cover the chip keep one pass
    w = configs.CONFIGS[name](**kw)
    _, kernels = _plan(compile_client, w.program)
    assert kernels == [kernel]


_EXIT_SCRIPT = r'''
import atexit, sys
sys.path.insert(0, sys.argv[1])
state = {}
atexit.register(lambda: print("after hook:", state["client"].handle is None, state["exe"].handle is None,
                              state["prof"].handle is None, flush=True))
from ryft_amd import pjrt  # its exit hook is registered after the one above, so it runs first
client = pjrt.load_plugin().client({"compile_only": True})
prof = client.profiler()
prof.start()  # left started
exe = client.compile(pjrt.Program.mlir(sys.argv[2]))
state.update(client=client, exe=exe, prof=prof)
print("compiled", flush=True)
'''


def test_wrappers_alive_at_interpreter_exit_are_destroyed():
    """Objects still referenced from __main__ at exit are destroyed by the module's exit hook (executables and a
    started profiler session before their client) while ctypes is intact, instead of reaching finalizers that can no longer call the plugin."""
    import sys
    r = subprocess.run([sys.executable, "-c", _EXIT_SCRIPT, ROOT, ADD_2X1], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    assert r.stdout.split() == ["compiled", "after", "hook:", "True", "True", "True"], r.stdout + r.stderr


# ----------------------------------------------------------------------------------------------- input donation
@pytest.mark.parametrize("name,expect", [
    ("SGD", ["alias: result 0 <- parameter 0 (in place)"]),
    ("GEMM", ["alias: result 0 <- parameter 0 (own buffer)"]),
    ("TRANSPOSED", ["alias: result 0 <- parameter 0 (own buffer)"]),
    ("PASSTHROUGH", ["alias: result 1 <- parameter 0 (in place)"]),
    ("DONOR", ["alias: result 1 <- parameter 0 (in place)"]),
])
@pytest.mark.parametrize("form", ["text", "bytecode"])
def test_aliasing_plans(compile_client, name, expect, form):
    """Aliasing declared on func arguments (text attribute dictionaries, or bytecode arg_attrs) reaches the plan; a
    result is computed in place over its donated parameter only when no step reads the parameter after (or, in the
    writing step, apart from) the element being written."""
    from tests import donation_programs as dp, mlir_bytecode
    text = getattr(dp, name)
    code = text if form == "text" else mlir_bytecode.to_bytecode(text)
    le = compile_client.compile(pjrt.Program.mlir(code))
    lines = [ln for ln in le.describe_plan().splitlines() if ln.startswith("alias:")]
    assert lines == expect
    st = le.executable().memory_statistics()
    nbytes = {"SGD": 4 << 16, "GEMM": 2 * 256 * 256, "TRANSPOSED": 4 * 64 * 64, "PASSTHROUGH": 4096, "DONOR": 2048}
    assert st["alias_size_in_bytes"] == nbytes[name]


def test_no_aliasing_without_attributes(compile_client):
    le = compile_client.compile(pjrt.Program.mlir(ADD_2X1))
    assert "alias:" not in le.describe_plan()
    assert le.executable().memory_statistics()["alias_size_in_bytes"] == 0


@pytest.mark.parametrize("name", ["result_out_of_range", "type_mismatch", "two_parameters_one_result"])
def test_malformed_aliasing_is_invalid_argument(compile_client, name):
    from tests import donation_programs as dp
    program, fragment = dp.BAD[name]
    with pytest.raises(pjrt.PjrtError) as e:
        compile_client.compile(pjrt.Program.mlir(program))
    assert e.value.code == pjrt.ErrorCode.INVALID_ARGUMENT and fragment in str(e.value), str(e.value)
