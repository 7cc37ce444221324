"""Host-side mirror of ryft-pjrt's runtime API over the PJRT C ABI (ctypes).

ryft-pjrt (Rust) cannot be built in this environment, so this module replays, call for call, what its safe wrappers
do against a plugin's ``GetPjrtApi`` table:

* ``load_plugin`` / ``Plugin`` — crates/ryft-pjrt/src/plugins.rs:67-80, 120-122 (resolve ``GetPjrtApi``, call
  ``PJRT_Plugin_Initialize`` once).
* ``Plugin.client`` — clients.rs:671-692 (``PJRT_Client_Create`` with NamedValue options, no KV store).
* ``Client.compile`` — programs.rs:1245-1263 (``PJRT_Program{format="mlir"}`` + serialized CompileOptionsProto).
* ``Client.buffer`` — buffers.rs:2099-2150 (``PJRT_Client_BufferFromHostBuffer``, kImmutableOnlyDuringCall, the
  device's default memory, the ``done_with_host_buffer`` event dropped).
* ``LoadedExecutable.execute`` — programs.rs:769-963 (addressable devices, ``GetExecutable`` → ``NumOutputs`` →
  ``Executable_Destroy`` on every call, then ``PJRT_LoadedExecutable_Execute``; null outputs / events are errors).
* ``Buffer.copy_to_host`` — buffers.rs:1237-1266 (``ToHostBuffer`` twice: size query, then the copy + event).
* errors — errors.rs:76-180 (message, code, payloads, then ``PJRT_Error_Destroy``); every table access is gated on
  ``PJRT_Api.struct_size`` like macros.rs:27-108.

Names and argument meaning follow ryft-pjrt; Python spellings replace Rust ones (``await_`` for ``r#await``).
"""
from __future__ import annotations

import atexit
import threading
import ctypes as C
import enum
import os
import re
import weakref
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional, Sequence, Tuple

_HERE = os.path.dirname(os.path.abspath(__file__))
_ROOT = os.path.dirname(_HERE)
DEFAULT_PLUGIN_PATH = os.path.join(_HERE, "lib", "libryft_pjrt_mi355x.so")
_HEADER = os.path.join(_ROOT, "include", "pjrt_c_api.h")

VERSION = (0, 104)  # crates/ryft-pjrt/src/versions.rs:33-34

# ----------------------------------------------------------------------------------------------- enums


class BufferType(enum.IntEnum):
    """PJRT_Buffer_Type (crates/ryft-pjrt/src/buffers.rs:2568-2600)."""

    INVALID = 0
    PRED = 1
    S8 = 2
    S16 = 3
    S32 = 4
    S64 = 5
    U8 = 6
    U16 = 7
    U32 = 8
    U64 = 9
    F16 = 10
    F32 = 11
    F64 = 12
    BF16 = 13
    C64 = 14
    C128 = 15
    F8E5M2 = 16
    F8E4M3FN = 17

    @property
    def size(self) -> int:
        return {1: 1, 2: 1, 3: 2, 4: 4, 5: 8, 6: 1, 7: 2, 8: 4, 9: 8, 10: 2, 11: 4, 12: 8, 13: 2, 16: 1, 17: 1}[int(self)]


class ErrorCode(enum.IntEnum):
    """PJRT_Error_Code (crates/ryft-pjrt/src/errors.rs:441-457)."""

    OK = 0
    CANCELLED = 1
    UNKNOWN = 2
    INVALID_ARGUMENT = 3
    DEADLINE_EXCEEDED = 4
    NOT_FOUND = 5
    ALREADY_EXISTS = 6
    PERMISSION_DENIED = 7
    RESOURCE_EXHAUSTED = 8
    FAILED_PRECONDITION = 9
    ABORTED = 10
    OUT_OF_RANGE = 11
    UNIMPLEMENTED = 12
    INTERNAL = 13
    UNAVAILABLE = 14
    DATA_LOSS = 15
    UNAUTHENTICATED = 16


class PjrtError(Exception):
    """A PJRT_Error converted like ryft-pjrt's ``Error::from_c_api``."""

    def __init__(self, code: ErrorCode, message: str, payload: Optional[List[Tuple[str, str]]] = None):
        super().__init__(f"{code.name}: {message}")
        self.code = code
        self.message = message
        self.payload = payload or []


# ----------------------------------------------------------------------------------------------- C layouts
_sz = C.c_size_t
_vp = C.c_void_p
_cp = C.c_char_p


class ExtensionBase(C.Structure):
    pass


ExtensionBase._fields_ = [("struct_size", _sz), ("extension_type", C.c_uint), ("next", C.POINTER(ExtensionBase))]


def _args(name: str, fields: Sequence[Tuple[str, object]]):
    return type(name, (C.Structure,), {"_fields_": [("struct_size", _sz), ("extension_start", _vp)] + list(fields)})


class ApiVersion(C.Structure):
    _fields_ = [("struct_size", _sz), ("extension_start", _vp), ("major_version", C.c_int), ("minor_version", C.c_int)]


class _Value(C.Union):
    _fields_ = [("string_value", _vp), ("int64_value", C.c_int64), ("int64_array_value", C.POINTER(C.c_int64)),
                ("float_value", C.c_float), ("bool_value", C.c_bool)]


class NamedValue(C.Structure):
    _anonymous_ = ("value",)
    _fields_ = [("struct_size", _sz), ("extension_start", _vp), ("name", _vp), ("name_size", _sz),
                ("type", C.c_uint), ("value", _Value), ("value_size", _sz)]


class Program_(C.Structure):
    _fields_ = [("struct_size", _sz), ("extension_start", _vp), ("code", _vp), ("code_size", _sz),
                ("format", _vp), ("format_size", _sz)]


class MemoryLayoutTiled(C.Structure):
    _fields_ = [("struct_size", _sz), ("extension_start", _vp), ("minor_to_major", C.POINTER(C.c_int64)),
                ("minor_to_major_size", _sz), ("tile_dims", _vp), ("tile_dim_sizes", _vp), ("num_tiles", _sz)]


class MemoryLayoutStrides(C.Structure):
    _fields_ = [("struct_size", _sz), ("extension_start", _vp), ("byte_strides", _vp), ("num_byte_strides", _sz)]


class _LayoutU(C.Union):
    _fields_ = [("tiled", MemoryLayoutTiled), ("strides", MemoryLayoutStrides)]


class MemoryLayout(C.Structure):
    _anonymous_ = ("u",)
    _fields_ = [("struct_size", _sz), ("extension_start", _vp), ("u", _LayoutU), ("type", C.c_uint)]


class LogicalDeviceIds(C.Structure):
    _fields_ = [("replica", C.c_int), ("partition", C.c_int)]


class ExecuteOptions(C.Structure):
    _fields_ = [("struct_size", _sz), ("extension_start", _vp), ("send_callbacks", _vp), ("recv_callbacks", _vp),
                ("num_send_ops", _sz), ("num_recv_ops", _sz), ("launch_id", C.c_int),
                ("non_donatable_input_indices", C.POINTER(C.c_int64)), ("num_non_donatable_input_indices", _sz),
                ("context", _vp), ("call_location", _vp), ("num_tasks", _sz), ("task_ids", _vp),
                ("incarnation_ids", _vp), ("multi_slice_config", _vp)]


OnReadyCallback = C.CFUNCTYPE(None, _vp, _vp)
PayloadVisitor = C.CFUNCTYPE(None, _vp, _sz, _vp, _sz, _vp)

A = {}  # args struct types by PJRT function name
for _n, _f in {
    "PJRT_Error_Destroy": [("error", _vp)],
    "PJRT_Error_Message": [("error", _vp), ("message", _vp), ("message_size", _sz)],
    "PJRT_Error_GetCode": [("error", _vp), ("code", C.c_uint)],
    "PJRT_Error_ForEachPayload": [("error", _vp), ("visitor", PayloadVisitor), ("user_arg", _vp)],
    "PJRT_Plugin_Initialize": [],
    "PJRT_Plugin_Attributes": [("attributes", C.POINTER(NamedValue)), ("num_attributes", _sz)],
    "PJRT_Event_Destroy": [("event", _vp)],
    "PJRT_Event_IsReady": [("event", _vp), ("is_ready", C.c_bool)],
    "PJRT_Event_Error": [("event", _vp)],
    "PJRT_Event_Await": [("event", _vp)],
    "PJRT_Event_OnReady": [("event", _vp), ("callback", OnReadyCallback), ("user_arg", _vp)],
    "PJRT_Event_Create": [("event", _vp)],
    "PJRT_Event_Set": [("event", _vp), ("error_code", C.c_uint), ("error_message", _vp), ("error_message_size", _sz)],
    "PJRT_Client_Create": [("create_options", C.POINTER(NamedValue)), ("num_options", _sz), ("kv_get_callback", _vp),
                           ("kv_get_user_arg", _vp), ("kv_put_callback", _vp), ("kv_put_user_arg", _vp),
                           ("client", _vp), ("kv_try_get_callback", _vp), ("kv_try_get_user_arg", _vp)],
    "PJRT_Client_Destroy": [("client", _vp)],
    "PJRT_Client_PlatformName": [("client", _vp), ("platform_name", _vp), ("platform_name_size", _sz)],
    "PJRT_Client_ProcessIndex": [("client", _vp), ("process_index", C.c_int)],
    "PJRT_Client_PlatformVersion": [("client", _vp), ("platform_version", _vp), ("platform_version_size", _sz)],
    "PJRT_Client_Devices": [("client", _vp), ("devices", C.POINTER(_vp)), ("num_devices", _sz)],
    "PJRT_Client_AddressableDevices": [("client", _vp), ("addressable_devices", C.POINTER(_vp)),
                                       ("num_addressable_devices", _sz)],
    "PJRT_Client_LookupDevice": [("client", _vp), ("id", C.c_int), ("device", _vp)],
    "PJRT_Client_LookupAddressableDevice": [("client", _vp), ("local_hardware_id", C.c_int),
                                            ("addressable_device", _vp)],
    "PJRT_Client_AddressableMemories": [("client", _vp), ("addressable_memories", C.POINTER(_vp)),
                                        ("num_addressable_memories", _sz)],
    "PJRT_Client_Compile": [("client", _vp), ("program", C.POINTER(Program_)), ("compile_options", _vp),
                            ("compile_options_size", _sz), ("executable", _vp)],
    "PJRT_Client_DefaultDeviceAssignment": [("client", _vp), ("num_replicas", C.c_int), ("num_partitions", C.c_int),
                                            ("default_assignment_size", _sz),
                                            ("default_assignment", C.POINTER(C.c_int))],
    "PJRT_Client_BufferFromHostBuffer": [("client", _vp), ("data", _vp), ("type", C.c_uint),
                                         ("dims", C.POINTER(C.c_int64)), ("num_dims", _sz),
                                         ("byte_strides", C.POINTER(C.c_int64)), ("num_byte_strides", _sz),
                                         ("host_buffer_semantics", C.c_uint), ("device", _vp), ("memory", _vp),
                                         ("device_layout", _vp), ("done_with_host_buffer", _vp), ("buffer", _vp)],
    "PJRT_DeviceDescription_Id": [("device_description", _vp), ("id", C.c_int)],
    "PJRT_DeviceDescription_ProcessIndex": [("device_description", _vp), ("process_index", C.c_int)],
    "PJRT_DeviceDescription_Attributes": [("device_description", _vp), ("num_attributes", _sz),
                                          ("attributes", C.POINTER(NamedValue))],
    "PJRT_DeviceDescription_Kind": [("device_description", _vp), ("device_kind", _vp), ("device_kind_size", _sz)],
    "PJRT_DeviceDescription_DebugString": [("device_description", _vp), ("debug_string", _vp),
                                           ("debug_string_size", _sz)],
    "PJRT_DeviceDescription_ToString": [("device_description", _vp), ("to_string", _vp), ("to_string_size", _sz)],
    "PJRT_Device_GetDescription": [("device", _vp), ("device_description", _vp)],
    "PJRT_Device_IsAddressable": [("device", _vp), ("is_addressable", C.c_bool)],
    "PJRT_Device_LocalHardwareId": [("device", _vp), ("local_hardware_id", C.c_int)],
    "PJRT_Device_AddressableMemories": [("device", _vp), ("memories", C.POINTER(_vp)), ("num_memories", _sz)],
    "PJRT_Device_DefaultMemory": [("device", _vp), ("memory", _vp)],
    "PJRT_Memory_Id": [("memory", _vp), ("id", C.c_int)],
    "PJRT_Memory_Kind": [("memory", _vp), ("kind", _vp), ("kind_size", _sz)],
    "PJRT_Memory_Kind_Id": [("memory", _vp), ("kind_id", C.c_int)],
    "PJRT_Memory_ToString": [("memory", _vp), ("to_string", _vp), ("to_string_size", _sz)],
    "PJRT_Memory_AddressableByDevices": [("memory", _vp), ("devices", C.POINTER(_vp)), ("num_devices", _sz)],
    "PJRT_Executable_Destroy": [("executable", _vp)],
    "PJRT_Executable_Name": [("executable", _vp), ("executable_name", _vp), ("executable_name_size", _sz)],
    "PJRT_Executable_NumReplicas": [("executable", _vp), ("num_replicas", _sz)],
    "PJRT_Executable_NumPartitions": [("executable", _vp), ("num_partitions", _sz)],
    "PJRT_Executable_NumOutputs": [("executable", _vp), ("num_outputs", _sz)],
    "PJRT_Executable_GetCostAnalysis": [("executable", _vp), ("num_properties", _sz),
                                        ("properties", C.POINTER(NamedValue))],
    "PJRT_Executable_Fingerprint": [("executable", _vp), ("executable_fingerprint", _vp),
                                    ("executable_fingerprint_size", _sz)],
    "PJRT_Executable_OutputElementTypes": [("executable", _vp), ("output_types", C.POINTER(C.c_uint)),
                                           ("num_output_types", _sz)],
    "PJRT_Executable_OutputDimensions": [("executable", _vp), ("num_outputs", _sz), ("dims", C.POINTER(C.c_int64)),
                                         ("dim_sizes", C.POINTER(_sz))],
    "PJRT_Executable_GetCompileOptions": [("executable", _vp), ("serialized_bytes", _vp),
                                          ("serialized_bytes_size", _sz), ("serialized_compile_options", _vp),
                                          ("serialized_compile_options_deleter", C.CFUNCTYPE(None, _vp))],
    "PJRT_LoadedExecutable_Destroy": [("executable", _vp)],
    "PJRT_LoadedExecutable_GetExecutable": [("loaded_executable", _vp), ("executable", _vp)],
    "PJRT_LoadedExecutable_AddressableDevices": [("executable", _vp), ("addressable_devices", C.POINTER(_vp)),
                                                 ("num_addressable_devices", _sz)],
    "PJRT_LoadedExecutable_Execute": [("executable", _vp), ("options", C.POINTER(ExecuteOptions)),
                                      ("argument_lists", C.POINTER(C.POINTER(_vp))), ("num_devices", _sz),
                                      ("num_args", _sz), ("output_lists", C.POINTER(C.POINTER(_vp))),
                                      ("device_complete_events", C.POINTER(_vp)), ("execute_device", _vp)],
    "PJRT_Client_CreateUninitializedBuffer": [("client", _vp), ("shape_dims", C.POINTER(C.c_int64)),
                                              ("shape_num_dims", _sz), ("shape_element_type", C.c_uint),
                                              ("shape_layout", _vp), ("device", _vp), ("memory", _vp),
                                              ("buffer", _vp)],
    "PJRT_Client_CreateErrorBuffer": [("client", _vp), ("error_code", C.c_uint), ("error_message", _vp),
                                      ("error_message_size", _sz), ("shape_dims", C.POINTER(C.c_int64)),
                                      ("shape_num_dims", _sz), ("shape_element_type", C.c_uint),
                                      ("shape_layout", _vp), ("memory", _vp), ("buffer", _vp),
                                      ("payload", C.POINTER(NamedValue)), ("payload_size", _sz)],
    "PJRT_Device_PoisonExecution": [("device", _vp), ("launch_id", C.c_int32), ("error_code", C.c_uint),
                                    ("error_message", _vp), ("error_message_size", _sz), ("poisoned", C.c_bool),
                                    ("payload", C.POINTER(NamedValue)), ("payload_size", _sz)],
    "PJRT_Buffer_UnsafePointer": [("buffer", _vp), ("buffer_pointer", C.c_size_t)],
    "PJRT_Buffer_Destroy": [("buffer", _vp)],
    "PJRT_Buffer_ElementType": [("buffer", _vp), ("type", C.c_uint)],
    "PJRT_Buffer_Dimensions": [("buffer", _vp), ("dims", C.POINTER(C.c_int64)), ("num_dims", _sz)],
    "PJRT_Buffer_GetMemoryLayout": [("buffer", _vp), ("layout", MemoryLayout)],
    "PJRT_Buffer_OnDeviceSizeInBytes": [("buffer", _vp), ("on_device_size_in_bytes", _sz)],
    "PJRT_Buffer_Device": [("buffer", _vp), ("device", _vp)],
    "PJRT_Buffer_Memory": [("buffer", _vp), ("memory", _vp)],
    "PJRT_Buffer_Delete": [("buffer", _vp)],
    "PJRT_Buffer_IsDeleted": [("buffer", _vp), ("is_deleted", C.c_bool)],
    "PJRT_Buffer_ToHostBuffer": [("src", _vp), ("host_layout", _vp), ("dst", _vp), ("dst_size", _sz),
                                 ("event", _vp)],
    "PJRT_Buffer_IsOnCpu": [("buffer", _vp), ("is_on_cpu", C.c_bool)],
    "PJRT_Buffer_ReadyEvent": [("buffer", _vp), ("event", _vp)],
    "PJRT_Buffer_CopyToDevice": [("buffer", _vp), ("dst_device", _vp), ("dst_buffer", _vp)],
    "PJRT_Buffer_CopyRawToHost": [("buffer", _vp), ("dst", _vp), ("offset", C.c_int64), ("transfer_size", C.c_int64),
                                  ("event", _vp)],
    "PJRT_Executable_Serialize": [("executable", _vp), ("serialized_bytes", _vp), ("serialized_bytes_size", _sz),
                                  ("serialized_executable", _vp),
                                  ("serialized_executable_deleter", C.CFUNCTYPE(None, _vp))],
    "PJRT_Executable_DeserializeAndLoad": [("client", _vp), ("serialized_executable", _vp),
                                           ("serialized_executable_size", _sz), ("loaded_executable", _vp),
                                           ("overridden_serialized_compile_options", _vp),
                                           ("overridden_serialized_compile_options_size", _sz)],
    "PJRT_LoadedExecutable_GetDeviceAssignment": [("executable", _vp), ("serialized_bytes", _vp),
                                                  ("serialized_bytes_size", _sz),
                                                  ("serialized_device_assignment", _vp),
                                                  ("serialized_device_assignment_deleter", C.CFUNCTYPE(None, _vp))],
    "PJRT_Executable_GetCompiledMemoryStats": [("executable", _vp)] + [(f, C.c_int64) for f in (
        "generated_code_size_in_bytes", "argument_size_in_bytes", "output_size_in_bytes", "alias_size_in_bytes",
        "temp_size_in_bytes", "host_generated_code_size_in_bytes", "host_argument_size_in_bytes",
        "host_output_size_in_bytes", "host_alias_size_in_bytes", "host_temp_size_in_bytes", "peak_memory_in_bytes",
        "total_size_in_bytes", "total_allocation_bytes", "indefinite_allocations", "peak_unpadded_heap_bytes")],
    "PJRT_Executable_ParameterMemoryKinds": [("executable", _vp), ("num_parameters", _sz),
                                             ("memory_kinds", C.POINTER(_vp)), ("memory_kind_sizes", C.POINTER(_sz))],
    "PJRT_Executable_OutputMemoryKinds": [("executable", _vp), ("num_outputs", _sz),
                                          ("memory_kinds", C.POINTER(_vp)), ("memory_kind_sizes", C.POINTER(_sz))],
    "PJRT_ExecuteContext_Create": [("context", _vp)],
    "PJRT_ExecuteContext_Destroy": [("context", _vp)],
}.items():
    A[_n] = _args(_n + "_Args", _f)


def _slot_names() -> List[str]:
    """PJRT_Api slot order, read from the C header that the plugin is compiled against (lib.rs:214-364)."""
    with open(_HEADER) as f:
        text = f.read()
    body = text[text.index("typedef struct PJRT_Api {"):text.index("} PJRT_Api;")]
    return re.findall(r"PJRT_(?:NO)?SLOT\((PJRT_\w+)\)", body)


SLOTS = _slot_names()
_SLOT_OFFSET = {name: 40 + 8 * i for i, name in enumerate(SLOTS)}

RYFT_MI355X_EXTENSION_TYPE = 0x52594654


class _RyftExtension(C.Structure):
    _fields_ = [("base", ExtensionBase),
                ("set_kernel_timing", C.CFUNCTYPE(_vp, _vp, C.c_bool)),
                ("kernel_timing", C.CFUNCTYPE(_vp, _vp, C.POINTER(_vp), C.POINTER(_sz))),
                ("describe_plan", C.CFUNCTYPE(_vp, _vp, C.POINTER(_vp), C.POINTER(_sz)))]


PJRT_EXTENSION_TYPE_LAYOUTS = 4
_LAYOUT_ARGS = {
    "PJRT_Layouts_MemoryLayout_Destroy": [("layout", _vp)],
    "PJRT_Layouts_MemoryLayout_Serialize": [("layout", _vp), ("serialized_bytes", _vp), ("serialized_bytes_size", _sz),
                                            ("serialized_layout", _vp),
                                            ("serialized_layout_deleter", C.CFUNCTYPE(None, _vp))],
    "PJRT_Layouts_PJRT_Client_GetDefaultLayout": [("client", _vp), ("element_type", C.c_uint),
                                                  ("dims", C.POINTER(C.c_int64)), ("num_dims", _sz), ("layout", _vp)],
    "PJRT_Layouts_PJRT_Buffer_MemoryLayout": [("buffer", _vp), ("layout", _vp)],
    "PJRT_Layouts_PJRT_Executable_GetOutputLayouts": [("executable", _vp), ("num_outputs", _sz),
                                                      ("layouts", C.POINTER(_vp))],
    "PJRT_Layouts_PJRT_Executable_GetParameterLayouts": [("executable", _vp), ("num_parameters", _sz),
                                                         ("layouts", C.POINTER(_vp))],
}
for _n, _f in _LAYOUT_ARGS.items():
    A[_n] = _args(_n + "_Args", _f)
# the extension's function table after its PJRT_Extension_Base (extensions/layouts.rs:798-807)
_LAYOUT_SLOTS = ["PJRT_Layouts_MemoryLayout_Destroy", "PJRT_Layouts_MemoryLayout_Serialize",
                 "PJRT_Layouts_PJRT_Client_GetDefaultLayout", "PJRT_Layouts_PJRT_Buffer_MemoryLayout",
                 "PJRT_Layouts_PJRT_Topology_GetDefaultLayout", "PJRT_Layouts_PJRT_Executable_GetOutputLayouts",
                 "PJRT_Layouts_PJRT_Executable_GetParameterLayouts"]


# Wrappers that own a plugin object destroy it in __del__. At interpreter exit CPython clears module globals
# (this module's and ctypes') before it finalizes the objects still referenced from __main__, so those finalizers
# could no longer call into the plugin and clients would stay alive, with their streams, device memory and pinned
# host memory, into the HIP runtime's own exit-time teardown. Every owning wrapper is therefore tracked, and an
# exit hook destroys the live ones while the interpreter is intact: clients last, after everything they own.
_LIVE: "weakref.WeakValueDictionary" = weakref.WeakValueDictionary()  # id → wrapper (some define __eq__)


class _Owned:
    _exit_order = 0  # clients are destroyed after the objects that belong to them

    def __new__(cls, *args, **kwargs):
        obj = super().__new__(cls)
        _LIVE[id(obj)] = obj
        return obj


@atexit.register
def _destroy_live_objects():
    for obj in sorted(list(_LIVE.values()), key=lambda o: o._exit_order):
        obj.__del__()


class LayoutsExtension:
    """PJRT_Layouts_Extension (extensions/layouts.rs:20-60): calls go through its own function table."""

    def __init__(self, api: "Api", address: int):
        self.api, self.address = api, address
        self.struct_size = C.c_size_t.from_address(address).value

    def call(self, name: str, **kw):
        off = 24 + 8 * _LAYOUT_SLOTS.index(name)
        fp = C.c_void_p.from_address(self.address + off).value if self.struct_size >= off + 8 else None
        if not fp:
            raise PjrtError(ErrorCode.UNIMPLEMENTED, f"{name} is not implemented by the loaded plugin")
        args = self.api.new_args(name, **kw)
        err = self.api.error(C.CFUNCTYPE(_vp, _vp)(fp)(C.addressof(args)))
        if err is not None:
            raise err
        return args


class Layout(_Owned):
    """A PJRT memory layout (extensions/layouts.rs:95-195); borrowed ones belong to their executable."""

    def __init__(self, ext: LayoutsExtension, handle: int, borrowed: bool):
        if not handle:
            raise PjrtError(ErrorCode.INVALID_ARGUMENT, "the provided PJRT layout handle is a null pointer")
        self.ext, self.handle, self.borrowed = ext, handle, borrowed

    def serialize(self) -> str:
        a = self.ext.call("PJRT_Layouts_MemoryLayout_Serialize", layout=self.handle)
        text = _str(a.serialized_bytes, a.serialized_bytes_size)
        a.serialized_layout_deleter(a.serialized_layout)
        return text

    def __eq__(self, other) -> bool:
        return isinstance(other, Layout) and self.serialize() == other.serialize()

    def __repr__(self) -> str:
        return f"Layout[{self.serialize()}]"

    def __del__(self):
        try:
            if self.handle and not self.borrowed:
                self.ext.call("PJRT_Layouts_MemoryLayout_Destroy", layout=self.handle)
                self.handle = None
        except Exception:
            pass


PJRT_EXTENSION_TYPE_MEMORY_DESCRIPTIONS = 6
A["PJRT_DeviceDescription_MemoryDescriptions"] = _args(
    "PJRT_DeviceDescription_MemoryDescriptions_Args",
    [("device_description", _vp), ("memory_descriptions", C.POINTER(_vp)), ("num_memory_descriptions", _sz),
     ("default_memory_index", C.c_ssize_t)])
A["PJRT_MemoryDescription_Kind"] = _args(
    "PJRT_MemoryDescription_Kind_Args", [("memory_description", _vp), ("kind", _vp), ("kind_size", _sz),
                                         ("kind_id", C.c_int)])


def _ext_call(api: "Api", address: int, slots: List[str], name: str, **kw):
    """Call `name` through an extension's function table (the slots after its PJRT_Extension_Base)."""
    off = 24 + 8 * slots.index(name)
    fp = C.c_void_p.from_address(address + off).value if C.c_size_t.from_address(address).value >= off + 8 else None
    if not fp:
        raise PjrtError(ErrorCode.UNIMPLEMENTED, f"{name} is not implemented by the loaded plugin")
    args = api.new_args(name, **kw)
    err = api.error(C.CFUNCTYPE(_vp, _vp)(fp)(C.addressof(args)))
    if err is not None:
        raise err
    return args


def _str(ptr, size) -> str:
    if not ptr or size == 0:
        return ""
    return C.string_at(ptr, size).decode("utf-8", errors="replace")


# ----------------------------------------------------------------------------------------------- Api
class Api:
    """A PJRT_Api table; every call is gated on struct_size and null slots (macros.rs:27-108)."""

    def __init__(self, handle: int, lib: C.CDLL):
        if not handle:
            raise PjrtError(ErrorCode.INVALID_ARGUMENT, "the provided PJRT API handle is a null pointer")
        self.handle = handle
        self.lib = lib
        self.struct_size = C.c_size_t.from_address(handle).value
        ver = ApiVersion.from_address(handle + 16)
        self.version = (ver.major_version, ver.minor_version)
        self._fns: Dict[str, object] = {}

    def fn(self, name: str):
        f = self._fns.get(name)
        if f is not None:
            return f
        off = _SLOT_OFFSET[name]
        if self.struct_size <= off:
            raise PjrtError(ErrorCode.UNIMPLEMENTED,
                            f"`{name}` is not available in the loaded PJRT plugin (version {self.version})")
        addr = C.c_void_p.from_address(self.handle + off).value
        if not addr:
            raise PjrtError(ErrorCode.UNIMPLEMENTED, f"`{name}` is not implemented in the loaded PJRT plugin")
        if name in ("PJRT_Error_Destroy", "PJRT_Error_Message"):
            proto = C.CFUNCTYPE(None, C.POINTER(A[name]))
        else:
            proto = C.CFUNCTYPE(_vp, C.POINTER(A[name]))
        f = proto(addr)
        self._fns[name] = f
        return f

    def new_args(self, name: str, **kw):
        args = A[name]()
        args.struct_size = C.sizeof(args)
        for k, v in kw.items():
            setattr(args, k, v)
        return args

    def error(self, handle) -> Optional[PjrtError]:
        """Error::from_c_api: message, code, payload, then always destroy (errors.rs:76-180)."""
        if not handle:
            return None
        m = self.new_args("PJRT_Error_Message", error=handle)
        self.fn("PJRT_Error_Message")(C.byref(m))
        message = _str(m.message, m.message_size)
        c = self.new_args("PJRT_Error_GetCode", error=handle)
        err2 = self.fn("PJRT_Error_GetCode")(C.byref(c))
        payload: List[Tuple[str, str]] = []
        try:
            def visit(k, ks, v, vs, _):
                payload.append((_str(k, ks), _str(v, vs)))
            cb = PayloadVisitor(visit)
            p = self.new_args("PJRT_Error_ForEachPayload", error=handle, visitor=cb, user_arg=None)
            perr = self.fn("PJRT_Error_ForEachPayload")(C.byref(p))
            if perr:
                self.fn("PJRT_Error_Destroy")(C.byref(self.new_args("PJRT_Error_Destroy", error=perr)))
        except PjrtError:
            pass
        self.fn("PJRT_Error_Destroy")(C.byref(self.new_args("PJRT_Error_Destroy", error=handle)))
        code = ErrorCode(c.code) if not err2 else ErrorCode.UNKNOWN
        if code == ErrorCode.OK:
            return None
        return PjrtError(code, message, sorted(payload))

    def call(self, name: str, **kw):
        """Invoke `name` with the given inputs; returns the args struct (outputs are read from it)."""
        args = self.new_args(name, **kw)
        err = self.error(self.fn(name)(C.byref(args)))
        if err is not None:
            raise err
        return args

    def extension(self, ext_type: int):
        p = C.c_void_p.from_address(self.handle + 8).value
        while p:
            base = ExtensionBase.from_address(p)
            if base.extension_type == ext_type:
                return p
            p = C.cast(base.next, C.c_void_p).value
        return None

    def layouts_extension(self) -> LayoutsExtension:
        p = self.extension(PJRT_EXTENSION_TYPE_LAYOUTS)
        if not p:
            raise PjrtError(ErrorCode.UNIMPLEMENTED, "the loaded plugin has no layouts extension")
        return LayoutsExtension(self, p)

    def attributes(self) -> Dict[str, object]:
        a = self.call("PJRT_Plugin_Attributes")
        return _named_values(a.attributes, a.num_attributes)


def _named_value_array(items):
    """A PJRT_NamedValue array of (name, value) pairs (bool, int, float, int list, else string), and the Python
    objects that must outlive it (values.rs:146, NamedValue::to_c_api)."""
    items = list(items)
    keep = []
    vals = (NamedValue * max(len(items), 1))()
    for i, (k, v) in enumerate(items):
        nv = vals[i]
        nv.struct_size = C.sizeof(NamedValue)
        kb = k.encode()
        keep.append(kb)
        nv.name = C.cast(C.c_char_p(kb), _vp)
        nv.name_size = len(kb)
        if isinstance(v, bool):
            nv.type, nv.bool_value, nv.value_size = 4, v, 1
        elif isinstance(v, int):
            nv.type, nv.int64_value, nv.value_size = 1, v, 1
        elif isinstance(v, float):
            nv.type, nv.float_value, nv.value_size = 3, v, 1
        elif isinstance(v, (list, tuple)):
            arr = (C.c_int64 * len(v))(*v)
            keep.append(arr)
            nv.type, nv.int64_array_value, nv.value_size = 2, arr, len(v)
        else:
            sb = str(v).encode()
            keep.append(sb)
            nv.type, nv.string_value, nv.value_size = 0, C.cast(C.c_char_p(sb), _vp), len(sb)
    return vals, keep


def _named_values(ptr, n) -> Dict[str, object]:
    out: Dict[str, object] = {}
    for i in range(n):
        v = ptr[i]
        name = _str(v.name, v.name_size)
        if v.type == 0:
            out[name] = _str(v.string_value, v.value_size)
        elif v.type == 1:
            out[name] = int(v.int64_value)
        elif v.type == 2:
            out[name] = [int(v.int64_array_value[k]) for k in range(v.value_size)]
        elif v.type == 3:
            out[name] = float(v.float_value)
        else:
            out[name] = bool(v.bool_value)
    return out


# ----------------------------------------------------------------------------------------------- plugin
_PLUGINS: Dict[str, "Plugin"] = {}


class Plugin:
    """A loaded PJRT plugin (plugins.rs:14-44)."""

    def __init__(self, path: str):
        self.path = path
        self.lib = C.CDLL(path, mode=C.RTLD_LOCAL)
        get = self.lib.GetPjrtApi
        get.restype = C.c_void_p
        get.argtypes = []
        self._api = Api(get(), self.lib)
        self._initialized = False

    def api(self) -> Api:
        if not self._initialized:  # `Once` → PJRT_Plugin_Initialize (plugins.rs:22-28)
            self._api.call("PJRT_Plugin_Initialize")
            self._initialized = True
        return self._api

    def version(self) -> Tuple[int, int]:
        return self.api().version

    def attributes(self) -> Dict[str, object]:
        return self.api().attributes()

    def attribute(self, name: str):
        attrs = self.attributes()
        if name not in attrs:
            raise PjrtError(ErrorCode.NOT_FOUND, f"no attribute named '{name}' found in this PJRT plugin")
        return attrs[name]

    def client(self, options: Optional[Dict[str, object]] = None) -> "Client":
        return Client._create(self, options or {})

    def profiler_extension(self):
        """Plugin::profiler_extension (extensions/profiler.rs:103-125)."""
        from . import profiler
        return profiler.extension(self.api())

    def profiler(self, options=None):
        """Plugin::profiler (extensions/profiler.rs:127-145): a profiler session of this plugin."""
        from . import profiler
        return self.profiler_extension().profiler(options or profiler.ProfileOptions())


def load_plugin(path: str = DEFAULT_PLUGIN_PATH) -> Plugin:
    """Loads (once per canonical path) the plugin at `path` (plugins.rs:91-106, 120-122)."""
    if not os.path.exists(path):
        raise PjrtError(ErrorCode.NOT_FOUND, f"PJRT plugin not found at {path} (run __graft_entry__.build())")
    key = os.path.realpath(path)
    if key not in _PLUGINS:
        _PLUGINS[key] = Plugin(key)
    return _PLUGINS[key]


# ----------------------------------------------------------------------------------------------- devices
class Memory:
    def __init__(self, client: "Client", handle: int):
        self.client, self.handle = client, handle

    def id(self) -> int:
        return self.client.api.call("PJRT_Memory_Id", memory=self.handle).id

    def kind(self) -> str:
        a = self.client.api.call("PJRT_Memory_Kind", memory=self.handle)
        return _str(a.kind, a.kind_size)

    def kind_id(self) -> int:
        return self.client.api.call("PJRT_Memory_Kind_Id", memory=self.handle).kind_id

    def __str__(self) -> str:
        a = self.client.api.call("PJRT_Memory_ToString", memory=self.handle)
        return _str(a.to_string, a.to_string_size)


class Device:
    def __init__(self, client: "Client", handle: int):
        self.client, self.handle = client, handle

    def __eq__(self, other) -> bool:  # devices.rs:335-343 compares ids
        return isinstance(other, Device) and self.id() == other.id()

    def _desc(self) -> int:
        return self.client.api.call("PJRT_Device_GetDescription", device=self.handle).device_description

    def id(self) -> int:
        return self.client.api.call("PJRT_DeviceDescription_Id", device_description=self._desc()).id

    def kind(self) -> str:
        a = self.client.api.call("PJRT_DeviceDescription_Kind", device_description=self._desc())
        return _str(a.device_kind, a.device_kind_size)

    def attributes(self) -> Dict[str, object]:
        a = self.client.api.call("PJRT_DeviceDescription_Attributes", device_description=self._desc())
        return _named_values(a.attributes, a.num_attributes)

    def memory_descriptions(self):
        """DeviceDescription::memory_descriptions (extensions/memory_descriptions.rs:130-205): [(kind, kind_id)] and
        the index of the default one (None if the plugin names none)."""
        api = self.client.api
        p = api.extension(PJRT_EXTENSION_TYPE_MEMORY_DESCRIPTIONS)
        if not p:
            raise PjrtError(ErrorCode.UNIMPLEMENTED, "the loaded plugin has no memory descriptions extension")
        slots = ["PJRT_DeviceDescription_MemoryDescriptions", "PJRT_MemoryDescription_Kind"]
        a = _ext_call(api, p, slots, "PJRT_DeviceDescription_MemoryDescriptions", device_description=self._desc())
        out = []
        for i in range(a.num_memory_descriptions):
            k = _ext_call(api, p, slots, "PJRT_MemoryDescription_Kind", memory_description=a.memory_descriptions[i])
            out.append((_str(k.kind, k.kind_size), int(k.kind_id)))
        idx = a.default_memory_index
        return out, (idx if 0 <= idx < len(out) else None)

    def local_hardware_id(self) -> int:
        return self.client.api.call("PJRT_Device_LocalHardwareId", device=self.handle).local_hardware_id

    def is_addressable(self) -> bool:
        return self.client.api.call("PJRT_Device_IsAddressable", device=self.handle).is_addressable

    def default_memory(self) -> Memory:
        m = self.client.api.call("PJRT_Device_DefaultMemory", device=self.handle).memory
        if not m:
            raise PjrtError(ErrorCode.INTERNAL, "device has no default memory")
        return Memory(self.client, m)

    def addressable_memories(self) -> List[Memory]:
        a = self.client.api.call("PJRT_Device_AddressableMemories", device=self.handle)
        return [Memory(self.client, a.memories[i]) for i in range(a.num_memories)]

    def poison_execution(self, launch_id: int, error: PjrtError, payload: Optional[Dict[str, str]] = None) -> bool:
        """Device::poison_execution(_with_payload) (devices.rs:257-300): the earliest unfinished execution on this
        device under `launch_id` completes with `error` (its results become error buffers); False when it had
        already finished."""
        msg = error.message.encode()
        vals, keep = _named_value_array((payload or {}).items())
        a = self.client.api.call("PJRT_Device_PoisonExecution", device=self.handle, launch_id=int(launch_id),
                                 error_code=int(error.code), error_message=C.cast(C.c_char_p(msg), _vp),
                                 error_message_size=len(msg), payload=vals, payload_size=len(payload or {}))
        return bool(a.poisoned)


# ----------------------------------------------------------------------------------------------- events
class Event(_Owned):
    """PJRT_Event wrapper (events.rs); `await_` blocks, `on_ready` registers a callback."""

    def __init__(self, api: Api, handle: int, value=None):
        if not handle:
            raise PjrtError(ErrorCode.INVALID_ARGUMENT, "the provided PJRT event handle is a null pointer")
        self.api, self.handle, self._value = api, handle, value
        self._callbacks = []

    def is_ready(self) -> bool:
        return self.api.call("PJRT_Event_IsReady", event=self.handle).is_ready

    def await_(self):
        self.api.call("PJRT_Event_Await", event=self.handle)
        return self._value() if callable(self._value) else self._value

    def on_ready(self, fn: Callable[[Optional[PjrtError]], None]):
        def cb(err, _):
            fn(self.api.error(err))
        c = OnReadyCallback(cb)
        self._callbacks.append(c)  # kept alive with the event
        self.api.call("PJRT_Event_OnReady", event=self.handle, callback=c, user_arg=None)

    def __del__(self):
        try:
            if self.handle:
                self.api.call("PJRT_Event_Destroy", event=self.handle)
                self.handle = None
        except Exception:
            pass


# ----------------------------------------------------------------------------------------------- buffers
class Buffer(_Owned):
    def __init__(self, client: "Client", handle: int):
        if not handle:
            raise PjrtError(ErrorCode.INVALID_ARGUMENT, "the provided PJRT buffer handle is a null pointer")
        self.client, self.handle = client, handle

    @property
    def api(self) -> Api:
        return self.client.api

    def element_type(self) -> BufferType:
        return BufferType(self.api.call("PJRT_Buffer_ElementType", buffer=self.handle).type)

    def dimensions(self) -> List[int]:
        a = self.api.call("PJRT_Buffer_Dimensions", buffer=self.handle)
        return [int(a.dims[i]) for i in range(a.num_dims)]

    def on_device_size_in_bytes(self) -> int:
        return self.api.call("PJRT_Buffer_OnDeviceSizeInBytes", buffer=self.handle).on_device_size_in_bytes

    def device(self) -> Device:
        return Device(self.client, self.api.call("PJRT_Buffer_Device", buffer=self.handle).device)

    def memory(self) -> Memory:
        return Memory(self.client, self.api.call("PJRT_Buffer_Memory", buffer=self.handle).memory)

    def is_on_cpu(self) -> bool:
        return self.api.call("PJRT_Buffer_IsOnCpu", buffer=self.handle).is_on_cpu

    def is_deleted(self) -> bool:
        return self.api.call("PJRT_Buffer_IsDeleted", buffer=self.handle).is_deleted

    def delete(self):
        self.api.call("PJRT_Buffer_Delete", buffer=self.handle)

    def minor_to_major(self) -> List[int]:
        a = self.api.call("PJRT_Buffer_GetMemoryLayout", buffer=self.handle)
        t = a.layout.tiled
        return [int(t.minor_to_major[i]) for i in range(t.minor_to_major_size)]

    def ready_event(self) -> Event:
        return Event(self.api, self.api.call("PJRT_Buffer_ReadyEvent", buffer=self.handle).event)

    def memory_layout(self) -> Layout:
        ext = self.api.layouts_extension()
        return Layout(ext, ext.call("PJRT_Layouts_PJRT_Buffer_MemoryLayout", buffer=self.handle).layout, False)

    def unsafe_pointer(self) -> int:
        """Buffer::unsafe_pointer (buffers.rs:1500-1505): the device address of the buffer's bytes."""
        return int(self.api.call("PJRT_Buffer_UnsafePointer", buffer=self.handle).buffer_pointer)

    def copy_to_host(self) -> Event:
        """ToHostBuffer twice: size query with dst=null, then the copy (buffers.rs:1237-1266)."""
        size = self.api.call("PJRT_Buffer_ToHostBuffer", src=self.handle, dst=None).dst_size
        out = (C.c_uint8 * max(size, 1))()
        a = self.api.call("PJRT_Buffer_ToHostBuffer", src=self.handle, dst=C.cast(out, _vp), dst_size=size)
        return Event(self.api, a.event, lambda: C.string_at(out, size))

    def copy_raw_to_host(self, size: int, offset: int = 0) -> Event:
        """Buffer::copy_raw_to_host_buffer (buffers.rs:1318-1340): `size` bytes of the on-device bytes from `offset`;
        the event's value is those bytes."""
        out = (C.c_uint8 * max(size, 1))()
        a = self.api.call("PJRT_Buffer_CopyRawToHost", buffer=self.handle, dst=C.cast(out, _vp), offset=offset,
                          transfer_size=size)
        return Event(self.api, a.event, lambda: bytes(out)[:size])

    def copy_to_device(self, device: Device) -> "Buffer":
        a = self.api.call("PJRT_Buffer_CopyToDevice", buffer=self.handle, dst_device=device.handle)
        return Buffer(self.client, a.dst_buffer)

    def to_numpy(self):
        """Copy to host and view as numpy (bf16 / f8 come back as raw uint16 / uint8 bits)."""
        import numpy as np
        t = self.element_type()
        np_t = {BufferType.PRED: np.bool_, BufferType.S8: np.int8, BufferType.S16: np.int16, BufferType.S32: np.int32,
                BufferType.S64: np.int64, BufferType.U8: np.uint8, BufferType.U16: np.uint16,
                BufferType.U32: np.uint32, BufferType.U64: np.uint64, BufferType.F16: np.float16,
                BufferType.F32: np.float32, BufferType.F64: np.float64, BufferType.BF16: np.uint16,
                BufferType.F8E4M3FN: np.uint8, BufferType.F8E5M2: np.uint8}[t]
        # the device bytes land directly in the array (ToHostBuffer: size query, then the copy)
        dims = self.dimensions()
        size = self.api.call("PJRT_Buffer_ToHostBuffer", src=self.handle, dst=None).dst_size
        out = np.empty(dims, dtype=np_t)
        if out.nbytes != size:
            raise PjrtError(ErrorCode.INTERNAL, f"buffer holds {size} bytes, its shape {out.nbytes}")
        if size:
            a = self.api.call("PJRT_Buffer_ToHostBuffer", src=self.handle, dst=C.c_void_p(out.ctypes.data),
                              dst_size=size)
            Event(self.api, a.event).await_()
        return out

    def __del__(self):
        try:
            if self.handle:
                self.api.call("PJRT_Buffer_Destroy", buffer=self.handle)
                self.handle = None
        except Exception:
            pass


# ----------------------------------------------------------------------------------------------- programs
@dataclass
class Program:
    """Program::Mlir (programs.rs:19-63). `code` is MLIR text or bytecode."""

    code: bytes
    format: str = "mlir"

    @staticmethod
    def mlir(code) -> "Program":
        return Program(code.encode() if isinstance(code, str) else bytes(code), "mlir")


def _varint(n: int) -> bytes:
    n &= (1 << 64) - 1
    out = bytearray()
    while True:
        b = n & 0x7F
        n >>= 7
        if n:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


@dataclass
class CompilationOptions:
    """The CompileOptionsProto fields the README example sets (README.md:93-106; protos.rs:2391-2504, 3298-3346)."""

    device_ordinal: int = -1
    replica_count: int = 1
    partition_count: int = 1
    matrix_unit_operand_precision: int = 0

    def encode(self) -> bytes:
        ebo = (b"\x08" + _varint(self.device_ordinal) + b"\x20" + _varint(self.replica_count) + b"\x28" +
               _varint(self.partition_count))
        out = b"\x1a" + _varint(len(ebo)) + ebo
        if self.matrix_unit_operand_precision:
            out += b"\x50" + _varint(self.matrix_unit_operand_precision)
        return out


def _read_varint(data: bytes, pos: int):
    n, shift = 0, 0
    while True:
        if pos >= len(data):
            raise PjrtError(ErrorCode.INVALID_ARGUMENT, "truncated varint")
        b = data[pos]
        pos += 1
        n |= (b & 0x7F) << shift
        shift += 7
        if not b & 0x80:
            return n, pos


def _proto_fields(data: bytes):
    """(field number, wire type, value) of a protobuf message (varint and length-delimited fields)."""
    pos, out = 0, []
    while pos < len(data):
        key, pos = _read_varint(data, pos)
        num, wt = key >> 3, key & 7
        if wt == 0:
            v, pos = _read_varint(data, pos)
        elif wt == 2:
            n, pos = _read_varint(data, pos)
            v, pos = data[pos:pos + n], pos + n
        else:
            raise PjrtError(ErrorCode.INVALID_ARGUMENT, f"unsupported protobuf wire type {wt}")
        out.append((num, wt, v))
    return out


@dataclass
class DeviceAssignment:
    """devices.rs:517-540: `assignment[replica * computation_count + computation]` = device id."""

    replica_count: int
    computation_count: int
    assignment: List[int]

    @staticmethod
    def decode(data: bytes) -> "DeviceAssignment":
        """xla.DeviceAssignmentProto (ryft-xla-sys/src/protos.rs:2318-2352), read as devices.rs:674-688 does."""
        replicas = computations = 0
        columns: List[List[int]] = []
        for num, wt, v in _proto_fields(data):
            if num == 1 and wt == 0:
                replicas = v
            elif num == 2 and wt == 0:
                computations = v
            elif num == 3 and wt == 2:
                ids: List[int] = []
                for n2, w2, v2 in _proto_fields(v):
                    if n2 == 1 and w2 == 2:  # packed int64
                        pos = 0
                        while pos < len(v2):
                            x, pos = _read_varint(v2, pos)
                            ids.append(x - (1 << 64) if x >> 63 else x)
                    elif n2 == 1 and w2 == 0:
                        ids.append(v2)
                columns.append(ids)
        out = []
        for r in range(replicas):
            for c in range(computations):
                if c >= len(columns) or r >= len(columns[c]):
                    raise PjrtError(ErrorCode.INVALID_ARGUMENT, "invalid device assignment")
                out.append(columns[c][r])
        return DeviceAssignment(replicas, computations, out)


class ExecutionContext(_Owned):
    """PJRT_ExecuteContext (programs.rs:1190-1235)."""

    def __init__(self, api: Api, handle: int):
        if not handle:
            raise PjrtError(ErrorCode.INVALID_ARGUMENT, "the provided PJRT execute context handle is a null pointer")
        self.api, self.handle = api, handle

    def __del__(self):
        try:
            if self.handle:
                self.api.call("PJRT_ExecuteContext_Destroy", context=self.handle)
                self.handle = None
        except Exception:
            pass


class Executable(_Owned):
    def __init__(self, api: Api, handle: int):
        self.api, self.handle = api, handle

    def name(self) -> str:
        a = self.api.call("PJRT_Executable_Name", executable=self.handle)
        return _str(a.executable_name, a.executable_name_size)

    def output_count(self) -> int:
        return self.api.call("PJRT_Executable_NumOutputs", executable=self.handle).num_outputs

    def replica_count(self) -> int:
        return self.api.call("PJRT_Executable_NumReplicas", executable=self.handle).num_replicas

    def computation_count(self) -> int:
        return self.api.call("PJRT_Executable_NumPartitions", executable=self.handle).num_partitions

    def output_element_types(self) -> List[BufferType]:
        a = self.api.call("PJRT_Executable_OutputElementTypes", executable=self.handle)
        return [BufferType(a.output_types[i]) for i in range(a.num_output_types)]

    def output_dimensions(self) -> List[List[int]]:
        a = self.api.call("PJRT_Executable_OutputDimensions", executable=self.handle)
        out, off = [], 0
        for i in range(a.num_outputs):
            r = a.dim_sizes[i]
            out.append([int(a.dims[off + k]) for k in range(r)])
            off += r
        return out

    def fingerprint(self) -> str:
        a = self.api.call("PJRT_Executable_Fingerprint", executable=self.handle)
        return _str(a.executable_fingerprint, a.executable_fingerprint_size)

    def cost_analysis(self) -> Dict[str, object]:
        a = self.api.call("PJRT_Executable_GetCostAnalysis", executable=self.handle)
        return _named_values(a.properties, a.num_properties)

    def compile_options(self) -> bytes:
        a = self.api.call("PJRT_Executable_GetCompileOptions", executable=self.handle)
        data = C.string_at(a.serialized_bytes, a.serialized_bytes_size)
        a.serialized_compile_options_deleter(a.serialized_compile_options)
        return data

    def serialize(self) -> bytes:
        """Executable::serialize (programs.rs:404-423): the plugin's bytes for this executable."""
        a = self.api.call("PJRT_Executable_Serialize", executable=self.handle)
        data = C.string_at(a.serialized_bytes, a.serialized_bytes_size)
        a.serialized_executable_deleter(a.serialized_executable)
        return data

    def input_layouts(self) -> List[Layout]:
        """Executable::input_layouts (extensions/layouts.rs:245-263): borrowed from the executable."""
        ext = self.api.layouts_extension()
        a = ext.call("PJRT_Layouts_PJRT_Executable_GetParameterLayouts", executable=self.handle)
        return [Layout(ext, a.layouts[i], True) for i in range(a.num_parameters)]

    def output_layouts(self) -> List[Layout]:
        ext = self.api.layouts_extension()
        a = ext.call("PJRT_Layouts_PJRT_Executable_GetOutputLayouts", executable=self.handle)
        return [Layout(ext, a.layouts[i], True) for i in range(a.num_outputs)]

    def memory_statistics(self) -> Dict[str, int]:
        """Executable::memory_statistics (programs.rs:318-360)."""
        a = self.api.call("PJRT_Executable_GetCompiledMemoryStats", executable=self.handle)
        return {name: int(getattr(a, name)) for name, _ in a._fields_[3:]}

    def input_memory_kinds(self) -> List[str]:
        a = self.api.call("PJRT_Executable_ParameterMemoryKinds", executable=self.handle)
        return [_str(a.memory_kinds[i], a.memory_kind_sizes[i]) for i in range(a.num_parameters)]

    def output_memory_kinds(self) -> List[str]:
        a = self.api.call("PJRT_Executable_OutputMemoryKinds", executable=self.handle)
        return [_str(a.memory_kinds[i], a.memory_kind_sizes[i]) for i in range(a.num_outputs)]

    def __del__(self):
        try:
            if self.handle:
                self.api.call("PJRT_Executable_Destroy", executable=self.handle)
                self.handle = None
        except Exception:
            pass


@dataclass
class ExecutionInput:
    buffer: Buffer
    donatable: bool = False


@dataclass
class ExecutionDeviceOutputs:
    outputs: List[Buffer]
    done: Event


class LoadedExecutable(_Owned):
    def __init__(self, client: "Client", handle: int):
        if not handle:
            raise PjrtError(ErrorCode.INVALID_ARGUMENT, "the provided PJRT loaded executable handle is a null pointer")
        self.client, self.handle = client, handle

    @property
    def api(self) -> Api:
        return self.client.api

    def addressable_devices(self) -> List[Device]:
        a = self.api.call("PJRT_LoadedExecutable_AddressableDevices", executable=self.handle)
        return [Device(self.client, a.addressable_devices[i]) for i in range(a.num_addressable_devices)]

    def executable(self) -> Executable:
        a = self.api.call("PJRT_LoadedExecutable_GetExecutable", loaded_executable=self.handle)
        return Executable(self.api, a.executable)

    def device_assignment(self) -> DeviceAssignment:
        """LoadedExecutable::device_assignment (programs.rs:704-736; decoding as devices.rs:674-688)."""
        a = self.api.call("PJRT_LoadedExecutable_GetDeviceAssignment", executable=self.handle)
        data = C.string_at(a.serialized_bytes, a.serialized_bytes_size)
        a.serialized_device_assignment_deleter(a.serialized_device_assignment)
        return DeviceAssignment.decode(data)

    def execute(self, inputs: Sequence[Sequence], launch_id: int = 0) -> List[ExecutionDeviceOutputs]:
        """LoadedExecutable::execute (programs.rs:769-963): one input list per addressable device."""
        counts = self.__dict__.get("_counts")
        if counts is None:  # fixed for a loaded executable: queried once, not on every execution
            counts = self._counts = (len(self.addressable_devices()), self.executable().output_count())
        device_count, output_count = counts
        # Repeated executions on the same plain (non-donated) buffers of one device reuse a prepared argument block
        # (per thread: the call releases the GIL, and its output arrays are written during it).
        if device_count == 1 and len(inputs) == 1 and all(type(x) is Buffer for x in inputs[0]):
            local = self.__dict__.get("_local")
            if local is None:
                local = self._local = threading.local()
            prepared = getattr(local, "prepared", None)
            if prepared is None:
                prepared = local.prepared = {}
            key = (tuple(x.handle for x in inputs[0]), launch_id)
            prep = prepared.get(key)
            if prep is None:
                if len(prepared) >= 32:
                    prepared.clear()
                prep = prepared[key] = self._prepare(inputs[0], launch_id, output_count)
            args, ref, outs, events, fn = prep
            err = fn(ref)
            if err:
                raise self.api.error(err)
            return [ExecutionDeviceOutputs([Buffer(self.client, outs[o]) for o in range(output_count)],
                                           Event(self.api, events[0]))]
        if len(inputs) != device_count:
            raise PjrtError(ErrorCode.INVALID_ARGUMENT,
                            f"expected inputs for {device_count} device(s) but got inputs for {len(inputs)} device(s)")
        norm = [[i if isinstance(i, ExecutionInput) else ExecutionInput(i) for i in dev] for dev in inputs]
        input_count = len(norm[0]) if norm else 0
        for d, dev in enumerate(norm):
            if len(dev) != input_count:
                raise PjrtError(ErrorCode.INVALID_ARGUMENT,
                                f"expected {input_count} input(s) for each device but got {len(dev)} for device {d}")
        donatable = tuple(x.donatable for x in norm[0]) if norm else ()
        for d, dev in enumerate(norm):
            for i, x in enumerate(dev):
                if x.donatable != donatable[i]:
                    raise PjrtError(ErrorCode.INVALID_ARGUMENT, f"input {i} is not marked consistently across all "
                                                                "devices as donatable or non-donatable")
        # the options depend only on which inputs are donatable and the launch id: built once each
        key = (donatable, launch_id)
        cached = self.__dict__.setdefault("_options", {}).get(key)
        if cached is None:
            keep = [i for i, dn in enumerate(donatable) if not dn]
            nd = (C.c_int64 * max(len(keep), 1))(*keep)
            opts = ExecuteOptions()
            opts.struct_size = C.sizeof(opts)
            opts.launch_id = launch_id
            opts.non_donatable_input_indices = nd
            opts.num_non_donatable_input_indices = len(keep)
            cached = self._options[key] = (nd, opts, C.pointer(opts))
        opts_ptr = cached[2]
        arg_arrays = [(_vp * max(input_count, 1))(*[x.buffer.handle for x in dev]) for dev in norm]
        arg_lists = (C.POINTER(_vp) * device_count)(*[C.cast(a, C.POINTER(_vp)) for a in arg_arrays])
        out_arrays = [(_vp * max(output_count, 1))() for _ in range(device_count)]
        out_lists = (C.POINTER(_vp) * device_count)(*[C.cast(a, C.POINTER(_vp)) for a in out_arrays])
        events = (_vp * device_count)()
        self.api.call("PJRT_LoadedExecutable_Execute", executable=self.handle, options=opts_ptr,
                      argument_lists=arg_lists, num_devices=device_count, num_args=input_count,
                      output_lists=out_lists, device_complete_events=events, execute_device=None)
        results = []
        for d in range(device_count):
            done = Event(self.api, events[d])
            outs = [Buffer(self.client, out_arrays[d][o]) for o in range(output_count)]
            results.append(ExecutionDeviceOutputs(outs, done))
        return results

    def _prepare(self, buffers, launch_id: int, output_count: int):
        """The argument block of an execution on `buffers` (one device, every input non-donatable)."""
        n = len(buffers)
        nd = (C.c_int64 * max(n, 1))(*range(n))
        opts = ExecuteOptions()
        opts.struct_size = C.sizeof(opts)
        opts.launch_id = launch_id
        opts.non_donatable_input_indices = nd
        opts.num_non_donatable_input_indices = n
        arr = (_vp * max(n, 1))(*[b.handle for b in buffers])
        lists = (C.POINTER(_vp) * 1)(C.cast(arr, C.POINTER(_vp)))
        outs = (_vp * max(output_count, 1))()
        olists = (C.POINTER(_vp) * 1)(C.cast(outs, C.POINTER(_vp)))
        events = (_vp * 1)()
        args = self.api.new_args("PJRT_LoadedExecutable_Execute", executable=self.handle, options=C.pointer(opts),
                                 argument_lists=lists, num_devices=1, num_args=n, output_lists=olists,
                                 device_complete_events=events, execute_device=None)
        args._keep = (nd, opts, arr, lists, olists)  # the arrays the block points into
        return args, C.byref(args), outs, events, self.api.fn("PJRT_LoadedExecutable_Execute")

    def describe_plan(self) -> str:
        ext = self.client._ext()
        p, n = C.c_void_p(), C.c_size_t()
        err = self.api.error(ext.describe_plan(self.handle, C.byref(p), C.byref(n)))
        if err:
            raise err
        return _str(p.value, n.value)

    def __del__(self):
        try:
            if self.handle:
                self.api.call("PJRT_LoadedExecutable_Destroy", executable=self.handle)
                self.handle = None
        except Exception:
            pass


# ----------------------------------------------------------------------------------------------- client
class Client(_Owned):
    _exit_order = 1

    def __init__(self, plugin: Plugin, handle: int):
        if not handle:
            raise PjrtError(ErrorCode.INVALID_ARGUMENT, "the provided PJRT client handle is a null pointer")
        self.plugin, self.handle = plugin, handle
        self.api = plugin.api()

    @staticmethod
    def _create(plugin: Plugin, options: Dict[str, object]) -> "Client":
        api = plugin.api()
        vals, keep = _named_value_array(options.items())
        a = api.call("PJRT_Client_Create", create_options=vals, num_options=len(options))
        return Client(plugin, a.client)

    def profiler_extension(self):
        """Client::profiler_extension (extensions/profiler.rs:26-60)."""
        return self.plugin.profiler_extension()

    def profiler(self, options=None):
        """Client::profiler (extensions/profiler.rs:62-80): a profiler session; it records the work of every client
        of the plugin while started."""
        return self.plugin.profiler(options)

    def platform_name(self) -> str:
        a = self.api.call("PJRT_Client_PlatformName", client=self.handle)
        return _str(a.platform_name, a.platform_name_size)

    def platform_version(self) -> str:
        a = self.api.call("PJRT_Client_PlatformVersion", client=self.handle)
        return _str(a.platform_version, a.platform_version_size)

    def process_index(self) -> int:
        return self.api.call("PJRT_Client_ProcessIndex", client=self.handle).process_index

    def attributes(self) -> Dict[str, object]:
        return self.api.attributes()

    def devices(self) -> List[Device]:
        a = self.api.call("PJRT_Client_Devices", client=self.handle)
        return [Device(self, a.devices[i]) for i in range(a.num_devices)]

    def addressable_devices(self) -> List[Device]:
        a = self.api.call("PJRT_Client_AddressableDevices", client=self.handle)
        return [Device(self, a.addressable_devices[i]) for i in range(a.num_addressable_devices)]

    def lookup_device(self, id: int) -> Device:
        return Device(self, self.api.call("PJRT_Client_LookupDevice", client=self.handle, id=id).device)

    def lookup_addressable_device(self, local_hardware_id: int) -> Device:
        a = self.api.call("PJRT_Client_LookupAddressableDevice", client=self.handle,
                          local_hardware_id=local_hardware_id)
        return Device(self, a.addressable_device)

    def addressable_memories(self) -> List[Memory]:
        a = self.api.call("PJRT_Client_AddressableMemories", client=self.handle)
        return [Memory(self, a.addressable_memories[i]) for i in range(a.num_addressable_memories)]

    def default_device_assignment(self, replicas: int, partitions: int) -> List[int]:
        n = replicas * partitions
        arr = (C.c_int * max(n, 1))()
        self.api.call("PJRT_Client_DefaultDeviceAssignment", client=self.handle, num_replicas=replicas,
                      num_partitions=partitions, default_assignment_size=n, default_assignment=arr)
        return list(arr)[:n]

    def compile(self, program: Program, options=None) -> LoadedExecutable:
        """Client::compile (programs.rs:1245-1263). `options`: CompilationOptions, or already-serialized
        CompileOptionsProto bytes."""
        opts = bytes(options) if isinstance(options, (bytes, bytearray)) else (options or CompilationOptions()).encode()
        code = C.create_string_buffer(program.code, len(program.code))
        fmt = C.create_string_buffer(program.format.encode(), len(program.format))
        p = Program_()
        p.struct_size = C.sizeof(p)
        p.code = C.cast(code, _vp)
        p.code_size = len(program.code)
        p.format = C.cast(fmt, _vp)
        p.format_size = len(program.format)
        ob = C.create_string_buffer(opts, len(opts))
        a = self.api.call("PJRT_Client_Compile", client=self.handle, program=C.pointer(p),
                          compile_options=C.cast(ob, _vp), compile_options_size=len(opts))
        return LoadedExecutable(self, a.executable)

    def deserialize_and_load_executable(self, data: bytes, options: Optional[CompilationOptions] = None
                                        ) -> LoadedExecutable:
        """Client::deserialize_and_load_executable (programs.rs:1303-1330)."""
        blob = C.create_string_buffer(bytes(data), len(data))
        opts = options.encode() if options is not None else b""
        ob = C.create_string_buffer(opts, max(len(opts), 1))
        a = self.api.call("PJRT_Executable_DeserializeAndLoad", client=self.handle, serialized_executable=C.cast(blob, _vp),
                          serialized_executable_size=len(data),
                          overridden_serialized_compile_options=C.cast(ob, _vp) if opts else None,
                          overridden_serialized_compile_options_size=len(opts))
        return LoadedExecutable(self, a.loaded_executable)

    def default_layout(self, element_type: BufferType, dims: Sequence[int]) -> Layout:
        """Client::default_layout (extensions/layouts.rs:198-217)."""
        ext = self.api.layouts_extension()
        d = (C.c_int64 * max(len(dims), 1))(*dims)
        a = ext.call("PJRT_Layouts_PJRT_Client_GetDefaultLayout", client=self.handle, element_type=int(element_type),
                     dims=d, num_dims=len(dims))
        return Layout(ext, a.layout, False)

    def execution_context(self) -> "ExecutionContext":
        return ExecutionContext(self.api, self.api.call("PJRT_ExecuteContext_Create").context)

    def buffer(self, data, element_type: BufferType, dims: Sequence[int], byte_strides: Optional[Sequence[int]] = None,
               device: Optional[Device] = None, memory: Optional[Memory] = None) -> Buffer:
        """Client::buffer (buffers.rs:2099-2150): host bytes → device buffer in the device's default memory."""
        if device is None:
            device = self.addressable_devices()[0]
        if memory is None:
            memory = device.default_memory()
        expected = int(BufferType(element_type).size)
        for d in dims:
            expected *= int(d)
        # a C-contiguous array is handed over in place (the plugin copies the bytes before the call returns);
        # anything else is copied into a contiguous block first
        if hasattr(data, "ctypes") and hasattr(data, "flags") and data.flags["C_CONTIGUOUS"]:
            keep, nbytes, ptr = data, int(data.nbytes), data.ctypes.data
        else:
            raw = data.tobytes() if hasattr(data, "tobytes") else bytes(data)
            keep = C.create_string_buffer(raw, max(len(raw), 1))
            nbytes, ptr = len(raw), C.addressof(keep)
        if byte_strides is None and nbytes != expected:
            raise PjrtError(ErrorCode.INVALID_ARGUMENT, f"expected {expected} bytes of host data, got {nbytes}")
        if not nbytes:  # (no bytes are read, but the pointer must not be null)
            keep = C.create_string_buffer(1)
            ptr = C.addressof(keep)
        src = C.c_void_p(ptr)
        dims_arr = (C.c_int64 * max(len(dims), 1))(*dims)
        kw = {}
        if byte_strides is not None:
            kw["byte_strides"] = (C.c_int64 * len(byte_strides))(*byte_strides)
            kw["num_byte_strides"] = len(byte_strides)
        a = self.api.call("PJRT_Client_BufferFromHostBuffer", client=self.handle, data=src,
                          type=int(element_type), dims=dims_arr, num_dims=len(dims), host_buffer_semantics=0,
                          device=None, memory=memory.handle, device_layout=None, **kw)
        del keep
        if a.done_with_host_buffer:
            Event(self.api, a.done_with_host_buffer)  # dropped, as ryft-pjrt does
        return Buffer(self, a.buffer)

    def uninitialized_buffer(self, element_type: BufferType, dims: Sequence[int],
                             memory: Optional[Memory] = None) -> Buffer:
        """Client::uninitialized_buffer (buffers.rs:2229-2252): a device buffer of the given type and dimensions whose
        bytes are unspecified, placed in `memory` (default: the first device's default memory); device = null."""
        if memory is None:
            memory = self.addressable_devices()[0].default_memory()
        dims_arr = (C.c_int64 * max(len(dims), 1))(*dims)
        a = self.api.call("PJRT_Client_CreateUninitializedBuffer", client=self.handle, shape_dims=dims_arr,
                          shape_num_dims=len(dims), shape_element_type=int(element_type), shape_layout=None,
                          device=None, memory=memory.handle)
        return Buffer(self, a.buffer)

    def error_buffer(self, error: PjrtError, element_type: BufferType, dims: Sequence[int],
                     memory: Optional[Memory] = None, payload: Optional[Dict[str, str]] = None) -> Buffer:
        """Client::error_buffer(_with_payload) (buffers.rs:2321-2392): a buffer of the given type and dimensions that
        holds `error` instead of data; its ready event, copies to host and executions that take it fail with it."""
        if memory is None:
            memory = self.addressable_devices()[0].default_memory()
        dims_arr = (C.c_int64 * max(len(dims), 1))(*dims)
        msg = error.message.encode()
        vals, keep = _named_value_array((payload or {}).items())
        a = self.api.call("PJRT_Client_CreateErrorBuffer", client=self.handle, error_code=int(error.code),
                          error_message=C.cast(C.c_char_p(msg), _vp), error_message_size=len(msg),
                          shape_dims=dims_arr, shape_num_dims=len(dims), shape_element_type=int(element_type),
                          shape_layout=None, memory=memory.handle, payload=vals, payload_size=len(payload or {}))
        return Buffer(self, a.buffer)

    # --- plugin extension: kernel timing on the device stream
    def _ext(self) -> _RyftExtension:
        p = self.api.extension(RYFT_MI355X_EXTENSION_TYPE)
        if not p:
            raise PjrtError(ErrorCode.UNIMPLEMENTED, "the loaded plugin has no ryft MI355X extension")
        return _RyftExtension.from_address(p)

    def set_kernel_timing(self, enable: bool):
        err = self.api.error(self._ext().set_kernel_timing(self.handle, bool(enable)))
        if err:
            raise err

    def kernel_timing(self) -> Dict[str, Dict[str, float]]:
        import json
        p, n = C.c_void_p(), C.c_size_t()
        err = self.api.error(self._ext().kernel_timing(self.handle, C.byref(p), C.byref(n)))
        if err:
            raise err
        return json.loads(_str(p.value, n.value))

    def __del__(self):
        try:
            if self.handle:
                self.api.call("PJRT_Client_Destroy", client=self.handle)
                self.handle = None
        except Exception:
            pass
