"""The PJRT profiler extension (crates/ryft-pjrt/src/extensions/profiler.rs:26-330) over ctypes.

A `Profiler` is created from a `Client` or `Plugin` with `ProfileOptions`, started, stopped, and its results read as
an `XSpace` (crates/ryft-xla-sys/src/protos.rs:3574-3810), decoded here into plain Python objects: planes of lines of
events, each event with its name (from the plane's event metadata), offset and duration in picoseconds and its stats
by name.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
from typing import Dict, List, Optional, Tuple

from . import pjrt as P

PJRT_EXTENSION_TYPE_PROFILER = 1
_sz, _vp = C.c_size_t, C.c_void_p


class _ErrorMessageArgs(C.Structure):
    _fields_ = [("struct_size", _sz), ("state", _vp), ("error", _vp), ("message", _vp), ("message_size", _sz)]


class _ErrorGetCodeArgs(C.Structure):
    _fields_ = [("struct_size", _sz), ("state", _vp), ("error", _vp), ("code", C.c_int)]


class _ErrorDestroyArgs(C.Structure):
    _fields_ = [("struct_size", _sz), ("state", _vp), ("error", _vp)]


class _CreateArgs(C.Structure):
    _fields_ = [("struct_size", _sz), ("options", _vp), ("options_size", _sz), ("profiler", _vp)]


class _HandleArgs(C.Structure):  # Destroy / Start / Stop
    _fields_ = [("struct_size", _sz), ("profiler", _vp)]


class _CollectDataArgs(C.Structure):
    _fields_ = [("struct_size", _sz), ("profiler", _vp), ("buffer", _vp), ("buffer_size_in_bytes", _sz)]


_API_SLOTS = ["PLUGIN_Profiler_Error_Destroy", "PLUGIN_Profiler_Error_Message", "PLUGIN_Profiler_Error_GetCode",
              "PLUGIN_Profiler_Create", "PLUGIN_Profiler_Destroy", "PLUGIN_Profiler_Start", "PLUGIN_Profiler_Stop",
              "PLUGIN_Profiler_CollectData"]
_ARGS = {"PLUGIN_Profiler_Error_Destroy": _ErrorDestroyArgs, "PLUGIN_Profiler_Error_Message": _ErrorMessageArgs,
         "PLUGIN_Profiler_Error_GetCode": _ErrorGetCodeArgs, "PLUGIN_Profiler_Create": _CreateArgs,
         "PLUGIN_Profiler_Destroy": _HandleArgs, "PLUGIN_Profiler_Start": _HandleArgs,
         "PLUGIN_Profiler_Stop": _HandleArgs, "PLUGIN_Profiler_CollectData": _CollectDataArgs}


# ----------------------------------------------------------------------------------------------- protobuf
def _varint(v: int) -> bytes:
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        out.append(b | (0x80 if v else 0))
        if not v:
            return bytes(out)


@dataclasses.dataclass
class ProfileOptions:
    """tensorflow.ProfileOptions (protos.rs:3423-3490); the fields a PJRT profiler reads. Version 0 asks for the
    default session (host tracing level 2, device tracing level 1)."""
    version: int = 1
    device_type: int = 0  # ProfileDeviceType: 0 unspecified, 1 CPU, 2 GPU, 3 TPU, 4 pluggable device
    include_dataset_operations: bool = False
    host_tracing_level: int = 2
    device_tracing_level: int = 1
    python_tracing_level: int = 0
    enable_hlo_proto: bool = False
    start_timestamp_ns: int = 0
    duration_ms: int = 0
    repository_path: str = ""

    def encode(self) -> bytes:
        out = bytearray()
        for field, value in ((1, int(self.include_dataset_operations)), (2, self.host_tracing_level),
                             (3, self.device_tracing_level), (4, self.python_tracing_level), (5, self.version),
                             (6, self.device_type), (7, int(self.enable_hlo_proto)), (8, self.start_timestamp_ns),
                             (9, self.duration_ms)):
            if value:
                out += _varint(field << 3) + _varint(value)
        if self.repository_path:
            b = self.repository_path.encode()
            out += _varint((10 << 3) | 2) + _varint(len(b)) + b
        return bytes(out)


def _fields(buf: bytes):
    """(field, wire type, value) of one message; length-delimited values are bytes, fixed64 values raw bytes."""
    i, n = 0, len(buf)

    def varint():
        nonlocal i
        v, shift = 0, 0
        while True:
            if i >= n:
                raise ValueError("truncated varint")
            b = buf[i]
            i += 1
            v |= (b & 0x7F) << shift
            if not b & 0x80:
                return v
            shift += 7

    while i < n:
        key = varint()
        field, wire = key >> 3, key & 7
        if wire == 0:
            yield field, wire, varint()
        elif wire == 1:
            yield field, wire, buf[i:i + 8]
            i += 8
        elif wire == 2:
            ln = varint()
            yield field, wire, buf[i:i + ln]
            i += ln
        elif wire == 5:
            yield field, wire, buf[i:i + 4]
            i += 4
        else:
            raise ValueError(f"wire type {wire}")


def _signed(v: int) -> int:
    return v - (1 << 64) if v >= 1 << 63 else v


@dataclasses.dataclass
class XEvent:
    name: str
    offset_ps: int
    duration_ps: int
    stats: Dict[str, object]


@dataclasses.dataclass
class XLine:
    id: int
    name: str
    display_name: str
    timestamp_ns: int
    duration_ps: int
    events: List[XEvent]


@dataclasses.dataclass
class XPlane:
    id: int
    name: str
    lines: List[XLine]


@dataclasses.dataclass
class XSpace:
    planes: List[XPlane]
    errors: List[str]
    warnings: List[str]
    hostnames: List[str]

    def plane(self, name: str) -> Optional[XPlane]:
        return next((p for p in self.planes if p.name == name), None)


def _stat(buf: bytes, names: Dict[int, str]) -> Tuple[str, object]:
    md, value = 0, None
    for f, w, v in _fields(buf):
        if f == 1:
            md = v
        elif f == 2:
            value = C.c_double.from_buffer_copy(v).value
        elif f in (3, 7):
            value = v
        elif f == 4:
            value = _signed(v)
        elif f == 5:
            value = v.decode("utf-8", "replace")
        elif f == 6:
            value = bytes(v)
    return names.get(md, str(md)), value


def _metadata_map(buf: bytes) -> Tuple[int, str]:
    key, name = 0, ""
    for f, w, v in _fields(buf):
        if f == 1:
            key = _signed(v)
        elif f == 2:
            for f2, w2, v2 in _fields(v):
                if f2 == 2:
                    name = v2.decode("utf-8", "replace")
    return key, name


def decode_xspace(buf: bytes) -> XSpace:
    space = XSpace([], [], [], [])
    for f, w, v in _fields(buf):
        if f == 1:
            pid, pname, raw_lines, ev_names, st_names = 0, "", [], {}, {}
            for f2, w2, v2 in _fields(v):
                if f2 == 1:
                    pid = _signed(v2)
                elif f2 == 2:
                    pname = v2.decode("utf-8", "replace")
                elif f2 == 3:
                    raw_lines.append(v2)
                elif f2 == 4:
                    k, n = _metadata_map(v2)
                    ev_names[k] = n
                elif f2 == 5:
                    k, n = _metadata_map(v2)
                    st_names[k] = n
            lines = []
            for lb in raw_lines:
                ln = XLine(0, "", "", 0, 0, [])
                for f3, w3, v3 in _fields(lb):
                    if f3 == 1:
                        ln.id = _signed(v3)
                    elif f3 == 2:
                        ln.name = v3.decode("utf-8", "replace")
                    elif f3 == 11:
                        ln.display_name = v3.decode("utf-8", "replace")
                    elif f3 == 3:
                        ln.timestamp_ns = _signed(v3)
                    elif f3 == 9:
                        ln.duration_ps = _signed(v3)
                    elif f3 == 4:
                        md, off, dur, stats = 0, 0, 0, {}
                        for f4, w4, v4 in _fields(v3):
                            if f4 == 1:
                                md = _signed(v4)
                            elif f4 == 2:
                                off = _signed(v4)
                            elif f4 == 3:
                                dur = _signed(v4)
                            elif f4 == 4:
                                k, val = _stat(v4, st_names)
                                stats[k] = val
                        ln.events.append(XEvent(ev_names.get(md, str(md)), off, dur, stats))
                lines.append(ln)
            space.planes.append(XPlane(pid, pname, lines))
        elif f in (2, 3, 4):
            [space.errors, space.warnings, space.hostnames][f - 2].append(v.decode("utf-8", "replace"))
    return space


# ----------------------------------------------------------------------------------------------- extension
class ProfilerExtension:
    """PJRT_Profiler_Extension: its PLUGIN_Profiler_Api table, with errors of the API's own type."""

    def __init__(self, api: "P.Api", address: int):
        self.api, self.address = api, address
        self.table = C.c_void_p.from_address(address + 24).value
        if not self.table:
            raise P.PjrtError(P.ErrorCode.UNIMPLEMENTED, "the profiler extension has no profiler API")
        self.table_size = C.c_size_t.from_address(self.table).value
        self.trace_me_context_id = C.c_int64.from_address(address + 32).value

    def _fn(self, name: str, restype=_vp):
        off = 16 + 8 * _API_SLOTS.index(name)
        fp = C.c_void_p.from_address(self.table + off).value if self.table_size >= off + 8 else None
        if not fp:
            raise P.PjrtError(P.ErrorCode.UNIMPLEMENTED, f"{name} is not implemented by the loaded plugin")
        return C.CFUNCTYPE(restype, C.POINTER(_ARGS[name]))(fp)

    def _error(self, handle) -> Optional[P.PjrtError]:
        if not handle:
            return None
        m = _ErrorMessageArgs(C.sizeof(_ErrorMessageArgs), None, handle, None, 0)
        self._fn("PLUGIN_Profiler_Error_Message", None)(C.byref(m))
        message = P._str(m.message, m.message_size)
        g = _ErrorGetCodeArgs(C.sizeof(_ErrorGetCodeArgs), None, handle, 0)
        gerr = self._fn("PLUGIN_Profiler_Error_GetCode")(C.byref(g))
        d = _ErrorDestroyArgs(C.sizeof(_ErrorDestroyArgs), None, handle)
        self._fn("PLUGIN_Profiler_Error_Destroy", None)(C.byref(d))
        if gerr:
            self._fn("PLUGIN_Profiler_Error_Destroy", None)(C.byref(_ErrorDestroyArgs(C.sizeof(_ErrorDestroyArgs),
                                                                                    None, gerr)))
        try:
            code = P.ErrorCode(g.code) if not gerr else P.ErrorCode.UNKNOWN
        except ValueError:
            code = P.ErrorCode.UNKNOWN
        return P.PjrtError(code, message)

    def call(self, name: str, args):
        args.struct_size = C.sizeof(args)
        err = self._error(self._fn(name)(C.byref(args)))
        if err is not None:
            raise err
        return args

    def profiler(self, options: ProfileOptions) -> "Profiler":
        raw = options.encode()
        buf = C.create_string_buffer(raw, len(raw))
        a = self.call("PLUGIN_Profiler_Create", _CreateArgs(0, C.cast(buf, _vp), len(raw), None))
        return Profiler(self, a.profiler)


def extension(api: "P.Api") -> ProfilerExtension:
    p = api.extension(PJRT_EXTENSION_TYPE_PROFILER)
    if not p:
        raise P.PjrtError(P.ErrorCode.UNIMPLEMENTED, "the profiler extension is not provided by the PJRT plugin")
    return ProfilerExtension(api, p)


class Profiler(P._Owned):
    """A profiling session (profiler.rs:173-255): create → start → (PJRT work) → stop → results."""
    _exit_order = 0  # destroyed before the clients

    def __init__(self, ext: ProfilerExtension, handle: int):
        if not handle:
            raise P.PjrtError(P.ErrorCode.INVALID_ARGUMENT, "the provided PJRT profiler handle is a null pointer")
        self.ext, self.handle = ext, handle

    def start(self) -> None:
        self.ext.call("PLUGIN_Profiler_Start", _HandleArgs(0, self.handle))

    def stop(self) -> None:
        self.ext.call("PLUGIN_Profiler_Stop", _HandleArgs(0, self.handle))

    def results_bytes(self) -> bytes:
        # one call with a null buffer: the plugin serializes into storage of its own and returns it (NUL included)
        a = self.ext.call("PLUGIN_Profiler_CollectData", _CollectDataArgs(0, self.handle, None, 0))
        if not a.buffer or not a.buffer_size_in_bytes:
            return b""
        return C.string_at(a.buffer, a.buffer_size_in_bytes - 1)  # the size counts the trailing NUL

    def results(self) -> XSpace:
        return decode_xspace(self.results_bytes())

    def __del__(self):
        try:
            if self.handle:
                self.ext.call("PLUGIN_Profiler_Destroy", _HandleArgs(0, self.handle))
                self.handle = None
        except Exception:
            pass
