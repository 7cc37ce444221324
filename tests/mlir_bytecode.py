"""MLIR bytecode writer for the tests: turns the StableHLO text modules the tests build (the pretty syntax ryft-mlir's
printer emits, for the supported op set) into MLIR bytecode, the form ryft-mlir's `Operation::bytecode()` hands to
`Program::Mlir` (crates/ryft-mlir/src/operations/operation.rs:805-819; README.md:88).

It follows MLIR's published bytecode format (versions 4-6): prefix varints, a string section, a dialect section with
op names, an attribute/type section located by an offset section (builtin and StableHLO dialect encodings; the f8
element types as assembly text), the IR section with isolated regions nested as sections, and - from version 5 on -
a properties section holding the inherent attributes of ops. Options select the variants a producer may emit
(properties vs attribute dictionaries, the order of property fields, StableHLO attributes in binary or text form,
isolated or inline reduce bodies) so the plugin's reader is exercised on each. Test infrastructure only: the
byte-level layout mirrors what the reader expects, so a round trip through it pins the reader against this writer's
reading of the format, not against bytes produced by MLIR itself.
"""
from __future__ import annotations

import re
import struct
from typing import Dict, List, Optional, Sequence, Tuple

# ------------------------------------------------------------------------------------------------ encoding
def varint(v: int) -> bytes:
    assert v >= 0
    for n in range(1, 9):
        if v < (1 << (7 * n)):
            return ((v << n) | (1 << (n - 1))).to_bytes(n, "little")
    return b"\x00" + v.to_bytes(8, "little")


def svarint(v: int) -> bytes:
    return varint(((v << 1) ^ (v >> 63)) & ((1 << 64) - 1))


def varint_flag(v: int, flag: bool) -> bytes:
    return varint((v << 1) | int(flag))


def section(sid: int, data: bytes) -> bytes:
    return bytes([sid]) + varint(len(data)) + data


# ------------------------------------------------------------------------------------------------ text subset
_TENSOR = re.compile(r"tensor<([^<>]*)>")
ELEM = {"f32", "bf16", "f16", "f64", "f8E4M3FN", "f8E5M2", "i1", "i8", "i16", "i32", "i64", "ui8", "ui16", "ui32",
        "ui64"}


def parse_tensor(t: str) -> Tuple[Tuple[int, ...], str]:
    t = t.strip()
    m = _TENSOR.fullmatch(t)
    if not m:
        assert t in ELEM, t
        return (), t
    parts = m.group(1).split("x")
    dims = []
    while parts and parts[0].isdigit():
        dims.append(int(parts.pop(0)))
    return tuple(dims), "x".join(parts)


def _split_top(s: str, sep: str = ",") -> List[str]:
    out, depth, cur = [], 0, ""
    for ch in s:
        if ch in "<[({":
            depth += 1
        elif ch in ">])}":
            depth -= 1
        if ch == sep and depth == 0:
            out.append(cur)
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur)
    return [x.strip() for x in out]


def _types_after_colon(s: str) -> Tuple[List[str], List[str]]:
    """`(A, B) -> C`, `(A) -> (B, C)` or `A, B` → (inputs, results)."""
    s = s.strip()
    if s.startswith("("):
        depth = 0
        for i, ch in enumerate(s):
            depth += ch == "("
            depth -= ch == ")"
            if depth == 0:
                break
        ins = _split_top(s[1:i])
        rest = s[i + 1:].strip()
        assert rest.startswith("->"), s
        rest = rest[2:].strip()
        outs = _split_top(rest[1:-1]) if rest.startswith("(") else [rest]
        return ins, outs
    return _split_top(s), []


def _ints(s: str) -> List[int]:
    return [int(x) for x in re.findall(r"-?\d+", s)]


class Op:
    def __init__(self, name, operands, results, result_types, attrs=None, body=None):
        self.name = name                  # "stablehlo.add"
        self.operands = operands          # SSA names
        self.results = results            # SSA names
        self.result_types = result_types  # type strings
        self.attrs = attrs or {}          # name → ("kind", value)
        self.body = body                  # reduce: (op name, arg type)
        self.region = None                # reduce with a general body: (arg names, arg types, ops, returned names)
        self.branches = None              # if / case: per branch (ops, returned names), no block arguments


def parse_module(text: str):
    """Returns (arg names, arg types, result types, ops, returned names) of `func.func @main`."""
    m = re.search(r"func\.func\s+(?:public\s+)?@main\((.*?)\)\s*->\s*(.*?)\s*\{\n", text, re.S)
    assert m, "no func.func @main"
    args = [a.strip() for a in _split_top(m.group(1))]
    arg_names = [a.split(":")[0].strip() for a in args]
    arg_types = [a.split(":", 1)[1].split("{")[0].strip() for a in args]  # (argument attributes: arg_attr_dicts)
    res = m.group(2).strip()
    res_types = _split_top(res[1:-1]) if res.startswith("(") else [res]
    body = text[m.end():]
    ops, returned = _parse_lines([ln.strip() for ln in body.split("\n")], "return")
    return arg_names, arg_types, res_types, ops, returned


def _parse_lines(lines: List[str], ret: str):
    """Ops of a block up to its `ret` line; returns (ops, returned names). A `%r:k = ...` op names its results
    %r#0 .. %r#(k-1); a reduce followed by a `reducer(...) {` line takes the region up to its closing brace."""
    ops: List[Op] = []
    returned: List[str] = []
    i = 0
    while i < len(lines):
        line = lines[i]
        i += 1
        if not line or line == "}":
            continue
        if line.startswith(ret):
            vals = line[len(ret):].split(":")[0]
            returned = [v.strip() for v in vals.split(",")]
            break
        lhs, rhs = line.split("=", 1)
        lhs, rhs = lhs.strip(), rhs.strip()
        name, rest = rhs.split(None, 1) if " " in rhs else (rhs, "")
        if name.startswith("stablehlo.reduce("):
            name, rest = "stablehlo.reduce", rhs[len("stablehlo.reduce"):]
        if rhs.startswith('"stablehlo.gather"('):
            ops.append(_parse_gather(lhs, rhs))
            continue
        if rhs.startswith('"stablehlo.if"(') or rhs.startswith('"stablehlo.case"('):
            # `%r = "stablehlo.if"(%p) ({`, branch ops and return, `}, {`, ..., then `}) : (I) -> R`: one block
            # without arguments per branch, using values of the enclosing scope
            branches, cur = [], []
            while not lines[i].startswith("})"):
                if lines[i] == "}, {":
                    branches.append(cur)
                    cur = []
                else:
                    cur.append(lines[i])
                i += 1
            branches.append(cur)
            m = re.fullmatch(r'"(stablehlo\.\w+)"\((%\w+)\) \(\{', rhs.strip())
            _, outs = _types_after_colon(lines[i][len("})"):].strip().lstrip(":").strip())
            op = Op(m.group(1), [m.group(2)], _result_names(lhs), outs)
            op.branches = [_parse_lines(b, "stablehlo.return") for b in branches]
            ops.append(op)
            i += 1
            continue
        if rhs.startswith('"stablehlo.scatter"('):
            region_lines = []
            while not lines[i].startswith("})"):
                region_lines.append(lines[i])
                i += 1
            ops.append(_parse_scatter(lhs, rhs, region_lines, lines[i]))
            i += 1
            continue
        if name == "stablehlo.reduce" and "applies" not in rest:
            region_lines = []
            while not lines[i].startswith("}"):
                region_lines.append(lines[i])
                i += 1
            i += 1
            ops.append(_parse_general_reduce(lhs, rest, region_lines))
            continue
        ops.append(_parse_op(lhs, name, rest))
    return ops, returned


def _result_names(lhs: str) -> List[str]:
    if ":" in lhs:
        nm, k = lhs.split(":")
        return [f"{nm.strip()}#{j}" for j in range(int(k))]
    return [lhs]


def _parse_general_reduce(lhs: str, rest: str, region_lines: List[str]) -> Op:
    # `(%x init: %i), (%y init: %j) across dimensions = [..] : (types) -> (types)`, then
    # `reducer(%a0: T, %b0: T) (%a1: U, %b1: U) {`, the body's ops and `stablehlo.return ...`
    head, ty = rest.split(" : ", 1)
    pairs = re.findall(r"\((%\w+) init: (%\w+)\)", head)
    dims = _ints(re.search(r"dimensions = \[(.*?)\]", head).group(1))
    ins, outs = _types_after_colon(ty)
    op = Op("stablehlo.reduce", [p[0] for p in pairs] + [p[1] for p in pairs], _result_names(lhs), outs,
            {"dimensions": ("i64s", dims)})
    decl = region_lines[0]
    arg_pairs = re.findall(r"\((%\w+): (tensor<[^>]*>), (%\w+): (tensor<[^>]*>)\)", decl)
    names = [a[0] for a in arg_pairs] + [a[2] for a in arg_pairs]
    types = [a[1] for a in arg_pairs] + [a[3] for a in arg_pairs]
    body_ops, returned = _parse_lines(region_lines[1:], "stablehlo.return")
    op.region = (names, types, body_ops, returned)
    return op


def arg_attr_dicts(text: str) -> List[Dict[str, Tuple[str, str]]]:
    """Per argument of `func.func @main`, its attribute dictionary: name → (value, type), e.g.
    {"tf.aliasing_output": ("0", "i32")}; a value without a type is a bool ("true") or a unit attribute ("")."""
    m = re.search(r"func\.func\s+(?:public\s+)?@main\((.*?)\)\s*->", text, re.S)
    out = []
    for a in _split_top(m.group(1)):
        d = {}
        if "{" in a:
            body = a[a.index("{") + 1:a.rindex("}")]
            for item in _split_top(body):
                k, _, v = item.partition("=")
                val, _, ty = v.partition(":")
                d[k.strip().strip('"')] = (val.strip(), ty.strip())
        out.append(d)
    return out


def _parse_gather(res: str, rhs: str) -> Op:
    # `"stablehlo.gather"(%a, %b) <{dimension_numbers = #stablehlo.gather<...>, indices_are_sorted = ...,
    # slice_sizes = array<i64: ...>}> : (A, B) -> R`
    m = re.fullmatch(r'"stablehlo\.gather"\((%\w+), (%\w+)\) <\{(.*)\}> : (.*)', rhs.strip())
    assert m, rhs
    attrs_txt = m.group(3)
    dn = re.search(r"#stablehlo\.gather<(.*?)>", attrs_txt).group(1)

    def field(name):
        f = re.search(name + r"\s*=\s*\[(.*?)\]", dn)
        return _ints(f.group(1)) if f else []

    g = {k: field(k) for k in ("offset_dims", "collapsed_slice_dims", "operand_batching_dims",
                               "start_indices_batching_dims", "start_index_map")}
    g["index_vector_dim"] = int(re.search(r"index_vector_dim\s*=\s*(\d+)", dn).group(1))
    sizes = _ints(re.search(r"slice_sizes\s*=\s*array<i64:(.*?)>", attrs_txt).group(1))
    ins, outs = _types_after_colon(m.group(4))
    attrs = {"dimension_numbers": ("gather_dims", g), "slice_sizes": ("i64s", sizes)}
    return Op("stablehlo.gather", [m.group(1), m.group(2)], [res], outs, attrs)


def _parse_scatter(res: str, rhs: str, region_lines: List[str], close: str) -> Op:
    # `"stablehlo.scatter"(%a, %i, %u) <{indices_are_sorted = .., scatter_dimension_numbers = #stablehlo.scatter<..>,
    # unique_indices = ..}> ({`, the region `^bb0(%x: T, %y: T):`, its ops and return, then `}) : (A, I, U) -> A`
    m = re.fullmatch(r'"stablehlo\.scatter"\((%\w+), (%\w+), (%\w+)\) <\{(.*)\}> \(\{', rhs.strip())
    assert m, rhs
    attrs_txt = m.group(4)
    dn = re.search(r"#stablehlo\.scatter<(.*?)>", attrs_txt).group(1)

    def field(name):
        f = re.search(name + r"\s*=\s*\[(.*?)\]", dn)
        return _ints(f.group(1)) if f else []

    g = {k: field(k) for k in ("update_window_dims", "inserted_window_dims", "input_batching_dims",
                               "scatter_indices_batching_dims", "scatter_dims_to_operand_dims")}
    g["index_vector_dim"] = int(re.search(r"index_vector_dim\s*=\s*(\d+)", dn).group(1))
    attrs = {"scatter_dimension_numbers": ("scatter_dims", g)}
    for b in ("indices_are_sorted", "unique_indices"):
        bm = re.search(b + r"\s*=\s*(true|false)", attrs_txt)
        if bm:
            attrs[b] = ("bool", bm.group(1) == "true")
    ins, outs = _types_after_colon(close[len("})"):].strip().lstrip(":").strip())
    op = Op("stablehlo.scatter", [m.group(1), m.group(2), m.group(3)], [res], outs, attrs)
    decl = region_lines[0]
    args = re.findall(r"(%\w+): (tensor<[^>]*>)", decl)
    body_ops, returned = _parse_lines(region_lines[1:], "stablehlo.return")
    op.region = ([a[0] for a in args], [a[1] for a in args], body_ops, returned)
    return op


def _parse_op(res: str, name: str, rest: str) -> Op:
    short = name.split(".", 1)[1]
    if short == "optimization_barrier":  # `%r:k = stablehlo.optimization_barrier %a, %b : A, B`
        body, ty = rest.split(" : ", 1)
        return Op(name, [x.strip() for x in body.split(",")], _result_names(res), [t.strip() for t in _split_top(ty)])
    if short == "constant":
        val, ty = rest.rsplit(":", 1)
        return Op(name, [], [res], [ty.strip()], {"value": ("dense", val.strip(), ty.strip())})
    if short == "reduce":
        m = re.fullmatch(r"\((%\w+) init: (%\w+)\) applies (\S+) across dimensions = \[(.*?)\] : (.*)", rest.strip())
        assert m, rest
        ins, outs = _types_after_colon(m.group(5))
        return Op(name, [m.group(1), m.group(2)], [res], outs,
                  {"dimensions": ("i64s", _ints(m.group(4)))}, body=(m.group(3), ins[1]))
    if short == "iota":
        m = re.fullmatch(r"dim = (\d+) : (.*)", rest.strip())
        return Op(name, [], [res], [m.group(2).strip()], {"iota_dimension": ("i64", int(m.group(1)))})
    if short == "compare":
        body, ty = rest.split(":", 1)
        parts = [p.strip() for p in body.split(",")]
        attrs = {"comparison_direction": ("cmp_dir", parts[0])}
        if len(parts) > 3:
            attrs["compare_type"] = ("cmp_type", parts[3])
        ins, outs = _types_after_colon(ty)
        return Op(name, parts[1:3], [res], outs, attrs)
    if short == "slice":
        m = re.fullmatch(r"(%\w+) \[(.*?)\] : (.*)", rest.strip())
        starts, limits, strides = [], [], []
        for part in [x for x in m.group(2).split(",") if x.strip()]:
            f = [int(v) for v in part.split(":")]
            starts.append(f[0])
            limits.append(f[1])
            strides.append(f[2] if len(f) > 2 else 1)
        ins, outs = _types_after_colon(m.group(3))
        return Op(name, [m.group(1)], [res], outs, {"start_indices": ("i64s", starts), "limit_indices": ("i64s", limits),
                                                    "strides": ("i64s", strides)})
    if short == "get_dimension_size":  # `%r = stablehlo.get_dimension_size %x, dim = 1 : (T) -> tensor<i32>`
        m = re.fullmatch(r"(%\w+), dim = (\d+) : (.*)", rest.strip())
        _, outs = _types_after_colon(m.group(3))
        return Op(name, [m.group(1)], [res], outs, {"dimension": ("i64", int(m.group(2)))})
    if short in ("replica_id", "partition_id"):  # `%r = stablehlo.replica_id : tensor<ui32>`
        return Op(name, [], [res], [rest.strip().lstrip(":").strip()])
    body, ty = rest.split(" : ", 1)
    ins, outs = _types_after_colon(ty)
    items = _split_top(body)
    operands = [x for x in items if x.startswith("%")]
    attrs = {}
    if short in ("broadcast_in_dim", "transpose"):
        key = "broadcast_dimensions" if short == "broadcast_in_dim" else "permutation"
        kv = [x for x in items if x.startswith("dims")][0]
        attrs[key] = ("i64s", _ints(kv.split("=", 1)[1]))
    if short == "reduce_precision":  # `%x, format = e5m10`
        kv = [x for x in items if x.startswith("format")][0]
        fm = re.match(r"format\s*=\s*e(\d+)m(\d+)", kv)
        attrs["exponent_bits"] = ("i32", int(fm.group(1)))
        attrs["mantissa_bits"] = ("i32", int(fm.group(2)))
    if short == "reverse":
        kv = [x for x in items if x.startswith("dims")][0]
        attrs["dimensions"] = ("i64s", _ints(kv.split("=", 1)[1]))
    if short == "dynamic_slice":
        kv = [x for x in items if x.startswith("sizes")][0]
        attrs["slice_sizes"] = ("i64s", _ints(kv.split("=", 1)[1]))
    if short == "concatenate":
        kv = [x for x in items if x.startswith("dim")][0]
        attrs["dimension"] = ("i64", int(kv.split("=", 1)[1]))
    if short == "pad":
        for key, attr in (("low", "edge_padding_low"), ("high", "edge_padding_high"), ("interior", "interior_padding")):
            kv = [x for x in items if x.startswith(key)][0]
            attrs[attr] = ("i64s", _ints(kv.split("=", 1)[1]))
    if short == "dot_general":
        dd = {"lhs_batch": [], "rhs_batch": [], "lhs_contract": [], "rhs_contract": []}
        for x in items:
            if x.startswith("batching_dims") or x.startswith("contracting_dims"):
                lr = x.split("=", 1)[1].split(" x ")
                k = "batch" if x.startswith("batching") else "contract"
                dd["lhs_" + k], dd["rhs_" + k] = _ints(lr[0]), _ints(lr[1])
        attrs["dot_dimension_numbers"] = ("dot_dims", dd)
    if not outs:  # `op %a, %b : T` (all types equal) or select's `: P, T`
        outs = [ins[-1]]
    return Op(name, operands, [res], outs, attrs)


# ------------------------------------------------------------------------------------------------ writer
CMP_DIR = {"EQ": 0, "NE": 1, "GE": 2, "GT": 3, "LE": 4, "LT": 5}
CMP_TYPE = {"NOTYPE": 0, "FLOAT": 1, "TOTALORDER": 2, "SIGNED": 3, "UNSIGNED": 4}
# inherent attributes of the ops this writer emits, sorted by name (the generated property readers' order) ...
SORTED = {
    "func.func": ["arg_attrs", "function_type", "res_attrs", "sym_name", "sym_visibility"],
    "stablehlo.compare": ["compare_type", "comparison_direction"],
    "stablehlo.dot_general": ["algorithm", "dot_dimension_numbers", "precision_config"],
    "stablehlo.slice": ["limit_indices", "start_indices", "strides"],
    "stablehlo.pad": ["edge_padding_high", "edge_padding_low", "interior_padding"],
    "stablehlo.gather": ["dimension_numbers", "indices_are_sorted", "slice_sizes"],
    "stablehlo.scatter": ["indices_are_sorted", "scatter_dimension_numbers", "unique_indices"],
}
# ... and in declaration order
DECLARED = {
    "func.func": ["sym_name", "function_type", "sym_visibility", "arg_attrs", "res_attrs"],
    "stablehlo.compare": ["comparison_direction", "compare_type"],
    "stablehlo.dot_general": ["dot_dimension_numbers", "precision_config", "algorithm"],
    # slice and pad: written sorted in every variant (three fields of one kind: a reader could not tell another
    # order apart)
    "stablehlo.slice": ["limit_indices", "start_indices", "strides"],
    "stablehlo.pad": ["edge_padding_high", "edge_padding_low", "interior_padding"],
    "stablehlo.gather": ["dimension_numbers", "slice_sizes", "indices_are_sorted"],
    "stablehlo.scatter": ["scatter_dimension_numbers", "indices_are_sorted", "unique_indices"],
}
REQUIRED = {"function_type", "sym_name", "comparison_direction", "dot_dimension_numbers", "value", "iota_dimension",
            "broadcast_dimensions", "permutation", "dimensions", "start_indices", "limit_indices", "strides",
            "dimension", "edge_padding_low", "edge_padding_high", "interior_padding", "slice_sizes",
            "dimension_numbers", "scatter_dimension_numbers", "exponent_bits", "mantissa_bits", "dimension"}


class Writer:
    def __init__(self, version=6, properties=True, order="sorted", stablehlo_attrs="binary",
                 isolated_reduce=False, producer="MLIR20.0.0git"):
        assert version >= 4 and (properties is False or version >= 5)
        self.version, self.properties, self.order = version, properties, order
        self.text_attrs = stablehlo_attrs == "text"
        self.isolated_reduce = isolated_reduce
        self.producer = producer
        self.strings: List[str] = []
        self.dialects = ["builtin", "func", "stablehlo"]
        self.opnames: List[Tuple[int, str]] = []
        self.entries = {"attr": [], "type": []}  # (dialect, custom, bytes)
        self.index = {"attr": {}, "type": {}}
        self.props: List[bytes] = []

    # -- tables
    def s(self, x: str) -> int:
        if x not in self.strings:
            self.strings.append(x)
        return self.strings.index(x)

    def opname(self, full: str) -> int:
        d, n = full.split(".", 1)
        key = (self.dialects.index(d), n)
        if key not in self.opnames:
            self.opnames.append(key)
        return self.opnames.index(key)

    def _entry(self, kind: str, dialect: str, custom: bool, data: bytes) -> int:
        key = (dialect, custom, data)
        if key not in self.index[kind]:
            self.index[kind][key] = len(self.entries[kind])
            self.entries[kind].append(key)
        return self.index[kind][key]

    # -- types
    def elem(self, e: str) -> int:
        codes = {"bf16": 3, "f16": 4, "f32": 5, "f64": 6}
        if e in codes:
            return self._entry("type", "builtin", True, varint(codes[e]))
        if e.startswith("i") or e.startswith("ui"):
            w = int(e.lstrip("ui"))
            return self._entry("type", "builtin", True, varint(0) + varint((w << 2) | (2 if e.startswith("ui") else 0)))
        return self._entry("type", "builtin", False, e.encode() + b"\0")  # f8 types: assembly text

    def tensor(self, t: str) -> int:
        dims, e = parse_tensor(t)
        el = self.elem(e)
        data = varint(13) + varint(len(dims)) + b"".join(svarint(d) for d in dims) + varint(el)
        return self._entry("type", "builtin", True, data)

    def fn_type(self, ins: Sequence[str], outs: Sequence[str]) -> int:
        i = [self.tensor(t) for t in ins]
        o = [self.tensor(t) for t in outs]
        data = varint(2) + varint(len(i)) + b"".join(map(varint, i)) + varint(len(o)) + b"".join(map(varint, o))
        return self._entry("type", "builtin", True, data)

    # -- attributes
    def battr(self, data: bytes) -> int:
        return self._entry("attr", "builtin", True, data)

    def string_attr(self, x: str) -> int:
        return self.battr(varint(2) + varint(self.s(x)))

    def unknown_loc(self) -> int:
        return self.battr(varint(15))

    def attr(self, spec) -> int:
        kind = spec[0]
        if kind == "i64s":
            raw = b"".join(struct.pack("<q", v) for v in spec[1])
            return self.battr(varint(17) + varint(self.elem("i64")) + varint(len(spec[1])) + varint(len(raw)) + raw)
        if kind == "i32":
            return self.battr(varint(8) + varint(self.elem("i32")) + svarint(spec[1]))
        if kind == "i64":
            return self.battr(varint(8) + varint(self.elem("i64")) + svarint(spec[1]))
        if kind == "dense":
            return self.battr(varint(18) + varint(self.tensor(spec[2])) + self._dense_blob(spec[1], spec[2]))
        if kind == "type":
            return self.battr(varint(6) + varint(spec[1]))
        if kind == "string":
            return self.string_attr(spec[1])
        if kind == "cmp_dir":
            if self.text_attrs:
                return self._entry("attr", "stablehlo", False, f"#stablehlo<comparison_direction {spec[1]}>".encode() + b"\0")
            return self._entry("attr", "stablehlo", True, varint(2) + varint(CMP_DIR[spec[1]]))
        if kind == "cmp_type":
            if self.text_attrs:
                return self._entry("attr", "stablehlo", False, f"#stablehlo<comparison_type {spec[1]}>".encode() + b"\0")
            return self._entry("attr", "stablehlo", True, varint(3) + varint(CMP_TYPE[spec[1]]))
        if kind == "dot_dims":
            d = spec[1]
            if self.text_attrs:
                txt = ("#stablehlo.dot<lhs_batching_dimensions = {}, rhs_batching_dimensions = {}, "
                       "lhs_contracting_dimensions = {}, rhs_contracting_dimensions = {}>").format(
                    d["lhs_batch"], d["rhs_batch"], d["lhs_contract"], d["rhs_contract"])
                return self._entry("attr", "stablehlo", False, txt.encode() + b"\0")
            data = varint(5)
            for k in ("lhs_batch", "rhs_batch", "lhs_contract", "rhs_contract"):
                data += varint(len(d[k])) + b"".join(svarint(v) for v in d[k])
            return self._entry("attr", "stablehlo", True, data)
        if kind == "bool":  # BoolAttr: an IntegerAttr of type i1 (builtin code 8)
            return self.battr(varint(8) + varint(self.elem("i1")) + bytes([1 if spec[1] else 0]))
        if kind == "scatter_dims":
            g = spec[1]
            lists = ("update_window_dims", "inserted_window_dims", "input_batching_dims",
                     "scatter_indices_batching_dims", "scatter_dims_to_operand_dims")
            if self.text_attrs:
                fields = [f"{k} = {g[k]}" for k in lists if g[k]] + [f"index_vector_dim = {g['index_vector_dim']}"]
                return self._entry("attr", "stablehlo", False, ("#stablehlo.scatter<" + ", ".join(fields) + ">").encode()
                                   + b"\0")
            data = varint(11)
            for k in lists:
                data += varint(len(g[k])) + b"".join(svarint(v) for v in g[k])
            data += svarint(g["index_vector_dim"])
            return self._entry("attr", "stablehlo", True, data)
        if kind == "gather_dims":
            g = spec[1]
            lists = ("offset_dims", "collapsed_slice_dims", "operand_batching_dims", "start_indices_batching_dims",
                     "start_index_map")
            if self.text_attrs:
                fields = [f"{k} = {g[k]}" for k in lists if g[k]] + [f"index_vector_dim = {g['index_vector_dim']}"]
                return self._entry("attr", "stablehlo", False, ("#stablehlo.gather<" + ", ".join(fields) + ">").encode()
                                   + b"\0")
            data = varint(7)
            for k in lists:
                data += varint(len(g[k])) + b"".join(svarint(v) for v in g[k])
            data += svarint(g["index_vector_dim"])
            return self._entry("attr", "stablehlo", True, data)
        raise ValueError(kind)

    def _dense_blob(self, val: str, ty: str) -> bytes:
        dims, e = parse_tensor(ty)
        n = 1
        for d in dims:
            n *= d
        payload = val[len("dense<"):-1].strip()
        toks = [t for t in re.split(r"[\[\],\s]+", payload) if t]
        fmt = {"f32": "<f", "f64": "<d", "i32": "<i", "i64": "<q", "i8": "<b", "i16": "<h", "ui8": "<B"}
        out = b""
        for t in toks:
            if t.startswith("0x"):
                size = {"f32": 4, "f64": 8, "bf16": 2, "f16": 2, "i32": 4, "i64": 8}.get(e, 1)
                out += int(t, 16).to_bytes(size, "little")
            elif e == "i1":
                out += bytes([0xFF if t == "true" else 0x00])
            elif e == "bf16":
                f = struct.unpack("<I", struct.pack("<f", float(t)))[0]
                out += (((f + 0x7FFF + ((f >> 16) & 1)) >> 16) & 0xFFFF).to_bytes(2, "little")
            else:
                out += struct.pack(fmt[e], float(t) if e.startswith("f") else int(t))
        assert len(toks) in (1, n), (val, ty)
        return varint(len(out)) + out

    # -- IR
    def _props(self, op_name: str, attrs: Dict[str, int]) -> bytes:
        names = (SORTED if self.order == "sorted" else DECLARED).get(op_name, sorted(attrs))
        data = b""
        for nm in names:
            if nm in REQUIRED:
                data += varint(attrs[nm])
            elif nm in attrs:
                data += varint_flag(attrs[nm], True)
            else:
                data += varint_flag(0, False)
        return data

    def _op(self, name: str, attrs: Dict[str, int], result_types: List[int], operands: List[int],
            regions: Optional[bytes] = None, isolated: bool = False, n_regions: int = 0) -> bytes:
        mask = 0
        out = b""
        if attrs:
            if self.properties:
                mask |= 0x40
                blob = self._props(name, attrs)
                entry = varint(len(blob)) + blob
                if entry not in self.props:
                    self.props.append(entry)
                out += varint(self.props.index(entry))
            else:
                mask |= 0x01
                d = varint(1) + varint(len(attrs))
                for k in sorted(attrs):
                    d += varint(self.string_attr(k)) + varint(attrs[k])
                out += varint(self.battr(d))
        if result_types:
            mask |= 0x02
            out += varint(len(result_types)) + b"".join(map(varint, result_types))
        if operands:
            mask |= 0x04
            out += varint(len(operands)) + b"".join(map(varint, operands))
        if n_regions:
            mask |= 0x10
            out += varint_flag(n_regions, isolated)
            out += section(4, regions) if isolated else regions
        return varint(self.opname(name)) + bytes([mask]) + varint(self.unknown_loc()) + out

    def _block(self, arg_types: List[int], ops: List[bytes]) -> bytes:
        out = varint_flag(len(ops), bool(arg_types))
        if arg_types:
            out += varint(len(arg_types)) + b"".join(varint_flag(t, False) for t in arg_types)
            out += b"\x00"  # no use-list orders
        return out + b"".join(ops)

    def module(self, text: str) -> bytes:
        arg_names, arg_types, res_types, ops, returned = parse_module(text)
        values: Dict[str, int] = {n: i for i, n in enumerate(arg_names)}
        n_func_values = len(arg_names) + sum(len(o.results) for o in ops)
        body_ops = []
        for op in ops:
            attrs = {k: self.attr(v) for k, v in op.attrs.items()}
            operands = [values[o] for o in op.operands]
            rtypes = [self.tensor(t) for t in op.result_types]
            regions, n_regions = None, 0
            if op.body:
                # reduce body: two scalar block arguments, the combiner, a return; its values follow the function
                # body's (or start at 0 in a scope of their own when the region is isolated)
                base = 0 if self.isolated_reduce else n_func_values
                st = self.tensor(op.body[1])
                comb = self._op(op.body[0], {}, [st], [base, base + 1])
                ret = self._op("stablehlo.return", {}, [], [base + 2])
                regions = varint(1) + varint(3) + self._block([st, st], [comb, ret])
                n_regions = 1
            elif op.region:
                # a general body: its block arguments, its ops (values numbered after the arguments) and a return
                base = 0 if self.isolated_reduce else n_func_values
                names, types, rops, rets = op.region
                rvals = {nm: base + k for k, nm in enumerate(names)}
                n_vals = len(names) + sum(len(o.results) for o in rops)
                enc = []
                for o in rops:
                    enc.append(self._op(o.name, {k: self.attr(v) for k, v in o.attrs.items()},
                                        [self.tensor(t) for t in o.result_types], [rvals[x] for x in o.operands]))
                    for r in o.results:
                        rvals[r] = base + len(rvals)
                enc.append(self._op("stablehlo.return", {}, [], [rvals[r] for r in rets]))
                regions = varint(1) + varint(n_vals) + self._block([self.tensor(t) for t in types], enc)
                n_regions = 1
            elif op.branches:
                # one region per branch: a block without arguments whose values are numbered after the function
                # body's (every sibling region from the same base); operands from the enclosing scope keep their ids
                regions, n_regions = b"", len(op.branches)
                for rops, rets in op.branches:
                    rvals: Dict[str, int] = {}
                    enc = []
                    for o in rops:
                        enc.append(self._op(o.name, {k: self.attr(v) for k, v in o.attrs.items()},
                                            [self.tensor(t) for t in o.result_types],
                                            [rvals[x] if x in rvals else values[x] for x in o.operands]))
                        for r in o.results:
                            rvals[r] = n_func_values + len(rvals)
                    enc.append(self._op("stablehlo.return", {}, [], [rvals[r] if r in rvals else values[r] for r in rets]))
                    regions += varint(1) + varint(len(rvals)) + self._block([], enc)
                body_ops.append(self._op(op.name, attrs, rtypes, operands, regions, False, n_regions))
                for r in op.results:
                    values[r] = len(values)
                continue
            body_ops.append(self._op(op.name, attrs, rtypes, operands, regions, self.isolated_reduce, n_regions))
            for r in op.results:
                values[r] = len(values)
        body_ops.append(self._op("func.return", {}, [], [values[r] for r in returned]))
        fbody = varint(1) + varint(n_func_values) + self._block([self.tensor(t) for t in arg_types], body_ops)
        fattrs = {"sym_name": self.string_attr("main"),
                  "function_type": self.attr(("type", self.fn_type(arg_types, res_types)))}
        dicts = arg_attr_dicts(text)
        if any(dicts):  # arg_attrs: ArrayAttr of DictionaryAttr (builtin codes 0 and 1)
            elems = []
            for d in dicts:
                entries = b""
                for k, (val, ty) in sorted(d.items()):
                    if ty:
                        v = self.battr(varint(8) + varint(self.elem(ty)) + svarint(int(val)))
                    elif val in ("true", "false"):
                        v = self.battr(varint(8) + varint(self.elem("i1")) + bytes([val == "true"]))
                    else:
                        v = self.battr(varint(7))
                    entries += varint(self.string_attr(k)) + varint(v)
                elems.append(self.battr(varint(1) + varint(len(d)) + entries))
            fattrs["arg_attrs"] = self.battr(varint(0) + varint(len(elems)) + b"".join(varint(e) for e in elems))
        func = self._op("func.func", fattrs, [], [], fbody, True, 1)
        mbody = varint(1) + varint(0) + self._block([], [func])
        module = self._op("builtin.module", {}, [], [], mbody, True, 1)
        ir = varint_flag(1, False) + module
        return self._finish(ir)

    def _finish(self, ir: bytes) -> bytes:
        # dialects and op names
        d = varint(len(self.dialects))
        for name in self.dialects:
            d += varint_flag(self.s(name), False)
        by_dialect: Dict[int, List[str]] = {}
        for di, n in self.opnames:
            by_dialect.setdefault(di, []).append(n)
        d += varint(len(self.opnames))
        for di, names in by_dialect.items():
            d += varint(di) + varint(len(names))
            for n in names:
                d += varint_flag(self.s(n), True) if self.version >= 5 else varint(self.s(n))
        # the reader numbers op names in section order: to_bytecode registers them grouped by dialect up front
        assert [(di, n) for di, names in by_dialect.items() for n in names] == self.opnames
        # attributes / types
        data, offsets = b"", b""
        counts = []
        for kind in ("attr", "type"):
            ents = self.entries[kind]
            counts.append(len(ents))
            groups, prev = [], None
            for dialect, custom, blob in ents:
                di = self.dialects.index(dialect)
                if di != prev:
                    groups.append([di, []])
                    prev = di
                groups[-1][1].append(varint_flag(len(blob), custom))
                data += blob
            for di, sizes in groups:
                offsets += varint(di) + varint(len(sizes)) + b"".join(sizes)
        offsets = varint(counts[0]) + varint(counts[1]) + offsets
        strings = varint(len(self.strings)) + b"".join(varint(len(x.encode()) + 1) for x in reversed(self.strings))
        strings += b"".join(x.encode() + b"\0" for x in self.strings)
        out = b"ML\xefR" + varint(self.version) + self.producer.encode() + b"\0"
        out += section(1, d) + section(2, data) + section(3, offsets) + section(4, ir) + section(0, strings)
        if self.version >= 5:
            out += section(8, varint(len(self.props)) + b"".join(self.props))
        return out


def to_bytecode(text: str, **options) -> bytes:
    """StableHLO text (the subset above) → MLIR bytecode; options as for Writer."""
    w = Writer(**options)
    # op names are numbered by the dialect-grouped order of the dialect section: register them in that order first
    _, _, _, ops, _ = parse_module(text)
    names = {"builtin.module", "func.func", "func.return"} | {o.name for o in ops}
    names |= {o.body[0] for o in ops if o.body} | ({"stablehlo.return"} if any(o.body or o.region for o in ops)
                                                   else set())
    names |= {r.name for o in ops if o.region for r in o.region[2]}
    names |= {r.name for o in ops if o.branches for b in o.branches for r in b[0]}
    names |= {"stablehlo.return"} if any(o.branches for o in ops) else set()
    for n in sorted(names, key=lambda x: (w.dialects.index(x.split(".")[0]), x)):
        w.opname(n)
    return w.module(text)
