"""StableHLO text parser and numpy interpreter (oracle; see oracle/__init__.py).

Parses the pretty syntax that ryft-mlir's printer emits for the supported op set (printer goldens:
crates/ryft-mlir/src/dialects/stable_hlo/operations/linear_algebra.rs:2240-2263, functional.rs:529-541,
manipulation.rs:2022,2154, control_flow.rs:596, miscellaneous.rs:1181, casting.rs:456, comparison.rs:500) and
evaluates it op by op. Floating-point values are carried as float64 holding exactly the value of their StableHLO
element type: each op computes in float64 and rounds its result to the result element type (through f32, as an f32
datapath would). Integers are carried as int64 and wrapped to their width. Per-op semantics cite the ryft-mlir
documentation of each builder (file:line in the evaluator below).
"""
from __future__ import annotations

import math
import re
from typing import Dict, List, Sequence, Tuple

import numpy as np

from . import numerics

FLOAT = {"f16", "bf16", "f32", "f64", "f8E4M3FN", "f8E5M2"}
INT_BITS = {"i1": 1, "i8": 8, "i16": 16, "i32": 32, "i64": 64, "ui8": 8, "ui16": 16, "ui32": 32, "ui64": 64}

_TENSOR = re.compile(r"tensor<([^>]*)>")


def parse_type(t: str) -> Tuple[Tuple[int, ...], str]:
    m = _TENSOR.search(t)
    if not m:
        raise ValueError(f"not a tensor type: {t}")
    parts = m.group(1).split("x")
    # element types such as f8E4M3FN contain no 'x'; dims are the leading integer parts
    dims = []
    while parts and parts[0].isdigit():
        dims.append(int(parts.pop(0)))
    return tuple(dims), "x".join(parts)


def _types(s: str) -> List[Tuple[Tuple[int, ...], str]]:
    return [parse_type("tensor<" + g + ">") for g in _TENSOR.findall(s)]


def _ints(s: str) -> List[int]:
    return [int(v) for v in re.findall(r"-?\d+", s)] if s and s.strip() else []


# ----------------------------------------------------------------------------------------------- values
def wrap_int(x: np.ndarray, dtype: str) -> np.ndarray:
    bits = INT_BITS[dtype]
    x = np.asarray(x, dtype=np.int64)
    if dtype == "i1":
        return (x != 0).astype(np.int64)
    if bits == 64:
        return x
    mask = (1 << bits) - 1
    u = x & mask
    if dtype.startswith("ui"):
        return u
    return np.where(u >= (1 << (bits - 1)), u - (1 << bits), u)


def normalize(x, dtype: str) -> np.ndarray:
    """Round / wrap an array to the values representable in `dtype`."""
    if dtype in FLOAT:
        return numerics.round_to(np.asarray(x, dtype=np.float64), dtype)
    return wrap_int(np.asarray(x), dtype)


def from_raw(raw: np.ndarray, dtype: str) -> np.ndarray:
    """PJRT buffer contents (bf16/f8 as raw bits) → oracle values."""
    raw = np.asarray(raw)
    if dtype in ("bf16", "f16", "f8E4M3FN", "f8E5M2"):
        return numerics.decode_bits(raw, dtype)
    if dtype in ("f32", "f64"):
        return raw.astype(np.float64)
    return wrap_int(raw.astype(np.int64), dtype)


def to_raw(x: np.ndarray, dtype: str) -> np.ndarray:
    """Oracle values → PJRT buffer contents."""
    if dtype in ("bf16", "f16", "f8E4M3FN", "f8E5M2"):
        return numerics.encode_bits(x, dtype)
    np_t = {"f32": np.float32, "f64": np.float64, "i1": np.bool_, "i8": np.int8, "i16": np.int16, "i32": np.int32,
            "i64": np.int64, "ui8": np.uint8, "ui16": np.uint16, "ui32": np.uint32, "ui64": np.uint64}[dtype]
    return np.asarray(x).astype(np_t)


def _dense(payload: str, shape, dtype: str) -> np.ndarray:
    p = payload.strip()
    n = int(np.prod(shape)) if shape else 1
    if p.startswith('"0x'):
        raw = bytes.fromhex(p[3:-1])
        np_bits = {"bf16": np.uint16, "f16": np.uint16, "f8E4M3FN": np.uint8, "f8E5M2": np.uint8, "f32": np.float32,
                   "f64": np.float64, "i8": np.int8, "i16": np.int16, "i32": np.int32, "i64": np.int64,
                   "i1": np.uint8}[dtype]
        arr = np.frombuffer(raw, dtype=np_bits)
        vals = from_raw(arr, dtype) if dtype not in ("i1",) else arr.astype(np.int64)
        return np.broadcast_to(vals, (n,)).reshape(shape).copy() if vals.size in (1, n) else vals.reshape(shape)
    toks = [t for t in re.split(r"[\[\],\s]+", p) if t]
    out = []
    for t in toks:
        if t.startswith("0x") or t.startswith("0X"):
            bits = int(t, 16)
            if dtype == "f32":
                out.append(float(np.array([bits], dtype=np.uint32).view(np.float32)[0]))
            elif dtype == "f64":
                out.append(float(np.array([bits], dtype=np.uint64).view(np.float64)[0]))
            elif dtype in ("bf16", "f16", "f8E4M3FN", "f8E5M2"):
                out.append(float(numerics.decode_bits(np.array([bits]), dtype)[0]))
            else:
                out.append(bits)
        elif t in ("true", "false"):
            out.append(1 if t == "true" else 0)
        elif dtype in FLOAT:
            out.append(float(t))
        else:
            out.append(int(float(t)) if any(c in t for c in ".eE") else int(t))
    arr = np.array(out, dtype=np.float64 if dtype in FLOAT else np.int64)
    if arr.size == 1:
        arr = np.broadcast_to(arr.reshape(()), shape).copy()
    return normalize(arr.reshape(shape), dtype)


# ----------------------------------------------------------------------------------------------- parsing
class Module:
    def __init__(self, text: str, entry: str = "main"):
        m = re.search(r"func\.func\s+(?:public\s+|private\s+)?@" + re.escape(entry) + r"\s*\((.*?)\)\s*->", text, re.S)
        if not m:
            raise ValueError(f"no func.func @{entry}")
        self.params: List[Tuple[str, Tuple[int, ...], str]] = []
        for a in re.finditer(r"(%[\w.$-]+)\s*:\s*(tensor<[^>]*>)", m.group(1)):
            shape, dt = parse_type(a.group(2))
            self.params.append((a.group(1), shape, dt))
        body = text[m.end():]
        body = body[body.index("{") + 1:]
        self.stmts = self._statements(body)

    @staticmethod
    def _statements(body: str) -> List[str]:
        out, lines = [], body.split("\n")
        i = 0
        while i < len(lines):
            ln = lines[i].strip()
            i += 1
            if not ln or ln.startswith("//") or ln == "}":
                continue
            if "reducer(" in ln or (ln.startswith("%") and "stablehlo.reduce(" in ln and "applies" not in ln):
                # pretty region form: collect up to the closing brace of the reducer block (line breaks kept)
                block = [ln]
                while "}" not in lines[i - 1] or len(block) == 1:
                    block.append(lines[i].strip())
                    i += 1
                    if block[-1].startswith("}"):
                        break
                out.append("\n".join(block))
                continue
            if ln.startswith("%") and ln.endswith("({"):
                # generic region form (reduce, map): up to the line that closes the region, `}) ... : (...) -> (...)`
                block = [ln]
                while not block[-1].startswith("})"):
                    block.append(lines[i].strip())
                    i += 1
                out.append("\n".join(block))
                continue
            out.append(ln)
        return out


_BIN = {"add", "subtract", "multiply", "divide", "maximum", "minimum", "and", "or", "xor", "power", "remainder"}
_UN = {"exponential", "log", "rsqrt", "sqrt", "tanh", "logistic", "negate", "abs", "not", "floor", "ceil", "sign",
       "exponential_minus_one", "log_plus_one"}


def evaluate(text: str, inputs: Sequence[np.ndarray], dot_precision: str = "f64") -> List[Tuple[np.ndarray, str]]:
    """Runs `func.func @main` on `inputs` (oracle values, see from_raw); returns [(values, dtype)] per result.

    dot_precision "f64" accumulates floating dots in float64 (parity checks); "f32" multiplies and accumulates in
    float32 the way XLA's CPU backend upcasts bf16 dots to an f32 GEMM (used only for the timed CPU baseline)."""
    mod = Module(text)
    if len(inputs) != len(mod.params):
        raise ValueError(f"expected {len(mod.params)} inputs, got {len(inputs)}")
    env: Dict[str, Tuple[np.ndarray, str]] = {}
    for (name, shape, dt), x in zip(mod.params, inputs):
        x = np.asarray(x)
        if tuple(x.shape) != tuple(shape):
            raise ValueError(f"{name}: expected shape {shape}, got {x.shape}")
        env[name] = (x, dt)
    out = _run(mod.stmts, env, dot_precision)
    if out is None:
        raise ValueError("function has no return")
    return out


def _run(stmts, env, dot_precision: str):
    """Evaluates statements into `env` up to a return; returns the returned values (None without a return)."""
    for st in stmts:
        r = _RET.match(st)
        if r:
            names = re.findall(r"%[\w.$#-]+", r.group(1))
            return [env[n] for n in names]
        m = re.match(r"(%[\w.$-]+)(?::\d+)?\s*=\s*(?:stablehlo|mhlo)\.(\w+)\s*(.*)$", st, re.S)
        if m:
            res, op, rest = m.group(1), m.group(2), m.group(3)
        else:
            # the generic form `%r = "stablehlo.op"(%a, %b) <{attrs}> : (types) -> type`, handed on as
            # `%a, %b <{attrs}> : (types) -> type`
            m = re.match(r'(%[\w.$-]+)(?::\d+)?\s*=\s*"(?:stablehlo|mhlo)\.(\w+)"\((.*?)\)\s*(.*)$', st, re.S)
            if not m:
                raise ValueError(f"cannot parse statement: {st}")
            res, op, rest = m.group(1), m.group(2), m.group(3) + " " + m.group(4)
        val = _eval_op(op, rest, env, dot_precision)
        if isinstance(val, list):  # a multi-result op (`%r:2 = ...`): %r#0, %r#1, ...
            for k, v in enumerate(val):
                env[f"{res}#{k}"] = v
        else:
            env[res] = val
    return None


_RET = re.compile(r'(?:func\.|stablehlo\.|"stablehlo\.)?return"?\s*\(?\s*(.*?)\)?(?:\s*:\s*.*)?$')


def _operands(rest: str, n: int, env) -> List[Tuple[np.ndarray, str]]:
    names = re.findall(r"%[\w.$#-]+", rest.split(":")[0])[:n]
    return [env[x] for x in names]


def _gather(rest: str, env, out_shape) -> Tuple[np.ndarray, str]:
    """gather (manipulation.rs:1235-1307), element by element as the StableHLO specification defines it: for result
    index i, batch_dims = the result dims not in offset_dims; the start-indices coordinate is i's batch coordinates
    with the index vector dim inserted; full_start_index[start_index_map[k]] = clamp(index_vector[k], 0,
    dim - slice_sizes); full_batching_index[operand_batching_dims[j]] = the batch coordinate of
    start_indices_batching_dims[j]; full_offset_index = i's offset coordinates placed on the operand dims that are
    neither collapsed nor batching, in order; operand index = the sum of the three."""
    head = rest.split("<{")[0]
    names = re.findall(r"%[\w.$-]+", head)
    (x, dt), (ix, idt) = env[names[0]], env[names[1]]
    x, ix = np.asarray(x), np.asarray(ix)
    attrs = rest[rest.index("<{"):rest.rindex("}>")]
    dn = re.search(r"#stablehlo\.gather<(.*?)>", attrs, re.S).group(1)

    def field(name):
        m = re.search(name + r"\s*=\s*\[(.*?)\]", dn)
        return _ints(m.group(1)) if m else []

    offset_dims, collapsed = field("offset_dims"), field("collapsed_slice_dims")
    op_batch, idx_batch = field("operand_batching_dims"), field("start_indices_batching_dims")
    start_map = field("start_index_map")
    ivd = int(re.search(r"index_vector_dim\s*=\s*(\d+)", dn).group(1))
    sizes = _ints(re.search(r"slice_sizes\s*=\s*array<i64:(.*?)>", attrs).group(1))
    if idt.startswith("ui"):
        ix = ix.astype(object) % (1 << INT_BITS[idt])
    out = np.empty(out_shape, dtype=x.dtype)
    batch_dims = [d for d in range(len(out_shape)) if d not in offset_dims]
    offset_operand = [d for d in range(x.ndim) if d not in collapsed and d not in op_batch]
    for i in np.ndindex(*out_shape):
        bi = [i[d] for d in batch_dims]
        if ivd < ix.ndim:
            vec = [ix[tuple(bi[:ivd] + [k] + bi[ivd:])] for k in range(ix.shape[ivd])]
        else:
            vec = [ix[tuple(bi)]]
        idx = [0] * x.ndim
        for k, d in enumerate(start_map):
            idx[d] += min(max(int(vec[k]), 0), x.shape[d] - sizes[d])
        for d_op, d_start in zip(op_batch, idx_batch):
            idx[d_op] += bi[d_start - (0 if d_start < ivd else 1)]
        for k, d in enumerate(offset_dims):
            idx[offset_operand[k]] += i[d]
        out[i] = x[tuple(idx)]
    return out, dt


def _region_fn(rest: str, dot_precision: str):
    """The one-block region of a generic op (`({ ^bb0(%a: T, %b: T): ... stablehlo.return %r : T })`) as a function
    of its block arguments ((values, dtype) pairs; values may be whole arrays), evaluated with this module's ops."""
    region = rest[rest.index("^bb"):rest.rindex("})")]
    first, _, body = region.partition("\n")
    args = re.findall(r"(%[\w.$-]+)\s*:", first[:first.index(")")])

    def fn(*vals):
        benv = dict(zip(args, vals))
        for ln in body.split("\n"):
            ln = ln.strip()
            if not ln:
                continue
            rm = re.match(r'"?stablehlo\.return"?\s*\(?(.*?)\)?\s*:', ln)
            if rm:
                return benv[re.findall(r"%[\w.$-]+", rm.group(1))[0]]
            m = re.match(r"(%[\w.$-]+)\s*=\s*(?:stablehlo|mhlo)\.(\w+)\s*(.*)$", ln)
            if m:
                benv[m.group(1)] = _eval_op(m.group(2), m.group(3), benv, dot_precision)
            else:
                m = re.match(r'(%[\w.$-]+)\s*=\s*"(?:stablehlo|mhlo)\.(\w+)"\((.*?)\)\s*(.*)$', ln)
                benv[m.group(1)] = _eval_op(m.group(2), m.group(3) + " " + m.group(4), benv, dot_precision)
        raise ValueError("region without a return")
    return fn


def _scatter(rest: str, env, dot_precision: str) -> Tuple[np.ndarray, str]:
    """scatter (manipulation.rs:1614-1690), one input, as the StableHLO specification defines it: for each scatter
    position (the updates' dims other than update_window_dims, in row-major order — the order XLA's CPU backend
    applies them in, which is what fixes the result when windows overlap), start = the index vector placed on
    scatter_dims_to_operand_dims plus the position's batching coordinates on input_batching_dims; the update window
    (the update_window_dims, walking the operand's non-inserted, non-batching dims in order) is combined into the
    result with the update computation (current value first). A window that does not lie inside the operand in every
    dimension is skipped whole (XLA's choice; the specification leaves out-of-bounds updates implementation-defined)."""
    head = rest.split("<{")[0]
    names = re.findall(r"%[\w.$#-]+", head)
    (x, dt), (ix, idt), (u, _) = env[names[0]], env[names[1]], env[names[2]]
    x, ix, u = np.asarray(x), np.asarray(ix), np.asarray(u)
    attrs = rest[rest.index("<{"):rest.index("}>")]
    dn = re.search(r"#stablehlo\.scatter<(.*?)>", attrs, re.S).group(1)

    def field(name):
        m = re.search(name + r"\s*=\s*\[(.*?)\]", dn)
        return _ints(m.group(1)) if m else []

    uwd, inserted = field("update_window_dims"), field("inserted_window_dims")
    in_batch, idx_batch = field("input_batching_dims"), field("scatter_indices_batching_dims")
    to_operand = field("scatter_dims_to_operand_dims")
    ivd = int(re.search(r"index_vector_dim\s*=\s*(\d+)", dn).group(1))
    fn = _region_fn(rest, dot_precision)
    if idt.startswith("ui"):
        ix = ix.astype(object) % (1 << INT_BITS[idt])
    out = x.copy()
    scatter_dims = [d for d in range(u.ndim) if d not in uwd]
    window_operand = [d for d in range(x.ndim) if d not in inserted and d not in in_batch]
    win = [1] * x.ndim
    for k, d in enumerate(uwd):
        win[window_operand[k]] = u.shape[d]
    for si in np.ndindex(*[u.shape[d] for d in scatter_dims]):
        si = list(si)
        if ivd < ix.ndim:
            vec = [ix[tuple(si[:ivd] + [k] + si[ivd:])] for k in range(ix.shape[ivd])]
        else:
            vec = [ix[tuple(si)]]
        start = [0] * x.ndim
        for k, d in enumerate(to_operand):
            start[d] += int(vec[k])
        for d_op, d_idx in zip(in_batch, idx_batch):
            start[d_op] += si[d_idx - (0 if d_idx < ivd else 1)]
        if any(start[d] < 0 or start[d] + win[d] > x.shape[d] for d in range(x.ndim)):
            continue
        usl = [slice(None)] * u.ndim
        for k, d in enumerate(scatter_dims):
            usl[d] = si[k]
        uw = u[tuple(usl)]  # the window, in update_window_dims order = the window operand dims' order
        osl = tuple(slice(start[d], start[d] + win[d]) for d in range(x.ndim))
        cur = out[osl].reshape(uw.shape)
        new, _ = fn((cur, dt), (uw, dt))
        out[osl] = np.broadcast_to(normalize(np.asarray(new), dt), uw.shape).reshape(out[osl].shape)
    return out, dt


def _eval_op(op: str, rest: str, env, dot_precision: str) -> Tuple[np.ndarray, str]:
    ty = rest[rest.rfind(":"):] if ":" in rest else ""
    if op == "constant":
        # miscellaneous.rs:16-60
        m = re.match(r"dense<(.*)>\s*:\s*(tensor<.*>)$", rest)
        shape, dt = parse_type(m.group(2))
        return _dense(m.group(1), shape, dt), dt
    if op == "iota":
        # miscellaneous.rs:67-130: element = its index along `dim`
        m = re.match(r"dim\s*=\s*(\d+)\s*:\s*(tensor<.*>)", rest)
        shape, dt = parse_type(m.group(2))
        d = int(m.group(1))
        idx = np.arange(shape[d]).reshape([-1 if i == d else 1 for i in range(len(shape))])
        return normalize(np.broadcast_to(idx, shape), dt), dt
    out_shape, out_dt = _types(ty)[-1]
    if op == "convert":
        # casting.rs:75-122: float→float rounds to nearest even; float→int truncates toward zero (saturating, NaN→0
        # here: out-of-range results are implementation-defined); int→float rounds; anything→i1 is x != 0.
        (x, dt), = _operands(rest, 1, env)
        if out_dt == "i1":
            return (np.asarray(x) != 0).astype(np.int64), out_dt
        if out_dt in FLOAT:
            return normalize(np.asarray(x, dtype=np.float64), out_dt), out_dt
        if dt in FLOAT:
            bits = INT_BITS[out_dt]
            lo, hi = (0, (1 << bits) - 1) if out_dt.startswith("ui") else (-(1 << (bits - 1)), (1 << (bits - 1)) - 1)
            xf = np.nan_to_num(np.trunc(np.asarray(x, dtype=np.float64)), nan=0.0)
            return np.clip(xf, lo, hi).astype(np.int64), out_dt
        return wrap_int(x, out_dt), out_dt
    if op == "broadcast_in_dim":
        # manipulation.rs:271-338: result[i] = operand[j] with j_k = i[dims[k]] (or 0 where the operand dim is 1)
        m = re.match(r"(%[\w.$-]+)\s*,\s*dims\s*=\s*\[(.*?)\]", rest)
        x, dt = env[m.group(1)]
        dims = _ints(m.group(2))
        view = np.asarray(x).reshape([x.shape[k] for k in range(x.ndim)])
        shape_in = [1] * len(out_shape)
        for k, d in enumerate(dims):
            shape_in[d] = x.shape[k]
        order = np.argsort(dims) if dims else []
        moved = np.transpose(view, order) if len(dims) > 1 else view
        return np.broadcast_to(moved.reshape(shape_in), out_shape).copy(), dt
    if op == "transpose":
        # manipulation.rs:76-133: result dim i = operand dim perm[i]
        m = re.match(r"(%[\w.$-]+)\s*,\s*dims\s*=\s*\[(.*?)\]", rest)
        x, dt = env[m.group(1)]
        return np.transpose(x, _ints(m.group(2))).copy(), dt
    if op == "reshape":
        (x, dt), = _operands(rest, 1, env)
        return np.asarray(x).reshape(out_shape), dt
    if op == "slice":
        # manipulation.rs:840-917: result[i] = operand[start + i·stride] for start ≤ index < limit, per dimension
        m = re.match(r"(%[\w.$-]+)\s*\[(.*?)\]", rest)
        x, dt = env[m.group(1)]
        sl = []
        for part in [p for p in m.group(2).split(",") if p.strip()]:
            f = [int(v) for v in part.split(":")]
            sl.append(slice(f[0], f[1], f[2] if len(f) > 2 else 1))
        return np.asarray(x)[tuple(sl)].copy(), dt
    if op in ("dynamic_slice", "dynamic_update_slice"):
        # manipulation.rs:943-1130: the window starts at clamp(0, start_indices, shape(operand) - window) per
        # dimension (window = slice_sizes, or the update's shape); dynamic_slice returns it, dynamic_update_slice
        # returns the operand with the window replaced by the update
        head = rest.split(":")[0]
        names = re.findall(r"%[\w.$-]+", head)
        x, dt = env[names[0]]
        x = np.asarray(x)
        upd = op == "dynamic_update_slice"
        if upd:
            u = np.asarray(env[names[1]][0])
            win = list(u.shape)
        else:
            win = _ints(re.search(r"sizes\s*=\s*\[(.*?)\]", head).group(1))
        starts = []
        for nm_ in names[2 if upd else 1:]:
            v, idt = env[nm_]
            v = int(np.asarray(v).reshape(()))
            if idt.startswith("ui"):  # unsigned: the stored value modulo 2^bits
                v %= 1 << INT_BITS[idt]
            starts.append(v)
        assert len(starts) == x.ndim and len(win) == x.ndim
        sl = tuple(slice(a, a + k) for a, k in ((min(max(v, 0), x.shape[d] - win[d]), win[d])
                                                for d, v in enumerate(starts)))
        if not upd:
            return x[sl].copy(), dt
        out = x.copy()
        out[sl] = u
        return out, dt
    if op == "gather":
        return _gather(rest, env, out_shape)
    if op == "reverse":
        # miscellaneous.rs:309-370: result[i] = operand[i with each listed dim d read from the end]
        (x, dt), = _operands(rest, 1, env)
        dm = re.search(r"(?:dims|dimensions)\s*=\s*(array<[^>]*>|\[[^\]]*\])", rest)
        dims = _ints(dm.group(1).split(":", 1)[1] if dm.group(1).startswith("array") else dm.group(1))
        return np.flip(np.asarray(x), axis=tuple(dims)).copy(), dt
    if op == "optimization_barrier":
        # miscellaneous.rs:405-450: the identity on each operand
        names = re.findall(r"%[\w.$#-]+", rest.split(":")[0])
        vals = [env[n] for n in names]
        return vals if len(vals) > 1 else vals[0]
    if op in ("if", "case"):
        # control_flow.rs: the branch the predicate picks (case: the one at the index, the last one for an index
        # outside the branches), its ops evaluated in the enclosing scope
        (sel, _), = _operands(rest, 1, env)
        body = rest[rest.index("({") + 2:rest.rindex("})")]
        branches = re.split(r"\n\s*\},\s*\{\s*(?=\n)", body)
        if op == "if":
            k = 0 if bool(np.asarray(sel)) else 1
        else:
            k = int(np.asarray(sel))
            k = k if 0 <= k < len(branches) else len(branches) - 1
        vals = _run(Module._statements(branches[k] + "\n"), dict(env), dot_precision)
        return vals if len(vals) != 1 else vals[0]
    if op == "get_dimension_size":
        # manipulation.rs:12-40: the extent of dimension `dim`, an i32 scalar
        (x, _), = _operands(rest, 1, env)
        d = int(re.search(r"dim(?:ension)?\s*=\s*(\d+)", rest).group(1))
        return np.array(np.shape(x)[d]), "i32"
    if op in ("replica_id", "partition_id"):
        # communication.rs:110-190: the id of the one replica / partition, 0
        return np.zeros((), np.int64), "ui32"
    if op == "reduce_precision":
        # casting.rs:259-300, on the element's own bits as XLA's emitter does: the mantissa rounded to m bits (ties to
        # even, a carry moving into the exponent), then exponents the e-bit format cannot hold overflow to ±inf or
        # underflow to ±0 (its subnormals included); NaN unchanged
        (x, dt), = _operands(rest, 1, env)
        fm = re.search(r"format\s*=\s*e(\d+)m(\d+)", rest)
        if fm:
            e, m = int(fm.group(1)), int(fm.group(2))
        else:
            e = int(re.search(r"exponent_bits\s*=\s*(\d+)", rest).group(1))
            m = int(re.search(r"mantissa_bits\s*=\s*(\d+)", rest).group(1))
        sm, se, width = {"f32": (23, 8, 32), "bf16": (7, 8, 16), "f16": (10, 5, 16)}[dt]
        xv = np.asarray(x)
        raw0 = np.asarray(to_raw(xv, dt))
        bits = (raw0.view(np.uint32) if dt == "f32" else raw0).astype(np.int64)  # the element's bits
        if m < sm:
            shift = sm - m
            last = 1 << shift
            bits = (bits + ((bits & last) >> shift) + ((last >> 1) - 1)) & ~(last - 1)
        if e < se:
            exp_mask, sign = ((1 << se) - 1) << sm, 1 << (sm + se)
            bias, rbias = (1 << (se - 1)) - 1, (1 << (e - 1)) - 1
            xe = bits & exp_mask
            bits = np.where(xe > ((bias + rbias) << sm), (bits & sign) | exp_mask,
                            np.where(xe <= ((bias - rbias) << sm), bits & sign, bits))
        bits &= (1 << width) - 1
        raw = bits.astype(np.uint32).view(np.float32) if width == 32 else bits.astype(np.uint16)
        out = np.asarray(from_raw(raw, dt), dtype=np.float64).reshape(xv.shape)
        return np.where(np.isnan(xv), xv, out), dt
    if op == "bitcast_convert":
        # casting.rs:8-73 (same element width): the element's bits reread as the result type
        (x, dt), = _operands(rest, 1, env)
        raw = np.ascontiguousarray(to_raw(np.asarray(x), dt))
        want = {"f32": np.float32, "i32": np.int32, "ui32": np.uint32, "bf16": np.uint16, "f16": np.uint16,
                "i16": np.int16, "ui16": np.uint16, "f8E4M3FN": np.uint8, "f8E5M2": np.uint8, "i8": np.int8,
                "ui8": np.uint8}[out_dt]
        if raw.dtype.itemsize != np.dtype(want).itemsize:
            raise NotImplementedError("bitcast_convert between widths")
        return from_raw(raw.view(want), out_dt), out_dt
    if op == "map":
        # functional.rs:13-104: the body applied to the inputs' elements (here to whole arrays at once)
        names = re.findall(r"%[\w.$-]+", rest[:rest.index("(")] if "(" in rest else rest)
        v, dt = _region_fn(rest, dot_precision)(*[env[n] for n in names])
        return normalize(np.broadcast_to(np.asarray(v), out_shape), out_dt), out_dt
    if op == "scatter":
        return _scatter(rest, env, dot_precision)
    if op == "concatenate":
        # manipulation.rs:778-822: the inputs one after another along `dim`, in operand order
        head = rest.split(":")[0]
        d = int(re.search(r"dim\s*=\s*(\d+)", head).group(1))
        names = re.findall(r"%[\w.$-]+", head)
        vals = [env[x] for x in names]
        return np.concatenate([np.asarray(v) for v, _ in vals], axis=d), vals[0][1]
    if op == "pad":
        # manipulation.rs:530-560: result[lo + i·(interior + 1)] = operand[i] where that index lies in the result,
        # the padding value elsewhere (negative edge padding removes elements; interior padding comes first)
        (x, dt), (v, _) = _operands(rest, 2, env)
        lo = _ints(re.search(r"low\s*=\s*\[(.*?)\]", rest).group(1))
        hi = _ints(re.search(r"high\s*=\s*\[(.*?)\]", rest).group(1))
        it = _ints(re.search(r"interior\s*=\s*\[(.*?)\]", rest).group(1))
        x = np.asarray(x)
        pv = np.asarray(v).reshape(())
        # interior padding first, then the edges: positive edges add padding, negative ones cut elements off
        inner = np.full([k + (k - 1) * it[d] if k > 0 else 0 for d, k in enumerate(x.shape)], pv, dtype=x.dtype)
        inner[tuple(slice(None, None, it[d] + 1) for d in range(x.ndim))] = x
        cut = tuple(slice(max(0, -lo[d]), inner.shape[d] - max(0, -hi[d]) if inner.shape[d] - max(0, -hi[d]) > 0
                          else 0) for d in range(x.ndim))
        inner = inner[cut]
        out = np.pad(inner, [(max(0, lo[d]), max(0, hi[d])) for d in range(x.ndim)], constant_values=pv)
        assert list(out.shape) == list(out_shape), (out.shape, out_shape)
        return out, dt
    if op == "compare":
        # comparison.rs:44-135
        m = re.match(r"(\w+)\s*,\s*(%[\w.$-]+)\s*,\s*(%[\w.$-]+)", rest)
        if m:
            direction, an, bn = m.group(1), m.group(2), m.group(3)
        else:  # generic: `%a, %b <{comparison_direction = #stablehlo<comparison_direction GT>, ...}> : ...`
            an, bn = re.findall(r"%[\w.$-]+", rest.split("<{")[0])[:2]
            direction = re.search(r"\b(EQ|NE|GE|GT|LE|LT)\b", rest).group(1)
        a, _ = env[an]
        b, _ = env[bn]
        fn = {"EQ": np.equal, "NE": np.not_equal, "GE": np.greater_equal, "GT": np.greater, "LE": np.less_equal,
              "LT": np.less}[direction]
        return fn(a, b).astype(np.int64), "i1"
    if op == "select":
        # control_flow.rs:216-300: pred ? on_true : on_false (a scalar predicate selects whole tensors)
        (p, _), (a, dt), (b, _) = _operands(rest, 3, env)
        return np.where(np.asarray(p) != 0, a, b), dt
    if op == "clamp":
        (lo, _), (x, dt), (hi, _) = _operands(rest, 3, env)
        return normalize(np.minimum(np.maximum(x, lo), hi), dt), dt
    if op in _BIN:
        # arithmetic.rs:190-420, comparison.rs:230-297 (maximum / minimum propagate NaN)
        (a, dt), (b, _) = _operands(rest, 2, env)
        if dt in FLOAT:
            a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
            with np.errstate(all="ignore"):
                r = {"add": lambda: a + b, "subtract": lambda: a - b, "multiply": lambda: a * b,
                     "divide": lambda: a / b, "maximum": lambda: np.maximum(a, b),
                     "minimum": lambda: np.minimum(a, b), "power": lambda: np.power(a, b),
                     "remainder": lambda: np.fmod(a, b)}[op]()
            return normalize(r, dt), dt
        a, b = np.asarray(a, dtype=np.int64), np.asarray(b, dtype=np.int64)
        if op == "divide":
            with np.errstate(all="ignore"):
                r = np.where(b == 0, -1, np.trunc(a / np.where(b == 0, 1, b))).astype(np.int64)
        elif op == "remainder":
            r = np.where(b == 0, a, np.fmod(a, np.where(b == 0, 1, b)))
        else:
            r = {"add": lambda: a + b, "subtract": lambda: a - b, "multiply": lambda: a * b,
                 "maximum": lambda: np.maximum(a, b), "minimum": lambda: np.minimum(a, b),
                 "and": lambda: a & b, "or": lambda: a | b, "xor": lambda: a ^ b}[op]()
        return wrap_int(r, dt), dt
    if op in _BITS:
        return _bit_op(op, rest, env)
    if op in _FLOAT_ONLY:
        return _float_op(op, rest, env)
    if op in _UN:
        # exponential.rs (exponential :245, rsqrt :151, logistic :434), arithmetic.rs:134 (negate)
        (x, dt), = _operands(rest, 1, env)
        if dt not in FLOAT:
            x = np.asarray(x, dtype=np.int64)
            r = {"negate": lambda: -x, "abs": lambda: np.abs(x), "sign": lambda: np.sign(x),
                 "not": lambda: (x == 0).astype(np.int64) if dt == "i1" else ~x}[op]()
            return wrap_int(r, dt), dt
        x = np.asarray(x, dtype=np.float64)
        with np.errstate(all="ignore"):
            r = {"exponential": lambda: np.exp(x), "log": lambda: np.log(x), "rsqrt": lambda: 1.0 / np.sqrt(x),
                 "sqrt": lambda: np.sqrt(x), "tanh": lambda: np.tanh(x),
                 "logistic": lambda: 1.0 / (1.0 + np.exp(-x)), "negate": lambda: -x, "abs": lambda: np.abs(x),
                 "floor": lambda: np.floor(x), "ceil": lambda: np.ceil(x),
                 # arithmetic.rs:15-25: NaN and signed zeros are their own sign
                 "sign": lambda: np.where(np.isnan(x) | (x == 0), x, np.sign(x)),
                 "exponential_minus_one": lambda: np.expm1(x), "log_plus_one": lambda: np.log1p(x)}[op]()
        return normalize(r, dt), dt
    if op == "dot_general":
        return _dot_general(rest, env, out_shape, out_dt, dot_precision)
    if op == "reduce":
        return _reduce(rest, env, out_shape, out_dt)
    raise NotImplementedError(f"stablehlo.{op}")


_BITS = {"shift_left", "shift_right_arithmetic", "shift_right_logical", "popcnt", "count_leading_zeros"}
_FLOAT_ONLY = {"sine", "cosine", "tan", "cbrt", "round_nearest_even", "round_nearest_afz", "is_finite", "atan2"}


def _bit_op(op, rest, env):
    """bit_manipulation.rs:5-280 on the two's complement bits of each element at its own width w: shift_left and
    shift_right_logical give 0 and shift_right_arithmetic the sign fill when the shift amount, read as a w-bit
    unsigned integer, is at least w; popcnt counts the set bits and count_leading_zeros the zero bits above the
    highest set one (w for 0)."""
    n = 2 if op.startswith("shift") else 1
    vals = _operands(rest, n, env)
    dt = vals[0][1]
    w = INT_BITS[dt]
    full = (1 << w) - 1 if w < 64 else 0xFFFFFFFFFFFFFFFF
    mask = np.uint64(full)
    u = np.asarray(vals[0][0], dtype=np.int64).view(np.uint64) & mask
    if op == "popcnt":
        return wrap_int(np.bitwise_count(u).astype(np.int64), dt), dt
    if op == "count_leading_zeros":
        length = np.zeros(u.shape, dtype=np.int64)
        v = u.copy()
        for k in (32, 16, 8, 4, 2, 1):
            big = v >= np.uint64(1 << k)
            v = np.where(big, v >> np.uint64(k), v)
            length += np.where(big, k, 0)
        length += (v > 0).astype(np.int64)
        return wrap_int(w - length, dt), dt
    amount = np.asarray(vals[1][0], dtype=np.int64).view(np.uint64) & mask
    inside = amount < np.uint64(w)
    s = np.where(inside, amount, np.uint64(0)).astype(np.uint64)
    if op == "shift_left":
        r = ((u << s) & mask).view(np.int64)
        r = np.where(inside, r, 0)
    elif op == "shift_right_logical":
        r = np.where(inside, (u >> s).view(np.int64), 0)
    else:
        signed = u.view(np.int64) if w == 64 else np.where(u >= np.uint64(1 << (w - 1)), u.astype(np.int64) - (1 << w),
                                                                   u.astype(np.int64))
        r = np.where(inside, signed >> s.astype(np.int64), np.where(signed < 0, -1, 0))
    return wrap_int(np.asarray(r, dtype=np.int64), dt), dt


def _float_op(op, rest, env):
    """trigonometric.rs:7-155, 203-262 (sine, cosine, tan, atan2), exponential.rs:166-210 (cbrt),
    rounding.rs:91-180 (round_nearest_afz: ties away from zero; round_nearest_even: ties to even),
    arithmetic.rs:470-515 (is_finite: i1, false for infinities and NaN)."""
    vals = _operands(rest, 2 if op == "atan2" else 1, env)
    dt = vals[0][1]
    x = np.asarray(vals[0][0], dtype=np.float64)
    if op == "is_finite":
        return np.isfinite(x).astype(np.int64), "i1"
    with np.errstate(all="ignore"):
        if op == "atan2":
            r = np.arctan2(x, np.asarray(vals[1][0], dtype=np.float64))
        elif op == "round_nearest_afz":
            t = np.trunc(x)
            r = np.where(np.abs(x - t) >= 0.5, t + np.sign(x), t)
        else:
            r = {"sine": np.sin, "cosine": np.cos, "tan": np.tan, "cbrt": np.cbrt, "round_nearest_even": np.rint}[op](x)
    return normalize(r, dt), dt


def _dot_general(rest, env, out_shape, out_dt, dot_precision):
    """linear_algebra.rs:561-705: transpose each operand to batch + free + contracting dims, flatten, multiply, and
    sum over the contracting dims; result dims are batch, lhs free, rhs free."""
    m = re.match(r"(%[\w.$-]+)\s*,\s*(%[\w.$-]+)\s*,(.*)", rest)
    (a, adt), (b, bdt) = env[m.group(1)], env[m.group(2)]
    attrs = m.group(3)
    bm = re.search(r"batching_dims\s*=\s*\[(.*?)\]\s*x\s*\[(.*?)\]", attrs)
    cm = re.search(r"contracting_dims\s*=\s*\[(.*?)\]\s*x\s*\[(.*?)\]", attrs)
    lb, rb = (_ints(bm.group(1)), _ints(bm.group(2))) if bm else ([], [])
    lc, rc = _ints(cm.group(1)), _ints(cm.group(2))
    a, b = np.asarray(a), np.asarray(b)
    lf = [d for d in range(a.ndim) if d not in lb and d not in lc]
    rf = [d for d in range(b.ndim) if d not in rb and d not in rc]
    at = np.transpose(a, lb + lf + lc)
    bt = np.transpose(b, rb + rc + rf)
    nb = int(np.prod([a.shape[d] for d in lb])) if lb else 1
    M = int(np.prod([a.shape[d] for d in lf])) if lf else 1
    K = int(np.prod([a.shape[d] for d in lc])) if lc else 1
    N = int(np.prod([b.shape[d] for d in rf])) if rf else 1
    A3, B3 = at.reshape(nb, M, K), bt.reshape(nb, K, N)
    if out_dt in FLOAT:
        if dot_precision == "f32":
            r = np.matmul(A3.astype(np.float32), B3.astype(np.float32)).astype(np.float64)
        else:
            r = np.matmul(A3.astype(np.float64), B3.astype(np.float64))
        return normalize(r.reshape(out_shape), out_dt), out_dt
    # integers: exact in float64 while |sum| < 2^53 (|acc| ≤ K·127² for i8), else int64 loop
    if K * float(np.max(np.abs(A3), initial=0)) * float(np.max(np.abs(B3), initial=0)) < 2.0 ** 52:
        r = np.rint(np.matmul(A3.astype(np.float64), B3.astype(np.float64))).astype(np.int64)
    else:
        r = np.einsum("bmk,bkn->bmn", A3.astype(np.int64), B3.astype(np.int64))
    return wrap_int(r.reshape(out_shape), out_dt), out_dt


def _reduce(rest, env, out_shape, out_dt):
    """functional.rs:109-230: reduce `dimensions` of N inputs together, starting from their N init values, with the
    body; the combination order is implementation-defined. One input with a single-op body (`applies`, or a region
    applying one op to its two arguments): numpy's reduction of the whole axis set (sums exact as float64, rounded
    once). Otherwise (several inputs, e.g. argmax's (value, index) pairs, or a longer body): the body's statements
    are evaluated element by element in index order over the reduced dims, acc = body(acc, x), acc starting at the
    init values. Returns one (values, dtype) per result (a list when N > 1)."""
    head = rest.split("\n")[0]
    pairs = re.findall(r"\((%[\w.$-]+)\s+init:\s*(%[\w.$-]+)\)", head)
    applies = re.search(r"applies\s+stablehlo\.(\w+)", head)
    if pairs:  # pretty form
        inputs, inits = [p[0] for p in pairs], [p[1] for p in pairs]
        dims = tuple(_ints(re.search(r"across\s+dimensions\s*=\s*\[(.*?)\]", head).group(1)))
        types = _types(head[head.index(":"):])
        region = None if applies else rest[rest.index("reducer"):]
    else:  # generic form: `%a, %b, %c, %d <{dimensions = ...}> ({ ^bb0(...): ... }) : (...) -> (...)`
        names = re.findall(r"%[\w.$-]+", rest[:rest.index("(")] if "(" in rest else rest)
        inputs, inits = names[:len(names) // 2], names[len(names) // 2:]
        dm = re.search(r"dimensions\s*=\s*(array<[^>]*>|dense<[^>]*>|\[[^\]]*\])", rest)
        dims = tuple(_ints(dm.group(1).split(":", 1)[1] if dm.group(1).startswith("array") else dm.group(1)))
        types = _types(rest[rest.rindex("})"):])
        region = rest[rest.index("^bb"):rest.rindex("})")]
    n = len(inputs)
    res_types = types[-n:]
    body = _region(region, n) if region is not None else None
    single = applies.group(1) if applies else (body[2] if body is not None and n == 1 else None)
    if n == 1 and single in ("add", "multiply", "maximum", "minimum", "and", "or"):
        x, dt = env[inputs[0]]
        return _reduce_single(single, np.asarray(x), dt, np.asarray(env[inits[0]][0]).reshape(()), dims,
                              res_types[0][1])
    args, stmts, _, rets = body
    xs, accs = [], []
    for i in range(n):
        x, dt = env[inputs[i]]
        x = np.asarray(x)
        kept = [d for d in range(x.ndim) if d not in dims]
        x = np.transpose(x, kept + sorted(dims))
        shape = x.shape[:len(kept)]
        xs.append((x.reshape(shape + (-1,)), dt))
        accs.append((np.broadcast_to(np.asarray(env[inits[i]][0]).reshape(()), shape).copy(), dt))
    for r in range(xs[0][0].shape[-1]):
        benv = dict(zip(args, accs + [(x[..., r], dt) for x, dt in xs]))
        for st in stmts:
            m = re.match(r"(%[\w.$-]+)\s*=\s*(?:stablehlo|mhlo)\.(\w+)\s*(.*)$", st, re.S)
            if m:
                benv[m.group(1)] = _eval_op(m.group(2), m.group(3), benv, "f64")
                continue
            m = re.match(r'(%[\w.$-]+)\s*=\s*"(?:stablehlo|mhlo)\.(\w+)"\((.*?)\)\s*(.*)$', st, re.S)
            benv[m.group(1)] = _eval_op(m.group(2), m.group(3) + " " + m.group(4), benv, "f64")
        accs = [(np.asarray(benv[v][0]), res_types[i][1]) for i, v in enumerate(rets)]
    out = [(normalize(np.asarray(a), dt), dt) for a, dt in accs]
    return out if n > 1 else out[0]


def _region(text, n):
    """A reduce body: (block arguments in order, body statements, the single op of a one-op body or None, returned
    names). Pretty `reducer(%a0: T, %b0: T) (%a1: U, %b1: U) { ... }` lists one (first, second) pair per input: the
    block arguments are the pairs' first members, then their second members. Generic `^bb0(%x: T, ...): ...`."""
    first_line, _, body = text.partition("\n")
    if text.startswith("reducer"):
        pairs = re.findall(r"\((%[\w.$-]+)\s*:\s*tensor<[^>]*>\s*,\s*(%[\w.$-]+)\s*:\s*tensor<[^>]*>\)", first_line)
        args = [p[0] for p in pairs] + [p[1] for p in pairs]
    else:
        args = re.findall(r"(%[\w.$-]+)\s*:", first_line[:first_line.index(")")])
    assert len(args) == 2 * n, (args, n)
    stmts, rets = [], None
    for ln in body.split("\n"):
        ln = ln.strip()
        if not ln or ln.startswith("}") or ln.startswith("{"):
            continue
        rm = re.match(r'"?stablehlo\.return"?\s*\(?(.*?)\)?\s*:', ln)
        if rm:
            rets = re.findall(r"%[\w.$-]+", rm.group(1))
            break
        stmts.append(ln)
    single = None
    if len(stmts) == 1:
        m = re.match(r'%[\w.$-]+\s*=\s*"?stablehlo\.(\w+)"?\s*\(?\s*(%[\w.$-]+)\s*,\s*(%[\w.$-]+)', stmts[0])
        if m and sorted(m.group(2, 3)) == sorted(args):
            single = m.group(1)
    return args, stmts, single, rets


def _reduce_single(body, x, dt, init, dims, out_dt):
    if dt in FLOAT:
        x = x.astype(np.float64)
        with np.errstate(all="ignore"):
            if body == "add":
                r = np.sum(x, axis=dims) + init
            elif body == "multiply":
                r = np.prod(x, axis=dims) * init
            elif body == "maximum":
                r = np.maximum(np.max(x, axis=dims, initial=-np.inf), init)
            elif body == "minimum":
                r = np.minimum(np.min(x, axis=dims, initial=np.inf), init)
            else:
                raise NotImplementedError(body)
        return normalize(r, out_dt), out_dt
    x = x.astype(np.int64)
    r = {"add": lambda: np.sum(x, axis=dims) + init, "multiply": lambda: np.prod(x, axis=dims) * init,
         "maximum": lambda: np.maximum(np.max(x, axis=dims, initial=np.iinfo(np.int64).min), init),
         "minimum": lambda: np.minimum(np.min(x, axis=dims, initial=np.iinfo(np.int64).max), init),
         "and": lambda: np.bitwise_and.reduce(x, axis=dims) & init,
         "or": lambda: np.bitwise_or.reduce(x, axis=dims) | init}[body]()
    return wrap_int(r, out_dt), out_dt


def rel_error(got: np.ndarray, want: np.ndarray) -> float:
    """Normwise relative error max|got - want| / max|want| (the tolerance metric of the parity tests)."""
    got, want = np.asarray(got, dtype=np.float64), np.asarray(want, dtype=np.float64)
    denom = float(np.max(np.abs(want))) if want.size else 0.0
    diff = float(np.max(np.abs(got - want))) if want.size else 0.0
    return diff / denom if denom > 0 else diff
