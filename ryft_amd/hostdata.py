"""Host-side data preparation: deterministic seeded inputs and bit-level encodings of narrow float types.

Inputs come from a counter-based splitmix64 stream so that every consumer (parity tests, the benchmark, the smoke
test) sees identical bytes for a given seed. Uniform floats use the top 24 bits of each draw; normals use
Box-Muller over consecutive pairs of draws. Encodings are IEEE-style round-to-nearest-even; they produce the raw
bits PJRT buffers carry for BF16 (PJRT_Buffer_Type 13) and F8E4M3FN (17), see crates/ryft-pjrt/src/buffers.rs:87-92,
134-136.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int) -> np.ndarray:
    """The first `n` outputs of splitmix64 started at `seed` (output i mixes seed + (i+1)·golden)."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (np.arange(1, n + 1, dtype=np.uint64) * _GOLDEN)
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, shape, lo: float, hi: float) -> np.ndarray:
    n = int(np.prod(shape))
    u = (splitmix64(seed, n) >> np.uint64(40)).astype(np.float64) * (1.0 / (1 << 24))
    return (lo + (hi - lo) * u).astype(np.float32).reshape(shape)


def normal(seed: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    r = splitmix64(seed, 2 * ((n + 1) // 2)) >> np.uint64(40)
    u1 = (r[0::2].astype(np.float64) + 1.0) * (1.0 / (1 << 24))  # (0, 1]
    u2 = r[1::2].astype(np.float64) * (1.0 / (1 << 24))
    rad = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * len(u1), dtype=np.float64)
    z[0::2] = rad * np.cos(2.0 * np.pi * u2)
    z[1::2] = rad * np.sin(2.0 * np.pi * u2)
    return (mean + std * z[:n]).astype(np.float32).reshape(shape)


def int_uniform(seed: int, shape, lo: int, hi: int) -> np.ndarray:
    """Integers uniform in [lo, hi] (inclusive)."""
    n = int(np.prod(shape))
    x = splitmix64(seed, n) >> np.uint64(32)
    return (lo + (x % np.uint64(hi - lo + 1)).astype(np.int64)).reshape(shape)


# ----------------------------------------------------------------------------------------------- encodings
def f32_to_bf16_bits(x) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    r = np.where(nan, (u >> np.uint32(16)) | np.uint32(0x40), r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_e4m3fn_bits(x) -> np.ndarray:
    """Round-to-nearest-even into f8E4M3FN; NaN/inf and values rounding above 448 become NaN (0x7f | sign)."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    sign = ((u >> np.uint32(24)) & np.uint32(0x80)).astype(np.uint32)
    a = u & np.uint32(0x7FFFFFFF)
    af = a.view(np.float32)
    sub = np.rint(af.astype(np.float64) * 512.0).astype(np.uint32)  # |x| < 2^-6: grid 2^-9
    with np.errstate(over="ignore"):
        r = (a + np.uint32(0x7FFFF) + ((a >> np.uint32(20)) & np.uint32(1))) >> np.uint32(20)
        norm = r.astype(np.int64) - ((127 - 7) << 3)
    code = np.where(a < np.uint32(0x3C800000), sub.astype(np.int64), norm)
    code = np.where((code > 0x7E) | (a >= np.uint32(0x7F800000)), 0x7F, code)
    return (sign | code.astype(np.uint32)).astype(np.uint8)


def e4m3fn_bits_to_f32(b) -> np.ndarray:
    b = np.asarray(b, dtype=np.uint8).astype(np.int64)
    s = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 15
    m = b & 7
    v = np.where(e == 0, m * 2.0 ** -9, (8 + m) * np.exp2(e - 10.0))
    v = np.where((b & 0x7F) == 0x7F, np.nan, v)
    return (s * v).astype(np.float32)
