"""Narrow floating-point formats for the oracle: value tables and round-to-nearest-even by search.

Formats (PJRT element types, crates/ryft-pjrt/src/buffers.rs:16-157; BF16 :134-136, F8E4M3FN :87-92):
  bf16      1-8-7, IEEE-like (inf, NaN)
  f16       1-5-10, IEEE
  f8E4M3FN  1-4-3, bias 7, no infinities, only S.1111.111 is NaN, max finite 448
  f8E5M2    1-5-2, bias 15, IEEE-like (inf, NaN)

Rounding of an f32 value x into a format: the nearest finite format value; on a tie, the one with an even code
(even mantissa); values beyond the largest finite value by at least half an ulp-of-the-next-binade become inf, or
NaN for f8E4M3FN (which has no inf). Implemented by binary search over the sorted table of finite values, which is
an independent construction from the product's bit-level conversions.
"""
from __future__ import annotations

import functools

import numpy as np


@functools.lru_cache(maxsize=None)
def table(fmt: str):
    """(codes, values) of all finite non-negative values of `fmt`, sorted by value; codes are the bit patterns."""
    if fmt == "f8E4M3FN":
        ebits, mbits, bias, ieee = 4, 3, 7, False
    elif fmt == "f8E5M2":
        ebits, mbits, bias, ieee = 5, 2, 15, True
    elif fmt == "f16":
        ebits, mbits, bias, ieee = 5, 10, 15, True
    elif fmt == "bf16":
        ebits, mbits, bias, ieee = 8, 7, 127, True
    else:
        raise ValueError(fmt)
    codes, values = [], []
    for e in range(1 << ebits):
        for m in range(1 << mbits):
            if ieee and e == (1 << ebits) - 1:
                continue  # inf / NaN
            if not ieee and e == (1 << ebits) - 1 and m == (1 << mbits) - 1:
                continue  # f8E4M3FN NaN
            if e == 0:
                v = m * 2.0 ** (1 - bias - mbits)
            else:
                v = (1.0 + m / (1 << mbits)) * 2.0 ** (e - bias)
            codes.append((e << mbits) | m)
            values.append(v)
    order = np.argsort(values, kind="stable")
    return np.array(codes, dtype=np.int64)[order], np.array(values, dtype=np.float64)[order], ebits, mbits, ieee


def _encode(x, fmt: str) -> np.ndarray:
    codes, vals, ebits, mbits, ieee = table(fmt)
    x = np.asarray(x, dtype=np.float64)
    sign = np.signbit(x)
    a = np.abs(x)
    hi_idx = np.clip(np.searchsorted(vals, a, side="left"), 0, len(vals) - 1)
    lo_idx = np.clip(hi_idx - 1, 0, len(vals) - 1)
    lo, hi = vals[lo_idx], vals[hi_idx]
    d_lo, d_hi = a - lo, hi - a
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & ((codes[hi_idx] & 1) == 0))
    idx = np.where(a <= lo, lo_idx, np.where(pick_hi, hi_idx, lo_idx))
    idx = np.where(a >= vals[-1], len(vals) - 1, idx)
    code = codes[idx]
    # overflow: at or beyond the midpoint between the max finite value and the next binade step
    maxv = vals[-1]
    step = 2.0 ** (np.floor(np.log2(maxv)) - mbits)
    # IEEE formats: the max finite value has an odd code, so the exact midpoint rounds (to even) up to inf.
    # f8E4M3FN: the value past 448 would be the NaN code 0x7f (odd), so the midpoint 464 rounds down to 448.
    over = (a >= maxv + step / 2.0) if ieee else (a > maxv + step / 2.0)
    top = (1 << (ebits + mbits)) - 1
    inf_code = (((1 << ebits) - 1) << mbits)
    nan_code = top if not ieee else inf_code | (1 << (mbits - 1))
    code = np.where(over, inf_code if ieee else nan_code, code)
    code = np.where(np.isnan(x), nan_code, code)
    code = np.where(np.isinf(x), inf_code if ieee else nan_code, code)
    nbits = 1 + ebits + mbits
    return (code | (sign.astype(np.int64) << (nbits - 1))).astype(np.int64)


def _decode(codes, fmt: str) -> np.ndarray:
    _, _, ebits, mbits, ieee = table(fmt)
    c = np.asarray(codes, dtype=np.int64)
    nbits = 1 + ebits + mbits
    s = np.where((c >> (nbits - 1)) & 1, -1.0, 1.0)
    e = (c >> mbits) & ((1 << ebits) - 1)
    m = c & ((1 << mbits) - 1)
    bias = (1 << (ebits - 1)) - 1
    v = np.where(e == 0, m * 2.0 ** (1 - bias - mbits), (1.0 + m / (1 << mbits)) * np.exp2(e - float(bias)))
    emax = (1 << ebits) - 1
    if ieee:
        v = np.where((e == emax) & (m == 0), np.inf, v)
        v = np.where((e == emax) & (m != 0), np.nan, v)
    else:
        v = np.where((e == emax) & (m == (1 << mbits) - 1), np.nan, v)
    return s * v


def round_to(x, dtype: str) -> np.ndarray:
    """Value of `x` (float64 array) after conversion to `dtype`, computed as f32 first (what an f32 datapath does),
    then narrowed; returned as float64."""
    x = np.asarray(x, dtype=np.float64)
    if dtype == "f64":
        return x
    f32 = x.astype(np.float32).astype(np.float64)
    if dtype == "f32":
        return f32
    return _decode(_encode(f32, dtype), dtype)


def encode_bits(x, dtype: str) -> np.ndarray:
    """Raw bit patterns of `x` converted to `dtype` (uint16 for bf16/f16, uint8 for f8)."""
    x32 = np.asarray(x, dtype=np.float64).astype(np.float32).astype(np.float64)
    codes = _encode(x32, dtype)
    return codes.astype(np.uint16 if dtype in ("bf16", "f16") else np.uint8)


def decode_bits(bits, dtype: str) -> np.ndarray:
    return _decode(np.asarray(bits).astype(np.int64), dtype)
