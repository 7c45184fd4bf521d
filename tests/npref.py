"""Independent numpy references used to pin the C oracle and to write the golden fixtures.

They do not share code with oracle/kvattn_oracle.c: attention is computed in float64
with vectorised numpy, bf16 rounding with integer arithmetic on the float bits, the E4M3
table is built with exact rational arithmetic from the OCP 8-bit floating point spec
(v1.0, 2023), and E4M3 encoding is a brute-force nearest-value search over that table.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np

HS = 64


def attention_f64(qkv, cache, totals, B, NH, maxT, hs=HS):
    """softmax(q K^T / sqrt(hs)) V per (b,h) over the first totals[b] positions, float64."""
    q = np.asarray(qkv, dtype=np.float64).reshape(B, 3, NH, hs)[:, 0]
    kv = np.asarray(cache, dtype=np.float64).reshape(2, B, NH, maxT, hs)
    out = np.zeros((B, NH, hs))
    for b in range(B):
        T = int(np.broadcast_to(totals, (B,))[b])
        s = np.einsum("hd,htd->ht", q[b], kv[0, b, :, :T]) / np.sqrt(hs)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        out[b] = np.einsum("ht,htd->hd", p, kv[1, b, :, :T]) / p.sum(axis=1, keepdims=True)
    return out


def bf16_round(x) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even, NaN kept quiet."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def bf16_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def e4m3_value(code: int):
    """Exact value of an OCP E4M3 ("FN") code as a Fraction, or None for NaN."""
    s, e, m = code >> 7, (code >> 3) & 0xF, code & 7
    if e == 15 and m == 7:
        return None
    v = Fraction(m, 8) * Fraction(2) ** -6 if e == 0 else (1 + Fraction(m, 8)) * Fraction(2) ** (e - 7)
    return -v if s else v


E4M3_TABLE = [e4m3_value(c) for c in range(256)]


def e4m3_encode_bruteforce(y: float) -> int:
    """Nearest finite E4M3 code to y, ties to the code with an even mantissa, saturating
    at +-448.  Zero keeps the sign of y."""
    if np.isnan(y):
        return 0x7F
    sign = 0x80 if np.signbit(y) else 0
    a = Fraction(abs(float(y)))
    if a >= 448:
        return sign | 0x7E
    best, best_d = None, None
    for code in range(0x7F):            # non-negative finite codes 0x00..0x7E
        d = abs(E4M3_TABLE[code] - a)
        if best is None or d < best_d or (d == best_d and (code & 1) == 0):
            best, best_d = code, d
    return sign | best


def int8_encode(x, scale) -> np.ndarray:
    """clamp(rint_half_even(float32(x) / float32(scale)), -127, 127) as bytes."""
    y = np.asarray(x, dtype=np.float32) / np.float32(scale)
    return np.clip(np.rint(y), -127, 127).astype(np.int8).view(np.uint8)


def quantise_row(x, fmt: str):
    """(codes uint8[64], scale float32) of one 64-element row of float32 values."""
    x = np.asarray(x, dtype=np.float32)
    limit = np.float32(448.0 if fmt == "fp8" else 127.0)
    scale = np.float32(np.abs(x).max()) / limit
    if scale == 0:
        return np.zeros(x.shape, np.uint8), np.float32(0.0)
    if fmt == "int8":
        return int8_encode(x, scale), scale
    y = x / scale
    return np.array([e4m3_encode_bruteforce(float(v)) for v in y], dtype=np.uint8), scale


def decode_w8(codes, fmt: str) -> np.ndarray:
    codes = np.asarray(codes, dtype=np.uint8)
    if fmt == "int8":
        return codes.view(np.int8).astype(np.float32)
    table = np.array([float(v) if v is not None else np.nan for v in E4M3_TABLE], dtype=np.float32)
    return table[codes]
