#!/usr/bin/env python3
"""Writes the golden fixtures of this directory from the independent numpy references
in tests/npref.py (float64 attention, brute-force E4M3, closed-form INT8, integer bf16).

Inputs come from numpy's legacy RandomState (a frozen stream).  Each fixture holds the
inputs in the device layouts and the expected outputs:

  g_f32.npz   FP32 cache, B=1, NH=2, maxT=48, 37 attended positions
  g_bf16.npz  BF16 cache, B=2, NH=2, maxT=80, ragged totals (80, 23)
  g_int8.npz  INT8 cache built by appending 40 positions of bf16 K/V rows (1% outliers
              x8 and one all-zero row), B=1, NH=2, maxT=40: expected codes, row scales and
              the attention output over the dequantised cache
  g_fp8.npz   the same for FP8-E4M3, plus a V row with a wide range (its maximum maps
              to the top code 448, its small entries to zero and subnormal codes)

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import npref  # noqa: E402

HS = 64


def fp_case(name, dtype, B, NH, maxT, totals, seed):
    rng = np.random.RandomState(seed)
    qkv = rng.standard_normal(B * 3 * NH * HS).astype(np.float32)
    cache = rng.standard_normal(2 * B * NH * maxT * HS).astype(np.float32)
    if dtype == "bf16":
        qkv_raw, cache_raw = npref.bf16_round(qkv), npref.bf16_round(cache)
        qv, cv = npref.bf16_to_f32(qkv_raw), npref.bf16_to_f32(cache_raw)
    else:
        qkv_raw, cache_raw, qv, cv = qkv, cache, qkv, cache
    out = npref.attention_f64(qv, cv, np.array(totals), B, NH, maxT)
    np.savez_compressed(os.path.join(HERE, name), B=B, NH=NH, maxT=maxT, totals=np.array(totals, np.int32),
                        qkv=qkv_raw, cache=cache_raw, out=out)


def w8_case(name, fmt, seed):
    B, NH, maxT = 1, 2, 40
    rng = np.random.RandomState(seed)
    # src[j] = the qkv vector of the token appended at position j (bf16 bits)
    src = rng.standard_normal((maxT, B, 3, NH, HS)).astype(np.float32)
    src = np.where(rng.random_sample(src.shape) < 0.01, src * 8.0, src).astype(np.float32)
    src[5, 0, 1, 1, :] = 0.0                       # an all-zero K row
    if fmt == "fp8":
        src[9, 0, 2, 0, :4] = [900.0, -1000.0, 3.0, 1e-3]
    src_raw = npref.bf16_round(src)
    srcf = npref.bf16_to_f32(src_raw)
    codes = np.zeros((2, B, NH, maxT, HS), np.uint8)
    scales = np.zeros((2, B, NH, maxT), np.float32)
    for j in range(maxT):
        for kv in range(2):
            for h in range(NH):
                c, s = npref.quantise_row(srcf[j, 0, 1 + kv, h], fmt)
                codes[kv, 0, h, j], scales[kv, 0, h, j] = c, s
    deq = npref.decode_w8(codes, fmt) * scales[..., None]
    q = srcf[maxT - 1].reshape(-1)                 # the last token's q
    out = npref.attention_f64(q, deq.reshape(-1), np.array([maxT]), B, NH, maxT)
    np.savez_compressed(os.path.join(HERE, name), B=B, NH=NH, maxT=maxT, src=src_raw, codes=codes.reshape(-1),
                        scales=scales.reshape(-1), out=out)


def main():
    fp_case("g_f32.npz", "f32", 1, 2, 48, [37], 101)
    fp_case("g_bf16.npz", "bf16", 2, 2, 80, [80, 23], 102)
    w8_case("g_int8.npz", "int8", 103)
    w8_case("g_fp8.npz", "fp8", 104)


if __name__ == "__main__":
    main()
