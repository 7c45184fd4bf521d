"""Shared builders for decode-attention test cases.

A case holds host copies (numpy, for the oracle) and device copies (torch, for the
HIP library) of the same bytes: qkv [B][3][NH][hs], the cache [2][B][NH][maxT][hs]
(and the row scales for 8-bit caches) and the per-sequence current lengths.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np

from oracle import oracle

HS = 64
FMT = {"int8": oracle.W8_INT8, "fp8": oracle.W8_FP8_E4M3}


@dataclass
class Case:
    dtype: str
    B: int
    NH: int
    maxT: int
    cur_lens: np.ndarray          # int32 [B], device length per sequence (total = cur+1)
    qkv_host: np.ndarray          # float32 [B*3*NH*HS] values as the kernels see them
    cache_host: np.ndarray        # float32 values (dequantised for 8-bit) [2*B*NH*maxT*HS]
    qkv_raw: np.ndarray           # bytes as stored on the device (f32 / uint16 bf16)
    cache_raw: np.ndarray         # f32 / uint16 / uint8
    scale_raw: Optional[np.ndarray] = None  # float32 [2*B*NH*maxT] for 8-bit

    @property
    def totals(self) -> np.ndarray:
        return (self.cur_lens + 1).astype(np.int32)

    def reference(self) -> np.ndarray:
        return oracle.attention_f32(self.qkv_host, self.cache_host, self.totals, self.B, self.NH, HS, self.maxT)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    return oracle.bf16_round(x)


def make_case(dtype: str, B: int, NH: int, maxT: int, cur_lens, seed: int = 0, outliers: float = 0.0,
              source: str = "normal") -> Case:
    """Seeded inputs: q, K, V ~ N(0,1) (or the reference lab's uniform stream)."""
    cur_lens = np.array(np.broadcast_to(np.asarray(cur_lens, dtype=np.int32), (B,)), dtype=np.int32)
    n_qkv = B * 3 * NH * HS
    n_cache = 2 * B * NH * maxT * HS
    if source == "lab":
        vals = oracle.lab_rand(seed, n_qkv + n_cache)
    else:
        vals = oracle.gen_normal(seed, n_qkv + n_cache)
    qkv = vals[:n_qkv].copy()
    cache = vals[n_qkv:].copy()
    if outliers > 0.0:
        rng = np.random.RandomState(seed + 7)
        mask = rng.random_sample(n_cache) < outliers
        cache[mask] *= 8.0
        qmask = rng.random_sample(n_qkv) < outliers
        qkv[qmask] *= 8.0
    if dtype == "f32":
        return Case(dtype, B, NH, maxT, cur_lens, qkv, cache, qkv, cache)
    qb = bf16_bits(qkv)
    cb = bf16_bits(cache)
    qf = oracle.bf16_decode(qb)
    cf = oracle.bf16_decode(cb)
    if dtype == "bf16":
        return Case(dtype, B, NH, maxT, cur_lens, qf, cf, qb, cb)
    # 8-bit: quantise every cache row with the oracle's append restatement, column by
    # column, from the bf16 source values.
    fmt = FMT[dtype]
    codes = np.zeros(n_cache, dtype=np.uint8)
    scales = np.zeros(2 * B * NH * maxT, dtype=np.float32)
    src = cf.reshape(2, B, NH, maxT, HS)
    for j in range(maxT):
        col = np.zeros((B, 3, NH, HS), dtype=np.float32)
        col[:, 1] = src[0, :, :, j]
        col[:, 2] = src[1, :, :, j]
        oracle.cache_write_w8(codes, scales, col.reshape(-1), np.full(B, j, np.int32), B, NH, HS, maxT, fmt)
    deq = oracle.dequant_w8(codes, scales, B, NH, HS, maxT, fmt)
    return Case(dtype, B, NH, maxT, cur_lens, qf, deq, qb, codes, scales)


def to_device(case: Case, dev):
    """Device tensors (qkv, cache, scale or None, cur_len)."""
    import torch
    if case.dtype == "f32":
        qkv = torch.from_numpy(case.qkv_raw).to(dev)
        cache = torch.from_numpy(case.cache_raw).to(dev)
    else:
        qkv = torch.from_numpy(case.qkv_raw.view(np.int16)).to(dev).view(torch.bfloat16)
        if case.dtype == "bf16":
            cache = torch.from_numpy(case.cache_raw.view(np.int16)).to(dev).view(torch.bfloat16)
        else:
            cache = torch.from_numpy(case.cache_raw).to(dev)
    scale = torch.from_numpy(case.scale_raw).to(dev) if case.scale_raw is not None else None
    cur = torch.from_numpy(case.cur_lens.copy()).to(dev)
    return qkv, cache, scale, cur


def out_tensor(case: Case, dev):
    import torch
    dt = torch.float32 if case.dtype == "f32" else torch.bfloat16
    return torch.full((case.B * case.NH * HS,), float("nan"), dtype=dt, device=dev)


TOL = {"f32": 1e-5, "bf16": 1e-2, "int8": 2e-2, "fp8": 2e-2}


def rel_errors(got: np.ndarray, ref: np.ndarray):
    """Per-(b,h) norm-wise relative error and max-abs error relative to max|ref|."""
    g = got.reshape(-1, HS).astype(np.float64)
    r = ref.reshape(-1, HS).astype(np.float64)
    nrm = np.linalg.norm(g - r, axis=1) / np.maximum(np.linalg.norm(r, axis=1), 1e-30)
    mabs = np.abs(g - r).max() / max(np.abs(r).max(), 1e-30)
    return float(nrm.max()), float(mabs)


def assert_close(got: np.ndarray, ref: np.ndarray, dtype: str, what: str = ""):
    tol = TOL[dtype]
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    nrm, mabs = rel_errors(got, ref)
    assert nrm <= tol and mabs <= tol, f"{what}: norm-rel {nrm:.3e}, max-abs-rel {mabs:.3e} > {tol}"
    return nrm, mabs
