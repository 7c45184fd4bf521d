"""numpy binding of the CPU oracle (libkvattn_oracle.so).

TEST INFRASTRUCTURE ONLY: used by tests/, by the smoke check and by the benchmark's
CPU-baseline leg, always as the checker or the reported CPU figure -- never as part of
the product path.  Each function mirrors one C function of kvattn_oracle.h, which cites
the reference file:line it restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libkvattn_oracle.so")

W8_INT8 = 0
W8_FP8_E4M3 = 1

_LIB = None
_vp = ctypes.c_void_p
_i = ctypes.c_int


def build() -> None:
    subprocess.run(["make", "-B", "-C", _HERE], check=True, stdout=subprocess.DEVNULL)


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "oracle_attention_f32": (None, [_vp, _vp, _vp, _i, _i, _i, _i, _i, ctypes.c_float]),
            "oracle_attention_f32_ragged": (None, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, ctypes.c_float]),
            "oracle_attention_f64_ragged": (None, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, ctypes.c_double]),
            "oracle_split_partials": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, ctypes.c_float]),
            "oracle_merge": (None, [_vp, _vp, _vp, _vp, _i, _i, _i, _i]),
            "oracle_bf16_from_f32": (ctypes.c_uint16, [ctypes.c_float]),
            "oracle_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "oracle_bf16_round_array": (None, [_vp, _vp, ctypes.c_size_t]),
            "oracle_bf16_decode_array": (None, [_vp, _vp, ctypes.c_size_t]),
            "oracle_w8_encode": (ctypes.c_uint8, [ctypes.c_float, ctypes.c_float, _i]),
            "oracle_w8_decode": (ctypes.c_float, [ctypes.c_uint8, _i]),
            "oracle_fp8_e4m3_from_f32": (ctypes.c_uint8, [ctypes.c_float]),
            "oracle_fp8_e4m3_to_f32": (ctypes.c_float, [ctypes.c_uint8]),
            "oracle_cache_write": (None, [_vp, _vp, ctypes.c_size_t, _vp, _i, _i, _i, _i]),
            "oracle_cache_write_w8": (None, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i]),
            "oracle_dequant_w8": (None, [_vp, _vp, _vp, _i, _i, _i, _i, _i]),
            "oracle_gen_normal": (None, [ctypes.c_uint64, _vp, ctypes.c_size_t]),
            "oracle_lab_rand": (None, [ctypes.c_uint, _vp, ctypes.c_size_t]),
            "oracle_time_attention_f32": (ctypes.c_double,
                                          [_vp, _vp, _vp, _i, _i, _i, _i, _i, ctypes.c_float, _i]),
            "oracle_gemv": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i]),
            "oracle_gelu_tanh": (ctypes.c_float, [ctypes.c_float]),
            "oracle_time_gemv": (ctypes.c_double, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def attention_f32(qkv, kv_cache, totals, B, NH, hs, maxT, scale=None) -> np.ndarray:
    """attention_kv_cpu restated (FP32); totals: int or per-sequence array."""
    qkv, kv = _f32(qkv), _f32(kv_cache)
    scale = np.float32(1.0 / np.sqrt(np.float32(hs))) if scale is None else np.float32(scale)
    out = np.empty(B * NH * hs, dtype=np.float32)
    t = np.ascontiguousarray(np.broadcast_to(np.asarray(totals, dtype=np.int32), (B,)))
    lib().oracle_attention_f32_ragged(_p(out), _p(qkv), _p(kv), _p(t), B, NH, hs, maxT, float(scale))
    return out.reshape(B, NH, hs)


def attention_f64(qkv, kv_cache, totals, B, NH, hs, maxT, scale=None) -> np.ndarray:
    qkv, kv = _f32(qkv), _f32(kv_cache)
    scale = 1.0 / np.sqrt(hs) if scale is None else float(scale)
    out = np.empty(B * NH * hs, dtype=np.float64)
    t = np.ascontiguousarray(np.broadcast_to(np.asarray(totals, dtype=np.int32), (B,)))
    lib().oracle_attention_f64_ragged(_p(out), _p(qkv), _p(kv), _p(t), B, NH, hs, maxT, scale)
    return out.reshape(B, NH, hs)


def split_partials(qkv, kv_cache, totals, B, NH, hs, maxT, S, scale=None):
    qkv, kv = _f32(qkv), _f32(kv_cache)
    scale = np.float32(1.0 / np.sqrt(np.float32(hs))) if scale is None else np.float32(scale)
    po = np.empty(B * NH * S * hs, dtype=np.float32)
    pl = np.empty(B * NH * S, dtype=np.float32)
    pm = np.empty(B * NH * S, dtype=np.float32)
    t = np.ascontiguousarray(np.broadcast_to(np.asarray(totals, dtype=np.int32), (B,)))
    lib().oracle_split_partials(_p(po), _p(pl), _p(pm), _p(qkv), _p(kv), _p(t), B, NH, hs, maxT, S, float(scale))
    return po.reshape(B, NH, S, hs), pl.reshape(B, NH, S), pm.reshape(B, NH, S)


def merge(part_out, part_lse, part_max, B, NH, hs, S) -> np.ndarray:
    po, pl, pm = _f32(part_out), _f32(part_lse), _f32(part_max)
    out = np.empty(B * NH * hs, dtype=np.float32)
    lib().oracle_merge(_p(out), _p(po), _p(pl), _p(pm), B, NH, hs, S)
    return out.reshape(B, NH, hs)


def bf16_round(x) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even."""
    x = _f32(x)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_bf16_round_array(_p(x), _p(out), x.size)
    return out


def bf16_decode(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    lib().oracle_bf16_decode_array(_p(b), _p(out), b.size)
    return out


def w8_encode(x: float, scale: float, fmt: int) -> int:
    return int(lib().oracle_w8_encode(float(x), float(scale), fmt))


def w8_decode(code: int, fmt: int) -> float:
    return float(lib().oracle_w8_decode(int(code), fmt))


def fp8_from_f32(y: float) -> int:
    return int(lib().oracle_fp8_e4m3_from_f32(float(y)))


def fp8_to_f32(code: int) -> float:
    return float(lib().oracle_fp8_e4m3_to_f32(int(code)))


def cache_write(kv_cache: np.ndarray, qkv: np.ndarray, cur_lens, B, NH, hs, maxT) -> None:
    """In-place append into kv_cache (any element type; qkv of the same dtype)."""
    assert kv_cache.dtype == qkv.dtype
    cl = np.ascontiguousarray(np.broadcast_to(np.asarray(cur_lens, dtype=np.int32), (B,)))
    q = np.ascontiguousarray(qkv)
    lib().oracle_cache_write(_p(kv_cache), _p(q), kv_cache.itemsize, _p(cl), B, NH, hs, maxT)


def cache_write_w8(kv_cache: np.ndarray, kv_scale: np.ndarray, qkv_f32: np.ndarray, cur_lens, B, NH, hs, maxT,
                   fmt: int) -> None:
    assert kv_cache.dtype == np.uint8 and kv_scale.dtype == np.float32
    cl = np.ascontiguousarray(np.broadcast_to(np.asarray(cur_lens, dtype=np.int32), (B,)))
    q = _f32(qkv_f32)
    lib().oracle_cache_write_w8(_p(kv_cache), _p(kv_scale), _p(q), _p(cl), B, NH, hs, maxT, fmt)


def dequant_w8(kv_cache: np.ndarray, kv_scale: np.ndarray, B, NH, hs, maxT, fmt: int) -> np.ndarray:
    out = np.empty(kv_cache.size, dtype=np.float32)
    lib().oracle_dequant_w8(_p(out), _p(np.ascontiguousarray(kv_cache)), _p(np.ascontiguousarray(kv_scale)),
                            B, NH, hs, maxT, fmt)
    return out


def gen_normal(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().oracle_gen_normal(ctypes.c_uint64(seed), _p(out), n)
    return out


def lab_rand(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().oracle_lab_rand(seed, _p(out), n)
    return out


def time_attention_f32(qkv, kv_cache, total, B, NH, hs, maxT, reps: int) -> float:
    """Median microseconds of one single-threaded attention_kv_cpu call."""
    qkv, kv = _f32(qkv), _f32(kv_cache)
    out = np.empty(B * NH * hs, dtype=np.float32)
    scale = np.float32(1.0 / np.sqrt(np.float32(hs)))
    return float(lib().oracle_time_attention_f32(_p(out), _p(qkv), _p(kv), B, total, NH, hs, maxT,
                                                 float(scale), reps))


def gemv(W, x, B, M, K, *, w_scale=None, bias=None, gelu=False, want_pre=False):
    """Fully connected decode layer (oracle_gemv): returns out [B*M] (and pre_gelu)."""
    Wf, xf = _f32(W), _f32(x)
    ws = None if w_scale is None else _f32(w_scale)
    bs = None if bias is None else _f32(bias)
    out = np.empty(B * M, dtype=np.float32)
    pre = np.empty(B * M, dtype=np.float32) if want_pre else None
    lib().oracle_gemv(_p(out), None if pre is None else _p(pre), _p(Wf), None if ws is None else _p(ws), _p(xf),
                      None if bs is None else _p(bs), B, M, K, int(bool(gelu)))
    return (out, pre) if want_pre else out


def gelu_tanh(v: float) -> float:
    return float(lib().oracle_gelu_tanh(float(v)))


def time_gemv(W, x, B, M, K, w_scale=None, bias=None, reps: int = 20) -> float:
    """Median microseconds of one single-threaded oracle_gemv call."""
    Wf, xf = _f32(W), _f32(x)
    ws = None if w_scale is None else _f32(w_scale)
    bs = None if bias is None else _f32(bias)
    out = np.empty(B * M, dtype=np.float32)
    return float(lib().oracle_time_gemv(_p(out), _p(Wf), None if ws is None else _p(ws), _p(xf),
                                        None if bs is None else _p(bs), B, M, K, reps))
