"""Pins the oracle's attention to the reference's own CPU routine, bit for bit (CPU only).

attention_kv_cpu (attention_kvcache/attention_kvcache.cu:74-102) is compiled from the
reference source where it lies by `make -C oracle ref` into oracle/_ref/ (gitignored; see
oracle/Makefile).  oracle_attention_f32 restates it with the same loop order and the same
individually rounded FP32 operations, so the two must agree exactly, not just within a
tolerance: a dropped term, a transposed index or a changed summation order would show as
differing bits.  Inputs: the lab's own check (B=1, NH=12, hs=64, maxT=1024, glibc srand(0)
stream, lengths {1, 64, 256, 512, 1024}; attention_kvcache.cu:911-917,952,1011-1041) and
seeded N(0,1) batches with B > 1 and maxT > length.  The reference keeps scores[1024] on its
stack, so lengths stay at or below 1024.  Skipped when neither the built library nor the
reference tree is present (the GPU box has no reference tree).
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

from oracle import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libattention_kv_cpu_ref.so")
REF_SRC = "/root/reference/attention_kvcache/attention_kvcache.cu"
HS = 64


@pytest.fixture(scope="module")
def ref():
    if not os.path.exists(REF_LIB):
        if not os.path.exists(REF_SRC):
            pytest.skip("reference CPU routine neither built (oracle/_ref) nor buildable here")
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "ref"], check=True, capture_output=True)
    lib = ctypes.CDLL(REF_LIB)
    fn = lib.attention_kv_cpu
    vp, i = ctypes.c_void_p, ctypes.c_int
    fn.argtypes = [vp, vp, vp, i, i, i, i, i, ctypes.c_float]
    fn.restype = None
    return fn


def _ref_call(fn, qkv, cache, B, T, NH, maxT):
    qkv = np.ascontiguousarray(qkv, np.float32)
    cache = np.ascontiguousarray(cache, np.float32)
    out = np.full(B * NH * HS, np.nan, np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(HS))
    # attention_kv_cpu(out, qkv, kv_cache, B, seq_len, NH, hs, maxT, scale)
    fn(out.ctypes.data, qkv.ctypes.data, cache.ctypes.data, B, T, NH, HS, maxT, float(scale))
    return out


def _bits(x):
    return np.asarray(x, np.float32).reshape(-1).view(np.uint32)


@pytest.mark.parametrize("T", [1, 64, 256, 512, 1024])
def test_oracle_matches_reference_on_lab_inputs(ref, T):
    B, NH, maxT = 1, 12, 1024
    vals = oracle.lab_rand(0, B * 3 * NH * HS + 2 * B * NH * maxT * HS)
    qkv, cache = vals[: B * 3 * NH * HS], vals[B * 3 * NH * HS:]
    want = _ref_call(ref, qkv, cache, B, T, NH, maxT)
    got = oracle.attention_f32(qkv, cache, T, B, NH, HS, maxT)
    assert np.isfinite(want).all()
    assert np.array_equal(_bits(got), _bits(want)), f"T={T}: oracle differs from attention_kv_cpu"


@pytest.mark.parametrize("B,NH,maxT,T", [(2, 3, 300, 257), (3, 2, 1024, 1024), (4, 5, 130, 1), (1, 12, 777, 700)])
def test_oracle_matches_reference_on_normal_inputs(ref, B, NH, maxT, T):
    vals = oracle.gen_normal(1000 + T, B * 3 * NH * HS + 2 * B * NH * maxT * HS)
    qkv, cache = vals[: B * 3 * NH * HS], vals[B * 3 * NH * HS:]
    want = _ref_call(ref, qkv, cache, B, T, NH, maxT)
    got = oracle.attention_f32(qkv, cache, T, B, NH, HS, maxT)
    assert np.array_equal(_bits(got), _bits(want)), f"B={B} NH={NH} maxT={maxT} T={T}"


def test_planted_mistake_in_a_copy_of_the_oracle_is_caught(ref):
    """The check has teeth: the oracle's result with the last position dropped (an
    off-by-one in the length) or with the scale applied twice no longer matches."""
    B, NH, maxT, T = 1, 12, 1024, 512
    vals = oracle.lab_rand(0, B * 3 * NH * HS + 2 * B * NH * maxT * HS)
    qkv, cache = vals[: B * 3 * NH * HS], vals[B * 3 * NH * HS:]
    want = _ref_call(ref, qkv, cache, B, T, NH, maxT)
    short = oracle.attention_f32(qkv, cache, T - 1, B, NH, HS, maxT)
    assert not np.array_equal(_bits(short), _bits(want))
    s = np.float32(1.0) / np.sqrt(np.float32(HS))
    twice = oracle.attention_f32(qkv, cache, T, B, NH, HS, maxT, scale=float(s * s))
    assert not np.array_equal(_bits(twice), _bits(want))
