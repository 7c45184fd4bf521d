"""CPU checks of the fully connected decode layer: the oracle's GEMV pinned against numpy
float64 and closed forms, and the argument checks of kvattn_gemv (made before any HIP call).

Pins of oracle_gemv (a restatement of GEMV6_fused, Inference_gpt2/GEMV.cuh:132-197, and
GEMV6_w8x2, GEMV_w8.cuh:64-157):
  * float64 numpy W @ x * scale + bias, at non-square shapes (a transposed operand or a
    dropped term fails);
  * the identity matrix reproduces x + bias exactly;
  * GELU: the tanh form's identity gelu(v) - gelu(-v) = v, gelu(0) = 0, gelu(v) -> v and
    -> 0 in the tails, and the float64 formula;
  * 8-bit: the row scale applied after the sum equals scaling every weight (to rounding).
"""
import math

import numpy as np
import pytest

from oracle import oracle


def _rng(seed):
    return np.random.RandomState(seed)


@pytest.mark.parametrize("B,M,K", [(1, 768, 768), (2, 40, 3072), (3, 2304, 64), (1, 5, 16)])
def test_gemv_matches_float64(B, M, K):
    r = _rng(B * 1000 + M)
    W = r.standard_normal((M, K)).astype(np.float32)
    x = r.standard_normal((B, K)).astype(np.float32)
    bias = r.standard_normal(M).astype(np.float32)
    got, pre = oracle.gemv(W, x, B, M, K, bias=bias, want_pre=True)
    ref = x.astype(np.float64) @ W.astype(np.float64).T + bias
    err = np.abs(got.reshape(B, M) - ref).max() / np.abs(ref).max()
    assert err < 1e-5
    assert np.array_equal(got, pre)                      # no GELU: out is the pre-GELU value


def test_gemv_planted_mistakes_fail():
    """Copies of the reference computation with a plausible mistake must miss the oracle."""
    r = _rng(7)
    M, K = 24, 48
    W = r.standard_normal((M, K)).astype(np.float32)
    x = r.standard_normal((1, K)).astype(np.float32)
    bias = r.standard_normal(M).astype(np.float32)
    got = oracle.gemv(W, x, 1, M, K, bias=bias).astype(np.float64)
    good = W.astype(np.float64) @ x[0] + bias
    assert np.abs(got - good).max() < 1e-4
    for bad in (W.astype(np.float64) @ x[0],                      # bias dropped
                W.astype(np.float64)[:, ::-1] @ x[0] + bias,       # reversed k index
                np.roll(W.astype(np.float64) @ x[0], 1) + bias):   # rows shifted
        assert np.abs(got - bad).max() > 1e-2


def test_gemv_identity_is_exact():
    K = 64
    x = _rng(3).standard_normal((2, K)).astype(np.float32)
    bias = _rng(4).standard_normal(K).astype(np.float32)
    got = oracle.gemv(np.eye(K, dtype=np.float32), x, 2, K, K, bias=bias)
    assert np.array_equal(got.reshape(2, K), (x + bias).astype(np.float32))


def test_gelu_closed_forms():
    vs = np.concatenate([np.linspace(-8, 8, 4001), [0.0, 1e-3, -1e-3, 20.0, -20.0]]).astype(np.float32)
    for v in vs:
        g = oracle.gelu_tanh(float(v))
        gm = oracle.gelu_tanh(float(-v))
        assert abs((g - gm) - float(v)) <= 2e-6 * max(1.0, abs(float(v)))
        ref = 0.5 * float(v) * (1.0 + math.tanh(math.sqrt(2.0 / math.pi) * (float(v) + 0.044715 * float(v) ** 3)))
        assert abs(g - ref) <= 2e-6 * max(1.0, abs(ref))
    assert oracle.gelu_tanh(0.0) == 0.0
    assert oracle.gelu_tanh(20.0) == 20.0
    assert abs(oracle.gelu_tanh(-20.0)) < 1e-30


def test_gemv_gelu_applies_to_pre():
    r = _rng(11)
    M, K = 64, 128
    W = r.standard_normal((M, K)).astype(np.float32)
    x = r.standard_normal((1, K)).astype(np.float32)
    out, pre = oracle.gemv(W, x, 1, M, K, gelu=True, want_pre=True)
    assert np.array_equal(out, np.array([oracle.gelu_tanh(float(p)) for p in pre], dtype=np.float32))


@pytest.mark.parametrize("fmt", [oracle.W8_INT8, oracle.W8_FP8_E4M3])
def test_gemv_8bit_row_scale(fmt):
    """Codes decoded and multiplied by the row scale after the sum (GEMV_w8.cuh:136)."""
    r = _rng(13 + fmt)
    M, K = 48, 256
    codes = r.randint(0, 256, size=(M, K)).astype(np.uint8)
    if fmt == oracle.W8_FP8_E4M3:
        codes[(codes & 0x7F) == 0x7F] = 0                  # no NaN codes
    dec = np.array([oracle.w8_decode(int(c), fmt) for c in range(256)], dtype=np.float32)[codes]
    scale = (r.random_sample(M) * 0.1 + 1e-3).astype(np.float32)
    x = r.standard_normal((1, K)).astype(np.float32)
    got = oracle.gemv(dec, x, 1, M, K, w_scale=scale).astype(np.float64)
    ref = (dec.astype(np.float64) * scale[:, None].astype(np.float64)) @ x[0].astype(np.float64)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 1e-5


ALIGNED = 1 << 20


@pytest.mark.parametrize("kw,status", [
    (dict(K=24), 4),                    # K % 16 != 0 -> KVATTN_ERR_SHAPE
    (dict(K=0), 4),
    (dict(M=0), 4),
    (dict(B=0), 4),
    (dict(w_dtype=7), 5),               # KVATTN_ERR_DTYPE
    (dict(w_dtype=2, w_scale=None), 5),  # 8-bit weights without row scales
    (dict(W=None), 1),                  # KVATTN_ERR_NULL_POINTER
    (dict(out=None), 1),
    (dict(x=ALIGNED + 8), 2),           # KVATTN_ERR_MISALIGNED
    (dict(out=ALIGNED + 1), 2),
])
def test_gemv_argument_errors(kw, status):
    from cuda_gpt2_inference_amd import kvattn
    a = dict(out=ALIGNED, pre=None, W=ALIGNED, w_scale=ALIGNED, x=ALIGNED, bias=None, B=1, M=768, K=768,
             w_dtype=1, gelu=0)
    a.update(kw)
    st = kvattn.lib().kvattn_gemv(a["out"], a["pre"], a["W"], a["w_scale"], a["x"], a["bias"], a["B"], a["M"],
                                  a["K"], a["w_dtype"], a["gelu"], None)
    assert st == status, kvattn.strerror(st)


@pytest.mark.parametrize("kw,status", [
    (dict(out_dtype=2), 5),             # out must be float or bf16 -> KVATTN_ERR_DTYPE
    (dict(out_dtype=7), 5),
    (dict(out=ALIGNED + 2), 2),         # float out, 2-byte aligned -> KVATTN_ERR_MISALIGNED
    (dict(K=24), 4),
])
def test_gemv_ex_argument_errors(kw, status):
    """kvattn_gemv_ex's output type and alignment checks (made before any HIP call)."""
    from cuda_gpt2_inference_amd import kvattn
    a = dict(out=ALIGNED, pre=None, W=ALIGNED, w_scale=ALIGNED, x=ALIGNED, bias=None, B=1, M=50304, K=768,
             w_dtype=2, out_dtype=0, gelu=0)
    a.update(kw)
    st = kvattn.lib().kvattn_gemv_ex(a["out"], a["pre"], a["W"], a["w_scale"], a["x"], a["bias"], a["B"], a["M"],
                                     a["K"], a["w_dtype"], a["out_dtype"], a["gelu"], None)
    assert st == status, kvattn.strerror(st)


@pytest.mark.parametrize("kw,status", [
    (dict(hs=32), 3),                   # KVATTN_ERR_HEAD_DIM
    (dict(B=0), 4),                     # KVATTN_ERR_SHAPE
    (dict(NH=0), 4),
    (dict(maxT=0), 4),
    (dict(maxT=(1 << 23) + 1), 4),
    (dict(K=24), 4),
    (dict(kv=None), 1),                 # KVATTN_ERR_NULL_POINTER
    (dict(W=None), 1),
    (dict(w_dtype=7), 5),               # KVATTN_ERR_DTYPE
    (dict(kv_dtype=0), 5),              # an FP32 cache behind bf16 activations
    (dict(kv_dtype=2, kv_scale=None), 5),   # 8-bit cache without row scales
    (dict(kv_dtype=3, w_dtype=0), 5),   # 8-bit cache behind FP32 activations
    (dict(kv_dtype=2, ws=None), 7),     # KVATTN_ERR_WORKSPACE
    (dict(kv_dtype=2, ws_bytes=64), 7),
    (dict(kv_dtype=2, ws=ALIGNED + 16), 2),  # KVATTN_ERR_MISALIGNED (workspace below 256 B)
    (dict(kv=ALIGNED + 1), 2),          # bf16 cache
    (dict(qkv=ALIGNED + 2, w_dtype=0, kv_dtype=0), 2),
])
def test_gemv_qkv_append_argument_errors(kw, status):
    """kvattn_gemv_qkv_append's checks, made before any HIP call (a device length is given,
    so the library's own length symbol is not looked up)."""
    from cuda_gpt2_inference_amd import kvattn
    a = dict(qkv=ALIGNED, W=ALIGNED, w_scale=ALIGNED, x=ALIGNED, bias=None, B=1, NH=12, hs=64, K=768, kv=ALIGNED,
             kv_scale=ALIGNED, maxT=1024, cur=ALIGNED, lens=0, w_dtype=1, kv_dtype=1, ws=ALIGNED, ws_bytes=1 << 20)
    a.update(kw)
    st = kvattn.lib().kvattn_gemv_qkv_append(a["qkv"], a["W"], a["w_scale"], a["x"], a["bias"], a["B"], a["NH"],
                                             a["hs"], a["K"], a["kv"], a["kv_scale"], a["maxT"], a["cur"], a["lens"],
                                             a["w_dtype"], a["kv_dtype"], a["ws"], a["ws_bytes"], None)
    assert st == status, kvattn.strerror(st)


def test_gemv_qkv_append_workspace_bytes():
    """One tagged 8-byte word per channel of the 2*B*NH appended K and V rows; 0 for shapes
    out of range."""
    from cuda_gpt2_inference_amd import kvattn
    for B, NH in ((1, 12), (3, 12), (64, 16), (1, 1)):
        assert kvattn.gemv_qkv_append_workspace_bytes(B, NH) == 2 * B * NH * 64 * 8
    assert kvattn.gemv_qkv_append_workspace_bytes(0, 12) == 0
