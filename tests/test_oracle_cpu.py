"""Pins the CPU oracle (oracle/kvattn_oracle.c) before it is trusted as the checker.

Every oracle function is checked against something it does not share code with: the
float64 numpy reference, closed forms and invariants of softmax attention, the exact
E4M3 table from the OCP spec with a brute-force encoder, torch's bf16 / float8 casts,
glibc's rand() stream used by the reference lab, and the committed golden fixtures.
A test that plants a mistake (in a copy of the reference, on the CPU) shows the
comparisons are sharp enough to catch it.
"""
import os

import numpy as np
import pytest

import npref
from oracle import oracle

HS = 64
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def normwise(got, ref):
    g = np.asarray(got, np.float64).reshape(-1, HS)
    r = np.asarray(ref, np.float64).reshape(-1, HS)
    return float((np.linalg.norm(g - r, axis=1) / np.linalg.norm(r, axis=1)).max())


def rand_case(B, NH, maxT, seed):
    rng = np.random.RandomState(seed)
    return (rng.standard_normal(B * 3 * NH * HS).astype(np.float32),
            rng.standard_normal(2 * B * NH * maxT * HS).astype(np.float32))


# ---------------------------------------------------------------------------------
# attention_kv_cpu restatement
# ---------------------------------------------------------------------------------
@pytest.mark.parametrize("totals", [[1, 5], [50, 17], [33, 50]])
def test_attention_f32_matches_float64_numpy(totals):
    B, NH, maxT = 2, 3, 50
    qkv, cache = rand_case(B, NH, maxT, 1)
    got = oracle.attention_f32(qkv, cache, totals, B, NH, HS, maxT)
    ref = npref.attention_f64(qkv, cache, np.array(totals), B, NH, maxT)
    assert normwise(got, ref) <= 1e-6


def test_attention_f64_twin_matches_numpy():
    B, NH, maxT = 2, 3, 40
    qkv, cache = rand_case(B, NH, maxT, 2)
    got = oracle.attention_f64(qkv, cache, [40, 9], B, NH, HS, maxT)
    ref = npref.attention_f64(qkv, cache, np.array([40, 9]), B, NH, maxT)
    assert np.abs(got - ref).max() <= 1e-12


def test_glibc_rand_stream_of_the_reference_lab():
    """make_random_float after srand(0) (attention_kvcache.cu:911-917,952): glibc's
    first rand() values are 1804289383, 846930886, 1681692777, 1714636915, 1957747793."""
    first = [1804289383, 846930886, 1681692777, 1714636915, 1957747793]
    expect = np.array([np.float32(v % 10000) / np.float32(5000.0) - np.float32(1.0) for v in first], np.float32)
    assert np.array_equal(oracle.lab_rand(0, 5), expect)


def test_reference_lab_shape_and_lengths():
    """The lab's own check: B=1, NH=12, hs=64, maxT=1024, srand(0) inputs, lengths
    {1,64,256,512,1024} (attention_kvcache.cu:955,979-980,1014), against float64."""
    B, NH, maxT = 1, 12, 1024
    vals = oracle.lab_rand(0, B * 3 * NH * HS + 2 * B * NH * maxT * HS)
    qkv, cache = vals[:B * 3 * NH * HS], vals[B * 3 * NH * HS:]
    for T in (1, 64, 256, 512, 1024):
        got = oracle.attention_f32(qkv, cache, T, B, NH, HS, maxT)
        ref = npref.attention_f64(qkv, cache, np.array([T]), B, NH, maxT)
        assert normwise(got, ref) <= 1e-6
        assert np.abs(got - ref).max() <= 1e-5


def test_single_position_returns_v0_exactly():
    B, NH, maxT = 1, 4, 8
    qkv, cache = rand_case(B, NH, maxT, 3)
    got = oracle.attention_f32(qkv, cache, 1, B, NH, HS, maxT)
    v0 = cache.reshape(2, B, NH, maxT, HS)[1, :, :, 0]
    assert np.array_equal(got, v0)


def test_equal_scores_give_mean_of_v():
    B, NH, maxT, T = 1, 3, 30, 23
    qkv, cache = rand_case(B, NH, maxT, 4)
    qkv.reshape(B, 3, NH, HS)[:, 0] = 0.0
    got = oracle.attention_f32(qkv, cache, T, B, NH, HS, maxT)
    mean = cache.reshape(2, B, NH, maxT, HS)[1, :, :, :T].astype(np.float64).mean(axis=2)
    assert np.abs(got - mean).max() <= 1e-6


def test_position_permutation_invariance_and_hull():
    B, NH, maxT, T = 1, 2, 40, 40
    qkv, cache = rand_case(B, NH, maxT, 5)
    perm = np.random.RandomState(0).permutation(T)
    c5 = cache.reshape(2, B, NH, maxT, HS)
    cp = c5[:, :, :, perm].copy().reshape(-1)
    a = oracle.attention_f32(qkv, cache, T, B, NH, HS, maxT)
    b = oracle.attention_f32(qkv, cp, T, B, NH, HS, maxT)
    assert normwise(a, b) <= 1e-6
    v = c5[1, 0]
    assert np.all(a[0] >= v.min(axis=1) - 1e-6) and np.all(a[0] <= v.max(axis=1) + 1e-6)


def test_one_hot_key_selects_its_value():
    B, NH, maxT, T, j = 1, 2, 16, 16, 11
    qkv, cache = rand_case(B, NH, maxT, 6)
    c5 = cache.reshape(2, B, NH, maxT, HS)
    q = qkv.reshape(B, 3, NH, HS)[0, 0]
    c5[0, 0, :, j] = 40.0 * q / np.linalg.norm(q, axis=1, keepdims=True)
    got = oracle.attention_f32(qkv, cache, T, B, NH, HS, maxT)
    assert np.abs(got[0] - c5[1, 0, :, j]).max() <= 1e-5


def test_planted_mistakes_are_caught():
    """Copies of the float64 reference with one deliberate mistake each (scale dropped,
    K and V swapped, off-by-one length) must fail the 1e-6 comparison."""
    B, NH, maxT, T = 1, 3, 32, 30
    qkv, cache = rand_case(B, NH, maxT, 7)
    got = oracle.attention_f32(qkv, cache, T, B, NH, HS, maxT)

    def ref(scale=1 / np.sqrt(HS), swap=False, T_=T):
        q = qkv.astype(np.float64).reshape(B, 3, NH, HS)[0, 0]
        kv = cache.astype(np.float64).reshape(2, B, NH, maxT, HS)[:, 0, :, :T_]
        k, v = (kv[1], kv[0]) if swap else (kv[0], kv[1])
        s = np.einsum("hd,htd->ht", q, k) * scale
        p = np.exp(s - s.max(axis=1, keepdims=True))
        return np.einsum("ht,htd->hd", p, v) / p.sum(axis=1, keepdims=True)

    assert normwise(got, ref()) <= 1e-6
    for bad in (ref(scale=1.0), ref(swap=True), ref(T_=T - 1)):
        assert normwise(got, bad) > 1e-3


# ---------------------------------------------------------------------------------
# split + merge
# ---------------------------------------------------------------------------------
@pytest.mark.parametrize("S", [1, 2, 3, 5, 8, 16, 32])
def test_merge_of_split_equals_unsplit(S):
    B, NH, maxT = 2, 3, 64
    totals = [64, 3]            # total < S leaves empty segments for S > 3
    qkv, cache = rand_case(B, NH, maxT, 8)
    po, pl, pm = oracle.split_partials(qkv, cache, totals, B, NH, HS, maxT, S)
    got = oracle.merge(po, pl, pm, B, NH, HS, S)
    ref = npref.attention_f64(qkv, cache, np.array(totals), B, NH, maxT)
    assert normwise(got, ref) <= 1e-6


def test_split_partials_against_float64_segments():
    """Each partial equals the float64 (max, sum exp, sum exp*V) of its segment of the
    reference partition chunk = ceil(total/S); empty segments carry the sentinel."""
    B, NH, maxT, S = 1, 2, 50, 8
    totals = [45]
    qkv, cache = rand_case(B, NH, maxT, 9)
    po, pl, pm = oracle.split_partials(qkv, cache, totals, B, NH, HS, maxT, S)
    q = qkv.astype(np.float64).reshape(B, 3, NH, HS)[0, 0]
    kv = cache.astype(np.float64).reshape(2, B, NH, maxT, HS)[:, 0]
    chunk = -(-totals[0] // S)
    for h in range(NH):
        for s in range(S):
            j0, j1 = s * chunk, min((s + 1) * chunk, totals[0])
            if j1 <= j0:
                assert pm[0, h, s] == np.float32(-3.4028234663852886e38) and pl[0, h, s] == 0
                assert np.all(po[0, h, s] == 0)
                continue
            sc = kv[0, h, j0:j1] @ q[h] / 8.0
            m = sc.max()
            e = np.exp(sc - m)
            assert abs(pm[0, h, s] - m) <= 1e-5 * max(1, abs(m))
            assert abs(pl[0, h, s] - e.sum()) <= 1e-5 * e.sum()
            assert np.abs(po[0, h, s] - e @ kv[1, h, j0:j1]).max() <= 1e-5 * np.abs(e @ kv[1, h, j0:j1]).max()


# ---------------------------------------------------------------------------------
# element codecs
# ---------------------------------------------------------------------------------
def test_bf16_rounding_matches_torch_and_integer_reference():
    import torch
    rng = np.random.RandomState(10)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32),
        (rng.standard_normal(2000) * 1e-39).astype(np.float32),           # subnormals
        np.array([0.0, -0.0, np.inf, -np.inf, 3.4028235e38, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8], np.float32),
        # exact ties: halfway between two bf16 values
        ((rng.randint(0, 1 << 15, 2000).astype(np.uint32) << 16) | 0x8000).view(np.float32),
    ])
    got = oracle.bf16_round(x)
    assert np.array_equal(got, npref.bf16_round(x))
    t = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], t[~nan])       # torch canonicalises NaN payloads
    assert np.all(np.isnan(oracle.bf16_decode(got[nan])))
    assert np.array_equal(oracle.bf16_decode(got).view(np.uint32), got.astype(np.uint32) << 16)


def test_fp8_decode_matches_ocp_table():
    for c in range(256):
        v = npref.E4M3_TABLE[c]
        got = oracle.fp8_to_f32(c)
        if v is None:
            assert np.isnan(got)
        else:
            assert got == float(v) and (np.signbit(got) == bool(c & 0x80))
    finite = [v for v in npref.E4M3_TABLE if v is not None]
    assert max(finite) == 448 and min(v for v in finite if v > 0) == 2.0 ** -9 and len(finite) == 254


def test_fp8_encode_bruteforce_every_bf16_in_range():
    """Every bf16 value in [-512, 512] (and both signs of zero) against the brute-force
    nearest-even E4M3 encoder; beyond 448 the code saturates to 0x7E / 0xFE."""
    bits = np.arange(1 << 16, dtype=np.uint32) << 16
    vals = bits.view(np.float32)
    vals = vals[np.isfinite(vals) & (np.abs(vals) <= 512)]
    for y in vals:
        assert oracle.fp8_from_f32(float(y)) == npref.e4m3_encode_bruteforce(float(y)), y


def test_fp8_encode_random_floats_and_torch():
    import torch
    rng = np.random.RandomState(11)
    y = np.concatenate([rng.standard_normal(3000) * 50, rng.standard_normal(1000) * 0.01,
                        rng.uniform(440, 470, 500), -rng.uniform(440, 470, 500)]).astype(np.float32)
    codes = np.array([oracle.fp8_from_f32(float(v)) for v in y], np.uint8)
    brute = np.array([npref.e4m3_encode_bruteforce(float(v)) for v in y], np.uint8)
    assert np.array_equal(codes, brute)
    ok = np.abs(y) <= 464          # torch's cast is RNE but does not saturate beyond 464
    tcodes = torch.from_numpy(y[ok]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(codes[ok], tcodes)
    assert np.all(codes[np.abs(y) > 464] & 0x7F == 0x7E)


def test_int8_encode_closed_form_and_ties():
    rng = np.random.RandomState(12)
    x = rng.standard_normal(5000).astype(np.float32) * 3
    for scale in (np.float32(0.0213), np.float32(1.0), np.float32(3.0) / np.float32(127.0)):
        got = np.array([oracle.w8_encode(float(v), float(scale), oracle.W8_INT8) for v in x], np.uint8)
        assert np.array_equal(got, npref.int8_encode(x, scale))
        dec = got.view(np.int8).astype(np.float64) * float(scale)
        inside = np.abs(x / scale) <= 127
        # half a step plus the float32 rounding of x/scale (|x/scale| <= 127)
        assert np.all(np.abs(dec[inside] - x[inside]) <= float(scale) * (0.5 + 127 * 2.0 ** -23))
    # ties round half to even: 0.5 -> 0, 1.5 -> 2, 2.5 -> 2, -0.5 -> 0, -1.5 -> -2
    for v, want in ((0.5, 0), (1.5, 2), (2.5, 2), (-0.5, 0), (-1.5, -2), (200.0, 127), (-300.0, -127)):
        assert np.int8(np.uint8(oracle.w8_encode(v, 1.0, oracle.W8_INT8)).view(np.int8)) == want
    for c in range(256):
        assert oracle.w8_decode(c, oracle.W8_INT8) == float(np.uint8(c).view(np.int8))


@pytest.mark.parametrize("fmt", ["int8", "fp8"])
def test_cache_write_w8_rows(fmt):
    B, NH, maxT = 2, 3, 6
    code = oracle.W8_INT8 if fmt == "int8" else oracle.W8_FP8_E4M3
    rng = np.random.RandomState(13)
    qkv = npref.bf16_to_f32(npref.bf16_round(rng.standard_normal(B * 3 * NH * HS).astype(np.float32) * 2))
    qkv.reshape(B, 3, NH, HS)[1, 2, 1] = 0.0          # zero V row of (b=1, h=1)
    kv = np.full(2 * B * NH * maxT * HS, 0xAB, np.uint8)
    sc = np.full(2 * B * NH * maxT, -1.0, np.float32)
    cur = np.array([4, 0], np.int32)
    oracle.cache_write_w8(kv, sc, qkv, cur, B, NH, HS, maxT, code)
    kv5 = kv.reshape(2, B, NH, maxT, HS)
    sc4 = sc.reshape(2, B, NH, maxT)
    q4 = qkv.reshape(B, 3, NH, HS)
    for which in range(2):
        for b in range(B):
            for h in range(NH):
                want_c, want_s = npref.quantise_row(q4[b, 1 + which, h], fmt)
                assert sc4[which, b, h, cur[b]].view(np.uint32) == np.float32(want_s).view(np.uint32)
                assert np.array_equal(kv5[which, b, h, cur[b]], want_c)
    assert sc4[1, 1, 1, 0] == 0.0 and np.all(kv5[1, 1, 1, 0] == 0)
    untouched = np.ones((2, B, NH, maxT), bool)
    untouched[:, 0, :, 4] = False
    untouched[:, 1, :, 0] = False
    assert np.all(sc4[untouched] == -1.0)


def test_cache_write_copy():
    B, NH, maxT = 2, 2, 5
    rng = np.random.RandomState(14)
    qkv = rng.standard_normal(B * 3 * NH * HS).astype(np.float32)
    kv = np.zeros(2 * B * NH * maxT * HS, np.float32)
    oracle.cache_write(kv, qkv, [3, 4], B, NH, HS, maxT)
    kv5 = kv.reshape(2, B, NH, maxT, HS)
    q4 = qkv.reshape(B, 3, NH, HS)
    assert np.array_equal(kv5[0, 0, :, 3], q4[0, 1]) and np.array_equal(kv5[1, 1, :, 4], q4[1, 2])
    assert np.count_nonzero(kv) == 2 * B * NH * HS


def test_gen_normal_moments_and_determinism():
    a = oracle.gen_normal(42, 200001)
    assert np.array_equal(a, oracle.gen_normal(42, 200001))
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1) < 0.01
    assert not np.array_equal(a[:100], oracle.gen_normal(43, 100))


# ---------------------------------------------------------------------------------
# golden fixtures
# ---------------------------------------------------------------------------------
@pytest.mark.parametrize("name", ["g_f32", "g_bf16"])
def test_golden_attention_fixtures(name):
    g = np.load(os.path.join(GOLDEN, name + ".npz"))
    B, NH, maxT = int(g["B"]), int(g["NH"]), int(g["maxT"])
    qkv, cache = g["qkv"], g["cache"]
    if qkv.dtype == np.uint16:
        qkv, cache = oracle.bf16_decode(qkv), oracle.bf16_decode(cache)
    got = oracle.attention_f32(qkv, cache, g["totals"], B, NH, HS, maxT)
    assert normwise(got, g["out"]) <= 1e-6


@pytest.mark.parametrize("fmt", ["int8", "fp8"])
def test_golden_w8_fixtures(fmt):
    g = np.load(os.path.join(GOLDEN, f"g_{fmt}.npz"))
    B, NH, maxT = int(g["B"]), int(g["NH"]), int(g["maxT"])
    code = oracle.W8_INT8 if fmt == "int8" else oracle.W8_FP8_E4M3
    src = oracle.bf16_decode(g["src"]).reshape(maxT, -1)
    kv = np.zeros(2 * B * NH * maxT * HS, np.uint8)
    sc = np.zeros(2 * B * NH * maxT, np.float32)
    for j in range(maxT):
        oracle.cache_write_w8(kv, sc, src[j], [j] * B, B, NH, HS, maxT, code)
    assert np.array_equal(kv, g["codes"])
    assert np.array_equal(sc.view(np.uint32), g["scales"].view(np.uint32))
    deq = oracle.dequant_w8(kv, sc, B, NH, HS, maxT, code)
    got = oracle.attention_f32(src[maxT - 1], deq, maxT, B, NH, HS, maxT)
    assert normwise(got, g["out"]) <= 1e-6
