"""GPU parity of kvattn_gemv (the decode step's fully connected layer) against the oracle.

Weights, inputs and biases are seeded and stored in the kernel's types (bf16 values and
8-bit codes are decoded exactly for the oracle).  Bars, as norm-wise relative error over
each output vector and max-abs error relative to max|ref|: FP32 1e-5; bf16 outputs 1e-2.
GPT-2 shapes: the QKV projection (2304 x 768), the attention output projection
(768 x 768), the MLP up projection with GELU (3072 x 768) and down projection (768 x 3072).
"""
import zlib

import numpy as np
import pytest

from oracle import oracle

pytestmark = pytest.mark.gpu

TOL = {"f32": 1e-5, "bf16": 1e-2, "int8": 1e-2, "fp8": 1e-2}
FMT = {"int8": oracle.W8_INT8, "fp8": oracle.W8_FP8_E4M3}


def _kv():
    from cuda_gpt2_inference_amd import kvattn
    return kvattn


def _make(dtype, B, M, K, seed, with_bias=True):
    """Host tensors in the kernel's types (moved to the GPU by _run) and the float values
    the oracle sees."""
    import torch
    r = np.random.RandomState(seed)
    x = r.standard_normal((B, K)).astype(np.float32)
    bias = r.standard_normal(M).astype(np.float32) if with_bias else None
    scale = None
    if dtype == "f32":
        W = (r.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32)
        dev = dict(W=torch.from_numpy(W), x=torch.from_numpy(x),
                   bias=None if bias is None else torch.from_numpy(bias))
        return dev, dict(W=W, x=x, bias=bias, scale=None)

    def bf16_tensor(bits):
        return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)

    xb = oracle.bf16_round(x)
    bb = None if bias is None else oracle.bf16_round(bias)
    if dtype == "bf16":
        Wb = oracle.bf16_round((r.standard_normal((M, K)) / np.sqrt(K)).astype(np.float32))
        dW = bf16_tensor(Wb)
        Wf = oracle.bf16_decode(Wb).reshape(M, K)
    else:
        codes = r.randint(0, 256, size=(M, K)).astype(np.uint8)
        if dtype == "fp8":
            codes[(codes & 0x7F) == 0x7F] = 0                 # no NaN codes
        table = np.array([oracle.w8_decode(c, FMT[dtype]) for c in range(256)], dtype=np.float32)
        Wf = table[codes]
        scale = (1.0 / (np.abs(Wf).max(axis=1) + 1.0) / np.sqrt(K)).astype(np.float32)
        dW = torch.from_numpy(codes)
    dev = dict(W=dW, x=bf16_tensor(xb), bias=None if bb is None else bf16_tensor(bb),
               scale=None if scale is None else torch.from_numpy(scale))
    host = dict(W=Wf, x=oracle.bf16_decode(xb).reshape(B, K),
                bias=None if bb is None else oracle.bf16_decode(bb), scale=scale)
    return dev, host


def _run(dev_t, dtype, B, M, K, gelu, want_pre, out_dtype=None):
    """kvattn_gemv (out in the activation type), or kvattn_gemv_ex with out_dtype."""
    import torch
    kvattn = _kv()
    d = {k: (None if v is None else v.to("cuda:0")) for k, v in dev_t.items()}
    if out_dtype is None:
        odt = torch.float32 if dtype == "f32" else torch.bfloat16
    else:
        odt = torch.float32 if out_dtype == "f32" else torch.bfloat16
    out = torch.full((B * M,), float("nan"), dtype=odt, device="cuda:0")
    pre = torch.full((B * M,), float("nan"), dtype=odt, device="cuda:0") if want_pre else None
    kvattn.gemv(out, d["W"], d["x"], B, M, K, w_dtype=dtype, w_scale=d.get("scale"), bias=d["bias"],
                pre_gelu=pre, gelu=gelu, out_dtype=out_dtype)
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), (None if pre is None else pre.float().cpu().numpy())


def _check(got, ref, dtype, B, M, what):
    assert np.all(np.isfinite(got)), what
    g = got.reshape(B, M).astype(np.float64)
    r = ref.reshape(B, M).astype(np.float64)
    nrm = (np.linalg.norm(g - r, axis=1) / np.linalg.norm(r, axis=1)).max()
    mabs = np.abs(g - r).max() / np.abs(r).max()
    assert nrm <= TOL[dtype] and mabs <= TOL[dtype], f"{what}: {nrm:.3e} {mabs:.3e}"


SHAPES = [("qkv", 2304, 768, False), ("attproj", 768, 768, False), ("fc", 3072, 768, True),
          ("fcproj", 768, 3072, False)]


@pytest.mark.parametrize("dtype", ["f32", "bf16", "int8", "fp8"])
@pytest.mark.parametrize("name,M,K,gelu", SHAPES)
def test_gemv_gpt2_shapes(dev, dtype, name, M, K, gelu):
    for B in (1, 3):
        d, h = _make(dtype, B, M, K, seed=zlib.crc32(f"{dtype} {name} {B}".encode()) % 10000)
        got, pre = _run(d, dtype, B, M, K, gelu, want_pre=gelu)
        ref, rpre = oracle.gemv(h["W"], h["x"], B, M, K, w_scale=h["scale"], bias=h["bias"], gelu=gelu,
                                want_pre=True)
        _check(got, ref, dtype, B, M, f"{name} {dtype} B={B}")
        if gelu:
            _check(pre, rpre, dtype, B, M, f"{name} {dtype} B={B} pre_gelu")


@pytest.mark.parametrize("dtype", ["f32", "bf16", "int8", "fp8"])
@pytest.mark.parametrize("M,K", [(1, 16), (5, 48), (7, 1040), (130, 4096)])
def test_gemv_ragged_shapes(dev, dtype, M, K):
    """Rows not a multiple of the 4 per workgroup, rows whose chunks do not fill the 64
    lanes, and the longest rows each dtype keeps in registers; no bias."""
    d, h = _make(dtype, 2, M, K, seed=M * 7 + K, with_bias=False)
    got, _ = _run(d, dtype, 2, M, K, False, False)
    ref = oracle.gemv(h["W"], h["x"], 2, M, K, w_scale=h["scale"])
    _check(got, ref, dtype, 2, M, f"M={M} K={K} {dtype}")


@pytest.mark.parametrize("dtype", ["f32", "bf16", "int8", "fp8"])
def test_gemv_vocabulary_projection_float_out(dev, dtype):
    """The reference engine's vocabulary projection, launch_GEMV6_w8x2<float, floatX> over the
    8-bit embedding table into float logits (inference_gpt2_opt.cu:389-394): Vp = 50304 rows
    of C = 768, no bias, float output (kvattn_gemv_ex), taken by the tall-matrix shape (several
    rows per wave).  The same call with bf16 output must equal the float result rounded."""
    M, K = 50304, 768
    d, h = _make(dtype, 1, M, K, seed=5030 + len(dtype), with_bias=False)
    got, _ = _run(d, dtype, 1, M, K, False, False, out_dtype="f32")
    ref = oracle.gemv(h["W"], h["x"], 1, M, K, w_scale=h["scale"])
    _check(got, ref, "f32" if dtype == "f32" else dtype, 1, M, f"logits {dtype} float out")
    got_b, _ = _run(d, dtype, 1, M, K, False, False, out_dtype="bf16")
    assert np.array_equal(got_b.view(np.uint32), oracle.bf16_decode(oracle.bf16_round(got)).view(np.uint32))


@pytest.mark.parametrize("dtype", ["f32", "bf16", "int8", "fp8"])
@pytest.mark.parametrize("M", [37, 8195])
def test_gemv_rows_beyond_one_block(dev, dtype, M):
    """Rows longer than one block of a wave's registers: with one row per wave (37 rows) a
    block is 64 x 16 chunks, so rows of 32 KB (FP32), 24 KB (bf16) and 20 KB (8-bit) take two
    blocks; with the tall shape (8195 rows, 2 rows per wave or 4 for 8-bit weights, a partial
    last wave) a block is 64 x 8 chunks (64 x 4 for 8-bit), and 9216-element rows take 3 to 5
    blocks.  B = 1 and B = 3 (the weights
    are read again per vector); with bias and GELU."""
    if M < 8192:
        K = {"f32": 8192, "bf16": 12288, "int8": 20480, "fp8": 20480}[dtype]
    else:
        K = 9216
    for B in (1, 3):
        d, h = _make(dtype, B, M, K, seed=M + B + K)
        got, pre = _run(d, dtype, B, M, K, True, True)
        ref, rpre = oracle.gemv(h["W"], h["x"], B, M, K, w_scale=h["scale"], bias=h["bias"], gelu=True,
                                want_pre=True)
        _check(got, ref, dtype, B, M, f"M={M} K={K} {dtype} B={B}")
        _check(pre, rpre, dtype, B, M, f"M={M} K={K} {dtype} B={B} pre_gelu")


@pytest.mark.parametrize("dtype", ["bf16", "int8"])
def test_gemv_tall_shape_equals_one_row_per_wave(dev, dtype):
    """A tall matrix (several rows per wave) against the same rows computed in pieces of
    fewer than 8192 rows (one row per wave): bit-identical, since both sum each row's chunks
    in the same order."""
    import torch
    M, K = 12288, 1024
    d, _ = _make(dtype, 2, M, K, seed=91)
    whole, _ = _run(d, dtype, 2, M, K, False, False)
    parts = []
    for m0 in range(0, M, 4096):
        sub = dict(d)
        sub["W"] = d["W"][m0:m0 + 4096].contiguous()
        sub["bias"] = d["bias"][m0:m0 + 4096].contiguous()
        if d.get("scale") is not None:
            sub["scale"] = d["scale"][m0:m0 + 4096].contiguous()
        p, _ = _run(sub, dtype, 2, 4096, K, False, False)
        parts.append(p.reshape(2, 4096))
    assert np.array_equal(whole.reshape(2, M), np.concatenate(parts, axis=1))


@pytest.mark.parametrize("dtype,kv", [("f32", "f32"), ("bf16", "bf16"), ("int8", "bf16"), ("bf16", "int8"),
                                      ("bf16", "fp8"), ("int8", "int8"), ("fp8", "fp8")])
@pytest.mark.parametrize("lens", ["uniform", "ragged", "library"])
def test_gemv_qkv_append_equals_gemv_then_append(dev, dtype, kv, lens):
    """kvattn_gemv_qkv_append against kvattn_gemv + kvattn_cache_write on copies of the same
    cache: identical qkv bytes and identical cache bytes (the appended K and V rows and every
    other row; for 8-bit caches the codes and the row scales), at GPT-2's QKV shape (NH = 12:
    2304 x 768), with one device length, per-sequence lengths (one of them beyond maxT,
    clamped), and the library's own length.  8-bit caches run two calls in a row on one
    workspace, so the second must not take the words the first staged there."""
    import torch
    kvattn = _kv()
    NH, HS, K, maxT = 12, 64, 768, 96
    B = 1 if lens == "uniform" else 3
    M = 3 * NH * HS
    d, _ = _make(dtype, B, M, K, seed=70 + B)
    W, x = d["W"].to(dev), d["x"].to(dev).contiguous()
    bias = None if d["bias"] is None else d["bias"].to(dev)
    scale = None if d.get("scale") is None else d["scale"].to(dev)
    act = torch.float32 if dtype == "f32" else torch.bfloat16
    w8 = kv in ("int8", "fp8")
    g = torch.Generator(device=dev)
    g.manual_seed(71)
    if w8:
        cache = torch.randint(0, 256, (2 * B * NH * maxT * HS,), generator=g, device=dev, dtype=torch.uint8)
        kscale = torch.rand(2 * B * NH * maxT, generator=g, device=dev)
        ws_bytes = kvattn.gemv_qkv_append_workspace_bytes(B, NH)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        kvattn.workspace_init(ws, ws_bytes)
    else:
        cache = torch.randn(2 * B * NH * maxT * HS, generator=g, device=dev).to(act)
        kscale, ws, ws_bytes = None, None, 0
    if lens == "uniform":
        cur, per_seq = torch.tensor([40], dtype=torch.int32, device=dev), False
    elif lens == "ragged":
        cur, per_seq = torch.tensor([0, maxT - 1, maxT + 10], dtype=torch.int32, device=dev), True
    else:
        kvattn.set_cur_len(17)
        cur, per_seq = None, False
    iview = torch.int32 if dtype == "f32" else torch.int16
    cview = torch.uint8 if w8 else iview
    c_a, c_b = cache.clone(), cache.clone()
    s_a = None if kscale is None else kscale.clone()
    s_b = None if kscale is None else kscale.clone()
    for call in range(2 if w8 else 1):
        xc = x if call == 0 else (x * -0.75).contiguous()
        q_a = torch.empty(B * M, dtype=act, device=dev)
        q_b = torch.empty_like(q_a)
        kvattn.gemv(q_a, W, xc, B, M, K, w_dtype=dtype, w_scale=scale, bias=bias)
        kvattn.kv_cache_write(c_a, q_a, B, NH, HS, maxT, kv_dtype=kv, kv_scale=s_a, cur_len=cur,
                              lens_per_seq=per_seq)
        kvattn.gemv_qkv_append(q_b, W, xc, B, NH, HS, K, c_b, maxT, w_dtype=dtype, kv_dtype=kv, w_scale=scale,
                               bias=bias, kv_scale=s_b, cur_len=cur, lens_per_seq=per_seq, workspace=ws,
                               workspace_nbytes=ws_bytes)
        torch.cuda.synchronize()
        tag = f"{dtype} weights, {kv} cache, {lens}, call {call}"
        assert torch.equal(q_a.view(iview), q_b.view(iview)), f"{tag}: qkv"
        assert torch.equal(c_a.view(cview), c_b.view(cview)), f"{tag}: cache"
        if w8:
            assert torch.equal(s_a.view(torch.int32), s_b.view(torch.int32)), f"{tag}: row scales"
        assert not torch.equal(c_a.view(cview), cache.view(cview)), f"{tag}: nothing appended"


@pytest.mark.parametrize("kv", ["int8", "fp8"])
def test_gemv_qkv_append_8bit_graph_replays(dev, kv):
    """The 8-bit QKV epilogue captured in a graph: its staged words carry the dispatch that
    wrote them (no memset node), so every replay must quantise afresh.  Three replays
    with new inputs and eager work in between, each against kvattn_gemv +
    kvattn_cache_write on a copy of the cache: qkv, codes and row scales bit for bit."""
    import torch
    kvattn = _kv()
    NH, HS, K, maxT, B = 12, 64, 768, 64, 2
    M = 3 * NH * HS
    d, _ = _make("int8", B, M, K, seed=91)
    W, scale = d["W"].to(dev), d["scale"].to(dev)
    bias = None if d["bias"] is None else d["bias"].to(dev)
    x = d["x"].to(dev).contiguous()
    cache = torch.zeros(2 * B * NH * maxT * HS, dtype=torch.uint8, device=dev)
    kscale = torch.zeros(2 * B * NH * maxT, device=dev)
    cur = torch.tensor([5, 40], dtype=torch.int32, device=dev)
    ws_bytes = kvattn.gemv_qkv_append_workspace_bytes(B, NH)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    kvattn.workspace_init(ws, ws_bytes)
    qkv = torch.empty(B * M, dtype=torch.bfloat16, device=dev)
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            kvattn.gemv_qkv_append(qkv, W, x, B, NH, HS, K, cache, maxT, w_dtype="int8", kv_dtype=kv, w_scale=scale,
                                   bias=bias, kv_scale=kscale, cur_len=cur, lens_per_seq=True, workspace=ws,
                                   workspace_nbytes=ws_bytes)
    torch.cuda.synchronize()
    gen = torch.Generator(device=dev)
    gen.manual_seed(92)
    for rep in range(3):
        x.copy_(torch.randn(x.numel(), generator=gen, device=dev).to(x.dtype).view_as(x))
        cur.copy_(torch.tensor([5 + rep, 40 + 7 * rep], dtype=torch.int32, device=dev))
        c_ref, s_ref = cache.clone(), kscale.clone()
        q_ref = torch.empty_like(qkv)
        kvattn.gemv(q_ref, W, x, B, M, K, w_dtype="int8", w_scale=scale, bias=bias)
        kvattn.kv_cache_write(c_ref, q_ref, B, NH, HS, maxT, kv_dtype=kv, kv_scale=s_ref, cur_len=cur,
                              lens_per_seq=True)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(qkv.view(torch.int16), q_ref.view(torch.int16)), f"{kv} replay {rep}: qkv"
        assert torch.equal(cache, c_ref), f"{kv} replay {rep}: codes"
        assert torch.equal(kscale.view(torch.int32), s_ref.view(torch.int32)), f"{kv} replay {rep}: row scales"


@pytest.mark.parametrize("kv", ["int8", "fp8"])
def test_gemv_qkv_append_8bit_fallback_and_dense_layout(dev, kv):
    """The 8-bit QKV epilogue (a) with its quantising wave's wait forced to give up from the
    host (poll bound 0: it computes every channel of its head row itself, with the owning
    waves' arithmetic) and (b) with 2 heads (6 head rows: the dense layout with write-through
    words instead of the XCD-local one), each against kvattn_gemv + kvattn_cache_write on a
    copy of the cache: qkv, codes and row scales bit for bit, two calls in a row."""
    import torch
    kvattn = _kv()
    HS, K, maxT, B = 64, 768, 48, 2
    for NH, bound in ((12, 0), (2, None), (2, 0)):
        M = 3 * NH * HS
        d, _ = _make("int8", B, M, K, seed=93 + NH)
        W, scale = d["W"].to(dev), d["scale"].to(dev)
        bias = d["bias"].to(dev)
        x = d["x"].to(dev).contiguous()
        cur = torch.tensor([3, 30], dtype=torch.int32, device=dev)
        ws_bytes = kvattn.gemv_qkv_append_workspace_bytes(B, NH)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        kvattn.workspace_init(ws, ws_bytes)
        cache = torch.zeros(2 * B * NH * maxT * HS, dtype=torch.uint8, device=dev)
        kscale = torch.zeros(2 * B * NH * maxT, device=dev)
        qkv = torch.empty(B * M, dtype=torch.bfloat16, device=dev)
        for call in range(2):
            cur.add_(call)
            c_ref, s_ref = cache.clone(), kscale.clone()
            q_ref = torch.empty_like(qkv)
            kvattn.gemv(q_ref, W, x, B, M, K, w_dtype="int8", w_scale=scale, bias=bias)
            kvattn.kv_cache_write(c_ref, q_ref, B, NH, HS, maxT, kv_dtype=kv, kv_scale=s_ref, cur_len=cur,
                                  lens_per_seq=True)
            prev = kvattn.set_merge_poll_limit(bound) if bound is not None else None
            try:
                kvattn.gemv_qkv_append(qkv, W, x, B, NH, HS, K, cache, maxT, w_dtype="int8", kv_dtype=kv,
                                       w_scale=scale, bias=bias, kv_scale=kscale, cur_len=cur, lens_per_seq=True,
                                       workspace=ws, workspace_nbytes=ws_bytes)
                torch.cuda.synchronize()
            finally:
                if prev is not None:
                    kvattn.set_merge_poll_limit(prev)
            what = f"NH={NH} bound={bound} call {call}"
            assert torch.equal(qkv.view(torch.int16), q_ref.view(torch.int16)), what + ": qkv"
            assert torch.equal(cache, c_ref), what + ": codes"
            assert torch.equal(kscale.view(torch.int32), s_ref.view(torch.int32)), what + ": row scales"


def test_gemv_seeded_shape_sweep(dev):
    """32 calls drawn from a fixed seed, each against the oracle: every weight type, B in
    1..4, M from 1 row to beyond the tall-matrix threshold (8192, with partial last waves),
    K any multiple of 16 up to 3072 (one or several blocks of a row), with and without
    bias and GELU, and float, bf16 or activation-typed output.  The bar follows the output
    type (bf16 outputs 1e-2)."""
    rng = np.random.RandomState(4242)
    for i in range(32):
        dtype = ["f32", "bf16", "int8", "fp8"][rng.randint(4)]
        B = int(rng.randint(1, 5))
        kind = rng.randint(3)
        M = int(rng.randint(1, 300)) if kind == 0 else (int(rng.randint(8190, 8201)) if kind == 1
                                                        else int(rng.randint(300, 12000)))
        K = 16 * int(rng.randint(1, 193))
        gelu = bool(rng.randint(2))
        with_bias = bool(rng.randint(2))
        out_dtype = [None, "f32", "bf16"][rng.randint(3)]
        name = f"case {i}: {dtype} B={B} M={M} K={K} gelu={gelu} bias={with_bias} out={out_dtype}"
        print(name, flush=True)
        d, h = _make(dtype, B, M, K, seed=7000 + i, with_bias=with_bias)
        got, pre = _run(d, dtype, B, M, K, gelu, want_pre=gelu, out_dtype=out_dtype)
        ref, rpre = oracle.gemv(h["W"], h["x"], B, M, K, w_scale=h["scale"], bias=h["bias"], gelu=gelu,
                                want_pre=True)
        out_bf16 = out_dtype == "bf16" or (out_dtype is None and dtype != "f32")
        key = "bf16" if out_bf16 else dtype
        _check(got, ref, key, B, M, name)
        if gelu:
            _check(pre, rpre, key, B, M, name + " pre_gelu")


def test_gemv_qkv_append_seeded_sweep(dev):
    """16 calls of kvattn_gemv_qkv_append drawn from a fixed seed, each against kvattn_gemv +
    kvattn_cache_write on a copy of the cache (qkv, cache bytes and 8-bit row scales bit for
    bit): every valid weight / cache type pair, NH 1..16 (the 8-bit epilogue's dense and
    XCD-local layouts), B 1..4, K up to 1536, maxT 1..200, one length or per-sequence
    lengths (some beyond maxT, clamped)."""
    import torch
    kvattn = _kv()
    pairs = [("f32", "f32"), ("bf16", "bf16"), ("int8", "bf16"), ("fp8", "bf16"), ("bf16", "int8"),
             ("bf16", "fp8"), ("int8", "int8"), ("fp8", "fp8"), ("int8", "fp8")]
    rng = np.random.RandomState(5150)
    HS = 64
    for i in range(16):
        dtype, kv = pairs[rng.randint(len(pairs))]
        NH, B = int(rng.randint(1, 17)), int(rng.randint(1, 5))
        K = 16 * int(rng.randint(1, 97))
        maxT = int(rng.randint(1, 201))
        per_seq = bool(rng.randint(2))
        lens = rng.randint(0, maxT + 8, B if per_seq else 1).astype(np.int32)
        name = f"case {i}: {dtype} weights, {kv} cache, NH={NH} B={B} K={K} maxT={maxT} cur_len={lens.tolist()}"
        print(name, flush=True)
        M = 3 * NH * HS
        d, _ = _make(dtype, B, M, K, seed=5200 + i, with_bias=bool(rng.randint(2)))
        W, x = d["W"].to(dev), d["x"].to(dev).contiguous()
        bias = None if d["bias"] is None else d["bias"].to(dev)
        scale = None if d.get("scale") is None else d["scale"].to(dev)
        act = torch.float32 if dtype == "f32" else torch.bfloat16
        w8 = kv in ("int8", "fp8")
        g = torch.Generator(device=dev)
        g.manual_seed(5300 + i)
        if w8:
            cache = torch.randint(0, 256, (2 * B * NH * maxT * HS,), generator=g, device=dev, dtype=torch.uint8)
            kscale = torch.rand(2 * B * NH * maxT, generator=g, device=dev)
            ws_bytes = kvattn.gemv_qkv_append_workspace_bytes(B, NH)
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
            kvattn.workspace_init(ws, ws_bytes)
        else:
            cache = torch.randn(2 * B * NH * maxT * HS, generator=g, device=dev).to(act)
            kscale, ws, ws_bytes = None, None, 0
        cur = torch.from_numpy(lens).to(dev)
        iview = torch.int32 if dtype == "f32" else torch.int16
        cview = torch.uint8 if w8 else iview
        c_a, c_b = cache.clone(), cache.clone()
        s_a = None if kscale is None else kscale.clone()
        s_b = None if kscale is None else kscale.clone()
        q_a = torch.empty(B * M, dtype=act, device=dev)
        q_b = torch.empty_like(q_a)
        kvattn.gemv(q_a, W, x, B, M, K, w_dtype=dtype, w_scale=scale, bias=bias)
        kvattn.kv_cache_write(c_a, q_a, B, NH, HS, maxT, kv_dtype=kv, kv_scale=s_a, cur_len=cur,
                              lens_per_seq=per_seq)
        kvattn.gemv_qkv_append(q_b, W, x, B, NH, HS, K, c_b, maxT, w_dtype=dtype, kv_dtype=kv, w_scale=scale,
                               bias=bias, kv_scale=s_b, cur_len=cur, lens_per_seq=per_seq, workspace=ws,
                               workspace_nbytes=ws_bytes)
        torch.cuda.synchronize()
        assert torch.equal(q_a.view(iview), q_b.view(iview)), f"{name}: qkv"
        assert torch.equal(c_a.view(cview), c_b.view(cview)), f"{name}: cache"
        if w8:
            assert torch.equal(s_a.view(torch.int32), s_b.view(torch.int32)), f"{name}: row scales"
