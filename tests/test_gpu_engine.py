"""Engine-level use of the decode attention on an MI355X: lengths planned on the device and a
12-layer decode step captured once and replayed token by token.

The reference engine captures two whole-step graphs (a "small" one with fused_single below
a length threshold and a "large" one with split + merge) and picks one per token, writing
the device length with a blocking cudaMemcpyToSymbol before each replay
(inference_gpt2_opt.cu:420-449,544-556).  Here the step is captured once with no length
hint, the kernels plan the segmentation from the device length, and the length is written
with a stream-ordered kernel.  Outputs are checked against the oracle at the stated
tolerance (BF16 1e-2, FP32 1e-5, 8-bit 2e-2); appended cache rows bit for bit.
"""
import numpy as np
import pytest

from kvcases import HS, assert_close, make_case, out_tensor, to_device
from oracle import oracle

pytestmark = pytest.mark.gpu

# Lengths around every change of the device plan: one segment up to 256 positions, then
# 128-row segments (257..512), 256-row (513..1024), 512-row (1025..); for the designated
# merger, 128-row segments from 257 on, and the quarters of the first 256 rows that segment 0
# splits among its waves (64/65, 128/129, 192/193).
PLAN_EDGES = (1, 2, 63, 64, 65, 127, 128, 129, 192, 193, 255, 256, 257, 300, 511, 512, 513, 1000, 1024, 1025,
              2048, 2049, 2100)


def _kv():
    from cuda_gpt2_inference_amd import kvattn
    return kvattn


@pytest.mark.parametrize("dtype", ["f32", "bf16", "int8", "fp8"])
def test_device_plan_uniform_length(dev, dtype):
    """One device length for the whole batch (dense grid), no host hint: every split
    strategy at every plan edge, from a single workspace sized for S = 0."""
    import torch
    kvattn = _kv()
    B, NH, maxT = 2, 3, 2100
    case = make_case(dtype, B, NH, maxT, 0, seed=31)
    qkv, cache, scale, _ = to_device(case, dev)
    cur = torch.zeros(1, dtype=torch.int32, device=dev)
    ws = kvattn.Workspace(B, NH, maxT, 0)
    for strategy in ("auto", "lastblock", "designated", "split_merge", "graph", "coop"):
        assert kvattn.plan(B, NH, HS, maxT, kv_dtype=dtype, strategy=strategy)[2] == -1
        for total in PLAN_EDGES:
            cur.fill_(total - 1)
            case.cur_lens[:] = total - 1
            out = out_tensor(case, dev)
            kvattn.decode(out, qkv, cache, B, NH, HS, maxT, kv_dtype=dtype, kv_scale=scale, cur_len=cur,
                          strategy=strategy, **ws.kwargs())
            torch.cuda.synchronize()
            assert_close(out.float().cpu().numpy(), case.reference(), dtype, f"{strategy} T={total}")


@pytest.mark.parametrize("dtype", ["bf16", "int8"])
def test_device_plan_past_64_segments(dev, dtype):
    """Past 64 segments of 512 rows (32768 positions) the device plan grows the rows instead
    (1024 from 32769, 2048 from 65537): split strategies with no hint, one length for the
    batch and per-sequence lengths, at and around those edges, against the oracle."""
    import torch
    kvattn = _kv()
    B, NH, maxT = 2, 2, 70000
    ws = kvattn.Workspace(B, NH, maxT, 0)
    for strategy in ("split_merge", "lastblock", "graph"):
        assert kvattn.plan(B, NH, HS, maxT, kv_dtype=dtype, strategy=strategy)[1:] == (64, -1)
    for lens in ([32768, 32768], [32769, 32769], [65536, 65536], [65537, 70000], [70000, 300], [40000, 33000]):
        case = make_case(dtype, B, NH, maxT, np.array(lens) - 1, seed=37 + lens[0] % 97)
        qkv, cache, scale, cur = to_device(case, dev)
        uniform = lens[0] == lens[1]
        if uniform:
            cur = cur[:1].contiguous()
        for strategy in ("split_merge", "lastblock", "graph"):
            out = out_tensor(case, dev)
            kvattn.decode(out, qkv, cache, B, NH, HS, maxT, kv_dtype=dtype, kv_scale=scale, cur_len=cur,
                          lens_per_seq=not uniform, strategy=strategy, **ws.kwargs())
            torch.cuda.synchronize()
            assert_close(out.float().cpu().numpy(), case.reference(), dtype, f"{strategy} lens={lens}")


@pytest.mark.parametrize("dtype", ["f32", "bf16", "fp8"])
def test_designated_device_plan_doubled_rows(dev, dtype):
    """The designated merger planned on the device beyond 64 segments of the base length:
    rows double (256 from 8193 positions, 512 from 16385 for 2 heads), so every segment but
    the first starts away from the first tile each workgroup requests before reading the
    length, and segment 0 outgrows it; the append path substitutes the fresh row there too."""
    import torch
    kvattn = _kv()
    B, NH, maxT = 1, 2, 16500
    case = make_case(dtype, B, NH, maxT, 0, seed=35)
    qkv, cache, scale, _ = to_device(case, dev)
    cur = torch.zeros(1, dtype=torch.int32, device=dev)
    ws = kvattn.Workspace(B, NH, maxT, 0)
    assert kvattn.plan(B, NH, HS, maxT, kv_dtype=dtype, strategy="designated")[1:] == (64, -1)
    for total in (256, 257, 8192, 8193, 8300, 16384, 16385, 16500):
        cur.fill_(total - 1)
        case.cur_lens[:] = total - 1
        kw = dict(kv_dtype=dtype, cur_len=cur, strategy="designated", **ws.kwargs())
        out = out_tensor(case, dev)
        kvattn.decode(out, qkv, cache, B, NH, HS, maxT, kv_scale=scale, **kw)
        torch.cuda.synchronize()
        assert_close(out.float().cpu().numpy(), case.reference(), dtype, f"designated T={total}")
        # Append and attend in one launch against the append followed by the attention.
        c_a, c_b = cache.clone(), cache.clone()
        s_a = scale.clone() if scale is not None else None
        s_b = scale.clone() if scale is not None else None
        o_a, o_b = out_tensor(case, dev), out_tensor(case, dev)
        kvattn.kv_cache_write(c_a, qkv, B, NH, HS, maxT, kv_dtype=dtype, kv_scale=s_a, cur_len=cur)
        kvattn.decode(o_a, qkv, c_a, B, NH, HS, maxT, kv_scale=s_a, **kw)
        kvattn.append_decode(o_b, qkv, c_b, B, NH, HS, maxT, kv_scale=s_b, **kw)
        torch.cuda.synchronize()
        assert np.array_equal(_cache_bytes(c_a), _cache_bytes(c_b)), f"append T={total}: cache"
        assert np.array_equal(o_a.float().cpu().numpy(), o_b.float().cpu().numpy()), f"append T={total}: out"


@pytest.mark.parametrize("dtype", ["bf16", "int8"])
def test_device_plan_ragged_lengths(dev, dtype):
    """Per-sequence lengths (compacted grid): each sequence plans its own segments."""
    import torch
    kvattn = _kv()
    B, NH, maxT = len(PLAN_EDGES), 2, 2100
    case = make_case(dtype, B, NH, maxT, np.array(PLAN_EDGES, np.int32) - 1, seed=32)
    qkv, cache, scale, cur = to_device(case, dev)
    ref = case.reference()
    ws = kvattn.Workspace(B, NH, maxT, 0)
    for strategy in ("auto", "lastblock", "designated", "split_merge", "graph", "coop"):
        out = out_tensor(case, dev)
        kvattn.decode(out, qkv, cache, B, NH, HS, maxT, kv_dtype=dtype, kv_scale=scale, cur_len=cur,
                      lens_per_seq=True, strategy=strategy, **ws.kwargs())
        torch.cuda.synchronize()
        assert_close(out.float().cpu().numpy(), ref, dtype, f"ragged {strategy}")


def test_set_cur_len_async(dev):
    """The stream-ordered length write, into a caller's int and into the library's own
    length (observed through an append that uses it)."""
    import torch
    kvattn = _kv()
    d = torch.full((4,), -7, dtype=torch.int32, device=dev)
    kvattn.set_cur_len_async(1234, d_cur_len=d[2:])
    torch.cuda.synchronize()
    assert d.cpu().tolist() == [-7, -7, 1234, -7]
    maxT = 8
    cache = torch.zeros(2 * maxT * HS, dtype=torch.float32, device=dev)
    qkv = torch.arange(3 * HS, dtype=torch.float32, device=dev) + 1.0
    kvattn.set_cur_len_async(5)
    kvattn.kv_cache_write(cache, qkv, 1, 1, HS, maxT, kv_dtype="f32")
    torch.cuda.synchronize()
    c = cache.view(2, maxT, HS).cpu()
    assert torch.equal(c[0, 5], qkv[HS:2 * HS].cpu()) and torch.equal(c[1, 5], qkv[2 * HS:].cpu())
    assert int((c != 0).any(dim=2).sum()) == 2


def _cache_bytes(t):
    import torch
    return t.view(torch.uint8).cpu().numpy().copy()


@pytest.mark.parametrize("dtype", ["f32", "bf16", "int8", "fp8"])
@pytest.mark.parametrize("lens", ["uniform", "ragged"])
def test_append_decode_equals_append_then_decode(dev, dtype, lens):
    """kvattn_append_decode against kvattn_cache_write + kvattn_decode on copies of the same
    cache: identical cache bytes (codes and scales included) and identical outputs, for every
    strategy and partition, at lengths inside one tile, at the fused_single / split edge and
    on the fused_single LDS path; outputs also against the oracle."""
    import torch
    kvattn = _kv()
    B, NH, maxT = 2, 3, 600
    totals = [[1, 1], [100, 100], [129, 129], [200, 200], [256, 256], [257, 257], [600, 600]] if lens == "uniform" else \
        [[600, 131], [1, 257], [256, 64]]
    runs = [("auto", 0, True), ("auto", 0, False), ("fused_single", 0, True), ("split_merge", 8, True),
            ("split_merge", 0, False), ("lastblock", 0, False), ("lastblock", -64, True), ("designated", 0, False),
            ("designated", -64, True), ("designated", 8, True), ("graph", 0, False),
            ("coop", 8, True), ("coop", 0, False)]
    for tt in totals:
        case = make_case(dtype, B, NH, maxT, np.array(tt, np.int32) - 1, seed=50 + tt[0])
        qkv, cache, scale, cur = to_device(case, dev)
        if lens == "uniform":
            cur = cur[:1].contiguous()
        hint = max(tt) - 1
        for strategy, S, hinted in runs:
            ws = kvattn.Workspace(B, NH, maxT, S)
            kw = dict(kv_dtype=dtype, cur_len=cur, lens_per_seq=(lens == "ragged"), S=S, strategy=strategy,
                      len_hint=hint if hinted else -1, **ws.kwargs())
            c_a, c_b = cache.clone(), cache.clone()
            s_a = scale.clone() if scale is not None else None
            s_b = scale.clone() if scale is not None else None
            o_a, o_b = out_tensor(case, dev), out_tensor(case, dev)
            kvattn.kv_cache_write(c_a, qkv, B, NH, HS, maxT, kv_dtype=dtype, kv_scale=s_a, cur_len=cur,
                                  lens_per_seq=(lens == "ragged"))
            kvattn.decode(o_a, qkv, c_a, B, NH, HS, maxT, kv_scale=s_a, **kw)
            kvattn.append_decode(o_b, qkv, c_b, B, NH, HS, maxT, kv_scale=s_b, **kw)
            torch.cuda.synchronize()
            what = f"{dtype} {lens} T={tt} {strategy} S={S} hint={hinted}"
            assert np.array_equal(_cache_bytes(c_a), _cache_bytes(c_b)), what + ": cache"
            if scale is not None:
                assert np.array_equal(_cache_bytes(s_a), _cache_bytes(s_b)), what + ": scales"
            ga, gb = o_a.float().cpu().numpy(), o_b.float().cpu().numpy()
            assert np.array_equal(ga, gb), what + f": outputs differ by {np.abs(ga - gb).max():.3e}"
        # The appended cache through the oracle's append, then the oracle's attention.
        ref_case = make_case(dtype, B, NH, maxT, np.array(tt, np.int32) - 1, seed=50 + tt[0])
        if dtype in ("int8", "fp8"):
            fmt = oracle.W8_INT8 if dtype == "int8" else oracle.W8_FP8_E4M3
            codes, scales = ref_case.cache_raw.copy(), ref_case.scale_raw.copy()
            oracle.cache_write_w8(codes, scales, ref_case.qkv_host, ref_case.cur_lens, B, NH, HS, maxT, fmt)
            assert np.array_equal(_cache_bytes(c_b), codes), f"{dtype} {lens} T={tt}: codes vs oracle"
            assert np.array_equal(_cache_bytes(s_b).view(np.uint32), scales.view(np.uint32))
            vals = oracle.dequant_w8(codes, scales, B, NH, HS, maxT, fmt)
        else:
            vals = ref_case.cache_host.copy()
            oracle.cache_write(vals, ref_case.qkv_host, ref_case.cur_lens, B, NH, HS, maxT)
        ref = oracle.attention_f32(ref_case.qkv_host, vals, ref_case.totals, B, NH, HS, maxT)
        assert_close(gb, ref, dtype, f"append_decode {dtype} {lens} T={tt}")


class Engine:
    """The attention block of a decode step for L layers (append, then attention, per
    layer), captured into a graph over per-layer qkv / out buffers and one KV cache
    allocation with the reference's layer stride 2*B*NH*maxT*hs (inference_gpt2_opt.cu:324)."""

    def __init__(self, dev, L, B, NH, maxT, dtype):
        import torch
        self.kvattn = _kv()
        self.L, self.B, self.NH, self.maxT, self.dtype = L, B, NH, maxT, dtype
        wide = torch.float32 if dtype == "f32" else torch.bfloat16
        n_cache = 2 * B * NH * maxT * HS
        self.cache = torch.zeros(L * n_cache, dtype=torch.uint8 if dtype in ("int8", "fp8") else wide, device=dev)
        self.scale = torch.zeros(L * 2 * B * NH * maxT, dtype=torch.float32, device=dev) \
            if dtype in ("int8", "fp8") else None
        self.qkv = torch.zeros(L, B * 3 * NH * HS, dtype=wide, device=dev)
        self.out = torch.zeros(L, B * NH * HS, dtype=wide, device=dev)
        self.cur = torch.zeros(1, dtype=torch.int32, device=dev)
        self.ws = self.kvattn.Workspace(B, NH, maxT, 0)
        self.n_cache = n_cache

    def layer_cache(self, l):
        return self.cache[l * self.n_cache:(l + 1) * self.n_cache]

    def layer_scale(self, l):
        n = 2 * self.B * self.NH * self.maxT
        return None if self.scale is None else self.scale[l * n:(l + 1) * n]

    def step(self, strategy="auto", S=0, fused=False, hint=-1):
        k = self.kvattn
        for l in range(self.L):
            args = (self.out[l], self.qkv[l], self.layer_cache(l), self.B, self.NH, HS, self.maxT)
            kw = dict(kv_dtype=self.dtype, kv_scale=self.layer_scale(l), cur_len=self.cur, S=S, strategy=strategy,
                      len_hint=hint, **self.ws.kwargs())
            if fused:
                k.append_decode(*args, **kw)
                continue
            k.kv_cache_write(self.layer_cache(l), self.qkv[l], self.B, self.NH, HS, self.maxT, kv_dtype=self.dtype,
                             kv_scale=self.layer_scale(l), cur_len=self.cur)
            k.decode(*args, **kw)

    def capture(self, strategy="auto", S=0, fused=False, hint=-1):
        import torch
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                self.step(strategy, S, fused, hint)
        torch.cuda.synchronize()
        return g


def _host_values(t, dtype):
    import torch
    if dtype == "f32":
        return t.cpu().numpy().astype(np.float32)
    return oracle.bf16_decode(t.view(torch.int16).cpu().numpy().view(np.uint16))


@pytest.mark.parametrize("dtype,mode", [("bf16", "one_graph"), ("bf16", "graph_pair"), ("fp8", "one_graph"),
                                        ("bf16", "fused"), ("int8", "fused"), ("bf16", "graph_trio"),
                                        ("int8", "graph_trio")])
def test_decode_step_token_by_token(dev, dtype, mode):
    """GPT-2 shape, 12 layers, B=1, NH=12, maxT=1024: the step graph is replayed for every
    token 1..1024 with fresh qkv and the device length advanced by set_cur_len_async.
    one_graph: one capture, AUTO with no hint.  fused: the same with kvattn_append_decode
    (append and attention in one launch per layer).  graph_pair: the reference's two graphs,
    fused_single below 150 positions and split + merge with S = 8 above (selection on the
    host per token, as inference_gpt2_opt.cu:556).  graph_trio: three fused append + attention
    graphs picked the same way, with length hints of 127 and 255 positions up to 128 and 256
    positions and no hint beyond.  Checked: every appended row bit for bit
    (8-bit: codes and scales against the oracle's quantiser) and the outputs of all layers
    at 40 tokens (every plan edge and a stride) against the oracle."""
    import torch
    kvattn = _kv()
    L, B, NH, maxT = 12, 1, 12, 1024
    eng = Engine(dev, L, B, NH, maxT, dtype)
    if mode in ("one_graph", "fused"):
        graphs = [eng.capture("auto", fused=(mode == "fused"))]
        pick = lambda cur_len: graphs[0]
    elif mode == "graph_trio":
        graphs = [eng.capture("auto", fused=True, hint=127), eng.capture("auto", fused=True, hint=255),
                  eng.capture("auto", fused=True)]
        pick = lambda cur_len: graphs[0] if cur_len < 128 else (graphs[1] if cur_len < 256 else graphs[2])
    else:
        graphs = [eng.capture("fused_single"), eng.capture("split_merge", S=8)]
        pick = lambda cur_len: graphs[0] if cur_len < 150 else graphs[1]
    g = torch.Generator(device=dev)
    g.manual_seed(41)
    wide = torch.float32 if dtype == "f32" else torch.bfloat16
    qkv_all = torch.randn(maxT, L, B * 3 * NH * HS, generator=g, device=dev).to(wide)
    check_tokens = sorted(set(PLAN_EDGES[:13]) | {149, 150, 151} | set(range(5, maxT, 41)))
    hist = {}
    for t in range(maxT):                  # token at position t, attends t + 1 positions
        eng.qkv.copy_(qkv_all[t])
        kvattn.set_cur_len_async(t, d_cur_len=eng.cur)
        pick(t).replay()
        if t + 1 in check_tokens:
            hist[t + 1] = eng.out.clone()
    torch.cuda.synchronize()

    qh = _host_values(qkv_all, dtype).reshape(maxT, L, B, 3, NH, HS)
    if dtype in ("bf16", "f32"):
        # Appended rows: column j of layer l holds K and V of token j.
        c = eng.cache.view(L, 2, B, NH, maxT, HS)
        got_k = _host_values(c[:, 0], dtype)
        got_v = _host_values(c[:, 1], dtype)
        assert np.array_equal(got_k, qh[:, :, :, 1].transpose(1, 2, 3, 0, 4))
        assert np.array_equal(got_v, qh[:, :, :, 2].transpose(1, 2, 3, 0, 4))
        caches = [c[l].reshape(-1) for l in range(L)]
        cache_vals = [_host_values(x, dtype) for x in caches]
    else:
        fmt = oracle.W8_FP8_E4M3 if dtype == "fp8" else oracle.W8_INT8
        codes = eng.cache.cpu().numpy()
        scales = eng.scale.cpu().numpy()
        n_sc = 2 * B * NH * maxT
        cache_vals = []
        for l in range(L):
            ref_codes = np.zeros(eng.n_cache, dtype=np.uint8)
            ref_scales = np.zeros(n_sc, dtype=np.float32)
            for j in range(maxT):
                oracle.cache_write_w8(ref_codes, ref_scales, qh[j, l].reshape(-1), [j] * B, B, NH, HS, maxT, fmt)
            lc = codes[l * eng.n_cache:(l + 1) * eng.n_cache]
            ls = scales[l * n_sc:(l + 1) * n_sc]
            assert np.array_equal(lc, ref_codes), f"layer {l} codes"
            assert np.array_equal(ls.view(np.uint32), ref_scales.view(np.uint32)), f"layer {l} scales"
            cache_vals.append(oracle.dequant_w8(ref_codes, ref_scales, B, NH, HS, maxT, fmt))
    for total, out in hist.items():
        o = out.float().cpu().numpy()
        for l in range(L):
            ref = oracle.attention_f32(qh[total - 1, l].reshape(-1), cache_vals[l], np.full(B, total, np.int32),
                                       B, NH, HS, maxT)
            assert_close(o[l], ref, dtype, f"{mode} layer {l} T={total}")
