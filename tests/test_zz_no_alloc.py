"""kvattn_decode_static, the entry point that allocates nothing (runs on an MI355X).

Its output must equal kvattn_decode's on the same inputs with a workspace of the caller's,
bit for bit (the same kernels, the same plan), on two calls in a row, the second with a
smaller input; both are also checked against the oracle at kvcases.TOL.  Every call goes
through the C ABI (ctypes, raw device pointers).
"""
import ctypes

import numpy as np
import pytest

from kvcases import HS, assert_close, make_case, out_tensor, to_device

pytestmark = pytest.mark.gpu


def _kv():
    from cuda_gpt2_inference_amd import kvattn
    return kvattn


def _static(kvattn, out, qkv, cache, scale, cur, case, S, strategy, lens_per_seq, len_hint):
    import torch
    return kvattn.lib().kvattn_decode_static(
        out.data_ptr(), qkv.data_ptr(), cache.data_ptr(), None if scale is None else scale.data_ptr(),
        case.B, case.NH, HS, case.maxT, cur.data_ptr(), int(lens_per_seq), int(len_hint), int(S),
        kvattn.strategy_code(strategy), kvattn.kv_dtype_code(case.dtype), torch.cuda.current_stream().cuda_stream)


def _with_workspace(kvattn, out, qkv, cache, scale, cur, case, S, strategy, lens_per_seq, len_hint):
    import torch
    ws = kvattn.Workspace(case.B, case.NH, case.maxT, S)
    return kvattn.lib().kvattn_decode(
        out.data_ptr(), qkv.data_ptr(), cache.data_ptr(), None if scale is None else scale.data_ptr(),
        case.B, case.NH, HS, case.maxT, cur.data_ptr(), int(lens_per_seq), int(len_hint), ws.buf.data_ptr(),
        ctypes.c_size_t(ws.nbytes), int(S), kvattn.strategy_code(strategy), kvattn.kv_dtype_code(case.dtype),
        torch.cuda.current_stream().cuda_stream), ws


def _compare(dev, case, strategy, S, lens_per_seq, len_hint, what):
    import torch
    kvattn = _kv()
    qkv, cache, scale, cur = to_device(case, dev)
    if not lens_per_seq:
        cur = cur[:1].contiguous()
    a, b = out_tensor(case, dev), out_tensor(case, dev)
    st = _static(kvattn, a, qkv, cache, scale, cur, case, S, strategy, lens_per_seq, len_hint)
    assert st == 0, f"{what}: kvattn_decode_static: {kvattn.strerror(st)}"
    st, ws = _with_workspace(kvattn, b, qkv, cache, scale, cur, case, S, strategy, lens_per_seq, len_hint)
    assert st == 0, f"{what}: kvattn_decode: {kvattn.strerror(st)}"
    torch.cuda.synchronize()
    ga, gb = a.float().cpu().numpy(), b.float().cpu().numpy()
    assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32)), f"{what}: static and workspace outputs differ"
    assert_close(ga, case.reference(), case.dtype, what)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "int8", "fp8"])
@pytest.mark.parametrize("strategy,S,hinted", [("auto", 0, True), ("auto", 0, False), ("designated", 8, True),
                                               ("lastblock", 0, True), ("split_merge", -128, False),
                                               ("fused_single", 0, True)])
def test_static_equals_workspace_two_calls_second_smaller(dev, dtype, strategy, S, hinted):
    """Call 1: B=3, NH=6, maxT=1100, ragged lengths; call 2: B=1, NH=4, maxT=700 (fewer
    heads, so its counters and partials sit where call 1 left other values)."""
    big = make_case(dtype, 3, 6, 1100, np.array([1100, 517, 260]) - 1, seed=501)
    small = make_case(dtype, 1, 4, 700, [699 if strategy != "fused_single" else 199], seed=502)
    for i, case in enumerate((big, small)):
        lens_per_seq = case.B > 1
        hint = int(case.cur_lens.max()) if hinted else -1
        _compare(dev, case, strategy, S, lens_per_seq, hint, f"{dtype} {strategy} S={S} call {i + 1}")


def test_static_rejects_what_it_cannot_serve(dev):
    import torch
    kvattn = _kv()
    case = make_case("bf16", 1, 2, 256, [255], seed=503)
    qkv, cache, scale, cur = to_device(case, dev)
    out = out_tensor(case, dev)
    for strategy in ("coop", "graph"):
        st = _static(kvattn, out, qkv, cache, scale, cur, case, 8, strategy, False, 255)
        assert st == kvattn.ERR_STRATEGY, strategy
    # A plan whose partials do not fit in the 8 MiB array: 64 x 12 heads x 128 slots (C5's
    # shape); refused before anything reads the (small) buffers passed here.
    st = kvattn.lib().kvattn_decode_static(out.data_ptr(), qkv.data_ptr(), cache.data_ptr(), None, 64, 12, HS, 8192,
                                           cur.data_ptr(), 0, -1, -64, kvattn.SPLIT_MERGE, kvattn.KV_BF16,
                                           torch.cuda.current_stream().cuda_stream)
    assert st == kvattn.ERR_WORKSPACE
    torch.cuda.synchronize()


def test_static_auto_takes_the_general_plan_when_the_tuned_one_does_not_fit(dev):
    """B=64, NH=12, maxT=4096, BF16, one length with a hint: AUTO's tuned plan streams 256-row
    segments (16 per head, 12,288 slots, ~11 MB of partials and tags: more than the 8 MiB
    array holds), so kvattn_decode_static takes the general plan, 512-row segments through
    the same split + merge kernels (8 per head).  Its output must equal, bit for bit,
    kvattn_decode's with that plan asked for explicitly (split_merge, S = -512) on a
    workspace of the caller's; 8 sampled heads are also checked against the oracle."""
    import torch
    from oracle import oracle
    kvattn = _kv()
    B, NH, maxT, T = 64, 12, 4096, 4096
    assert kvattn.plan(B, NH, HS, maxT, kv_dtype="bf16", len_hint=T - 1) == (kvattn.SPLIT_MERGE, 16, 256)
    g = torch.Generator(device=dev)
    g.manual_seed(77)
    cache = torch.randn(2 * B * NH * maxT * HS, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    qkv = torch.randn(B * 3 * NH * HS, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    cur = torch.tensor([T - 1], dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    a = torch.full((B * NH * HS,), float("nan"), dtype=torch.bfloat16, device=dev)
    st = kvattn.lib().kvattn_decode_static(a.data_ptr(), qkv.data_ptr(), cache.data_ptr(), None, B, NH, HS, maxT,
                                           cur.data_ptr(), 0, T - 1, 0, kvattn.AUTO, kvattn.KV_BF16, stream)
    assert st == 0, kvattn.strerror(st)
    b = torch.full_like(a, float("nan"))
    ws = kvattn.Workspace(B, NH, maxT, -512)
    kvattn.decode(b, qkv, cache, B, NH, HS, maxT, kv_dtype="bf16", cur_len=cur, len_hint=T - 1, S=-512,
                  strategy="split_merge", **ws.kwargs())
    torch.cuda.synchronize()
    ga, gb = a.float().cpu().numpy(), b.float().cpu().numpy()
    assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32)), "static AUTO differs from split_merge S=-512"
    kv5 = cache.view(2, B, NH, maxT, HS)
    q = qkv.float().view(B, 3, NH, HS)
    rng = np.random.RandomState(78)
    for bb, h in zip(rng.randint(0, B, 8), rng.randint(0, NH, 8)):
        k = kv5[0, bb, h].float().cpu().numpy()
        v = kv5[1, bb, h].float().cpu().numpy()
        q1 = np.zeros((1, 3, 1, HS), np.float32)
        q1[0, 0, 0] = q[bb, 0, h].cpu().numpy()
        ref = oracle.attention_f32(q1.reshape(-1), np.stack([k, v]).reshape(-1), T, 1, 1, HS, T)
        assert_close(ga.reshape(B, NH, HS)[bb, h], ref, "bf16", f"static AUTO b={bb} h={h}")
