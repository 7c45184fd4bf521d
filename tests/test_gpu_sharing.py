"""Buffers shared between calls (runs on an MI355X): tagged partial words across hardware
queues, the static scratch array shared by kvattn_decode_static and kvattn_forward_large, and
one caller workspace serving plans of different head counts.

HIP spreads its streams over several hardware queues, and every queue counts its dispatch ids
from 0, so calls on two streams carry equal ids all the time.  The designated merger's words
carry the dispatch id and a hash of the queue address, so a word another queue's call left in
a shared slot is never taken for this call's.  The alternating tests below line the two
queues' dispatch counters up first, so that without the queue term every call on one stream
would find words with its own tag left by the other stream's previous call.
"""
import numpy as np
import pytest

from kvcases import HS, assert_close, make_case, out_tensor, to_device

pytestmark = pytest.mark.gpu

ALL_DT = ["f32", "bf16", "int8", "fp8"]


def _kv():
    from cuda_gpt2_inference_amd import kvattn
    return kvattn


def _identity(kvattn, stream, dev):
    """(dispatch id, queue address, tag) of one dispatch on `stream`."""
    import torch
    buf = torch.zeros(3, dtype=torch.int64, device=dev)
    # The zero fill runs on the current stream: order `stream` after it, or the fill can land
    # after the identity dispatch's store.
    stream.wait_stream(torch.cuda.current_stream())
    kvattn.call_identity(buf, stream=stream)
    stream.synchronize()
    return [int(v) & (2**64 - 1) for v in buf.cpu().numpy().view(np.uint64)]


def _two_streams_on_two_queues(kvattn, dev):
    """Two torch streams whose dispatches go to different hardware queues, or None."""
    import torch
    streams = [torch.cuda.Stream(device=dev) for _ in range(8)]
    seen = {}
    for s in streams:
        q = _identity(kvattn, s, dev)[1]
        seen.setdefault(q, s)
        if len(seen) == 2:
            return list(seen.values())
    return None


def _align(kvattn, a, b, dev):
    """Pad the stream whose queue is behind with identity dispatches so that the next dispatch
    ids of a and b are equal (best effort, at most four rounds: synchronisations and copies may
    add packets to a queue).  Returns whether they were lined up."""
    import torch
    buf = torch.zeros(9, dtype=torch.int64, device=dev)
    torch.cuda.synchronize()
    for _ in range(4):
        kvattn.call_identity(buf[0:3], stream=a)
        kvattn.call_identity(buf[3:6], stream=b)
        a.synchronize()
        b.synchronize()
        ids = buf.cpu().numpy().view(np.uint64)
        ia, ib = int(ids[0]), int(ids[3])
        if ia == ib:
            return True
        lag, n = (a, ib - ia) if ia < ib else (b, ia - ib)
        for _ in range(min(n, 4096)):
            kvattn.call_identity(buf[6:9], stream=lag)
    return False


def test_call_identity_distinct_across_queues(dev):
    """Dispatch ids coincide across hardware queues; tags do not.  On one queue the tag is the
    dispatch id plus a fixed offset (so 2^31 consecutive dispatches have distinct tags)."""
    import torch
    kvattn = _kv()
    streams = [torch.cuda.Stream(device=dev) for _ in range(6)] + [torch.cuda.current_stream()]
    recs = [_identity(kvattn, s, dev) for _ in range(4) for s in streams]
    queues = {q for _, q, _ in recs}
    if len(queues) < 2:
        pytest.skip("every stream shares one hardware queue here")
    for d, q, t in recs:
        assert t >> 31 == 1 and t < 2**32, f"tag {t:#x}: top bit of 32 not set"
    offset = {}
    for d, q, t in recs:
        off = ((t & 0x7FFFFFFF) - (d & 0x7FFFFFFF)) % 2**31
        assert offset.setdefault(q, off) == off, f"queue {q:#x}: tag minus dispatch id not constant"
    coincide = 0
    for i, (d1, q1, t1) in enumerate(recs):
        for d2, q2, t2 in recs[i + 1:]:
            if (d1, q1) != (d2, q2):
                assert t1 != t2, f"dispatch {d1} on {q1:#x} and {d2} on {q2:#x} share tag {t1:#x}"
            if d1 == d2 and q1 != q2:
                coincide += 1
    assert coincide > 0, "no pair of dispatches with equal ids on different queues was observed"


def _alternate(kvattn, dev, call, n_iter=16):
    """call(i, stream) on two streams of different hardware queues in alternation, each call
    ordered after the other stream's previous one by an event; their dispatch counters are
    lined up first.  Returns the per-call outputs (list of (i, out tensor, case))."""
    import torch
    pair = _two_streams_on_two_queues(kvattn, dev)
    if pair is None:
        pytest.skip("every stream shares one hardware queue here")
    a, b = pair
    _align(kvattn, a, b, dev)
    ev_a, ev_b = torch.cuda.Event(), torch.cuda.Event()
    ev_b.record(b)
    results = []
    for i in range(n_iter):
        for s, ev_wait, ev_rec in ((a, ev_b, ev_a), (b, ev_a, ev_b)):
            s.wait_event(ev_wait)
            results.append(call(len(results), s))
            ev_rec.record(s)
    torch.cuda.synchronize()
    return results


def _cases(dtype, n, B, NH, maxT, seed):
    return [make_case(dtype, B, NH, maxT, [maxT - 1 - 3 * (k % 5)] * B, seed=seed + k) for k in range(n)]


@pytest.mark.parametrize("dtype", ["bf16", "int8"])
def test_designated_two_streams_one_workspace(dev, dtype):
    """Ordered designated calls (GPT-2 layer, 8 segments) on two streams in alternation,
    sharing one caller workspace, every output against the oracle, no merge timeout."""
    import torch
    kvattn = _kv()
    B, NH, maxT = 1, 12, 1024
    cases = _cases(dtype, 4, B, NH, maxT, 700)
    dev_in = [to_device(c, dev) for c in cases]
    ws = kvattn.Workspace(B, NH, maxT, 8)
    outs = [out_tensor(cases[0], dev) for _ in range(32)]
    torch.cuda.synchronize()

    def call(i, s):
        c = i % len(cases)
        qkv, cache, scale, cur = dev_in[c]
        kvattn.decode(outs[i], qkv, cache, B, NH, HS, maxT, kv_dtype=dtype, kv_scale=scale, cur_len=cur[:1],
                      len_hint=int(cases[c].cur_lens[0]), S=8, strategy="designated", stream=s, **ws.kwargs())
        return i, c

    for i, c in _alternate(kvattn, dev, call):
        assert_close(outs[i].float().cpu().numpy(), cases[c].reference(), dtype, f"call {i} (case {c})")
    assert ws.status() == 0


@pytest.mark.parametrize("dtype", ["bf16", "fp8"])
def test_static_scratch_two_streams(dev, dtype):
    """kvattn_decode_static (AUTO: the designated merger) and kvattn_forward_large (B = 1: the
    designated merger over the reference partition) alternating on two streams, all in the one
    static scratch array, every output against the oracle, no merge timeout in the array."""
    import torch
    kvattn = _kv()
    B, NH, maxT, S = 1, 12, 1024, 8
    cases = _cases(dtype, 4, B, NH, maxT, 800)
    dev_in = [to_device(c, dev) for c in cases]
    outs = [out_tensor(cases[0], dev) for _ in range(32)]
    po = torch.empty(B * NH * S * HS, dtype=torch.float32, device=dev)
    pl = torch.empty(B * NH * S, dtype=torch.float32, device=dev)
    pm = torch.empty(B * NH * S, dtype=torch.float32, device=dev)
    kvattn.scratch_status(clear=True)
    torch.cuda.synchronize()

    def call(i, s):
        c = i % len(cases)
        qkv, cache, scale, cur = dev_in[c]
        if (i // 2) % 2 == 0:
            kvattn.decode_static(outs[i], qkv, cache, B, NH, HS, maxT, kv_dtype=dtype, kv_scale=scale,
                                 cur_len=cur[:1], len_hint=int(cases[c].cur_lens[0]), stream=s)
        else:
            kvattn.attention_forward_kv_large(outs[i], qkv, cache, B, NH, HS, maxT, po, pl, pm, S, kv_dtype=dtype,
                                              kv_scale=scale, cur_len=cur[:1], stream=s)
        return i, c

    for i, c in _alternate(kvattn, dev, call):
        assert_close(outs[i].float().cpu().numpy(), cases[c].reference(), dtype, f"call {i} (case {c})")
    assert kvattn.scratch_status() == 0


def test_forward_large_static_interleaved_with_decode_static(dev):
    """kvattn_forward_large with B = 1 (its single launch takes its words from the static
    scratch array) in every dtype, interleaved on one stream with kvattn_decode_static calls of
    other shapes and strategies in the same array; every output against the oracle."""
    import torch
    kvattn = _kv()
    NH, maxT, S = 12, 1024, 8
    po = torch.empty(NH * S * HS, dtype=torch.float32, device=dev)
    pl = torch.empty(NH * S, dtype=torch.float32, device=dev)
    pm = torch.empty(NH * S, dtype=torch.float32, device=dev)
    kvattn.scratch_status(clear=True)
    others = [("lastblock", 3, 6, 1100, np.array([1100, 517, 260]) - 1, 0),
              ("designated", 1, 4, 700, [699], 8),
              ("split_merge", 2, 5, 900, np.array([900, 33]) - 1, -128),
              ("auto", 1, 12, 1024, [300], 0)]
    for k, dtype in enumerate(ALL_DT):
        for rep in range(2):
            big = make_case(dtype, 1, NH, maxT, [1023 - 100 * rep], seed=900 + 10 * k + rep)
            qkv, cache, scale, cur = to_device(big, dev)
            out = out_tensor(big, dev)
            kvattn.attention_forward_kv_large(out, qkv, cache, 1, NH, HS, maxT, po, pl, pm, S, kv_dtype=dtype,
                                              kv_scale=scale, cur_len=cur)
            strategy, B2, NH2, maxT2, lens2, S2 = others[(k + rep) % len(others)]
            small = make_case(dtype, B2, NH2, maxT2, lens2, seed=950 + 10 * k + rep)
            q2, c2, s2, l2 = to_device(small, dev)
            out2 = out_tensor(small, dev)
            kvattn.decode_static(out2, q2, c2, B2, NH2, HS, maxT2, kv_dtype=dtype, kv_scale=s2, cur_len=l2,
                                 lens_per_seq=B2 > 1, len_hint=int(small.cur_lens.max()), S=S2, strategy=strategy)
            torch.cuda.synchronize()
            assert_close(out.float().cpu().numpy(), big.reference(), dtype, f"forward_large {dtype} #{rep}")
            assert_close(out2.float().cpu().numpy(), small.reference(), dtype, f"decode_static {strategy} {dtype}")
    assert kvattn.scratch_status() == 0


def test_workspace_counters_across_head_counts(dev):
    """One caller buffer, sized for the largest plan, serves last-block calls of 24, 96, 24,
    96 heads (B = 2, 8 with NH = 12) and split + merge calls in between: the counters sit in a
    region whose size follows from the buffer's, so the 96-head call never finds them on the
    24-head call's partials (where they would start at garbage, the merge would never fire and
    `out` would keep its stale values).  Every output against the oracle."""
    import torch
    kvattn = _kv()
    NH, maxT = 12, 1024
    nbytes = max(kvattn.workspace_bytes(B, NH, HS, maxT, 0) for B in (2, 8))
    buf = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    kvattn.workspace_init(buf, nbytes)
    kw = dict(workspace=buf, workspace_nbytes=nbytes)
    seq = [("lastblock", 2), ("lastblock", 8), ("split_merge", 2), ("lastblock", 2), ("split_merge", 8),
           ("lastblock", 8), ("lastblock", 2)]
    for i, (strategy, B) in enumerate(seq):
        case = make_case("bf16", B, NH, maxT, [1023 - 7 * i] * B, seed=1000 + i)
        qkv, cache, _, cur = to_device(case, dev)
        out = out_tensor(case, dev)
        assert kvattn.plan(B, NH, HS, maxT, kv_dtype="bf16", len_hint=int(case.cur_lens[0]),
                           strategy=strategy)[1] > 1
        kvattn.decode(out, qkv, cache, B, NH, HS, maxT, kv_dtype="bf16", cur_len=cur[:1],
                      len_hint=int(case.cur_lens[0]), strategy=strategy, **kw)
        torch.cuda.synchronize()
        assert_close(out.float().cpu().numpy(), case.reference(), "bf16", f"call {i} {strategy} B={B}")
