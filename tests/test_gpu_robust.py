"""Robustness of the HIP decode attention on an MI355X (runs on the GPU box).

* Cache rows at and past a sequence's length hold garbage, as in the reference engine,
  which allocates its cache with cudaMalloc and never clears it
  (inference_gpt2_opt.cu:692-699): NaN and Inf bits (f32 / bf16), FP8 NaN codes 0x7F/0xFF
  and NaN / Inf row scales (8-bit).  Kernels that request rows before they know the length
  (a stale host hint, the device-planned first tile) must not let them into the result.
* The designated merger's bounded wait: a merger that stops waiting (forced from the host
  with a poll bound of 0, so every kernel still exits normally) computes its producers'
  segments itself, so the output still matches the oracle; it is counted in the
  workspace's status, and the partials its producers publish afterwards are never taken
  for a later call's.

Bars as in kvcases.TOL (FP32 1e-5, BF16 1e-2, 8-bit 2e-2 against the oracle on the
dequantised cache).
"""
import numpy as np
import pytest

from kvcases import FMT, HS, assert_close, make_case, out_tensor, to_device
from oracle import oracle

pytestmark = pytest.mark.gpu

ALL_DT = ["f32", "bf16", "int8", "fp8"]


def _kv():
    from cuda_gpt2_inference_amd import kvattn
    return kvattn


def poison_past_length(case):
    """Overwrite every cache row at or beyond each sequence's attended length, in place:
    even rows NaN, odd rows +Inf (K) / -Inf (V); 8-bit caches get FP8 NaN codes and NaN /
    Inf row scales.  The oracle never reads those rows."""
    B, NH, maxT = case.B, case.NH, case.maxT
    raw = case.cache_raw.reshape(2, B, NH, maxT, HS)
    sc = None if case.scale_raw is None else case.scale_raw.reshape(2, B, NH, maxT)
    for b, t in enumerate(case.totals):
        rows = np.arange(t, maxT)
        even, odd = rows[rows % 2 == 0], rows[rows % 2 == 1]
        if case.dtype == "f32":
            raw[:, b, :, even, :] = np.nan
            raw[0, b, :, odd, :] = np.inf
            raw[1, b, :, odd, :] = -np.inf
        elif case.dtype == "bf16":
            raw[:, b, :, even, :] = 0x7FC0
            raw[0, b, :, odd, :] = 0x7F80
            raw[1, b, :, odd, :] = 0xFF80
        else:
            raw[:, b, :, even, :] = 0x7F
            raw[:, b, :, odd, :] = 0xFF
            sc[:, b, :, even] = np.nan
            sc[:, b, :, odd] = np.inf
    return case


def _uniform(dtype, NH, maxT, total, seed):
    return poison_past_length(make_case(dtype, 1, NH, maxT, [total - 1], seed=seed))


def _decode(case, dev, strategy, len_hint, S=0, append=False):
    """One call with a single device length for the batch (lens_per_seq = 0), so that the
    host's hint may steer the first requests."""
    import torch
    kvattn = _kv()
    qkv, cache, scale, _ = to_device(case, dev)
    cur = torch.tensor([int(case.cur_lens[0])], dtype=torch.int32, device=dev)
    out = out_tensor(case, dev)
    ws = kvattn.Workspace(case.B, case.NH, case.maxT, S)
    fn = kvattn.append_decode if append else kvattn.decode
    fn(out, qkv, cache, case.B, case.NH, HS, case.maxT, kv_dtype=case.dtype, kv_scale=scale, cur_len=cur,
       len_hint=len_hint, S=S, strategy=strategy, **ws.kwargs())
    torch.cuda.synchronize()
    assert ws.status() == 0
    return out.float().cpu().numpy(), cache, scale


@pytest.mark.parametrize("dtype", ALL_DT)
def test_fused_single_stale_hint_ignores_rows_past_length(dev, dtype):
    """fused_single requests its one tile per wave for the hinted 256 positions before it
    reads the device length (100 or 201 positions)."""
    for total in (100, 201):
        case = _uniform(dtype, 12, 256, total, seed=300 + total)
        got, _, _ = _decode(case, dev, "fused_single", len_hint=255)
        assert_close(got, case.reference(), dtype, f"fused_single stale hint T={total}")


@pytest.mark.parametrize("dtype", ALL_DT)
def test_fused_single_short_tiles(dev, dtype):
    """Hinted lengths up to 128 take fused_single's 4 waves of 32-row tiles: exact hints at
    and around the tile edges, a stale hint longer than the device length (rows past it are
    poisoned), and hints shorter than it, whose device length leaves the one-tile-per-wave
    shape for the scores staged in LDS (up to 700 positions)."""
    for maxT, hint_total, total in ((256, 1, 1), (256, 32, 32), (256, 33, 33), (1024, 100, 100), (256, 128, 128),
                                    (256, 128, 60), (1024, 100, 230), (1024, 64, 700)):
        case = _uniform(dtype, 12, maxT, total, seed=400 + total + maxT)
        for strategy in ("fused_single", "auto"):
            got, _, _ = _decode(case, dev, strategy, len_hint=hint_total - 1)
            assert_close(got, case.reference(), dtype, f"{strategy} hint {hint_total} T={total} maxT={maxT}")
    case = poison_past_length(make_case(dtype, 8, 12, 512, [96] * 8, seed=470))
    got, _, _ = _decode(case, dev, "auto", len_hint=96)
    assert_close(got, case.reference(), dtype, "auto B=8 hint 97 T=97")


@pytest.mark.parametrize("dtype", ALL_DT)
def test_fused_single_short_tiles_per_sequence_lengths(dev, dtype):
    """Per-sequence lengths with a hinted longest length up to 128 take the 32-row tiles too
    (the hint picks the shape; no tile is requested before the lengths): rows past each
    sequence's length are poisoned, and a stale hint shorter than some lengths sends those
    sequences to the scores staged in LDS."""
    import torch
    kvattn = _kv()
    for maxT, lens, hint in ((256, [1, 37, 64, 128, 100, 5], 128), (1024, [90, 300, 17, 128, 700, 64], 100)):
        B = len(lens)
        case = poison_past_length(make_case(dtype, B, 12, maxT, np.array(lens) - 1, seed=490 + maxT))
        qkv, cache, scale, cur = to_device(case, dev)
        out = out_tensor(case, dev)
        ws = kvattn.Workspace(B, 12, maxT, 0)
        kvattn.decode(out, qkv, cache, B, 12, HS, maxT, kv_dtype=dtype, kv_scale=scale, cur_len=cur,
                      lens_per_seq=True, len_hint=hint - 1, strategy="auto", **ws.kwargs())
        torch.cuda.synchronize()
        assert_close(out.float().cpu().numpy(), case.reference(), dtype, f"lens {lens} hint {hint}")


@pytest.mark.parametrize("B,NH", [(24, 12), (21, 12), (16, 17)])
def test_fused_single_fp32_across_the_head_count_switch(dev, B, NH):
    """FP32 fused_single takes 4 waves of 64-row tiles beyond 256 heads (B * NH = 288 and
    272 here) and 8 waves of 32-row tiles up to it (252): exact hints from 129 to 256
    positions, a stale hint longer than the device length, and one shorter than it whose
    device length needs the scores staged in LDS."""
    for maxT, hint_total, total in ((256, 129, 129), (256, 200, 200), (256, 256, 256), (256, 256, 150),
                                    (1024, 150, 600)):
        case = poison_past_length(make_case("f32", B, NH, maxT, [total - 1] * B, seed=480 + total))
        got, _, _ = _decode(case, dev, "fused_single", len_hint=hint_total - 1)
        assert_close(got, case.reference(), "f32", f"B={B} NH={NH} hint {hint_total} T={total} maxT={maxT}")


@pytest.mark.parametrize("dtype", ALL_DT)
def test_device_planned_designated_ignores_rows_past_length(dev, dtype):
    """AUTO without a hint plans on the device; the designated instance requests its
    nominal first tile (segment 0: up to 256 rows) before the length: T below and above 256."""
    kvattn = _kv()
    assert kvattn.plan(1, 12, HS, 1024, kv_dtype=dtype, len_hint=-1)[0] == kvattn.SPLIT_DESIGNATED
    for total in (70, 200, 300, 700):
        case = _uniform(dtype, 12, 1024, total, seed=320 + total)
        got, _, _ = _decode(case, dev, "auto", len_hint=-1)
        assert_close(got, case.reference(), dtype, f"device-planned designated T={total}")


@pytest.mark.parametrize("dtype", ALL_DT)
@pytest.mark.parametrize("strategy", ["designated", "lastblock", "split_merge", "graph", "coop"])
def test_hinted_split_ignores_rows_past_length(dev, dtype, strategy):
    """A host hint of 1024 positions (segments of fixed rows, first tiles requested before
    the length) while the device length is 600 or 130."""
    for total in (600, 130):
        case = _uniform(dtype, 12, 1024, total, seed=340 + total)
        got, _, _ = _decode(case, dev, strategy, len_hint=1023)
        assert_close(got, case.reference(), dtype, f"{strategy} hint 1024, T={total}")


@pytest.mark.parametrize("dtype", ALL_DT)
def test_append_decode_ignores_rows_past_length(dev, dtype):
    """Append and attend in one launch over a poisoned cache: the fresh row replaces the
    garbage at position cur_len, every row after it stays out of the result."""
    for strategy, len_hint, total, maxT in (("auto", -1, 500, 1024), ("auto", 1023, 500, 1024),
                                            ("fused_single", 255, 150, 256), ("fused_single", 99, 100, 256),
                                            ("fused_single", 63, 150, 256)):
        case = _uniform(dtype, 12, maxT, total, seed=360 + total)
        got, cache, scale = _decode(case, dev, strategy, len_hint=len_hint, append=True)
        # The reference: the oracle's append into the host copy, then attention over it.
        B, NH = case.B, case.NH
        if dtype in ("int8", "fp8"):
            codes, scales = case.cache_raw.copy(), case.scale_raw.copy()
            oracle.cache_write_w8(codes, scales, case.qkv_host, case.cur_lens, B, NH, HS, maxT, FMT[dtype])
            assert np.array_equal(cache.cpu().numpy(), codes)
            assert np.array_equal(scale.cpu().numpy().view(np.uint32), scales.view(np.uint32))
            host = oracle.dequant_w8(codes, scales, B, NH, HS, maxT, FMT[dtype])
        elif dtype == "bf16":
            import torch
            bits = case.cache_raw.copy()
            oracle.cache_write(bits, case.qkv_raw, case.cur_lens, B, NH, HS, maxT)
            assert np.array_equal(cache.view(torch.int16).cpu().numpy().view(np.uint16), bits)
            host = oracle.bf16_decode(bits)
        else:
            host = case.cache_raw.copy()
            oracle.cache_write(host, case.qkv_raw, case.cur_lens, B, NH, HS, maxT)
            assert np.array_equal(cache.cpu().numpy().view(np.uint32), host.view(np.uint32))
        ref = oracle.attention_f32(case.qkv_host, host, case.totals, B, NH, HS, maxT)
        assert_close(got, ref, dtype, f"append_decode {strategy} hint {len_hint} T={total}")


@pytest.mark.parametrize("dtype", ALL_DT)
def test_designated_fallback_matches_oracle_and_workspace_stays_usable(dev, dtype):
    """Poll bound 0: every multi-segment merger stops waiting at once and computes its
    producers' segments on its own wave (counted in the workspace status) while the
    producers publish anyway.  Its output matches the oracle.  The next call on the same
    workspace, with different q, K and V, must not take those late partials for its own
    and matches the oracle; the count stays until cleared."""
    import torch
    kvattn = _kv()
    B, NH, maxT, total = 1, 12, 1024, 1024
    first = make_case(dtype, B, NH, maxT, [total - 1], seed=401)
    second = make_case(dtype, B, NH, maxT, [total - 1], seed=402)
    ws = kvattn.Workspace(B, NH, maxT, 8)
    assert ws.status() == 0
    for strategy, S in (("designated", 8), ("auto", 0)):
        qkv, cache, scale, cur = to_device(first, dev)
        out = out_tensor(first, dev)
        prev = kvattn.set_merge_poll_limit(0)
        try:
            kvattn.decode(out, qkv, cache, B, NH, HS, maxT, kv_dtype=dtype, kv_scale=scale, cur_len=cur,
                          len_hint=total - 1, S=S, strategy=strategy, **ws.kwargs())
            torch.cuda.synchronize()
        finally:
            kvattn.set_merge_poll_limit(prev)
        assert_close(out.float().cpu().numpy(), first.reference(), dtype, f"{strategy}: merger's own fallback")
        assert ws.status() == B * NH
        qkv2, cache2, scale2, cur2 = to_device(second, dev)
        out2 = out_tensor(second, dev)
        for rep in range(3):
            kvattn.decode(out2, qkv2, cache2, B, NH, HS, maxT, kv_dtype=dtype, kv_scale=scale2, cur_len=cur2,
                          len_hint=total - 1, S=S, strategy=strategy, **ws.kwargs())
            torch.cuda.synchronize()
            assert_close(out2.float().cpu().numpy(), second.reference(), dtype,
                         f"{strategy}: call {rep + 1} after the fallback")
        assert ws.status() == B * NH, "the count is sticky until cleared"
        assert ws.status(clear=True) == B * NH
        assert ws.status() == 0


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_designated_empty_segments_ignore_stale_words(dev, dtype):
    """The reference partition leaves segments empty when the length is short (10 positions
    over 8 segments: segments 5..7).  Their slots publish nothing, so they still hold the words
    of an earlier call: here NaN partials, from a call whose V rows are all NaN.  The merger
    requests every slot of its batch and must drop those words by more than a zero weight
    (0 x NaN is NaN): the second call matches the oracle."""
    import torch
    kvattn = _kv()
    B, NH, maxT, S = 1, 12, 1024, 8
    ws = kvattn.Workspace(B, NH, maxT, S)
    first = make_case(dtype, B, NH, maxT, [maxT - 1], seed=431)
    qkv, cache, scale, cur = to_device(first, dev)
    cache.view(2, -1)[1].fill_(float("nan"))
    out = out_tensor(first, dev)
    kvattn.decode(out, qkv, cache, B, NH, HS, maxT, kv_dtype=dtype, kv_scale=scale, cur_len=cur, len_hint=maxT - 1,
                  S=S, strategy="designated", **ws.kwargs())
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all(), "the first call should have published NaN partials"
    second = make_case(dtype, B, NH, maxT, [9], seed=432)
    qkv2, cache2, scale2, cur2 = to_device(second, dev)
    out2 = out_tensor(second, dev)
    kvattn.decode(out2, qkv2, cache2, B, NH, HS, maxT, kv_dtype=dtype, kv_scale=scale2, cur_len=cur2, len_hint=9,
                  S=S, strategy="designated", **ws.kwargs())
    torch.cuda.synchronize()
    assert_close(out2.float().cpu().numpy(), second.reference(), dtype, "short length after NaN partials")
    assert ws.status() == 0


@pytest.mark.parametrize("dtype", ALL_DT)
def test_designated_fallback_with_fresh_row_equals_normal_path(dev, dtype):
    """Append and attend in one launch with the merger's fallback forced (poll bound 0): the
    merger's own computation of the segment holding the current position takes the fresh row
    as its producer does, so output and cache bytes equal those of the normal path, and the
    output matches the oracle over the appended cache (poisoned rows past the length)."""
    import torch
    kvattn = _kv()
    B, NH, maxT, total = 1, 12, 1024, 1000
    case = _uniform(dtype, NH, maxT, total, seed=421)
    res = {}
    for bound in (None, 0):
        qkv, cache, scale, cur = to_device(case, dev)
        out = out_tensor(case, dev)
        ws = kvattn.Workspace(B, NH, maxT, 0)
        prev = kvattn.set_merge_poll_limit(0) if bound == 0 else None
        try:
            kvattn.append_decode(out, qkv, cache, B, NH, HS, maxT, kv_dtype=dtype, kv_scale=scale, cur_len=cur,
                                 len_hint=total - 1, strategy="auto", **ws.kwargs())
            torch.cuda.synchronize()
        finally:
            if prev is not None:
                kvattn.set_merge_poll_limit(prev)
        assert ws.status() == (B * NH if bound == 0 else 0)
        res[bound] = (out.float().cpu().numpy(), cache.view(torch.uint8).cpu().numpy().copy(),
                      None if scale is None else scale.cpu().numpy().view(np.uint32).copy())
    got, c0, s0 = res[0]
    ref_out, c1, s1 = res[None]
    assert np.array_equal(c0, c1), "cache bytes differ between the fallback and the normal path"
    if s0 is not None:
        assert np.array_equal(s0, s1)
    assert_close(got, ref_out, dtype, "fallback against the normal path")


def test_cooperative_barrier_give_up_is_reported(dev):
    """The cooperative strategy's grid barrier is bounded like the designated merger's wait:
    with a poll bound of 0 every merger that is not the last to arrive gives up (NaN,
    counted); with the bound restored the next calls on the same workspace, with other
    inputs and another segment count, match the oracle."""
    import torch
    kvattn = _kv()
    B, NH, maxT, total = 1, 12, 1024, 1024
    first = make_case("bf16", B, NH, maxT, [total - 1], seed=411)
    second = make_case("bf16", B, NH, maxT, [total - 1], seed=412)
    ws = kvattn.Workspace(B, NH, maxT, 16)
    qkv, cache, _, cur = to_device(first, dev)
    out = out_tensor(first, dev)
    prev = kvattn.set_merge_poll_limit(0)
    try:
        kvattn.decode(out, qkv, cache, B, NH, HS, maxT, kv_dtype="bf16", cur_len=cur, len_hint=total - 1, S=8,
                      strategy="coop", **ws.kwargs())
        torch.cuda.synchronize()
    finally:
        kvattn.set_merge_poll_limit(prev)
    got = out.float().cpu().numpy().reshape(B * NH, HS)
    gave_up = int(np.isnan(got).all(axis=1).sum())
    assert gave_up >= B * NH - 1 and ws.status(clear=True) == gave_up
    qkv2, cache2, _, cur2 = to_device(second, dev)
    for S in (8, 16, 5):
        out2 = out_tensor(second, dev)
        kvattn.decode(out2, qkv2, cache2, B, NH, HS, maxT, kv_dtype="bf16", cur_len=cur2, len_hint=total - 1, S=S,
                      strategy="coop", **ws.kwargs())
        torch.cuda.synchronize()
        assert_close(out2.float().cpu().numpy(), second.reference(), "bf16", f"coop S={S} after the give-up")
    assert ws.status() == 0


def _xcd_words(ws):
    """The workspace's status words 4 and 5: designated producers of XCD-local grids that
    published write-through because their merger's XCD word named another XCD (4) or was not
    there yet when they looked (5)."""
    w = ws.buf[:256].cpu().numpy().view(np.uint32)
    return int(w[4]), int(w[5])


@pytest.mark.parametrize("rot", [0, 1, 3, 7])
def test_designated_producers_on_other_xcds(dev, rot):
    """kvattn_set_xcd_layout_offset(rot) moves every producer of an XCD-local designated grid
    rot XCDs away from its merger, where its plain stores would stay in an L2 the merger does
    not poll.  Each producer reads the XCD its merger publishes and then stores write-through,
    so every output still matches the oracle and no merger stops waiting (a plain-store
    producer elsewhere would hold its merger for the whole poll bound and count a timeout).
    With rot != 0 every producer counts itself as remote (or as having not seen the merger's
    word yet); with rot = 0 none finds its merger elsewhere.  Every kernel exits normally:
    the setting only rotates the host's grid layout."""
    import torch
    kvattn = _kv()
    calls = [("bf16", 1, 12, 1024, [1023], True), ("bf16", 1, 12, 1024, [1023], False),
             ("int8", 1, 12, 1024, [1023], True), ("f32", 1, 8, 1024, [700], True),
             ("fp8", 2, 12, 700, [699, 299], True), ("bf16", 3, 4, 2048, [2047, 1500, 900], False)]
    prev = kvattn.set_xcd_layout_offset(rot)
    try:
        for i, (dtype, B, NH, maxT, cur, hinted) in enumerate(calls):
            case = make_case(dtype, B, NH, maxT, cur, seed=1200 + 10 * rot + i)
            qkv, cache, scale, curd = to_device(case, dev)
            out = out_tensor(case, dev)
            ws = kvattn.Workspace(B, NH, maxT, 0)
            hint = int(case.cur_lens.max()) if hinted else -1
            st, slots, rows = kvattn.plan(B, NH, HS, maxT, kv_dtype=dtype, len_hint=hint)
            assert st == kvattn.SPLIT_DESIGNATED and B * NH >= 8, (dtype, B, NH, st)
            rows = rows if rows > 0 else 128
            producers = sum(NH * (-(-int(t) // rows) - 1) for t in case.totals)
            before = _xcd_words(ws)
            kvattn.decode(out, qkv, cache, B, NH, HS, maxT, kv_dtype=dtype, kv_scale=scale, cur_len=curd,
                          lens_per_seq=B > 1, len_hint=hint, **ws.kwargs())
            torch.cuda.synchronize()
            what = f"rot {rot} call {i} {dtype} B={B} NH={NH}"
            assert_close(out.float().cpu().numpy(), case.reference(), dtype, what)
            assert ws.status() == 0, f"{what}: a merger stopped waiting"
            after = _xcd_words(ws)
            remote, unseen = after[0] - before[0], after[1] - before[1]
            if rot:
                assert remote + unseen == producers and remote > 0, f"{what}: remote {remote} unseen {unseen} " \
                                                                     f"of {producers} producers"
            else:
                assert remote == 0, f"{what}: {remote} producers found their merger on another XCD"
    finally:
        kvattn.set_xcd_layout_offset(prev)
