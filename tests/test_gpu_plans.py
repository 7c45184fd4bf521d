"""AUTO's plans for batches and long contexts on an MI355X: one shape per branch of the plan
choice, with a length hint (one length for the batch) and without one (the plan a captured
graph replays at every length), checked against the oracle.

Each case first asserts, through kvattn_plan, that AUTO takes the branch it is there for
(the one-segment-per-head last-block plan, the designated merger on grids of up to 768
workgroups, or the split + merge streaming plans of 256 or 512 rows).  Inputs are drawn on
the device from torch's seeded generator (8-bit caches: random codes and row scales), as the
bandwidth-bound shapes hold 64-100 MB of cache.  Then:
- 16 sampled (b,h) (and the first and last) against the oracle at kvcases.TOL, from their
  rows copied back (8-bit rows decoded by the oracle's dequantiser);
- every (b,h) inside the hull min_j V <= out <= max_j V of its rows;
- every (b,h) within TOL of the last-block merge over the reference partition (S = 8).
"""
import numpy as np
import pytest

from kvcases import HS, TOL, assert_close
from oracle import oracle

pytestmark = pytest.mark.gpu


def _kv():
    from cuda_gpt2_inference_amd import kvattn
    return kvattn


# dtype, B, NH, maxT, attended length T, (strategy name, segment slots, rows per segment)
CASES = [
    # bandwidth bound (100 MB of BF16): 256-row segments, split + merge kernels
    ("bf16", 32, 12, 1024, 1024, ("split_merge", 4, 256)),
    # bandwidth bound INT8 (80 MB): 256-row segments
    ("int8", 12, 12, 4096, 4096, ("split_merge", 16, 256)),
    # bandwidth bound INT8 at a context of 8192 (71 MB): 512-row segments
    ("int8", 2, 32, 8192, 8192, ("split_merge", 16, 512)),
    # long contexts: at most 64 segments per head, longer rows in the streaming shape
    ("bf16", 1, 12, 32768, 32000, ("split_merge", 64, 512)),
    ("int8", 1, 12, 65536, 65536, ("split_merge", 64, 1024)),
    # 192 heads of at most 512 rows: one segment per head, no merge
    ("fp8", 16, 12, 512, 512, ("lastblock", 1, 512)),
    ("int8", 32, 12, 512, 480, ("lastblock", 1, 512)),
    ("bf16", 16, 12, 512, 400, ("lastblock", 1, 512)),
    # designated merger on 768 workgroups
    ("bf16", 8, 12, 1024, 1024, ("designated", 8, 128)),
    ("fp8", 4, 12, 2048, 2000, ("designated", 16, 128)),
    # designated merger, 8-bit streaming tiles (256-row segments, 192 workgroups)
    ("int8", 1, 12, 4096, 4096, ("designated", 16, 256)),
    # up to 64 heads with long segments: designated grids past 768 workgroups
    ("bf16", 2, 25, 4096, 4096, ("designated", 16, 256)),
    ("fp8", 1, 49, 8192, 8000, ("designated", 16, 512)),
    # FP32 beyond the designated window keeps the general plan (last-block merge)
    ("f32", 16, 12, 1024, 1024, ("lastblock", 4, 256)),
]


def _inputs(torch, dev, dtype, B, NH, maxT, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    n = 2 * B * NH * maxT * HS
    act = torch.float32 if dtype == "f32" else torch.bfloat16
    qkv = torch.randn(B * 3 * NH * HS, generator=g, device=dev, dtype=torch.float32).to(act)
    if dtype in ("f32", "bf16"):
        return qkv, torch.randn(n, generator=g, device=dev, dtype=torch.float32).to(act), None
    codes = torch.randint(0, 256, (n,), generator=g, device=dev, dtype=torch.int32)
    if dtype == "fp8":
        codes = codes & 0x77          # finite E4M3 codes only (0x7f / 0xff are NaN)
    else:
        codes = torch.where(codes == 128, torch.zeros_like(codes), codes)   # the quantiser's range
    scale = torch.rand(2 * B * NH * maxT, generator=g, device=dev, dtype=torch.float32) * 0.05 + 1e-3
    return qkv, codes.to(torch.uint8), scale


def _rows_f32(cache, scale, dtype, B, NH, maxT, b, h, T):
    """K and V rows [T][HS] of (b,h) as the kernels see them, as float32 host arrays."""
    kv = cache.view(2, B, NH, maxT, HS)
    if dtype in ("f32", "bf16"):
        return kv[0, b, h, :T].float().cpu().numpy(), kv[1, b, h, :T].float().cpu().numpy()
    sc = scale.view(2, B, NH, maxT)
    codes = np.stack([kv[0, b, h, :T].cpu().numpy(), kv[1, b, h, :T].cpu().numpy()]).reshape(-1)
    scales = np.stack([sc[0, b, h, :T].cpu().numpy(), sc[1, b, h, :T].cpu().numpy()]).reshape(-1)
    fmt = oracle.W8_INT8 if dtype == "int8" else oracle.W8_FP8_E4M3
    deq = oracle.dequant_w8(codes, scales.astype(np.float32), 1, 1, HS, T, fmt).reshape(2, T, HS)
    return deq[0], deq[1]


@pytest.mark.parametrize("dtype,B,NH,maxT,T,expect", CASES,
                         ids=[f"{c[0]}-B{c[1]}-NH{c[2]}-maxT{c[3]}-T{c[4]}-{c[5][0]}" for c in CASES])
def test_auto_plan_branches(dev, dtype, B, NH, maxT, T, expect):
    import torch
    kvattn = _kv()
    plan = kvattn.plan(B, NH, HS, maxT, kv_dtype=dtype, len_hint=T - 1)
    assert (kvattn.STRATEGY_NAMES[plan[0]], plan[1], plan[2]) == expect, plan
    print(f"{dtype} B={B} NH={NH} maxT={maxT} T={T} plan {expect}", flush=True)
    qkv, cache, scale = _inputs(torch, dev, dtype, B, NH, maxT, seed=B * 1000 + maxT + T)
    cur = torch.tensor([T - 1], dtype=torch.int32, device=dev)
    act = torch.float32 if dtype == "f32" else torch.bfloat16
    outs = {}
    for name, strategy, S in (("auto", "auto", 0), ("reference partition", "lastblock", 8)):
        ws = kvattn.Workspace(B, NH, maxT, S)
        out = torch.full((B * NH * HS,), float("nan"), dtype=act, device=dev)
        kvattn.decode(out, qkv, cache, B, NH, HS, maxT, kv_dtype=dtype, kv_scale=scale, cur_len=cur,
                      len_hint=T - 1, S=S, strategy=strategy, **ws.kwargs())
        torch.cuda.synchronize()
        st = ws.status()
        assert st == 0, f"{name}: {st} designated merges timed out"
        outs[name] = out.float().view(B, NH, HS)
    got = outs["auto"]
    assert bool(torch.isfinite(got).all()), "non-finite output"
    # sampled (b,h) against the oracle
    q = qkv.float().view(B, 3, NH, HS)
    rng = np.random.RandomState(B + NH + T)
    picks = {(int(b), int(h)) for b, h in zip(rng.randint(0, B, 16), rng.randint(0, NH, 16))}
    picks |= {(0, 0), (B - 1, NH - 1)}
    for b, h in sorted(picks):
        k, v = _rows_f32(cache, scale, dtype, B, NH, maxT, b, h, T)
        q1 = np.zeros((1, 3, 1, HS), np.float32)
        q1[0, 0, 0] = q[b, 0, h].cpu().numpy()
        ref = oracle.attention_f32(q1.reshape(-1), np.stack([k, v]).reshape(-1), T, 1, 1, HS, T)
        assert_close(got[b, h].cpu().numpy(), ref, dtype, f"{dtype} b={b} h={h}")
    # every (b,h): inside the hull of its V rows, and close to the reference partition's result
    if dtype in ("f32", "bf16"):
        vv = cache.view(2, B, NH, maxT, HS)[1, :, :, :T].float()
    else:
        sc = scale.view(2, B, NH, maxT)[1, :, :, :T].unsqueeze(-1)
        raw = cache.view(2, B, NH, maxT, HS)[1, :, :, :T]
        if dtype == "int8":
            vals = raw.view(torch.int8).float()
        else:
            vals = raw.view(torch.float8_e4m3fn).float()
        vv = vals * sc
    vmin, vmax = vv.amin(dim=2), vv.amax(dim=2)
    slack = TOL[dtype] * (vmax - vmin).abs() + 1e-3
    assert bool(((got >= vmin - slack) & (got <= vmax + slack)).all()), "output outside the V hull"
    ref2 = outs["reference partition"]
    d = (got - ref2).norm(dim=2) / ref2.norm(dim=2).clamp_min(1e-30)
    assert float(d.max()) <= TOL[dtype], f"AUTO and the reference partition differ ({float(d.max()):.3e})"


# Without a length hint (a graph captured once and replayed at every length): beyond the
# device-planned grid of a few heads, AUTO takes the hinted plan's designated window (or one
# segment per head) at maxT with fixed rows, and the same launch serves every length.
# dtype, B, NH, maxT, attended lengths (one per call; per sequence when ragged), plan, ragged
NO_HINT = [
    ("int8", 2, 12, 1024, [300, 1024], ("designated", 8, 128), False),
    ("bf16", 1, 12, 4096, [1000, 4096], ("designated", 16, 256), False),
    ("fp8", 32, 12, 1024, [300, 1024], ("designated", 2, 512), False),
    ("bf16", 16, 12, 512, [300, 512], ("lastblock", 1, 512), False),
    ("int8", 5, 12, 8192, [700, 8192], ("designated", 16, 512), False),
    ("int8", 8, 12, 1024, [1024, 77, 512, 1000, 129, 300, 1024, 1], ("designated", 8, 128), True),
]


@pytest.mark.parametrize("dtype,B,NH,maxT,Ts,expect,ragged", NO_HINT,
                         ids=[f"{c[0]}-B{c[1]}-maxT{c[3]}-{c[5][0]}{'-ragged' if c[6] else ''}" for c in NO_HINT])
def test_auto_without_hint_plan_branches(dev, dtype, B, NH, maxT, Ts, expect, ragged):
    import torch
    kvattn = _kv()
    plan = kvattn.plan(B, NH, HS, maxT, kv_dtype=dtype)
    assert (kvattn.STRATEGY_NAMES[plan[0]], plan[1], plan[2]) == expect, plan
    qkv, cache, scale = _inputs(torch, dev, dtype, B, NH, maxT, seed=B * 100 + maxT)
    act = torch.float32 if dtype == "f32" else torch.bfloat16
    ws = kvattn.Workspace(B, NH, maxT, 0)
    q = qkv.float().view(B, 3, NH, HS)
    calls = [Ts] if ragged else [[T] * B for T in Ts]
    for lens in calls:
        print(f"{dtype} B={B} maxT={maxT} lengths {lens} plan {expect}", flush=True)
        cur = torch.tensor([t - 1 for t in lens], dtype=torch.int32, device=dev)
        if not ragged:
            cur = cur[:1].contiguous()
        out = torch.full((B * NH * HS,), float("nan"), dtype=act, device=dev)
        kvattn.decode(out, qkv, cache, B, NH, HS, maxT, kv_dtype=dtype, kv_scale=scale, cur_len=cur,
                      lens_per_seq=ragged, **ws.kwargs())
        torch.cuda.synchronize()
        assert ws.status() == 0
        got = out.float().view(B, NH, HS)
        rng = np.random.RandomState(sum(lens))
        picks = {(int(b), int(h)) for b, h in zip(rng.randint(0, B, 12), rng.randint(0, NH, 12))}
        picks |= {(0, 0), (B - 1, NH - 1)}
        for b, h in sorted(picks):
            T = lens[b]
            k, v = _rows_f32(cache, scale, dtype, B, NH, maxT, b, h, T)
            q1 = np.zeros((1, 3, 1, HS), np.float32)
            q1[0, 0, 0] = q[b, 0, h].cpu().numpy()
            ref = oracle.attention_f32(q1.reshape(-1), np.stack([k, v]).reshape(-1), T, 1, 1, HS, T)
            assert_close(got[b, h].cpu().numpy(), ref, dtype, f"{dtype} lengths {lens} b={b} h={h}")


# A paged cache (page pool [num_pages][2][NH][P][hs], shuffled block table) takes the same
# designated window and one-segment plan, with and without a hint; its split + merge plans
# stay planned on the device.  dtype, B, NH, P, maxT, lengths per sequence
PAGED = [
    ("bf16", 16, 12, 256, 512, [512] * 16),                 # 192 heads of 512 rows: one segment per head
    ("int8", 1, 12, 256, 4096, [4096]),                     # designated 16 x 256, 8-bit streaming tiles
    ("fp8", 8, 12, 64, 1024, [1024, 1, 300, 64, 65, 1000, 777, 129]),   # designated 8 x 128, ragged
]


@pytest.mark.parametrize("dtype,B,NH,P,maxT,lens", PAGED,
                         ids=[f"{c[0]}-B{c[1]}-P{c[3]}-maxT{c[4]}" for c in PAGED])
def test_auto_paged_plan_branches(dev, dtype, B, NH, P, maxT, lens):
    import torch
    kvattn = _kv()
    rs = np.random.RandomState(B * 7 + maxT)
    need = [(t + P - 1) // P for t in lens]
    npg = sum(need) + 2
    perm = rs.permutation(npg)
    table = np.full((B, maxT // P), -1, np.int32)
    k = 0
    for b in range(B):
        table[b, :need[b]] = perm[k:k + need[b]]
        k += need[b]
    qkv, pool, scale = _inputs(torch, dev, dtype, npg, NH, P, seed=B + maxT + P)   # [npg][2][NH][P][hs]
    qkv = qkv[: B * 3 * NH * HS].contiguous()    # npg >= B, so the generated q/k/v cover B sequences
    d_table = torch.from_numpy(table).to(dev)
    cache = kvattn.PagedCache(pool, d_table, maxT // P, P, npg, page_scales=scale)
    ragged = len(set(lens)) > 1
    cur = torch.tensor([t - 1 for t in lens], dtype=torch.int32, device=dev)
    if not ragged:
        cur = cur[:1].contiguous()
    act = torch.float32 if dtype == "f32" else torch.bfloat16
    q = qkv.float().view(B, 3, NH, HS)
    pool5 = pool.view(npg, 2, NH, P, HS)
    sc4 = scale.view(npg, 2, NH, P) if scale is not None else None
    for hint in (max(lens) - 1, -1):
        print(f"paged {dtype} B={B} P={P} maxT={maxT} hint={hint}", flush=True)
        ws = kvattn.Workspace(B, NH, maxT, 0)
        out = torch.full((B * NH * HS,), float("nan"), dtype=act, device=dev)
        kvattn.paged_decode(out, qkv, cache, B, NH, HS, kv_dtype=dtype, cur_len=cur, lens_per_seq=ragged,
                            len_hint=hint, **ws.kwargs())
        torch.cuda.synchronize()
        assert ws.status() == 0
        got = out.float().view(B, NH, HS)
        rng = np.random.RandomState(hint + 5)
        picks = {(int(b), int(h)) for b, h in zip(rng.randint(0, B, 10), rng.randint(0, NH, 10))}
        picks |= {(0, 0), (B - 1, NH - 1)}
        for b, h in sorted(picks):
            T = lens[b]
            pages = [int(table[b, i]) for i in range((T + P - 1) // P)]
            if dtype in ("f32", "bf16"):
                k_rows = torch.cat([pool5[p, 0, h] for p in pages])[:T].float().cpu().numpy()
                v_rows = torch.cat([pool5[p, 1, h] for p in pages])[:T].float().cpu().numpy()
            else:
                codes = np.stack([torch.cat([pool5[p, kv, h] for p in pages])[:T].cpu().numpy() for kv in (0, 1)])
                scs = np.stack([torch.cat([sc4[p, kv, h] for p in pages])[:T].cpu().numpy() for kv in (0, 1)])
                fmt = oracle.W8_INT8 if dtype == "int8" else oracle.W8_FP8_E4M3
                deq = oracle.dequant_w8(codes.reshape(-1), scs.reshape(-1).astype(np.float32), 1, 1, HS, T,
                                        fmt).reshape(2, T, HS)
                k_rows, v_rows = deq[0], deq[1]
            q1 = np.zeros((1, 3, 1, HS), np.float32)
            q1[0, 0, 0] = q[b, 0, h].cpu().numpy()
            ref = oracle.attention_f32(q1.reshape(-1), np.stack([k_rows, v_rows]).reshape(-1), T, 1, 1, HS, T)
            assert_close(got[b, h].cpu().numpy(), ref, dtype, f"paged {dtype} hint={hint} b={b} h={h} T={T}")


def test_auto_paged_long_max_context_keeps_segments_a_wave_walks(dev):
    """A paged cache of maxT = 2^20 positions over 2 heads: the hinted rule would plan
    16,384-row segments, longer than a paged wave walks (it follows at most 64 tiles, one page
    id per lane), so AUTO keeps the general plan.  20,000 attended positions, both heads
    against the oracle, with and without the hint."""
    import torch
    kvattn = _kv()
    B, NH, P, maxT, T = 1, 2, 256, 1 << 20, 20000
    need = (T + P - 1) // P
    npg = need + 3
    rs = np.random.RandomState(11)
    table = np.full((B, maxT // P), -1, np.int32)
    table[0, :need] = rs.permutation(npg)[:need]
    g = torch.Generator(device=dev)
    g.manual_seed(12)
    pool = torch.randn(npg * 2 * NH * P * HS, generator=g, device=dev).to(torch.bfloat16)
    qkv = torch.randn(B * 3 * NH * HS, generator=g, device=dev).to(torch.bfloat16)
    cache = kvattn.PagedCache(pool, torch.from_numpy(table).to(dev), maxT // P, P, npg)
    cur = torch.tensor([T - 1], dtype=torch.int32, device=dev)
    pool5 = pool.view(npg, 2, NH, P, HS)
    q = qkv.float().view(B, 3, NH, HS)
    for hint in (T - 1, -1):
        ws = kvattn.Workspace(B, NH, maxT, 0)
        out = torch.full((B * NH * HS,), float("nan"), dtype=torch.bfloat16, device=dev)
        kvattn.paged_decode(out, qkv, cache, B, NH, HS, kv_dtype="bf16", cur_len=cur, len_hint=hint, **ws.kwargs())
        torch.cuda.synchronize()
        got = out.float().view(B, NH, HS)
        for h in range(NH):
            pages = [int(table[0, i]) for i in range(need)]
            k_rows = torch.cat([pool5[p, 0, h] for p in pages])[:T].float().cpu().numpy()
            v_rows = torch.cat([pool5[p, 1, h] for p in pages])[:T].float().cpu().numpy()
            q1 = np.zeros((1, 3, 1, HS), np.float32)
            q1[0, 0, 0] = q[0, 0, h].cpu().numpy()
            ref = oracle.attention_f32(q1.reshape(-1), np.stack([k_rows, v_rows]).reshape(-1), T, 1, 1, HS, T)
            assert_close(got[0, h].cpu().numpy(), ref, "bf16", f"paged maxT=2^20 hint={hint} h={h}")
