"""Paged KV cache on the GPU: the append and the attention through a block table, against the
oracle on the same values laid out contiguously.

A case's contiguous cache [2][B][NH][maxT][hs] is scattered into a page pool
[num_pages][2][NH][page_rows][hs] through a shuffled block table; spare pages are filled
with NaN (bf16 / f32) or NaN codes and scales (8-bit), so a read from a wrong page shows up
as a non-finite output.  Bars as for the contiguous cache (kvcases.TOL); appended bytes bit
for bit; append + attention in one launch bit-identical to the two calls.
"""
import numpy as np
import pytest

from kvcases import HS, assert_close, make_case, out_tensor
from oracle import oracle

pytestmark = pytest.mark.gpu


def _kv():
    from cuda_gpt2_inference_amd import kvattn
    return kvattn


def _scatter(arr, B, NH, maxT, P, table, num_pages, row_elems, fill):
    """[2][B][NH][maxT][row_elems] -> [num_pages][2][NH][P][row_elems] through table."""
    mp = maxT // P
    src = arr.reshape(2, B, NH, mp, P, row_elems).transpose(1, 3, 0, 2, 4, 5)   # b, page idx, kv, h, P, e
    pool = np.full((num_pages, 2, NH, P, row_elems), fill, dtype=arr.dtype)
    for b in range(B):
        for i in range(mp):
            if 0 <= table[b, i] < num_pages:
                pool[table[b, i]] = src[b, i]
    return pool


class Paged:
    """Host case + device paged cache built from it."""

    def __init__(self, case, P, dev, seed=0, spare=3):
        import torch
        self.case, self.P = case, P
        B, NH, maxT = case.B, case.NH, case.maxT
        assert maxT % P == 0
        self.max_pages = maxT // P
        self.num_pages = B * self.max_pages + spare
        r = np.random.RandomState(seed)
        self.table = r.permutation(self.num_pages)[:B * self.max_pages].reshape(B, self.max_pages).astype(np.int32)
        if case.dtype == "f32":
            raw = case.cache_raw.view(np.uint32)
            fill = np.uint32(0x7FC00000)
        elif case.dtype == "bf16":
            raw = case.cache_raw
            fill = np.uint16(0x7FC0)
        else:
            raw = case.cache_raw
            fill = np.uint8(0x7F)                     # INT8 127 / FP8 NaN, with NaN scales below
        pool = _scatter(raw.reshape(-1), B, NH, maxT, P, self.table, self.num_pages, HS, fill)
        self.pool_raw = pool
        if case.dtype == "f32":
            self.pages = torch.from_numpy(pool.reshape(-1).view(np.float32).copy()).to(dev)
        elif case.dtype == "bf16":
            self.pages = torch.from_numpy(pool.reshape(-1).view(np.int16).copy()).to(dev).view(torch.bfloat16)
        else:
            self.pages = torch.from_numpy(pool.reshape(-1).copy()).to(dev)
        self.scales = None
        if case.scale_raw is not None:
            sp = _scatter(case.scale_raw.reshape(-1, 1), B, NH, maxT, P, self.table, self.num_pages, 1,
                          np.float32(np.nan))
            self.scales = torch.from_numpy(sp.reshape(-1).copy()).to(dev)
        self.d_table = torch.from_numpy(self.table.copy()).to(dev)
        kvattn = _kv()
        self.cache = kvattn.PagedCache(self.pages, self.d_table, self.max_pages, P, self.num_pages,
                                       page_scales=self.scales)

    def host_pool(self, raw_cache, raw_scale=None):
        """Expected pool bytes for a contiguous cache image (spare pages untouched)."""
        c = self.case
        pool = _scatter(raw_cache.reshape(-1), c.B, c.NH, c.maxT, self.P, self.table, self.num_pages, HS,
                        self.pool_raw.reshape(-1)[0] * 0)
        keep = np.ones(self.num_pages, bool)
        keep[self.table.reshape(-1)] = False
        pool[keep] = self.pool_raw[keep]
        return pool


def _dev_bytes(t):
    import torch
    return t.view(torch.uint8).cpu().numpy()


@pytest.mark.parametrize("dtype", ["f32", "bf16", "int8", "fp8"])
@pytest.mark.parametrize("P", [64, 256])
def test_paged_decode_matches_oracle(dev, dtype, P):
    """Every paged strategy and partition, uniform and ragged lengths, with and without a
    host hint, against the oracle on the contiguous values."""
    import torch
    kvattn = _kv()
    B, NH, maxT = 3, 4, 1024
    lens_sets = {"ragged": [1024, 300, 64], "ragged2": [1, 256, 257], "uniform": [777] * 3}
    for name, lens in lens_sets.items():
        case = make_case(dtype, B, NH, maxT, np.array(lens, np.int32) - 1, seed=60 + P)
        pg = Paged(case, P, dev, seed=P)
        ref = case.reference()
        cur = torch.from_numpy(case.cur_lens.copy()).to(dev)
        qkv = torch.from_numpy(case.qkv_raw.view(np.int16 if dtype != "f32" else np.float32)).to(dev)
        if dtype != "f32":
            qkv = qkv.view(torch.bfloat16)
        for strategy in ("auto", "lastblock", "designated", "split_merge", "graph"):
            for S in (0, -64, -128 if P == 64 else -256):
                for hint in (-1, max(lens) - 1):
                    ws = kvattn.Workspace(B, NH, maxT, S)
                    out = out_tensor(case, dev)
                    kvattn.paged_decode(out, qkv, pg.cache, B, NH, HS, kv_dtype=dtype, cur_len=cur,
                                        lens_per_seq=True, len_hint=hint, S=S, strategy=strategy, **ws.kwargs())
                    torch.cuda.synchronize()
                    assert_close(out.float().cpu().numpy(), ref, dtype,
                                 f"paged P={P} {name} {strategy} S={S} hint={hint}")


@pytest.mark.parametrize("dtype", ["f32", "bf16", "int8", "fp8"])
def test_paged_append_and_fused(dev, dtype):
    """paged_cache_write writes exactly the oracle's append through the table;
    append_decode on the pool equals paged_cache_write + paged_decode bit for bit."""
    import torch
    kvattn = _kv()
    B, NH, maxT, P = 3, 2, 512, 64
    lens = [512, 65, 200]
    case = make_case(dtype, B, NH, maxT, np.array(lens, np.int32) - 1, seed=71)
    qkv = torch.from_numpy(case.qkv_raw.view(np.int16 if dtype != "f32" else np.float32)).to(dev)
    if dtype != "f32":
        qkv = qkv.view(torch.bfloat16)
    cur = torch.from_numpy(case.cur_lens.copy()).to(dev)
    # Expected cache after the append, contiguous, from the oracle.
    exp_cache = case.cache_raw.copy()
    exp_scale = None if case.scale_raw is None else case.scale_raw.copy()
    if dtype in ("int8", "fp8"):
        fmt = oracle.W8_INT8 if dtype == "int8" else oracle.W8_FP8_E4M3
        oracle.cache_write_w8(exp_cache, exp_scale, case.qkv_host, case.cur_lens, B, NH, HS, maxT, fmt)
    else:
        oracle.cache_write(exp_cache, case.qkv_raw, case.cur_lens, B, NH, HS, maxT)

    pg_a = Paged(case, P, dev, seed=5)
    kvattn.paged_cache_write(pg_a.cache, qkv, B, NH, HS, kv_dtype=dtype, cur_len=cur, lens_per_seq=True)
    torch.cuda.synchronize()
    want = pg_a.host_pool(exp_cache.view(pg_a.pool_raw.dtype) if dtype == "f32" else exp_cache)
    assert np.array_equal(_dev_bytes(pg_a.pages), want.reshape(-1).view(np.uint8)), "paged append bytes"
    if exp_scale is not None:
        ws_pool = _scatter(exp_scale.reshape(-1, 1), B, NH, maxT, P, pg_a.table, pg_a.num_pages, 1,
                           np.float32(np.nan)).reshape(-1)
        got = pg_a.scales.cpu().numpy()
        used = ~np.isnan(ws_pool)
        assert np.array_equal(got[used].view(np.uint32), ws_pool[used].view(np.uint32)), "paged append scales"

    for strategy, S, hint in (("auto", 0, -1), ("lastblock", -64, max(lens) - 1), ("designated", -64, -1),
                              ("designated", 0, max(lens) - 1), ("split_merge", 0, -1), ("graph", -128, -1)):
        pa, pb = Paged(case, P, dev, seed=9), Paged(case, P, dev, seed=9)
        wsp = kvattn.Workspace(B, NH, maxT, S)
        oa, ob = out_tensor(case, dev), out_tensor(case, dev)
        kw = dict(kv_dtype=dtype, cur_len=cur, lens_per_seq=True, len_hint=hint, S=S, strategy=strategy,
                  **wsp.kwargs())
        kvattn.paged_cache_write(pa.cache, qkv, B, NH, HS, kv_dtype=dtype, cur_len=cur, lens_per_seq=True)
        kvattn.paged_decode(oa, qkv, pa.cache, B, NH, HS, **kw)
        kvattn.paged_decode(ob, qkv, pb.cache, B, NH, HS, append=True, **kw)
        torch.cuda.synchronize()
        what = f"{dtype} {strategy} S={S}"
        assert np.array_equal(_dev_bytes(pa.pages), _dev_bytes(pb.pages)), what + ": pool"
        if pa.scales is not None:
            assert np.array_equal(_dev_bytes(pa.scales), _dev_bytes(pb.scales)), what + ": scales"
        ga, gb = oa.float().cpu().numpy(), ob.float().cpu().numpy()
        assert np.array_equal(ga, gb), what + ": outputs"
        # ... and both against the oracle on the appended values.
        if dtype in ("int8", "fp8"):
            vals = oracle.dequant_w8(exp_cache, exp_scale, B, NH, HS, maxT,
                                     oracle.W8_INT8 if dtype == "int8" else oracle.W8_FP8_E4M3)
        else:
            vals = case.cache_host.copy()
            oracle.cache_write(vals, case.qkv_host, case.cur_lens, B, NH, HS, maxT)
        ref = oracle.attention_f32(case.qkv_host, vals, case.totals, B, NH, HS, maxT)
        assert_close(gb, ref, dtype, what)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "int8", "fp8"])
def test_paged_designated_fallback_matches_oracle(dev, dtype):
    """The designated merger's fallback on a paged cache (poll bound 0: every merger of a
    multi-segment head computes its producers' segments itself, walking the block table):
    the output matches the oracle, and with the append fused the pool bytes and the output
    equal those of the normal path."""
    import torch
    kvattn = _kv()
    B, NH, maxT, P = 3, 4, 1024, 64
    lens = [1024, 300, 64]
    case = make_case(dtype, B, NH, maxT, np.array(lens, np.int32) - 1, seed=81)
    ref = case.reference()
    cur = torch.from_numpy(case.cur_lens.copy()).to(dev)
    qkv = torch.from_numpy(case.qkv_raw.view(np.int16 if dtype != "f32" else np.float32)).to(dev)
    if dtype != "f32":
        qkv = qkv.view(torch.bfloat16)
    for S, hint in ((-64, -1), (0, max(lens) - 1)):
        runs = {}
        for bound in (None, 0):
            for append in (False, True):
                pg = Paged(case, P, dev, seed=3)
                ws = kvattn.Workspace(B, NH, maxT, S)
                out = out_tensor(case, dev)
                prev = kvattn.set_merge_poll_limit(0) if bound == 0 else None
                try:
                    kvattn.paged_decode(out, qkv, pg.cache, B, NH, HS, kv_dtype=dtype, cur_len=cur,
                                        lens_per_seq=True, len_hint=hint, S=S, strategy="designated",
                                        append=append, **ws.kwargs())
                    torch.cuda.synchronize()
                finally:
                    if prev is not None:
                        kvattn.set_merge_poll_limit(prev)
                what = f"paged designated S={S} hint={hint} bound={bound} append={append}"
                assert (ws.status() > 0) == (bound == 0), what + ": status count"
                runs[(bound, append)] = (out.float().cpu().numpy(), _dev_bytes(pg.pages).copy())
                if not append:
                    assert_close(runs[(bound, append)][0], ref, dtype, what)
        assert np.array_equal(runs[(0, True)][1], runs[(None, True)][1]), f"S={S}: pool bytes of the fallback"
        assert_close(runs[(0, True)][0], runs[(None, True)][0], dtype, f"S={S}: fused append, fallback")


def test_paged_invalid_table_entries_are_skipped(dev):
    """A table entry outside [0, num_pages) inside a sequence's length: those positions are
    skipped, never read (the result equals attention over the remaining positions)."""
    import torch
    kvattn = _kv()
    B, NH, maxT, P = 2, 3, 512, 64
    case = make_case("bf16", B, NH, maxT, [511, 300], seed=81)
    pg = Paged(case, P, dev, seed=2)
    table = pg.table.copy()
    table[0, 2] = -1                 # positions 128..191 of sequence 0
    table[1, 4] = pg.num_pages + 7   # positions 256..299 of sequence 1
    pg.d_table.copy_(torch.from_numpy(table))
    qkv = torch.from_numpy(case.qkv_raw.view(np.int16)).to(dev).view(torch.bfloat16)
    cur = torch.from_numpy(case.cur_lens.copy()).to(dev)
    ws = kvattn.Workspace(B, NH, maxT, 0)
    out = out_tensor(case, dev)
    kvattn.paged_decode(out, qkv, pg.cache, B, NH, HS, kv_dtype="bf16", cur_len=cur, lens_per_seq=True,
                        **ws.kwargs())
    torch.cuda.synchronize()
    got = out.float().cpu().numpy().reshape(B, NH, HS)
    c = case.cache_host.reshape(2, B, NH, maxT, HS)
    q = case.qkv_host.reshape(B, 3, NH, HS)
    for b, (lo, hi) in ((0, (128, 192)), (1, (256, 320))):
        total = int(case.totals[b])
        keep = [j for j in range(total) if not lo <= j < hi]
        for h in range(NH):
            k = c[0, b, h, keep].astype(np.float64)
            v = c[1, b, h, keep].astype(np.float64)
            s = k @ q[b, 0, h].astype(np.float64) / 8.0
            p = np.exp(s - s.max())
            ref = (p @ v) / p.sum()
            assert np.linalg.norm(got[b, h] - ref) / np.linalg.norm(ref) <= 1e-2, (b, h)


@pytest.mark.parametrize("dtype", ["bf16", "int8", "fp8"])
@pytest.mark.parametrize("hint", [-1, 249])
def test_paged_invalid_entries_in_either_tile(dev, dtype, hint):
    """One segment per (b,h) of up to 256 positions in 64-row pages: each wave walks two
    32-row tiles, rows [32w, 32w + 32) and [32w + 128, 32w + 160) (the 8-bit caches request
    the second with the first).  Page 0 of sequence 0 is invalid (the first tile of waves 0
    and 1), page 3 of sequence 1 too (the second tile of waves 2 and 3, at the sequence's
    end): those positions are skipped, never read, and the rest attended as usual."""
    import torch
    kvattn = _kv()
    B, NH, maxT, P = 2, 3, 256, 64
    case = make_case(dtype, B, NH, maxT, [249, 199], seed=83)
    pg = Paged(case, P, dev, seed=4)
    table = pg.table.copy()
    table[0, 0] = -1                  # positions 0..63 of sequence 0
    table[1, 3] = pg.num_pages + 7    # positions 192..199 of sequence 1
    pg.d_table.copy_(torch.from_numpy(table))
    qkv = torch.from_numpy(case.qkv_raw.view(np.int16)).to(dev).view(torch.bfloat16)
    cur = torch.from_numpy(case.cur_lens.copy()).to(dev)
    ws = kvattn.Workspace(B, NH, maxT, 0)
    out = out_tensor(case, dev)
    kvattn.paged_decode(out, qkv, pg.cache, B, NH, HS, kv_dtype=dtype, cur_len=cur, lens_per_seq=True,
                        len_hint=hint, **ws.kwargs())
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    c = case.cache_host.reshape(2, B, NH, maxT, HS)
    q = case.qkv_host.reshape(B, 3, NH, HS)
    ref = np.zeros((B, NH, HS), np.float64)
    for b, (lo, hi) in ((0, (0, 64)), (1, (192, 256))):
        keep = [j for j in range(int(case.totals[b])) if not lo <= j < hi]
        for h in range(NH):
            k = c[0, b, h, keep].astype(np.float64)
            v = c[1, b, h, keep].astype(np.float64)
            sc = k @ q[b, 0, h].astype(np.float64) / 8.0
            p_ = np.exp(sc - sc.max())
            ref[b, h] = (p_ @ v) / p_.sum()
    assert_close(got, ref.reshape(-1).astype(np.float32), dtype, f"{dtype} hint={hint}")


def test_paged_c5_shape_matches_contiguous(dev):
    """64 sequences x NH=12, lengths U[1, 8192], 256-row pages shuffled in a pool holding
    only the pages in use (~0.82 GB instead of 1.6 GB): every (b,h) agrees with the
    contiguous cache's result to the BF16 bar, and 16 slots agree with the oracle."""
    import torch
    kvattn = _kv()
    B, NH, maxT, P = 64, 12, 8192, 256
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    lens = torch.randint(1, maxT + 1, (B,), generator=g, device=dev, dtype=torch.int32)
    cur = (lens - 1).contiguous()
    qkv = torch.randn(B * 3 * NH * HS, generator=g, device=dev).to(torch.bfloat16)
    lens_h = lens.cpu().numpy()
    need = [(int(L) + P - 1) // P for L in lens_h]
    num_pages = sum(need)
    perm = np.random.RandomState(3).permutation(num_pages)
    table = np.full((B, maxT // P), -1, np.int32)
    k = 0
    for b in range(B):
        table[b, :need[b]] = perm[k:k + need[b]]
        k += need[b]
    pages = torch.empty(num_pages * 2 * NH * P * HS, device=dev, dtype=torch.bfloat16)
    chunk = 1 << 26
    for i in range(0, pages.numel(), chunk):
        n = min(chunk, pages.numel() - i)
        pages[i:i + n] = torch.randn(n, generator=g, device=dev).to(torch.bfloat16)
    d_table = torch.from_numpy(table).to(dev)
    cache = kvattn.PagedCache(pages, d_table, maxT // P, P, num_pages)
    ws = kvattn.Workspace(B, NH, maxT, 0)
    out_p = torch.empty(B * NH * HS, device=dev, dtype=torch.bfloat16)
    kvattn.paged_decode(out_p, qkv, cache, B, NH, HS, kv_dtype="bf16", cur_len=cur, lens_per_seq=True,
                        **ws.kwargs())
    # The same values gathered into a contiguous cache, decoded by the contiguous kernels.
    pv = pages.view(num_pages, 2, NH, P, HS)
    contig = torch.zeros(2, B, NH, maxT, HS, device=dev, dtype=torch.bfloat16)
    for b in range(B):
        for i in range(need[b]):
            contig[:, b, :, i * P:(i + 1) * P] = pv[int(table[b, i])]
    out_c = torch.empty_like(out_p)
    kvattn.decode(out_c, qkv, contig.view(-1), B, NH, HS, maxT, kv_dtype="bf16", cur_len=cur, lens_per_seq=True,
                  **ws.kwargs())
    torch.cuda.synchronize()
    a = out_p.float().view(B, NH, HS)
    c = out_c.float().view(B, NH, HS)
    assert bool(torch.isfinite(a).all())
    rel = ((a - c).norm(dim=2) / c.norm(dim=2)).max().item()
    assert rel <= 1e-2, rel
    q_h = qkv.float().cpu().numpy().reshape(B, 3, NH, HS)
    rng = np.random.RandomState(1)
    for b, h in zip(rng.randint(0, B, 16), rng.randint(0, NH, 16)):
        T = int(lens_h[b])
        kk = contig[0, b, h, :T].float().cpu().numpy()
        vv = contig[1, b, h, :T].float().cpu().numpy()
        q1 = np.zeros((1, 3, 1, HS), np.float32)
        q1[0, 0, 0] = q_h[b, 0, h]
        ref = oracle.attention_f32(q1.reshape(-1), np.stack([kk, vv]).reshape(-1), T, 1, 1, HS, T)
        assert_close(a[b, h].cpu().numpy(), ref, "bf16", f"paged C5 b={b} h={h} T={T}")


def test_paged_seeded_shape_sweep(dev):
    """24 paged calls drawn from a fixed seed, each against the oracle on the contiguous
    values: page rows 64 / 128 / 256 / 512, B 1..4, NH 1..12, up to 16 pages per sequence
    with ragged lengths, every cache type, AUTO and the explicit split strategies, device-
    planned or fixed rows per segment (multiples of 64), and an absent, exact or stale
    length hint.  An explicit designated plan the library refuses (a grid beyond residency,
    or segments longer than a wave walks) runs with the last-block merge instead."""
    import torch
    kvattn = _kv()
    rng = np.random.RandomState(777)
    strategies = ("auto", "lastblock", "designated", "split_merge", "graph")
    for i in range(24):
        dtype = ["f32", "bf16", "int8", "fp8"][rng.randint(4)]
        P = int(rng.choice([64, 128, 256, 512]))
        B, NH = int(rng.randint(1, 5)), int(rng.randint(1, 13))
        maxT = P * int(rng.randint(1, 17))
        lens = rng.randint(1, maxT + 1, B).astype(np.int32)
        strategy = strategies[rng.randint(len(strategies))]
        S = 0 if strategy == "auto" or rng.randint(2) == 0 else -64 * int(rng.randint(1, 9))
        hint_kind = rng.randint(3)
        hint = -1 if hint_kind == 0 else (int(lens.max()) - 1 if hint_kind == 1 else int(rng.randint(0, maxT)))
        name = (f"case {i}: {dtype} P={P} B={B} NH={NH} maxT={maxT} {strategy} S={S} hint={hint} "
                f"lens={lens.tolist()}")
        print(name, flush=True)
        case = make_case(dtype, B, NH, maxT, lens - 1, seed=8000 + i)
        pg = Paged(case, P, dev, seed=i)
        cur = torch.from_numpy(case.cur_lens.copy()).to(dev)
        qkv = torch.from_numpy(case.qkv_raw.view(np.int16 if dtype != "f32" else np.float32)).to(dev)
        if dtype != "f32":
            qkv = qkv.view(torch.bfloat16)
        ws = kvattn.Workspace(B, NH, maxT, S)
        out = out_tensor(case, dev)
        kw = dict(kv_dtype=dtype, cur_len=cur, lens_per_seq=True, len_hint=hint, S=S, **ws.kwargs())
        try:
            kvattn.paged_decode(out, qkv, pg.cache, B, NH, HS, strategy=strategy, **kw)
        except kvattn.KvAttnError as e:
            assert strategy == "designated" and e.status in (kvattn.ERR_GRID_TOO_LARGE, kvattn.ERR_SPLIT), \
                f"{name}: {e}"
            print(f"  refused ({e}); last-block instead", flush=True)
            kvattn.paged_decode(out, qkv, pg.cache, B, NH, HS, strategy="lastblock", **kw)
        torch.cuda.synchronize()
        assert_close(out.float().cpu().numpy(), case.reference(), dtype, name)


@pytest.mark.parametrize("rot", [0, 2])
@pytest.mark.parametrize("dtype", ["bf16", "int8"])
def test_paged_designated_producers_on_other_xcds(dev, dtype, rot):
    """The run-time XCD check on a paged cache: 12 (b,h) rows (an XCD-local designated grid),
    64-row segments, producers rotated `rot` XCDs away from their merger
    (kvattn_set_xcd_layout_offset).  Outputs against the oracle, no merge timeout; at rot 0 no
    producer finds its merger elsewhere, otherwise every producer (76 here) publishes
    write-through, counted in status words 4 (merger elsewhere) and 5 (its word not there yet)."""
    import torch
    kvattn = _kv()
    B, NH, maxT, P = 3, 4, 1024, 64
    lens = [1024, 300, 64]
    case = make_case(dtype, B, NH, maxT, np.array(lens, np.int32) - 1, seed=83 + rot)
    cur = torch.from_numpy(case.cur_lens.copy()).to(dev)
    qkv = torch.from_numpy(case.qkv_raw.view(np.int16)).to(dev).view(torch.bfloat16)
    producers = NH * sum(-(-L // 64) - 1 for L in lens)
    prev = kvattn.set_xcd_layout_offset(rot)
    try:
        pg = Paged(case, P, dev, seed=5)
        ws = kvattn.Workspace(B, NH, maxT, -64)
        out = out_tensor(case, dev)
        kvattn.paged_decode(out, qkv, pg.cache, B, NH, HS, kv_dtype=dtype, cur_len=cur, lens_per_seq=True,
                            len_hint=max(lens) - 1, S=-64, strategy="designated", **ws.kwargs())
        torch.cuda.synchronize()
    finally:
        kvattn.set_xcd_layout_offset(prev)
    what = f"paged designated {dtype} rot {rot}"
    assert_close(out.float().cpu().numpy(), case.reference(), dtype, what)
    assert ws.status() == 0, f"{what}: a merger stopped waiting"
    words = ws.buf[:256].cpu().numpy().view(np.uint32)
    remote, unseen = int(words[4]), int(words[5])
    if rot:
        assert remote + unseen == producers and remote > 0, f"{what}: remote {remote} unseen {unseen} of {producers}"
    else:
        assert remote == 0, f"{what}: {remote} producers found their merger on another XCD"


def test_paged_auto_ragged_between_the_stream_bounds(dev):
    """The same band in a paged cache (64 sequences x 12 heads x up to 1024 positions, 256-row
    pages, INT8): AUTO's last-block merge on the latency shape through the table, against the
    oracle."""
    import torch
    kvattn = _kv()
    B, NH, maxT, P = 64, 12, 1024, 256
    rng = np.random.RandomState(517)
    lens = rng.randint(1, maxT + 1, B).astype(np.int32)
    lens[3] = maxT
    case = make_case("int8", B, NH, maxT, lens - 1, seed=518)
    pg = Paged(case, P, dev, seed=6)
    qkv = torch.from_numpy(case.qkv_raw.view(np.int16)).to(dev).view(torch.bfloat16)
    cur = torch.from_numpy(case.cur_lens.copy()).to(dev)
    ws = kvattn.Workspace(B, NH, maxT, 0)
    out = out_tensor(case, dev)
    kvattn.paged_decode(out, qkv, pg.cache, B, NH, HS, kv_dtype="int8", cur_len=cur, lens_per_seq=True,
                        len_hint=maxT - 1, **ws.kwargs())
    torch.cuda.synchronize()
    assert ws.status() == 0
    assert_close(out.float().cpu().numpy(), case.reference(), "int8", "paged int8 ragged band")
