"""CPU checks of the host-side planning (AUTO strategy, segmentation, workspace sizing) and
of the Python binding's error mapping.  No GPU call is made: planning and argument
validation happen before any HIP call."""
import pytest

from cuda_gpt2_inference_amd import kvattn

ALIGNED = 1 << 20


def up(x):
    return (x + 255) // 256 * 256


def carve_bytes(B, NH, slots):
    return (up(B * NH * 4) + 2 * up(B * NH * slots * 4) + up(B * NH * slots * 64 * 4)
            + up(B * NH * slots * 2 * 8) + up(B * NH * slots * 64 * 8))


def test_auto_short_context_is_fused_single():
    for hint in (0, 1, 100, 255):
        assert kvattn.plan(1, 12, 64, 1024, kv_dtype="bf16", len_hint=hint) == (kvattn.FUSED_SINGLE, 1, 0)


def test_auto_gpt2_layer_is_single_launch_split():
    # T = 1024 at B=1, NH=12: 128-row segments (8 per head), merged in-kernel by segment 0
    # (the designated merger).
    assert kvattn.plan(1, 12, 64, 1024, kv_dtype="bf16", len_hint=1023) == (kvattn.SPLIT_DESIGNATED, 8, 128)
    # 257 positions: three 128-row segments used; the grid covers every length up to maxT.
    assert kvattn.plan(1, 12, 64, 1024, kv_dtype="int8", len_hint=256) == (kvattn.SPLIT_DESIGNATED, 8, 128)
    # More heads: 128-row segments while heads x segments stays within 768 workgroups, then
    # 256 rows.
    assert kvattn.plan(2, 12, 64, 1024, kv_dtype="bf16", len_hint=1023) == (kvattn.SPLIT_DESIGNATED, 8, 128)
    assert kvattn.plan(16, 12, 64, 1024, kv_dtype="bf16", len_hint=1023) == (kvattn.SPLIT_DESIGNATED, 4, 256)
    # The lastblock strategy keeps its own segmentation (about four segments).
    assert kvattn.plan(1, 12, 64, 1024, kv_dtype="bf16", len_hint=1023, strategy="lastblock") == \
        (kvattn.SPLIT_LASTBLOCK, 4, 256)


def test_designated_follows_at_most_64_segments():
    # Explicitly requested with more than 64 segments per (b,h): refused; AUTO falls back to
    # the last-block merge instead.
    with pytest.raises(kvattn.KvAttnError) as ei:
        kvattn.plan(1, 12, 64, 8192, kv_dtype="bf16", S=-64, strategy="designated")
    assert ei.value.status == kvattn.ERR_SPLIT
    assert kvattn.plan(1, 12, 64, 4096, kv_dtype="bf16", S=-64, strategy="designated") == \
        (kvattn.SPLIT_DESIGNATED, 64, 64)
    # Long contexts: longer segments keep the count at 64 or fewer.
    assert kvattn.plan(1, 1, 64, 40000, kv_dtype="bf16", len_hint=39999) == (kvattn.SPLIT_DESIGNATED, 40, 1024)
    assert kvattn.plan(1, 1, 64, 40000, kv_dtype="bf16") == (kvattn.SPLIT_DESIGNATED, 64, -1)


def test_auto_large_batch_streams_with_split_merge():
    st, slots, rows = kvattn.plan(64, 12, 64, 8192, kv_dtype="bf16", len_hint=8191)
    assert (st, slots, rows) == (kvattn.SPLIT_MERGE, 32, 256)
    # FP32 and FP8 keep the general streaming plan (512-row segments).
    assert kvattn.plan(64, 12, 64, 8192, kv_dtype="fp8", len_hint=8191) == (kvattn.SPLIT_MERGE, 16, 512)
    assert kvattn.plan(64, 12, 64, 8192, kv_dtype="int8", len_hint=8191) == (kvattn.SPLIT_MERGE, 16, 512)
    assert kvattn.plan(64, 12, 64, 4096, kv_dtype="int8", len_hint=4095) == (kvattn.SPLIT_MERGE, 16, 256)


# (B, NH, maxT, hint, dtype) -> AUTO's plan, one shape per branch of the tuned choice.
TUNED = [
    # one segment per head: >= 192 heads of at most 512 rows
    ((16, 12, 512, 511, "fp8"), (kvattn.SPLIT_LASTBLOCK, 1, 512)),
    ((64, 12, 512, 299, "f32"), (kvattn.SPLIT_LASTBLOCK, 1, 512)),
    ((15, 12, 512, 511, "bf16"), (kvattn.SPLIT_DESIGNATED, 4, 128)),     # 180 heads: designated
    ((64, 12, 512, 511, "int8"), (kvattn.SPLIT_LASTBLOCK, 1, 512)),
    # designated: rows max(128, maxT / 16) (a power of two), doubled while the grid exceeds 768
    ((8, 12, 1024, 1023, "bf16"), (kvattn.SPLIT_DESIGNATED, 8, 128)),    # 96 x 8 = 768
    ((1, 12, 4096, 4095, "int8"), (kvattn.SPLIT_DESIGNATED, 16, 256)),
    ((1, 12, 8192, 8191, "bf16"), (kvattn.SPLIT_DESIGNATED, 16, 512)),
    ((32, 12, 1024, 1023, "fp8"), (kvattn.SPLIT_DESIGNATED, 2, 512)),    # doubled twice, 53.6 MB
    ((8, 12, 2048, 2047, "int8"), (kvattn.SPLIT_DESIGNATED, 8, 256)),    # doubled, 8 segments, 26.8 MB
    ((1, 2, 8192, 8191, "bf16"), (kvattn.SPLIT_DESIGNATED, 64, 128)),    # 2 heads: up to 64 segments
    # up to 64 heads with long segments (256 rows, 512 for 8-bit): grids of up to 1024
    ((2, 25, 4096, 4095, "bf16"), (kvattn.SPLIT_DESIGNATED, 16, 256)),   # 50 x 16 = 800
    ((1, 64, 4096, 4095, "bf16"), (kvattn.SPLIT_DESIGNATED, 16, 256)),   # 64 x 16 = 1024, 64 MiB
    ((5, 12, 8192, 8191, "fp8"), (kvattn.SPLIT_DESIGNATED, 16, 512)),    # 60 x 16 = 960
    ((5, 12, 2048, 2047, "bf16"), (kvattn.SPLIT_DESIGNATED, 8, 256)),    # 128-row segments: 768 still
    ((5, 12, 4096, 4095, "int8"), (kvattn.SPLIT_DESIGNATED, 8, 512)),    # 8-bit 256-row segments: 768 still
    # not designated: doubled to 8 segments above 40 MB, or above 64 MB, or a grid beyond 768
    ((8, 12, 2048, 2047, "bf16"), (kvattn.SPLIT_MERGE, 8, 256)),
    ((8, 12, 4096, 4095, "fp8"), (kvattn.SPLIT_LASTBLOCK, 8, 512)),      # FP8: the general plan
    ((32, 12, 1024, 1023, "bf16"), (kvattn.SPLIT_MERGE, 4, 256)),
    ((16, 12, 1024, 1023, "f32"), (kvattn.SPLIT_LASTBLOCK, 4, 256)),
    ((2, 32, 8192, 8191, "int8"), (kvattn.SPLIT_MERGE, 16, 512)),
    # split + merge: at most 64 segments per head, longer rows past that
    ((2, 12, 16384, 16383, "bf16"), (kvattn.SPLIT_MERGE, 64, 256)),
    ((1, 12, 32768, 32767, "bf16"), (kvattn.SPLIT_MERGE, 64, 512)),
    ((1, 12, 65536, 65535, "int8"), (kvattn.SPLIT_MERGE, 64, 1024)),
    ((16, 12, 20000, 19999, "bf16"), (kvattn.SPLIT_MERGE, 40, 512)),
]


@pytest.mark.parametrize("args,plan", TUNED, ids=[f"B{a[0]}-NH{a[1]}-maxT{a[2]}-{a[4]}" for a, _ in TUNED])
def test_auto_with_hint_takes_the_measured_plan(args, plan):
    B, NH, maxT, hint, dt = args
    assert kvattn.plan(B, NH, 64, maxT, kv_dtype=dt, len_hint=hint) == plan


def test_auto_tuned_plans_stay_within_their_bounds():
    """Every hinted AUTO plan over a grid of shapes: a designated grid of at most 768
    workgroups (1024 for up to 64 heads with segments of 256 rows or more, 512 for 8-bit
    caches) and 64 segments per head, at most 16 once there are 12 or more heads; the
    one-segment plan only for 192+ heads of at most 512 rows; and the GPT-2 layer (B = 1,
    NH = 12, maxT = 1024) unchanged at every length past fused_single."""
    for dt in ("f32", "bf16", "int8", "fp8"):
        for B in (1, 2, 3, 5, 8, 16, 33, 64, 200):
            for NH in (1, 4, 12, 25):
                for maxT in (300, 512, 1000, 1024, 2048, 5000, 8192, 20000):
                    for hint in {maxT // 3, maxT - 1}:
                        st, slots, rows = kvattn.plan(B, NH, 64, maxT, kv_dtype=dt, len_hint=hint)
                        heads = B * NH
                        if st == kvattn.SPLIT_DESIGNATED:
                            wide = heads <= 64 and rows >= (512 if dt in ("int8", "fp8") else 256)
                            assert heads * slots <= (1024 if wide else 768) and slots <= 64, (dt, B, NH, maxT, hint)
                            if heads >= 12:
                                assert slots <= 16, (dt, B, NH, maxT, hint)
                        if st == kvattn.SPLIT_LASTBLOCK and slots == 1 and rows == 512:
                            assert heads >= 192 and maxT <= 512
                        if st != kvattn.FUSED_SINGLE:
                            assert slots * rows >= maxT
    for hint in range(256, 1024, 37):
        assert kvattn.plan(1, 12, 64, 1024, kv_dtype="bf16", len_hint=hint) == (kvattn.SPLIT_DESIGNATED, 8, 128)


def test_auto_without_hint_plans_on_the_device():
    # No length hint (a graph replayed at every length): the kernels pick the rows per
    # segment from the device length; the grid holds the most segments any length needs.
    assert kvattn.plan(1, 12, 64, 1024, kv_dtype="bf16") == (kvattn.SPLIT_DESIGNATED, 8, -1)
    assert kvattn.plan(1, 12, 64, 300, kv_dtype="bf16") == (kvattn.SPLIT_DESIGNATED, 3, -1)
    assert kvattn.plan(1, 12, 64, 1024, kv_dtype="bf16", strategy="lastblock") == (kvattn.SPLIT_LASTBLOCK, 4, -1)
    assert kvattn.plan(64, 12, 64, 8192, kv_dtype="bf16") == (kvattn.SPLIT_MERGE, 16, -1)
    assert kvattn.plan(1, 12, 64, 20000, kv_dtype="fp8", strategy="lastblock") == (kvattn.SPLIT_LASTBLOCK, 40, -1)
    # Every length fits fused_single: no split at all.
    assert kvattn.plan(1, 12, 64, 256, kv_dtype="bf16") == (kvattn.FUSED_SINGLE, 1, 0)
    # An explicit partition keeps its meaning without a hint.
    assert kvattn.plan(1, 12, 64, 1024, kv_dtype="bf16", S=8, strategy="split_merge") == (kvattn.SPLIT_MERGE, 8, 0)
    assert kvattn.plan(1, 12, 64, 1024, kv_dtype="bf16", S=-128, strategy="lastblock") == \
        (kvattn.SPLIT_LASTBLOCK, 8, 128)


def test_auto_without_hint_beyond_a_few_heads_takes_fixed_rows():
    # More than 16 heads, or a device-planned designated grid beyond 256 workgroups: the
    # hinted plan's designated window (or one segment per head) at maxT, fixed rows.
    assert kvattn.plan(2, 12, 64, 1024, kv_dtype="int8") == (kvattn.SPLIT_DESIGNATED, 8, 128)
    assert kvattn.plan(1, 12, 64, 4096, kv_dtype="bf16") == (kvattn.SPLIT_DESIGNATED, 16, 256)
    assert kvattn.plan(32, 12, 64, 1024, kv_dtype="fp8") == (kvattn.SPLIT_DESIGNATED, 2, 512)
    assert kvattn.plan(16, 12, 64, 512, kv_dtype="bf16") == (kvattn.SPLIT_LASTBLOCK, 1, 512)
    # ... but never its split + merge streaming plans: those stay planned on the device.
    assert kvattn.plan(32, 12, 64, 1024, kv_dtype="bf16") == (kvattn.SPLIT_LASTBLOCK, 4, -1)
    assert kvattn.plan(16, 12, 64, 4096, kv_dtype="int8") == (kvattn.SPLIT_MERGE, 8, -1)
    # A few heads whose device-planned designated grid fits keep it (GPT-2's layer).
    assert kvattn.plan(1, 12, 64, 2048, kv_dtype="bf16") == (kvattn.SPLIT_DESIGNATED, 16, -1)
    assert kvattn.plan(1, 16, 64, 1024, kv_dtype="fp8") == (kvattn.SPLIT_DESIGNATED, 8, -1)


def test_auto_skips_fused_single_when_scores_exceed_lds():
    # 64 KB of LDS holds 16384 scores; maxT beyond that rules fused_single out.
    st, _, _ = kvattn.plan(1, 12, 64, 20000, kv_dtype="bf16", len_hint=10)
    assert st != kvattn.FUSED_SINGLE


def test_explicit_strategies_and_partitions():
    assert kvattn.plan(1, 12, 64, 1024, kv_dtype="f32", len_hint=1023, S=8, strategy="coop") == \
        (kvattn.SINGLE_LAUNCH_COOP, 8, 0)
    assert kvattn.plan(2, 3, 64, 1000, kv_dtype="bf16", S=-100, strategy="split_merge") == \
        (kvattn.SPLIT_MERGE, 10, 100)
    assert kvattn.plan(2, 3, 64, 1000, kv_dtype="bf16", S=0, strategy="graph")[0] == kvattn.SINGLE_LAUNCH_GRAPH


@pytest.mark.parametrize("B,NH,maxT", [(1, 12, 1024), (64, 12, 8192), (3, 5, 777), (1, 1, 1)])
def test_workspace_for_S0_covers_every_auto_plan(B, NH, maxT):
    ws = kvattn.workspace_bytes(B, NH, 64, maxT, 0)
    for hint in sorted(h for h in {-1, 0, 1, maxT // 7, maxT // 2, maxT - 1} if h < maxT):
        for strategy in ("auto", "split_merge", "lastblock", "designated", "graph"):
            try:
                _, slots, _ = kvattn.plan(B, NH, 64, maxT, kv_dtype="bf16", len_hint=hint, strategy=strategy)
            except kvattn.KvAttnError as e:
                # The designated merger follows at most 64 segments per (b,h).
                assert strategy == "designated" and e.status == kvattn.ERR_SPLIT
                continue
            assert carve_bytes(B, NH, slots) <= ws


@pytest.mark.parametrize("kw,status", [
    (dict(len_hint=1024), kvattn.ERR_LENGTH),
    (dict(len_hint=-2), kvattn.ERR_LENGTH),
    (dict(strategy=9), kvattn.ERR_STRATEGY),
    (dict(S=1 << 20, strategy="split_merge"), kvattn.ERR_SPLIT),
])
def test_plan_errors(kw, status):
    a = dict(len_hint=-1, S=0, strategy="auto")
    a.update(kw)
    with pytest.raises(kvattn.KvAttnError) as ei:
        kvattn.plan(1, 12, 64, 1024, kv_dtype="bf16", **a)
    assert ei.value.status == status


def test_binding_raises_with_status_and_text():
    with pytest.raises(kvattn.KvAttnError) as ei:
        kvattn.decode(ALIGNED, ALIGNED, ALIGNED, 1, 12, 48, 1024, kv_dtype="bf16", stream=0)
    assert ei.value.status == kvattn.ERR_HEAD_DIM
    assert "head size must be 64" in str(ei.value)
    with pytest.raises(kvattn.KvAttnError) as ei:
        kvattn.attention_kv_merge(ALIGNED, ALIGNED, ALIGNED, ALIGNED, 1, 12, 64, 0, kv_dtype="bf16", stream=0)
    assert ei.value.status == kvattn.ERR_SPLIT
    with pytest.raises(kvattn.KvAttnError) as ei:
        kvattn.kv_cache_write(ALIGNED, ALIGNED, 1, 12, 64, 1024, kv_dtype="fp8", stream=0)
    assert ei.value.status == kvattn.ERR_DTYPE
    with pytest.raises(kvattn.KvAttnError) as ei:
        kvattn.decode(ALIGNED, ALIGNED, ALIGNED, 1, 12, 64, 1024, kv_dtype="bf16", len_hint=1023, stream=0)
    assert ei.value.status == kvattn.ERR_WORKSPACE     # split plan without a workspace


def _designated_rows_loop(total, heads):
    """The designated merger's segment length, as the rule reads: the whole length up to 256
    positions; otherwise 128 rows (256 beyond 16 heads), doubled while 64 segments do not
    cover the length."""
    if total <= 256:
        return max(total, 1)
    r = 128 if heads <= 16 else 256
    while r * 64 < total:
        r <<= 1
    return r


@pytest.mark.parametrize("heads", [1, 16, 17])
def test_designated_rows_closed_form_matches_the_rule(heads):
    """The library computes the designated rows without a loop (a power of two from a count
    of leading zeros); the host plan, with maxT = the hinted length, reports them."""
    totals = sorted({t for e in (256, 8192, 16384, 32768, 1 << 20) for t in (e - 1, e, e + 1)} |
                    {257, 300, 1000, 4097, 12345, 65536, 100000, 777777, (1 << 22) - 3, 1 << 22})
    for total in totals:
        rows = _designated_rows_loop(total, heads)
        st, slots, got = kvattn.plan(1, heads, 64, total, kv_dtype="bf16", len_hint=total - 1,
                                     strategy="designated")
        assert (st, got) == (kvattn.SPLIT_DESIGNATED, rows if total > 256 else total), (total, heads)
        assert slots == -(-total // got)


def test_auto_caps_hinted_split_segments_at_64_per_head():
    """AUTO with one length for the batch grows the rows instead of passing 64 segments per
    head of the hinted length (general plan: FP8 / FP32; tuned plan: BF16 / INT8, sized from
    the hint, not maxT); explicit strategies keep 512-row segments."""
    assert kvattn.plan(1, 12, 64, 65536, kv_dtype="fp8", len_hint=65535) == (kvattn.SPLIT_MERGE, 64, 1024)
    assert kvattn.plan(1, 12, 64, 65536, kv_dtype="f32", len_hint=65535) == (kvattn.SPLIT_MERGE, 64, 1024)
    assert kvattn.plan(1, 12, 64, 65536, kv_dtype="fp8", len_hint=65535, strategy="lastblock") == \
        (kvattn.SPLIT_LASTBLOCK, 128, 512)
    # a hint of 16384 in a 65536-row cache: 256-row segments for the hinted length, the grid
    # covering maxT
    assert kvattn.plan(8, 12, 64, 65536, kv_dtype="bf16", len_hint=16383) == (kvattn.SPLIT_MERGE, 256, 256)
    assert kvattn.plan(4, 12, 64, 32768, kv_dtype="fp8", len_hint=32767) == (kvattn.SPLIT_MERGE, 64, 512)
