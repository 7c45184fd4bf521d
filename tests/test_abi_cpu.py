"""CPU checks of the C ABI: the library loads, exports every symbol include/kvattn.h
declares, and rejects bad arguments with status codes before touching a GPU."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kvattn.h")


def _kv():
    from cuda_gpt2_inference_amd import kvattn
    return kvattn


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kvattn_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    kvattn = _kv()
    lib = kvattn.lib()
    declared = header_functions()
    assert len(declared) >= 12
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in kvattn.h but not exported"
    assert set(declared) == set(kvattn.SIGNATURES), "ctypes signatures out of sync with kvattn.h"


def test_symbols_are_c_linkage():
    """extern "C": exported names are unmangled (dlsym by plain name works)."""
    so = ctypes.CDLL(_kv().LIB_PATH)
    for name in header_functions():
        assert getattr(so, name) is not None


def test_strerror_covers_every_status():
    kvattn = _kv()
    seen = set()
    for st in range(0, 16):
        msg = kvattn.strerror(st)
        assert msg and msg != "unknown status"
        seen.add(msg)
    assert len(seen) == 16
    assert kvattn.strerror(99) == "unknown status"


def test_workspace_bytes():
    kvattn = _kv()
    # 256 bytes of status words, part_max, part_lse (B*NH*S f32), part_out (B*NH*S*64 f32), the
    # designated merger's tagged words ({max, exp-sum} in a 128-byte line per slot, B*NH*S*16
    # u64, and B*NH*S*64 u64 channel words), every region rounded up to 256 bytes; then room for
    # a counter region of 4 bytes per 904 bytes of buffer (904 = the partial and tag bytes of
    # one slot, so every plan the buffer holds finds a counter per head there): the smallest
    # size x with x - (4 x / 904 + 255) >= that sum, rounded up to 256.
    def expect(B, NH, S):
        up = lambda x: (x + 255) // 256 * 256  # noqa: E731
        fixed = (256 + 2 * up(B * NH * S * 4) + up(B * NH * S * 64 * 4)
                 + up(B * NH * S * 16 * 8) + up(B * NH * S * 64 * 8))
        x = up(-(-(fixed + 255) * 904 // 900))
        counters = up(x // 904 * 4)
        assert x >= fixed + counters and counters >= B * NH * 4
        return x
    assert kvattn.workspace_bytes(1, 12, 64, 1024, 8) == expect(1, 12, 8)
    assert kvattn.workspace_bytes(64, 12, 64, 8192, 0) == expect(64, 12, 8192 // 64)
    assert kvattn.workspace_bytes(2, 3, 64, 1000, -100) == expect(2, 3, 10)
    assert kvattn.workspace_bytes(1, 12, 32, 1024, 8) == 0      # hs != 64
    assert kvattn.workspace_bytes(0, 12, 64, 1024, 8) == 0      # B < 1


ALIGNED = 1 << 20   # a fake, 16-byte aligned address; never dereferenced by these calls


@pytest.mark.parametrize("kw,status", [
    (dict(hs=32), 3),                       # KVATTN_ERR_HEAD_DIM
    (dict(B=0), 4),                         # KVATTN_ERR_SHAPE
    (dict(maxT=0), 4),
    (dict(kv_dtype=7), 5),                  # KVATTN_ERR_DTYPE
    (dict(kv_dtype=2, kv_scale=None), 5),   # 8-bit without scales
    (dict(qkv=None), 1),                    # KVATTN_ERR_NULL_POINTER
    (dict(out=None), 1),
    (dict(kv=ALIGNED + 8), 2),              # KVATTN_ERR_MISALIGNED
    (dict(strategy=9), 6),                  # KVATTN_ERR_STRATEGY
    (dict(len_hint=5000), 12),              # KVATTN_ERR_LENGTH
])
@pytest.mark.parametrize("entry", ["kvattn_decode", "kvattn_append_decode"])
def test_decode_argument_errors(kw, status, entry):
    kvattn = _kv()
    a = dict(out=ALIGNED, qkv=ALIGNED, kv=ALIGNED, kv_scale=ALIGNED, B=1, NH=12, hs=64, maxT=1024,
             kv_dtype=1, strategy=0, len_hint=-1)
    a.update(kw)
    st = getattr(kvattn.lib(), entry)(a["out"], a["qkv"], a["kv"], a["kv_scale"], a["B"], a["NH"], a["hs"],
                                      a["maxT"], None, 0, a["len_hint"], None, 0, 0, a["strategy"],
                                      a["kv_dtype"], None)
    assert st == status, kvattn.strerror(st)


def test_other_entry_point_errors():
    kvattn = _kv()
    L = kvattn.lib()
    assert L.kvattn_cache_write(ALIGNED, None, ALIGNED, 1, 12, 48, 1024, None, 0, 1, None) == kvattn.ERR_HEAD_DIM
    assert L.kvattn_cache_write(ALIGNED, None, ALIGNED, 1, 12, 64, 1024, None, 0, 3, None) == kvattn.ERR_DTYPE
    assert L.kvattn_append(ALIGNED, None, ALIGNED, 1, 12, 48, 1024, None, 1, None) == kvattn.ERR_HEAD_DIM
    assert L.kvattn_append(ALIGNED, None, ALIGNED, 1, 12, 64, 1024, None, 3, None) == kvattn.ERR_DTYPE
    assert L.kvattn_append(None, None, ALIGNED, 1, 12, 64, 1024, None, 1, None) == kvattn.ERR_NULL_POINTER
    assert L.kvattn_forward_small(None, ALIGNED, ALIGNED, None, 1, 12, 64, 1024, None, 0, 1, None) == \
        kvattn.ERR_NULL_POINTER
    assert L.kvattn_forward_large(ALIGNED, ALIGNED, ALIGNED, None, 1, 12, 64, 1024, None, 0, ALIGNED, ALIGNED,
                                  ALIGNED, 0, 1, None) == kvattn.ERR_SPLIT
    assert L.kvattn_split(ALIGNED, None, ALIGNED, ALIGNED, ALIGNED, None, 1, 12, 64, 1024, None, 0, 8, 1,
                          None) == kvattn.ERR_NULL_POINTER
    assert L.kvattn_merge(ALIGNED, ALIGNED, ALIGNED, ALIGNED, 1, 12, 64, 1 << 20, 1, None) == kvattn.ERR_SPLIT
    assert L.kvattn_merge(ALIGNED + 4, ALIGNED, ALIGNED, ALIGNED, 1, 12, 64, 8, 1, None) == kvattn.ERR_MISALIGNED
    assert L.kvattn_cur_len_symbol(None) == kvattn.ERR_NULL_POINTER
    assert L.kvattn_set_cur_len_async(ALIGNED, -1, None) == kvattn.ERR_LENGTH
    assert L.kvattn_set_cur_len_async(ALIGNED, 1 << 23, None) == kvattn.ERR_LENGTH
    assert L.kvattn_workspace_init(None, 0, None) == kvattn.ERR_NULL_POINTER


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    kvattn = _kv()
    monkeypatch.setattr(kvattn, "_LIB", None)
    monkeypatch.setattr(kvattn, "LIB_PATH", str(tmp_path / "libkvattn.so"))
    with pytest.raises(kvattn.KvAttnError):
        kvattn.lib()


@pytest.mark.parametrize("kw,status", [
    (dict(table=None), 1),               # KVATTN_ERR_NULL_POINTER
    (dict(table=ALIGNED + 2), 2),        # KVATTN_ERR_MISALIGNED
    (dict(page_rows=32), 4),             # below one 64-row tile: KVATTN_ERR_SHAPE
    (dict(page_rows=100), 4),            # not a multiple of 64
    (dict(max_pages=0), 4),
    (dict(num_pages=0), 4),
    (dict(max_pages=1 << 20, page_rows=1 << 10), 4),   # more positions than a cache may hold
    (dict(strategy=1), 6),               # FUSED_SINGLE: KVATTN_ERR_STRATEGY
    (dict(strategy=3), 6),               # cooperative
    (dict(S=8), 8),                      # reference partition: KVATTN_ERR_SPLIT
    (dict(S=-100), 8),                   # rows per segment not a multiple of 64
    (dict(S=-8192), 8),                  # more than 4096 rows per segment
    (dict(len_hint=1 << 20), 12),        # KVATTN_ERR_LENGTH
])
def test_paged_decode_argument_errors(kw, status):
    kvattn = _kv()
    a = dict(table=ALIGNED, max_pages=16, page_rows=64, num_pages=16, strategy=0, S=0, len_hint=-1)
    a.update(kw)
    st = kvattn.lib().kvattn_paged_decode(ALIGNED, ALIGNED, ALIGNED, None, a["table"], a["max_pages"],
                                          a["page_rows"], a["num_pages"], 1, 12, 64, None, 0, a["len_hint"],
                                          ALIGNED, 1 << 30, a["S"], a["strategy"], 1, 0, None)
    assert st == status, kvattn.strerror(st)
    if "strategy" not in kw and "S" not in kw and "len_hint" not in kw:
        st = kvattn.lib().kvattn_paged_cache_write(ALIGNED, None, a["table"], a["max_pages"], a["page_rows"],
                                                   a["num_pages"], ALIGNED, 1, 12, 64, None, 0, 1, None)
        assert st == status, kvattn.strerror(st)


def test_set_merge_poll_limit_round_trip():
    """The designated merger's poll bound is host state only (no GPU call)."""
    kvattn = _kv()
    prev = kvattn.set_merge_poll_limit(5)
    try:
        assert kvattn.set_merge_poll_limit(-1) == 5
        assert kvattn.set_merge_poll_limit(-1) == 1 << 16
    finally:
        kvattn.set_merge_poll_limit(prev)


def test_workspace_status_rejects_bad_arguments():
    kvattn = _kv()
    n = ctypes.c_int(-1)
    assert kvattn.lib().kvattn_workspace_status(None, 4096, 0, None, ctypes.byref(n)) == kvattn.ERR_NULL_POINTER
    assert kvattn.lib().kvattn_workspace_status(ALIGNED + 4, 4096, 0, None, ctypes.byref(n)) == kvattn.ERR_MISALIGNED
    assert kvattn.lib().kvattn_workspace_status(ALIGNED, 100, 0, None, ctypes.byref(n)) == kvattn.ERR_WORKSPACE
