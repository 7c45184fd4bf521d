"""ctypes binding of libkvattn.so (the C ABI declared in include/kvattn.h).

Two layers:

* ``lib()`` returns the loaded library with every entry point's argtypes/restype set;
  arguments are raw device pointers (ints) and sizes, exactly the C ABI.
* The functions named after the reference's host entry points
  (``kv_cache_write``, ``attention_forward_kv_small``, ``attention_forward_kv_large``,
  ``attention_kv_split``, ``attention_kv_merge``) and ``decode`` accept torch tensors
  (or raw pointers), pass ``torch.cuda.current_stream()`` unless a stream is given, and
  raise ``KvAttnError`` on a non-zero status -- the reference's ``cudaCheck`` prints and
  exits (Inference_gpt2/common.h:123-130); a Python caller gets an exception instead.

There is no fallback: if the shared library is missing, importing the binding works
but the first call raises ``KvAttnError`` telling the caller to build it.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libkvattn.so")

# kvattn_status
OK = 0
ERR_NULL_POINTER = 1
ERR_MISALIGNED = 2
ERR_HEAD_DIM = 3
ERR_SHAPE = 4
ERR_DTYPE = 5
ERR_STRATEGY = 6
ERR_WORKSPACE = 7
ERR_SPLIT = 8
ERR_COOP_TOO_LARGE = 9
ERR_LDS = 10
ERR_CAPTURE = 11
ERR_LENGTH = 12
ERR_HIP = 13
ERR_GRID_TOO_LARGE = 14
ERR_MERGE_TIMEOUT = 15

# kvattn_dtype
KV_F32 = 0
KV_BF16 = 1
KV_INT8 = 2
KV_FP8_E4M3 = 3
KV_DTYPES = {"f32": KV_F32, "bf16": KV_BF16, "int8": KV_INT8, "fp8": KV_FP8_E4M3}

# kvattn_strategy
AUTO = 0
FUSED_SINGLE = 1
SPLIT_MERGE = 2
SINGLE_LAUNCH_COOP = 3
SINGLE_LAUNCH_GRAPH = 4
SPLIT_LASTBLOCK = 5
SPLIT_DESIGNATED = 6
STRATEGIES = {
    "auto": AUTO,
    "fused_single": FUSED_SINGLE,
    "split_merge": SPLIT_MERGE,
    "coop": SINGLE_LAUNCH_COOP,
    "graph": SINGLE_LAUNCH_GRAPH,
    "lastblock": SPLIT_LASTBLOCK,
    "designated": SPLIT_DESIGNATED,
}

HEAD_DIM = 64

_vp = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/kvattn.h one to one.
SIGNATURES = {
    "kvattn_strerror": (ctypes.c_char_p, [_i]),
    "kvattn_last_hip_error": (_i, []),
    "kvattn_cur_len_symbol": (_i, [ctypes.POINTER(_vp)]),
    "kvattn_set_cur_len": (_i, [_i]),
    "kvattn_set_cur_len_async": (_i, [_vp, _i, _vp]),
    "kvattn_cache_write": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp, _i, _i, _vp]),
    "kvattn_append": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp, _i, _vp]),
    "kvattn_forward_small": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _i, _i, _vp]),
    "kvattn_forward_large": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _i, _vp, _vp, _vp, _i, _i, _vp]),
    "kvattn_split": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _i, _i, _i, _vp]),
    "kvattn_merge": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "kvattn_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "kvattn_workspace_init": (_i, [_vp, _sz, _vp]),
    "kvattn_workspace_status": (_i, [_vp, _sz, _i, _vp, ctypes.POINTER(_i)]),
    "kvattn_set_merge_poll_limit": (_i, [_i]),
    "kvattn_scratch_status": (_i, [_i, _vp, ctypes.POINTER(_i)]),
    "kvattn_call_identity": (_i, [_vp, _vp]),
    "kvattn_set_xcd_layout_offset": (_i, [_i]),
    "kvattn_plan": (_i, [_i, _i, _i, _i, _i, _i, _i, _i, ctypes.POINTER(_i), ctypes.POINTER(_i),
                         ctypes.POINTER(_i)]),
    "kvattn_decode": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _i, _i, _vp, _sz, _i, _i, _i, _vp]),
    "kvattn_append_decode": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _i, _i, _vp, _sz, _i, _i, _i, _vp]),
    "kvattn_decode_static": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _i, _i, _i, _i, _i, _vp]),
    "kvattn_gemv": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "kvattn_gemv_ex": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "kvattn_gemv_qkv_append": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _i, _vp, _i, _i, _i, _vp,
                                    _sz, _vp]),
    "kvattn_gemv_qkv_append_workspace_bytes": (_sz, [_i, _i]),
    "kvattn_paged_cache_write": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp, _i, _i, _i, _vp, _i, _i, _vp]),
    "kvattn_paged_decode": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _i, _i, _vp, _sz, _i, _i,
                                 _i, _i, _vp]),
}


class KvAttnError(RuntimeError):
    def __init__(self, status: int, where: str):
        self.status = status
        text = strerror(status) if _LIB is not None else "library not loaded"
        hip = ""
        if status == ERR_HIP and _LIB is not None:
            hip = f" (hipError {_LIB.kvattn_last_hip_error()})"
        super().__init__(f"{where}: kvattn status {status}: {text}{hip}")


_LIB: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """Load libkvattn.so once; raise if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise KvAttnError(-1, f"{LIB_PATH} is missing; build it with __graft_entry__.build() "
                                  "or `make -C cuda_gpt2_inference_amd/csrc`")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def strerror(status: int) -> str:
    return lib().kvattn_strerror(status).decode()


def _check(status: int, where: str) -> None:
    if status != OK:
        raise KvAttnError(status, where)


def _ptr(x) -> Optional[int]:
    """Device address of a tensor, an int address, or None."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


def _stream(stream) -> Optional[int]:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def kv_dtype_code(kv_dtype) -> int:
    if isinstance(kv_dtype, str):
        return KV_DTYPES[kv_dtype]
    return int(kv_dtype)


def strategy_code(strategy) -> int:
    if isinstance(strategy, str):
        return STRATEGIES[strategy]
    return int(strategy)


def cur_len_symbol() -> int:
    """Device address of the library's own device-resident length."""
    p = _vp()
    _check(lib().kvattn_cur_len_symbol(ctypes.byref(p)), "kvattn_cur_len_symbol")
    return int(p.value)


def set_cur_len(cur_len: int) -> None:
    _check(lib().kvattn_set_cur_len(int(cur_len)), "kvattn_set_cur_len")


def set_cur_len_async(cur_len: int, d_cur_len=None, stream=None) -> None:
    """Stream-ordered write of the device length (no host synchronisation)."""
    _check(lib().kvattn_set_cur_len_async(_ptr(d_cur_len), int(cur_len), _stream(stream)),
           "kvattn_set_cur_len_async")


def kv_cache_write(kv_cache, qkv, B, NH, hs, maxT, *, kv_dtype, kv_scale=None, cur_len=None,
                   lens_per_seq=False, stream=None) -> None:
    """Append the current token's K/V (reference kv_cache_write_kernel[_w8])."""
    _check(lib().kvattn_cache_write(_ptr(kv_cache), _ptr(kv_scale), _ptr(qkv), B, NH, hs, maxT,
                                    _ptr(cur_len), int(bool(lens_per_seq)), kv_dtype_code(kv_dtype),
                                    _stream(stream)), "kvattn_cache_write")


def attention_forward_kv_small(out, qkv, kv_cache, B, NH, hs, maxT, *, kv_dtype, kv_scale=None,
                               cur_len=None, lens_per_seq=False, stream=None) -> None:
    """fused_single (reference attention_forward_kv_small[_w8])."""
    _check(lib().kvattn_forward_small(_ptr(out), _ptr(qkv), _ptr(kv_cache), _ptr(kv_scale), B, NH, hs, maxT,
                                      _ptr(cur_len), int(bool(lens_per_seq)), kv_dtype_code(kv_dtype),
                                      _stream(stream)), "kvattn_forward_small")


def attention_forward_kv_large(out, qkv, kv_cache, B, NH, hs, maxT, part_out, part_lse, part_max, S, *,
                               kv_dtype, kv_scale=None, cur_len=None, lens_per_seq=False,
                               stream=None) -> None:
    """Split + merge or cooperative (reference attention_forward_kv_large[_w8])."""
    _check(lib().kvattn_forward_large(_ptr(out), _ptr(qkv), _ptr(kv_cache), _ptr(kv_scale), B, NH, hs, maxT,
                                      _ptr(cur_len), int(bool(lens_per_seq)), _ptr(part_out), _ptr(part_lse),
                                      _ptr(part_max), S, kv_dtype_code(kv_dtype), _stream(stream)),
           "kvattn_forward_large")


def attention_kv_split(part_out, part_lse, part_max, qkv, kv_cache, B, NH, hs, maxT, S, *, kv_dtype,
                       kv_scale=None, cur_len=None, lens_per_seq=False, stream=None) -> None:
    """Split phase (reference attention_kv_split_kernel[_w8])."""
    _check(lib().kvattn_split(_ptr(part_out), _ptr(part_lse), _ptr(part_max), _ptr(qkv), _ptr(kv_cache),
                              _ptr(kv_scale), B, NH, hs, maxT, _ptr(cur_len), int(bool(lens_per_seq)), S,
                              kv_dtype_code(kv_dtype), _stream(stream)), "kvattn_split")


def attention_kv_merge(out, part_out, part_lse, part_max, B, NH, hs, S, *, kv_dtype, stream=None) -> None:
    """Merge phase (reference attention_kv_merge_kernel[_w8])."""
    _check(lib().kvattn_merge(_ptr(out), _ptr(part_out), _ptr(part_lse), _ptr(part_max), B, NH, hs, S,
                              kv_dtype_code(kv_dtype), _stream(stream)), "kvattn_merge")


def workspace_bytes(B, NH, hs, maxT, S=0) -> int:
    return int(lib().kvattn_workspace_bytes(B, NH, hs, maxT, S))


def workspace_init(workspace, nbytes, stream=None) -> None:
    _check(lib().kvattn_workspace_init(_ptr(workspace), nbytes, _stream(stream)), "kvattn_workspace_init")


def workspace_status(workspace, nbytes, clear=False, stream=None) -> int:
    """Merges that stopped waiting since the workspace was initialised or last cleared
    (kvattn_workspace_status; synchronises the stream): designated mergers that computed
    their producers' segments themselves, cooperative mergers that wrote NaN.  Returns the
    count; it is not an error to find one here."""
    n = _i()
    st = lib().kvattn_workspace_status(_ptr(workspace), int(nbytes), int(bool(clear)), _stream(stream),
                                       ctypes.byref(n))
    if st not in (OK, ERR_MERGE_TIMEOUT):
        _check(st, "kvattn_workspace_status")
    return n.value


def scratch_status(clear=False, stream=None) -> int:
    """Merges that stopped waiting in the library's static scratch array on the current device
    (kvattn_scratch_status; the workspace of decode_static and of forward_large's single
    launch; synchronises the stream).  Returns the count."""
    n = _i()
    st = lib().kvattn_scratch_status(int(bool(clear)), _stream(stream), ctypes.byref(n))
    if st not in (OK, ERR_MERGE_TIMEOUT):
        _check(st, "kvattn_scratch_status")
    return n.value


def call_identity(out, stream=None) -> None:
    """Enqueue one dispatch that writes {dispatch id, queue address, tag} into out (3 int64
    words on the device): the identity a tagged partial word of that stream carries."""
    _check(lib().kvattn_call_identity(_ptr(out), _stream(stream)), "kvattn_call_identity")


def set_xcd_layout_offset(rot: int) -> int:
    """Test setting: designated producers `rot` XCDs away from their merger (0: the layout in
    use).  Returns the previous setting."""
    return int(lib().kvattn_set_xcd_layout_offset(int(rot)))


def set_merge_poll_limit(polls: int) -> int:
    """Bound on a merger's polls for later launches (0: stop waiting at once, a
    fault-injection setting; < 0: the default, 2^16).  Returns the previous bound."""
    return int(lib().kvattn_set_merge_poll_limit(int(polls)))


def plan(B, NH, hs, maxT, *, kv_dtype, len_hint=-1, S=0, strategy="auto"):
    """(strategy code, segment slots per (b,h), rows per segment) kvattn_decode would use."""
    st, seg, rows = _i(), _i(), _i()
    _check(lib().kvattn_plan(B, NH, hs, maxT, int(len_hint), int(S), strategy_code(strategy),
                             kv_dtype_code(kv_dtype), ctypes.byref(st), ctypes.byref(seg), ctypes.byref(rows)),
           "kvattn_plan")
    return st.value, seg.value, rows.value


STRATEGY_NAMES = {v: k for k, v in STRATEGIES.items()}


def decode(out, qkv, kv_cache, B, NH, hs, maxT, *, kv_dtype, kv_scale=None, cur_len=None,
           lens_per_seq=False, len_hint=-1, workspace=None, workspace_nbytes=0, S=0, strategy="auto",
           stream=None) -> None:
    """One decode-attention call with an explicit strategy (kvattn_decode)."""
    _check(lib().kvattn_decode(_ptr(out), _ptr(qkv), _ptr(kv_cache), _ptr(kv_scale), B, NH, hs, maxT,
                               _ptr(cur_len), int(bool(lens_per_seq)), int(len_hint), _ptr(workspace),
                               int(workspace_nbytes), int(S), strategy_code(strategy),
                               kv_dtype_code(kv_dtype), _stream(stream)), "kvattn_decode")


def decode_static(out, qkv, kv_cache, B, NH, hs, maxT, *, kv_dtype, kv_scale=None, cur_len=None,
                  lens_per_seq=False, len_hint=-1, S=0, strategy="auto", stream=None) -> None:
    """decode with the library's static device scratch as workspace (kvattn_decode_static):
    allocates nothing; calls that overlap in time on one GPU race."""
    _check(lib().kvattn_decode_static(_ptr(out), _ptr(qkv), _ptr(kv_cache), _ptr(kv_scale), B, NH, hs, maxT,
                                      _ptr(cur_len), int(bool(lens_per_seq)), int(len_hint), int(S),
                                      strategy_code(strategy), kv_dtype_code(kv_dtype), _stream(stream)),
           "kvattn_decode_static")


def append_decode(out, qkv, kv_cache, B, NH, hs, maxT, *, kv_dtype, kv_scale=None, cur_len=None,
                  lens_per_seq=False, len_hint=-1, workspace=None, workspace_nbytes=0, S=0, strategy="auto",
                  stream=None) -> None:
    """kv_cache_write + decode in one launch (kvattn_append_decode)."""
    _check(lib().kvattn_append_decode(_ptr(out), _ptr(qkv), _ptr(kv_cache), _ptr(kv_scale), B, NH, hs, maxT,
                                      _ptr(cur_len), int(bool(lens_per_seq)), int(len_hint), _ptr(workspace),
                                      int(workspace_nbytes), int(S), strategy_code(strategy),
                                      kv_dtype_code(kv_dtype), _stream(stream)), "kvattn_append_decode")


def gemv(out, W, x, B, M, K, *, w_dtype, w_scale=None, bias=None, pre_gelu=None, gelu=False, out_dtype=None,
         stream=None) -> None:
    """Decode-step fully connected layer out = [GELU](W x [* w_scale] + bias) (kvattn_gemv;
    kvattn_gemv_ex when out_dtype, "f32" or "bf16", is given)."""
    if out_dtype is None:
        _check(lib().kvattn_gemv(_ptr(out), _ptr(pre_gelu), _ptr(W), _ptr(w_scale), _ptr(x), _ptr(bias), B, M, K,
                                 kv_dtype_code(w_dtype), int(bool(gelu)), _stream(stream)), "kvattn_gemv")
        return
    _check(lib().kvattn_gemv_ex(_ptr(out), _ptr(pre_gelu), _ptr(W), _ptr(w_scale), _ptr(x), _ptr(bias), B, M, K,
                                kv_dtype_code(w_dtype), kv_dtype_code(out_dtype), int(bool(gelu)),
                                _stream(stream)), "kvattn_gemv_ex")


def gemv_qkv_append(qkv, W, x, B, NH, hs, K, kv_cache, maxT, *, w_dtype, kv_dtype=None, w_scale=None, bias=None,
                    kv_scale=None, cur_len=None, lens_per_seq=False, workspace=None, workspace_nbytes=0,
                    stream=None) -> None:
    """QKV projection with the KV append in its epilogue (kvattn_gemv_qkv_append).  kv_dtype
    defaults to the activation type (f32 for f32 weights, else bf16); 8-bit caches need
    kv_scale and a workspace of gemv_qkv_append_workspace_bytes(B, NH), zeroed once."""
    if kv_dtype is None:
        kv_dtype = "f32" if kv_dtype_code(w_dtype) == KV_F32 else "bf16"
    _check(lib().kvattn_gemv_qkv_append(_ptr(qkv), _ptr(W), _ptr(w_scale), _ptr(x), _ptr(bias), B, NH, hs, K,
                                        _ptr(kv_cache), _ptr(kv_scale), maxT, _ptr(cur_len),
                                        int(bool(lens_per_seq)), kv_dtype_code(w_dtype), kv_dtype_code(kv_dtype),
                                        _ptr(workspace), int(workspace_nbytes), _stream(stream)),
           "kvattn_gemv_qkv_append")


def gemv_qkv_append_workspace_bytes(B: int, NH: int) -> int:
    """Workspace bytes gemv_qkv_append needs for an 8-bit cache."""
    return int(lib().kvattn_gemv_qkv_append_workspace_bytes(B, NH))


class PagedCache:
    """A paged KV cache: a page pool [num_pages][2][NH][page_rows][hs] (+ row scales for
    8-bit caches) and a block table [B][max_pages] of page ids (device tensors)."""

    def __init__(self, pages, block_table, max_pages, page_rows, num_pages, page_scales=None):
        self.pages, self.block_table, self.page_scales = pages, block_table, page_scales
        self.max_pages, self.page_rows, self.num_pages = int(max_pages), int(page_rows), int(num_pages)

    @property
    def maxT(self) -> int:
        return self.max_pages * self.page_rows

    def _args(self):
        return (_ptr(self.pages), _ptr(self.page_scales), _ptr(self.block_table), self.max_pages, self.page_rows,
                self.num_pages)


def paged_cache_write(cache: PagedCache, qkv, B, NH, hs, *, kv_dtype, cur_len=None, lens_per_seq=False,
                      stream=None) -> None:
    """kv_cache_write into a paged cache (kvattn_paged_cache_write)."""
    _check(lib().kvattn_paged_cache_write(*cache._args(), _ptr(qkv), B, NH, hs, _ptr(cur_len),
                                          int(bool(lens_per_seq)), kv_dtype_code(kv_dtype), _stream(stream)),
           "kvattn_paged_cache_write")


def paged_decode(out, qkv, cache: PagedCache, B, NH, hs, *, kv_dtype, cur_len=None, lens_per_seq=False,
                 len_hint=-1, workspace=None, workspace_nbytes=0, S=0, strategy="auto", append=False,
                 stream=None) -> None:
    """decode / append_decode on a paged cache (kvattn_paged_decode)."""
    p = cache._args()
    _check(lib().kvattn_paged_decode(_ptr(out), _ptr(qkv), p[0], p[1], p[2], p[3], p[4], p[5], B, NH, hs,
                                     _ptr(cur_len), int(bool(lens_per_seq)), int(len_hint), _ptr(workspace),
                                     int(workspace_nbytes), int(S), strategy_code(strategy),
                                     kv_dtype_code(kv_dtype), int(bool(append)), _stream(stream)),
           "kvattn_paged_decode")


class Workspace:
    """Device workspace for ``decode``: allocated with torch, counters zeroed once."""

    def __init__(self, B, NH, maxT, S=0, device="cuda"):
        import torch
        self.nbytes = workspace_bytes(B, NH, HEAD_DIM, maxT, S)
        if self.nbytes == 0:
            raise KvAttnError(ERR_SHAPE, "kvattn_workspace_bytes")
        self.buf = torch.empty(self.nbytes, dtype=torch.uint8, device=device)
        workspace_init(self.buf, self.nbytes)

    def kwargs(self):
        return {"workspace": self.buf, "workspace_nbytes": self.nbytes}

    def status(self, clear=False, stream=None) -> int:
        """Designated merges on this workspace that stopped waiting (see workspace_status)."""
        return workspace_status(self.buf, self.nbytes, clear=clear, stream=stream)
