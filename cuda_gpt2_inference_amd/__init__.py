"""MI355X (gfx950) decode-phase KV-cache attention.

The compute lives in ``libkvattn.so`` (hand-written HIP kernels behind the C ABI of
``include/kvattn.h``); ``kvattn`` is its ctypes binding.
"""
from . import kvattn  # noqa: F401
from .kvattn import KvAttnError, Workspace, decode  # noqa: F401

__all__ = ["kvattn", "KvAttnError", "Workspace", "decode"]
