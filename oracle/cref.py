"""ctypes loader of the oracle's C restatement (TEST INFRASTRUCTURE ONLY)."""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

_LIB = Path(__file__).resolve().parent / "_build" / "liboracle_ref.so"
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not _LIB.exists():
            from . import build
            build.build()
        _lib = ctypes.CDLL(str(_LIB))
        _lib.inl_ref_attn_f32.restype = ctypes.c_int
        _lib.inl_ref_attn_f32.argtypes = [
            ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_void_p]
        _lib.inl_ref_threads.restype = ctypes.c_int
    return _lib


def threads() -> int:
    return int(lib().inl_ref_threads())


def attention_f32(q, k, v, cu_seqlens, *, causal, window=-1, scale=1.0):
    """f32 packed attention (``q [N,Hq,D]``, ``k, v [N,Hkv,D]``) on the CPU."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
    out = np.zeros(q.shape, dtype=np.float32)
    rc = lib().inl_ref_attn_f32(len(cu) - 1, cu.ctypes.data, q.shape[1], k.shape[1], q.shape[2],
                                int(causal), int(window), float(scale), q.ctypes.data,
                                k.ctypes.data, v.ctypes.data, out.ctypes.data)
    if rc != 0:
        raise ValueError("inl_ref_attn_f32: bad arguments")
    return out
