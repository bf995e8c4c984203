"""Python binding of ``libinl_hip.so`` (the gfx950 encoder-attention C ABI).

This is the host-side mirror of the reference's attention call for Python
callers, tests and the benchmark. Torch tensors are used only as device
buffers: every computation runs in the HIP library. If the library is
missing, importing this module raises - there is no fallback path.

The functions take packed tensors (texts back to back, token-major) and a
``cu_seqlens`` host sequence, the layout of ``include/inl_hip.h``.
"""
from __future__ import annotations

import ctypes
import math
import os
from pathlib import Path
from typing import Optional, Sequence

_LIB_PATH = Path(__file__).resolve().parent / "libinl_hip.so"

if not _LIB_PATH.exists():
    raise ImportError(
        f"{_LIB_PATH} is not built; run `python im-not-llm_amd/build.py` "
        "(the HIP path has no fallback)")

_lib = ctypes.CDLL(str(_LIB_PATH))

INL_F32 = 0
INL_BF16 = 1

c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_void_p = ctypes.c_void_p


class AttnDesc(ctypes.Structure):
    _fields_ = [
        ("n_texts", c_i32),
        ("cu_seqlens_host", ctypes.POINTER(c_i32)),
        ("h_q", c_i32),
        ("h_kv", c_i32),
        ("head_dim", c_i32),
        ("causal", c_i32),
        ("window", c_i32),
        ("scale", ctypes.c_float),
        ("dtype", c_i32),
        ("out_dtype", c_i32),
        ("q_row_stride", c_i64),
        ("k_row_stride", c_i64),
        ("v_row_stride", c_i64),
        ("o_row_stride", c_i64),
        ("flags", c_i32),
    ]


ATTN_PV_BF16 = 1


class NormRopeDesc(ctypes.Structure):
    _fields_ = [
        ("n_texts", c_i32),
        ("cu_seqlens_host", ctypes.POINTER(c_i32)),
        ("heads", c_i32),
        ("head_dim", c_i32),
        ("x_row_stride", c_i64),
        ("y_row_stride", c_i64),
        ("dtype", c_i32),
        ("out_dtype", c_i32),
        ("norm", c_i32),
        ("eps", ctypes.c_float),
        ("rotary_dim", c_i32),
        ("sections", c_i32),
        ("table_rows", c_i32),
        ("round_tables", c_i32),
        ("round_norm", c_i32),
    ]


def _sig(name, restype, *argtypes):
    fn = getattr(_lib, name, None)
    if fn is None:
        return None
    fn.restype = restype
    fn.argtypes = list(argtypes)
    return fn


_lib.inl_last_error.restype = ctypes.c_char_p
_lib.inl_abi_version.restype = c_i32
_plan_create = _sig("inl_attn_plan_create", ctypes.c_int,
                    ctypes.POINTER(AttnDesc), ctypes.POINTER(c_void_p))
_plan_destroy = _sig("inl_attn_plan_destroy", ctypes.c_int, c_void_p)
_plan_info = _sig("inl_attn_plan_info", ctypes.c_int, c_void_p,
                  ctypes.POINTER(c_i64), ctypes.POINTER(c_i32), ctypes.POINTER(c_i32))
_attn_fwd = _sig("inl_attn_fwd", ctypes.c_int, c_void_p, c_void_p, c_void_p,
                 c_void_p, c_void_p, c_void_p)
_ws_size = _sig("inl_attn_workspace_size", ctypes.c_int, ctypes.POINTER(AttnDesc),
                ctypes.POINTER(ctypes.c_size_t))
_varlen_fwd = _sig("inl_attn_varlen_fwd", ctypes.c_int, ctypes.POINTER(AttnDesc),
                   c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, ctypes.c_size_t,
                   c_void_p)


class InlError(RuntimeError):
    """A non-zero status from the library, with its message."""

    def __init__(self, code: int, message: str):
        super().__init__(f"inl_hip error {code}: {message}")
        self.code = code
        self.message = message


def last_error() -> str:
    return (_lib.inl_last_error() or b"").decode()


def _check(rc: int) -> None:
    if rc != 0:
        raise InlError(rc, last_error())


def library_path() -> Path:
    return _LIB_PATH


def abi_version() -> int:
    return int(_lib.inl_abi_version())


def exported_symbols() -> list:
    """Names of the inl_* entry points this build exports (ctypes lookup)."""
    names = []
    for n in ("inl_attn_plan_create", "inl_attn_plan_destroy", "inl_attn_plan_info",
              "inl_attn_fwd", "inl_attn_workspace_size", "inl_attn_varlen_fwd",
              "inl_norm_rope_fwd", "inl_rope_table_host", "inl_pool_last_fwd",
              "inl_pool_mean_fwd", "inl_l2_normalize_fwd", "inl_pool_splade_fwd",
              "inl_last_error", "inl_abi_version"):
        if getattr(_lib, n, None) is not None:
            names.append(n)
    return names


def _cu_array(cu_seqlens: Sequence[int]):
    arr = (c_i32 * len(cu_seqlens))(*[int(x) for x in cu_seqlens])
    return arr


def _dtype_code(t) -> int:
    import torch
    if t == torch.bfloat16:
        return INL_BF16
    if t == torch.float32:
        return INL_F32
    raise InlError(-1, f"unsupported dtype {t}")


def _stream_ptr(stream) -> int:
    import torch
    if stream is None:
        stream = torch.cuda.current_stream()
    return int(stream.cuda_stream)


def make_attn_desc(cu_seqlens, h_q, h_kv, head_dim, *, causal, window=-1, scale=None,
                   dtype="bf16", out_dtype=None, q_row_stride=0, k_row_stride=0,
                   v_row_stride=0, o_row_stride=0, flags=0):
    """Build an ``AttnDesc``; the cu_seqlens array is kept alive on it."""
    cu = _cu_array(cu_seqlens)
    codes = {"bf16": INL_BF16, "f32": INL_F32, INL_BF16: INL_BF16, INL_F32: INL_F32}
    d = AttnDesc()
    d.n_texts = len(cu_seqlens) - 1
    d.cu_seqlens_host = cu
    d.h_q, d.h_kv, d.head_dim = int(h_q), int(h_kv), int(head_dim)
    d.causal = int(bool(causal))
    d.window = int(window if window is not None else -1)
    d.scale = float(scale if scale is not None else head_dim ** -0.5)
    d.dtype = codes[dtype]
    d.out_dtype = codes[out_dtype if out_dtype is not None else dtype]
    d.q_row_stride, d.k_row_stride = int(q_row_stride), int(k_row_stride)
    d.v_row_stride, d.o_row_stride = int(v_row_stride), int(o_row_stride)
    d.flags = int(flags)
    d._cu_keepalive = cu
    return d


class AttnPlan:
    """A device-resident tile schedule for one packed batch and one attention
    form (``inl_attn_plan_create``); reusable across layers of that form."""

    def __init__(self, desc: AttnDesc):
        self.desc = desc
        h = c_void_p()
        _check(_plan_create(ctypes.byref(desc), ctypes.byref(h)))
        self._h = h

    @property
    def handle(self) -> int:
        return self._h.value or 0

    def info(self):
        n = c_i64()
        bm = c_i32()
        bn = c_i32()
        _check(_plan_info(self._h, ctypes.byref(n), ctypes.byref(bm), ctypes.byref(bn)))
        return {"tiles": n.value, "block_m": bm.value, "block_n": bn.value}

    def run(self, q, k, v, out, stream=None) -> None:
        """Enqueue ``out = attention(q, k, v)`` (torch device tensors)."""
        _check(_attn_fwd(self._h, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                         out.data_ptr(), _stream_ptr(stream)))

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            _check(_plan_destroy(self._h))
            self._h = c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def varlen_attention(q, k, v, cu_seqlens, *, causal: bool, window: int = -1,
                     scale: Optional[float] = None, out_dtype=None, out=None,
                     stream=None, flags: int = 0):
    """Packed attention over torch device tensors ``q [N, Hq, D]``,
    ``k, v [N, Hkv, D]`` (token rows may be strided views of a fused QKV
    buffer). Returns ``out [N, Hq, D]``. Uses the one-shot C entry point
    (``inl_attn_varlen_fwd``) with a workspace from torch's allocator."""
    import torch
    n, hq, d = q.shape
    hkv = k.shape[1]
    dt = "bf16" if q.dtype == torch.bfloat16 else "f32"
    od = out_dtype if out_dtype is not None else q.dtype
    if out is None:
        out = torch.empty((n, hq, d), dtype=od, device=q.device)
    desc = make_attn_desc(cu_seqlens, hq, hkv, d, causal=causal, window=window, scale=scale,
                          dtype=dt, out_dtype="bf16" if out.dtype == torch.bfloat16 else "f32",
                          q_row_stride=q.stride(0), k_row_stride=k.stride(0),
                          v_row_stride=v.stride(0), o_row_stride=out.stride(0), flags=flags)
    for name, t in (("q", q), ("k", k), ("v", v), ("out", out)):
        if t.stride(2) != 1 or t.stride(1) != d:
            raise InlError(-1, f"{name}: heads must be contiguous inside a token row")
    nbytes = ctypes.c_size_t()
    _check(_ws_size(ctypes.byref(desc), ctypes.byref(nbytes)))
    ws = torch.empty(max(16, nbytes.value), dtype=torch.uint8, device=q.device)
    _check(_varlen_fwd(ctypes.byref(desc), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                       out.data_ptr(), ws.data_ptr(), nbytes.value, _stream_ptr(stream)))
    out._inl_workspace = ws  # keep alive until the stream has consumed it
    return out


def attention_flops(lengths, h_q, head_dim, causal, window=-1) -> int:
    """Algorithmic FLOPs of one call: ``4 * H_q * d * visible (q, k) pairs``."""
    total = 0
    for t in lengths:
        t = int(t)
        if t <= 0:
            continue
        if window is None or window < 0:
            total += t * (t + 1) // 2 if causal else t * t
        else:
            w = int(window)
            for qi in range(t):
                hi = min(t, qi + w + 1)
                if causal:
                    hi = min(hi, qi + 1)
                total += hi - max(0, qi - w)
    return 4 * h_q * head_dim * total
