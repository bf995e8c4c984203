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

# torch ships its own HIP runtime with the same soname (libamdhip64.so.7).
# Loading torch first makes this library bind to that runtime; loaded the
# other way round the process holds two HIP runtimes, and the second one to
# open the device finds none.
try:
    import torch  # noqa: F401
except ImportError:
    pass

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
        ("seq_starts_host", ctypes.POINTER(c_i32)),
    ]


ATTN_PV_BF16 = 1
ATTN_NO_SPLIT = 2


class NormRopeDesc(ctypes.Structure):
    _fields_ = [
        ("n_tokens", c_i64),
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
_kernel_name = _sig("inl_attn_kernel_name", ctypes.c_int, ctypes.POINTER(AttnDesc),
                    ctypes.POINTER(ctypes.c_char_p))


_norm_rope = _sig("inl_norm_rope_fwd", ctypes.c_int, ctypes.POINTER(NormRopeDesc), c_void_p,
                  c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p)
_norm_rope_qk = _sig("inl_norm_rope_qk_fwd", ctypes.c_int, ctypes.POINTER(NormRopeDesc), c_i32, c_void_p, c_void_p,
                  c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p)
_rope_table = _sig("inl_rope_table_host", ctypes.c_int, c_i32, ctypes.c_double, c_i32, c_i32,
                   c_void_p, c_void_p)
_positions = _sig("inl_positions_host", ctypes.c_int, c_i32, c_void_p, c_void_p)
_pool_last = _sig("inl_pool_last_fwd", ctypes.c_int, c_i32, c_void_p, c_i32, c_i64, c_i32,
                  c_void_p, c_void_p, ctypes.c_float, c_i32, c_void_p, c_void_p)
_pool_mean = _sig("inl_pool_mean_fwd", ctypes.c_int, c_i32, c_void_p, c_i32, c_i64, c_i32,
                  c_void_p, c_i32, c_void_p, c_void_p)
_l2 = _sig("inl_l2_normalize_fwd", ctypes.c_int, c_i32, c_i32, c_i64, c_void_p, c_i64,
           c_void_p, ctypes.c_float, c_i32, c_void_p)
_splade = _sig("inl_pool_splade_fwd", ctypes.c_int, c_i32, c_void_p, c_i32, c_void_p, c_i64,
               c_void_p, ctypes.c_float, c_void_p, c_i32, c_void_p, c_i32, c_void_p, c_void_p)


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
              "inl_attn_kernel_name",
              "inl_norm_rope_fwd", "inl_norm_rope_qk_fwd", "inl_rope_table_host", "inl_positions_host",
              "inl_pool_last_fwd",
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


def _weight(weights, name, shape, dtype):
    """``weights[name]`` as a contiguous device tensor, after checking its
    dtype and shape: the runners take bare pointers and size every read from
    the configuration, so a tensor of another shape would be read past its
    end."""
    t = weights.get(name)
    if t is None:
        raise InlError(-1, f"weight {name} is missing")
    if t.dtype != dtype:
        raise InlError(-1, f"weight {name}: dtype {t.dtype}, the runner's is {dtype}")
    if tuple(t.shape) != tuple(int(s) for s in shape):
        raise InlError(-1, f"weight {name}: shape {tuple(t.shape)}, the configuration needs {tuple(shape)}")
    if not t.is_cuda:
        raise InlError(-1, f"weight {name}: not a device tensor ({t.device})")
    return t.contiguous()


def _stream_ptr(stream) -> int:
    import torch
    if stream is None:
        stream = torch.cuda.current_stream()
    return int(stream.cuda_stream)


def make_attn_desc(cu_seqlens, h_q, h_kv, head_dim, *, causal, window=-1, scale=None,
                   dtype="bf16", out_dtype=None, q_row_stride=0, k_row_stride=0,
                   v_row_stride=0, o_row_stride=0, flags=0, seq_starts=None):
    """Build an ``AttnDesc``; the cu_seqlens (and seq_starts) arrays are kept
    alive on it. ``seq_starts[b]`` is the first row of text b when texts are
    not packed back to back (a padded batch); None = packed."""
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
    if seq_starts is not None:
        if len(seq_starts) != d.n_texts:
            raise ValueError(f"seq_starts must have {d.n_texts} entries, got {len(seq_starts)}")
        st = _cu_array(seq_starts)
        d.seq_starts_host = st
        d._starts_keepalive = st
    return d


def desc_rows(desc: AttnDesc) -> int:
    """Rows of q, k, v and out that ``desc`` reads or writes: the packed
    total ``cu_seqlens[-1]``, or with ``seq_starts`` the end of the last text."""
    n = desc.n_texts
    if n <= 0:
        return 0
    cu = desc.cu_seqlens_host
    if desc.seq_starts_host:
        st = desc.seq_starts_host
        return max(int(st[b]) + int(cu[b + 1]) - int(cu[b]) for b in range(n))
    return int(cu[n])


def kernel_name(desc: AttnDesc) -> str:
    """The kernel a plan for ``desc`` launches (``inl_attn_kernel_name``)."""
    name = ctypes.c_char_p()
    _check(_kernel_name(ctypes.byref(desc), ctypes.byref(name)))
    return name.value.decode()


def _check_tensors(desc: AttnDesc, q, k, v, out) -> None:
    """Refuse tensors the kernels would read or write past: every tensor must
    hold the rows ``desc`` covers, with its dtype and row strides, and live on a
    GPU. The library sees only pointers, so these checks are the binding's."""
    import torch
    rows = desc_rows(desc)
    want_in = torch.bfloat16 if desc.dtype == INL_BF16 else torch.float32
    want_out = torch.bfloat16 if desc.out_dtype == INL_BF16 else torch.float32
    d = desc.head_dim
    specs = (("q", q, desc.h_q, desc.q_row_stride, want_in), ("k", k, desc.h_kv, desc.k_row_stride, want_in),
             ("v", v, desc.h_kv, desc.v_row_stride, want_in), ("out", out, desc.h_q, desc.o_row_stride, want_out))
    for name, t, heads, stride, dt in specs:
        if t.dtype != dt:
            raise InlError(-1, f"{name}: dtype {t.dtype}, the desc needs {dt}")
        if t.dim() != 3 or t.shape[1] != heads or t.shape[2] != d:
            raise InlError(-1, f"{name}: shape {tuple(t.shape)}, the desc needs [rows, {heads}, {d}]")
        if t.stride(2) != 1 or t.stride(1) != d:
            raise InlError(-1, f"{name}: heads must be contiguous inside a token row")
        if t.shape[0] < rows:
            raise InlError(-1, f"{name}: {t.shape[0]} rows, the desc covers {rows}")
        if rows > 0 and t.stride(0) != (stride if stride else heads * d):
            raise InlError(-1, f"{name}: row stride {t.stride(0)} differs from the desc's")
    for name, t, _, _, _ in specs:
        if not t.is_cuda:
            raise InlError(-1, f"{name}: not a device tensor")


class AttnPlan:
    """A device-resident tile schedule for one packed batch and one attention
    form (``inl_attn_plan_create``); reusable across layers of that form."""

    def __init__(self, desc: AttnDesc):
        self.desc = desc
        h = c_void_p()
        _check(_plan_create(ctypes.byref(desc), ctypes.byref(h)))
        self._h = h
        self.rows = desc_rows(desc)

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
        _check_tensors(self.desc, q, k, v, out)
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
                     stream=None, flags: int = 0, seq_starts=None):
    """Packed attention over torch device tensors ``q [N, Hq, D]``,
    ``k, v [N, Hkv, D]`` (token rows may be strided views of a fused QKV
    buffer). Returns ``out [N, Hq, D]``. Uses the one-shot C entry point
    (``inl_attn_varlen_fwd``) with a workspace from torch's allocator.
    ``seq_starts`` places text b at rows ``[seq_starts[b], seq_starts[b] +
    len_b)`` (a padded batch); rows outside every text are not written."""
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
                          v_row_stride=v.stride(0), o_row_stride=out.stride(0), flags=flags,
                          seq_starts=seq_starts)
    _check_tensors(desc, q, k, v, out)
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
_plan_packed = _sig("inl_plan_packed_batches", ctypes.c_int, c_void_p, c_i64, c_i64, c_i64,
                    c_void_p, ctypes.POINTER(c_i64))


# ---------------------------------------------------------------------------
# Packed batch planner
# ---------------------------------------------------------------------------

def plan_packed_batches(lengths, max_items: int, max_tokens: int):
    """Consecutive batches (``range`` objects over the inputs, in order) of at
    most ``max_items`` inputs and ``max_tokens`` real tokens; the packed
    counterpart of the reference's padded ``plan_batches``
    (crates/inl-sparse/src/native.rs:557-582, crates/inl-text/src/native.rs:
    698-735). An input over ``max_tokens`` forms a batch by itself."""
    import numpy as np
    ln = np.ascontiguousarray(lengths, dtype=np.int32)
    ends = np.empty(max(len(ln), 1), dtype=np.int64)
    nb = c_i64()
    _check(_plan_packed(ln.ctypes.data, len(ln), int(max_items), int(max_tokens), ends.ctypes.data,
                        ctypes.byref(nb)))
    out, start = [], 0
    for e in ends[:nb.value]:
        out.append(range(start, int(e)))
        start = int(e)
    return out


# ---------------------------------------------------------------------------
# Prologue
# ---------------------------------------------------------------------------

def rope_table(rotary_dim: int, theta: float, positions: int, mode: int = 0):
    """(cos, sin) float32 numpy arrays ``[positions, rotary_dim/2]`` built by
    the library exactly as the reference builds them (mode 0: f64 angles;
    mode 1: f32, the Qwen3.5 table)."""
    import numpy as np
    half = rotary_dim // 2
    c = np.empty((positions, half), dtype=np.float32)
    s_ = np.empty((positions, half), dtype=np.float32)
    _check(_rope_table(rotary_dim, float(theta), positions, mode, c.ctypes.data, s_.ctypes.data))
    return c, s_


def positions(cu_seqlens):
    """Text-local positions (int32 numpy) of the packed tokens."""
    import numpy as np
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
    out = np.empty(int(cu[-1]) if len(cu) else 0, dtype=np.int32)
    _check(_positions(len(cu) - 1, cu.ctypes.data, out.ctypes.data))
    return out


def norm_rope(x, rows=None, cos=None, sin=None, *, weight=None, eps=1e-6, norm=True,
              rotary_dim=None, sections=1, cos2=None, sin2=None, out=None, out_dtype=None,
              round_tables=False, round_norm=False, stream=None):
    """Fused per-head RMSNorm + RoPE over ``x [N, heads, head_dim]`` (torch
    device tensor; token rows may be strided). ``rows`` (int32 device [N]) is
    the table row of each token; ``cos``/``sin`` are f32 device tables.
    ``rotary_dim=0`` (or no tables) skips the rope."""
    import torch
    n, heads, hd = x.shape
    od = out_dtype if out_dtype is not None else x.dtype
    if out is None:
        out = torch.empty((n, heads, hd), dtype=od, device=x.device)
    rd = (hd if cos is not None else 0) if rotary_dim is None else rotary_dim
    d = NormRopeDesc()
    d.n_tokens, d.heads, d.head_dim = n, heads, hd
    d.x_row_stride, d.y_row_stride = x.stride(0), out.stride(0)
    d.dtype, d.out_dtype = _dtype_code(x.dtype), _dtype_code(out.dtype)
    d.norm, d.eps = int(bool(norm)), float(eps)
    d.rotary_dim, d.sections = int(rd), int(sections)
    d.table_rows = int(cos.shape[0]) if cos is not None else 0
    d.round_tables, d.round_norm = int(bool(round_tables)), int(bool(round_norm))
    ptr = lambda t: t.data_ptr() if t is not None else None
    _check(_norm_rope(ctypes.byref(d), x.data_ptr(), out.data_ptr(), ptr(weight), ptr(rows),
                      ptr(cos), ptr(sin), ptr(cos2), ptr(sin2), _stream_ptr(stream)))
    return out


def norm_rope_qk(x, q_heads, rows=None, cos=None, sin=None, *, q_weight=None, k_weight=None, eps=1e-6,
                 norm=True, rotary_dim=None, sections=1, cos2=None, sin2=None, out=None, out_dtype=None,
                 round_tables=False, round_norm=False, stream=None):
    """norm_rope over the q heads (``x[:, :q_heads]``, ``q_weight``) and k
    heads (``x[:, q_heads:]``, ``k_weight``) of ``x [N, heads, head_dim]`` in
    one launch (inl_norm_rope_qk_fwd)."""
    import torch
    n, heads, hd = x.shape
    od = out_dtype if out_dtype is not None else x.dtype
    if out is None:
        out = torch.empty((n, heads, hd), dtype=od, device=x.device)
    rd = (hd if cos is not None else 0) if rotary_dim is None else rotary_dim
    d = NormRopeDesc()
    d.n_tokens, d.heads, d.head_dim = n, heads, hd
    d.x_row_stride, d.y_row_stride = x.stride(0), out.stride(0)
    d.dtype, d.out_dtype = _dtype_code(x.dtype), _dtype_code(out.dtype)
    d.norm, d.eps = int(bool(norm)), float(eps)
    d.rotary_dim, d.sections = int(rd), int(sections)
    d.table_rows = int(cos.shape[0]) if cos is not None else 0
    d.round_tables, d.round_norm = int(bool(round_tables)), int(bool(round_norm))
    ptr = lambda t: t.data_ptr() if t is not None else None
    _check(_norm_rope_qk(ctypes.byref(d), int(q_heads), x.data_ptr(), out.data_ptr(), ptr(q_weight),
                         ptr(k_weight), ptr(rows), ptr(cos), ptr(sin), ptr(cos2), ptr(sin2),
                         _stream_ptr(stream)))
    return out


# ---------------------------------------------------------------------------
# Epilogues (``cu`` is an int32 device tensor of packed row offsets)
# ---------------------------------------------------------------------------

def pool_last(hidden, cu, *, weight=None, eps=1e-6, round_norm=False, stream=None):
    import torch
    if weight is not None and weight.dtype != hidden.dtype:
        raise ValueError(f"pool_last: weight dtype {weight.dtype} must match hidden dtype {hidden.dtype}")
    n_texts = cu.numel() - 1
    out = torch.empty((n_texts, hidden.shape[1]), dtype=torch.float32, device=hidden.device)
    _check(_pool_last(n_texts, cu.data_ptr(), hidden.shape[1], hidden.stride(0),
                      _dtype_code(hidden.dtype), hidden.data_ptr(),
                      weight.data_ptr() if weight is not None else None, float(eps),
                      int(bool(round_norm)), out.data_ptr(), _stream_ptr(stream)))
    return out


def pool_mean(hidden, cu, *, normalize=False, stream=None):
    import torch
    n_texts = cu.numel() - 1
    out = torch.empty((n_texts, hidden.shape[1]), dtype=torch.float32, device=hidden.device)
    _check(_pool_mean(n_texts, cu.data_ptr(), hidden.shape[1], hidden.stride(0),
                      _dtype_code(hidden.dtype), hidden.data_ptr(), int(bool(normalize)),
                      out.data_ptr(), _stream_ptr(stream)))
    return out


def l2_normalize(x, dim=None, *, eps_inside=1e-12, skip_zero=False, out=None, stream=None):
    import torch
    rows, width = x.shape
    dim = width if dim is None else dim
    if out is None:
        out = torch.empty((rows, dim), dtype=torch.float32, device=x.device)
    _check(_l2(rows, dim, x.stride(0), x.data_ptr(), out.stride(0), out.data_ptr(),
               float(eps_inside), int(bool(skip_zero)), _stream_ptr(stream)))
    return out


def pool_splade(logits, offs, *, bias=None, shift=0.0, masked_ids=(), canonical=None,
                out_dim=None, stream=None):
    """SPLADE pooling over bias-free f32 logits ``[n_speak, vocab]`` with
    speaking-position offsets ``offs`` (int32 device [rows+1])."""
    import torch
    rows = offs.numel() - 1
    vocab = logits.shape[1]
    if out_dim is None:
        out_dim = vocab if canonical is None else int(canonical.max().item()) + 1
    out = torch.empty((rows, out_dim), dtype=torch.float32, device=logits.device)
    m = (c_i32 * max(1, len(masked_ids)))(*[int(v) for v in masked_ids])
    _check(_splade(rows, offs.data_ptr(), vocab, logits.data_ptr(), logits.stride(0),
                   bias.data_ptr() if bias is not None else None, float(shift), m,
                   len(masked_ids), canonical.data_ptr() if canonical is not None else None,
                   out_dim, out.data_ptr(), _stream_ptr(stream)))
    return out


# ---------------------------------------------------------------------------
# Encoder layer ops and the Qwen3 encoder runner (include/inl_encoder.h)
# ---------------------------------------------------------------------------

_linear_ws = _sig("inl_linear_workspace_size", ctypes.c_int, ctypes.POINTER(ctypes.c_size_t))
_linear_stats = _sig("inl_linear_stats", ctypes.c_int, ctypes.POINTER(c_i64), ctypes.POINTER(c_i64),
                     ctypes.POINTER(c_i64))
_linear = _sig("inl_linear_fwd", ctypes.c_int, c_i64, c_i64, c_i64, c_i32, c_void_p, c_i64, c_void_p, c_i64,
               c_i32, c_void_p, c_i64, ctypes.c_float, ctypes.c_float, c_void_p, ctypes.c_size_t, c_void_p)
_gemm = _sig("inl_gemm_bf16_fwd", ctypes.c_int, c_i64, c_i64, c_i64, c_void_p, c_i64, c_void_p, c_i64, c_i32,
             c_void_p, c_i64, ctypes.c_float, ctypes.c_float, c_void_p)
_gemm_gated = _sig("inl_gemm_bf16_gated_fwd", ctypes.c_int, c_i64, c_i64, c_i64, c_void_p, c_i64, c_void_p, c_i64,
                   c_i32, c_void_p, c_i64, c_i32, c_void_p, c_i64, c_void_p)
INL_GATE_GEGLU, INL_GATE_GELU_MUL = 1, 2
_embed = _sig("inl_embed_fwd", ctypes.c_int, c_i64, c_void_p, c_void_p, c_i64, c_i32, c_i32, c_void_p, c_i64,
              c_void_p)
_rms_rows = _sig("inl_rms_norm_rows_fwd", ctypes.c_int, c_i64, c_i32, c_void_p, c_i64, c_void_p, c_i32,
                 ctypes.c_float, c_i32, c_void_p, c_i64, c_void_p)
_swiglu = _sig("inl_swiglu_fwd", ctypes.c_int, c_i64, c_i32, c_i32, c_void_p, c_i64, c_void_p, c_i64, c_void_p)


class Qwen3Config(ctypes.Structure):
    _fields_ = [("vocab", c_i32), ("hidden", c_i32), ("intermediate", c_i32), ("layers", c_i32),
                ("heads", c_i32), ("kv_heads", c_i32), ("head_dim", c_i32), ("eps", ctypes.c_float),
                ("rope_theta", ctypes.c_double), ("max_positions", c_i32), ("dtype", c_i32),
                ("attn_flags", c_i32)]


class Qwen3LayerWeights(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in ("qkv_proj", "o_proj", "gate_up_proj", "down_proj", "q_norm", "k_norm",
                                        "input_norm", "post_attention_norm")]


_q3_create = _sig("inl_qwen3_create", ctypes.c_int, ctypes.POINTER(Qwen3Config), c_void_p,
                  ctypes.POINTER(Qwen3LayerWeights), c_void_p, ctypes.POINTER(c_void_p))
_q3_destroy = _sig("inl_qwen3_destroy", ctypes.c_int, c_void_p)
_q3_ws = _sig("inl_qwen3_workspace_size", ctypes.c_int, c_void_p, c_i32, c_void_p, ctypes.POINTER(ctypes.c_size_t))
_q3_graphs = _sig("inl_qwen3_set_graphs", ctypes.c_int, c_void_p, c_i32)
_q3_ginfo = _sig("inl_qwen3_graph_info", ctypes.c_int, c_void_p, ctypes.POINTER(c_i32), ctypes.POINTER(c_i32))
_q3_encode = _sig("inl_qwen3_encode", ctypes.c_int, c_void_p, c_i32, c_void_p, c_void_p, c_void_p, c_void_p,
                  ctypes.c_size_t, c_void_p)

_LINEAR_WS = {}


def _linear_workspace(dev):
    import torch
    key = str(dev)
    if key not in _LINEAR_WS:
        n = ctypes.c_size_t()
        _check(_linear_ws(ctypes.byref(n)))
        _LINEAR_WS[key] = torch.empty(n.value, dtype=torch.uint8, device=dev)
    return _LINEAR_WS[key]


def linear(x, w, *, out=None, out_dtype=None, alpha=1.0, beta=0.0, stream=None):
    """``out = alpha * x @ w.T + beta * out`` on hipBLASLt (``inl_linear_fwd``):
    ``x [m, k]``, ``w [n, k]`` row-major, rows may be strided."""
    import torch
    m, k = x.shape
    n = w.shape[0]
    if w.shape[1] != k or x.dtype != w.dtype:
        raise InlError(-1, "linear: x [m, k] and w [n, k] must agree in k and dtype")
    if x.stride(1) != 1 or w.stride(1) != 1:
        raise InlError(-1, "linear: rows must be contiguous")
    od = out_dtype if out_dtype is not None else (out.dtype if out is not None else x.dtype)
    if out is None:
        out = torch.empty((m, n), dtype=od, device=x.device)
    if out.shape != (m, n) or out.stride(1) != 1:
        raise InlError(-1, f"linear: out must be [{m}, {n}] with contiguous rows")
    ws = _linear_workspace(x.device)
    _check(_linear(m, n, k, _dtype_code(x.dtype), x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0),
                   _dtype_code(out.dtype), out.data_ptr(), out.stride(0), float(alpha), float(beta),
                   ws.data_ptr(), ws.numel(), _stream_ptr(stream)))
    return out


def gemm_bf16(x, w, *, out=None, out_dtype=None, alpha=1.0, beta=0.0, stream=None):
    """``out = alpha * x @ w.T + beta * out`` on the library's own bf16 MFMA
    kernel (``inl_gemm_bf16_fwd``): bf16 ``x [m, k]`` and ``w [n, k]``, rows
    may be strided; ``out`` f32 or bf16."""
    import torch
    m, k = x.shape
    n = w.shape[0]
    if w.shape[1] != k or x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise InlError(-1, "gemm_bf16: x [m, k] and w [n, k] must be bf16 and agree in k")
    if x.stride(1) != 1 or w.stride(1) != 1:
        raise InlError(-1, "gemm_bf16: rows must be contiguous")
    od = out_dtype if out_dtype is not None else (out.dtype if out is not None else torch.bfloat16)
    if out is None:
        out = torch.empty((m, n), dtype=od, device=x.device)
    if out.shape != (m, n) or out.stride(1) != 1:
        raise InlError(-1, f"gemm_bf16: out must be [{m}, {n}] with contiguous rows")
    _check(_gemm(m, n, k, x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), _dtype_code(out.dtype),
                 out.data_ptr(), out.stride(0), float(alpha), float(beta), _stream_ptr(stream)))
    return out


def gemm_bf16_gated(x, w, mode, *, mul=None, out=None, out_dtype=None, stream=None):
    """``inl_gemm_bf16_gated_fwd``: ``mode="geglu"``: ``w [2n, k]`` (gate rows
    then up rows), ``out = gelu_tanh(x @ w[:n].T) * (x @ w[n:].T)``;
    ``mode="gelu_mul"``: ``out = gelu_tanh(x @ w.T) * mul`` (bf16 ``[m, n]``)."""
    import torch
    m, k = x.shape
    if mode == "geglu":
        code, n = INL_GATE_GEGLU, w.shape[0] // 2
        if w.shape[0] % 2:
            raise InlError(-1, "gemm_bf16_gated: geglu needs an even number of w rows")
    elif mode == "gelu_mul":
        code, n = INL_GATE_GELU_MUL, w.shape[0]
        if mul is None or mul.shape != (m, n) or mul.dtype != torch.bfloat16 or mul.stride(1) != 1:
            raise InlError(-1, f"gemm_bf16_gated: gelu_mul needs a bf16 mul [{m}, {n}] with contiguous rows")
    else:
        raise InlError(-1, f"gemm_bf16_gated: unknown mode {mode!r}")
    if w.shape[1] != k or x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise InlError(-1, "gemm_bf16_gated: x and w must be bf16 and agree in k")
    if x.stride(1) != 1 or w.stride(1) != 1:
        raise InlError(-1, "gemm_bf16_gated: rows must be contiguous")
    od = out_dtype if out_dtype is not None else (out.dtype if out is not None else torch.bfloat16)
    if out is None:
        out = torch.empty((m, n), dtype=od, device=x.device)
    if out.shape != (m, n) or out.stride(1) != 1:
        raise InlError(-1, f"gemm_bf16_gated: out must be [{m}, {n}] with contiguous rows")
    _check(_gemm_gated(m, n, k, x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), code,
                       mul.data_ptr() if mul is not None else None, mul.stride(0) if mul is not None else 0,
                       _dtype_code(out.dtype), out.data_ptr(), out.stride(0), _stream_ptr(stream)))
    return out


def linear_stats():
    """``inl_linear_stats``: dict of hipBLASLt timing passes run so far, (shape,
    row-count bucket) choices held and exact-row-count entries cached."""
    t, b, c = c_i64(), c_i64(), c_i64()
    _check(_linear_stats(ctypes.byref(t), ctypes.byref(b), ctypes.byref(c)))
    return {"tunings": t.value, "buckets": b.value, "cached_shapes": c.value}


def embed(ids, table, *, stream=None):
    """``table[ids]`` as f32 rows (``inl_embed_fwd``); ids int32 on the device."""
    import torch
    out = torch.empty((ids.numel(), table.shape[1]), dtype=torch.float32, device=table.device)
    _check(_embed(ids.numel(), ids.data_ptr(), table.data_ptr(), table.shape[0], table.shape[1],
                  _dtype_code(table.dtype), out.data_ptr(), out.stride(0), _stream_ptr(stream)))
    return out


def rms_norm_rows(x, weight=None, *, eps=1e-6, out_dtype=None, stream=None):
    """RMSNorm of f32 rows into ``out_dtype`` (``inl_rms_norm_rows_fwd``)."""
    import torch
    rows, dim = x.shape
    od = out_dtype if out_dtype is not None else torch.float32
    out = torch.empty((rows, dim), dtype=od, device=x.device)
    wdt = _dtype_code(weight.dtype) if weight is not None else INL_F32
    _check(_rms_rows(rows, dim, x.data_ptr(), x.stride(0), weight.data_ptr() if weight is not None else None,
                     wdt, float(eps), _dtype_code(od), out.data_ptr(), out.stride(0), _stream_ptr(stream)))
    return out


def swiglu(gate_up, intermediate, *, stream=None):
    """``silu(gate_up[:, :I]) * gate_up[:, I:2I]`` (``inl_swiglu_fwd``)."""
    import torch
    rows = gate_up.shape[0]
    out = torch.empty((rows, intermediate), dtype=gate_up.dtype, device=gate_up.device)
    _check(_swiglu(rows, intermediate, _dtype_code(gate_up.dtype), gate_up.data_ptr(), gate_up.stride(0),
                   out.data_ptr(), out.stride(0), _stream_ptr(stream)))
    return out


class Qwen3Encoder:
    """The GPU Qwen3 embedder (``inl_qwen3_*``): packed texts in, unit-length
    last-token embeddings out. ``weights`` maps the checkpoint's tensor names
    (``embed_tokens.weight``, ``layers.{i}.self_attn.q_proj.weight``, ...,
    ``norm.weight``) to device tensors of one dtype; the q/k/v and gate/up
    projections are stacked once here (the runner takes them fused)."""

    def __init__(self, cfg, weights, *, max_positions=4096, attn_flags=0):
        import torch
        t0 = weights["embed_tokens.weight"]
        self.dtype = t0.dtype
        self.cfg = cfg
        c = Qwen3Config()
        c.vocab, c.hidden, c.intermediate, c.layers = cfg.vocab, cfg.hidden, cfg.intermediate, cfg.layers
        c.heads, c.kv_heads, c.head_dim = cfg.heads, cfg.kv_heads, cfg.head_dim
        c.eps, c.rope_theta, c.max_positions = cfg.eps, cfg.theta, max_positions
        c.dtype, c.attn_flags = _dtype_code(self.dtype), attn_flags
        dt, hs, ff = self.dtype, cfg.hidden, cfg.intermediate
        qd, kvd = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
        t0 = _weight(weights, "embed_tokens.weight", (cfg.vocab, hs), dt)
        self._keep = [t0, _weight(weights, "norm.weight", (hs,), dt)]
        layers = (Qwen3LayerWeights * cfg.layers)()
        for i in range(cfg.layers):
            p = f"layers.{i}."
            W = lambda n, *shape: _weight(weights, p + n, shape, dt)
            qkv = torch.cat([W("self_attn.q_proj.weight", qd, hs), W("self_attn.k_proj.weight", kvd, hs),
                             W("self_attn.v_proj.weight", kvd, hs)], 0).contiguous()
            gu = torch.cat([W("mlp.gate_proj.weight", ff, hs), W("mlp.up_proj.weight", ff, hs)], 0).contiguous()
            parts = [qkv, W("self_attn.o_proj.weight", hs, qd), gu, W("mlp.down_proj.weight", hs, ff),
                     W("self_attn.q_norm.weight", cfg.head_dim), W("self_attn.k_norm.weight", cfg.head_dim),
                     W("input_layernorm.weight", hs), W("post_attention_layernorm.weight", hs)]
            self._keep += parts
            for name, t in zip([f[0] for f in Qwen3LayerWeights._fields_], parts):
                setattr(layers[i], name, t.data_ptr())
        h = c_void_p()
        _check(_q3_create(ctypes.byref(c), t0.data_ptr(), layers, self._keep[1].data_ptr(), ctypes.byref(h)))
        self._h = h

    def workspace_bytes(self, cu_seqlens) -> int:
        cu = _cu_array(cu_seqlens)
        n = ctypes.c_size_t()
        _check(_q3_ws(self._h, len(cu_seqlens) - 1, cu, ctypes.byref(n)))
        return n.value

    def set_graphs(self, enable: bool) -> None:
        """``inl_qwen3_set_graphs``: keep (True, the default) or stop keeping
        the launch sequence of a batch shape as a HIP graph."""
        _check(_q3_graphs(self._h, 1 if enable else 0))

    def graph_info(self):
        """(graphs enabled, a graph of the last batch shape is held)."""
        en, held = c_i32(), c_i32()
        _check(_q3_ginfo(self._h, ctypes.byref(en), ctypes.byref(held)))
        return bool(en.value), bool(held.value)

    def encode(self, ids, cu_seqlens, *, out=None, workspace=None, stream=None):
        """``ids``: host int sequence of the packed token ids; returns f32
        ``[texts, hidden]`` unit vectors on the device."""
        import numpy as np
        import torch
        cu = _cu_array(cu_seqlens)
        nt = len(cu_seqlens) - 1
        idv = np.ascontiguousarray(ids, dtype=np.int32)
        if len(idv) != int(cu_seqlens[-1]):
            raise InlError(-1, f"encode: {len(idv)} ids for {int(cu_seqlens[-1])} tokens")
        dev = self._keep[0].device
        if out is None:
            out = torch.empty((nt, self.cfg.hidden), dtype=torch.float32, device=dev)
        need = self.workspace_bytes(cu_seqlens)
        if workspace is None:   # reuse the last one: same addresses let a batch shape keep its graph
            workspace = getattr(self, "_last_ws", None)
        if workspace is None or workspace.numel() < need + 256:
            workspace = torch.empty(need + 256, dtype=torch.uint8, device=dev)
        ptr = workspace.data_ptr()
        ptr += (-ptr) % 256
        _check(_q3_encode(self._h, nt, cu, idv.ctypes.data, out.data_ptr(), ptr, need, _stream_ptr(stream)))
        self._last_ws = workspace
        return out

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            _check(_q3_destroy(self._h))
            self._h = c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Gemma2Config(ctypes.Structure):
    _fields_ = [("vocab", c_i32), ("hidden", c_i32), ("intermediate", c_i32), ("layers", c_i32),
                ("heads", c_i32), ("kv_heads", c_i32), ("head_dim", c_i32), ("ple_dim", c_i32),
                ("embedding_dim", c_i32), ("sliding_window", c_i32), ("eps", ctypes.c_float),
                ("theta_sliding", ctypes.c_double), ("theta_full", ctypes.c_double), ("max_positions", c_i32),
                ("dtype", c_i32), ("attn_flags", c_i32)]


_G2_WEIGHTS = ("qkv_proj", "o_proj", "gate_up_proj", "down_proj", "q_norm", "k_norm", "input_norm",
               "post_attention_norm", "pre_feedforward_norm", "post_feedforward_norm", "ple_input_gate",
               "ple_projection", "ple_post_norm", "layer_scalar")


class Gemma2LayerWeights(ctypes.Structure):
    _fields_ = [("full", c_i32), ("head_dim", c_i32), ("kv_heads", c_i32)] + [(n, c_void_p) for n in _G2_WEIGHTS]


_g2_create = _sig("inl_gemma2_create", ctypes.c_int, ctypes.POINTER(Gemma2Config), c_void_p,
                  ctypes.POINTER(Gemma2LayerWeights), c_void_p, c_void_p, c_void_p, c_void_p, ctypes.POINTER(c_void_p))
_g2_destroy = _sig("inl_gemma2_destroy", ctypes.c_int, c_void_p)
_g2_ws = _sig("inl_gemma2_workspace_size", ctypes.c_int, c_void_p, c_i32, c_void_p, ctypes.POINTER(ctypes.c_size_t))
_g2_encode = _sig("inl_gemma2_encode", ctypes.c_int, c_void_p, c_i32, c_void_p, c_void_p, c_i32, c_void_p, c_void_p,
                  ctypes.c_size_t, c_void_p)


class Gemma2Encoder:
    """The GPU EmbeddingGemma 2 text tower (``inl_gemma2_*``): packed texts
    in, unit-length mean-pooled embeddings out. ``text_config`` is the
    checkpoint's ``text_config`` dict (``layer_types``, ``per_layer_config``,
    ``rope_parameters``, ...); ``weights`` maps the text model's tensor names
    (``embed_tokens.weight``, ``layers.{i}.self_attn.q_proj.weight``, ...,
    ``ple.per_layer_model_projection.weight``, ``embedding_projection.weight``)
    to device tensors of one dtype. q/k/v and gate/up are stacked once here."""

    def __init__(self, text_config, weights, *, max_positions=None, attn_flags=0):
        import torch
        tc = text_config
        t0 = weights["embed_tokens.weight"]
        self.dtype = t0.dtype
        self.embedding_dim = int(tc["embedding_dim"])
        c = Gemma2Config()
        c.vocab, c.hidden, c.intermediate = tc["vocab_size"], tc["hidden_size"], tc["intermediate_size"]
        c.layers, c.heads, c.kv_heads = tc["num_hidden_layers"], tc["num_attention_heads"], tc["num_key_value_heads"]
        c.head_dim, c.ple_dim, c.embedding_dim = tc["head_dim"], tc["hidden_size_per_layer_input"], tc["embedding_dim"]
        c.sliding_window, c.eps = tc["sliding_window"], tc["rms_norm_eps"]
        c.theta_sliding = tc["rope_parameters"]["sliding_attention"]["rope_theta"]
        c.theta_full = tc["rope_parameters"]["full_attention"]["rope_theta"]
        c.max_positions = max_positions or tc.get("max_position_embeddings", 8192)
        c.dtype, c.attn_flags = _dtype_code(self.dtype), attn_flags
        dt, hs, ff, ple = self.dtype, c.hidden, c.intermediate, c.ple_dim
        t0 = _weight(weights, "embed_tokens.weight", (c.vocab, hs), dt)
        self._keep = [t0, _weight(weights, "ple.per_layer_model_projection.weight", (c.layers * ple, hs), dt),
                      _weight(weights, "ple.per_layer_projection_norm.weight", (ple,), dt),
                      _weight(weights, "norm.weight", (hs,), dt),
                      _weight(weights, "embedding_projection.weight", (c.embedding_dim, hs), dt)]
        over = tc.get("per_layer_config", {})
        layers = (Gemma2LayerWeights * c.layers)()
        for i in range(c.layers):
            p = f"layers.{i}."
            W = lambda n, *shape: _weight(weights, p + n, shape, dt)
            o = over.get(f"{i:02d}", {})
            layers[i].full = 1 if tc["layer_types"][i] == "full_attention" else 0
            layers[i].head_dim = o.get("head_dim", 0)
            layers[i].kv_heads = o.get("num_key_value_heads", 0)
            hd = layers[i].head_dim or c.head_dim
            qd, kvd = c.heads * hd, (layers[i].kv_heads or c.kv_heads) * hd
            qkv = torch.cat([W("self_attn.q_proj.weight", qd, hs), W("self_attn.k_proj.weight", kvd, hs),
                             W("self_attn.v_proj.weight", kvd, hs)], 0).contiguous()
            gu = torch.cat([W("mlp.gate_proj.weight", ff, hs), W("mlp.up_proj.weight", ff, hs)], 0).contiguous()
            parts = [qkv, W("self_attn.o_proj.weight", hs, qd), gu, W("mlp.down_proj.weight", hs, ff),
                     W("self_attn.q_norm.weight", hd), W("self_attn.k_norm.weight", hd),
                     W("input_layernorm.weight", hs), W("post_attention_layernorm.weight", hs),
                     W("pre_feedforward_layernorm.weight", hs), W("post_feedforward_layernorm.weight", hs),
                     W("ple_block.per_layer_input_gate.weight", ple, hs),
                     W("ple_block.per_layer_projection.weight", hs, ple),
                     W("ple_block.post_per_layer_input_norm.weight", hs), W("layer_scalar", 1)]
            self._keep += parts
            for name, t in zip(_G2_WEIGHTS, parts):
                setattr(layers[i], name, t.data_ptr())
        h = c_void_p()
        _check(_g2_create(ctypes.byref(c), t0.data_ptr(), layers, *[t.data_ptr() for t in self._keep[1:5]],
                          ctypes.byref(h)))
        self._h = h

    def workspace_bytes(self, cu_seqlens) -> int:
        cu = _cu_array(cu_seqlens)
        n = ctypes.c_size_t()
        _check(_g2_ws(self._h, len(cu_seqlens) - 1, cu, ctypes.byref(n)))
        return n.value

    def encode(self, ids, cu_seqlens, *, out_dim=None, out=None, workspace=None, stream=None):
        """``ids``: host int sequence of the packed token ids; returns f32
        ``[texts, out_dim]`` unit vectors on the device (``out_dim`` below
        ``embedding_dim``: Matryoshka truncation, renormalised)."""
        import numpy as np
        import torch
        cu = _cu_array(cu_seqlens)
        nt = len(cu_seqlens) - 1
        od = int(out_dim or self.embedding_dim)
        idv = np.ascontiguousarray(ids, dtype=np.int32)
        if len(idv) != int(cu_seqlens[-1]):
            raise InlError(-1, f"encode: {len(idv)} ids for {int(cu_seqlens[-1])} tokens")
        dev = self._keep[0].device
        if out is None:
            out = torch.empty((nt, od), dtype=torch.float32, device=dev)
        need = self.workspace_bytes(cu_seqlens)
        if workspace is None:
            workspace = getattr(self, "_last_ws", None)
        if workspace is None or workspace.numel() < need + 256:
            workspace = torch.empty(need + 256, dtype=torch.uint8, device=dev)
        ptr = workspace.data_ptr()
        ptr += (-ptr) % 256
        _check(_g2_encode(self._h, nt, cu, idv.ctypes.data, od, out.data_ptr(), ptr, need, _stream_ptr(stream)))
        self._last_ws = workspace
        return out

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            _check(_g2_destroy(self._h))
            self._h = c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_sd_ws = _sig("inl_splade_decoder_workspace_size", ctypes.c_int, c_i32, c_i32, ctypes.POINTER(ctypes.c_size_t))
_sd_max = _sig("inl_splade_decoder_max_fwd", ctypes.c_int, c_i32, c_void_p, c_void_p, c_i64, c_i32, c_void_p, c_i64,
               c_i32, c_i32, c_void_p, c_void_p, ctypes.c_size_t, c_void_p)
_sp_finish = _sig("inl_splade_finish_fwd", ctypes.c_int, c_i32, c_i32, c_void_p, c_i64, c_void_p, ctypes.c_float,
                  c_void_p, c_i32, c_void_p, c_i32, c_void_p, c_void_p)


def splade_decoder_max(head, w_dec, offs, *, out=None, stream=None):
    """Per-text maxima over speaking positions of ``head @ w_dec.T`` without
    materialising the logits (``inl_splade_decoder_max_fwd``): ``head [S, H]``
    and ``w_dec [V, H]`` bf16 device tensors, ``offs`` a host sequence of
    ``rows + 1`` position offsets. Returns f32 ``[rows, V]``."""
    import numpy as np
    import torch
    rows = len(offs) - 1
    S, H = head.shape
    V = w_dec.shape[0]
    if w_dec.shape[1] != H or head.dtype != w_dec.dtype:
        raise InlError(-1, "splade_decoder_max: head [S, H] and w_dec [V, H] must agree in H and dtype")
    if int(offs[-1]) > S:
        raise InlError(-1, f"splade_decoder_max: offsets cover {int(offs[-1])} positions, head has {S}")
    if head.stride(1) != 1 or w_dec.stride(1) != 1:
        raise InlError(-1, "splade_decoder_max: rows must be contiguous")
    if out is None:
        out = torch.empty((rows, V), dtype=torch.float32, device=head.device)
    ofs = np.ascontiguousarray(offs, dtype=np.int32)
    n = ctypes.c_size_t()
    _check(_sd_ws(rows, V, ctypes.byref(n)))
    ws = torch.empty(n.value, dtype=torch.uint8, device=head.device)
    _check(_sd_max(rows, ofs.ctypes.data, head.data_ptr(), head.stride(0), H, w_dec.data_ptr(), w_dec.stride(0),
                   V, _dtype_code(head.dtype), out.data_ptr(), ws.data_ptr(), n.value, _stream_ptr(stream)))
    out._inl_workspace = ws
    return out


def splade_finish(maxima, *, bias=None, shift=0.0, masked_ids=(), canonical=None, out_dim=None, stream=None):
    """``inl_splade_finish_fwd``: finish and fold per-row maxima [rows, V]."""
    import torch
    rows, vocab = maxima.shape
    if out_dim is None:
        out_dim = vocab if canonical is None else int(canonical.max().item()) + 1
    out = torch.empty((rows, out_dim), dtype=torch.float32, device=maxima.device)
    m = (c_i32 * max(1, len(masked_ids)))(*[int(v) for v in masked_ids])
    _check(_sp_finish(rows, vocab, maxima.data_ptr(), maxima.stride(0),
                      bias.data_ptr() if bias is not None else None, float(shift), m, len(masked_ids),
                      canonical.data_ptr() if canonical is not None else None, out_dim, out.data_ptr(),
                      _stream_ptr(stream)))
    return out


# ---------------------------------------------------------------------------
# Gated-delta-net ops (include/inl_gdn.h)
# ---------------------------------------------------------------------------

_gdn_conv = _sig("inl_gdn_conv_fwd", ctypes.c_int, c_i64, c_i32, c_void_p, c_i32, c_i32, c_i32, c_void_p, c_i64,
                 c_void_p, c_void_p, c_i64, c_void_p)
_gdn_gates = _sig("inl_gdn_gates_fwd", ctypes.c_int, c_i64, c_i32, c_i32, c_void_p, c_i64, c_void_p, c_i64,
                  c_void_p, c_void_p, c_void_p, c_void_p, c_void_p)
_gdn_rule = _sig("inl_gdn_rule_fwd", ctypes.c_int, c_i64, c_i32, c_void_p, c_i32, c_i32, c_i32, c_i32, c_i32,
                 c_void_p, c_i64, c_void_p, c_void_p, c_i64, c_void_p, c_i64, c_void_p)
_gdn_norm = _sig("inl_gdn_gated_norm_fwd", ctypes.c_int, c_i64, c_i32, c_i32, c_i32, c_i32, c_void_p, c_i64,
                 c_void_p, c_i64, c_void_p, ctypes.c_float, c_void_p, c_i64, c_void_p)
_gdn_inverse = _sig("inl_gdn_unit_lower_inverse_fwd", ctypes.c_int, c_i64, c_i32, c_void_p, c_void_p, c_void_p)


def _cu_device(cu, device):
    import torch
    if isinstance(cu, torch.Tensor):
        if cu.dtype != torch.int32 or not cu.is_cuda or cu.dim() != 1 or not cu.is_contiguous():
            raise InlError(-1, "cu_seqlens must be a contiguous int32 device vector")
        return cu
    return torch.tensor([int(c) for c in cu], dtype=torch.int32, device=device)


def _rows2d(x, name):
    if x.dim() != 2 or x.stride(1) != 1 or not x.is_cuda:
        raise InlError(-1, f"{name} must be a 2-D device tensor with unit column stride")


def gdn_conv(x, cu_seqlens, weight, *, stream=None):
    """``inl_gdn_conv_fwd``: silu(causal depthwise conv) per packed text; x
    [N, C], weight [C, taps] (same dtype) -> [N, C]."""
    import torch
    _rows2d(x, "x")
    cu = _cu_device(cu_seqlens, x.device)
    n, ch = x.shape
    weight = weight.contiguous()
    if weight.dtype != x.dtype or weight.dim() != 2 or weight.shape[0] != ch:
        raise InlError(-1, "weight must be [channels, taps] in x's dtype")
    out = torch.empty_like(x, memory_format=torch.contiguous_format)
    _check(_gdn_conv(n, cu.numel() - 1, cu.data_ptr(), ch, weight.shape[1], _dtype_code(x.dtype), x.data_ptr(),
                     x.stride(0), weight.data_ptr(), out.data_ptr(), out.stride(0), _stream_ptr(stream)))
    return out


def gdn_gates(a, b, dt_bias, neg_a, *, stream=None):
    """``inl_gdn_gates_fwd``: (g, beta), f32 [N, nv], from the a/b projections."""
    import torch
    _rows2d(a, "a")
    _rows2d(b, "b")
    n, nv = a.shape
    if b.shape != a.shape or b.dtype != a.dtype:
        raise InlError(-1, "a and b must share shape and dtype")
    dt_bias = dt_bias.float().contiguous()
    neg_a = neg_a.float().contiguous()
    g = torch.empty((n, nv), dtype=torch.float32, device=a.device)
    beta = torch.empty_like(g)
    _check(_gdn_gates(n, nv, _dtype_code(a.dtype), a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0),
                      dt_bias.data_ptr(), neg_a.data_ptr(), g.data_ptr(), beta.data_ptr(), _stream_ptr(stream)))
    return g, beta


def gdn_rule(mixed, cu_seqlens, key_heads, value_heads, key_dim, value_dim, g, beta, *, stream=None):
    """``inl_gdn_rule_fwd``: the gated delta rule over packed texts; mixed
    [N, 2 nk dk + nv dv] (model dtype), g/beta f32 [N, nv] -> f32 [N, nv, dv]."""
    import torch
    _rows2d(mixed, "mixed")
    _rows2d(g, "g")
    if beta.stride() != g.stride() or beta.shape != g.shape or g.dtype != torch.float32 or beta.dtype != torch.float32:
        raise InlError(-1, "g and beta must be f32 tensors of one shape and stride")
    cu = _cu_device(cu_seqlens, mixed.device)
    n = mixed.shape[0]
    if mixed.shape[1] != 2 * key_heads * key_dim + value_heads * value_dim or g.shape != (n, value_heads):
        raise InlError(-1, "mixed must be [N, 2 nk dk + nv dv] and g [N, nv]")
    out = torch.empty((n, value_heads, value_dim), dtype=torch.float32, device=mixed.device)
    _check(_gdn_rule(n, cu.numel() - 1, cu.data_ptr(), key_heads, value_heads, key_dim, value_dim,
                     _dtype_code(mixed.dtype), mixed.data_ptr(), mixed.stride(0), g.data_ptr(), beta.data_ptr(),
                     g.stride(0), out.data_ptr(), out.stride(0), _stream_ptr(stream)))
    return out


def gdn_gated_norm(core, z, weight, eps, *, stream=None):
    """``inl_gdn_gated_norm_fwd``: core [N, heads, dv] (f32 or z's dtype), z
    [N, heads, dv], weight [dv] (z's dtype) -> [N, heads, dv] in z's dtype."""
    import torch
    if core.dim() != 3 or z.shape != core.shape or not core.is_contiguous() or not z.is_contiguous():
        raise InlError(-1, "core and z must be contiguous [N, heads, dv] tensors")
    n, heads, dv = core.shape
    weight = weight.contiguous()
    if weight.dtype != z.dtype or weight.numel() != dv:
        raise InlError(-1, "weight must be [dv] in z's dtype")
    out = torch.empty_like(z)
    _check(_gdn_norm(n, heads, dv, _dtype_code(z.dtype), _dtype_code(core.dtype), core.data_ptr(), core.stride(0),
                     z.data_ptr(), z.stride(0), weight.data_ptr(), float(eps), out.data_ptr(), out.stride(0),
                     _stream_ptr(stream)))
    return out


def unit_lower_inverse(a, *, stream=None):
    """``inl_gdn_unit_lower_inverse_fwd``: (I + A)^-1 of f32 [n, S, S]
    strictly lower-triangular matrices."""
    import torch
    if a.dim() != 3 or a.shape[1] != a.shape[2] or a.dtype != torch.float32 or not a.is_cuda:
        raise InlError(-1, "a must be an f32 device tensor [n, S, S]")
    a = a.contiguous()
    out = torch.empty_like(a)
    _check(_gdn_inverse(a.shape[0], a.shape[1], a.data_ptr(), out.data_ptr(), _stream_ptr(stream)))
    return out
