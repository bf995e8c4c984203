"""The C++ interface above the C ABI (include/inl_attention.hpp), driven
through the ctypes shim tests/cpp/attend_check.cpp.

It mirrors crates/inl-core/src/attention.rs:40-234: AttentionBackend::resolve
and its error text (:73-112), score_rows (:114-123), BatchMask (:126-160) and
attend (:215-234). CPU tests cover resolution and argument checks (which
raise before any GPU call); GPU tests compare attend on padded batches with
the oracle's forms of the reference masks, calling it twice so the second call
reuses the mask's plan. Tolerance: 2e-3 max-abs for bf16 inputs (f32 output).
"""
import ctypes
from pathlib import Path

import numpy as np
import pytest

from oracle import attention as oa

SHIM = Path(__file__).resolve().parent / "cpp" / "libattend_check.so"
AUTO, FUSED, TILED, EAGER = range(4)
CPU, HIP = range(2)
F32, BF16 = 0, 1


@pytest.fixture(scope="module")
def shim(inl):
    if not SHIM.exists():
        pytest.fail(f"{SHIM} is not built: run im-not-llm_amd/build.py")
    lib = ctypes.CDLL(str(SHIM))
    lib.inl_test_resolve.argtypes = [ctypes.c_int] * 4 + [ctypes.c_int64, ctypes.POINTER(ctypes.c_int64),
                                                          ctypes.c_char_p, ctypes.c_int]
    lib.inl_test_attend.argtypes = ([ctypes.c_int, ctypes.c_void_p] + [ctypes.c_int] * 9 + [ctypes.c_float]
                                    + [ctypes.c_void_p] * 5 + [ctypes.c_int, ctypes.c_char_p, ctypes.c_int])
    return lib


def _resolve(shim, request, device, dtype, head_dim, padded=128):
    rows = ctypes.c_int64(-1)
    msg = ctypes.create_string_buffer(512)
    rc = shim.inl_test_resolve(request, device, dtype, head_dim, padded, ctypes.byref(rows), msg, 512)
    return rc, rows.value, msg.value.decode()


def _attend(shim, form, pl, b, t, causal, window, hq, hkv, d, dtype, out_dtype, scale, q=0, k=0, v=0, out=0,
            repeat=1):
    arr = (ctypes.c_int32 * max(len(pl), 1))(*pl)
    msg = ctypes.create_string_buffer(512)
    rc = shim.inl_test_attend(form, ctypes.cast(arr, ctypes.c_void_p), b, t, causal, window, hq, hkv, d, dtype,
                              out_dtype, scale, q, k, v, out, None, repeat, msg, 512)
    return rc, msg.value.decode()


def test_resolve_mirrors_the_reference(shim):
    # auto / fused on the HIP device: the fused kernels, no score rows (:114-123)
    for req in (AUTO, FUSED):
        for dt, hd in ((BF16, 128), (F32, 64), (BF16, 256), (BF16, 16)):
            rc, rows, _ = _resolve(shim, req, HIP, dt, hd, padded=2048)
            assert rc == 0 and rows == 0
    # the reference's message for an unavailable fused backend (:84-86)
    rc, _, msg = _resolve(shim, FUSED, HIP, BF16, 512)
    assert rc != 0 and msg.startswith('attention = "fused" is unavailable: ') and "head_dim 512" in msg
    rc, _, msg = _resolve(shim, FUSED, CPU, F32, 128)
    assert rc != 0 and 'attention = "fused" is unavailable' in msg
    rc, _, msg = _resolve(shim, FUSED, HIP, 7, 128)
    assert rc != 0 and "dtype" in msg
    # no eager or tiled path in this library: an error, never a silent fallback
    for req, name in ((EAGER, "eager"), (TILED, "tiled")):
        rc, _, msg = _resolve(shim, req, HIP, BF16, 128)
        assert rc != 0 and f'attention = "{name}"' in msg


def test_mask_and_shape_errors_raise_before_any_launch(shim, inl):
    # pad length outside [0, T] (BatchMask::new takes left pads < T)
    rc, msg = _attend(shim, 0, [0, 9], 2, 8, 1, -1, 16, 8, 128, BF16, F32, 0.1)
    assert rc == -1 and "pad length 9" in msg
    rc, msg = _attend(shim, 1, [3, -1], 2, 8, 0, 4, 3, 1, 256, BF16, F32, 1.0)
    assert rc == -1 and "length -1" in msg
    rc, msg = _attend(shim, 1, [3, 3], 2, 8, 0, -2, 3, 1, 256, BF16, F32, 1.0)
    assert rc == -1 and "window" in msg
    # q heads not a multiple of the KV heads (repeat_kv, :202-210)
    rc, msg = _attend(shim, 0, [0, 0], 2, 8, 1, -1, 15, 8, 128, BF16, F32, 0.1)
    assert rc == -1 and "n_rep" in msg


def _rms(x):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6)


def _inputs(b, t, hq, hkv, d, seed):
    rng = np.random.default_rng(seed)
    q = _rms(rng.standard_normal((b, t, hq, d))).astype(np.float32)
    k = _rms(rng.standard_normal((b, t, hkv, d))).astype(np.float32)
    v = rng.standard_normal((b, t, hkv, d)).astype(np.float32)
    return q, k, v


def _dev(x, torch, cuda):
    return torch.from_numpy(x).to(cuda).to(torch.bfloat16).contiguous()


def _host(t):
    return t.float().cpu().numpy().astype(np.float64).transpose(0, 2, 1, 3)   # [B, H, T, D]


@pytest.mark.gpu
def test_attend_qwen3_left_padded(shim, cuda):
    """attend on a left-padded causal GQA batch vs the reference's eager form
    with its summed -1e4 mask (attention.rs:170-199,236-249)."""
    import torch
    b, t, hq, hkv, d = 3, 130, 16, 8, 128
    pads = [0, 129, 57]
    q, k, v = _inputs(b, t, hq, hkv, d, 21)
    qd, kd, vd = (_dev(x, torch, cuda) for x in (q, k, v))
    ref = oa.qwen3_eager(_host(qd), _host(kd), _host(vd), oa.qwen3_additive_mask(pads, t), d ** -0.5, hq // hkv)
    out = torch.full((b, t, hq, d), 4321.0, dtype=torch.float32, device=cuda)
    print(f"C++ attend qwen3 left-padded pads={pads}", flush=True)
    rc, msg = _attend(shim, 0, pads, b, t, 1, -1, hq, hkv, d, BF16, F32, d ** -0.5,
                      qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(), repeat=2)
    torch.cuda.synchronize()
    assert rc == 0, msg
    got = out.cpu().numpy().transpose(0, 2, 1, 3)
    for i, p in enumerate(pads):
        err = np.abs(got[i, :, p:] - ref[i, :, p:]).max()
        assert err <= 2e-3, f"row {i}: max abs err {err:.3g}"
        assert np.all(got[i, :, :p] == 4321.0), f"row {i}: a padded row was written"


@pytest.mark.gpu
@pytest.mark.parametrize("window", [-1, 24], ids=["full", "sliding24"])
def test_attend_gemma2_right_padded(shim, cuda, window):
    """attend on a right-padded bidirectional batch, GQA 3/1, scale 1, with
    the -1e9 f32 mask and inclusive window (gemma2.rs:414-441,499-523)."""
    import torch
    b, t, hq, hkv, d = 2, 100, 3, 1, 256
    lens = [100, 31]
    q, k, v = _inputs(b, t, hq, hkv, d, 22)
    q *= np.float32(d ** -0.5)
    qd, kd, vd = (_dev(x, torch, cuda) for x in (q, k, v))
    mask = oa.gemma2_attention_mask(lens, t, None if window < 0 else window)
    ref = oa.gemma2_attention(_host(qd), _host(kd), _host(vd), None if mask is None else mask.astype(np.float64))
    out = torch.full((b, t, hq, d), 99.0, dtype=torch.float32, device=cuda)
    print(f"C++ attend gemma2 right-padded window={window}", flush=True)
    rc, msg = _attend(shim, 1, lens, b, t, 0, window, hq, hkv, d, BF16, F32, 1.0,
                      qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(), repeat=2)
    torch.cuda.synchronize()
    assert rc == 0, msg
    got = out.cpu().numpy().transpose(0, 2, 1, 3)
    for i, n in enumerate(lens):
        err = np.abs(got[i, :, :n] - ref[i, :, :n]).max()
        assert err <= 2e-3, f"row {i}: max abs err {err:.3g}"
        assert np.all(got[i, :, n:] == 99.0), f"row {i}: a padded row was written"
