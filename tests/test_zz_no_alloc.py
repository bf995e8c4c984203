"""The allocation-free attention entry point (inl_attn_varlen_fwd_static),
called through the C ABI: its output must equal inl_attn_varlen_fwd's bit for
bit (same kernels, same schedule), on two calls in a row whose second is
smaller, so that a schedule left in the shared static buffer by the first
call cannot leak into the second. A batch whose schedule exceeds the static
buffer is refused on the host, before any device work."""
import ctypes

import numpy as np
import pytest

from oracle import attention as oa


def _static_fn(inl):
    fn = inl._lib.inl_attn_varlen_fwd_static
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.POINTER(inl.AttnDesc)] + [ctypes.c_void_p] * 5
    return fn


def test_static_entry_refuses_an_oversized_schedule(inl):
    """1,700 texts of 2,048 tokens, 16 heads x 64 with one K/V head each:
    8 head pairs x 16 row blocks per text is 217,600 units, 4,353,040 bytes
    of schedule, beyond the 4 MiB buffer. Nothing reaches the device: the
    pointers are never read."""
    fn = _static_fn(inl)
    desc = inl.make_attn_desc([2048 * i for i in range(1701)], 16, 16, 64, causal=False, dtype="bf16")
    n = ctypes.c_size_t()
    assert inl._ws_size(ctypes.byref(desc), ctypes.byref(n)) == 0 and n.value == 4_353_040
    fake = 1 << 20
    rc = fn(ctypes.byref(desc), fake, fake, fake, fake, None)
    assert rc == -1
    assert "static buffer" in inl.last_error() and "4194304" in inl.last_error()


def _case(lengths, seed, torch, dev):
    rng = np.random.default_rng(seed)
    n = int(sum(lengths))
    q = torch.from_numpy(rng.standard_normal((n, 16, 128)).astype(np.float32) * 0.1).to(dev).to(torch.bfloat16)
    k = torch.from_numpy(rng.standard_normal((n, 8, 128)).astype(np.float32)).to(dev).to(torch.bfloat16)
    v = torch.from_numpy(rng.standard_normal((n, 8, 128)).astype(np.float32)).to(dev).to(torch.bfloat16)
    return q, k, v


@pytest.mark.gpu
def test_static_entry_matches_the_workspace_entry(cuda, inl):
    import torch
    fn = _static_fn(inl)
    stream = torch.cuda.current_stream()
    for call, lengths in enumerate(([300, 1000, 77, 2048, 1, 129], [5, 130, 64])):
        print(f"case=no_alloc call={call} lengths={lengths}", flush=True)
        q, k, v = _case(lengths, 11 + call, torch, cuda)
        cu = oa.cu_from_lengths(lengths).tolist()
        want = inl.varlen_attention(q, k, v, cu, causal=True, out_dtype=torch.float32)
        got = torch.full_like(want, float("nan"))
        desc = inl.make_attn_desc(cu, 16, 8, 128, causal=True, scale=128 ** -0.5, dtype="bf16",
                                  out_dtype="f32")
        inl._check_tensors(desc, q, k, v, got)
        rc = fn(ctypes.byref(desc), q.data_ptr(), k.data_ptr(), v.data_ptr(), got.data_ptr(),
                stream.cuda_stream)
        assert rc == 0, inl.last_error()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {call}: static-buffer output differs from the workspace form"
        h = lambda t: t.float().cpu().numpy().astype(np.float64)
        ref = oa.varlen_attention(h(q), h(k), h(v), np.asarray(cu), causal=True, scale=128 ** -0.5)
        assert np.abs(got.cpu().numpy() - ref).max() <= 2e-3
