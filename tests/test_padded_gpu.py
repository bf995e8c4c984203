"""GPU parity on padded batches run in place (``seq_starts``).

The reference engines hand attention ``[B, T]`` padded batches with additive
masks: Qwen3 pads on the left (crates/inl-core/src/attention.rs:126-199),
EmbeddingGemma 2 and ModernBERT on the right (gemma2.rs:499-523,
modernbert.rs:594-617). With ``seq_starts`` the HIP kernel runs on the same
``[B*T, H, D]`` rows, text b starting at ``b*T + pad_b`` (left) or ``b*T``
(right). The reference leaves padded rows unspecified
(attention.rs:213-214); these tests compare the real rows against the
oracle's padded forms with the reference masks, and check that the kernel
does not write the padded rows.
Tolerance: 2e-3 max-abs for bf16 inputs (f32 output), 1e-5 for f32.
"""
import numpy as np
import pytest

from oracle import attention as oa

pytestmark = pytest.mark.gpu


def _rms(x):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6)


def _padded_inputs(b, t, hq, hkv, d, seed):
    rng = np.random.default_rng(seed)
    q = _rms(rng.standard_normal((b, t, hq, d))).astype(np.float32)
    k = _rms(rng.standard_normal((b, t, hkv, d))).astype(np.float32)
    v = rng.standard_normal((b, t, hkv, d)).astype(np.float32)
    return q, k, v


def _to_dev(x, dtype, torch, dev):
    b, t, h, d = x.shape
    return torch.from_numpy(x.reshape(b * t, h, d)).to(dev).to(dtype)


def _host(t):
    return t.float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("dtype_name", ["bf16", "f32"])
def test_qwen3_left_padded_matches_eager(dtype_name, cuda, inl):
    """Left-padded causal GQA vs the reference's eager path with its summed
    -1e4 causal+padding mask (attention.rs:236-249)."""
    import torch
    dtype = torch.bfloat16 if dtype_name == "bf16" else torch.float32
    b, t, hq, hkv, d = 4, 150, 16, 8, 128
    lens = [150, 1, 77, 129]
    pads = [t - n for n in lens]
    q, k, v = _padded_inputs(b, t, hq, hkv, d, 11)
    qd, kd, vd = (_to_dev(x, dtype, torch, cuda) for x in (q, k, v))
    # the oracle runs on the values the device holds
    qh, kh, vh = (_host(x).reshape(b, t, -1, d).transpose(0, 2, 1, 3) for x in (qd, kd, vd))
    mask = oa.qwen3_additive_mask(pads, t)
    ref = oa.qwen3_eager(qh, kh, vh, mask, d ** -0.5, hq // hkv)      # [B, H, T, D]
    sentinel = 12345.0
    out = torch.full((b * t, hq, d), sentinel, dtype=torch.float32, device=cuda)
    print(f"left-padded qwen3 {dtype_name} lens={lens}", flush=True)
    inl.varlen_attention(qd, kd, vd, oa.cu_from_lengths(lens).tolist(), causal=True,
                         out=out, seq_starts=[i * t + p for i, p in enumerate(pads)])
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(b, t, hq, d).transpose(0, 2, 1, 3)
    tol = 2e-3 if dtype_name == "bf16" else 1e-5
    for i, p in enumerate(pads):
        err = np.abs(got[i, :, p:] - ref[i, :, p:]).max()
        assert err <= tol, f"text {i}: max abs err {err:.3g}"
        assert np.all(got[i, :, :p] == sentinel), f"text {i}: a padded row was written"


@pytest.mark.parametrize("window", [None, 16], ids=["full", "sliding16"])
def test_gemma2_right_padded_matches_reference(window, cuda, inl):
    """Right-padded bidirectional GQA 3/1, scale 1, -1e9 f32 mask with an
    optional inclusive window (gemma2.rs:414-441,499-523)."""
    import torch
    b, t, hq, hkv, d = 3, 90, 3, 1, 256
    lens = [90, 40, 7]
    q, k, v = _padded_inputs(b, t, hq, hkv, d, 12)
    q *= np.float32(d ** -0.5)        # unit-variance logits at scale 1
    qd, kd, vd = (_to_dev(x, torch.bfloat16, torch, cuda) for x in (q, k, v))
    qh, kh, vh = (_host(x).reshape(b, t, -1, d).transpose(0, 2, 1, 3) for x in (qd, kd, vd))
    mask = oa.gemma2_attention_mask(lens, t, window)
    ref = oa.gemma2_attention(qh, kh, vh, None if mask is None else mask.astype(np.float64))
    out = torch.full((b * t, hq, d), 777.0, dtype=torch.float32, device=cuda)
    print(f"right-padded gemma2 window={window}", flush=True)
    inl.varlen_attention(qd, kd, vd, oa.cu_from_lengths(lens).tolist(), causal=False,
                         window=-1 if window is None else window, scale=1.0, out=out,
                         seq_starts=[i * t for i in range(b)])
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(b, t, hq, d).transpose(0, 2, 1, 3)
    for i, n in enumerate(lens):
        err = np.abs(got[i, :, :n] - ref[i, :, :n]).max()
        assert err <= 2e-3, f"text {i}: max abs err {err:.3g}"
        assert np.all(got[i, :, n:] == 777.0), f"text {i}: a padded row was written"


def test_modernbert_right_padded_local(cuda, inl):
    """Right-padded ModernBERT local layer: radius 64, -1e4 masks, q scaled by
    64^-0.5 (modernbert.rs:366-401,594-617)."""
    import torch
    b, t, h, d = 2, 200, 12, 64
    lens = [200, 133]
    q, k, v = _padded_inputs(b, t, h, h, d, 13)
    qd, kd, vd = (_to_dev(x, torch.bfloat16, torch, cuda) for x in (q, k, v))
    qh, kh, vh = (_host(x).reshape(b, t, -1, d).transpose(0, 2, 1, 3) for x in (qd, kd, vd))
    _, local = oa.modernbert_masks(lens, t, 64)
    ref = oa.modernbert_attend(qh, kh, vh, local, d ** -0.5)
    out = torch.zeros((b * t, h, d), dtype=torch.float32, device=cuda)
    print("right-padded modernbert local", flush=True)
    inl.varlen_attention(qd, kd, vd, oa.cu_from_lengths(lens).tolist(), causal=False, window=64,
                         out=out, seq_starts=[0, t])
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(b, t, h, d).transpose(0, 2, 1, 3)
    for i, n in enumerate(lens):
        err = np.abs(got[i, :, :n] - ref[i, :, :n]).max()
        assert err <= 2e-3, f"text {i}: max abs err {err:.3g}"

