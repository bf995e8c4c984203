"""End-to-end pins against the reference's tiny HF golden fixtures.

The tiny EmbeddingGemma 2 checkpoint (6 layers, GQA 4/2 heads of 16 on the
sliding layers with radius 3, 4/1 heads of 32 on the full layers) is run by
``tests/tiny_encoders.py``. Its attention, per-head norms, RoPE, mean pooling
and L2 go through the oracle (CPU tests) or the HIP library (GPU test); the
result must match the vectors HF ``transformers`` produced, within the
reference's own bound for this test, 2e-5 max-abs
(crates/inl-text/src/gemma2.rs:942-967), for every text both batched and
alone, at max_length 64 and 9.
"""
import numpy as np
import pytest

import tiny_encoders as te

TOL = 2e-5   # gemma2.rs:953,963


@pytest.fixture(scope="module")
def gemma2():
    return te.load_fixture("tiny_embeddinggemma2")


def _check_gemma2(fx, ops, tol=TOL):
    golden = fx[2]
    worst = 0.0
    for case in golden["cases"]:
        emb, lens = te.gemma2_embed(fx, golden["texts"], case["max_length"], ops)
        assert lens == case["lengths"], "tokenization differs from the golden's"
        assert emb.shape == (len(golden["texts"]), golden["dim"])
        err = np.abs(emb - np.asarray(case["batched"])).max()
        assert err < tol, f"max_length {case['max_length']} batched: {err:.3g}"
        worst = max(worst, err)
        for i, text in enumerate(golden["texts"]):
            alone, _ = te.gemma2_embed(fx, [text], case["max_length"], ops)
            err = np.abs(alone[0] - np.asarray(case["alone"][i])).max()
            assert err < tol, f"max_length {case['max_length']} alone row {i}: {err:.3g}"
            worst = max(worst, err)
    return worst


def test_gemma2_tiny_oracle_matches_golden(gemma2):
    worst = _check_gemma2(gemma2, te.OracleOps())
    print(f"tiny EmbeddingGemma2 oracle: worst max-abs {worst:.3g}")


class _Planted(te.OracleOps):
    """The oracle with one plausible mistake in the attention mask."""

    def __init__(self, kind):
        self.kind = kind

    def attention(self, q, k, v, cu, *, causal, window, scale):
        if self.kind == "window+1" and window >= 0:
            window += 1
        elif self.kind == "window-1" and window >= 0:
            window -= 1
        elif self.kind == "causal":
            causal = True
        elif self.kind == "scaled":
            scale = q.shape[-1] ** -0.5
        return super().attention(q, k, v, cu, causal=causal, window=window, scale=scale)


@pytest.mark.parametrize("kind", ["window+1", "window-1", "causal", "scaled"])
def test_gemma2_tiny_golden_rejects_mask_mistakes(gemma2, kind):
    """The golden discriminates: an off-by-one window radius, a causal mask
    or the usual 1/sqrt(d) scale (EmbeddingGemma uses 1) each move the
    embeddings far outside the bound."""
    golden = gemma2[2]
    case = golden["cases"][0]
    emb, _ = te.gemma2_embed(gemma2, golden["texts"], case["max_length"], _Planted(kind))
    assert np.abs(emb - np.asarray(case["batched"])).max() > 100 * TOL


@pytest.mark.gpu
def test_gemma2_tiny_hip_matches_golden(gemma2, cuda, inl):
    """The same forward with attention (f32, head dims 16 and 32, sliding and
    full), the per-head norms + RoPE, mean pooling and L2 on the GPU."""
    import torch
    worst = _check_gemma2(gemma2, te.HipOps(inl, torch, cuda))
    print(f"tiny EmbeddingGemma2 HIP: worst max-abs {worst:.3g}")
