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


def test_gemma2_tiny_oracle_f32_mode_matches_golden(gemma2):
    """oracle.gemma2.encode in f32 arithmetic (the CPU baseline's mode) on the
    golden texts: within 1e-5 of the golden vectors (f32 rounding of six
    32-wide layers; the f64 mode is held to the reference's 2e-5 above)."""
    from oracle import attention as oa
    from oracle import gemma2 as og
    cfg, W, golden, fdir = gemma2
    case = golden["cases"][0]
    ids = te.tokenize(fdir, golden["texts"], case["max_length"])
    cu = oa.cu_from_lengths([len(x) for x in ids])
    emb = og.encode(W, cfg["text_config"], np.concatenate(ids), cu, prefix="language_model.", dtype=np.float32)
    assert emb.dtype == np.float32
    err = np.abs(emb - np.asarray(case["batched"])).max()
    print(f"tiny EmbeddingGemma2 oracle f32: max-abs {err:.3g}")
    assert err < 1e-5, err


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


# ---------------------------------------------------------------------------
# Tiny SPLADE (ModernBERT MLM, 5 layers, 4 heads of 8, local radius 4)
# ---------------------------------------------------------------------------

SPLADE_TOL = 1e-4   # modernbert.rs:1045,1054 (exact index sets, weights to 1e-4)


@pytest.fixture(scope="module")
def splade():
    return te.load_fixture("tiny_splade")


def _check_splade(fx, ops, tol=SPLADE_TOL):
    """Every case (document / query prefix, max_length 64 / 12), batched and
    alone: the active-term set exactly, the weights within ``tol``."""
    worst = 0.0
    for case in fx[2]["cases"]:
        label = f"{case['kind']}/{case['max_length']}"
        rows = [r["ids"] for r in case["batched"]]
        runs = [("batched", case["batched"], te.modernbert_splade(fx, rows, ops))]
        runs.append(("alone", case["alone"], [te.modernbert_splade(fx, [r["ids"]], ops)[0]
                                                for r in case["alone"]]))
        for mode, want, got in runs:
            for i, (row, (idx, val)) in enumerate(zip(want, got)):
                assert idx.tolist() == row["indices"], f"{label} {mode}[{i}]: active terms differ"
                err = float(np.abs(val - np.asarray(row["values"], dtype=np.float32)).max())
                assert err <= tol, f"{label} {mode}[{i}]: weight error {err:.3g}"
                worst = max(worst, err)
    return worst


def test_splade_tiny_oracle_matches_golden(splade):
    worst = _check_splade(splade, te.OracleOps())
    print(f"tiny SPLADE oracle: worst weight error {worst:.3g}")


@pytest.mark.parametrize("kind", ["window+1", "window-1", "causal"])
def test_splade_tiny_golden_rejects_mask_mistakes(splade, kind):
    """An off-by-one local radius or a causal mask changes the 43-token
    row's active terms or moves its weights past the bound."""
    case = splade[2]["cases"][0]
    row = case["batched"][1]
    idx, val = te.modernbert_splade(splade, [row["ids"]], _Planted(kind))[0]
    same = idx.tolist() == row["indices"]
    assert not same or np.abs(val - np.asarray(row["values"])).max() > 10 * SPLADE_TOL


@pytest.mark.gpu
def test_splade_tiny_hip_matches_golden(splade, cuda, inl):
    """The same forward with attention (f32, head dim 8, local and global),
    RoPE and the SPLADE epilogue (row max, finish, canonical fold) on the
    GPU."""
    import torch
    worst = _check_splade(splade, te.HipOps(inl, torch, cuda))
    print(f"tiny SPLADE HIP: worst weight error {worst:.3g}")
