"""CPU pins of the end-to-end Qwen3 encoder oracle (oracle/qwen3.py).

- Against an independent implementation of the same architecture:
  transformers' ``Qwen3Model`` (float64), loaded with the oracle's weights
  under the checkpoint's names. Its final hidden state at each text's last
  position must equal the oracle's ``forward_last``. transformers builds the
  RoPE tables in f32 where the reference uses f64 angles, so the two agree to
  about 1e-6, not to rounding; the bound is 1e-5.
- Planted mistakes in the oracle (no rotation, bidirectional attention, the
  MLP's gate and up swapped, the q/k norm skipped) fail that bound by orders
  of magnitude.
- The reference's own invariants (qwen3/mod.rs:647-669): unit-length
  embeddings, and a text batched with a longer one embeds as it does alone.
"""
import numpy as np
import pytest

from oracle import attention as oa
from oracle import prologue as op
from oracle import qwen3 as oq

TINY = oq.Qwen3Config(vocab=24, hidden=48, intermediate=96, layers=2, heads=4, kv_heads=2, head_dim=32,
                      eps=1e-6, theta=10_000.0)
TEXTS = [[1, 2, 3, 4, 5, 6, 1, 2, 3, 4], [1, 2], [3, 4, 5], [6]]   # "a b c d e f a b c d", "a b", ...


def _hf_last_hidden(weights, cfg, texts):
    torch = pytest.importorskip("torch")
    transformers = pytest.importorskip("transformers")
    hf_cfg = transformers.Qwen3Config(
        vocab_size=cfg.vocab, hidden_size=cfg.hidden, intermediate_size=cfg.intermediate,
        num_hidden_layers=cfg.layers, num_attention_heads=cfg.heads, num_key_value_heads=cfg.kv_heads,
        head_dim=cfg.head_dim, rms_norm_eps=cfg.eps, rope_theta=cfg.theta, attention_bias=False,
        hidden_act="silu", max_position_embeddings=64)
    model = transformers.Qwen3Model(hf_cfg).double().eval()
    state = {k: torch.from_numpy(np.asarray(v, dtype=np.float64)) for k, v in weights.items()}
    missing, unexpected = model.load_state_dict(state, strict=False)
    assert not unexpected and all("rotary" in m for m in missing), (missing, unexpected)
    out = []
    with torch.no_grad():
        for t in texts:
            hs = model(input_ids=torch.tensor([t])).last_hidden_state
            out.append(hs[0, -1].numpy())
    return np.stack(out)


def _packed(texts):
    ids = np.concatenate([np.asarray(t) for t in texts])
    return ids, oa.cu_from_lengths([len(t) for t in texts])


@pytest.fixture(scope="module")
def tiny():
    w = oq.random_weights(TINY, seed=3, dtype=np.float64)
    return w, _hf_last_hidden(w, TINY, TEXTS)


def test_oracle_matches_transformers_qwen3(tiny):
    w, ref = tiny
    ids, cu = _packed(TEXTS)
    got = oq.encode(w, TINY, ids, cu, last_hidden=True)
    assert np.abs(got - ref).max() < 1e-5
    assert np.abs(ref).max() > 0.5   # a real signal, not a near-zero output


@pytest.mark.parametrize("mistake", ["no_rope", "bidirectional", "gate_up_swapped", "no_qk_norm"])
def test_planted_mistakes_fail(tiny, mistake, monkeypatch):
    w, ref = tiny
    ids, cu = _packed(TEXTS)
    if mistake == "no_rope":
        monkeypatch.setattr(op, "rope", lambda x, c, s: x)
    elif mistake == "bidirectional":
        real = oa.varlen_attention
        monkeypatch.setattr(oa, "varlen_attention", lambda q, k, v, cu, **kw: real(q, k, v, cu, **{**kw, "causal": False}))
    elif mistake == "gate_up_swapped":
        w = dict(w)
        for i in range(TINY.layers):
            g, u = f"layers.{i}.mlp.gate_proj.weight", f"layers.{i}.mlp.up_proj.weight"
            w[g], w[u] = w[u], w[g]
    elif mistake == "no_qk_norm":
        w = dict(w)
        for i in range(TINY.layers):
            for n in ("q_norm", "k_norm"):
                w[f"layers.{i}.self_attn.{n}.weight"] = np.ones(TINY.head_dim)
        real = op.rms_norm
        monkeypatch.setattr(op, "rms_norm", lambda x, wt, eps, dtype=np.float64:
                            x.astype(dtype) * (np.asarray(wt, dtype) if wt is not None else 1)
                            if x.ndim == 3 else real(x, wt, eps, dtype))
    got = oq.encode(w, TINY, ids, cu, last_hidden=True)
    assert np.abs(got - ref).max() > 1e-2, mistake


def test_unit_length_and_batch_invariance():
    """qwen3/mod.rs:647-669: unit norm within 1e-5; "c d e" batched with a
    longer text has cosine > 0.99999 with "c d e" alone."""
    w = oq.random_weights(TINY, seed=4, dtype=np.float64)
    alone = oq.encode(w, TINY, *_packed([[3, 4, 5]]))[0]
    assert abs(np.linalg.norm(alone) - 1) < 1e-5
    batched = oq.encode(w, TINY, *_packed([[1, 2, 3, 4, 5, 6, 1, 2, 3, 4], [3, 4, 5]]))[1]
    assert float(alone @ batched) > 0.99999


def test_forward_flops_count():
    """2 flops per multiply-add of the four projections and the MLP per token
    and layer, plus the causal attention: for the 0.6B shape that is 31.5
    MFLOP of matrix work per token per layer."""
    cfg = oq.QWEN3_0_6B
    per_token = 2 * (1024 * (2048 + 2 * 1024) + 2048 * 1024 + 3 * 1024 * 3072)
    assert per_token == 31_457_280
    assert oq.forward_flops(cfg, [10]) == 28 * (10 * per_token + 4 * 16 * 128 * 55)
