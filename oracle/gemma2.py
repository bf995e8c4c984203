"""EmbeddingGemma 2 text-tower oracle (numpy): the end-to-end forward of the
reference's Gemma2 embedder over packed texts. TEST INFRASTRUCTURE ONLY -
never on the product path.

It follows crates/inl-text/src/gemma2.rs:
- ``Gemma2Model::forward_pooled_from_embeds`` (:622-662): the embedding scale
  ``sqrt(hidden)`` (:576-587, :606-609), the per-layer inputs
  ``rms_norm(embeds . Wple^T * hidden^-0.5) * ple_norm`` per layer slice
  (:625-628), the layers, the final RMSNorm, the mean over each text's real
  tokens, ``embedding_projection`` and L2 with ``1e-12`` inside the sqrt;
- ``Layer::forward`` (:473-494): attention and MLP blocks with a pre- and a
  post-norm each, then the per-layer-input block (:279-283) and the
  ``layer_scalar``;
- ``Attention::forward`` (:381-441): q/k RMSNorm with weight, weightless v
  norm, half-split RoPE from the f64 ``RotaryTable`` of the layer kind
  (θ of ``sliding_attention`` / ``full_attention``, :292-315), scale 1,
  bidirectional, sliding layers masked to ``|q - k| <= sliding_window``;
- ``Mlp::forward`` (:249-254): ``down(gelu_tanh(gate(x)) * up(x))``.

Texts are packed (positions restart at 0 for every text, attention stays
inside a text): the reference right-pads and masks the padding, which is the
same function on the real rows. The attention, RMSNorm, RoPE and pooling
steps are the pinned functions of ``oracle.attention``, ``oracle.prologue``
and ``oracle.pooling``; the composition is pinned against the reference's
own golden vectors (tests/golden/tiny_embeddinggemma2, gemma2.rs:942-967) by
``tests/test_tiny_golden.py``.
"""
from __future__ import annotations

import numpy as np

from . import attention as oa
from . import pooling as opool
from . import prologue as opro


def gelu_tanh(x):
    """candle ``Tensor::gelu`` (the tanh approximation, ``gelu_pytorch_tanh``)."""
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def layer_shape(tc, i):
    """(kind, head_dim, kv_heads) of layer i: ``layer_types`` and the
    ``per_layer_config`` overrides keyed by zero-padded index (gemma2.rs:186-201)."""
    over = tc.get("per_layer_config", {}).get(f"{i:02d}", {})
    return (tc["layer_types"][i], over.get("head_dim", tc["head_dim"]),
            over.get("num_key_value_heads", tc["num_key_value_heads"]))


class Ops:
    """The hot-path steps as the pinned oracle functions compute them, in
    ``dtype`` (f64 for parity checks, f32 for the CPU baseline)."""

    def __init__(self, dtype=np.float64):
        self.dtype = dtype

    def norm_rope(self, x, weight, eps, table=None, pos=None):
        y = opro.rms_norm(x, weight, eps, dtype=self.dtype)
        if table is not None:
            cos, sin = table
            y = opro.rope(y, cos[pos][:, None, :].astype(self.dtype), sin[pos][:, None, :].astype(self.dtype))
        return y

    def attention(self, q, k, v, cu, *, causal, window, scale):
        return oa.varlen_attention(q, k, v, cu, causal=causal, window=window, scale=scale, dtype=self.dtype)

    def mean_pool(self, h, cu):
        return opool.mean_pool(h, cu, dtype=self.dtype)

    def l2(self, x):
        return opool.l2_normalize(x, dtype=self.dtype)


def encode(W, tc, ids, cu, ops=None, prefix="", dtype=np.float64):
    """Unit-length embeddings ``[texts, embedding_dim]`` of packed token ids
    (``cu`` the packed offsets). ``W`` maps tensor names (after ``prefix``)
    to arrays; ``dtype`` is the arithmetic type."""
    ops = ops or Ops(dtype)
    lens = np.diff(np.asarray(cu))
    pos = np.concatenate([np.arange(n) for n in lens])
    hs, eps = tc["hidden_size"], tc["rms_norm_eps"]
    n_layers, ple_dim = tc["num_hidden_layers"], tc["hidden_size_per_layer_input"]
    w = lambda name: np.asarray(W[prefix + name], dtype=dtype)

    def lin(x, name):
        return x @ w(name + ".weight").T

    positions = int(lens.max())
    tables = {}
    for kind in ("sliding_attention", "full_attention"):
        hd = next((layer_shape(tc, i)[1] for i in range(n_layers) if layer_shape(tc, i)[0] == kind),
                  tc["head_dim"])
        tables[kind] = opro.rope_table(hd, tc["rope_parameters"][kind]["rope_theta"], positions)

    h = w("embed_tokens.weight")[np.asarray(ids)] * dtype(np.sqrt(float(hs)))
    per_layer = (lin(h, "ple.per_layer_model_projection") * dtype(hs ** -0.5)).reshape(-1, n_layers, ple_dim)
    per_layer = opro.rms_norm(per_layer, w("ple.per_layer_projection_norm.weight"), eps, dtype=dtype)
    heads = tc["num_attention_heads"]
    n = h.shape[0]
    for i in range(n_layers):
        kind, hd, kvh = layer_shape(tc, i)
        lp = f"layers.{i}."
        x = opro.rms_norm(h, w(lp + "input_layernorm.weight"), eps, dtype=dtype)
        q = lin(x, lp + "self_attn.q_proj").reshape(n, heads, hd)
        k = lin(x, lp + "self_attn.k_proj").reshape(n, kvh, hd)
        v = lin(x, lp + "self_attn.v_proj").reshape(n, kvh, hd)
        q = ops.norm_rope(q, w(lp + "self_attn.q_norm.weight"), eps, tables[kind], pos)
        k = ops.norm_rope(k, w(lp + "self_attn.k_norm.weight"), eps, tables[kind], pos)
        v = ops.norm_rope(v, None, eps)
        window = tc["sliding_window"] if kind == "sliding_attention" else -1
        a = ops.attention(q, k, v, np.asarray(cu), causal=False, window=window, scale=1.0)
        a = lin(a.reshape(n, heads * hd), lp + "self_attn.o_proj")
        h = h + opro.rms_norm(a, w(lp + "post_attention_layernorm.weight"), eps, dtype=dtype)
        m = opro.rms_norm(h, w(lp + "pre_feedforward_layernorm.weight"), eps, dtype=dtype)
        m = lin(gelu_tanh(lin(m, lp + "mlp.gate_proj")) * lin(m, lp + "mlp.up_proj"), lp + "mlp.down_proj")
        h = h + opro.rms_norm(m, w(lp + "post_feedforward_layernorm.weight"), eps, dtype=dtype)
        g = gelu_tanh(lin(h, lp + "ple_block.per_layer_input_gate")) * per_layer[:, i, :]
        h = h + opro.rms_norm(lin(g, lp + "ple_block.per_layer_projection"),
                              w(lp + "ple_block.post_per_layer_input_norm.weight"), eps, dtype=dtype)
        h = h * w(lp + "layer_scalar")[0]
    h = opro.rms_norm(h, w("norm.weight"), eps, dtype=dtype)
    pooled = ops.mean_pool(h, np.asarray(cu))
    return ops.l2(lin(pooled, "embedding_projection"))
