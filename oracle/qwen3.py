"""Qwen3 encoder oracle (numpy): the end-to-end forward of the reference's
Qwen3 embedder over packed texts. TEST INFRASTRUCTURE ONLY - never on the
product path.

It follows crates/inl-text/src/qwen3/mod.rs:
- ``Mlp::forward`` (:109-116): ``down(silu(gate(x)) * up(x))``, every Linear
  without bias (:99-104);
- ``Attention::forward`` (:227-254): q/k/v projections, the per-head q/k
  RMSNorm, the half-split RoPE from the f64 ``RotaryTable`` (:123-159),
  causal GQA attention with scale ``head_dim^-0.5`` (:211,250), o_proj;
- ``DecoderLayer::forward`` (:280-297): pre-norm residual blocks;
- ``Qwen3Model::forward_last`` (:339-358): the final RMSNorm of each text's
  last position;
- ``Qwen3Embedder::embed`` (:464-469): L2 with ``1e-12`` inside the sqrt.

Texts are packed (positions restart at 0 for every text, attention stays
inside a text), which equals the reference's left-padded batch by its own
padding-invariance test (qwen3/mod.rs:647-669). The attention, RMSNorm, RoPE
and pooling steps are the pinned functions of ``oracle.attention``,
``oracle.prologue`` and ``oracle.pooling``; the composition is pinned against
an independent implementation of the same architecture (transformers'
``Qwen3Model``) in ``tests/test_oracle_qwen3.py``.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import attention as oa
from . import pooling as opl
from . import prologue as op


@dataclass(frozen=True)
class Qwen3Config:
    """The fields of qwen3/mod.rs's ``Config`` the forward uses."""
    vocab: int = 151669
    hidden: int = 1024
    intermediate: int = 3072
    layers: int = 28
    heads: int = 16
    kv_heads: int = 8
    head_dim: int = 128
    eps: float = 1e-6
    theta: float = 1e6


# The benchmark's configuration 1 (Qwen3-Embedding-0.6B architecture).
QWEN3_0_6B = Qwen3Config()


def layer_shapes(cfg: Qwen3Config):
    """(name, shape, is_norm) of one decoder layer's weights, in the
    checkpoint's names (qwen3/mod.rs:188-209, :262-278)."""
    q_out, kv_out = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    return [
        ("self_attn.q_proj.weight", (q_out, cfg.hidden), False),
        ("self_attn.k_proj.weight", (kv_out, cfg.hidden), False),
        ("self_attn.v_proj.weight", (kv_out, cfg.hidden), False),
        ("self_attn.o_proj.weight", (cfg.hidden, q_out), False),
        ("self_attn.q_norm.weight", (cfg.head_dim,), True),
        ("self_attn.k_norm.weight", (cfg.head_dim,), True),
        ("mlp.gate_proj.weight", (cfg.intermediate, cfg.hidden), False),
        ("mlp.up_proj.weight", (cfg.intermediate, cfg.hidden), False),
        ("mlp.down_proj.weight", (cfg.hidden, cfg.intermediate), False),
        ("input_layernorm.weight", (cfg.hidden,), True),
        ("post_attention_layernorm.weight", (cfg.hidden,), True),
    ]


def random_weights(cfg: Qwen3Config, seed: int = 0, dtype=np.float32) -> dict:
    """Random weights distributed as the reference's test weights
    (qwen3/mod.rs:522-589): matrices ``u * 2 / sqrt(fan_in)`` and norm
    weights ``1 + 0.2 u``, u uniform in [-0.5, 0.5) (here from numpy's
    generator, not the test's LCG)."""
    rng = np.random.default_rng(seed)

    def draw(shape, norm):
        u = rng.random(shape, dtype=np.float32) - np.float32(0.5)
        return (1 + 0.2 * u if norm else u * (2 / np.sqrt(shape[-1]))).astype(dtype)

    w = {"embed_tokens.weight": draw((cfg.vocab, cfg.hidden), False)}
    for i in range(cfg.layers):
        for name, shape, norm in layer_shapes(cfg):
            w[f"layers.{i}.{name}"] = draw(shape, norm)
    w["norm.weight"] = draw((cfg.hidden,), True)
    return w


def silu(x):
    """``x * sigmoid(x)`` (candle ``Activation::Silu``, qwen3/mod.rs:111)."""
    return x / (1.0 + np.exp(-x))


def encode(weights: dict, cfg: Qwen3Config, ids, cu_seqlens, dtype=np.float64, last_hidden=False):
    """Unit-length embeddings ``[texts, hidden]`` of packed texts ``ids``
    (text b = ``ids[cu[b]:cu[b+1]]``), or with ``last_hidden`` the final
    RMSNorm of each text's last row before the L2 (forward_last)."""
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    ids = np.asarray(ids, dtype=np.int64)
    n = int(cu[-1])
    W = lambda name: np.asarray(weights[name], dtype=dtype)
    hq, hkv, d = cfg.heads, cfg.kv_heads, cfg.head_dim
    lengths = np.diff(cu)
    cos, sin = op.rope_table(d, cfg.theta, int(lengths.max()) if len(lengths) else 1)
    pos = op.positions_of(cu)
    c = cos[pos][:, None, :].astype(dtype)
    s = sin[pos][:, None, :].astype(dtype)
    h = W("embed_tokens.weight")[ids]                                  # [n, hidden]
    for i in range(cfg.layers):
        p = f"layers.{i}."
        x = op.rms_norm(h, W(p + "input_layernorm.weight"), cfg.eps, dtype)
        q = (x @ W(p + "self_attn.q_proj.weight").T).reshape(n, hq, d)
        k = (x @ W(p + "self_attn.k_proj.weight").T).reshape(n, hkv, d)
        v = (x @ W(p + "self_attn.v_proj.weight").T).reshape(n, hkv, d)
        q = op.rope(op.rms_norm(q, W(p + "self_attn.q_norm.weight"), cfg.eps, dtype), c, s)
        k = op.rope(op.rms_norm(k, W(p + "self_attn.k_norm.weight"), cfg.eps, dtype), c, s)
        a = oa.varlen_attention(q, k, v, cu, causal=True, scale=d ** -0.5)
        h = h + a.reshape(n, hq * d) @ W(p + "self_attn.o_proj.weight").T
        x = op.rms_norm(h, W(p + "post_attention_layernorm.weight"), cfg.eps, dtype)
        g = x @ W(p + "mlp.gate_proj.weight").T
        u = x @ W(p + "mlp.up_proj.weight").T
        h = h + (silu(g) * u) @ W(p + "mlp.down_proj.weight").T
    if last_hidden:
        return op.rms_norm(h[cu[1:] - 1], W("norm.weight"), cfg.eps, dtype)
    return opl.last_token(h, cu, W("norm.weight"), cfg.eps, dtype)


def forward_flops(cfg: Qwen3Config, lengths) -> int:
    """Algorithmic FLOPs of one encode: the projections and MLP (2 per
    multiply-add) and the causal attention's visible pairs; the final norm,
    pooling and elementwise work are not counted."""
    n = int(sum(int(t) for t in lengths))
    q_out, kv_out = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    per_token = 2 * (cfg.hidden * (q_out + 2 * kv_out) + q_out * cfg.hidden + 3 * cfg.hidden * cfg.intermediate)
    return cfg.layers * (n * per_token + oa.attention_flops(lengths, cfg.heads, cfg.head_dim, True))
