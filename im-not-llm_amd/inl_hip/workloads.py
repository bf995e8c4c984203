"""Synthetic packed workloads of the benchmark configurations (seeded numpy).

Lengths only - inputs are drawn by the callers. The generators reproduce the
token counts the measurement plan fixes for seed 0 (numpy ``default_rng``):
config 2 gives 713 texts / 200,179 tokens / 0.5034 TFLOP causal (12 batches
of up to 64 texts).
"""
from __future__ import annotations

import numpy as np


def qwen3_op_lengths(seed: int = 0, sigma: float = 1.0, median: float = 180.0,
                     max_len: int = 2048, min_total: int = 200_000):
    """Config 2: lengths ``clip(round(lognormal(ln median, sigma)), 1, max_len)``
    drawn one text at a time until at least ``min_total`` tokens."""
    rng = np.random.default_rng(seed)
    lens, total = [], 0
    while total < min_total:
        t = int(np.clip(np.round(rng.lognormal(np.log(median), sigma)), 1, max_len))
        lens.append(t)
        total += t
    return lens


def batches(lengths, size: int = 64):
    """Split lengths into consecutive batches of ``size`` texts."""
    return [list(lengths[i:i + size]) for i in range(0, len(lengths), size)]


def uniform_lengths(n: int, lo: int, hi: int, seed: int = 0):
    """``n`` lengths uniform in ``[lo, hi]`` (configs 1, 3 and 4)."""
    rng = np.random.default_rng(seed)
    return [int(x) for x in rng.integers(lo, hi + 1, size=n)]


def cu_seqlens(lengths):
    out = [0]
    for t in lengths:
        out.append(out[-1] + int(t))
    return out


class Qwen3Shape:
    """Architecture fields of a Qwen3 encoder (the attributes
    ``inl_hip.Qwen3Encoder`` reads); the default is Qwen3-Embedding-0.6B
    28 layers, hidden 1024, 16 q / 8 kv heads of
    128, intermediate 3072, vocab 151669, RoPE theta 1e6, eps 1e-6."""

    def __init__(self, vocab=151669, hidden=1024, intermediate=3072, layers=28, heads=16, kv_heads=8,
                 head_dim=128, eps=1e-6, theta=1e6):
        self.vocab, self.hidden, self.intermediate, self.layers = vocab, hidden, intermediate, layers
        self.heads, self.kv_heads, self.head_dim, self.eps, self.theta = heads, kv_heads, head_dim, eps, theta


def qwen3_random_weights(shape, torch, dev, dtype, seed=0):
    """Seeded random weights on the device, named as the checkpoint:
    matrices ``u * 2 / sqrt(fan_in)`` and norm weights ``1 + 0.2 u`` with u
    uniform in [-0.5, 0.5), the distribution of the reference's test weights
    (crates/inl-text/src/qwen3/mod.rs:522-589)."""
    g = torch.Generator(device=dev).manual_seed(seed)

    def draw(shape_, norm):
        u = torch.rand(*shape_, generator=g, device=dev) - 0.5
        return (1 + 0.2 * u if norm else u * (2 / shape_[-1] ** 0.5)).to(dtype)

    c = shape
    q_out, kv_out = c.heads * c.head_dim, c.kv_heads * c.head_dim
    w = {"embed_tokens.weight": draw((c.vocab, c.hidden), False)}
    for i in range(c.layers):
        p = f"layers.{i}."
        for name, shp, norm in (("self_attn.q_proj.weight", (q_out, c.hidden), False),
                                ("self_attn.k_proj.weight", (kv_out, c.hidden), False),
                                ("self_attn.v_proj.weight", (kv_out, c.hidden), False),
                                ("self_attn.o_proj.weight", (c.hidden, q_out), False),
                                ("self_attn.q_norm.weight", (c.head_dim,), True),
                                ("self_attn.k_norm.weight", (c.head_dim,), True),
                                ("mlp.gate_proj.weight", (c.intermediate, c.hidden), False),
                                ("mlp.up_proj.weight", (c.intermediate, c.hidden), False),
                                ("mlp.down_proj.weight", (c.hidden, c.intermediate), False),
                                ("input_layernorm.weight", (c.hidden,), True),
                                ("post_attention_layernorm.weight", (c.hidden,), True)):
            w[p + name] = draw(shp, norm)
    w["norm.weight"] = draw((c.hidden,), True)
    return w


# EmbeddingGemma 2 text tower (crates/inl-text/src/gemma2.rs)

def gemma2_config3(vocab=262144, layers=24):
    """The configuration-3 shape (24 layers, hidden 768, 3 Q / 1 KV heads x
    256, sliding radius 512, every sixth layer full as gemma2.rs:11-13 says)
    in the checkpoint's ``text_config`` form. Not in the benchmark's
    description, so chosen here: intermediate 1152 (the EmbeddingGemma text
    tower's), per-layer input 256, embedding_dim 768, rope θ 1e4 / 1e6
    (crates/inl-text/src/gemma2.rs:76-102 lists the fields)."""
    return {
        "vocab_size": vocab, "hidden_size": 768, "intermediate_size": 1152, "num_hidden_layers": layers,
        "num_attention_heads": 3, "num_key_value_heads": 1, "head_dim": 256, "rms_norm_eps": 1e-6,
        "sliding_window": 512,
        "layer_types": ["full_attention" if (i + 1) % 6 == 0 else "sliding_attention" for i in range(layers)],
        "hidden_size_per_layer_input": 256, "embedding_dim": 768,
        "rope_parameters": {"sliding_attention": {"rope_theta": 1e4}, "full_attention": {"rope_theta": 1e6}},
        "per_layer_config": {}, "max_position_embeddings": 8192,
    }


def gemma2_random_weights(tc, seed=0):
    """Seeded random-init f32 weights of ``tc`` by tensor name: projections
    N(0, 1/in), norm weights 1 + N(0, 0.05^2) (q/k norms a quarter of that),
    embeddings N(0, 0.05^2) (rows of norm ~1.4 after the sqrt(768) scale),
    layer scalars U[0.5, 1]."""
    rng = np.random.default_rng(seed)
    hs, ff, ple = tc["hidden_size"], tc["intermediate_size"], tc["hidden_size_per_layer_input"]
    L, heads = tc["num_hidden_layers"], tc["num_attention_heads"]
    f = lambda *shape: rng.standard_normal(shape, dtype=np.float32)
    lin = lambda out, inp: f(out, inp) / np.float32(np.sqrt(inp))
    norm = lambda d: (1.0 + 0.05 * f(d)).astype(np.float32)
    # Attention is unscaled on RMS-normed q and k: with norm weights near 1 the
    # scores of random vectors have a standard deviation of sqrt(head_dim) = 16
    # and the softmax is nearly one-hot, so bf16 rounding flips which key wins
    # from layer to layer. q/k norm weights near 0.25 give scores of deviation ~1.
    qk_norm = lambda d: (0.25 * (1.0 + 0.05 * f(d))).astype(np.float32)
    W = {"embed_tokens.weight": (f(tc["vocab_size"], hs) * np.float32(0.05)),
         "ple.per_layer_model_projection.weight": lin(L * ple, hs),
         "ple.per_layer_projection_norm.weight": norm(ple),
         "norm.weight": norm(hs), "embedding_projection.weight": lin(tc["embedding_dim"], hs)}
    for i in range(L):
        over = tc.get("per_layer_config", {}).get(f"{i:02d}", {})
        hd = over.get("head_dim", tc["head_dim"])
        kvh = over.get("num_key_value_heads", tc["num_key_value_heads"])
        p = f"layers.{i}."
        W.update({
            p + "self_attn.q_proj.weight": lin(heads * hd, hs), p + "self_attn.k_proj.weight": lin(kvh * hd, hs),
            p + "self_attn.v_proj.weight": lin(kvh * hd, hs), p + "self_attn.o_proj.weight": lin(hs, heads * hd),
            p + "self_attn.q_norm.weight": qk_norm(hd), p + "self_attn.k_norm.weight": qk_norm(hd),
            p + "input_layernorm.weight": norm(hs), p + "post_attention_layernorm.weight": norm(hs),
            p + "pre_feedforward_layernorm.weight": norm(hs), p + "post_feedforward_layernorm.weight": norm(hs),
            p + "mlp.gate_proj.weight": lin(ff, hs), p + "mlp.up_proj.weight": lin(ff, hs),
            p + "mlp.down_proj.weight": lin(hs, ff),
            p + "ple_block.per_layer_input_gate.weight": lin(ple, hs),
            p + "ple_block.per_layer_projection.weight": lin(hs, ple),
            p + "ple_block.post_per_layer_input_norm.weight": norm(hs),
            p + "layer_scalar": rng.uniform(0.5, 1.0, 1).astype(np.float32),
        })
    return W
