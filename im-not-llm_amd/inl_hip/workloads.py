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
