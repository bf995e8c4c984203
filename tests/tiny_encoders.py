"""Tiny-checkpoint encoders for the reference's HF golden fixtures (test
infrastructure).

The fixtures under ``tests/golden/<name>/`` are the reference's own test data
(a tiny random ``model.safetensors``, its ``config.json`` and
``tokenizer.json``, and the ``golden.json`` vectors HF ``transformers``
produced for them). The encoders below run the whole tiny model in numpy,
following the reference's forward pass, and route the ops of the attention
hot path (per-head RMSNorm + RoPE, packed varlen attention, pooling, L2) to
an ``ops`` object: the numpy oracle (``OracleOps``) or the HIP library through
its C ABI (``HipOps``). Everything else (projections, MLP, embeddings) stays
in numpy f64.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

from oracle import attention as oa
from oracle import gdn as ogdn
from oracle import gemma2 as og
from oracle import pooling as opool
from oracle import prologue as opro

GOLDEN = Path(__file__).resolve().parent / "golden"


def load_fixture(name: str):
    """(config dict, f64 weights dict, golden dict, tokenizer directory)."""
    from safetensors.numpy import load_file
    d = GOLDEN / name
    cfg = json.loads((d / "config.json").read_text())
    weights = {k: v.astype(np.float64) for k, v in load_file(str(d / "model.safetensors")).items()}
    golden = json.loads((d / "golden.json").read_text())
    return cfg, weights, golden, d


def tokenize(fixture_dir: Path, texts, max_length: int):
    """Token ids per text: the fixture's tokenizer with its post-processor
    (special tokens) and truncation to ``max_length``, no padding (rows are
    packed)."""
    import tokenizers
    tok = tokenizers.Tokenizer.from_file(str(fixture_dir / "tokenizer.json"))
    tok.enable_truncation(max_length)
    return [e.ids for e in tok.encode_batch(list(texts))]


def gelu_tanh(x):
    """candle ``Tensor::gelu`` (the tanh approximation, ``gelu_pytorch_tanh``)."""
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


class OracleOps:
    """The hot-path ops as the numpy oracle computes them (f64)."""

    def norm_rope(self, x, weight, eps, table=None, pos=None):
        y = opro.rms_norm(x, weight, eps)
        if table is not None:
            cos, sin = table
            y = opro.rope(y, cos[pos][:, None, :].astype(np.float64), sin[pos][:, None, :].astype(np.float64))
        return y

    def rope(self, x, table, pos):
        cos, sin = table
        return opro.rope(x.astype(np.float64), cos[pos][:, None, :].astype(np.float64),
                         sin[pos][:, None, :].astype(np.float64))

    def attention(self, q, k, v, cu, *, causal, window, scale):
        return oa.varlen_attention(q, k, v, cu, causal=causal, window=window, scale=scale)

    def mean_pool(self, h, cu):
        return opool.mean_pool(h, cu)

    def splade(self, logits, ends, bias, shift, masked, canonical):
        return opool.splade_pool(logits, ends, bias, shift, masked, canonical)

    def l2(self, x):
        return opool.l2_normalize(x)

    def gdn_conv(self, x, cu, weight):
        return ogdn.causal_conv(x, cu, weight)

    def gdn_gates(self, a, b, dt_bias, neg_a):
        return ogdn.gates(a, b, dt_bias, neg_a)

    def gdn_rule(self, mixed, cu, nk, nv, dk, dv, g, beta):
        return ogdn.rule_packed(mixed, cu, nk, nv, dk, dv, g, beta)

    def gdn_gated_norm(self, core, z, weight, eps):
        return ogdn.gated_norm(core, z, weight, eps)


class HipOps:
    """The same ops through the HIP library in f32 (device tensors in and out
    of each call; the numpy glue converts)."""

    def __init__(self, inl, torch, device):
        self.inl, self.torch, self.dev = inl, torch, device
        self._tables = {}

    def _t(self, x):
        return self.torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(self.dev)

    def norm_rope(self, x, weight, eps, table=None, pos=None):
        w = self._t(weight) if weight is not None else None
        kw = {}
        if table is not None:
            cos, sin = table
            kw = dict(rows=self.torch.from_numpy(np.ascontiguousarray(pos, dtype=np.int32)).to(self.dev),
                      cos=self._t(cos), sin=self._t(sin))
        y = self.inl.norm_rope(self._t(x), weight=w, eps=eps, **kw)
        return y.cpu().numpy().astype(np.float64)

    def rope(self, x, table, pos):
        cos, sin = table
        rows = self.torch.from_numpy(np.ascontiguousarray(pos, dtype=np.int32)).to(self.dev)
        y = self.inl.norm_rope(self._t(x), rows, self._t(cos), self._t(sin), norm=False)
        return y.cpu().numpy().astype(np.float64)

    def splade(self, logits, ends, bias, shift, masked, canonical):
        offs = np.concatenate([[0], np.asarray(ends)]).astype(np.int32)
        out = self.inl.pool_splade(
            self._t(logits), self.torch.from_numpy(offs).to(self.dev), bias=self._t(bias), shift=shift,
            masked_ids=masked,
            canonical=self.torch.from_numpy(np.asarray(canonical, dtype=np.int32)).to(self.dev))
        return out.cpu().numpy()

    def attention(self, q, k, v, cu, *, causal, window, scale):
        o = self.inl.varlen_attention(self._t(q), self._t(k), self._t(v), [int(c) for c in cu],
                                      causal=causal, window=window, scale=scale)
        return o.cpu().numpy().astype(np.float64)

    def mean_pool(self, h, cu):
        cu_d = self.torch.from_numpy(np.ascontiguousarray(cu, dtype=np.int32)).to(self.dev)
        return self.inl.pool_mean(self._t(h), cu_d).cpu().numpy().astype(np.float64)

    def l2(self, x):
        return self.inl.l2_normalize(self._t(x)).cpu().numpy().astype(np.float64)

    def _cu(self, cu):
        return self.torch.from_numpy(np.ascontiguousarray(cu, dtype=np.int32)).to(self.dev)

    def gdn_conv(self, x, cu, weight):
        return self.inl.gdn_conv(self._t(x), self._cu(cu), self._t(weight)).cpu().numpy().astype(np.float64)

    def gdn_gates(self, a, b, dt_bias, neg_a):
        g, beta = self.inl.gdn_gates(self._t(a), self._t(b), self._t(dt_bias), self._t(neg_a))
        return g.cpu().numpy().astype(np.float64), beta.cpu().numpy().astype(np.float64)

    def gdn_rule(self, mixed, cu, nk, nv, dk, dv, g, beta):
        out = self.inl.gdn_rule(self._t(mixed), self._cu(cu), nk, nv, dk, dv, self._t(g), self._t(beta))
        return out.cpu().numpy().astype(np.float64)

    def gdn_gated_norm(self, core, z, weight, eps):
        out = self.inl.gdn_gated_norm(self._t(core), self._t(z), self._t(weight), eps)
        return out.cpu().numpy().astype(np.float64)


def _positions(lens):
    return np.concatenate([np.arange(n) for n in lens]) if lens else np.zeros(0, dtype=np.int64)


# ---------------------------------------------------------------------------
# EmbeddingGemma 2 (crates/inl-text/src/gemma2.rs)
# ---------------------------------------------------------------------------

def gemma2_embed(fixture, texts, max_length: int, ops):
    """Unit-length embeddings ``[B, embedding_dim]`` of the fixture's tokens
    for ``texts`` (and their lengths): ``oracle.gemma2.encode`` (the forward
    of gemma2.rs:606-662 over packed rows) with the hot-path ops routed to
    ``ops``. The reference right pads the rows and masks the padding, which
    is the same function for the real rows."""
    cfg, W, _, fdir = fixture
    ids = tokenize(fdir, texts, max_length)
    lens = [len(x) for x in ids]
    cu = oa.cu_from_lengths(lens)
    flat = np.concatenate([np.asarray(x, dtype=np.int64) for x in ids])
    return og.encode(W, cfg["text_config"], flat, cu, ops=ops, prefix="language_model."), lens


# ---------------------------------------------------------------------------
# ModernBERT MLM + SPLADE pooling (crates/inl-sparse/src/modernbert.rs)
# ---------------------------------------------------------------------------

def layer_norm(x, weight, eps):
    """candle ``LayerNorm::new_no_bias``: ``(x - mean) / sqrt(var + eps) * w``."""
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * weight


def gelu_erf(x):
    """candle ``Tensor::gelu_erf``."""
    from scipy.special import erf
    return 0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))


def modernbert_splade(fixture, rows, ops):
    """Sparse SPLADE vectors ``[(indices, values)]`` of the pre-tokenized
    ``rows``, following modernbert.rs:621-655 (embedding norm, layers with
    the identity pre-attention norm on layer 0, global layers every
    ``global_attn_every_n_layers`` with the full-attention RoPE base, local
    layers masked to ``|q - k| <= local_attention / 2``, scale
    ``head_dim^-0.5``, GeGLU MLP with erf gelu), the MLM head and tied decoder
    of :657-662 on the speaking positions (:703-716), and the pooling of
    :806-907 (row max, ``ln(1 + relu(max + bias - shift))`` with the masked
    vocabulary, canonical fold), then ``SparseVector::from_pairs``
    (crates/inl-sparse/src/lib.rs:51-62)."""
    cfg, W, _, fdir = fixture
    pool = json.loads((fdir / "pooling_config.json").read_text())
    lens = [len(r) for r in rows]
    cu = oa.cu_from_lengths(lens)
    flat = np.concatenate([np.asarray(r, dtype=np.int64) for r in rows])
    pos = _positions(lens)
    hs, heads, eps = cfg["hidden_size"], cfg["num_attention_heads"], cfg.get("norm_eps", 1e-5)
    hd, inter = hs // heads, cfg["intermediate_size"]
    n = flat.shape[0]
    emb = W["model.embeddings.tok_embeddings.weight"]
    rope = cfg["rope_parameters"]
    positions = max(lens)
    tables = {True: opro.rope_table(hd, rope["full_attention"]["rope_theta"], positions),
              False: opro.rope_table(hd, rope["sliding_attention"]["rope_theta"], positions)}
    h = layer_norm(emb[flat], W["model.embeddings.norm.weight"], eps)
    for i in range(cfg["num_hidden_layers"]):
        lp = f"model.layers.{i}."
        glob = i % cfg["global_attn_every_n_layers"] == 0
        x = h if i == 0 else layer_norm(h, W[lp + "attn_norm.weight"], eps)
        wqkv = W[lp + "attn.Wqkv.weight"]
        q = (x @ wqkv[:hs].T).reshape(n, heads, hd)
        k = (x @ wqkv[hs:2 * hs].T).reshape(n, heads, hd)
        v = (x @ wqkv[2 * hs:].T).reshape(n, heads, hd)
        q = ops.rope(q, tables[glob], pos)
        k = ops.rope(k, tables[glob], pos)
        window = -1 if glob else cfg["local_attention"] // 2
        a = ops.attention(q, k, v, cu, causal=False, window=window, scale=hd ** -0.5)
        h = h + a.reshape(n, hs) @ W[lp + "attn.Wo.weight"].T
        m = layer_norm(h, W[lp + "mlp_norm.weight"], eps)
        wi = W[lp + "mlp.Wi.weight"]
        h = h + (gelu_erf(m @ wi[:inter].T) * (m @ wi[inter:].T)) @ W[lp + "mlp.Wo.weight"].T
    h = layer_norm(h, W["model.final_norm.weight"], eps)
    index, ends = opool.speakers(rows, pool["prefix_token_ids"])
    head = layer_norm(gelu_erf(h[index] @ W["head.dense.weight"].T), W["head.norm.weight"], eps)
    logits = (head @ emb.T).astype(np.float32)
    dense = ops.splade(logits, ends, W["decoder.bias"].astype(np.float32), pool["logit_shift"],
                       pool["masked_vocab_ids"], pool["canonical_ids"])
    return [opool.sparse_from_pairs(row) for row in dense]


# ---------------------------------------------------------------------------
# Qwen3.5 late-interaction tower (crates/inl-late/src/qwen3_5.rs, native.rs)
# ---------------------------------------------------------------------------

def load_late_fixture(name: str = "tiny_qwen3_5_late"):
    """(config, weights, golden, fixture dir, dense weight [out, hidden],
    sentence-transformers prompts, lengths and mask config)."""
    from safetensors.numpy import load_file
    cfg, weights, golden, d = load_fixture(name)
    dense = load_file(str(d / "dense.safetensors"))["linear.weight"].astype(np.float64)
    st = {
        "prompts": json.loads((d / "config_sentence_transformers.json").read_text())["prompts"],
        "lengths": json.loads((d / "sentence_bert_config.json").read_text()),
        "mask": json.loads((d / "mask_config.json").read_text()),
        "dense": json.loads((d / "dense_config.json").read_text()),
    }
    return cfg, weights, golden, d, dense, st


def _zero_centred_rms(x, weight, eps):
    """Qwen3.5 RmsNorm: ``x / rms(x) * (1 + w)`` (qwen3_5.rs:189-210)."""
    return opro.rms_norm(x, 1.0 + weight, eps)


def qwen35_late_encode(fixture, texts, task: str, ops):
    """Per-token unit vectors per text, following native.rs:281-311 (prompt
    prepended, special tokens, cut to the task's length), qwen3_5.rs:893-910
    (embedding, layers, final norm) with the layer of :788-799, the gated
    delta net of :481-545 and the full attention of :302-348 (zero-centred
    q/k RMSNorm, partial half-split RoPE on the first rotary_dim features,
    bidirectional or causal per ``is_causal``, sigmoid output gate), then
    native.rs:640-689 (the Dense projection, ``x / max(|x|, 1e-12)``, the
    document skiplist). Rows are packed; the reference right pads them,
    which leaves the real rows unchanged (qwen3_5.rs:1-7)."""
    import tokenizers
    cfg, W, _, fdir, dense, st = fixture
    tc = cfg["text_config"]
    length = min(st["lengths"][f"{task}_length"], tc["max_position_embeddings"])
    tok = tokenizers.Tokenizer.from_file(str(fdir / "tokenizer.json"))
    tok.no_truncation()
    tok.no_padding()
    ids = [tok.encode(st["prompts"][task] + t, add_special_tokens=True).ids[:length] for t in texts]
    skip = []
    if task in st["mask"].get("skiplist_tasks", []):
        skip = [i for i in (tok.token_to_id(w) for w in st["mask"]["skiplist_words"]) if i is not None]
    lens = [len(x) for x in ids]
    cu = oa.cu_from_lengths(lens)
    flat = np.concatenate([np.asarray(x, dtype=np.int64) for x in ids])
    pos = _positions(lens)
    n = flat.shape[0]
    eps = tc["rms_norm_eps"]
    p = "language_model."

    def lin(x, name):
        return x @ W[p + name + ".weight"].T

    heads, kvh, hd = tc["num_attention_heads"], tc["num_key_value_heads"], tc["head_dim"]
    rot = int(hd * tc["rope_parameters"].get("partial_rotary_factor", 1.0))
    cos, sin = opro.rope_table_f32(rot, tc["rope_parameters"]["rope_theta"], max(lens))
    nk, nv = tc["linear_num_key_heads"], tc["linear_num_value_heads"]
    dk, dv = tc["linear_key_head_dim"], tc["linear_value_head_dim"]
    h = W[p + "embed_tokens.weight"][flat]
    for i, kind in enumerate(tc["layer_types"]):
        lp = f"layers.{i}."
        x = _zero_centred_rms(h, W[p + lp + "input_layernorm.weight"], eps)
        if kind == "linear_attention":
            a_ = lp + "linear_attn."
            mixed = ops.gdn_conv(lin(x, a_ + "in_proj_qkv"), cu, W[p + a_ + "conv1d.weight"][:, 0, :])
            neg_a = -np.exp(W[p + a_ + "A_log"])
            g, beta = ops.gdn_gates(lin(x, a_ + "in_proj_a"), lin(x, a_ + "in_proj_b"), W[p + a_ + "dt_bias"], neg_a)
            core = ops.gdn_rule(mixed, cu, nk, nv, dk, dv, g, beta)
            z = lin(x, a_ + "in_proj_z").reshape(n, nv, dv)
            y = ops.gdn_gated_norm(core, z, W[p + a_ + "norm.weight"], eps)
            mix = lin(y.reshape(n, nv * dv), a_ + "out_proj")
        else:
            s_ = lp + "self_attn."
            qg = lin(x, s_ + "q_proj").reshape(n, heads, 2 * hd)
            q, gate = qg[..., :hd], qg[..., hd:].reshape(n, heads * hd)
            q = _zero_centred_rms(q, W[p + s_ + "q_norm.weight"], eps)
            k = _zero_centred_rms(lin(x, s_ + "k_proj").reshape(n, kvh, hd), W[p + s_ + "k_norm.weight"], eps)
            v = lin(x, s_ + "v_proj").reshape(n, kvh, hd)
            c, s = cos[pos][:, None, :].astype(np.float64), sin[pos][:, None, :].astype(np.float64)
            q = opro.partial_rope(q, c, s, rot)
            k = opro.partial_rope(k, c, s, rot)
            a = ops.attention(q, k, v, cu, causal=bool(tc.get("is_causal", True)), window=-1, scale=hd ** -0.5)
            a = a.reshape(n, heads * hd) * (1.0 / (1.0 + np.exp(-gate)))
            mix = lin(a, s_ + "o_proj")
        h = h + mix
        m = _zero_centred_rms(h, W[p + lp + "post_attention_layernorm.weight"], eps)
        m = lin(m, lp + "mlp.gate_proj")
        m = (m / (1.0 + np.exp(-m))) * lin(_zero_centred_rms(h, W[p + lp + "post_attention_layernorm.weight"], eps),
                                          lp + "mlp.up_proj")
        h = h + lin(m, lp + "mlp.down_proj")
    h = _zero_centred_rms(h, W[p + "norm.weight"], eps)
    y = h @ dense.T
    y = y / np.maximum(np.linalg.norm(y, axis=1, keepdims=True), 1e-12)
    out = []
    for b in range(len(ids)):
        keep = [j for j, t in enumerate(ids[b]) if t not in skip]
        out.append(y[cu[b] + np.asarray(keep, dtype=np.int64)] if keep else np.zeros((0, y.shape[1])))
    return out, lens
