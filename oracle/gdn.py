"""Gated DeltaNet oracle (numpy): the linear-attention layers of the
reference's Qwen3.5 late-interaction encoder. TEST INFRASTRUCTURE ONLY -
never on the product path.

It restates crates/inl-late/src/qwen3_5.rs:
- ``causal_conv`` (:465-479): depthwise convolution with ``taps - 1`` zeros
  of left padding, cut to the input length, then silu; per packed text here
  (each text starts from zeros, as each row of the reference's batch does);
- the gates (:494-500): ``beta = sigmoid(b)``, ``g = softplus(a + dt_bias) *
  neg_a``, ``neg_a = -exp(A_log)`` (:452), with ``softplus(x) = relu(x) +
  log(1 + exp(-|x|))`` (:546-551);
- ``l2norm`` (:553-557): ``x / sqrt(sum(x^2) + 1e-6)``;
- the per-token gated delta rule (its tests' ``recurrent``, :975-1010, and
  late.metal:172-197), state ``[dk, dv]`` from zero per text and head;
- ``chunk_gated_delta_rule`` (:607-728), the chunked form the reference runs,
  restated to pin the per-token form the way the reference's own tests do;
- ``unit_lower_inverse`` (:733-760, late.metal:32-93);
- the gated RMSNorm (:519-534).
"""
from __future__ import annotations

import numpy as np


def silu(x):
    return x / (1.0 + np.exp(-x))


def softplus(x):
    """qwen3_5.rs:546-551."""
    return np.maximum(x, 0.0) + np.log1p(np.exp(-np.abs(x)))


def l2norm(x, eps=1e-6):
    """qwen3_5.rs:553-557 (the FLA l2norm), over the last axis."""
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + eps)


def causal_conv(x, cu_seqlens, weight):
    """``silu(conv1d(x))`` per text: ``x [N, C]`` packed rows, ``weight
    [C, K]``; output row t of a text is ``silu(sum_k x[t + k - (K-1)] *
    w[:, k])`` with rows before the text's start read as zero."""
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(weight, dtype=np.float64)
    K = w.shape[1]
    out = np.zeros_like(x)
    cu = np.asarray(cu_seqlens)
    for b in range(len(cu) - 1):
        seg = x[cu[b]:cu[b + 1]]
        t = len(seg)
        padded = np.concatenate([np.zeros((K - 1, x.shape[1])), seg], 0)
        acc = np.zeros((t, x.shape[1]))
        for k in range(K):
            acc = acc + padded[k:k + t] * w[:, k]
        out[cu[b]:cu[b + 1]] = silu(acc)
    return out


def gates(a, b, dt_bias, neg_a):
    """``(g, beta)`` from the a/b projections ``[N, nv]`` (qwen3_5.rs:494-500);
    ``neg_a = -exp(A_log)`` per value head, as the reference stores it
    (qwen3_5.rs:452)."""
    beta = 1.0 / (1.0 + np.exp(-np.asarray(b, dtype=np.float64)))
    g = softplus(np.asarray(a, dtype=np.float64) + np.asarray(dt_bias, dtype=np.float64)) * \
        np.asarray(neg_a, dtype=np.float64)
    return g, beta


def recurrent_rule(q, k, v, g, beta):
    """The per-token gated delta rule of one sequence and head: ``q, k
    [T, dk]`` (raw: normalised here), ``v [T, dv]``, ``g, beta [T]``;
    returns ``[T, dv]`` (qwen3_5.rs:975-1010)."""
    T, dk = q.shape
    dv = v.shape[1]
    qn = l2norm(np.asarray(q, dtype=np.float64)) / np.sqrt(dk)
    kn = l2norm(np.asarray(k, dtype=np.float64))
    state = np.zeros((dk, dv))
    out = np.zeros((T, dv))
    for i in range(T):
        state *= np.exp(g[i])
        mem = kn[i] @ state
        delta = (v[i] - mem) * beta[i]
        state += np.outer(kn[i], delta)
        out[i] = qn[i] @ state
    return out


def chunked_rule(q, k, v, g, beta, chunk=64):
    """qwen3_5.rs:607-728 for one sequence and head (no initial state), in
    f64: per chunk, ``(I + A)^-1`` of the strictly lower ``A = (k_beta k^T) o
    decay``, the intra-chunk attention and the carried state."""
    T, dk = q.shape
    dv = v.shape[1]
    c = max(1, min(chunk, 1 << (max(T, 1) - 1).bit_length()))
    pad = (c - T % c) % c
    qn = np.pad(l2norm(np.asarray(q, np.float64)) / np.sqrt(dk), ((0, pad), (0, 0)))
    kn = np.pad(l2norm(np.asarray(k, np.float64)), ((0, pad), (0, 0)))
    vv = np.pad(np.asarray(v, np.float64), ((0, pad), (0, 0)))
    gg = np.pad(np.asarray(g, np.float64), (0, pad))
    bb = np.pad(np.asarray(beta, np.float64), (0, pad))
    lower = np.tril(np.ones((c, c)))
    strict = np.tril(np.ones((c, c)), -1)
    out = []
    state = None
    for s in range(0, T + pad, c):
        qc, kc, vc, gc, bc = qn[s:s + c], kn[s:s + c], vv[s:s + c], gg[s:s + c], bb[s:s + c]
        cum = np.cumsum(gc)
        decay = np.exp(np.minimum(cum[:, None] - cum[None, :], 0.0)) * lower
        kb, vb = kc * bc[:, None], vc * bc[:, None]
        inv = unit_lower_inverse((kb @ kc.T) * decay * strict)
        values = inv @ vb
        intra = (qc @ kc.T) * decay
        if state is None:
            v_new = values
            o = intra @ v_new
        else:
            k_cumdecay = inv @ (kb * np.exp(cum)[:, None])
            v_new = values - k_cumdecay @ state
            o = (qc * np.exp(cum)[:, None]) @ state + intra @ v_new
        out.append(o)
        last = cum[-1]
        update = (kc * np.exp(last - cum)[:, None]).T @ v_new
        state = update if state is None else state * np.exp(last) + update
    return np.concatenate(out, 0)[:T]


def unit_lower_inverse(a):
    """``(I + A)^-1`` for strictly lower-triangular ``a [..., S, S]`` by forward
    substitution, one column at a time (late.metal:32-93)."""
    a = np.asarray(a, dtype=np.float64)
    s = a.shape[-1]
    x = np.zeros_like(a)
    for j in range(s):
        col = np.zeros(a.shape[:-1])
        col[..., j] = 1.0
        for i in range(j + 1, s):
            col[..., i] = -(a[..., i, j:i] * col[..., j:i]).sum(-1)
        x[..., :, j] = col
    return x


def round_to(x, dtype):
    """Round to the model dtype (bf16: round to nearest even) and back."""
    if dtype == "f32":
        return np.asarray(x, np.float32).astype(np.float64)
    f = np.asarray(x, np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return u.astype(np.uint32).view(np.float32).astype(np.float64)


def gated_norm(core, z, weight, eps, dtype="f32"):
    """qwen3_5.rs:519-534 per row of ``dv``: the rule's output rounded to the
    model dtype, normalised in f32, rounded, times the weight (rounded), times
    ``silu(z)`` in f32, rounded."""
    c = round_to(core, dtype)
    var = (c * c).mean(-1, keepdims=True)
    normed = round_to(c / np.sqrt(var + eps), dtype)
    scaled = round_to(normed * np.asarray(weight, np.float64), dtype)
    return round_to(scaled * silu(np.asarray(z, np.float64)), dtype)


def rule_packed(mixed, cu_seqlens, nk, nv, dk, dv, g, beta):
    """The delta rule over packed texts: ``mixed [N, 2 nk dk + nv dv]`` (the
    conv output: q heads, k heads, v heads), ``g, beta [N, nv]``; value head h
    reads key head ``h // (nv // nk)`` (qwen3_5.rs:510-520). Returns
    ``[N, nv, dv]``."""
    mixed = np.asarray(mixed, np.float64)
    cu = np.asarray(cu_seqlens)
    rep = nv // nk
    out = np.zeros((mixed.shape[0], nv, dv))
    for b in range(len(cu) - 1):
        a, e = cu[b], cu[b + 1]
        if e == a:
            continue
        for h in range(nv):
            kh = h // rep
            q = mixed[a:e, kh * dk:(kh + 1) * dk]
            k = mixed[a:e, (nk + kh) * dk:(nk + kh + 1) * dk]
            v = mixed[a:e, 2 * nk * dk + h * dv:2 * nk * dk + (h + 1) * dv]
            out[a:e, h] = recurrent_rule(q, k, v, g[a:e, h], beta[a:e, h])
    return out


# ---------------------------------------------------------------------------
# The reference kernels' operation sequences, every step rounded as they
# round it (numpy float32 arithmetic is IEEE; bf16 rounding is emulated).
# ---------------------------------------------------------------------------

def _r(x, dtype):
    """Round float32 values to the model dtype, staying float32."""
    x = np.asarray(x, np.float32)
    if dtype == "f32":
        return x
    u = x.view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return u.astype(np.uint32).view(np.float32)


def causal_conv_ops(x, cu_seqlens, weight, dtype="f32"):
    """late.metal:131-151 (and the candle op sequence of qwen3_5.rs:465-479):
    per tap in order, ``term = T(sample * w)``, ``acc = T(acc + term)``, then
    silu with every step in T: ``x / (1 + exp(-x))``. x, weight hold values
    of dtype T; returns float32 values of T."""
    x = _r(x, dtype)
    w = _r(weight, dtype)
    K = w.shape[1]
    out = np.zeros_like(x)
    cu = np.asarray(cu_seqlens)
    for b in range(len(cu) - 1):
        seg = x[cu[b]:cu[b + 1]]
        t = len(seg)
        padded = np.concatenate([np.zeros((K - 1, x.shape[1]), np.float32), seg], 0)
        acc = np.zeros((t, x.shape[1]), np.float32)
        for k in range(K):
            term = _r(padded[k:k + t] * w[:, k], dtype)
            acc = _r(acc + term, dtype)
        e = _r(np.exp(_r(-acc, dtype)), dtype)
        out[cu[b]:cu[b + 1]] = _r(acc / _r(np.float32(1) + e, dtype), dtype)
    return out


def gates_ops(a, b, dt_bias, neg_a):
    """qwen3_5.rs:494-500 in float32: ``beta = 1 / (1 + exp(-b))``,
    ``g = (relu(a + dt) + log(exp(-|a + dt|) + 1)) * neg_a``."""
    a = np.asarray(a, np.float32) + np.asarray(dt_bias, np.float32)
    tail = np.log(np.exp(-np.abs(a)) + np.float32(1))
    g = (np.maximum(a, np.float32(0)) + tail) * np.asarray(neg_a, np.float32)
    beta = np.float32(1) / (np.exp(-np.asarray(b, np.float32)) + np.float32(1))
    return g.astype(np.float32), beta.astype(np.float32)


def gated_norm_ops(core, z, weight, eps, dtype="f32"):
    """late.metal:315-352 on rows of the last axis: ``c = T(core)``,
    ``var = sum(c^2) * (1 / dv)``, ``n = T(c / sqrt(var + eps))``,
    ``s = T(n * w)``, ``out = T(s * (z / (1 + exp(-z))))`` in float32 (the sum
    of squares in float64 here; the kernels' orders differ by rounding)."""
    c = _r(core, dtype)
    dv = c.shape[-1]
    var = np.float32((c.astype(np.float64) ** 2).sum(-1, keepdims=True).astype(np.float32)) * \
        (np.float32(1) / np.float32(dv))
    scale = np.sqrt(var.astype(np.float32) + np.float32(eps)).astype(np.float32)
    n = _r(c / scale, dtype)
    s = _r(n * _r(weight, dtype), dtype)
    zf = _r(z, dtype)
    sz = zf / (np.float32(1) + np.exp(-zf))
    return _r(s * sz, dtype)


def unit_lower_inverse_ops(a):
    """late.metal:64-91 in float32: column j, rows i > j:
    ``x[i] = -(sum over k = j .. i-1, ascending, of f32(A[i, k] * x[k]))``.
    Vectorised over matrices and columns; ``a [n, S, S]``."""
    a = np.asarray(a, np.float32)
    n, s, _ = a.shape
    x = np.zeros((n, s, s), np.float32)       # x[m, i, j]
    cols = np.arange(s)
    for i in range(s):
        acc = np.zeros((n, s), np.float32)
        for k in range(i):
            prod = a[:, i, k][:, None] * x[:, k, :]
            acc = np.where(cols[None, :] <= k, acc + prod, acc).astype(np.float32)
        x[:, i, :] = np.where(cols[None, :] == i, np.float32(1),
                              np.where(cols[None, :] < i, -acc, np.float32(0)))
    return x
