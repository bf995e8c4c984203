"""Pins of the gated-delta-net oracle (oracle/gdn.py), on the CPU.

- The whole tiny pplx-late tower (tests/tiny_encoders.py) against the HF
  golden vectors the reference's own test holds (crates/inl-late/tests/
  tiny_golden.rs, tolerance 1e-4): this pins the convolution, the gates, the
  rule and the gated norm as HF runs them; planted mistakes in each fail it.
- The reference's unit tests, restated on its own pseudo-random inputs
  (qwen3_5.rs:963-971 generator): the chunked rule equals the per-token
  recurrence for short, exact and partial chunks and across chunks
  (qwen3_5.rs:1063-1160); the unit-lower inverse inverts (:1163-1190).
- Closed forms: the convolution per channel equals numpy's full convolution
  cut to the causal part; the inverse equals numpy's; the op-by-op f32
  restatements of the reference kernels (the GPU checkers) agree with the
  f64 forms to rounding.
"""
import numpy as np
import pytest

from oracle import gdn as og

import tiny_encoders as te


def pseudo(n, seed):
    """qwen3_5.rs:963-971: u32 LCG, (state >> 8) / 2^24 - 0.5, as f32."""
    state = (seed * 2654435761 + 1) & 0xFFFFFFFF
    out = np.empty(n, np.float32)
    for i in range(n):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32(state >> 8) / np.float32(1 << 24) - np.float32(0.5)
    return out


@pytest.fixture(scope="module")
def late():
    return te.load_late_fixture()


def _worst(out, golden):
    assert len(out) == len(golden)
    worst = 0.0
    for a, b in zip(out, golden):
        b = np.asarray(b)
        assert a.shape == b.shape
        if a.size:
            worst = max(worst, float(np.abs(a - b).max()))
    return worst


@pytest.mark.parametrize("task", ["query", "document"])
def test_tiny_late_oracle_matches_golden(late, task):
    g = late[2]
    case = next(c for c in g["cases"] if c["task"] == task)
    out, lens = te.qwen35_late_encode(late, g["texts"], task, te.OracleOps())
    assert lens == case["lengths"]
    assert _worst(out, case["alone"]) < 1e-4
    assert _worst(out, case["batched"]) < 1e-4


class _Planted(te.OracleOps):
    def __init__(self, kind):
        self.kind = kind

    def gdn_conv(self, x, cu, w):
        if self.kind == "conv_taps_reversed":
            w = w[:, ::-1]
        return super().gdn_conv(x, cu, w)

    def gdn_gates(self, a, b, dt, neg_a):
        if self.kind == "gates_a_log":
            neg_a = -np.exp(neg_a)    # neg_a taken for A_log
        g, beta = super().gdn_gates(a, b, dt, neg_a)
        if self.kind == "no_beta":
            beta = np.ones_like(beta)
        return g, beta

    def gdn_rule(self, mixed, cu, nk, nv, dk, dv, g, beta):
        if self.kind == "rule_carries_state_across_texts":
            return og.rule_packed(mixed, [0, cu[-1]], nk, nv, dk, dv, g, beta)
        if self.kind == "kv_head_modulo":
            mixed = np.asarray(mixed)
            out = np.zeros((mixed.shape[0], nv, dv))
            for b in range(len(cu) - 1):
                a, e = cu[b], cu[b + 1]
                for h in range(nv):
                    kh = h % nk
                    out[a:e, h] = og.recurrent_rule(mixed[a:e, kh * dk:(kh + 1) * dk],
                                                    mixed[a:e, (nk + kh) * dk:(nk + kh + 1) * dk],
                                                    mixed[a:e, 2 * nk * dk + h * dv:2 * nk * dk + (h + 1) * dv],
                                                    g[a:e, h], beta[a:e, h])
            return out
        return super().gdn_rule(mixed, cu, nk, nv, dk, dv, g, beta)

    def gdn_gated_norm(self, core, z, w, eps):
        if self.kind == "norm_without_gate":
            return og.gated_norm(core, np.full_like(z, 40.0), w, eps)
        return super().gdn_gated_norm(core, z, w, eps)


@pytest.mark.parametrize("kind", ["conv_taps_reversed", "gates_a_log", "no_beta",
                                  "rule_carries_state_across_texts", "kv_head_modulo", "norm_without_gate"])
def test_tiny_late_golden_rejects_planted_mistakes(late, kind):
    g = late[2]
    case = next(c for c in g["cases"] if c["task"] == "document")
    out, _ = te.qwen35_late_encode(late, g["texts"], "document", _Planted(kind))
    assert _worst(out, case["alone"]) > 1e-3


@pytest.mark.parametrize("t", [1, 7, 8, 63, 64, 65, 145])
def test_chunked_rule_matches_recurrence_heads_and_partial_chunks(t):
    """qwen3_5.rs:1063-1122 (b=2, h=3, dk=4, dv=3)."""
    b, h, dk, dv = 2, 3, 4, 3
    q = pseudo(b * t * h * dk, 11).reshape(b, t, h, dk)
    k = pseudo(b * t * h * dk, 12).reshape(b, t, h, dk)
    v = pseudo(b * t * h * dv, 13).reshape(b, t, h, dv)
    g = (-0.3 * (pseudo(b * t * h, 14) + 0.5)).reshape(b, t, h)
    beta = (pseudo(b * t * h, 15) + 0.5).reshape(b, t, h)
    for bb in range(b):
        for hh in range(h):
            args = (q[bb, :, hh], k[bb, :, hh], v[bb, :, hh], g[bb, :, hh], beta[bb, :, hh])
            assert np.abs(og.chunked_rule(*args) - og.recurrent_rule(*args)).max() < 1e-4


def test_chunked_rule_matches_recurrence_across_chunks():
    """qwen3_5.rs:1124-1160: t = 2 * 64 + 17, dk = 8, dv = 6."""
    t, dk, dv = 2 * 64 + 17, 8, 6
    q, k = pseudo(t * dk, 1).reshape(t, dk), pseudo(t * dk, 2).reshape(t, dk)
    v = pseudo(t * dv, 3).reshape(t, dv)
    g, beta = -0.3 * (pseudo(t, 4) + 0.5), pseudo(t, 5) + 0.5
    assert np.abs(og.chunked_rule(q, k, v, g, beta) - og.recurrent_rule(q, k, v, g, beta)).max() < 1e-4


def test_rule_without_decay_or_beta_is_the_delta_rule_closed_form():
    """g = 0, beta = 1, one token: S = k v^T, out = (q.k) v with q, k unit
    (q scaled by 1/sqrt(dk)); two orthogonal keys store both values."""
    dk, dv = 4, 3
    q = np.array([[1.0, 0, 0, 0], [0, 1.0, 0, 0]])
    k = np.array([[1.0, 0, 0, 0], [0, 1.0, 0, 0]])
    v = np.array([[1.0, 2, 3], [4.0, 5, 6]])
    out = og.recurrent_rule(q, k, v, np.zeros(2), np.ones(2))
    s = 1.0 / np.sqrt(1.0 + 1e-6) ** 2 / np.sqrt(dk)
    assert np.allclose(out, v * s, atol=1e-9)


def test_unit_lower_inverse_inverts():
    """qwen3_5.rs:1163-1190 (s = 16, pseudo seed 9, upper part zeroed), plus
    numpy's inverse and the kernel-order f32 form."""
    s = 16
    a = pseudo(2 * s * s, 9).reshape(2, s, s)
    a = np.tril(a, -1)
    x = og.unit_lower_inverse(a)
    eye = np.eye(s)
    assert np.abs((eye + a) @ x - eye).max() < 1e-4
    assert np.allclose(x, np.linalg.inv(eye + a), atol=1e-9)
    x32 = og.unit_lower_inverse_ops(a)
    assert np.abs(x32 - x).max() < 1e-5
    assert np.array_equal(np.triu(x32, 1), np.zeros_like(x32)) and np.all(np.diagonal(x32, 0, 1, 2) == 1)


def test_conv_is_numpy_causal_convolution():
    rng = np.random.default_rng(3)
    lens = [5, 0, 1, 9]
    cu = np.concatenate([[0], np.cumsum(lens)])
    x = rng.standard_normal((cu[-1], 6))
    w = rng.standard_normal((6, 4))
    out = og.causal_conv(x, cu, w)
    for b in range(len(lens)):
        for c in range(6):
            seg = x[cu[b]:cu[b + 1], c]
            # tap k multiplies x[t + k - 3]: a convolution with the reversed taps
            ref = np.convolve(seg, w[c, ::-1])[:len(seg)] if len(seg) else seg
            assert np.allclose(out[cu[b]:cu[b + 1], c], og.silu(ref), atol=1e-12)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_op_sequence_forms_agree_with_f64_forms(dtype):
    rng = np.random.default_rng(4)
    cu = np.array([0, 3, 3, 20])
    x = og._r(rng.standard_normal((20, 16)).astype(np.float32), dtype)
    w = og._r((rng.standard_normal((16, 4)) * 0.5).astype(np.float32), dtype)
    tol = 1e-5 if dtype == "f32" else 0.05
    assert np.abs(og.causal_conv_ops(x, cu, w, dtype) - og.causal_conv(x, cu, w)).max() < tol
    a, b = rng.standard_normal((20, 4)).astype(np.float32), rng.standard_normal((20, 4)).astype(np.float32)
    dt, neg_a = rng.standard_normal(4).astype(np.float32), -rng.uniform(0.5, 4, 4).astype(np.float32)
    g32, b32 = og.gates_ops(a, b, dt, neg_a)
    g64, b64 = og.gates(a, b, dt, neg_a)
    assert np.abs(g32 - g64).max() < 1e-5 and np.abs(b32 - b64).max() < 1e-6
    core = rng.standard_normal((20, 4, 8)).astype(np.float32)
    z = og._r(rng.standard_normal((20, 4, 8)).astype(np.float32), dtype)
    nw = og._r((1 + 0.3 * rng.standard_normal(8)).astype(np.float32), dtype)
    assert np.abs(og.gated_norm_ops(core, z, nw, 1e-6, dtype) - og.gated_norm(core, z, nw, 1e-6, dtype)).max() < \
        (1e-5 if dtype == "f32" else 0.05)
