"""Configuration 3 at full size (32 texts of U[64, 8192] tokens = 139,124) in
the EmbeddingGemma 2 runner's own buffer layout, one launch kind at a time:
q/k/v are strided slices of one fused QKV row of 2304 bf16 (q 3 x 256 at
column 0, k at 768, v at 1024), the attention output goes to rows of 1152
bf16, and the prologue runs in place on those rows with the runner's RoPE
tables (8192 positions, θ 1e4 for sliding and 1e6 for full layers).

Checks are size-independent properties and sampled rows:
- attention with K = 0 gives each query the mean of its visible V rows
  (exact from prefix sums in f64); unwritten rows keep a NaN sentinel and
  columns outside the output slice must stay untouched. Tolerance 1e-3 plus
  the bf16 rounding of the output (2^-8 relative);
- attention on RMS-normalised random q/k: sampled queries of every text
  against the textbook softmax over their visible keys in f64, <= 2e-3
  (plus the bf16 output rounding), the north star's bf16 bound;
- the prologue: sampled rows of every text against the oracle's RMSNorm and
  RoPE (f64) on the same bf16 inputs, within the bf16 output rounding; the
  rows outside the rotated slices unchanged.
"""
import numpy as np
import pytest

from oracle import prologue as opro

pytestmark = pytest.mark.gpu

QKV_W, O_W, HQ, HKV, D = 2304, 1152, 3, 1, 256


def _lengths():
    from inl_hip import workloads as w
    return w.uniform_lengths(32, 64, 8192)


def _cu(lengths):
    cu = [0]
    for t in lengths:
        cu.append(cu[-1] + int(t))
    return cu


def _views(A, B, n):
    q = A[:, 0:HQ * D].view(n, HQ, D)
    k = A[:, HQ * D:(HQ + HKV) * D].view(n, HKV, D)
    v = A[:, (HQ + HKV) * D:(HQ + 2 * HKV) * D].view(n, HKV, D)
    o = B[:, 0:HQ * D].view(n, HQ, D)
    return q, k, v, o


def _expected_means(vh, lengths, window):
    n, d = vh.shape
    out = np.empty((n, d), dtype=np.float64)
    s = 0
    for t in lengths:
        c = np.zeros((t + 1, d), dtype=np.float64)
        np.cumsum(vh[s:s + t], axis=0, out=c[1:])
        i = np.arange(t)
        lo = np.zeros(t, dtype=np.int64) if window < 0 else np.maximum(0, i - window)
        hi = np.full(t, t - 1) if window < 0 else np.minimum(t - 1, i + window)
        out[s:s + t] = (c[hi + 1] - c[lo]) / (hi - lo + 1)[:, None]
        s += t
    return out


@pytest.mark.parametrize("window", [512, -1], ids=["sliding512", "full"])
def test_runner_layout_attention_uniform_keys(window, cuda, inl):
    import torch
    lengths = _lengths()
    cu = _cu(lengths)
    n = cu[-1]
    g = torch.Generator(device=cuda).manual_seed(21)
    A = torch.randn(n, QKV_W, generator=g, device=cuda).to(torch.bfloat16)
    A[:, HQ * D:(HQ + HKV) * D] = 0          # K = 0: uniform weights over the visible keys
    B = torch.full((n, O_W), float("nan"), device=cuda, dtype=torch.bfloat16)
    q, k, v, o = _views(A, B, n)
    print(f"case=gemma2 runner-layout attention uniform keys window={window} tokens={n}", flush=True)
    inl.varlen_attention(q, k, v, cu, causal=False, window=window, scale=1.0, out=o)
    torch.cuda.synchronize()
    exp = _expected_means(v[:, 0].float().cpu().numpy().astype(np.float64), lengths, window)
    worst = 0.0
    for h in range(HQ):
        got = o[:, h].float().cpu().numpy().astype(np.float64)
        assert np.isfinite(got).all(), f"head {h}: unwritten or non-finite rows"
        err = np.abs(got - exp) - 2.0 ** -8 * np.abs(exp)
        worst = max(worst, float(err.max()))
    assert torch.isnan(B[:, HQ * D:]).all().item(), "columns past the output slice were written"
    print(f"case=gemma2 runner-layout uniform keys window={window}: worst excess {worst:.3g}", flush=True)
    assert worst <= 1e-3


@pytest.mark.parametrize("window", [512, -1], ids=["sliding512", "full"])
def test_runner_layout_attention_sampled_rows(window, cuda, inl):
    import torch
    lengths = _lengths()
    cu = _cu(lengths)
    n = cu[-1]
    g = torch.Generator(device=cuda).manual_seed(22)
    A = torch.randn(n, QKV_W, generator=g, device=cuda)
    for lo, hi in ((0, HQ * D), (HQ * D, (HQ + HKV) * D)):
        x = A[:, lo:hi].view(n, -1, D)
        A[:, lo:hi] = (x * torch.rsqrt((x * x).mean(-1, keepdim=True) + 1e-6)).reshape(n, hi - lo)
    A = A.to(torch.bfloat16)
    B = torch.full((n, O_W), float("nan"), device=cuda, dtype=torch.bfloat16)
    q, k, v, o = _views(A, B, n)
    print(f"case=gemma2 runner-layout attention sampled rows window={window} tokens={n}", flush=True)
    inl.varlen_attention(q, k, v, cu, causal=False, window=window, scale=1.0, out=o)
    torch.cuda.synchronize()
    rng = np.random.default_rng(6)
    kh = k[:, 0].float().cpu().numpy().astype(np.float64)
    vh = v[:, 0].float().cpu().numpy().astype(np.float64)
    worst = 0.0
    for b, t in enumerate(lengths):
        s = cu[b]
        picks = np.unique(np.concatenate([[0, 1, t // 2, t - 1], rng.integers(0, t, 6)]))
        rows = torch.from_numpy(s + picks).to(cuda)
        qs = q[rows].float().cpu().numpy().astype(np.float64)
        got = o[rows].float().cpu().numpy().astype(np.float64)
        for j, i in enumerate(picks):
            lo = 0 if window < 0 else max(0, i - window)
            hi = t if window < 0 else min(t, i + window + 1)
            kk, vv = kh[s + lo:s + hi], vh[s + lo:s + hi]
            for h in range(HQ):
                sc = kk @ qs[j, h]
                p = np.exp(sc - sc.max())
                want = (p / p.sum()) @ vv
                worst = max(worst, float((np.abs(got[j, h] - want) - 2.0 ** -8 * np.abs(want)).max()))
    print(f"case=gemma2 runner-layout sampled window={window}: worst excess {worst:.3g}", flush=True)
    assert worst <= 2e-3


def test_runner_layout_prologue_in_place(cuda, inl):
    """q (3 heads, weight), k (1 head, weight) and v (weightless, no rope) of
    the fused rows normalised and rotated in place, as the runner calls it."""
    import torch
    lengths = _lengths()
    cu = np.asarray(_cu(lengths), dtype=np.int32)
    n = int(cu[-1])
    g = torch.Generator(device=cuda).manual_seed(23)
    A = (torch.randn(n, QKV_W, generator=g, device=cuda) * 2.0).to(torch.bfloat16)
    before = A.clone()
    qw = (0.25 * (1 + 0.05 * torch.randn(D, generator=g, device=cuda))).to(torch.bfloat16)
    kw = (0.25 * (1 + 0.05 * torch.randn(D, generator=g, device=cuda))).to(torch.bfloat16)
    pos = torch.from_numpy(inl.positions(cu)).to(cuda)
    c_np, s_np = inl.rope_table(D, 1e4, 8192)
    cos, sin = torch.from_numpy(c_np).to(cuda), torch.from_numpy(s_np).to(cuda)
    q, k, v, _ = _views(A, A, n)
    print(f"case=gemma2 runner-layout prologue in place tokens={n}", flush=True)
    inl.norm_rope(q, pos, cos, sin, weight=qw, eps=1e-6, out=q, round_tables=True, round_norm=True)
    inl.norm_rope(k, pos, cos, sin, weight=kw, eps=1e-6, out=k, round_tables=True, round_norm=True)
    inl.norm_rope(v, eps=1e-6, out=v, rotary_dim=0, round_norm=True)
    torch.cuda.synchronize()
    assert torch.equal(A[:, (HQ + 2 * HKV) * D:], before[:, (HQ + 2 * HKV) * D:])
    rng = np.random.default_rng(7)
    picks = np.unique(np.concatenate([cu[:-1], cu[1:] - 1, rng.integers(0, n, 2000)]))
    rows = torch.from_numpy(picks.astype(np.int64)).to(cuda)
    src = before[rows].float().cpu().numpy().astype(np.float64)
    got = A[rows].float().cpu().numpy().astype(np.float64)
    p = inl.positions(cu)[picks]
    # the oracle's f64 norm and rope on the same bf16 inputs; the runner's
    # bf16 mode rounds the tables and the normed values to bf16 as the
    # reference does, so the bound is a few bf16 ulps of each output
    tc = c_np.astype(np.float64)[p][:, None, :]
    ts = s_np.astype(np.float64)[p][:, None, :]
    worst = 0.0
    for lo, heads, w, rot in ((0, HQ, qw, True), (HQ * D, HKV, kw, True), ((HQ + HKV) * D, HKV, None, False)):
        x = src[:, lo:lo + heads * D].reshape(-1, heads, D)
        wt = None if w is None else w.float().cpu().numpy().astype(np.float64)
        y = opro.rms_norm(x, wt, 1e-6)
        if rot:
            y = opro.rope(y, tc, ts)
        gv = got[:, lo:lo + heads * D].reshape(-1, heads, D)
        scale = np.abs(y).max(axis=-1, keepdims=True)
        worst = max(worst, float((np.abs(gv - y) / scale).max()))
    print(f"case=gemma2 runner-layout prologue: worst error / row max {worst:.3g}", flush=True)
    assert worst <= 2.0 ** -6
