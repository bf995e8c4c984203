"""Full-size GPU checks through a size-independent property.

With K = 0 every score is 0, so each query weighs its visible keys equally
and its output is the mean of their V rows, which numpy computes exactly
from prefix sums at any size. The shapes and lengths are the benchmark
configurations at full size (and the whole config-2 workload in one launch).
A tile that is skipped or run twice, a unit that is lost, or a mask, window
or text boundary that is wrong changes that mean. Unwritten rows keep a NaN
sentinel. The QK^T product itself is covered by the oracle parity tests at
smaller sizes. Tolerance: 1e-3 max-abs (f32 output; the means are O(1)).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


CASES = ["config2_all_in_one_launch", "qwen3_2048_causal", "gemma_window512", "gemma_full",
         "modernbert_local64", "modernbert_global", "pplx_causal", "vision",
         "gemma_full_long_in_mix", "pplx_causal_mix"]


def _mix(n, median, longest, seed):
    """Log-normal lengths (sigma 1) with one text of ``longest`` rows: the
    planner splits that text's (text, KV head) stream over several XCDs."""
    rng = np.random.default_rng(seed)
    lens = [int(x) for x in np.clip(rng.lognormal(np.log(median), 1.0, n), 16, longest)]
    lens[n // 3] = longest
    return lens


def _case(name):
    """(lengths, hq, hkv, d, causal, window); built at run time, not at
    collection, so that nothing loads the library before torch."""
    from inl_hip import workloads as w
    return {
        "config2_all_in_one_launch": (w.qwen3_op_lengths(), 16, 8, 128, True, -1),
        "qwen3_2048_causal": ([2048] * 32, 16, 8, 128, True, -1),
        "gemma_window512": (w.uniform_lengths(32, 64, 8192), 3, 1, 256, False, 512),
        "gemma_full": (w.uniform_lengths(32, 64, 8192), 3, 1, 256, False, -1),
        "modernbert_local64": (w.uniform_lengths(128, 32, 2048), 12, 12, 64, False, 64),
        "modernbert_global": (w.uniform_lengths(128, 32, 2048), 12, 12, 64, False, -1),
        "pplx_causal": ([4096] * 16, 16, 2, 256, True, -1),
        "vision": ([256] * 64, 16, 16, 64, False, -1),
        "gemma_full_long_in_mix": (_mix(48, 600, 8192, 100), 3, 1, 256, False, -1),
        "pplx_causal_mix": (_mix(32, 1000, 8192, 101), 16, 2, 256, True, -1),
    }[name]


def _expected_means(vh, lengths, causal, window):
    """[N, d] per KV head: mean of the visible V rows of each query (f64)."""
    n, d = vh.shape
    out = np.empty((n, d), dtype=np.float64)
    s = 0
    for t in lengths:
        if t == 0:
            continue
        c = np.zeros((t + 1, d), dtype=np.float64)
        np.cumsum(vh[s:s + t], axis=0, out=c[1:])
        i = np.arange(t)
        lo = np.zeros(t, dtype=np.int64) if window < 0 else np.maximum(0, i - window)
        hi = i if causal else np.full(t, t - 1)
        if window >= 0:
            hi = np.minimum(hi, np.minimum(t - 1, i + window))
        out[s:s + t] = (c[hi + 1] - c[lo]) / (hi - lo + 1)[:, None]
        s += t
    return out


F32_CASES = ["modernbert_local64", "modernbert_global", "qwen3_2048_causal"]


@pytest.mark.parametrize("name,dtype", [(c, "bf16") for c in CASES] + [(c, "f32") for c in F32_CASES],
                         ids=[c for c in CASES] + [c + "-f32" for c in F32_CASES])
def test_uniform_keys_give_visible_means(name, dtype, cuda, inl):
    import torch
    lengths, hq, hkv, d, causal, window = _case(name)
    n = int(sum(lengths))
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    g = torch.Generator(device=cuda).manual_seed(7)
    q = torch.randn(n, hq, d, generator=g, device=cuda).to(tdt)
    k = torch.zeros(n, hkv, d, device=cuda, dtype=tdt)
    v = torch.randn(n, hkv, d, generator=g, device=cuda).to(tdt)
    out = torch.full((n, hq, d), float("nan"), device=cuda, dtype=torch.float32)
    cu = [0]
    for t in lengths:
        cu.append(cu[-1] + int(t))
    print(f"full-size {name} {dtype}: {len(lengths)} texts, {n} tokens", flush=True)
    inl.varlen_attention(q, k, v, cu, causal=causal, window=window, scale=d ** -0.5, out=out)
    torch.cuda.synchronize()
    group = hq // hkv
    worst = 0.0
    for kv in range(hkv):
        exp = _expected_means(v[:, kv].float().cpu().numpy().astype(np.float64), lengths, causal, window)
        for h in range(kv * group, (kv + 1) * group):
            got = out[:, h].cpu().numpy()
            assert np.isfinite(got).all(), f"{name}: head {h} has unwritten or non-finite rows"
            worst = max(worst, float(np.abs(got - exp).max()))
    print(f"full-size {name}: max abs err {worst:.3g}", flush=True)
    assert worst <= 1e-3


def _sample_rows(lengths, per_text, rng):
    """Row indices per text: the first two, the middle, the last, and
    ``per_text`` more at random (all of them for short texts)."""
    rows, s = [], 0
    for t in lengths:
        if t <= per_text + 4:
            pick = np.arange(t)
        else:
            pick = np.unique(np.concatenate([[0, 1, t // 2, t - 1], rng.integers(0, t, per_text)]))
        rows.append(s + pick)
        s += t
    return rows


def _textbook_rows(qrows, kh, vh, lengths, rows, hq, hkv, causal, window, scale):
    """softmax(scale q.k) V over each sampled query's visible keys, f64, for
    every query head (head h reads KV head h // (hq/hkv)). ``qrows`` maps a
    sampled row to its f64 ``[hq, d]`` queries; ``kh``/``vh`` are the f32
    keys and values, converted to f64 one text at a time."""
    group = hq // hkv
    out = {}
    s = 0
    for t, picks in zip(lengths, rows):
        kt, vt = kh[s:s + t].astype(np.float64), vh[s:s + t].astype(np.float64)
        for r in picks:
            i = r - s
            lo = 0 if window < 0 else max(0, i - window)
            hi = i + 1 if causal else t
            if window >= 0:
                hi = min(hi, i + window + 1)
            kk, vv = kt[lo:hi], vt[lo:hi]           # [keys, hkv, d]
            for h in range(hq):
                sc = kk[:, h // group] @ qrows[r][h] * scale
                p = np.exp(sc - sc.max())
                out[(r, h)] = (p / p.sum()) @ vv[:, h // group]
        s += t
    return out


SAMPLED = [(c, "bf16") for c in ("config2_all_in_one_launch", "qwen3_2048_causal", "gemma_window512",
                                 "gemma_full", "modernbert_local64", "modernbert_global", "pplx_causal",
                                 "gemma_full_long_in_mix", "pplx_causal_mix")] + \
          [(c, "f32") for c in ("modernbert_local64", "modernbert_global")]


@pytest.mark.parametrize("name,dtype", SAMPLED, ids=[f"{c}-{d}" for c, d in SAMPLED])
def test_sampled_rows_match_textbook_full_size(name, dtype, cuda, inl):
    """Random RMS-normalised q/k and N(0,1) v at the benchmark shapes and full
    sizes, in one launch; the first, second, middle and last query of every
    text and 12 more at random are checked against the textbook softmax over
    their visible keys (f64 on the host, from the same rounded inputs):
    <= 2e-3 max-abs in bf16, <= 1e-5 in f32 (the north star's bounds)."""
    import torch
    lengths, hq, hkv, d, causal, window = _case(name)
    n = int(sum(lengths))
    scale = d ** -0.5
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    g = torch.Generator(device=cuda).manual_seed(11)

    def normed(h):
        x = torch.randn(n, h, d, generator=g, device=cuda)
        return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + 1e-6)

    q = normed(hq).to(tdt)
    k = normed(hkv).to(tdt)
    v = torch.randn(n, hkv, d, generator=g, device=cuda).to(tdt)
    out = torch.full((n, hq, d), float("nan"), device=cuda, dtype=torch.float32)
    cu = [0]
    for t in lengths:
        cu.append(cu[-1] + int(t))
    print(f"full-size sampled {name} {dtype}: {len(lengths)} texts, {n} tokens", flush=True)
    inl.varlen_attention(q, k, v, cu, causal=causal, window=window, scale=scale, out=out)
    torch.cuda.synchronize()
    rows = _sample_rows(lengths, 12, np.random.default_rng(5))
    flat_np = np.concatenate(rows)
    flat = torch.from_numpy(flat_np).to(cuda)
    qs = q[flat].float().cpu().numpy().astype(np.float64)
    qrows = {int(r): qs[j] for j, r in enumerate(flat_np)}
    kh, vh = k.float().cpu().numpy(), v.float().cpu().numpy()
    got = out[flat].cpu().numpy()
    want = _textbook_rows(qrows, kh, vh, lengths, rows, hq, hkv, causal, window, scale)
    pos = {int(r): j for j, r in enumerate(flat_np)}
    worst = max(float(np.abs(got[pos[r], h] - ref).max()) for (r, h), ref in want.items())
    print(f"full-size sampled {name} {dtype}: {len(pos)} rows x {hq} heads, max abs err {worst:.3g}", flush=True)
    assert np.isfinite(got).all()
    assert worst <= (2e-3 if dtype == "bf16" else 1e-5)
