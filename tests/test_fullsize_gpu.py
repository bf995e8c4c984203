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


CASES = ["config2_all_in_one_launch", "qwen3_2048_causal", "gemma_window512", "modernbert_local64",
         "pplx_causal"]


def _case(name):
    """(lengths, hq, hkv, d, causal, window); built at run time, not at
    collection, so that nothing loads the library before torch."""
    from inl_hip import workloads as w
    return {
        "config2_all_in_one_launch": (w.qwen3_op_lengths(), 16, 8, 128, True, -1),
        "qwen3_2048_causal": ([2048] * 32, 16, 8, 128, True, -1),
        "gemma_window512": (w.uniform_lengths(32, 64, 8192), 3, 1, 256, False, 512),
        "modernbert_local64": (w.uniform_lengths(128, 32, 2048), 12, 12, 64, False, 64),
        "pplx_causal": ([4096] * 16, 16, 2, 256, True, -1),
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


@pytest.mark.parametrize("name", CASES)
def test_uniform_keys_give_visible_means(name, cuda, inl):
    import torch
    lengths, hq, hkv, d, causal, window = _case(name)
    n = int(sum(lengths))
    g = torch.Generator(device=cuda).manual_seed(7)
    q = torch.randn(n, hq, d, generator=g, device=cuda).to(torch.bfloat16)
    k = torch.zeros(n, hkv, d, device=cuda, dtype=torch.bfloat16)
    v = torch.randn(n, hkv, d, generator=g, device=cuda).to(torch.bfloat16)
    out = torch.full((n, hq, d), float("nan"), device=cuda, dtype=torch.float32)
    cu = [0]
    for t in lengths:
        cu.append(cu[-1] + int(t))
    print(f"full-size {name}: {len(lengths)} texts, {n} tokens", flush=True)
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
