"""Full-size GPU checks of the prologue and the epilogues through properties
that hold at any size, on the whole config-2 workload (713 texts, 200,179
tokens, Qwen3-0.6B shape: 16 q heads / 8 kv heads x 128, hidden 1024).

- RMSNorm then RoPE: the rotation keeps each head row's L2 norm, and the
  unit-weight RMSNorm makes it sqrt(head_dim) (qwen3/mod.rs:72-90,123-159);
  position 0 is not rotated, so a text's first row equals its plain
  RMSNorm.
- Last-token pooling (qwen3/mod.rs:339-358,464-469): each text's output is
  the L2-normalised RMSNorm of its last row, which the host computes from
  the gathered rows.
- Mean pooling (gemma2.rs:647-656): a hidden state that is constant within
  each text pools to that constant.
Tolerances (f32 outputs from bf16 inputs): 1e-4 relative on the head norms,
1e-5 absolute on position 0 and the last-token vectors, 4e-5 on the means.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _lengths():
    from inl_hip import workloads
    return workloads.qwen3_op_lengths()


def test_norm_rope_keeps_head_norms_full_size(cuda, inl):
    import torch
    lens = _lengths()
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    n, heads, hd = int(cu[-1]), 16, 128
    g = torch.Generator(device=cuda).manual_seed(3)
    x = (torch.randn(n, heads, hd, generator=g, device=cuda) * 3.0).to(torch.bfloat16)
    pos = torch.from_numpy(inl.positions(cu)).to(cuda)
    c, s = inl.rope_table(hd, 1e6, int(max(lens)))
    cos, sin = torch.from_numpy(c).to(cuda), torch.from_numpy(s).to(cuda)
    print(f"full-size norm_rope: {n} tokens x {heads} heads", flush=True)
    y = inl.norm_rope(x, pos, cos, sin, out_dtype=torch.float32)
    plain = inl.norm_rope(x, out_dtype=torch.float32, rotary_dim=0)
    torch.cuda.synchronize()
    norms = torch.linalg.vector_norm(y, dim=-1).cpu().numpy()
    rel = np.abs(norms / np.sqrt(hd) - 1.0).max()
    first = torch.from_numpy(cu[:-1].astype(np.int64)).to(cuda)
    d0 = (y[first] - plain[first]).abs().max().item()
    print(f"full-size norm_rope: max rel norm err {rel:.3g}, position-0 diff {d0:.3g}", flush=True)
    assert rel <= 1e-4      # f32 output: the rotation and norm in f32
    assert d0 <= 1e-5


def test_pool_last_and_mean_full_size(cuda, inl):
    import torch
    lens = _lengths()
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    n, hidden = int(cu[-1]), 1024
    g = torch.Generator(device=cuda).manual_seed(4)
    h = torch.randn(n, hidden, generator=g, device=cuda).to(torch.bfloat16)
    w = (1.0 + 0.1 * torch.randn(hidden, generator=g, device=cuda)).to(torch.bfloat16)   # hidden's dtype
    cud = torch.from_numpy(cu).to(cuda)
    print(f"full-size pooling: {len(lens)} texts, {n} rows", flush=True)
    got = inl.pool_last(h, cud, weight=w, eps=1e-6).cpu().numpy()
    last = h[torch.from_numpy(cu[1:].astype(np.int64) - 1).to(cuda)].float().cpu().numpy().astype(np.float64)
    ww = w.float().cpu().numpy().astype(np.float64)
    r = last / np.sqrt((last * last).mean(-1, keepdims=True) + 1e-6) * ww
    exp = r / np.sqrt((r * r).sum(-1, keepdims=True) + 1e-12)
    e_last = np.abs(got - exp).max()
    # a per-text constant hidden state pools to itself
    vals = torch.randn(len(lens), hidden, generator=g, device=cuda).to(torch.bfloat16)
    text_of = torch.from_numpy(np.repeat(np.arange(len(lens)), lens)).to(cuda)
    hc = vals[text_of].contiguous()
    mean = inl.pool_mean(hc, cud).cpu().numpy()
    e_mean = np.abs(mean - vals.float().cpu().numpy()).max()
    print(f"full-size pooling: last max abs err {e_last:.3g}, mean-of-constant err {e_mean:.3g}", flush=True)
    assert e_last <= 1e-5
    assert e_mean <= 1e-5 * 4
