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


def test_splade_full_vocab_config4_planted_maxima(cuda, inl):
    """SPLADE pooling at config 4's full size: 128 texts of U[32,2048] tokens,
    every token but the first (the prefix) speaking, 135,764 speaking rows of
    f32 logits over the 50,002-term vocabulary (27.2 GB), folded onto 36,282
    canonical terms, shift 10, masked ids 50000/50001, a random bias in
    [-1, 1] (crates/inl-sparse/src/modernbert.rs:806-907).

    Planted maxima make the answer known exactly: the background logits lie
    in [-8, shift - 2], so with the bias every background term finishes at 0.
    Each row gets 64 planted terms (some masked, some folded onto the same
    canonical term), each planted at 3 of its row's positions with the
    largest value above the shift. The expected output is the oracle's
    finish and fold of the row maxima; values within 1e-6 and the active-term
    sets bit-exact, as the north star asks of f32 mode."""
    import torch
    from inl_hip import workloads
    from oracle import pooling as opl
    lens = workloads.uniform_lengths(128, 32, 2048)
    speak = np.array([t - 1 for t in lens], dtype=np.int64)
    offs = np.concatenate([[0], np.cumsum(speak)]).astype(np.int32)
    n_rows, vocab, terms, shift = len(lens), 50002, 36282, 10.0
    masked = [50000, 50001]
    rng = np.random.default_rng(21)
    canonical = np.concatenate([rng.permutation(terms), rng.integers(0, terms, vocab - terms)]).astype(np.int32)
    bias = rng.uniform(-1.0, 1.0, vocab).astype(np.float32)
    S = int(offs[-1])
    print(f"full-size splade: {n_rows} rows, {S} speaking positions x {vocab} terms", flush=True)
    logits = torch.empty((S, vocab), dtype=torch.float32, device=cuda)
    logits.uniform_(-8.0, shift - 2.0, generator=torch.Generator(device=cuda).manual_seed(5))
    m = np.full((n_rows, vocab), shift - 2.0, dtype=np.float32)   # finishes at 0 like the background
    pos_all, term_all, val_all = [], [], []
    for r in range(n_rows):
        t_pick = rng.choice(vocab, size=64, replace=False)
        t_pick[:2] = masked                                # planted but masked
        t_pick[2] = 0
        t_pick[3] = int(np.nonzero(canonical == canonical[0])[0][-1])  # shares term 0's canonical id
        t_pick = np.unique(t_pick)
        for t in t_pick:
            p = rng.choice(np.arange(offs[r], offs[r + 1]), size=min(3, int(speak[r])), replace=False)
            vals = (shift + rng.uniform(0.5, 6.0, size=len(p))).astype(np.float32)
            pos_all.append(p)
            term_all.append(np.full(len(p), t))
            val_all.append(vals)
            m[r, t] = vals.max()
    pi = torch.from_numpy(np.concatenate(pos_all)).to(cuda)
    ti = torch.from_numpy(np.concatenate(term_all)).to(cuda)
    logits[pi, ti] = torch.from_numpy(np.concatenate(val_all)).to(cuda)
    out = inl.pool_splade(logits, torch.from_numpy(offs).to(cuda), bias=torch.from_numpy(bias).to(cuda),
                          shift=shift, masked_ids=masked, canonical=torch.from_numpy(canonical).to(cuda),
                          out_dim=terms)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    del logits
    want = opl.splade_fold(opl.splade_finish(m, bias, shift, masked), canonical)
    err = float(np.abs(got - want).max())
    n_active = 0
    for r in range(n_rows):
        gi, _ = opl.sparse_from_pairs(got[r])
        wi, _ = opl.sparse_from_pairs(want[r])
        assert np.array_equal(gi, wi), f"row {r}: active sets differ"
        n_active += len(wi)
    print(f"full-size splade: max abs err {err:.3g}, {n_active} active terms", flush=True)
    assert err <= 1e-6
    assert n_active >= n_rows * 50
