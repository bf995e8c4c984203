"""GPU parity of the fused SPLADE decoder + max (inl_splade_decoder_max_fwd)
and of the finish/fold on its output (inl_splade_finish_fwd), through the C
ABI.

The reference product is plain PyTorch in fp32 on the same bf16 inputs
(``head.float() @ w.float().T``, then the per-text max), i.e. the logits the
fused kernel never writes. Inputs: head ~ N(0, 1), w ~ N(0, 1/hidden) * 4, so
logits are ~N(0, 16) and the shift of 10 leaves a few active terms per text.
Tolerance on the maxima: 1e-4 absolute (both sides accumulate 768 exact
bf16 x bf16 products in f32; only the order differs, ~1e-6). The finish and
fold then go through the oracle (oracle/pooling.py) within 1e-6, and the
active terms of the fused path equal those of the unfused one (materialised
logits through inl_pool_splade_fwd) wherever the finished logit is not within
1e-4 of the threshold: the two sum the same products in different orders.
"""
import numpy as np
import pytest

from oracle import pooling as opl

pytestmark = pytest.mark.gpu


def _inputs(lengths, vocab, hidden, torch, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    S = int(sum(lengths))
    head = torch.randn(max(S, 1), hidden, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(vocab, hidden, generator=g, device=dev) * (4.0 / hidden ** 0.5)).to(torch.bfloat16)
    offs = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    return head, w, offs


def _reference_maxima(head, w, offs, torch):
    wf = w.float()
    out = torch.full((len(offs) - 1, w.shape[0]), float("-inf"), device=head.device)
    for r in range(len(offs) - 1):
        a, b = int(offs[r]), int(offs[r + 1])
        for c in range(a, b, 1024):   # bounded logits per step
            blk = head[c:min(b, c + 1024)].float() @ wf.T
            out[r] = torch.maximum(out[r], blk.max(0).values)
    return out


CASES = [
    ("ragged_small", [0, 1, 127, 128, 129, 300, 2, 1000], 5003, 768),
    ("one_chunk", [77], 512, 64),
    ("config4_full", "config4", 50002, 768),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_fused_maxima_match_fp32_product(case, cuda, inl):
    import torch
    name, lengths, vocab, hidden = case
    if lengths == "config4":
        from inl_hip import workloads
        lengths = [t - 1 for t in workloads.uniform_lengths(128, 32, 2048)]   # the prefix does not speak
    head, w, offs = _inputs(lengths, vocab, hidden, torch, cuda, 3)
    print(f"case={name}: {len(lengths)} texts, {int(offs[-1])} positions, vocab {vocab}, hidden {hidden}", flush=True)
    got = inl.splade_decoder_max(head, w, offs)
    ref = _reference_maxima(head, w, offs, torch)
    torch.cuda.synchronize()
    empty = torch.tensor([n == 0 for n in lengths], device=cuda)
    assert torch.isneginf(got[empty]).all(), "a text without speaking positions pools to -inf"
    live = ~empty
    err = (got[live] - ref[live]).abs().max().item()
    print(f"case={name}: max abs err {err:.3g}", flush=True)
    assert err <= 1e-4


def test_fused_path_equals_materialised_logits(cuda, inl):
    """Fused max + finish/fold against the unfused path (fp32 logits through
    inl_pool_splade_fwd) and the oracle: values within 1e-6, active-term sets
    equal, with a bias, masked ids (50000, 50001) and a canonical fold."""
    import torch
    lengths, vocab, hidden = [40, 0, 700, 129, 1], 50002, 768
    head, w, offs = _inputs(lengths, vocab, hidden, torch, cuda, 4)
    rng = np.random.default_rng(1)
    terms = 36282
    canonical = np.concatenate([rng.permutation(terms), rng.integers(0, terms, vocab - terms)]).astype(np.int32)
    bias = rng.uniform(-1, 1, vocab).astype(np.float32)
    can_d, bias_d = torch.from_numpy(canonical).to(cuda), torch.from_numpy(bias).to(cuda)
    kw = dict(bias=bias_d, shift=10.0, masked_ids=(50000, 50001), canonical=can_d, out_dim=terms)
    m = inl.splade_decoder_max(head, w, offs)
    fused = inl.splade_finish(m, **kw)
    logits = head[:int(offs[-1])].float() @ w.float().T
    unfused = inl.pool_splade(logits, torch.from_numpy(offs).to(cuda), **kw)
    torch.cuda.synchronize()
    mh = m.cpu().numpy()
    want = opl.splade_fold(opl.splade_finish(mh, bias, 10.0, [50000, 50001]), canonical)
    f, u = fused.cpu().numpy(), unfused.cpu().numpy()
    assert np.abs(f - want).max() <= 1e-6
    assert np.abs(f - u).max() <= 1e-4
    # active terms before the fold: equal wherever the finished logit is not
    # within 1e-4 of the threshold (the two paths sum in different orders)
    um = torch.stack([logits[int(offs[r]):int(offs[r + 1])].max(0).values if lengths[r] else
                      torch.full((vocab,), float("-inf"), device=cuda) for r in range(len(lengths))]).cpu().numpy()
    x_f, x_u = mh + bias - 10.0, um + bias - 10.0
    clear = np.abs(x_u) > 1e-4
    open_ = np.ones(vocab, bool)
    open_[[50000, 50001]] = False
    act_f, act_u = (x_f > 0) & open_, (x_u > 0) & open_
    assert np.array_equal(act_f[clear], act_u[clear])
    assert not f[1].any() and act_f.sum() > 50
