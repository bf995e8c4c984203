"""GPU parity of the pooling epilogues against the numpy oracle, including
the reference's own SPLADE known-answer cases (crates/inl-sparse/src/
modernbert.rs:1299-1393) and a bit-exact active-term set check."""
import numpy as np
import pytest

from oracle import pooling as opl
from oracle import attention as oa

pytestmark = pytest.mark.gpu


def _cu(lengths, torch, dev):
    return torch.tensor(oa.cu_from_lengths(lengths), dtype=torch.int32, device=dev)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_last_token(dtype, cuda, inl):
    import torch
    lengths = [1, 5, 0, 300, 17]
    rng = np.random.default_rng(5)
    h = 1024
    x = rng.standard_normal((sum(lengths), h)).astype(np.float32) * 3
    w = (1 + 0.2 * (rng.random(h) - 0.5)).astype(np.float32)
    td = torch.float32 if dtype == "f32" else torch.bfloat16
    xt = torch.from_numpy(x).to(cuda).to(td)
    wt = torch.from_numpy(w).to(cuda).to(td)
    out = inl.pool_last(xt, _cu(lengths, torch, cuda), weight=wt, eps=1e-6)
    torch.cuda.synchronize()
    xh = xt.float().cpu().numpy().astype(np.float64)
    wh = wt.float().cpu().numpy().astype(np.float64)
    cu = oa.cu_from_lengths(lengths)
    got = out.cpu().numpy()
    for b, t in enumerate(lengths):
        if t == 0:
            assert np.all(got[b] == 0)
            continue
        ref = opl.l2_normalize(opl.rms_norm(xh[cu[b + 1] - 1][None], wh, 1e-6))[0]
        assert np.abs(got[b] - ref).max() <= 1e-6
        assert abs(np.linalg.norm(got[b]) - 1) <= 1e-5


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_mean_and_matryoshka(dtype, cuda, inl):
    import torch
    lengths = [3, 1, 700, 0, 64]
    rng = np.random.default_rng(6)
    h = 768
    x = rng.standard_normal((sum(lengths), h)).astype(np.float32)
    td = torch.float32 if dtype == "f32" else torch.bfloat16
    xt = torch.from_numpy(x).to(cuda).to(td)
    xh = xt.float().cpu().numpy().astype(np.float64)
    cu = oa.cu_from_lengths(lengths)
    mean = inl.pool_mean(xt, _cu(lengths, torch, cuda))
    unit = inl.pool_mean(xt, _cu(lengths, torch, cuda), normalize=True)
    torch.cuda.synchronize()
    ref = opl.mean_pool(xh, cu)
    assert np.abs(mean.cpu().numpy() - ref).max() <= 2e-6
    refu = opl.l2_normalize(ref)
    assert np.abs(unit.cpu().numpy() - refu).max() <= 1e-6
    # Matryoshka: truncate to k and renormalise (native.rs:822-830)
    for k in (128, 256, 512):
        t = inl.l2_normalize(unit, k, eps_inside=0.0, skip_zero=True)
        torch.cuda.synchronize()
        want = opl.truncate_and_normalize(unit.cpu().numpy(), k)
        assert np.abs(t.cpu().numpy() - want).max() <= 1e-6


@pytest.mark.parametrize("h,dtype,sliced", [(104, "bf16", False), (100, "f32", False), (766, "bf16", True),
                                            (1024, "bf16", False)])
def test_mean_shapes_and_determinism(h, dtype, sliced, cuda, inl):
    """The vector kernel (16-byte rows: partial last column slice, f32 and
    bf16) and the generic one (a column slice of a wider buffer, rows not
    16-byte multiples), each within 2e-6 of the oracle on ragged texts,
    including a long one and an empty one; the vector kernel's result is
    bit-identical across calls (fixed summation order, no atomics)."""
    import torch
    lengths = [5, 0, 3000, 1, 257, 64]
    rng = np.random.default_rng(8)
    td = torch.float32 if dtype == "f32" else torch.bfloat16
    width = h + 2 if sliced else h
    xt = torch.from_numpy(rng.standard_normal((sum(lengths), width)).astype(np.float32)).to(cuda).to(td)
    if sliced:
        xt = xt[:, 1:h + 1]
    xh = xt.float().cpu().numpy().astype(np.float64)
    cu = _cu(lengths, torch, cuda)
    a = inl.pool_mean(xt, cu)
    b = inl.pool_mean(xt, cu)
    torch.cuda.synchronize()
    ref = opl.mean_pool(xh, oa.cu_from_lengths(lengths))
    assert np.abs(a.cpu().numpy() - ref).max() <= 2e-6
    assert torch.equal(a, b)


def _splade_gpu(inl, torch, dev, logits, rows, prefix, vocab, **kw):
    """Gather speaking positions on the host (as the reference's Speakers
    index does), then pool on the GPU."""
    idx, ends = opl.speakers(rows, prefix, seq=logits.shape[1])
    flat = logits.reshape(-1, vocab)
    packed = flat[idx] if len(idx) else np.zeros((1, vocab), np.float32)
    offs = np.concatenate([[0], ends]).astype(np.int32)
    return inl.pool_splade(torch.from_numpy(np.ascontiguousarray(packed)).to(dev),
                           torch.from_numpy(offs).to(dev), **kw)


def test_splade_known_answers(cuda, inl):
    import torch
    # shift 1: term 0 -> ln 3, term 1 absent, term 2 -> ln 4 (modernbert.rs:1299-1309)
    out = _splade_gpu(inl, torch, cuda, np.array([[[3.0, 0.5, 1.5], [0.0, 0.9, 4.0]]], np.float32),
                      [[5, 6]], [], 3, shift=1.0).cpu().numpy()
    assert abs(out[0, 0] - np.log(3)) < 1e-6 and out[0, 1] == 0 and abs(out[0, 2] - np.log(4)) < 1e-6
    # prefix position and masked term (modernbert.rs:1311-1322)
    out = _splade_gpu(inl, torch, cuda, np.array([[[50.0, 50.0, 50.0], [1.0, 0.0, 30.0]]], np.float32),
                      [[9, 5]], [9], 3, masked_ids=[2]).cpu().numpy()
    assert abs(out[0, 0] - np.log(2)) < 1e-6 and out[0, 1] == 0 and out[0, 2] == 0
    # canonical fold takes the max per term (modernbert.rs:1336-1345)
    can = torch.tensor([0, 1, 0], dtype=torch.int32, device=cuda)
    out = _splade_gpu(inl, torch, cuda, np.array([[[1.0, 5.0, 3.0]]], np.float32), [[5]], [], 3,
                      canonical=can).cpu().numpy()
    assert out.shape == (1, 2) and abs(out[0, 0] - np.log(4)) < 1e-6 and abs(out[0, 1] - np.log(6)) < 1e-6


def test_splade_random_bit_exact_active_set(cuda, inl):
    """Random logits, ragged rows, a prefix token, masked terms, a bias and a
    canonical fold: values vs the f32 oracle, active-term sets bit-exact."""
    import torch
    rng = np.random.default_rng(9)
    vocab, rows_n = 5003, 6
    rows = [list(rng.integers(0, 50, size=int(n))) for n in (1, 9, 40, 200, 3, 1)]
    rows[0] = [49]  # only the prefix token: silent row
    prefix, masked = [49], [3, 11, 4000]
    seq = max(len(r) for r in rows)
    logits = (rng.standard_normal((rows_n, seq, vocab)) * 4).astype(np.float32)
    bias = (rng.standard_normal(vocab) * 2).astype(np.float32)
    canonical = rng.integers(0, 4000, size=vocab).astype(np.int32)
    out = _splade_gpu(inl, torch, cuda, logits, rows, prefix, vocab, bias=torch.from_numpy(bias).to(cuda),
                      shift=2.0, masked_ids=masked, canonical=torch.from_numpy(canonical).to(cuda),
                      out_dim=4000).cpu().numpy()
    idx, ends = opl.speakers(rows, prefix, seq=seq)
    ref = opl.splade_pool(logits.reshape(-1, vocab)[idx], ends, bias, 2.0, masked, canonical)
    assert np.abs(out - ref).max() <= 1e-6
    for r in range(rows_n):
        gi, _ = opl.sparse_from_pairs(out[r])
        ri, _ = opl.sparse_from_pairs(ref[r])
        assert np.array_equal(gi, ri), f"row {r}: active sets differ"
    assert not out[0].any(), "a row with no speaking position pools to zero"
