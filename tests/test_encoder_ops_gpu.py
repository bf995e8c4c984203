"""GPU parity of the encoder's layer ops (include/inl_encoder.h) through the
C ABI: the hipBLASLt Linear against a plain PyTorch fp32 reference of the same
product (and the oracle's formula for the element-wise ops).

Tolerances: f32 GEMMs within 1e-5 relative to the output's scale (f32 MFMA
products, f32 accumulation in a different order); bf16 GEMMs within 2^-8
relative of the f32 reference plus the output rounding (bf16 inputs are exact
in f32, so only the accumulation order and the final rounding differ);
element-wise ops within 1e-6 (f32) or half a bf16 ulp (bf16 output).
"""
import numpy as np
import pytest

from oracle import prologue as op
from oracle import qwen3 as oq

pytestmark = pytest.mark.gpu


def _rand(torch, dev, shape, seed, scale=1.0):
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn(*shape, generator=g, device=dev) * scale


@pytest.mark.parametrize("m,n,k", [(1, 64, 32), (778, 4096, 1024), (777, 1024, 3072), (33, 6144, 1024)])
def test_linear_f32(m, n, k, cuda, inl):
    import torch
    x = _rand(torch, cuda, (m, k), 1)
    w = _rand(torch, cuda, (n, k), 2, k ** -0.5)
    print(f"case=linear_f32 m={m} n={n} k={k}", flush=True)
    y = inl.linear(x, w)
    ref = x.double() @ w.double().T
    torch.cuda.synchronize()
    err = (y.double() - ref).abs().max().item() / ref.abs().max().item()
    assert err <= 1e-5, err


@pytest.mark.parametrize("out", ["bf16", "f32_accumulate"])
def test_linear_bf16(out, cuda, inl):
    """bf16 inputs into bf16 output, and into an f32 output with beta = 1 (the
    residual-add form of the o_proj and down_proj GEMMs); strided x rows."""
    import torch
    m, n, k = 300, 1024, 2048
    xs = _rand(torch, cuda, (m, k + 64), 3).to(torch.bfloat16)
    x = xs[:, :k]
    w = _rand(torch, cuda, (n, k), 4, k ** -0.5).to(torch.bfloat16)
    ref = x.double() @ w.double().T
    print(f"case=linear_bf16 out={out}", flush=True)
    if out == "bf16":
        y = inl.linear(x, w)
        torch.cuda.synchronize()
        assert y.dtype == torch.bfloat16
        bound = 2.0 ** -8 * ref.abs() + 2.0 ** -8 * ref.abs().max() * 1e-2
        assert ((y.double() - ref).abs() <= bound + 1e-6).all()
    else:
        base = _rand(torch, cuda, (m, n), 5)
        y = base.clone()
        inl.linear(x, w, out=y, beta=1.0)
        torch.cuda.synchronize()
        err = (y.double() - (base.double() + ref)).abs().max().item()
        assert err <= 1e-4 * ref.abs().max().item(), err


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_linear_one_tuning_per_row_bucket(dtype, cuda, inl):
    """50 distinct row counts of one shape, all in the bucket (256, 512]: at
    most one timing pass for the shape, every product still exact to the
    same bound as the single-shape tests. A row count of another bucket adds
    at most one more pass; a repeated row count adds none."""
    import torch
    td = torch.float32 if dtype == "f32" else torch.bfloat16
    n, k = 640, 384   # a shape no other test uses, so its bucket starts untimed
    w = _rand(torch, cuda, (n, k), 11, k ** -0.5).to(td)
    xall = _rand(torch, cuda, (600, k), 12).to(td)
    before = inl.linear_stats()
    print(f"case=linear_buckets {dtype} stats before {before}", flush=True)
    worst = 0.0
    for m in range(300, 350):
        x = xall[:m]
        y = inl.linear(x, w, out_dtype=torch.float32)
        ref = x.double() @ w.double().T
        torch.cuda.synchronize()
        worst = max(worst, (y.double() - ref).abs().max().item() / ref.abs().max().item())
    mid = inl.linear_stats()
    assert mid["tunings"] - before["tunings"] <= 1, (before, mid)
    assert worst <= (1e-5 if dtype == "f32" else 1e-4), worst
    for m in (349, 520, 349):   # repeated: cached; 520: bucket (512, 1024]
        inl.linear(xall[:m], w, out_dtype=torch.float32)
    after = inl.linear_stats()
    print(f"case=linear_buckets {dtype} stats after {after}", flush=True)
    assert after["tunings"] - mid["tunings"] <= 1, (mid, after)
    assert after["cached_shapes"] <= 512


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_embed_rms_swiglu(dtype, cuda, inl):
    import torch
    td = torch.float32 if dtype == "f32" else torch.bfloat16
    vocab, hidden, inter, n = 500, 1024, 3072, 257
    table = _rand(torch, cuda, (vocab, hidden), 6).to(td)
    ids = torch.from_numpy(np.random.default_rng(0).integers(0, vocab, n).astype(np.int32)).to(cuda)
    print(f"case=embed_rms_swiglu {dtype}", flush=True)
    e = inl.embed(ids, table)
    torch.cuda.synchronize()
    assert e.dtype == torch.float32 and torch.equal(e, table.float()[ids.long()])
    # an id outside the vocabulary gives a NaN row, not an out-of-range read
    bad = inl.embed(torch.tensor([vocab, -1, 3], dtype=torch.int32, device=cuda), table)
    torch.cuda.synchronize()
    assert torch.isnan(bad[:2]).all() and torch.equal(bad[2], table.float()[3])

    w = (1 + 0.2 * (_rand(torch, cuda, (hidden,), 7))).to(td)
    y = inl.rms_norm_rows(e, w, eps=1e-6, out_dtype=td)
    torch.cuda.synchronize()
    ref = op.rms_norm(e.cpu().numpy().astype(np.float64), w.float().cpu().numpy().astype(np.float64), 1e-6)
    got = y.float().cpu().numpy()
    if dtype == "f32":
        assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
    else:
        assert np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-6)

    gu = _rand(torch, cuda, (n, 2 * inter), 8, 2.0).to(td)
    a = inl.swiglu(gu, inter)
    torch.cuda.synchronize()
    g64 = gu.float().cpu().numpy().astype(np.float64)
    ref = oq.silu(g64[:, :inter]) * g64[:, inter:]
    got = a.float().cpu().numpy()
    if dtype == "f32":
        assert np.abs(got - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())
    else:
        assert np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-5)


@pytest.mark.parametrize("dim", [256, 1000, 1024, 3000])
def test_rms_rows_vector_and_scalar_paths(dim, cuda, inl):
    """RMSNorm rows at every register layout (one chunk, a partial last
    chunk, four chunks, two passes), with no weight, an aligned weight (the
    4-value vector path) and a weight and output one element off alignment
    (the scalar path), in f32 and bf16."""
    import torch
    n = 37
    x = _rand(torch, cuda, (n, dim), 11)
    x64 = x.cpu().numpy().astype(np.float64)
    for td in (torch.float32, torch.bfloat16):
        big = (1 + 0.2 * _rand(torch, cuda, (dim + 8,), 12)).to(td)
        for wname, w in (("none", None), ("aligned", big[:dim]), ("offset", big[1:1 + dim])):
            w64 = np.ones(dim) if w is None else w.float().cpu().numpy().astype(np.float64)
            ref = op.rms_norm(x64, w64, 1e-6)
            outs = {"contiguous": inl.rms_norm_rows(x, w, eps=1e-6, out_dtype=td)}
            buf = torch.full((n, dim + 8), float("nan"), dtype=td, device=cuda)
            view = buf[:, 1:1 + dim]
            wdt = inl.INL_F32 if w is None else inl._dtype_code(w.dtype)
            rc = inl._rms_rows(n, dim, x.data_ptr(), x.stride(0), None if w is None else w.data_ptr(), wdt, 1e-6,
                               inl._dtype_code(td), view.data_ptr(), buf.stride(0), None)
            assert rc == 0, inl.last_error()
            outs["offset"] = view
            torch.cuda.synchronize()
            print(f"case=rms_rows dim={dim} {td} weight={wname}", flush=True)
            for oname, y in outs.items():
                got = y.float().cpu().numpy()
                if td == torch.float32:
                    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max(), (wname, oname)
                else:
                    assert np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-6), (wname, oname)
            # the padding around the offset view is untouched
            assert torch.isnan(buf[:, 0]).all() and torch.isnan(buf[:, 1 + dim:]).all()
