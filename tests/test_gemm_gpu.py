"""GPU parity of the hand-written bf16 GEMM (inl_gemm_bf16_fwd) through the C
ABI, against a plain PyTorch fp32 reference of the same product.

bf16 inputs are exact in f32 and f64, so the reference is the f64 product of
the same bf16 values; the kernel accumulates in f32 in another order, so the
bound is a few f32 ulps of sum |x| |w| per element (1e-5 relative to the
largest |y| is far above that and far below any indexing mistake, which moves
whole rows or columns by O(1)). bf16 outputs add their own rounding (half an
ulp, 2^-9 relative).

At configuration 3's sizes (M = 139,124 packed tokens) no library GEMM runs:
sampled rows are compared against the f64 product on the CPU, and every row
is covered by a checksum: the column sums of y equal (the column sums of x)
. w^T (an exact identity of the product), computed in f64 on the CPU.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _rand(torch, dev, shape, seed, scale=1.0):
    g = torch.Generator(device=dev).manual_seed(seed)
    return (torch.randn(*shape, generator=g, device=dev) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("m,n,k,out", [
    (1, 256, 32, "f32"), (255, 256, 64, "f32"), (257, 264, 96, "bf16"), (778, 4096, 1024, "f32"),
    (1408, 2304, 768, "bf16"), (1408, 256, 768, "f32"), (1408, 768, 256, "f32"), (3001, 1280, 768, "bf16"),
    (600, 1024, 1152, "f32"), (64, 8, 32, "f32")])
def test_gemm_against_fp32(m, n, k, out, cuda, inl):
    import torch
    x = _rand(torch, cuda, (m, k), 1)
    w = _rand(torch, cuda, (n, k), 2, k ** -0.5)
    od = torch.float32 if out == "f32" else torch.bfloat16
    print(f"case=gemm m={m} n={n} k={k} out={out}", flush=True)
    y = inl.gemm_bf16(x, w, out_dtype=od)
    ref = x.double() @ w.double().T
    torch.cuda.synchronize()
    scale = ref.abs().max().item()
    err = (y.double() - ref).abs()
    if out == "f32":
        assert err.max().item() <= 1e-5 * scale, err.max().item() / scale
    else:
        assert (err <= 2.0 ** -8 * ref.abs() + 1e-5 * scale).all()


@pytest.mark.parametrize("n", [512, 200])
def test_gemm_strides_alpha_beta(n, cuda, inl):
    """Strided x, w and y rows (q/k/v-style slices of wider rows), alpha, and
    beta = 1 accumulation into f32 and into bf16 outputs; columns of y outside
    [0, n) are left untouched. n = 200 is one n-tile (the 128-row kernel
    shape), n = 512 two (the 256-row shape)."""
    import torch
    m, k = 700, 256
    xs = _rand(torch, cuda, (m, k + 72), 3)
    ws = _rand(torch, cuda, (n, k + 40), 4, k ** -0.5)
    x, w = xs[:, 8:8 + k], ws[:, :k]
    ref = x.double() @ w.double().T
    print(f"case=gemm strides alpha beta n={n}", flush=True)
    for od in (torch.float32, torch.bfloat16):
        base = torch.randn(m, n + 24, device=cuda).to(od)
        y = base.clone()
        inl.gemm_bf16(x, w, out=y[:, 16:16 + n], alpha=0.5, beta=1.0)
        torch.cuda.synchronize()
        want = base[:, 16:16 + n].double() + 0.5 * ref
        tol = 1e-5 * ref.abs().max().item() + (2.0 ** -8 * want.abs() if od == torch.bfloat16 else 0)
        assert ((y[:, 16:16 + n].double() - want).abs() <= tol).all()
        assert torch.equal(y[:, :16], base[:, :16]) and torch.equal(y[:, 16 + n:], base[:, 16 + n:])


def test_gemm_refusals(cuda, inl):
    import torch
    x = torch.zeros(4, 40, dtype=torch.bfloat16, device=cuda)
    w = torch.zeros(8, 40, dtype=torch.bfloat16, device=cuda)
    with pytest.raises(inl.InlError):
        inl.gemm_bf16(x, w)   # k = 40 is not a multiple of 32
    x = torch.zeros(4, 32, dtype=torch.bfloat16, device=cuda)
    w = torch.zeros(12, 32, dtype=torch.bfloat16, device=cuda)
    with pytest.raises(inl.InlError):
        inl.gemm_bf16(x, w)   # n = 12 is not a multiple of 8
    assert inl.gemm_bf16(x[:0], w[:8]).shape == (0, 8)


# The GEMM shapes of the configuration-3 EmbeddingGemma 2 encoder (139,124
# tokens; hidden 768, q/k/v 1280 in rows of 2304, intermediate 1152, per-layer
# input 256): (n, k, x row stride, y row stride, output dtype)
CONFIG3_GEMMS = [
    (256, 768, 768, 256, "f32"),     # per-layer-input projection slice
    (1280, 768, 768, 2304, "bf16"),  # fused q/k/v
    (768, 768, 1152, 768, "f32"),    # o_proj
    (2304, 768, 768, 2304, "bf16"),  # gate/up
    (768, 1152, 1152, 768, "f32"),   # down_proj
    (256, 768, 768, 2304, "bf16"),   # per-layer input gate
    (768, 256, 1152, 768, "f32"),    # per-layer projection
]


@pytest.mark.parametrize("n,k,xs,ys,out", CONFIG3_GEMMS)
def test_gemm_config3_shapes(n, k, xs, ys, out, cuda, inl):
    import torch
    m = 139124
    x = _rand(torch, cuda, (m, xs), 5)[:, :k]
    w = _rand(torch, cuda, (n, k), 6, k ** -0.5)
    od = torch.float32 if out == "f32" else torch.bfloat16
    y = torch.full((m, ys), float("nan"), dtype=od, device=cuda)
    print(f"case=gemm config3 n={n} k={k} xs={xs} ys={ys} out={out}", flush=True)
    inl.gemm_bf16(x, w, out=y[:, :n])
    torch.cuda.synchronize()
    yv = y[:, :n]
    assert not torch.isnan(yv).any().item()
    # sampled rows, including both ends and tile boundaries
    rows = np.unique(np.concatenate([[0, 1, 255, 256, m - 257, m - 256, m - 1],
                                     np.random.default_rng(0).integers(0, m, 400)]))
    xr = x[torch.from_numpy(rows).to(cuda)].double().cpu().numpy()
    wd = w.double().cpu().numpy()
    ref = xr @ wd.T
    got = yv[torch.from_numpy(rows).to(cuda)].double().cpu().numpy()
    scale = np.abs(ref).max()
    tol = 1e-5 * scale + (2.0 ** -8 * np.abs(ref) if out == "bf16" else 0)
    assert (np.abs(got - ref) <= tol).all(), np.abs(got - ref).max() / scale
    # every row: column sums of y against (column sums of x) . w^T in f64
    colsum_x = x.double().sum(0).cpu().numpy()
    colsum_y = yv.double().sum(0).cpu().numpy()
    want = colsum_x @ wd.T
    rel = np.abs(colsum_y - want).max() / np.abs(want).max()
    # f32 outputs: f32 accumulation only. bf16: each element's rounding is
    # random, so a column sum drifts by ~0.4 sqrt(m) ulps of a typical |y|
    # against a sum of ~sqrt(m) |y|: ~1e-3 of the largest sum. One 256-row
    # tile left at zero would move the sums by ~1e-2; unwritten elements stay
    # NaN and fail above.
    assert rel <= (1e-4 if out == "f32" else 5e-3), rel


def _gelu_tanh(v):
    return 0.5 * v * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (v + 0.044715 * v ** 3)))


@pytest.mark.parametrize("mode,m,n,k", [("geglu", 300, 200, 64), ("geglu", 3001, 1152, 768), ("geglu", 517, 96, 128),
                                        ("gelu_mul", 257, 264, 96), ("gelu_mul", 3001, 256, 768),
                                        ("gelu_mul", 130, 72, 64)])
def test_gated_gemm_against_fp64(mode, m, n, k, cuda, inl):
    """The fused GEGLU and GELU x multiplier epilogues against the f64
    product of the same bf16 values, gelu_tanh in f64: within the bf16
    output rounding (2^-8 relative) plus 1e-5 of the largest |y| (the f32
    accumulation and f32 tanh)."""
    import torch
    x = _rand(torch, cuda, (m, k), 7)
    w = _rand(torch, cuda, (2 * n if mode == "geglu" else n, k), 8, k ** -0.5)
    mul = _rand(torch, cuda, (m, n), 9) if mode == "gelu_mul" else None
    print(f"case=gated gemm {mode} m={m} n={n} k={k}", flush=True)
    y = inl.gemm_bf16_gated(x, w, mode, mul=mul)
    xd, wd = x.double().cpu().numpy(), w.double().cpu().numpy()
    if mode == "geglu":
        ref = _gelu_tanh(xd @ wd[:n].T) * (xd @ wd[n:].T)
    else:
        ref = _gelu_tanh(xd @ wd.T) * mul.double().cpu().numpy()
    got = y.double().cpu().numpy()
    tol = 2.0 ** -8 * np.abs(ref) + 1e-5 * np.abs(ref).max()
    assert (np.abs(got - ref) <= tol).all(), np.abs(got - ref).max()


@pytest.mark.parametrize("mode", ["geglu", "gelu_mul"])
def test_gated_gemm_config3_full_size(mode, cuda, inl):
    """Configuration 3's two gates at 139,124 rows (MLP: gate/up 2 x 1152
    rows of 768, output rows of 1152; per-layer input: 256 columns times the
    per-layer input rows): no row left unwritten, sampled rows within the
    bound above."""
    import torch
    m, k = 139124, 768
    n = 1152 if mode == "geglu" else 256
    x = _rand(torch, cuda, (m, k), 10)
    w = _rand(torch, cuda, (2 * n if mode == "geglu" else n, k), 11, k ** -0.5)
    mul = _rand(torch, cuda, (m, n), 12) if mode == "gelu_mul" else None
    y = torch.full((m, 1152), float("nan"), dtype=torch.bfloat16, device=cuda)
    print(f"case=gated gemm {mode} config3 full size", flush=True)
    inl.gemm_bf16_gated(x, w, mode, mul=mul, out=y[:, :n])
    torch.cuda.synchronize()
    assert not torch.isnan(y[:, :n]).any().item()
    if n < 1152:
        assert torch.isnan(y[:, n:]).all().item()
    rows = np.unique(np.concatenate([[0, 1, 255, 256, m - 1], np.random.default_rng(1).integers(0, m, 300)]))
    ri = torch.from_numpy(rows).to(cuda)
    xd, wd = x[ri].double().cpu().numpy(), w.double().cpu().numpy()
    if mode == "geglu":
        ref = _gelu_tanh(xd @ wd[:n].T) * (xd @ wd[n:].T)
    else:
        ref = _gelu_tanh(xd @ wd.T) * mul[ri].double().cpu().numpy()
    got = y[ri, :n].double().cpu().numpy()
    tol = 2.0 ** -8 * np.abs(ref) + 1e-5 * np.abs(ref).max()
    assert (np.abs(got - ref) <= tol).all(), np.abs(got - ref).max()
