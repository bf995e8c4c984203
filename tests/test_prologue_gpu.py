"""GPU parity of the fused RMSNorm + RoPE prologue against the numpy oracle.

Every reference form: Qwen3 q/k (weighted norm, RoPE theta 1e6, head_dim
128), EmbeddingGemma q/k (theta 1e4, head_dim 256) and the weightless v norm,
ModernBERT (RoPE only, head_dim 64), Qwen3.5 (zero-centred norm weight, partial
RoPE on 64 of 256 dims, f32-built table) and the vision tower (axial RoPE on
per-token 2-D tables). Bounds: f32 mode 1e-5 (scaled by max(1, term size)); bf16
output compared with the float64 oracle evaluated with the same
rounding points (bf16 norm output and bf16 tables, as the reference
materialises them in the model dtype), to one bf16 ulp of the rotation's
terms.
"""
import numpy as np
import pytest

from oracle import prologue as op
from oracle import attention as oa

pytestmark = pytest.mark.gpu


def _bf16(x, torch):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def _ulp_bf16(x):
    ax = np.maximum(np.abs(x), 1e-30)
    return np.exp2(np.floor(np.log2(ax)) - 7)


def _run(inl, torch, dev, x, cu, *, weight, eps, norm, theta, rotary_dim, dtype, mode=0,
         round_tables=False, round_norm=False):
    n, h, d = x.shape
    xt = torch.from_numpy(x).to(dev).to(dtype)
    xh = xt.float().cpu().numpy().astype(np.float64)
    pos = inl.positions(cu)
    maxpos = int(pos.max()) + 1 if len(pos) else 1
    rd = rotary_dim
    cos = sin = rows = None
    if rd:
        c, s = inl.rope_table(rd, theta, maxpos, mode)
        cos, sin = torch.from_numpy(c).to(dev), torch.from_numpy(s).to(dev)
        rows = torch.from_numpy(pos).to(dev)
    w = None
    if weight is not None:
        w = torch.from_numpy(weight.astype(np.float32)).to(dev).to(dtype)
    y = inl.norm_rope(xt, rows, cos, sin, weight=w, eps=eps, norm=norm, rotary_dim=rd or 0,
                      round_tables=round_tables, round_norm=round_norm)
    torch.cuda.synchronize()
    got = y.float().cpu().numpy().astype(np.float64)
    # oracle with the same rounding points; the table values are the
    # library's (their construction is checked against the oracle's tables
    # on the CPU), so only the kernel's arithmetic is compared here.
    wh = w.float().cpu().numpy().astype(np.float64) if w is not None else None
    ref = op.rms_norm(xh, wh, eps) if norm else xh
    if round_norm:
        ref = _bf16(ref, torch).astype(np.float64)
    mag = np.abs(ref)
    if rd:
        c, s = cos.cpu().numpy(), sin.cpu().numpy()
        if round_tables:
            c, s = _bf16(c, torch), _bf16(s, torch)
        cc, ss = c[pos][:, None, :].astype(np.float64), s[pos][:, None, :].astype(np.float64)
        mag = op.partial_rope(np.abs(ref), np.abs(cc), -np.abs(ss), rd)
        half = rd // 2
        mag[..., :half] = np.abs(ref[..., :half]) * np.abs(cc) + np.abs(ref[..., half:rd]) * np.abs(ss)
        mag[..., half:rd] = np.abs(ref[..., half:rd]) * np.abs(cc) + np.abs(ref[..., :half]) * np.abs(ss)
        ref = op.partial_rope(ref, cc, ss, rd)
    return got, ref, mag


CASES = [
    # name, heads, head_dim, norm, weighted, theta, rotary_dim, mode
    ("qwen3_qk", 16, 128, True, True, 1e6, 128, 0),
    ("gemma_qk_sliding", 3, 256, True, True, 1e4, 256, 0),
    ("gemma_v_weightless", 1, 256, True, False, None, 0, 0),
    ("modernbert_rope_only", 12, 64, False, False, 160000.0, 64, 0),
    ("qwen35_partial", 16, 256, True, True, 1e7, 64, 1),
    ("tiny_head_dim16", 4, 16, True, True, 1e4, 16, 0),
    ("tiny_head_dim8", 4, 8, False, False, 1e4, 8, 0),
    ("partial_rotary8", 4, 32, True, True, 1e4, 8, 0),
    # partner lanes 32 apart (v_permlane32_swap) and a 64-lane norm sum
    ("wide_head_dim512", 2, 512, True, True, 1e4, 512, 0),
    # partner lanes 3 apart: not a power of two, the shuffle path
    ("partial_rotary48", 4, 64, True, True, 1e4, 48, 0),
    # five heads of 256 (the fused q/k/v row's count): the kernel's 5-head step
    ("five_heads_256", 5, 256, True, True, 1e6, 256, 0),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("mode", ["f32", "bf16"])
def test_norm_rope_matches_oracle(case, mode, cuda, inl):
    import torch
    name, heads, hd, norm, weighted, theta, rd, tmode = case
    lengths = [1, 7, 64, 130]
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((sum(lengths), heads, hd)) * 1.5).astype(np.float32)
    weight = (1.0 + 0.2 * (rng.random(hd) - 0.5)) if weighted else None
    cu = oa.cu_from_lengths(lengths)
    dtype = torch.float32 if mode == "f32" else torch.bfloat16
    rb = mode == "bf16"
    print(f"case={name} mode={mode}", flush=True)
    got, ref, mag = _run(inl, torch, cuda, x, cu, weight=weight, eps=1e-6, norm=norm, theta=theta,
                         rotary_dim=rd, dtype=dtype, mode=tmode, round_tables=rb, round_norm=rb)
    if mode == "f32":
        err = np.abs(got - ref) / np.maximum(1.0, mag)
        assert err.max() <= 1e-5, f"{name}: {err.max():.3g}"
    else:
        # the normed value is rounded to bf16 by both sides (f32 kernel vs
        # f64 oracle may land on adjacent bf16 values: one ulp, at most 2^-7
        # relative), then the output is rounded again (half an ulp, at most
        # 2^-8 relative); relative to the sizes of the rotation's terms. The
        # f32 test checks the arithmetic to 1e-5.
        bound = (2.0 ** -7 + 2.0 ** -8) * mag + 1e-6
        assert np.all(np.abs(got - ref) <= bound), f"{name}: {np.max(np.abs(got - ref) / bound):.3g} x bound"


def test_axial_rope_vision(cuda, inl):
    """Vision tower: weighted q norm then axial RoPE from per-token 2-D
    positions (vision.rs:760-800), f32."""
    import torch
    rng = np.random.default_rng(3)
    n, heads, hd = 2 * 49, 16, 64
    x = rng.standard_normal((n, heads, hd)).astype(np.float32)
    w = (1.0 + 0.2 * (rng.random(hd) - 0.5)).astype(np.float32)
    pos_xy = np.stack(np.meshgrid(np.arange(7), np.arange(7), indexing="ij"), -1).reshape(-1, 2)
    pos_xy = np.concatenate([pos_xy, pos_xy]).astype(np.float32)
    inv = op.vision_inv_freq(hd, 100.0)
    cx, sx, cy, sy = op.axial_tables(inv, pos_xy)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    rows = torch.arange(n, dtype=torch.int32, device=cuda)
    y = inl.norm_rope(t(x), rows, t(cx), t(sx), weight=t(w), eps=1e-6, rotary_dim=hd, sections=2,
                      cos2=t(cy), sin2=t(sy))
    torch.cuda.synchronize()
    ref = op.axial_rope(op.rms_norm(x.astype(np.float64), w.astype(np.float64), 1e-6),
                        cx.astype(np.float64), sx.astype(np.float64), cy.astype(np.float64), sy.astype(np.float64))
    assert np.abs(y.cpu().numpy() - ref).max() <= 1e-5


def test_strided_rows_in_place_and_bad_position(cuda, inl):
    """q slice of a fused QKV buffer normalised in place; a token whose
    table row is out of range becomes NaN (no out-of-range read)."""
    import torch
    n, hq, hkv, d = 20, 4, 2, 128
    g = torch.Generator().manual_seed(1)
    qkv = torch.randn(n, (hq + 2 * hkv) * d, generator=g).to(cuda)
    q = qkv[:, : hq * d].view(n, hq, d)
    before = qkv.clone()
    c, s = inl.rope_table(d, 1e6, 8)
    rows = torch.tensor([i % 8 for i in range(n)], dtype=torch.int32, device=cuda)
    rows[5] = 8  # out of range
    inl.norm_rope(q, rows, torch.from_numpy(c).to(cuda), torch.from_numpy(s).to(cuda), out=q)
    torch.cuda.synchronize()
    got = q.cpu().numpy()
    assert np.isnan(got[5]).all() and not np.isnan(np.delete(got, 5, axis=0)).any()
    # k and v columns untouched
    assert torch.equal(qkv[:, hq * d:], before[:, hq * d:])
    pos = np.array([i % 8 for i in range(n)])
    ref = op.rope(op.rms_norm(before[:, : hq * d].view(n, hq, d).cpu().numpy().astype(np.float64), None, 1e-6),
                  c[pos][:, None, :].astype(np.float64), s[pos][:, None, :].astype(np.float64))
    ok = np.ones(n, bool)
    ok[5] = False
    assert np.abs(got[ok] - ref[ok]).max() <= 1e-5


@pytest.mark.parametrize("case", ["qwen3", "gemma_bf16_rounding", "k_weightless", "five_heads_256"])
def test_qk_one_launch_equals_two(case, cuda, inl):
    """inl_norm_rope_qk_fwd over the q and k heads of fused projection rows
    equals the two per-tensor launches bit for bit (the per-tensor path is
    pinned to the oracle above); in place on the fused rows, the v columns
    stay untouched; q_heads outside (0, heads) is refused."""
    import torch
    hq, hkv, d, theta, rnd = {"gemma_bf16_rounding": (3, 1, 256, 1e4, True),
                              "five_heads_256": (3, 2, 256, 1e6, True)}.get(case, (16, 8, 128, 1e6, False))
    lens = [1, 37, 200, 5, 64]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    n = int(cu[-1])
    g = torch.Generator(device=cuda).manual_seed(11)
    qkv = (torch.randn(n, (hq + 2 * hkv) * d, generator=g, device=cuda) * 1.5).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(d, generator=g, device=cuda)).to(torch.bfloat16)
    kw = None if case == "k_weightless" else (1 + 0.1 * torch.randn(d, generator=g, device=cuda)).to(torch.bfloat16)
    rows = torch.from_numpy(inl.positions(cu)).to(cuda)
    c, s = inl.rope_table(d, theta, max(lens))
    cos, sin = torch.from_numpy(c).to(cuda), torch.from_numpy(s).to(cuda)
    view = qkv.view(n, hq + 2 * hkv, d)
    kw_ = dict(eps=1e-6, round_tables=rnd, round_norm=rnd)
    print(f"case=norm_rope_qk {case} tokens={n}", flush=True)
    qo = inl.norm_rope(view[:, :hq], rows, cos, sin, weight=qw, **kw_)
    ko = inl.norm_rope(view[:, hq:hq + hkv], rows, cos, sin, weight=kw, **kw_)
    both = inl.norm_rope_qk(view[:, :hq + hkv], hq, rows, cos, sin, q_weight=qw, k_weight=kw, **kw_)
    torch.cuda.synchronize()
    assert torch.equal(both[:, :hq], qo) and torch.equal(both[:, hq:], ko)
    before = qkv.clone()
    inl.norm_rope_qk(view[:, :hq + hkv], hq, rows, cos, sin, q_weight=qw, k_weight=kw, out=view[:, :hq + hkv], **kw_)
    torch.cuda.synchronize()
    assert torch.equal(view[:, :hq], qo) and torch.equal(view[:, hq:hq + hkv], ko)
    assert torch.equal(qkv[:, (hq + hkv) * d:], before[:, (hq + hkv) * d:])
    for bad in (0, hq + hkv):
        with pytest.raises(inl.InlError):
            inl.norm_rope_qk(view[:, :hq + hkv], bad, rows, cos, sin, q_weight=qw, k_weight=kw)
