"""GPU parity: the HIP varlen attention against the numpy oracle.

Inputs are seeded; bf16 cases compare against the float64 oracle evaluated on
the same bf16-rounded inputs. Tolerances (north star): attention output
max-abs error <= 2e-3 in bf16 (checked on f32 output, so the bound covers
the kernel's arithmetic: bf16 MFMA products, bf16 P, fp32 softmax and
accumulation) plus, for bf16 output, the output's own rounding
(half a bf16 ulp of the value); <= 1e-5 in f32 mode.
"""
import numpy as np
import pytest

from oracle import attention as oa

pytestmark = pytest.mark.gpu


def _inputs(lengths, hq, hkv, d, seed, dtype, torch, dev, scale=None, logit_std=1.0):
    """N(0,1) q/k/v; q and k RMS-normalised per head (as the prologue leaves
    them), q then scaled so that ``scale * q.k`` has std ``logit_std``."""
    rng = np.random.default_rng(seed)
    n = int(sum(lengths))
    q = rng.standard_normal((n, hq, d)).astype(np.float32)
    k = rng.standard_normal((n, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n, hkv, d)).astype(np.float32)
    q /= np.sqrt((q * q).mean(-1, keepdims=True) + 1e-6)
    k /= np.sqrt((k * k).mean(-1, keepdims=True) + 1e-6)
    if scale is not None:
        q *= np.float32(logit_std * d ** -0.5 / scale)
    ts = [torch.from_numpy(x).to(dev).to(dtype) for x in (q, k, v)]
    host = [t.float().cpu().numpy().astype(np.float64) for t in ts]
    return ts, host


def _half_ulp_bf16(x):
    # half a bf16 ulp of |x|: 2^(floor(log2|x|) - 8)
    ax = np.maximum(np.abs(x), 1e-30)
    return np.exp2(np.floor(np.log2(ax)) - 8)


CASES = [
    # (name, lengths, hq, hkv, d, causal, window, scale)
    ("qwen3_causal_gqa", [1, 2, 31, 32, 33, 64, 65, 127, 200, 300], 16, 8, 128, True, -1, 128 ** -0.5),
    ("gemma_full_gqa3", [5, 70, 129, 257], 3, 1, 256, False, -1, 1.0),
    ("gemma_sliding", [3, 100, 700, 1100], 3, 1, 256, False, 512, 1.0),
    ("modernbert_local", [1, 40, 129, 300], 12, 12, 64, False, 64, 64 ** -0.5),
    ("modernbert_global", [2, 97, 260], 12, 12, 64, False, -1, 64 ** -0.5),
    ("vision_full", [256, 256, 17], 16, 16, 64, False, -1, 1.0),
    ("qwen35_causal_d256", [1, 77, 300], 16, 2, 256, True, -1, 256 ** -0.5),
    ("causal_window", [90, 200], 4, 2, 128, True, 16, 128 ** -0.5),
    ("tiny_head_dims", [9, 13], 4, 2, 16, False, 3, 1.0),
    # Many short texts: several work units per workgroup for every persistent
    # kernel, so unit switches (the next unit's Q, K/V streams, output
    # stores) are exercised with real scores (the cases above fit one unit
    # per workgroup).
    ("d128_many_units", "many:0:300:1:260", 16, 8, 128, True, -1, 128 ** -0.5),
    ("d256_many_units_window", "many:1:160:1:400", 3, 1, 256, False, 96, 1.0),
    ("d256_many_units_full", "many:2:160:1:400", 3, 1, 256, False, -1, 1.0),
    ("d256_many_units_causal", "many:3:60:1:300", 16, 2, 256, True, -1, 256 ** -0.5),
    ("d64_many_units", "many:4:200:1:300", 12, 12, 64, False, 64, 64 ** -0.5),
]


def _lengths(spec):
    """A literal list, or "many:seed:n:lo:hi" = n seeded lengths in [lo, hi]."""
    if not isinstance(spec, str):
        return spec
    _, seed, n, lo, hi = spec.split(":")
    return [int(x) for x in np.random.default_rng(int(seed)).integers(int(lo), int(hi) + 1, int(n))]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_bf16_matches_oracle(case, cuda, inl):
    import torch
    name, lengths, hq, hkv, d, causal, window, scale = case
    lengths = _lengths(lengths)
    (q, k, v), (qh, kh, vh) = _inputs(lengths, hq, hkv, d, 1, torch.bfloat16, torch, cuda, scale)
    cu = oa.cu_from_lengths(lengths)
    ref = oa.varlen_attention(qh, kh, vh, cu, causal=causal, window=window, scale=scale)
    print(f"case={name} lengths={lengths}", flush=True)
    out32 = inl.varlen_attention(q, k, v, cu.tolist(), causal=causal, window=window,
                                 scale=scale, out_dtype=torch.float32)
    torch.cuda.synchronize()
    err = np.abs(out32.cpu().numpy().astype(np.float64) - ref)
    assert err.max() <= 2e-3, f"{name}: max abs err {err.max():.3g} (f32 out)"
    out16 = inl.varlen_attention(q, k, v, cu.tolist(), causal=causal, window=window, scale=scale)
    torch.cuda.synchronize()
    got = out16.float().cpu().numpy().astype(np.float64)
    bound = 2e-3 + _half_ulp_bf16(ref)
    assert np.all(np.abs(got - ref) <= bound), f"{name}: bf16 out beyond 2e-3 + half ulp"


F32_CASES = [c for c in CASES if c[0] in (
    "qwen3_causal_gqa", "gemma_sliding", "modernbert_local", "tiny_head_dims", "qwen35_causal_d256")]


@pytest.mark.parametrize("case", F32_CASES, ids=[c[0] for c in F32_CASES])
def test_f32_matches_oracle(case, cuda, inl):
    import torch
    name, lengths, hq, hkv, d, causal, window, scale = case
    (q, k, v), (qh, kh, vh) = _inputs(lengths, hq, hkv, d, 2, torch.float32, torch, cuda, scale)
    cu = oa.cu_from_lengths(lengths)
    ref = oa.varlen_attention(qh, kh, vh, cu, causal=causal, window=window, scale=scale)
    print(f"case={name} f32", flush=True)
    out = inl.varlen_attention(q, k, v, cu.tolist(), causal=causal, window=window, scale=scale)
    torch.cuda.synchronize()
    err = np.abs(out.cpu().numpy().astype(np.float64) - ref).max()
    assert err <= 1e-5, f"{name}: f32 max abs err {err:.3g}"


SPLIT_CASES = [
    # f32 batches small enough that the plan splits their longer query
    # blocks' key ranges over several workgroups and merges the parts.
    ("config1_like", [16, 100, 256, 37, 200, 129, 64, 250], 16, 8, 128, True, -1, 128 ** -0.5),
    ("one_long_causal", [1024], 16, 8, 128, True, -1, 128 ** -0.5),
    ("window_d64", [1500, 3], 12, 12, 64, False, 64, 64 ** -0.5),
    ("d256_causal_gqa8", [700, 5], 16, 2, 256, True, -1, 256 ** -0.5),
]


@pytest.mark.parametrize("case", SPLIT_CASES, ids=[c[0] for c in SPLIT_CASES])
def test_f32_split_key_ranges(case, cuda, inl):
    """The split plan launches more work items than the unsplit one; both
    match the oracle within 1e-5 (f32 output) and within 1e-5 plus half a
    bf16 ulp (bf16 output of f32 inputs)."""
    import torch
    name, lengths, hq, hkv, d, causal, window, scale = case
    (q, k, v), (qh, kh, vh) = _inputs(lengths, hq, hkv, d, 5, torch.float32, torch, cuda, scale)
    cu = oa.cu_from_lengths(lengths)
    mk = lambda flags: inl.make_attn_desc(cu.tolist(), hq, hkv, d, causal=causal, window=window, scale=scale,
                                          dtype="f32", out_dtype="f32", flags=flags)
    split, whole = inl.AttnPlan(mk(0)), inl.AttnPlan(mk(inl.ATTN_NO_SPLIT))
    assert split.info()["tiles"] > whole.info()["tiles"], (split.info(), whole.info())
    split.close()
    whole.close()
    ref = oa.varlen_attention(qh, kh, vh, cu, causal=causal, window=window, scale=scale)
    print(f"case={name} f32 split", flush=True)
    for flags in (0, inl.ATTN_NO_SPLIT):
        out = inl.varlen_attention(q, k, v, cu.tolist(), causal=causal, window=window, scale=scale, flags=flags)
        torch.cuda.synchronize()
        err = np.abs(out.cpu().numpy().astype(np.float64) - ref).max()
        assert err <= 1e-5, f"{name} flags={flags}: f32 max abs err {err:.3g}"
    out16 = inl.varlen_attention(q, k, v, cu.tolist(), causal=causal, window=window, scale=scale,
                                 out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    got = out16.float().cpu().numpy().astype(np.float64)
    assert np.all(np.abs(got - ref) <= 1e-5 + _half_ulp_bf16(ref)), f"{name}: bf16 output of the merge"


def test_plan_reuse_and_empty_texts(cuda, inl):
    """A plan is reusable across calls; zero-length texts own no rows."""
    import torch
    lengths = [0, 50, 0, 1, 130, 0]
    (q, k, v), (qh, kh, vh) = _inputs(lengths, 8, 4, 128, 3, torch.bfloat16, torch, cuda)
    cu = oa.cu_from_lengths(lengths)
    desc = inl.make_attn_desc(cu.tolist(), 8, 4, 128, causal=True, dtype="bf16", out_dtype="f32")
    plan = inl.AttnPlan(desc)
    ref = oa.varlen_attention(qh, kh, vh, cu, causal=True, scale=128 ** -0.5)
    for _ in range(3):
        out = torch.full((q.shape[0], 8, 128), float("nan"), device=cuda)
        plan.run(q, k, v, out)
        torch.cuda.synchronize()
        assert np.abs(out.cpu().numpy() - ref).max() <= 2e-3
    plan.close()


def test_fused_qkv_strided_rows(cuda, inl):
    """q, k, v as column slices of one fused projection output."""
    import torch
    lengths = [33, 100]
    n, hq, hkv, d = sum(lengths), 16, 8, 128
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(n, (hq + 2 * hkv) * d, generator=g).to(torch.bfloat16).to(cuda)
    q = qkv[:, : hq * d].view(n, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].view(n, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(n, hkv, d)
    cu = oa.cu_from_lengths(lengths)
    ref = oa.varlen_attention(*(t.float().cpu().numpy().astype(np.float64) for t in (q, k, v)),
                              cu, causal=True, scale=d ** -0.5)
    out = inl.varlen_attention(q, k, v, cu.tolist(), causal=True, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert np.abs(out.cpu().numpy() - ref).max() <= 2e-3


def test_config2_batch_bf16(cuda, inl):
    """The first 64-text batch of the config-2 workload (log-normal lengths,
    median 180, max 2048), causal GQA 16/8 x 128, q/k RMS-normalised N(0,1)."""
    import torch
    from inl_hip import workloads
    lengths = workloads.batches(workloads.qwen3_op_lengths())[0]
    (q, k, v), (qh, kh, vh) = _inputs(lengths, 16, 8, 128, 0, torch.bfloat16, torch, cuda)
    cu = oa.cu_from_lengths(lengths)
    ref = oa.varlen_attention(qh, kh, vh, cu, causal=True, scale=128 ** -0.5)
    out = inl.varlen_attention(q, k, v, cu.tolist(), causal=True, out_dtype=torch.float32)
    torch.cuda.synchronize()
    err = np.abs(out.cpu().numpy() - ref).max()
    print(f"config2 batch0 tokens={sum(lengths)} max abs err={err:.3g}", flush=True)
    assert err <= 2e-3


@pytest.mark.parametrize("pv_bf16", [False, True], ids=["pv_f16", "pv_bf16"])
def test_peaky_logits_bf16(pv_bf16, cuda, inl):
    """Logit std 4 (few keys carry the weight) stresses the rounding of P:
    fp16 P stays within 2e-3; the bf16-P option is bounded by 8e-3."""
    import torch
    lengths = [2, 3, 5, 17, 130]
    (q, k, v), (qh, kh, vh) = _inputs(lengths, 8, 4, 128, 7, torch.bfloat16, torch, cuda,
                                      128 ** -0.5, logit_std=4.0)
    cu = oa.cu_from_lengths(lengths)
    ref = oa.varlen_attention(qh, kh, vh, cu, causal=True, scale=128 ** -0.5)
    out = inl.varlen_attention(q, k, v, cu.tolist(), causal=True, out_dtype=torch.float32,
                               flags=inl.ATTN_PV_BF16 if pv_bf16 else 0)
    torch.cuda.synchronize()
    err = np.abs(out.cpu().numpy() - ref).max()
    print(f"peaky pv_bf16={pv_bf16} max abs err={err:.3g}", flush=True)
    assert err <= (8e-3 if pv_bf16 else 2e-3)


def test_pv_fp16_range_contract(cuda, inl):
    """The default bf16 path runs PV in fp16 (include/inl_hip.h): a value
    |v| >= 65520 becomes inf. Text 1 holds one key row of 70,000 at position
    40. By default its rows that see that key are non-finite, while the
    other texts of the batch stay within 2e-3 of the oracle. With
    INL_ATTN_PV_BF16 every row is finite. There the weights that multiply V
    are bf16-rounded P divided by the sum of the same rounded values: each
    carries at most 2u relative error (u = 2^-8, bf16's unit roundoff), so
    a row is within 2e-3 + 2^-7 * sum_j p_j |v_j| of the oracle."""
    import torch
    lengths, hq, hkv, d, scale = [70, 90, 33], 16, 8, 128, 128 ** -0.5
    (q, k, v), (qh, kh, vh) = _inputs(lengths, hq, hkv, d, 7, torch.bfloat16, torch, cuda, scale)
    cu = oa.cu_from_lengths(lengths)
    big = int(cu[1]) + 40
    v[big] = 70000.0
    vh = v.float().cpu().numpy().astype(np.float64)
    assert np.all(np.abs(vh[big]) >= 65520)
    ref = oa.varlen_attention(qh, kh, vh, cu, causal=True, scale=scale)
    mag = oa.varlen_attention(qh, kh, np.abs(vh), cu, causal=True, scale=scale)
    print("case=pv_fp16_range lengths=", lengths, flush=True)
    out = inl.varlen_attention(q, k, v, cu.tolist(), causal=True, scale=scale, out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    t1 = slice(int(cu[1]), int(cu[2]))
    others = np.r_[int(cu[0]):int(cu[1]), int(cu[2]):int(cu[3])]
    assert not np.isfinite(got[big:int(cu[2])]).any(), "rows that see the key must overflow in fp16 PV"
    assert np.abs(got[others] - ref[others]).max() <= 2e-3
    out = inl.varlen_attention(q, k, v, cu.tolist(), causal=True, scale=scale, out_dtype=torch.float32,
                               flags=inl.ATTN_PV_BF16)
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    assert np.isfinite(got).all()
    ratio = (np.abs(got - ref) / (2e-3 + 2.0 ** -7 * mag)).max()
    print(f"pv_bf16: worst error / bound = {ratio:.3f}", flush=True)
    assert ratio <= 1.0
    assert np.abs(got[t1]).max() > 1000.0  # the large key is really in play
