#!/usr/bin/env python3
"""Benchmark of the encoder attention hot path on one MI355X.

Default workload (the metric's configuration):
packed variable-length causal GQA attention at the Qwen3-0.6B shape
(16 query heads, 8 KV heads, head_dim 128, bf16), 713 texts with log-normal
lengths (median 180, sigma 1.0, max 2048; 200,179 tokens) in 12 batches of
64 texts. Q/K/V are N(0,1) after a seeded RMSNorm. A step is one pass of
the attention op over all 12 batches (12 launches, one plan per batch built
before timing, as an engine builds one per batch and reuses it for every
layer).

Prints one JSON line: attention-op tokens/s (value: tokens through one
attention layer per second), attention TFLOP/s, the roofline of the
attention kernel and the CPU baseline. The roofline divides the algorithmic
work of one launch (FLOPs: 4 * head_dim per visible (q, k) pair per query
head; HBM bytes: Q, K, V read once and O written once) by the average launch
time from HIP events on the launch stream (a separate pass, each step queued
behind a GPU sleep so that the events bracket back-to-back kernels; the
wall-clock pass has no sleep). `bound` is "mfma": attention is
graded against the 2516.6 TFLOP/s bf16 dense MFMA peak, with the 8 TB/s HBM
figure under `other`. `traffic` is the measured HBM bytes per launch from
the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary for the workload. The
CPU baseline is the oracle's multi-threaded f32 C restatement of the
reference CPU flash path, timed on a bounded sample of the same workload.

Other attention workloads (--workload): gemma_window, gemma_full,
modernbert_local, modernbert_global, vision, pplx_causal, qwen3_2048,
qwen3_2048_full - reported the same way, and each of them in f32 with an
`_f32` suffix (e.g. `qwen3_f32`: the f32 kernel against the 157.3 TFLOP/s
fp32 matrix peak). Op workloads (--workload norm_rope, norm_rope_qk,
pool_last, pool_mean, splade, gdn_conv, gdn_gated_norm) time the prologue,
epilogue and gated-delta-net element-wise kernels at their configurations'
full sizes against the 8 TB/s HBM roofline; splade_decoder (a GEMM) against
the bf16 MFMA peak and gdn_rule (f32 vector work) against the 157.3 TFLOP/s
fp32 vector peak. The
end-to-end workloads (--workload qwen3_e2e, f32 as configuration 1, and
qwen3_e2e_bf16) time a whole Qwen3-0.6B encode of 8 texts (778 tokens) and
report encoded tokens/s, with the numpy f32 forward as the CPU baseline;
--workload gemma_e2e does the same for configuration 3 (the
EmbeddingGemma-2 text tower, bf16, 32 texts of U[64,8192] tokens, every GEMM
on the library's own bf16 kernel); its CPU leg also checks three of the
timed batch's texts against the oracle. The default line nests the
configuration-1 end-to-end measurement (f32, a new 8-text draw every step)
under `e2e_config1`; --workload gemm times one configuration-3 layer's GEMMs
on the library's bf16 kernel. --stream-reference times torch's own streaming
kernels (copy, in-place add, fill, sum over 1 and 4 GiB): what a plain
element-wise kernel reaches on the GPU's HBM, next to the 8 TB/s peak.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "im-not-llm_amd"))

METRIC = "encoded tokens/sec + attention TFLOP/s (% bf16 MFMA peak), Qwen3-0.6B-shape"
PEAK_BF16_TFLOPS = 2516.6   # 256 CU x 2.4 GHz x 4096 flop/clk/CU, dense
PEAK_HBM_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def workload(name: str):
    """(lengths per batch, h_q, h_kv, head_dim, causal, window, scale, label)."""
    from inl_hip import workloads as w
    if name == "qwen3":
        lens = w.qwen3_op_lengths()
        return (w.batches(lens, 64), 16, 8, 128, True, -1, 128 ** -0.5,
                "config2: packed causal GQA attention, Qwen3-0.6B shape (16 Q / 8 KV heads, "
                "head_dim 128, bf16); 713 texts log-normal(median 180, sigma 1.0, max 2048) = "
                f"{sum(lens)} tokens in 12 batches of 64")
    if name in ("gemma_window", "gemma_full"):
        lens = w.uniform_lengths(32, 64, 8192)
        win = 512 if name == "gemma_window" else -1
        return ([lens], 3, 1, 256, False, win, 1.0,
                f"config3: EmbeddingGemma-text bidirectional attention, 3 Q / 1 KV heads, head_dim "
                f"256, {'sliding radius 512' if win > 0 else 'full'}; 32 texts U[64,8192] = {sum(lens)} tokens")
    if name in ("modernbert_local", "modernbert_global"):
        lens = w.uniform_lengths(128, 32, 2048)
        win = 64 if name == "modernbert_local" else -1
        return ([lens], 12, 12, 64, False, win, 64 ** -0.5,
                f"config4: ModernBERT attention, 12 heads x 64, {'local radius 64' if win > 0 else 'global'}; "
                f"128 texts U[32,2048] = {sum(lens)} tokens")
    if name in ("qwen3_2048", "qwen3_2048_full"):
        lens = [2048] * 32
        causal = name == "qwen3_2048"
        return ([lens], 16, 8, 128, causal, -1, 128 ** -0.5,
                f"Qwen3-0.6B-shape attention at 2048-token texts ({'causal' if causal else 'bidirectional'} "
                "GQA 16 Q / 8 KV heads x 128, bf16); 32 texts x 2048")
    if name == "pplx_causal":
        lens = [4096] * 16
        return ([lens], 16, 2, 256, True, -1, 256 ** -0.5,
                "config5a: pplx-late full attention, causal GQA 16 Q / 2 KV heads x 256; 16 texts x 4096")
    if name == "vision":
        lens = [256] * 64
        return ([lens], 16, 16, 64, False, -1, 1.0,
                "config5b: vision ViT block attention, 16 heads x 64, bidirectional; 64 images x 256 patches")
    raise SystemExit(f"unknown workload {name}")


def make_inputs(lengths, hq, hkv, d, scale, seed, torch, dev, dtype=None):
    """Seeded N(0,1) q/k/v through an RMSNorm with weights 1 + 0.2 u (u in
    [-0.5, 0.5)), q scaled so that scale * q.k has unit variance; bf16
    unless `dtype` says otherwise."""
    dtype = dtype or torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(seed)
    n = int(sum(lengths))

    def normed(h, s):
        x = torch.randn(n, h, d, generator=g, device=dev)
        w = 1.0 + 0.2 * (torch.rand(d, generator=g, device=dev) - 0.5)
        x = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + 1e-6) * w
        return (x * s).to(dtype)

    q = normed(hq, d ** -0.5 / scale)
    k = normed(hkv, 1.0)
    v = normed(hkv, 1.0)
    return q, k, v


def cpu_baseline(batches, inputs, hq, hkv, d, causal, window, scale, seconds):
    """The oracle's f32 C restatement on host cores over the workload's
    batches in order, wrapping round, until `seconds` of work (at least one
    batch)."""
    from oracle import cref, attention as oa
    cref.lib()
    host = [tuple(t.float().cpu().numpy() for t in qkv) for qkv in inputs]
    tokens, flops, spent, used = 0, 0, 0.0, 0
    while spent < seconds:
        i = used % len(batches)
        lens = batches[i]
        qh, kh, vh = host[i]
        cu = oa.cu_from_lengths(lens)
        t0 = time.perf_counter()
        cref.attention_f32(qh, kh, vh, cu, causal=causal, window=window, scale=scale)
        spent += time.perf_counter() - t0
        tokens += int(sum(lens))
        flops += oa.attention_flops(lens, hq, d, causal, window)
        used += 1
    return {
        "value": round(tokens / spent, 1),
        "unit": "tokens/s",
        "cores": cref.threads(),
        "kind": "port",
        "cpu_model": cpu_model(),
        "sample": (f"{used} batch launches ({used / len(batches):.2f} passes over the {len(batches)} batches; "
                   f"{tokens} tokens, {flops / 1e12:.4f} TFLOP) through oracle/attn_ref.c (f32 per-text "
                   f"online-softmax attention as candle's CPU flash path, 64-key blocks, 8-wide AVX2 dot "
                   f"products, OpenMP over (text, head, 16-row block)), {spent:.2f} s"),
        "tflops": round(flops / spent / 1e12, 4),
        "cross_check": torch_cpu_sdpa(batches, host, hq, hkv, causal, window, scale, min(3.0, seconds / 4)),
    }


def torch_cpu_sdpa(batches, host, hq, hkv, causal, window, scale, seconds):
    """A sanity cross-check beside the CPU baseline, not the baseline: torch's
    CPU scaled_dot_product_attention in f32, one call per text (GQA through
    enable_gqa, the window as a boolean mask), over the workload's batches in
    order until `seconds` of work. Its first batch is compared with the
    oracle's C restatement on the same inputs."""
    import numpy as np
    import torch
    import torch.nn.functional as F
    from oracle import cref, attention as oa

    def run(i):
        qh, kh, vh = host[i]
        cu = oa.cu_from_lengths(batches[i])
        out = np.empty_like(qh)
        for a, b in zip(cu[:-1], cu[1:]):
            q = torch.from_numpy(qh[a:b]).transpose(0, 1).unsqueeze(0)
            k = torch.from_numpy(kh[a:b]).transpose(0, 1).unsqueeze(0)
            v = torch.from_numpy(vh[a:b]).transpose(0, 1).unsqueeze(0)
            mask = None
            if window >= 0:
                r = torch.arange(b - a)
                mask = (r[None, :] - r[:, None]).abs() <= window
                if causal:
                    mask &= r[None, :] <= r[:, None]
            o = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, is_causal=causal and mask is None,
                                               scale=scale, enable_gqa=hq != hkv)
            out[a:b] = o[0].transpose(0, 1).numpy()
        return out

    with torch.inference_mode():
        first = run(0)
        qh, kh, vh = host[0]
        ref = cref.attention_f32(qh, kh, vh, oa.cu_from_lengths(batches[0]), causal=causal, window=window,
                                 scale=scale)
        diff = float(np.abs(first - ref).max())
        tokens, spent, used = 0, 0.0, 0
        while spent < seconds:
            i = used % len(batches)
            t0 = time.perf_counter()
            run(i)
            spent += time.perf_counter() - t0
            tokens += int(sum(batches[i]))
            used += 1
    return {"what": "torch CPU scaled_dot_product_attention, f32, per text (a cross-check, not the baseline)",
            "value": round(tokens / spent, 1), "unit": "tokens/s", "threads": torch.get_num_threads(),
            "sample": f"{used} batch launches, {tokens} tokens, {spent:.2f} s",
            "max_abs_diff_vs_port": diff}


def read_traffic(name: str):
    """HBM bytes per launch of the workload's kernel from the committed
    FETCH_SIZE/WRITE_SIZE summary (profiles/hbm_traffic.md), if present."""
    f = ROOT / "profiles" / "hbm_traffic.md"
    if not f.exists():
        return None
    key = f"traffic_bytes_per_launch[{name}]:"
    for line in f.read_text().splitlines():
        if line.startswith(key):
            return float(line.split(":", 1)[1])
    return None


def cpu_model() -> str:
    """The host CPU's model line (lscpu's "Model name" with family/model)."""
    info = {}
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if ":" in line:
                k, v = (x.strip() for x in line.split(":", 1))
                info.setdefault(k, v)
    except OSError:
        return "unknown"
    return f"{info.get('model name', 'unknown')} (family {info.get('cpu family', '?')}, model {info.get('model', '?')})"


def roofline(tflops, gbs, traffic, kernel, avg_ms, flop_launch, bytes_launch, peak=PEAK_BF16_TFLOPS):
    """The attention kernel against the dense MFMA peak of its dtype (bf16
    2516.6, f32 157.3 TFLOP/s: attention is a dense contraction and is
    graded on matrix-core use), with its HBM bandwidth beside it under
    ``other``; ``hbm_floor_exceeds_mfma_floor`` says when the launch's
    bytes, not its flops, set the lower bound on time."""
    mfma_floor = flop_launch / (peak * 1e12)
    hbm_floor = bytes_launch / (PEAK_HBM_GBS * 1e9)
    return {"bound": "mfma", "achieved": round(tflops, 2), "peak": peak, "unit": "TFLOP/s",
            "frac": round(tflops / peak, 4), "traffic": traffic,
            "kernel": kernel, "avg_launch_us": round(avg_ms * 1e3, 2),
            "algorithmic_per_launch": {"flop": flop_launch, "hbm_bytes": bytes_launch},
            "hbm_floor_exceeds_mfma_floor": hbm_floor > mfma_floor,
            "other": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                      "frac": round(gbs / PEAK_HBM_GBS, 4)}}


OP_WORKLOADS = ("norm_rope", "norm_rope_qk", "pool_last", "pool_mean", "splade", "splade_decoder", "gemm",
                "gdn_conv", "gdn_rule", "gdn_gated_norm")
# What bounds each op workload that is not HBM-bound: the decoder is a GEMM
# on the bf16 matrix cores; the delta rule is f32 vector (VALU) work, graded
# against MI355X's 157.3 TFLOP/s fp32 vector peak (which counts packed-fp32
# FMAs; this build disables packed fp32, so 78.6 TFLOP/s is its ceiling).
OP_BOUND = {"splade_decoder": "mfma", "gemm": "mfma", "gdn_rule": "valu"}
E2E_WORKLOADS = ("qwen3_e2e", "qwen3_e2e_bf16")
PEAK_F32_TFLOPS = 157.3     # MI355X fp32 peak: dense matrix, and vector with packed FMAs


def e2e_cpu_baseline(weights, shape, ids, cu, seconds):
    """The oracle's numpy Qwen3 forward (oracle/qwen3.py) in f32 on the host
    cores, over the same weights and texts, repeated until `seconds` of work
    (at least one encode). BLAS threads: all the process is given."""
    import numpy as np
    from oracle import qwen3 as oq
    cfg = oq.Qwen3Config(vocab=shape.vocab, hidden=shape.hidden, intermediate=shape.intermediate,
                         layers=shape.layers, heads=shape.heads, kv_heads=shape.kv_heads,
                         head_dim=shape.head_dim, eps=shape.eps, theta=shape.theta)
    host = {k: v.float().cpu().numpy() for k, v in weights.items()}
    try:
        from threadpoolctl import threadpool_info
        cores = max((i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"), default=1)
    except Exception:
        cores = os.cpu_count() or 1
    spent, runs = 0.0, 0
    while spent < seconds or runs == 0:
        t0 = time.perf_counter()
        oq.encode(host, cfg, ids, cu, dtype=np.float32)
        spent += time.perf_counter() - t0
        runs += 1
    tokens = int(cu[-1]) * runs
    return {"value": round(tokens / spent, 1), "unit": "tokens/s", "cores": int(cores), "kind": "port",
            "cpu_model": cpu_model(),
            "sample": (f"{runs} encodes of the same {len(cu) - 1} texts ({int(cu[-1])} tokens each) through "
                       f"oracle/qwen3.py (numpy f32 forward: BLAS GEMMs, per-text attention), {spent:.2f} s"),
            "reference_published": {"value": 178, "unit": "tokens/s",
                                    "what": ("the reference's own CPU f32 figure for Qwen3-Embedding-0.6B at "
                                             "batch 8 on a Ryzen 5 3600 (6 cores; other hardware, real "
                                             "checkpoint and text)"),
                                    "source": "docs/DEVICES.md:429"}}


def qwen3_e2e_measure(torch, inl_hip, dev, bf16, steps, warmup, cpu_seconds, no_cpu):
    """Configuration 1 end to end: the Qwen3-0.6B-architecture encoder on
    batches of 8 texts of U[16, 256] tokens, embed -> 28 layers -> last-token
    pooling -> L2, f32 or bf16.

    Every timed step encodes a different draw of 8 texts (seeds 0..steps-1;
    warm-up draws use other seeds), as an engine sees them: no two steps share
    a batch shape, so no launch graph is ever replayed (graphs are off) and
    each GEMM reuses its row-count bucket's algorithm choice instead of
    tuning. For comparison, `repeated_batch` times draw 0 over and over with
    the runner's launch graph on. Returns a dict (tokens/s, roofline, CPU
    baseline)."""
    import numpy as np
    from inl_hip import workloads as w
    td = torch.bfloat16 if bf16 else torch.float32
    shape = w.Qwen3Shape()

    def draw(seed):
        lengths = w.uniform_lengths(8, 16, 256, seed=seed)
        cu = w.cu_seqlens(lengths)
        ids = np.random.default_rng(seed).integers(0, shape.vocab, cu[-1]).astype(np.int32)
        return lengths, cu, ids

    timed = [draw(s) for s in range(steps)]
    warm = [draw(1000 + s) for s in range(max(warmup, 1))]
    weights = w.qwen3_random_weights(shape, torch, dev, td, seed=0)
    enc = inl_hip.Qwen3Encoder(shape, weights, max_positions=256)
    out = torch.empty((8, shape.hidden), dtype=torch.float32, device=dev)
    ws = torch.empty(max(enc.workspace_bytes(c) for _, c, _ in timed + warm) + 256, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()
    q_out, kv_out = shape.heads * shape.head_dim, shape.kv_heads * shape.head_dim
    per_token = 2 * (shape.hidden * (q_out + 2 * kv_out) + q_out * shape.hidden + 3 * shape.hidden * shape.intermediate)

    def flops_of(lengths):
        return shape.layers * (sum(lengths) * per_token
                               + inl_hip.attention_flops(lengths, shape.heads, shape.head_dim, True))

    enc.set_graphs(False)
    for _, cu, ids in warm:
        enc.encode(ids, cu, out=out, workspace=ws, stream=stream)
    torch.cuda.synchronize()
    tuned0 = inl_hip.linear_stats()["tunings"]
    t0 = time.perf_counter()
    for _, cu, ids in timed:
        enc.encode(ids, cu, out=out, workspace=ws, stream=stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    tunings = inl_hip.linear_stats()["tunings"] - tuned0
    # GPU time per encode from HIP events on the launch stream (same draws)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in timed]
    for (a, b), (_, cu, ids) in zip(evs, timed):
        a.record(stream)
        enc.encode(ids, cu, out=out, workspace=ws, stream=stream)
        b.record(stream)
    torch.cuda.synchronize()
    gpu_ms = sum(a.elapsed_time(b) for a, b in evs)
    tokens = sum(c[-1] for _, c, _ in timed)
    flops = sum(flops_of(l) for l, _, _ in timed)
    # the same encoder on one repeated batch, launch graph on
    enc.set_graphs(True)
    _, cu0, ids0 = timed[0]
    for _ in range(3):
        enc.encode(ids0, cu0, out=out, workspace=ws, stream=stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(steps):
        enc.encode(ids0, cu0, out=out, workspace=ws, stream=stream)
    torch.cuda.synchronize()
    rep_wall = time.perf_counter() - t1
    peak = PEAK_BF16_TFLOPS if bf16 else PEAK_F32_TFLOPS
    ach = flops / (gpu_ms * 1e-3) / 1e12
    res = {
        "metric": "encoded tokens/s", "value": round(tokens / wall, 1), "unit": "tokens/s",
        "dtype": "bf16" if bf16 else "f32", "steps": steps, "warmup": len(warm),
        "ms_per_step": round(wall / steps * 1e3, 4), "tokens": int(tokens),
        "workload": (f"config1: Qwen3-Embedding-0.6B-architecture encoder end to end "
                     f"({'bf16' if bf16 else 'f32'}): 28 layers, hidden 1024, 16 Q / 8 KV heads x 128, RoPE "
                     f"theta 1e6, last-token pooling, L2; each step a new draw of 8 texts U[16,256] (seeds "
                     f"0..{steps - 1}), random ids in [0,151669), random-init weights"),
        "graphs": "off (every step is a new batch shape)",
        "gemm_tunings_in_timed_steps": int(tunings),
        "roofline": {"bound": "mfma", "achieved": round(ach, 2), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(ach / peak, 4), "traffic": None,
                     "kernel": "whole encode (hipBLASLt GEMMs, attention, prologue, norms, SwiGLU, pooling)",
                     "avg_launch_us": round(gpu_ms / steps * 1e3, 2),
                     "algorithmic_per_launch": {"flop": int(flops // steps)}},
        "repeated_batch": {"value": round(cu0[-1] * steps / rep_wall, 1), "unit": "tokens/s",
                           "ms_per_step": round(rep_wall / steps * 1e3, 4), "tokens_per_step": int(cu0[-1]),
                           "graphs": "on (replayed from the third call)"},
    }
    if not no_cpu:
        l0, c0, i0 = timed[0]
        res["cpu_baseline"] = e2e_cpu_baseline(weights, shape, i0, np.asarray(c0), cpu_seconds)
    enc.close()
    return res


def e2e_main(args):
    """--workload qwen3_e2e (f32, configuration 1) or qwen3_e2e_bf16: the
    configuration-1 measurement above as the line itself."""
    import torch
    import inl_hip
    dev = torch.device("cuda:0")
    bf16 = args.workload.endswith("bf16")
    r = qwen3_e2e_measure(torch, inl_hip, dev, bf16, args.steps, args.warmup, args.cpu_seconds, args.no_cpu)
    log(f"workload: {r['workload']}")
    result = {
        "metric": METRIC, "value": r["value"], "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": r["warmup"], "ms_per_step": r["ms_per_step"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": r["dtype"],
        "data": "synthetic (random token ids, seeded random-init weights; no checkpoint)",
        "config": {"workload": r["workload"], "tokens_timed": r["tokens"], "graphs": r["graphs"],
                   "gemm_tunings_in_timed_steps": r["gemm_tunings_in_timed_steps"],
                   "value_is": "end-to-end encoded tokens/s (embed, 28 layers, pooling, L2 per step)"},
        "roofline": r["roofline"], "repeated_batch": r["repeated_batch"],
    }
    if "cpu_baseline" in r:
        result["cpu_baseline"] = r["cpu_baseline"]
    print(json.dumps(result), flush=True)


def gemma_e2e_cpu_baseline(host_w, tc, seconds):
    """The oracle's numpy EmbeddingGemma 2 forward (oracle/gemma2.py) in f32
    on the host cores (the reference's CPU path is f32: bf16 is refused on
    the CPU, gemma2.rs:685-691), over the benchmark's weights and a bounded
    sample of 4 texts of U[64, 512] tokens, repeated until `seconds`."""
    import numpy as np
    from oracle import gemma2 as og
    from inl_hip import workloads as w
    lengths = w.uniform_lengths(4, 64, 512, seed=1)
    cu = np.asarray(w.cu_seqlens(lengths))
    ids = np.random.default_rng(1).integers(0, tc["vocab_size"], int(cu[-1]))
    try:
        from threadpoolctl import threadpool_info
        cores = max((i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"), default=1)
    except Exception:
        cores = os.cpu_count() or 1
    spent, runs = 0.0, 0
    while spent < seconds or runs == 0:
        t0 = time.perf_counter()
        og.encode(host_w, tc, ids, cu, dtype=np.float32)
        spent += time.perf_counter() - t0
        runs += 1
    tokens = int(cu[-1]) * runs
    return {"value": round(tokens / spent, 1), "unit": "tokens/s", "cores": int(cores), "kind": "port",
            "cpu_model": cpu_model(),
            "sample": (f"{runs} encodes of 4 texts U[64,512] ({int(cu[-1])} tokens each) through oracle/gemma2.py "
                       f"(numpy f32 forward: BLAS GEMMs, per-text attention) with the same weights, {spent:.2f} s"),
            "reference_published": {"value": 424, "unit": "tokens/s",
                                    "what": ("the reference's own CPU f32 figure for EmbeddingGemma 2 at batch 8 "
                                             "on a Ryzen 5 3600 (6 cores; other hardware, real checkpoint and "
                                             "text)"),
                                    "source": "docs/DEVICES.md:430"}}


def gemma_e2e_main(args):
    """Configuration 3 end to end: the EmbeddingGemma-2 text tower of
    gemma2.rs at the benchmark's shape (24 layers, hidden 768, 3 Q / 1 KV
    heads x 256, sliding radius 512 with every sixth layer full) on 32 texts
    of U[64, 8192] tokens, bf16; embed -> per-layer inputs -> 24 layers ->
    mean pool -> projection -> L2; one step = one encode."""
    # Every GEMM of this workload runs on the library's own bf16 kernel
    # (inl_gemm_bf16_fwd); the runner refuses batches this large whenever
    # one would go to hipBLASLt.
    import numpy as np
    import torch
    import inl_hip
    from inl_hip import workloads as w
    dev = torch.device("cuda:0")
    tc = w.gemma2_config3()
    host_w = w.gemma2_random_weights(tc, seed=0)
    weights = {k: torch.from_numpy(v).to(dev).to(torch.bfloat16) for k, v in host_w.items()}
    lengths = w.uniform_lengths(32, 64, 8192)
    cu = np.asarray(w.cu_seqlens(lengths))
    tokens = int(cu[-1])
    ids = np.random.default_rng(0).integers(0, tc["vocab_size"], tokens).astype(np.int32)
    enc = inl_hip.Gemma2Encoder(tc, weights, max_positions=8192)
    out = torch.empty((len(lengths), tc["embedding_dim"]), dtype=torch.float32, device=dev)
    ws = torch.empty(enc.workspace_bytes(cu.tolist()) + 256, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()
    H, I, E, heads, hd, kvh = (tc["hidden_size"], tc["intermediate_size"], tc["hidden_size_per_layer_input"],
                               tc["num_attention_heads"], tc["head_dim"], tc["num_key_value_heads"])
    per_token = 2 * (H * (heads + 2 * kvh) * hd + heads * hd * H + 2 * H * I + I * H + 3 * H * E)
    flops = 0
    for kind in tc["layer_types"]:
        window = tc["sliding_window"] if kind == "sliding_attention" else -1
        flops += tokens * per_token + inl_hip.attention_flops(lengths, heads, hd, False, window)
    label = (f"config3: EmbeddingGemma-2 text tower end to end (bf16): 24 layers (every sixth full), hidden 768, "
             f"3 Q / 1 KV heads x 256, sliding radius 512, intermediate 1152, per-layer input 256, embedding_dim 768, "
             f"vocab 262144; mean pooling, projection, L2; 32 texts U[64,8192] = {tokens} tokens, random ids, "
             f"random-init weights")
    log(f"workload: {label}; {flops / 1e12:.3f} TFLOP per encode")

    def step(evs=None):
        if evs is not None:
            evs[0][0].record(stream)
        enc.encode(ids, cu.tolist(), out=out, workspace=ws, stream=stream)
        if evs is not None:
            evs[0][1].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    avg_ms = timed_launches(torch, step, 1, args.steps)
    ach = flops / (avg_ms * 1e-3) / 1e12
    result = {
        "metric": METRIC, "value": round(tokens * args.steps / wall, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random token ids, seeded random-init weights; no checkpoint)",
        "config": {"workload": label, "tokens_per_step": tokens, "texts": len(lengths),
                   "tflop_per_step": round(flops / 1e12, 6),
                   "value_is": "end-to-end encoded tokens/s (embed, 24 layers, pooling, projection, L2 per step)"},
        "roofline": {"bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(ach / PEAK_BF16_TFLOPS, 4), "traffic": None,
                     "kernel": "whole encode (own bf16 MFMA GEMMs, attention, prologue, norms, GEGLU, pooling)",
                     "avg_launch_us": round(avg_ms * 1e3, 2), "algorithmic_per_launch": {"flop": flops}},
    }
    if not args.no_cpu:
        # the CPU leg: the oracle's forward as the baseline, and as the
        # checker of three texts of the timed batch
        result["cpu_baseline"] = gemma_e2e_cpu_baseline(host_w, tc, args.cpu_seconds)
        result["cpu_baseline"]["oracle_check"] = gemma_e2e_parity(host_w, tc, ids, cu, out, weights)
    enc.close()
    print(json.dumps(result), flush=True)


def gemma_e2e_parity(host_w, tc, ids, cu, out, weights):
    """(Part of the CPU leg.) Cosines of three texts of the timed batch (the shortest and the two
    nearest 1,000 tokens) against oracle/gemma2.py in f32 on the bf16-rounded
    weights: texts are independent in a packed batch, so the oracle encodes
    just those texts. The reference's bf16 floor is cosine >= 0.999."""
    import numpy as np
    from oracle import gemma2 as og
    lens = np.diff(np.asarray(cu))
    order = [int(np.argmin(lens))] + [int(i) for i in np.argsort(np.abs(lens - 1000))[:3]]
    picks = list(dict.fromkeys(order))[:3]
    wb = {k: v.float().cpu().numpy() for k, v in weights.items()}
    sub_ids = np.concatenate([ids[cu[b]:cu[b + 1]] for b in picks])
    sub_cu = np.concatenate([[0], np.cumsum([lens[b] for b in picks])])
    t0 = time.perf_counter()
    ref = og.encode(wb, tc, sub_ids, sub_cu, dtype=np.float32).astype(np.float64)
    got = out[picks].double().cpu().numpy()
    cos = (got * ref).sum(1) / np.linalg.norm(got, axis=1) / np.linalg.norm(ref, axis=1)
    log(f"gemma_e2e parity: texts {picks} ({[int(lens[b]) for b in picks]} tokens): cosines "
        f"{[round(float(c), 6) for c in cos]} ({time.perf_counter() - t0:.1f} s)")
    return {"texts": picks, "tokens": [int(lens[b]) for b in picks], "cosine": [round(float(c), 6) for c in cos],
            "against": "oracle/gemma2.py f32 on the bf16-rounded weights", "min_cosine": round(float(cos.min()), 6)}


def op_workload(name, torch, inl_hip, dev):
    """The prologue and epilogue kernels at their configurations' full sizes.
    Returns (label, kernel, launches per step, step(evs), tokens per step,
    algorithmic HBM bytes per step, dtype). Bytes are what the op must move:
    its inputs read once and its outputs written once (per-unit figures,
    stated in each label)."""
    from inl_hip import workloads as w
    g = torch.Generator(device=dev).manual_seed(3)
    stream = torch.cuda.current_stream()

    def timed(launches):
        def step(evs=None):
            for i, fn in enumerate(launches):
                if evs is not None:
                    evs[i][0].record(stream)
                fn()
                if evs is not None:
                    evs[i][1].record(stream)
        return step

    if name == "norm_rope":
        # config 2 batches: per batch, q (16 heads, q_norm weight) and k (8 heads,
        # k_norm weight) of a fused [T, 32, 128] bf16 QKV projection output,
        # RMSNorm (eps 1e-6) + RoPE (theta 1e6), bf16 out
        lens = w.qwen3_op_lengths()
        bats = w.batches(lens, 64)
        c, s_ = inl_hip.rope_table(128, 1e6, 2048)
        cos, sin = torch.from_numpy(c).to(dev), torch.from_numpy(s_).to(dev)
        launches, nbytes = [], 0
        for b in bats:
            cu = w.cu_seqlens(b)
            T = cu[-1]
            qkv = torch.randn(T, 32, 128, generator=g, device=dev).to(torch.bfloat16)
            rows = torch.from_numpy(inl_hip.positions(cu)).to(dev)
            wq = (1 + 0.1 * torch.randn(128, generator=g, device=dev)).to(torch.bfloat16)
            wk = (1 + 0.1 * torch.randn(128, generator=g, device=dev)).to(torch.bfloat16)
            qo = torch.empty(T, 16, 128, device=dev, dtype=torch.bfloat16)
            ko = torch.empty(T, 8, 128, device=dev, dtype=torch.bfloat16)
            launches.append(lambda qkv=qkv, rows=rows, wq=wq, qo=qo: inl_hip.norm_rope(
                qkv[:, :16], rows, cos, sin, weight=wq, eps=1e-6, out=qo, stream=stream))
            launches.append(lambda qkv=qkv, rows=rows, wk=wk, ko=ko: inl_hip.norm_rope(
                qkv[:, 16:24], rows, cos, sin, weight=wk, eps=1e-6, out=ko, stream=stream))
            # per launch: x read and y written (heads*128*2 B each per token), the
            # positions (4 B per token), the weight, and the cos/sin rows of the
            # batch's longest text (2 tables x 64 floats per position)
            for heads in (16, 8):
                nbytes += T * heads * 128 * 2 * 2 + T * 4 + 128 * 2 + max(b) * 64 * 4 * 2
        label = (f"config2 prologue: q/k RMSNorm+RoPE (Qwen3-0.6B: 16 q / 8 k heads x 128, bf16 in/out, "
                 f"theta 1e6) over {sum(lens)} tokens in 12 batches, 2 launches per batch")
        return label, "norm_rope_kernel<bf16, bf16>", len(launches), timed(launches), sum(lens), nbytes, "bf16"
    if name == "norm_rope_qk":
        # the same prologue with q and k of each batch in one launch
        # (inl_norm_rope_qk_fwd over the 24 q/k heads of the fused rows), as the
        # encoder runners call it
        lens = w.qwen3_op_lengths()
        bats = w.batches(lens, 64)
        c, s_ = inl_hip.rope_table(128, 1e6, 2048)
        cos, sin = torch.from_numpy(c).to(dev), torch.from_numpy(s_).to(dev)
        launches, nbytes = [], 0
        for b in bats:
            cu = w.cu_seqlens(b)
            T = cu[-1]
            qkv = torch.randn(T, 32, 128, generator=g, device=dev).to(torch.bfloat16)
            rows = torch.from_numpy(inl_hip.positions(cu)).to(dev)
            wq = (1 + 0.1 * torch.randn(128, generator=g, device=dev)).to(torch.bfloat16)
            wk = (1 + 0.1 * torch.randn(128, generator=g, device=dev)).to(torch.bfloat16)
            qko = torch.empty(T, 24, 128, device=dev, dtype=torch.bfloat16)
            launches.append(lambda qkv=qkv, rows=rows, wq=wq, wk=wk, qko=qko: inl_hip.norm_rope_qk(
                qkv[:, :24], 16, rows, cos, sin, q_weight=wq, k_weight=wk, eps=1e-6, out=qko, stream=stream))
            # x read and y written (24 heads x 128 x 2 B each per token), the
            # positions, both weights and the cos/sin rows of the longest text
            nbytes += T * 24 * 128 * 2 * 2 + T * 4 + 2 * 128 * 2 + max(b) * 64 * 4 * 2
        label = (f"config2 prologue, q and k in one launch per batch (inl_norm_rope_qk_fwd; Qwen3-0.6B: 16 q / 8 k "
                 f"heads x 128, bf16 in/out, theta 1e6) over {sum(lens)} tokens in 12 batches")
        return label, "norm_rope_kernel<bf16, bf16>", len(launches), timed(launches), sum(lens), nbytes, "bf16"
    if name == "pool_last":
        # config 2 batches: final RMSNorm of each text's last row (hidden 1024,
        # bf16) and the f32 L2 normalisation
        lens = w.qwen3_op_lengths()
        bats = w.batches(lens, 64)
        launches, nbytes = [], 0
        wt = (1 + 0.1 * torch.randn(1024, generator=g, device=dev)).to(torch.bfloat16)
        for b in bats:
            cu = torch.tensor(w.cu_seqlens(b), dtype=torch.int32, device=dev)
            h = torch.randn(int(sum(b)), 1024, generator=g, device=dev).to(torch.bfloat16)
            launches.append(lambda h=h, cu=cu: inl_hip.pool_last(h, cu, weight=wt, eps=1e-6, stream=stream))
            nbytes += len(b) * 1024 * 2 + 1024 * 2 + len(b) * 1024 * 4 + (len(b) + 1) * 4
        label = ("config2 last-token epilogue: final RMSNorm + L2 of each text's last row (hidden 1024, bf16 "
                 "in, f32 out), 12 batches of 64 texts")
        return label, "pool_last_kernel<bf16>", len(launches), timed(launches), sum(lens), nbytes, "bf16"
    if name == "pool_mean":
        # config 3: mean over each text's rows (hidden 768, bf16) + L2
        lens = w.uniform_lengths(32, 64, 8192)
        cu = torch.tensor(w.cu_seqlens(lens), dtype=torch.int32, device=dev)
        h = torch.randn(int(sum(lens)), 768, generator=g, device=dev).to(torch.bfloat16)
        launches = [lambda: inl_hip.pool_mean(h, cu, normalize=True, stream=stream)]
        nbytes = int(sum(lens)) * 768 * 2 + len(lens) * 768 * 4 + (len(lens) + 1) * 4
        label = (f"config3 mean epilogue: mean over {sum(lens)} rows of 32 texts U[64,8192] (hidden 768, bf16 "
                 "in, f32 out) + L2")
        return label, "pool_mean_vec_kernel<bf16>", 1, timed(launches), sum(lens), nbytes, "bf16"
    if name == "splade":
        # config 4: SPLADE max-pool over every speaking row's f32 logits
        # (vocab 50002) of 128 texts U[32,2048], finish, fold to 36282 terms
        lens = w.uniform_lengths(128, 32, 2048)
        speak = [t - 1 for t in lens]
        offs = torch.tensor(w.cu_seqlens(speak), dtype=torch.int32, device=dev)
        S, V, terms = int(sum(speak)), 50002, 36282
        logits = torch.empty(S, V, device=dev)
        logits.normal_(0.0, 4.0, generator=g)
        bias = torch.randn(V, generator=g, device=dev)
        import numpy as np
        rng = np.random.default_rng(0)
        canonical = torch.from_numpy(np.concatenate([rng.permutation(terms), rng.integers(0, terms, V - terms)])
                                     .astype(np.int32)).to(dev)
        launches = [lambda: inl_hip.pool_splade(logits, offs, bias=bias, shift=10.0, masked_ids=(50000, 50001),
                                                canonical=canonical, out_dim=terms, stream=stream)]
        nbytes = S * V * 4 + V * 4 + V * 4 + len(lens) * terms * 4
        label = (f"config4 SPLADE epilogue: max over {S} speaking rows x {V} f32 logits of 128 texts "
                 f"U[32,2048], finish (shift 10), fold to {terms} terms")
        return label, "splade_kernel", 1, timed(launches), S, nbytes, "f32"
    if name == "gemm":
        # config 3: one layer's projections on the hand-written bf16 GEMM at
        # 139,124 tokens, as the EmbeddingGemma 2 runner issues them
        # (q/k/v rows of 2304, the fused GEGLU and per-layer-input gates)
        import numpy as np
        m, H, I, E = 139124, 768, 1152, 256
        x = torch.randn(m, H, generator=g, device=dev).to(torch.bfloat16)
        xb = torch.randn(m, I, generator=g, device=dev).to(torch.bfloat16)
        A = torch.empty(m, 2304, device=dev, dtype=torch.bfloat16)
        B = torch.empty(m, I, device=dev, dtype=torch.bfloat16)
        T = torch.empty(m, H, device=dev)
        Tp = torch.empty(m, E, device=dev)
        P = torch.randn(m, E, generator=g, device=dev).to(torch.bfloat16)
        wt = lambda r, c: (torch.randn(r, c, generator=g, device=dev) * c ** -0.5).to(torch.bfloat16)
        w_ple, w_qkv, w_o, w_gu, w_d, w_g, w_p = wt(E, H), wt(1280, H), wt(H, 768), wt(2 * I, H), wt(H, I), \
            wt(E, H), wt(H, E)
        launches = [
            lambda: inl_hip.gemm_bf16(x, w_ple, out=Tp, alpha=H ** -0.5, stream=stream),
            lambda: inl_hip.gemm_bf16(x, w_qkv, out=A[:, :1280], stream=stream),
            lambda: inl_hip.gemm_bf16(xb[:, :768], w_o, out=T, stream=stream),
            lambda: inl_hip.gemm_bf16_gated(x, w_gu, "geglu", out=B, stream=stream),
            lambda: inl_hip.gemm_bf16(xb, w_d, out=T, stream=stream),
            lambda: inl_hip.gemm_bf16_gated(x, w_g, "gelu_mul", mul=P, out=B[:, :E], stream=stream),
            lambda: inl_hip.gemm_bf16(xb[:, :E], w_p, out=T, stream=stream),
        ]
        flops = 2 * m * H * (E + 1280 + 768 + 2 * I + I + E) + 2 * m * E * H
        return ("config3 GEMMs of one EmbeddingGemma 2 layer on inl_gemm_bf16_fwd / _gated_fwd (139,124 rows: "
                "per-layer input 768->256, q/k/v 768->1280, o 768->768, GEGLU 768->2x1152, down 1152->768, "
                "per-layer gate 768->256 x multiplier, per-layer projection 256->768), bf16 in, f32 accumulation",
                "gemm_bf16_kernel", len(launches), timed(launches), m, flops, "bf16")

    if name == "splade_decoder":
        # config 4: the fused decoder GEMM + per-text max over every speaking
        # row (bf16 head [S, 768] x decoder [50002, 768]^T), no logits written
        import numpy as np
        lens = w.uniform_lengths(128, 32, 2048)
        speak = [t - 1 for t in lens]
        offs = np.asarray(w.cu_seqlens(speak), dtype=np.int32)
        S, V, H = int(offs[-1]), 50002, 768
        head = torch.randn(S, H, generator=g, device=dev).to(torch.bfloat16)
        wd = (torch.randn(V, H, generator=g, device=dev) * (4.0 / H ** 0.5)).to(torch.bfloat16)
        out = torch.empty(len(speak), V, device=dev)
        launches = [lambda: inl_hip.splade_decoder_max(head, wd, offs, out=out, stream=stream)]
        flops = 2 * S * V * H
        label = (f"config4 SPLADE decoder GEMM + per-text max, fused: {S} speaking rows x {V} terms x {H} "
                 f"(bf16, f32 accumulation) of 128 texts U[32,2048]; the {S * V * 4 / 1e9:.1f} GB of f32 logits "
                 "are never written")
        return label, "splade_decoder_max_kernel", 1, timed(launches), S, flops, "bf16"
    if name.startswith("gdn_"):
        # configuration 5's pplx-late linear-attention layer: 16 texts x 4096
        # tokens, 16 key / 16 value heads of 128 (Qwen3.5-0.8B shape), conv 4
        nk = nv = 16
        dk = dv = 128
        lens = [4096] * 16
        cu = torch.tensor(w.cu_seqlens(lens), dtype=torch.int32, device=dev)
        N, ch = sum(lens), 2 * nk * dk + nv * dv
        shape = f"16 texts x 4096 tokens, {nk}/{nv} heads, dk = dv = {dk}, bf16"
        if name == "gdn_conv":
            proj = torch.randn(N, ch, generator=g, device=dev).to(torch.bfloat16)
            wt = (torch.randn(ch, 4, generator=g, device=dev) * 0.5).to(torch.bfloat16)
            launches = [lambda: inl_hip.gdn_conv(proj, cu, wt, stream=stream)]
            label = f"config5 gated-delta-net causal conv (4 taps) + silu over {ch} channels, {shape}"
            return label, "gdn_conv_kernel", 1, timed(launches), N, N * ch * 2 * 2, "bf16"
        mixed = torch.randn(N, ch, generator=g, device=dev).to(torch.bfloat16)
        gg = -torch.rand(N, nv, generator=g, device=dev) * 0.2
        beta = torch.rand(N, nv, generator=g, device=dev)
        if name == "gdn_rule":
            launches = [lambda: inl_hip.gdn_rule(mixed, cu, nk, nv, dk, dv, gg, beta, stream=stream)]
            label = (f"config5 gated delta rule, f32 state per (text, head), {shape}; 7 dk dv flops per "
                     "token and head (decay, S^T k, update, S^T q)")
            return label, "gdn_rule_kernel", 1, timed(launches), N, 7 * N * nv * dk * dv, "f32"
        if name == "gdn_gated_norm":
            core = torch.randn(N, nv, dv, generator=g, device=dev)
            z = torch.randn(N, nv, dv, generator=g, device=dev).to(torch.bfloat16)
            nw = torch.ones(dv, device=dev).to(torch.bfloat16)
            launches = [lambda: inl_hip.gdn_gated_norm(core, z, nw, 1e-6, stream=stream)]
            label = f"config5 gated RMSNorm of the rule's f32 output with silu(z) gate, {shape}"
            return label, "gdn_gated_norm_kernel", 1, timed(launches), N, N * nv * dv * (4 + 2 + 2), "bf16"
    raise SystemExit(f"unknown op workload {name}")


def timed_launches(torch, step, n_launch, steps):
    """Per-launch GPU durations from HIP events on the launch stream. Each
    step is queued behind a GPU-side sleep, so that the host has enqueued all
    of the step's launches before the first one starts: the events then
    bracket back-to-back kernels, not host-side gaps between short ones.
    Returns the mean launch duration in ms."""
    probe = time.perf_counter()
    step()
    torch.cuda.synchronize()
    host = time.perf_counter() - probe
    sleep = getattr(torch.cuda, "_sleep", None)
    events = [[[torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)]
               for _ in range(n_launch)] for _ in range(steps)]
    for s in range(steps):
        if sleep is not None:
            sleep(int(max(host, 1e-4) * 4e9))   # about twice the host time at ~2 GHz
        step(events[s])
    torch.cuda.synchronize()
    if n_launch > 1:
        per = [sum(events[s][i][0].elapsed_time(events[s][i][1]) for s in range(steps)) / steps
               for i in range(n_launch)]
        log("per-launch average (us): " + ", ".join(f"{1e3 * x:.1f}" for x in per))
    return sum(a.elapsed_time(b) for ev in events for a, b in ev) / (steps * n_launch)


def op_main(args):
    import torch
    import inl_hip
    dev = torch.device("cuda:0")
    label, kernel, n_launch, step, tokens, nbytes, dtype = op_workload(args.workload, torch, inl_hip, dev)
    bound = OP_BOUND.get(args.workload, "hbm")
    mfma = bound != "hbm"   # work counted in flops, not bytes
    log(f"workload: {label}; {nbytes / 1e9:.3f} {'GFLOP' if mfma else 'GB'} per step, {n_launch} launches")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    avg_ms = timed_launches(torch, step, n_launch, args.steps)
    gbs = nbytes / n_launch / (avg_ms * 1e-3) / 1e9
    if mfma:
        tf = nbytes / n_launch / (avg_ms * 1e-3) / 1e12
        peak = PEAK_BF16_TFLOPS if bound == "mfma" else PEAK_F32_TFLOPS
        roof = {"bound": bound, "achieved": round(tf, 2), "peak": peak, "unit": "TFLOP/s",
                "frac": round(tf / peak, 4), "traffic": read_traffic(args.workload), "kernel": kernel,
                "avg_launch_us": round(avg_ms * 1e3, 2), "algorithmic_per_launch": {"flop": nbytes / n_launch}}
    else:
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": read_traffic(args.workload), "kernel": kernel,
                "avg_launch_us": round(avg_ms * 1e3, 2), "algorithmic_per_launch": {"hbm_bytes": nbytes / n_launch}}
    print(json.dumps({
        "metric": f"{args.workload} op throughput ("
                  + {"mfma": "TFLOP/s vs bf16 MFMA peak", "valu": "TFLOP/s vs fp32 vector peak",
                     "hbm": "HBM GB/s vs 8 TB/s"}[bound] + ")",
        "value": round(tokens * args.steps / wall, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
        "data": "synthetic (seeded random inputs; no checkpoint)",
        "config": {"workload": label, "tokens_per_step": tokens, "launches_per_step": n_launch,
                   ("flop_per_step" if mfma else "hbm_bytes_per_step"): nbytes},
        "roofline": roof,
    }), flush=True)


def stream_reference():
    """HBM bandwidth that torch's own streaming kernels reach (HIP events, 20
    launches each after 3 warm-up launches): the practical ceiling next to
    the 8 TB/s peak that the HBM-bound rows are measured against. Sizes of
    1 GiB and more keep the data out of the 256 MB last-level cache."""
    import torch
    dev = torch.device("cuda:0")
    out = {"what": "torch streaming kernels, f32, bytes moved per launch / launch time", "unit": "TB/s"}
    for gib in (1, 4):
        n = gib * (1 << 30) // 4
        x = torch.randn(n, device=dev)
        y = torch.randn(n, device=dev)

        def rate(f, nbytes):
            for _ in range(3):
                f()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(20):
                f()
            b.record()
            torch.cuda.synchronize()
            return round(nbytes / (a.elapsed_time(b) / 20 * 1e-3) / 1e12, 2)

        out[f"{gib}_GiB"] = {
            "copy (1 read + 1 write)": rate(lambda: y.copy_(x), 2 * n * 4),
            "add in place (2 reads + 1 write)": rate(lambda: y.add_(x), 3 * n * 4),
            "fill (1 write)": rate(lambda: y.fill_(0.5), n * 4),
            "sum (1 read)": rate(lambda: torch.sum(x), n * 4),
        }
        del x, y
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="qwen3")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-e2e", action="store_true",
                    help="default workload only: skip the nested configuration-1 end-to-end measurement")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run device-to-device copies of MIB MiB (3 launches): the known-size "
                         "reference that scales the FETCH_SIZE / WRITE_SIZE counters")
    ap.add_argument("--stream-reference", action="store_true",
                    help="only time torch's own streaming kernels (copy, in-place add, fill, sum) over 1 and "
                         "4 GiB: what a plain element-wise kernel reaches on this GPU's HBM")
    args = ap.parse_args()

    if args.stream_reference:
        stream_reference()
        return

    if args.copy_calibration:
        import torch
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.randn(n, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n * 4, "launches": 3}))
        return

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the path shards by independent texts (one GPU's texts per rank)", file=sys.stderr)
        sys.exit(2)

    if args.workload in OP_WORKLOADS:
        op_main(args)
        return
    if args.workload == "gemma_e2e":
        gemma_e2e_main(args)
        return
    if args.workload in E2E_WORKLOADS:
        e2e_main(args)
        return

    import torch
    import inl_hip
    from inl_hip import attention_flops

    dev = torch.device("cuda:0")
    # "<workload>_f32": the same shapes in f32 (configuration 1's dtype), on the
    # f32 kernel, graded against the 157.3 TFLOP/s fp32 matrix peak
    f32 = args.workload.endswith("_f32")
    base = args.workload[:-4] if f32 else args.workload
    dt_name, td, es = ("f32", torch.float32, 4) if f32 else ("bf16", torch.bfloat16, 2)
    peak = PEAK_F32_TFLOPS if f32 else PEAK_BF16_TFLOPS
    batches, hq, hkv, d, causal, window, scale, label = workload(base)
    if f32:
        label = label.replace("bf16", "f32")
    inputs = [make_inputs(lens, hq, hkv, d, scale, 1000 + i, torch, dev, td) for i, lens in enumerate(batches)]
    plans, outs = [], []
    for lens, (q, k, v) in zip(batches, inputs):
        cu = inl_hip.workloads.cu_seqlens(lens)
        desc = inl_hip.make_attn_desc(cu, hq, hkv, d, causal=causal, window=window, scale=scale,
                                      dtype=dt_name, out_dtype=dt_name)
        plans.append(inl_hip.AttnPlan(desc))
        outs.append(torch.empty_like(q))
    tokens = sum(sum(b) for b in batches)
    flops = sum(attention_flops(b, hq, d, causal, window) for b in batches)
    # algorithmic HBM bytes: Q, K, V read once and O written once
    hbm_bytes = tokens * (hq * d + 2 * hkv * d + hq * d) * es
    kernel = inl_hip.kernel_name(plans[0].desc)
    n_launch = len(batches)
    stream = torch.cuda.current_stream()
    log(f"workload: {label}; {flops / 1e12:.4f} TFLOP per step, {n_launch} launches")

    def step(evs=None):
        for i, (pl, (q, k, v), o) in enumerate(zip(plans, inputs, outs)):
            if evs is not None:
                evs[i][0].record(stream)
            pl.run(q, k, v, o, stream)
            if evs is not None:
                evs[i][1].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    avg_launch_ms = timed_launches(torch, step, n_launch, args.steps)
    kernel_ms = avg_launch_ms * args.steps * n_launch
    achieved = flops / n_launch / (avg_launch_ms * 1e-3) / 1e12
    achieved_gbs = hbm_bytes / n_launch / (avg_launch_ms * 1e-3) / 1e9
    tok_s = tokens * args.steps / wall
    traffic = read_traffic(args.workload)
    log(f"wall {wall:.4f} s for {args.steps} steps; kernel {kernel_ms:.3f} ms; "
        f"avg launch {avg_launch_ms * 1e3:.1f} us; {achieved:.1f} TFLOP/s")

    result = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dt_name,
        "data": "synthetic (seeded N(0,1) q/k/v after RMSNorm; no checkpoint)",
        "config": {"workload": label, "tokens_per_step": tokens, "launches_per_step": n_launch,
                   "attention_tflop_per_step": round(flops / 1e12, 6),
                   "value_is": ("attention-op tokens/s: tokens passed through ONE attention layer per "
                                "second (a step runs the op once over every batch), not end-to-end "
                                "encoded tokens/s")},
        "attention_tflops": round(flops * args.steps / wall / 1e12, 2),
        "attention_frac_of_peak": round(flops * args.steps / wall / 1e12 / peak, 4),
        "roofline": roofline(achieved, achieved_gbs, traffic, kernel, avg_launch_ms, flops / n_launch,
                             hbm_bytes / n_launch, peak),
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(batches, inputs, hq, hkv, d, causal, window, scale,
                                              args.cpu_seconds)
    for pl in plans:
        pl.close()
    if args.workload == "qwen3" and not args.no_e2e:
        # the metric's other half: configuration 1 encoded tokens/s end to end
        del inputs, outs
        torch.cuda.empty_cache()
        result["e2e_config1"] = qwen3_e2e_measure(torch, inl_hip, dev, False, args.steps, args.warmup,
                                                  args.cpu_seconds, args.no_cpu)
        log(f"e2e config1: {result['e2e_config1']['value']} tokens/s")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
