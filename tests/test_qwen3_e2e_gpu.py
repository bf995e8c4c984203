"""GPU end-to-end Qwen3 encode (inl_qwen3_* through the C ABI) against the
numpy oracle (oracle/qwen3.py, pinned against transformers' Qwen3Model).

- Full width, 2 layers (hidden 1024, 16/8 heads x 128, intermediate 3072),
  ragged texts, f32: every embedding within cosine 0.99999 of the f64 oracle
  and 2e-4 max-abs; bf16 (weights rounded to bf16, the oracle on those same
  weights): cosine >= 0.999 (28 bf16 roundings per layer of activations).
- Configuration 1 at full size (28 layers, vocab 151,669, 8 texts of
  U[16, 256] tokens = 778 tokens), f32: cosine >= 0.9999 against the oracle
  in f32 (the north star's pooled-embedding bound).
- The runner refuses ids outside the vocabulary and empty texts on the host,
  and weights of another shape, dtype or device when it is built.
"""
import numpy as np
import pytest

from oracle import attention as oa
from oracle import qwen3 as oq

pytestmark = pytest.mark.gpu


def _to_device(weights, torch, dev, dtype):
    return {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev).to(dtype) for k, v in weights.items()}


def _cosines(a, b):
    a = a / np.linalg.norm(a, axis=1, keepdims=True)
    b = b / np.linalg.norm(b, axis=1, keepdims=True)
    return (a * b).sum(1)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_two_layers_full_width(dtype, cuda, inl):
    import torch
    cfg = oq.Qwen3Config(vocab=2048, layers=2)
    w = oq.random_weights(cfg, seed=1)
    td = torch.float32 if dtype == "f32" else torch.bfloat16
    wd = _to_device(w, torch, cuda, td)
    if dtype == "bf16":   # the oracle runs on the bf16-rounded weights
        w = {k: v.float().cpu().numpy() for k, v in wd.items()}
    lengths = [1, 17, 200, 64, 129, 3]
    ids = np.random.default_rng(2).integers(0, cfg.vocab, sum(lengths))
    cu = oa.cu_from_lengths(lengths)
    print(f"case=qwen3_2layer {dtype} lengths={lengths}", flush=True)
    enc = inl.Qwen3Encoder(cfg, wd, max_positions=256)
    got = enc.encode(ids, cu.tolist()).cpu().numpy().astype(np.float64)
    enc.close()
    ref = oq.encode(w, cfg, ids, cu)
    cos = _cosines(got, ref)
    err = np.abs(got - ref).max()
    print(f"qwen3_2layer {dtype}: min cosine {cos.min():.8f}, max abs {err:.3g}", flush=True)
    assert np.allclose(np.linalg.norm(got, axis=1), 1.0, atol=1e-5)
    if dtype == "f32":
        assert cos.min() >= 0.99999 and err <= 2e-4
    else:
        assert cos.min() >= 0.999


def test_config1_full_size_f32(cuda, inl):
    """28 layers of the 0.6B shape with random f32 weights; the oracle runs in
    f32 on the host (about 0.7 TFLOP)."""
    import torch
    from inl_hip import workloads
    cfg = oq.QWEN3_0_6B
    lengths = workloads.uniform_lengths(8, 16, 256)
    assert sum(lengths) == 778
    w = oq.random_weights(cfg, seed=0)
    ids = np.random.default_rng(0).integers(0, cfg.vocab, sum(lengths))
    cu = oa.cu_from_lengths(lengths)
    print(f"case=qwen3_config1 f32 lengths={lengths}", flush=True)
    enc = inl.Qwen3Encoder(cfg, _to_device(w, torch, cuda, torch.float32), max_positions=256)
    got = enc.encode(ids, cu.tolist()).cpu().numpy().astype(np.float64)
    enc.close()
    ref = oq.encode(w, cfg, ids, cu, dtype=np.float32).astype(np.float64)
    cos = _cosines(got, ref)
    print(f"qwen3_config1 f32: min cosine {cos.min():.8f}, max abs {np.abs(got - ref).max():.3g}", flush=True)
    assert cos.min() >= 0.9999


def test_runner_refuses_bad_inputs(cuda, inl):
    import torch
    cfg = oq.Qwen3Config(vocab=64, hidden=256, intermediate=512, layers=1, heads=4, kv_heads=2, head_dim=64)
    enc = inl.Qwen3Encoder(cfg, _to_device(oq.random_weights(cfg, seed=5), torch, cuda, torch.float32),
                           max_positions=32)
    with pytest.raises(inl.InlError, match="outside the vocabulary"):
        enc.encode([1, 2, 64], [0, 3])
    with pytest.raises(inl.InlError, match="empty"):
        enc.encode([1, 2], [0, 2, 2])
    with pytest.raises(inl.InlError, match="max_positions"):
        enc.encode(list(range(1, 34)), [0, 33])
    out = enc.encode([1, 2, 3], [0, 3])
    torch.cuda.synchronize()
    assert np.isfinite(out.cpu().numpy()).all()
    enc.close()
    # weights of another shape, dtype or device are refused before any launch
    w = _to_device(oq.random_weights(cfg, seed=5), torch, cuda, torch.float32)
    w["layers.0.mlp.down_proj.weight"] = w["layers.0.mlp.down_proj.weight"][:, :-8]
    with pytest.raises(inl.InlError, match="shape"):
        inl.Qwen3Encoder(cfg, w, max_positions=32)
    w = _to_device(oq.random_weights(cfg, seed=5), torch, cuda, torch.float32)
    w["norm.weight"] = w["norm.weight"].cpu()
    with pytest.raises(inl.InlError, match="not a device tensor"):
        inl.Qwen3Encoder(cfg, w, max_positions=32)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_graph_replays_match_eager(dtype, cuda, inl):
    """The runner's launch-sequence graph (captured on a shape's second call,
    replayed after) gives bit-identical embeddings to eager launches, for
    new ids on every call, with eager work of another encoder and
    synchronisations between the replays; a new shape drops the graph and
    the first shape builds it again."""
    import torch
    cfg = oq.Qwen3Config(vocab=2048, layers=2)
    td = torch.float32 if dtype == "f32" else torch.bfloat16
    wd = _to_device(oq.random_weights(cfg, seed=3), torch, cuda, td)
    eager = inl.Qwen3Encoder(cfg, wd, max_positions=256)
    eager.set_graphs(False)
    graph = inl.Qwen3Encoder(cfg, wd, max_positions=256)
    rng = np.random.default_rng(7)

    def run(lengths, calls):
        cu = oa.cu_from_lengths(lengths).tolist()
        out = torch.empty((len(lengths), cfg.hidden), dtype=torch.float32, device=cuda)
        ws = torch.empty(graph.workspace_bytes(cu) + 256, dtype=torch.uint8, device=cuda)
        for i in range(calls):
            ids = rng.integers(0, cfg.vocab, sum(lengths))
            got = graph.encode(ids, cu, out=out, workspace=ws).clone()
            want = eager.encode(ids, cu)
            torch.cuda.synchronize()
            held = graph.graph_info()
            print(f"{dtype} {lengths} call {i}: graph info {held}", flush=True)
            assert torch.equal(got, want), f"call {i} differs by {(got - want).abs().max().item():.3g}"
            if i >= 1:
                assert held == (True, True), "the second call of a shape should leave a graph held"

    run([1, 17, 200, 64, 129, 3], 5)
    run([5, 40], 3)
    run([1, 17, 200, 64, 129, 3], 3)
    eager.close()
    graph.close()
