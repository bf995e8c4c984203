"""CPU oracle for the encoder attention path. TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU and in plain numpy (float64 unless a
function says otherwise), the arithmetic the reference im-not-llm candle
implementation performs on the encoder attention hot path:

* ``attention``  - the five attention forms (Qwen3 causal GQA, EmbeddingGemma
  bidirectional full/sliding, ModernBERT global/local, Qwen3.5 full attention,
  vision ViT) over padded batches with the reference's additive masks, and the
  packed variable-length form the HIP kernels implement;
* ``prologue``   - per-head RMSNorm and the half-split / partial / axial RoPE;
* ``pooling``    - last-token, mean and SPLADE epilogues, L2 normalisation,
  Matryoshka truncation and the sparse active-term set;
* ``planner``    - the reference's padded batch planner, its packed
  counterpart and a brute-force optimum for small inputs;
* ``cref``       - a ctypes loader for ``attn_ref.c``, the multi-threaded f32
  C restatement used as the CPU baseline.

The tiny EmbeddingGemma 2 and ModernBERT-SPLADE encoders that run the
reference's golden fixtures over these functions (pinning the forms in situ)
live beside the tests, in ``tests/tiny_encoders.py``.

Parity unpinned: none of the functions here. Each is checked against the
reference's known answers, its golden fixtures or a closed form in
``tests/test_oracle_*.py``; the RoPE tables and the partial and axial
rotations in ``tests/test_oracle_rope_pins.py``.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker: the
product path (``im-not-llm_amd/``) never calls into it.

Every function cites the reference file:line it follows (paths relative to
the reference repository root).
"""
