"""Batch planner oracle (pure Python). TEST INFRASTRUCTURE ONLY - never on
the product path.

``padded_plan`` restates the reference's padded planner; ``packed_plan`` is the
same greedy split with the padded-token cap (inputs x longest) replaced by the
real-token cap (sum of lengths) that a packed varlen batch costs;
``min_batches`` is the brute-force optimum that pins the greedy split on small
inputs.
"""
from __future__ import annotations

from functools import lru_cache


def padded_plan(lengths, batch_size, max_batch_tokens):
    """crates/inl-sparse/src/native.rs:557-582 (identical to
    crates/inl-late/src/native.rs:694-719): consecutive batches of at most
    ``batch_size`` inputs and ``len * max(length.max(1))`` padded tokens; the
    first input of a batch is always taken."""
    out, start, padded = [], 0, 0
    for i, n in enumerate(lengths):
        cand_padded = max(padded, max(n, 1))
        cand_len = i - start + 1
        if i > start and (cand_len > batch_size or cand_len * cand_padded > max_batch_tokens):
            out.append(range(start, i))
            start, padded = i, max(n, 1)
        else:
            padded = cand_padded
    if start < len(lengths):
        out.append(range(start, len(lengths)))
    return out


def packed_plan(lengths, batch_size, max_tokens):
    """The split above with ``sum(length.max(1))`` in place of the padded
    count (crates/inl-ane/src/layout.rs:258-456 packs texts the same way: a
    segment per text, no padding rows)."""
    out, start, tokens = [], 0, 0
    for i, n in enumerate(lengths):
        n = max(n, 1)
        if i > start and (i - start + 1 > batch_size or tokens + n > max_tokens):
            out.append(range(start, i))
            start, tokens = i, 0
        tokens += n
    if start < len(lengths):
        out.append(range(start, len(lengths)))
    return out


def min_batches(lengths, batch_size, max_tokens):
    """Fewest consecutive batches under the packed caps (a single input may
    exceed ``max_tokens`` alone), by dynamic programming over split points."""
    n = len(lengths)

    def ok(s, e):
        return e - s == 1 or (e - s <= batch_size and sum(max(x, 1) for x in lengths[s:e]) <= max_tokens)

    @lru_cache(maxsize=None)
    def best(s):
        if s == n:
            return 0
        return min(1 + best(e) for e in range(s + 1, n + 1) if ok(s, e))

    return best(0)
