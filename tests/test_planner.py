"""Packed batch planner: oracle pins and the C-ABI host entry point.

The reference's planners (crates/inl-sparse/src/native.rs:557-582,
crates/inl-late/src/native.rs:694-719, crates/inl-text/src/native.rs:698-735)
split inputs in order under an input cap and a PADDED-token cap; the packed
planner caps real tokens. The oracle's padded planner is pinned on the
reference's own test cases (crates/inl-sparse/src/native.rs:816-835,
crates/inl-text/src/native.rs:906-918); the packed planner on the same cases,
on a brute-force optimum and on the padded planner's batch count.
No GPU needed: the planner is host code.
"""
import numpy as np
import pytest

from oracle import planner as op


SPARSE_CASE = [5, 5, 200, 5, 5, 5, 90, 90, 90]


def _check_cover(batches, lengths, cap_items, cap_tokens, cost):
    nxt = 0
    for r in batches:
        assert r.start == nxt and len(r) >= 1
        assert len(r) <= cap_items
        assert len(r) == 1 or cost([lengths[i] for i in r]) <= cap_tokens
        nxt = r.stop
    assert nxt == len(lengths)


def test_oracle_padded_plan_matches_reference_tests():
    # crates/inl-sparse/src/native.rs:816-835
    b = op.padded_plan(SPARSE_CASE, 4, 100)
    _check_cover(b, SPARSE_CASE, 4, 100, lambda x: len(x) * max(x))
    assert b == [range(0, 2), range(2, 3), range(3, 6), range(6, 7), range(7, 8), range(8, 9)]
    assert op.padded_plan([], 4, 100) == []
    assert op.padded_plan([500], 4, 100) == [range(0, 1)]
    # crates/inl-text/src/native.rs:906-918: 130 short texts, batch size 64
    assert op.padded_plan([40] * 130, 64, 16384) == [range(0, 64), range(64, 128), range(128, 130)]
    # crates/inl-sparse/src/native.rs:843-860: sorting cuts padding
    alt = [20 if i % 2 == 0 else 400 for i in range(64)]
    padded = lambda ls: sum(len(r) * max(ls[i] for i in r) for r in op.padded_plan(ls, 64, 2048))
    assert padded(sorted(alt, reverse=True)) * 10 < padded(alt) * 7


def test_oracle_packed_plan_is_optimal_on_small_inputs():
    rng = np.random.default_rng(3)
    for _ in range(300):
        n = int(rng.integers(0, 9))
        ls = [int(x) for x in rng.integers(0, 60, size=n)]
        items, cap = int(rng.integers(1, 5)), int(rng.integers(1, 120))
        b = op.packed_plan(ls, items, cap)
        _check_cover(b, ls, items, cap, lambda x: sum(max(v, 1) for v in x))
        assert len(b) == op.min_batches(ls, items, cap)


def test_oracle_packed_never_needs_more_batches_than_padded():
    rng = np.random.default_rng(4)
    for _ in range(200):
        ls = [int(x) for x in rng.integers(1, 2048, size=int(rng.integers(1, 200)))]
        items, cap = int(rng.integers(1, 80)), int(rng.integers(512, 40000))
        assert len(op.packed_plan(ls, items, cap)) <= len(op.padded_plan(ls, items, cap))


def test_library_matches_oracle(inl):
    rng = np.random.default_rng(5)
    cases = [(SPARSE_CASE, 4, 100), ([], 4, 100), ([500], 4, 100), ([0, 0, 0], 2, 1),
             ([40] * 130, 64, 16384), ([1, 1, 1, 1, 1], 2, 1000), ([5000, 10, 10], 8, 100)]
    for _ in range(200):
        ls = [int(x) for x in rng.integers(0, 3000, size=int(rng.integers(0, 300)))]
        cases.append((ls, int(rng.integers(1, 100)), int(rng.integers(1, 50000))))
    for ls, items, cap in cases:
        assert inl.plan_packed_batches(ls, items, cap) == op.packed_plan(ls, items, cap), (ls, items, cap)
    # packed form of the reference case: same split here, every batch within 100 real tokens
    assert inl.plan_packed_batches(SPARSE_CASE, 4, 100) == op.padded_plan(SPARSE_CASE, 4, 100)


def test_library_rejects_bad_arguments(inl):
    for args in [([1, 2], 0, 10), ([1, 2], 3, 0), ([1, -2], 3, 10)]:
        with pytest.raises(inl.InlError):
            inl.plan_packed_batches(*args)


def test_config2_mix_fits_fewer_packed_batches(inl):
    """The benchmark mix (713 texts, median 180) in reference order: under
    the reference's default caps of 64 inputs and 4,096 tokens the packed
    planner needs fewer batches than the padded one."""
    from inl_hip import workloads
    lens = workloads.qwen3_op_lengths()
    # crates/inl-text/src/native.rs:29: DEFAULT_MAX_BATCH_TOKENS = 4096
    packed = inl.plan_packed_batches(lens, 64, 4096)
    padded = op.padded_plan(lens, 64, 4096)
    assert sum(len(r) for r in packed) == len(lens)
    assert len(packed) < len(padded)
    assert all(len(r) == 1 or sum(lens[i] for i in r) <= 4096 for r in packed)
