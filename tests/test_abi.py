"""The C-ABI library loads on a machine without a GPU, exports every entry
point include/inl_hip.h declares, and validates arguments on the host (no
GPU call is made by these tests)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def _declared():
    text = (ROOT / "include" / "inl_hip.h").read_text()
    return sorted(set(re.findall(r"\b(inl_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    import inl_hip
    lib = ctypes.CDLL(str(inl_hip.library_path()))
    declared = _declared()
    assert len(declared) >= 15
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    assert inl_hip.abi_version() == 1


def test_attention_desc_validation_errors():
    import inl_hip
    cu = [0, 5, 9]
    ok = inl_hip.make_attn_desc(cu, 16, 8, 128, causal=True)
    n = ctypes.c_size_t()
    assert inl_hip._ws_size(ctypes.byref(ok), ctypes.byref(n)) == 0
    assert n.value > 0 and n.value % 16 == 0
    cases = [
        (inl_hip.make_attn_desc(cu, 16, 6, 128, causal=True), -1, "multiple of h_kv"),
        (inl_hip.make_attn_desc(cu, 16, 8, 100, causal=True), -2, "head_dim"),
        (inl_hip.make_attn_desc(cu, 16, 8, 128, causal=True, window=-5), -1, "window"),
        (inl_hip.make_attn_desc([0, 5, 3], 16, 8, 128, causal=True), -1, "nondecreasing"),
        (inl_hip.make_attn_desc([1, 5], 16, 8, 128, causal=True), -1, "cu_seqlens[0]"),
        (inl_hip.make_attn_desc(cu, 16, 8, 128, causal=True, scale=-1.0), -1, "scale"),
        (inl_hip.make_attn_desc(cu, 16, 8, 128, causal=True, q_row_stride=100), -1, "stride"),
        (inl_hip.make_attn_desc(cu, 16, 8, 128, causal=True, flags=8), -1, "flags"),
        (inl_hip.make_attn_desc(cu, 16, 8, 128, causal=True, seq_starts=[-1, 0]), -1, "seq_starts"),
        (inl_hip.make_attn_desc(cu, 16, 8, 128, causal=True, seq_starts=[0, 2**31 - 3]), -1,
         "seq_starts"),
    ]
    for desc, code, word in cases:
        rc = inl_hip._ws_size(ctypes.byref(desc), ctypes.byref(n))
        assert rc == code, (word, rc, inl_hip.last_error())
        assert word in inl_hip.last_error()


def test_workspace_counts_visible_tiles_only():
    """The schedule skips tiles above the causal diagonal and outside the
    window: a causal 2048-token text needs fewer tiles than a full one."""
    import inl_hip
    n = ctypes.c_size_t()
    sizes = {}
    for causal, window in [(True, -1), (False, -1), (False, 64)]:
        d = inl_hip.make_attn_desc([0, 2048], 12, 12, 64, causal=causal, window=window)
        assert inl_hip._ws_size(ctypes.byref(d), ctypes.byref(n)) == 0
        sizes[(causal, window)] = n.value
    # one work item per query block either way; items are 16 bytes
    assert sizes[(True, -1)] == sizes[(False, -1)] == sizes[(False, 64)] > 0


def test_host_helpers_validate():
    import inl_hip
    with pytest.raises(inl_hip.InlError):
        inl_hip.rope_table(7, 1e4, 4)
    with pytest.raises(inl_hip.InlError):
        inl_hip.positions([0, 4, 2])
