"""The C-ABI library loads on a machine without a GPU, exports every entry
point include/inl_hip.h declares, and validates arguments on the host (no
GPU call is made by these tests)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def _declared():
    text = "".join(p.read_text() for p in sorted((ROOT / "include").glob("*.h")))
    return sorted(set(re.findall(r"\b(inl_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    import inl_hip
    lib = ctypes.CDLL(str(inl_hip.library_path()))
    declared = _declared()
    assert len(declared) >= 28
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    assert inl_hip.abi_version() == 2


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


def test_kernel_selection_counts_output_row_bytes():
    """The fast kernels address a text's rows with 32-bit offsets. A Qwen3
    text of 524,288 tokens has 4 KiB bf16 q rows (2.1 GiB per text) but 8 KiB
    f32 output rows (4.3 GiB): it must take the generic kernel, which uses
    64-bit offsets. The same text with bf16 output fits, and so does a short
    text with f32 output; a wide caller output stride counts too."""
    import inl_hip
    long = [0, 524_288]
    mk = lambda cu, **kw: inl_hip.make_attn_desc(cu, 16, 8, 128, causal=True, dtype="bf16", **kw)
    assert inl_hip.kernel_name(mk(long, out_dtype="bf16")) == "attn_pp_kernel<128, 64>"
    assert inl_hip.kernel_name(mk(long, out_dtype="f32")).startswith("attn_fwd_kernel<bf16, 128")
    assert inl_hip.kernel_name(mk([0, 4096], out_dtype="f32")) == "attn_pp_kernel<128, 64>"
    assert inl_hip.kernel_name(mk(long, out_dtype="bf16", o_row_stride=8192)).startswith("attn_fwd_kernel")
    # the other fast kernels by shape
    assert inl_hip.kernel_name(inl_hip.make_attn_desc([0, 100], 3, 1, 256, causal=False)) == \
        "attn_wide_kernel<256, 32>"
    assert inl_hip.kernel_name(inl_hip.make_attn_desc([0, 100], 12, 12, 64, causal=False)) == \
        "attn_pp64_kernel<64, 64>"
    assert inl_hip.kernel_name(inl_hip.make_attn_desc([0, 100], 12, 12, 64, causal=False, dtype="f32")) == \
        "attn_fwd_kernel<f32, 64, 64, 4>"
    assert inl_hip.kernel_name(inl_hip.make_attn_desc([0, 100], 16, 8, 128, causal=True,
                                                      flags=inl_hip.ATTN_PV_BF16)).endswith("pv_bf16>")


def test_tile_ranges_fit_their_16_bit_fields():
    """A work item packs its first and last key tile into 16 bits each. With
    32-key tiles (head_dim 256) a text of 2^21 - 1 tokens needs 65,536 tiles
    and is refused; one of 2^21 - 33 tokens needs 65,535 and is planned, with
    and without a window."""
    import inl_hip
    n = ctypes.c_size_t()
    for window in (-1, 512):
        bad = inl_hip.make_attn_desc([0, 2**21 - 1], 3, 1, 256, causal=False, window=window)
        assert inl_hip._ws_size(ctypes.byref(bad), ctypes.byref(n)) == -2
        assert "65535 key tiles" in inl_hip.last_error()
        ok = inl_hip.make_attn_desc([0, 2**21 - 33], 3, 1, 256, causal=False, window=window)
        assert inl_hip._ws_size(ctypes.byref(ok), ctypes.byref(n)) == 0, inl_hip.last_error()


def test_binding_refuses_tensors_the_kernels_would_overrun():
    """The library sees pointers only, so the Python binding checks that q, k,
    v and out hold every row the desc covers, with its dtypes and strides,
    before it calls the library (CPU tensors: the device check comes last)."""
    import torch
    import inl_hip
    cu = [0, 5, 9]
    desc = inl_hip.make_attn_desc(cu, 4, 2, 16, causal=True, dtype="bf16", out_dtype="f32")
    mk = lambda n, h, dt=torch.bfloat16: torch.zeros(n, h, 16, dtype=dt)
    good = (mk(9, 4), mk(9, 2), mk(9, 2), mk(9, 4, torch.float32))
    with pytest.raises(inl_hip.InlError, match="not a device tensor"):
        inl_hip._check_tensors(desc, *good)
    cases = [
        ((mk(8, 4), mk(9, 2), mk(9, 2), mk(9, 4, torch.float32)), "q: 8 rows, the desc covers 9"),
        ((mk(9, 4), mk(9, 2), mk(7, 2), mk(9, 4, torch.float32)), "v: 7 rows"),
        ((mk(9, 4), mk(9, 2), mk(9, 2), mk(8, 4, torch.float32)), "out: 8 rows"),
        ((mk(9, 4), mk(9, 2, torch.float32), mk(9, 2), mk(9, 4, torch.float32)), "k: dtype"),
        ((mk(9, 4), mk(9, 2), mk(9, 2), mk(9, 4)), "out: dtype"),
        ((mk(9, 4), mk(9, 3), mk(9, 2), mk(9, 4, torch.float32)), "k: shape"),
    ]
    for tensors, msg in cases:
        with pytest.raises(inl_hip.InlError, match=msg.replace("[", r"\[")):
            inl_hip._check_tensors(desc, *tensors)
    # padded batches: seq_starts move the last text's end
    padded = inl_hip.make_attn_desc(cu, 4, 2, 16, causal=True, dtype="bf16", out_dtype="f32",
                                    seq_starts=[0, 12])
    assert inl_hip.desc_rows(padded) == 16
    with pytest.raises(inl_hip.InlError, match="the desc covers 16"):
        inl_hip._check_tensors(padded, *good)


def test_encoder_weights_are_checked_against_the_configuration():
    """The encoder runners read every weight at the size the configuration
    gives, so the binding checks each tensor's dtype and shape before the
    device (CPU tensors here: the device check comes last)."""
    import torch
    import inl_hip
    w = {"a": torch.zeros(6, 4), "b": torch.zeros(6, 4, dtype=torch.bfloat16)}
    with pytest.raises(inl_hip.InlError, match="weight c is missing"):
        inl_hip._weight(w, "c", (6, 4), torch.float32)
    with pytest.raises(inl_hip.InlError, match="weight b: dtype"):
        inl_hip._weight(w, "b", (6, 4), torch.float32)
    with pytest.raises(inl_hip.InlError, match=r"weight a: shape \(6, 4\), the configuration needs \(4, 6\)"):
        inl_hip._weight(w, "a", (4, 6), torch.float32)
    with pytest.raises(inl_hip.InlError, match="weight a: not a device tensor"):
        inl_hip._weight(w, "a", (6, 4), torch.float32)


def test_gdn_entry_points_validate_on_the_host():
    """Shapes outside what the gated-delta-net kernels hold are refused
    before any device call (null device pointers are never dereferenced)."""
    import inl_hip
    L = inl_hip._lib
    bad = inl_hip.INL_E_INVALID if hasattr(inl_hip, "INL_E_INVALID") else -1
    # taps beyond 8, zero channels
    assert L.inl_gdn_conv_fwd(ctypes.c_int64(4), 1, None, 8, 9, 0, None, ctypes.c_int64(0), None, None,
                              ctypes.c_int64(0), None) == bad
    assert L.inl_gdn_conv_fwd(ctypes.c_int64(4), 1, None, 0, 4, 0, None, ctypes.c_int64(0), None, None,
                              ctypes.c_int64(0), None) == bad
    # no rows: nothing to do
    assert L.inl_gdn_conv_fwd(ctypes.c_int64(0), 1, None, 8, 4, 0, None, ctypes.c_int64(0), None, None,
                              ctypes.c_int64(0), None) == 0
    # key_dim 129, value heads not a multiple of key heads
    args = (ctypes.c_int64(4), 1, None)
    assert L.inl_gdn_rule_fwd(*args, 1, 1, 129, 64, 0, None, ctypes.c_int64(0), None, None, ctypes.c_int64(0),
                              None, ctypes.c_int64(0), None) == bad
    assert L.inl_gdn_rule_fwd(*args, 2, 3, 64, 64, 0, None, ctypes.c_int64(0), None, None, ctypes.c_int64(0),
                              None, ctypes.c_int64(0), None) == bad
    # a stride shorter than a row
    assert L.inl_gdn_rule_fwd(*args, 1, 1, 8, 8, 0, ctypes.c_void_p(16), ctypes.c_int64(8), ctypes.c_void_p(16),
                              ctypes.c_void_p(16), ctypes.c_int64(0), ctypes.c_void_p(16), ctypes.c_int64(0),
                              None) == bad
    # gated norm: value_dim 129, core dtype neither f32 nor the model dtype
    assert L.inl_gdn_gated_norm_fwd(ctypes.c_int64(4), 2, 129, 0, 0, None, ctypes.c_int64(0), None,
                                    ctypes.c_int64(0), None, ctypes.c_float(1e-6), None, ctypes.c_int64(0), None) == bad
    assert L.inl_gdn_gated_norm_fwd(ctypes.c_int64(4), 2, 64, 0, 1, None, ctypes.c_int64(0), None,
                                    ctypes.c_int64(0), None, ctypes.c_float(1e-6), None, ctypes.c_int64(0), None) == bad
    # inverse: size 65
    assert L.inl_gdn_unit_lower_inverse_fwd(ctypes.c_int64(3), 65, None, None, None) == bad
    assert L.inl_gdn_gates_fwd(ctypes.c_int64(4), 0, 0, None, ctypes.c_int64(0), None, ctypes.c_int64(0), None,
                               None, None, None, None) == bad
    assert "value_dim" in inl_hip.last_error() or "gdn" in inl_hip.last_error()


def test_asm_load_kernels_use_no_scratch():
    """Kernels that issue global loads from inline asm must compile without
    scratch: the build reads the compiler's resource remarks for them and
    fails on a spill. Checks the parser on the remark text the compiler
    prints, and that those sources are the ones with inline-asm loads."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("inl_build", ROOT / "im-not-llm_amd" / "build.py")
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    text = ("x.hip:62:1: remark: Function Name: _Z1kv [-Rpass-analysis=kernel-resource-usage]\n"
            "x.hip:62:1: remark:     VGPRs: 237 [-Rpass-analysis=kernel-resource-usage]\n"
            "x.hip:62:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]\n"
            "x.hip:90:1: remark: Function Name: _Z1jv [-Rpass-analysis=kernel-resource-usage]\n"
            "x.hip:90:1: remark:     ScratchSize [bytes/lane]: 284 [-Rpass-analysis=kernel-resource-usage]\n")
    assert b.scratch_users(text) == ["_Z1jv (284 B/lane)"]
    with pytest.raises(RuntimeError, match="use scratch"):
        b.check_no_scratch("x.hip", text)
    # no remarks at all (flag ignored, remarks elsewhere) and a block with no
    # ScratchSize line both fail the check instead of passing it
    with pytest.raises(RuntimeError, match="no kernel-resource-usage remarks"):
        b.check_no_scratch("x.hip", "")
    with pytest.raises(RuntimeError, match="without a ScratchSize"):
        b.check_no_scratch("x.hip", text.splitlines()[0] + "\n")
    b.check_no_scratch("x.hip", "\n".join(text.splitlines()[:3]))
    asm_loads = {p.name for p in (ROOT / "im-not-llm_amd" / "csrc").glob("*.hip")
                 if re.search(r'asm volatile\("buffer_load', p.read_text())
                 or re.search(r'vmcnt\(%', p.read_text()) or '"attn_stream.hpp"' in p.read_text()}
    assert asm_loads <= b.NO_SCRATCH, asm_loads - b.NO_SCRATCH


def test_no_scratch_remarks_are_parsed_from_a_real_compile(tmp_path):
    """Compile the smallest no-scratch source with the build's own flags and
    remark options: the compiler's remarks must describe its kernels, so the
    build's check sees real input, not an empty string."""
    import importlib.util
    import subprocess
    spec = importlib.util.spec_from_file_location("inl_build", ROOT / "im-not-llm_amd" / "build.py")
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    src = ROOT / "im-not-llm_amd" / "csrc" / "splade_decoder.hip"
    assert src.name in b.NO_SCRATCH
    r = subprocess.run([b.HIPCC, *b.FLAGS, "-c", *b.RESOURCE_REMARKS, str(src), "-o", str(tmp_path / "s.o")],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    parsed = b.parse_scratch(r.stderr)
    kernels = [n for n, _ in parsed if "splade_decoder_max_kernel" in n]
    assert kernels and all(s == 0 for _, s in parsed), parsed
    b.check_no_scratch(src.name, r.stderr)


def _asmcheck():
    import importlib.util
    import sys
    spec = importlib.util.spec_from_file_location("inl_asmcheck", ROOT / "im-not-llm_amd" / "asmcheck.py")
    m = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = m   # dataclasses look their module up there
    spec.loader.exec_module(m)
    return m


def _listing(body):
    return "\t.globl\tk\nk:\n" + "\n".join("\t" + l if not l.endswith(":") else l for l in body) + "\n.Lfunc_end0:\n"


def test_inflight_register_check_on_listings():
    """The build walks the device listing of every kernel with inline-asm
    loads for instructions that name a register whose load is still in
    flight (the compiler treats the asm output as written when the asm
    statement ends). A copy before the wait is caught, on any path of the
    control flow; a wait that has enough younger memory operations behind it
    retires the load; direct-to-LDS loads write no register."""
    ac = _asmcheck()
    load = [";;#ASMSTART", "buffer_load_dwordx4 v[4:7], v1, s[0:3], 0 offen offset:32", ";;#ASMEND"]
    dma = [";;#ASMSTART", "buffer_load_dwordx4 v2, s[0:3], 0 offen lds", ";;#ASMEND"]
    copy = ["v_mov_b64_e32 v[8:9], v[6:7]"]
    end = ["s_endpgm"]
    bad = ac.check_listing(_listing(load + copy + ["s_waitcnt vmcnt(0)"] + end))
    assert len(bad) == 1 and bad[0].registers == ["v6", "v7"], bad
    assert ac.check_listing(_listing(load + ["s_waitcnt vmcnt(0)"] + copy + end)) == []
    # vmcnt(1) retires the load only with one younger memory operation
    assert ac.check_listing(_listing(load + dma + ["s_waitcnt vmcnt(1)"] + copy + end)) == []
    assert len(ac.check_listing(_listing(load + ["s_waitcnt vmcnt(1)"] + copy + end))) == 1
    # the register-writing load of a wait-free branch reaches the copy at the join
    branchy = load + ["s_cbranch_scc1 .LBB0_2", "s_waitcnt vmcnt(0)", "s_branch .LBB0_3", ".LBB0_2:",
                      "s_nop 0", ".LBB0_3:"] + copy + end
    assert len(ac.check_listing(_listing(branchy))) == 1
    both = load + ["s_cbranch_scc1 .LBB0_2", "s_waitcnt vmcnt(0)", "s_branch .LBB0_3", ".LBB0_2:",
                   "s_waitcnt vmcnt(0)", ".LBB0_3:"] + copy + end
    assert ac.check_listing(_listing(both)) == []
    # a loop: the load at the bottom reaches the copy at the top on the next
    # turn; the load itself may write registers still in flight from its
    # previous turn (loads write in issue order, the younger value stays)
    loop = [".LBB0_1:"] + copy + load + ["s_cbranch_scc1 .LBB0_1", "s_waitcnt vmcnt(0)"] + end
    assert [v.text.split()[0] for v in ac.check_listing(_listing(loop))] == ["v_mov_b64_e32"]
    assert ac.check_listing(_listing(load + load + ["s_waitcnt vmcnt(0)"] + copy + end)) == []
    # ... but not a VALU write into them, nor an address taken from them
    overwrite = ["v_mov_b32_e32 v5, 0"]
    assert len(ac.check_listing(_listing(load + overwrite + ["s_waitcnt vmcnt(0)"] + end))) == 1
    addr = [";;#ASMSTART", "buffer_load_dwordx4 v[8:11], v5, s[0:3], 0 offen", ";;#ASMEND"]
    bad = ac.check_listing(_listing(load + addr + ["s_waitcnt vmcnt(0)"] + end))
    assert len(bad) == 1 and bad[0].registers == ["v5"], bad
    assert ac.count_asm_loads(_listing(load + dma + end)) == 1


def test_inflight_register_check_on_a_real_listing(tmp_path):
    """attn_pp64's listing, compiled with the build's flags, holds its
    register-writing asm loads (the next unit's Q) and names none of their
    registers before the wait that retires them."""
    import importlib.util
    import subprocess
    spec = importlib.util.spec_from_file_location("inl_build", ROOT / "im-not-llm_amd" / "build.py")
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    src = ROOT / "im-not-llm_amd" / "csrc" / "attn_pp64.hip"
    assert src.name in b.ASM_REGISTER_LOADS <= b.NO_SCRATCH
    out = tmp_path / "pp64.s"
    r = subprocess.run([b.HIPCC, *b.FLAGS, "-S", "--cuda-device-only", str(src), "-o", str(out)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    ac = _asmcheck()
    text = out.read_text()
    assert ac.count_asm_loads(text) > 0
    assert ac.check_listing(text) == []
    b.check_inflight(src.name, text)


def test_small_f32_batches_split_their_key_ranges():
    """f32 batches too small to fill the GPU get a key-range split (partial
    outputs in the plan's memory, so a larger workspace); bf16 descs, large
    batches and INL_ATTN_NO_SPLIT do not."""
    import inl_hip
    n = ctypes.c_size_t()

    def ws(cu, dtype, flags=0):
        d = inl_hip.make_attn_desc(cu, 16, 8, 128, causal=True, dtype=dtype, flags=flags)
        assert inl_hip._ws_size(ctypes.byref(d), ctypes.byref(n)) == 0, inl_hip.last_error()
        return n.value

    small = [0, 16, 116, 372, 409, 609, 738, 802, 1052]   # configuration 1's size: 8 texts
    one_slot_group = 8 * 4 * 32 * (8 + 128 * 4)           # head groups x waves x rows x (max, sum, O)
    assert ws(small, "f32") >= ws(small, "f32", inl_hip.ATTN_NO_SPLIT) + one_slot_group
    assert ws(small, "bf16") == ws(small, "bf16", inl_hip.ATTN_NO_SPLIT)
    big = list(range(0, 64 * 2048 + 1, 2048))              # 64 texts x 2048 fill the GPU
    assert ws(big, "f32") == ws(big, "f32", inl_hip.ATTN_NO_SPLIT)
    bad = inl_hip.make_attn_desc(small, 16, 8, 128, causal=True, dtype="f32", flags=4)
    assert inl_hip._ws_size(ctypes.byref(bad), ctypes.byref(n)) != 0
    assert "unknown flags" in inl_hip.last_error()
