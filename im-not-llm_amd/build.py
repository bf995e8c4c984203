"""Build the gfx950 library ``inl_hip/libinl_hip.so`` in-tree with hipcc.

Usage: ``python im-not-llm_amd/build.py`` (or ``build()`` from Python).
The shared object is written next to the Python binding so it travels with
the source tree; it is listed in .gitignore.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "inl_hip" / "libinl_hip.so"
INCLUDE = PKG.parent / "include"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed fp32 VALU instructions (v_pk_fma_f32 and the like) are disabled for
# all device code: some of their forms have produced wrong results without
# any error on these GPUs. hipcc's host pass warns that it does not know the
# feature, which is harmless.
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", f"-I{INCLUDE}",
]
# hipBLASLt (the encoder's plain GEMMs). When torch is loaded first, its
# bundled copy of the same soname is the one bound.
LINK_FLAGS = [f"--offload-arch={ARCH}", "-shared", "-fPIC", "-L/opt/rocm/lib", "-lhipblaslt",
              "-Wl,-rpath,/opt/rocm/lib"]


# Per-source flags. attn_wide.hip (head_dim 256, one wave per SIMD, ~450 of
# 512 registers): MFMA accumulators in VGPRs, so that O^T, which the softmax
# rescales with VALU instructions, is not copied between AGPRs and VGPRs on
# every tile; the MFMA operands then take the AGPRs.
EXTRA = {
    "attn_wide.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}

# Sources whose kernels issue global loads from inline asm and wait for them
# with hand-counted `s_waitcnt vmcnt`: the compiler believes an asm load's
# destination register is written when the asm statement ends, so a register
# spill could store that register, or hand it to another value, while the
# load is still in flight. Their kernels must use no scratch; the build reads
# the compiler's resource-usage remarks and fails if any of them does.
NO_SCRATCH = {"attn_pp.hip", "attn_pp64.hip", "attn_wide.hip", "gemm.hip", "splade_decoder.hip"}
RESOURCE_REMARKS = ["-Rpass-analysis=kernel-resource-usage", "-fno-caret-diagnostics"]
# The same sources are also compiled to a device assembly listing, which
# asmcheck.py walks for instructions that name a register an inline-asm
# load has not yet written (a copy placed before the load's wait). These
# have register-writing asm loads; the check must find some there, so that a
# listing format the parser no longer reads cannot pass silently.
ASM_REGISTER_LOADS = {"attn_pp.hip", "attn_pp64.hip", "attn_wide.hip"}


def scratch_users(remarks: str) -> list[str]:
    """Kernels that the compiler's kernel-resource-usage remarks report with
    a nonzero ScratchSize (bytes per lane)."""
    return [f"{name} ({size} B/lane)" for name, size in parse_scratch(remarks) if size]


def parse_scratch(remarks: str) -> list[tuple[str, int]]:
    """(function name, ScratchSize) of every function the kernel-resource-usage
    remarks describe. A function whose remark block has no ScratchSize line
    is reported with size -1, so that a format change cannot pass silently."""
    out, name = [], None
    for line in remarks.splitlines():
        if "Function Name:" in line:
            if name is not None:
                out.append((name, -1))
            name = line.split("Function Name:", 1)[1].split()[0]
        elif "ScratchSize [bytes/lane]:" in line and name is not None:
            out.append((name, int(line.split("ScratchSize [bytes/lane]:", 1)[1].split()[0])))
            name = None
    if name is not None:
        out.append((name, -1))
    return out


def check_no_scratch(src_name: str, remarks: str) -> None:
    """Raise unless the remarks describe at least one kernel, every described
    function has a ScratchSize, and none of them is nonzero."""
    parsed = parse_scratch(remarks)
    if not parsed:
        raise RuntimeError(f"{src_name}: no kernel-resource-usage remarks were parsed, so the no-scratch "
                           "check cannot be made")
    unsized = [n for n, s in parsed if s < 0]
    if unsized:
        raise RuntimeError(f"{src_name}: remarks without a ScratchSize for " + ", ".join(unsized))
    users = scratch_users(remarks)
    if users:
        raise RuntimeError(f"{src_name}: kernels with inline-asm loads use scratch: " + ", ".join(users))


def check_inflight(src_name: str, listing: str) -> None:
    """Raise if the device listing of a source with inline-asm loads names a
    register before the wait that retires its load (see asmcheck.py)."""
    sys.path.insert(0, str(PKG))
    try:
        import asmcheck
    finally:
        sys.path.pop(0)
    loads = asmcheck.count_asm_loads(listing)
    if src_name in ASM_REGISTER_LOADS and loads == 0:
        raise RuntimeError(f"{src_name}: no register-writing inline-asm loads found in its listing, so the "
                           "in-flight register check cannot be made")
    bad = asmcheck.check_listing(listing)
    if bad:
        shown = "\n".join(str(v) for v in bad[:10])
        raise RuntimeError(f"{src_name}: {len(bad)} instructions name registers whose inline-asm loads are "
                           f"still in flight:\n{shown}")


def sources():
    return sorted(CSRC.glob("*.hip"))


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    return res.returncode, err


def build(verbose: bool = False) -> Path:
    """Compile every HIP source into the shared library; raises on failure."""
    if not Path(HIPCC).exists() and shutil.which(HIPCC) is None:
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    tmp = OUT.with_suffix(".so.tmp")
    with tempfile.TemporaryDirectory(prefix="inl_hip_build_") as objdir:
        jobs, listings = [], []
        for src in sources():
            obj = Path(objdir) / (src.stem + ".o")
            cmd = [HIPCC, *FLAGS, "-c", *EXTRA.get(src.name, []),
                   *(RESOURCE_REMARKS if src.name in NO_SCRATCH else []), str(src), "-o", str(obj)]
            jobs.append((src, obj, cmd))
            if src.name in NO_SCRATCH:
                lst = Path(objdir) / (src.stem + ".s")
                listings.append((src, lst, [HIPCC, *FLAGS, "-S", "--cuda-device-only", *EXTRA.get(src.name, []),
                                            str(src), "-o", str(lst)]))
        with ThreadPoolExecutor(max_workers=min(len(jobs), os.cpu_count() or 1, 8)) as pool:
            results = list(pool.map(lambda j: _run(j[2]), jobs + listings))
        for (src, _, _), (rc, err) in zip(jobs, results):
            if rc != 0:
                raise RuntimeError(f"hipcc failed on {src.name} ({rc}):\n{err}")
            if src.name in NO_SCRATCH:
                check_no_scratch(src.name, err)
                err = "\n".join(l for l in err.splitlines() if "kernel-resource-usage" not in l)
            if verbose and err.strip():
                print(err, file=sys.stderr)
        for (src, lst, _), (rc, err) in zip(listings, results[len(jobs):]):
            if rc != 0:
                raise RuntimeError(f"hipcc -S failed on {src.name} ({rc}):\n{err}")
            check_inflight(src.name, lst.read_text())
        rc, err = _run([HIPCC, *LINK_FLAGS, *(str(o) for _, o, _ in jobs), "-o", str(tmp)])
        if rc != 0:
            raise RuntimeError(f"hipcc link failed ({rc}):\n{err}")
    os.replace(tmp, OUT)
    _build_test_shims()
    return OUT


# Test shims under tests/cpp/: host C++ that drives the library's C++
# interface (include/inl_attention.hpp) from pytest through ctypes. Built
# here, beside the library, so that no test compiles anything.
TEST_CPP = PKG.parent / "tests" / "cpp"


def _build_test_shims():
    if not TEST_CPP.is_dir():
        return
    for src in sorted(TEST_CPP.glob("*.cpp")):
        out = TEST_CPP / f"lib{src.stem}.so"
        rel = os.path.relpath(OUT.parent, TEST_CPP)
        rc, err = _run([HIPCC, "-O2", "-std=c++17", "-fPIC", "-shared", f"-I{INCLUDE}", str(src),
                        f"-L{OUT.parent}", "-linl_hip", f"-Wl,-rpath,$ORIGIN/{rel}", "-o", str(out)])
        if rc != 0:
            raise RuntimeError(f"hipcc failed on {src.name} ({rc}):\n{err}")


if __name__ == "__main__":
    print(build(verbose=True))
