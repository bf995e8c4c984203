"""AddressSanitizer + UndefinedBehaviorSanitizer run of the library's host
code and of the oracle's C restatement, on the CPU.

Usage: ``python im-not-llm_amd/sanitize.py`` (or ``run()`` from Python).

- Every ``csrc/*.hip`` is compiled as for the library, with the host side
  (only) under ``-fsanitize=address,undefined`` (``-Xarch_host``), and linked
  with ``tests/cpp/sanitize/host_driver.cpp``, which runs the host-side entry
  points over random and adversarial inputs and never launches a kernel (see
  that file), so it runs on a machine without a GPU.
- ``oracle/attn_ref.c`` is compiled with gcc under the same sanitizers and
  linked with ``tests/cpp/sanitize/oracle_driver.c``.

Both binaries are built in a temporary directory and must exit 0 with no
sanitizer report. Leak detection is off: the HIP runtime's own process-
lifetime allocations are not this code's.
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
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
DRIVERS = ROOT / "tests" / "cpp" / "sanitize"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CLANGXX = "/opt/rocm/lib/llvm/bin/clang++"

SAN_HOST = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]
ENV = {"ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:abort_on_error=0",
       "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"}


def _run(cmd, **kw):
    return subprocess.run(cmd, capture_output=True, text=True, **kw)


def _noise(err: str) -> str:
    return "\n".join(l for l in err.splitlines() if "is not a recognized feature" not in l)


def build_host(out_dir: Path) -> Path:
    srcs = sorted(CSRC.glob("*.hip"))
    objs = [out_dir / (s.stem + ".o") for s in srcs]
    base = [HIPCC, "--offload-arch=gfx950", "-O3", "-Xarch_host", "-O1", "-g", "-std=c++17", "-fPIC", f"-I{INCLUDE}",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", *SAN_HOST]
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as pool:
        res = list(pool.map(lambda so: _run([*base, "-c", str(so[0]), "-o", str(so[1])]), zip(srcs, objs)))
    for s, r in zip(srcs, res):
        if r.returncode != 0:
            raise RuntimeError(f"sanitizer build of {s.name} failed:\n{_noise(r.stderr)}")
    drv = out_dir / "host_driver.o"
    r = _run([*base, "-c", str(DRIVERS / "host_driver.cpp"), "-o", str(drv)])
    if r.returncode != 0:
        raise RuntimeError(f"sanitizer build of host_driver.cpp failed:\n{_noise(r.stderr)}")
    # objects only: the clang driver links the HIP runtime and the host sanitizer runtimes
    exe = out_dir / "host_driver"
    r = _run([CLANGXX, "--hip-link", "-fsanitize=address,undefined", str(drv), *map(str, objs),
              "-L/opt/rocm/lib", "-lamdhip64", "-lhipblaslt", "-Wl,-rpath,/opt/rocm/lib", "-o", str(exe)])
    if r.returncode != 0:
        raise RuntimeError(f"sanitizer link failed:\n{_noise(r.stderr)}")
    return exe


def build_oracle(out_dir: Path) -> Path:
    exe = out_dir / "oracle_driver"
    r = _run(["gcc", "-O1", "-g", "-std=c11", "-fopenmp", "-fsanitize=address,undefined",
              "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", str(ROOT / "oracle" / "attn_ref.c"),
              str(DRIVERS / "oracle_driver.c"), "-lm", "-o", str(exe)])
    if r.returncode != 0:
        raise RuntimeError(f"oracle sanitizer build failed:\n{r.stderr}")
    return exe


CANARY = r"""
#include <cstdlib>
int main(int argc, char**) {
  int* p = static_cast<int*>(std::malloc(4 * sizeof(int)));
  const int v = p[4 + argc];   // one past the end (argc >= 1): must be reported
  std::free(p);
  return v == 12345;
}
"""


def canary(out_dir: Path) -> bool:
    """A heap overflow built with the host flags above must be reported:
    proof that the instrumentation is live in this toolchain."""
    src = out_dir / "canary.hip"
    src.write_text(CANARY)
    exe = out_dir / "canary"
    r = _run([HIPCC, "--offload-arch=gfx950", "-O1", "-g", *SAN_HOST, "-c", str(src), "-o", str(exe) + ".o"])
    if r.returncode != 0:
        raise RuntimeError(f"canary build failed:\n{_noise(r.stderr)}")
    r = _run([CLANGXX, "--hip-link", "-fsanitize=address,undefined", str(exe) + ".o", "-L/opt/rocm/lib",
              "-lamdhip64", "-o", str(exe)])
    if r.returncode != 0:
        raise RuntimeError(f"canary link failed:\n{_noise(r.stderr)}")
    r = _run([str(exe)], env=dict(os.environ, **ENV), timeout=60)
    return r.returncode != 0 and "heap-buffer-overflow" in r.stderr


def run(verbose: bool = False) -> dict:
    """Build both drivers, run them; returns {name: last output line}.
    Raises RuntimeError on a build failure, a nonzero exit or a report."""
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    results = {}
    with tempfile.TemporaryDirectory(prefix="inl_sanitize_") as d:
        out = Path(d)
        if not canary(out):
            raise RuntimeError("the sanitizer canary was not reported: instrumentation is not active")
        results["canary"] = "heap-buffer-overflow reported"
        for name, exe in (("host", build_host(out)), ("oracle", build_oracle(out))):
            env = dict(os.environ, **ENV, OMP_NUM_THREADS="4")
            r = _run([str(exe)], env=env, timeout=600)
            text = r.stdout + r.stderr
            if verbose:
                print(text, file=sys.stderr)
            if r.returncode != 0 or "runtime error" in text or "ERROR: AddressSanitizer" in text:
                raise RuntimeError(f"{name} driver failed ({r.returncode}):\n{text[-4000:]}")
            results[name] = r.stdout.strip().splitlines()[-1] if r.stdout.strip() else ""
    return results


if __name__ == "__main__":
    print(run(verbose="-v" in sys.argv))
