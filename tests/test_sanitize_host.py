"""ASan + UBSan run of the library's host code and of the oracle's C
restatement (im-not-llm_amd/sanitize.py), on the CPU: a planted heap
overflow must be reported (the instrumentation is live), then both drivers
(tests/cpp/sanitize/) must finish with no report."""
import shutil
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.skipif(shutil.which("gcc") is None or not Path("/opt/rocm/bin/hipcc").exists(),
                    reason="needs hipcc and gcc")
def test_host_code_and_oracle_are_sanitizer_clean():
    import importlib.util
    spec = importlib.util.spec_from_file_location("inl_sanitize", ROOT / "im-not-llm_amd" / "sanitize.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    res = mod.run()
    assert res["canary"] == "heap-buffer-overflow reported"
    assert res["host"].endswith(" 0 failures") and res["oracle"].endswith(" 0 failures")
