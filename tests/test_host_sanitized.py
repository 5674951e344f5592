"""Host error paths under AddressSanitizer + UndefinedBehaviorSanitizer.

Builds tests/native/host_status (all runtime sources, the CPU oracle and a
driver; host code sanitized) and runs it on the CPU.  The driver forces
every status code the host can produce without a device on a runtime made
with QM_DEVICE_NONE, and checks oracle known answers; any sanitizer report
aborts it.  The status codes that need device objects are forced by the GPU
tests named in the driver's header.
"""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
OUT = ROOT / "qwen38-metal_amd" / "_build" / "asan"
EXE = OUT / "host_status"

# Codes the reference's error enum has but this path never produces.
NEVER_PRODUCED = {"QM_ERR_ZERO_CAPACITY", "QM_ERR_EMPTY_APPEND"}
# Forced by GPU tests (they need a cache, a state, a graph or a HIP failure).
ON_GPU = {"QM_ERR_INVALID_SEQUENCE_LENGTH", "QM_ERR_CAPACITY_EXCEEDED", "QM_ERR_INVALID_SNAPSHOT",
          "QM_ERR_INVALID_SNAPSHOT_ROW", "QM_ERR_GRAPH_STALE", "QM_ERR_OUT_OF_MEMORY", "QM_ERR_COMMAND_FAILED"}


def _stale() -> bool:
    if not EXE.exists():
        return True
    built = EXE.stat().st_mtime
    srcs = list((ROOT / "qwen38-metal_amd" / "csrc").glob("*")) + [ROOT / "oracle" / "qm_oracle.cpp",
                                                                     ROOT / "include" / "qm38.h"]
    srcs += list((ROOT / "tests" / "native").glob("*"))
    return any(p.stat().st_mtime > built for p in srcs)


def _all_codes():
    text = (ROOT / "include" / "qm38.h").read_text()
    import re
    return set(re.findall(r"\b(QM_(?:OK|ERR_[A-Z_]+))\s*=", text))


@pytest.fixture(scope="module")
def driver():
    if not Path("/opt/rocm/bin/hipcc").exists():
        pytest.skip("hipcc is not installed")
    if _stale():
        subprocess.run(["sh", str(ROOT / "tests" / "native" / "build_host_status.sh"), str(OUT)], check=True,
                       capture_output=True, text=True)
    return EXE


def test_host_status_codes_under_sanitizers(driver):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    res = subprocess.run([str(driver)], capture_output=True, text=True, env=env, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "ERROR: AddressSanitizer" not in res.stderr and "runtime error:" not in res.stderr, res.stderr
    forced = {line.split()[1] for line in res.stdout.splitlines() if line.startswith("forced ")}
    assert "failures 0" in res.stdout
    codes = _all_codes()
    missing = codes - forced - ON_GPU - NEVER_PRODUCED
    assert not missing, f"status codes forced nowhere: {sorted(missing)}"
    assert not (forced & ON_GPU), "update ON_GPU: the host now forces " + str(sorted(forced & ON_GPU))
