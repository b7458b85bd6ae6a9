"""The host code under AddressSanitizer and UndefinedBehaviorSanitizer.

`make -C oracle sanitize` builds libfmx.so (its host code: the C ABI's
validation, workspace and geometry arithmetic, fault state, packing sizes) and
the oracle's C restatement with ASan + UBSan (clang's runtime; UBSan findings
abort). This test runs the host-only tests of both against those builds in a
child process that preloads the sanitizer runtime: the C-ABI host tests, the
oracle's quantisation, math and reference-comparison tests, the GGUF
writer/reader and the workload builders. Any report fails
the child and so this test. No GPU is used."""
import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
ORACLE = ROOT / "oracle"
SAN_FMX = ORACLE / "_san" / "libfmx.so"
SAN_ORACLE = ORACLE / "_san" / "libfmoracle.so"
HOST_TESTS = ["tests/test_capi_host.py", "tests/test_oracle_quant.py", "tests/test_oracle_math.py",
              "tests/test_oracle_reference.py", "tests/test_gguf.py", "tests/test_workloads.py"]


def asan_runtime():
    clang = Path("/opt/rocm/llvm/bin/clang")
    if not clang.exists():
        return None
    out = subprocess.run([str(clang), "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True,
                         text=True)
    path = Path(out.stdout.strip())
    return path if path.is_absolute() and path.exists() else None


def test_host_code_under_asan_and_ubsan():
    rt = asan_runtime()
    if rt is None or shutil.which("make") is None or not Path("/opt/rocm/bin/hipcc").exists():
        pytest.skip("clang's sanitizer runtime or hipcc is not in this image")
    build = subprocess.run(["make", "-C", str(ORACLE), "-j8", "sanitize"], capture_output=True, text=True,
                           timeout=1200)
    assert build.returncode == 0, build.stderr[-4000:]
    assert SAN_FMX.exists() and SAN_ORACLE.exists()
    env = dict(os.environ, LD_PRELOAD=str(rt), FMX_LIBRARY=str(SAN_FMX), FMORACLE_LIBRARY=str(SAN_ORACLE),
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    run = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider", "-m", "not gpu",
                          *HOST_TESTS], cwd=ROOT, env=env, capture_output=True, text=True, timeout=1200)
    report = run.stdout[-3000:] + run.stderr[-3000:]
    assert run.returncode == 0, report
    assert "ERROR: AddressSanitizer" not in report and "runtime error:" not in report, report
    assert " passed" in run.stdout, report
