"""The host-side tests again, against AddressSanitizer + UndefinedBehaviorSanitizer
builds (CPU only; nothing launches, no GPU needed).

- libloom_hip_asan.so (`make -C loom-dataflow_amd/csrc asan`): the host code
  of every source -- argument validation, the block-size JSON reader, the
  variant-name parser, the memref unpacking, the constraint scopes -- built
  with -fsanitize=address,undefined (device code uninstrumented), loaded via
  LOOM_HIP_LIB with clang's ASan runtime preloaded.  The ABI, materialization,
  constraint, memref, Python-validation and fuzz tests run against it.
- liboracle_asan.so (`make -C oracle liboracle_asan.so`, gcc): the CPU oracle,
  loaded via LOOM_ORACLE_LIB with gcc's runtime preloaded; the oracle tests
  run against it.
A sanitizer report aborts the child run (halt_on_error, no recovery), so the
child's exit status and output decide.  (Checked: putting back the old order
of JParser::num's range test -- a double-to-long-long conversion of 1e300 --
makes the first run stop at the corpus file that carries it.)
"""
import glob
import os
import subprocess
import sys

import pytest

from tests.conftest import ROOT

HOST_TESTS = ["tests/test_abi.py", "tests/test_materialize.py", "tests/test_constraints.py",
              "tests/test_memref.py", "tests/test_python_validation.py", "tests/test_fuzz_abi.py"]
REPORTS = ("ERROR: AddressSanitizer", "runtime error:", "ERROR: LeakSanitizer")


def _run(env_extra, tests):
    env = dict(os.environ)
    env.update(env_extra)
    env["ASAN_OPTIONS"] = "detect_leaks=0:halt_on_error=1:abort_on_error=0"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    env["PYTHONDONTWRITEBYTECODE"] = "1"
    # --capture=sys: a sanitizer writes its report to file descriptor 2 and
    # exits at once, so fd-level capture would swallow it
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                        "--capture=sys", "-m", "not gpu", *tests], cwd=ROOT, env=env, capture_output=True,
                       text=True, timeout=1200)
    out = r.stdout + r.stderr
    assert not any(rep in out for rep in REPORTS), out[-6000:]
    assert r.returncode == 0, out[-6000:]
    return out


def test_host_code_under_asan_ubsan():
    subprocess.run(["make", "-s", "-j8", "-C", os.path.join(ROOT, "loom-dataflow_amd", "csrc"),
                    "asan"], check=True, capture_output=True)
    lib = os.path.join(ROOT, "loom-dataflow_amd", "_build_asan", "libloom_hip_asan.so")
    rt = sorted(glob.glob("/opt/rocm/lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not rt:
        pytest.skip("clang's ASan runtime is not installed")
    out = _run({"LD_PRELOAD": rt[-1], "LOOM_HIP_LIB": lib}, HOST_TESTS)
    assert " passed" in out


def test_oracle_under_asan_ubsan():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "liboracle_asan.so"],
                   check=True, capture_output=True)
    rt = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True,
                        text=True).stdout.strip()
    if not os.path.isabs(rt):
        pytest.skip("gcc's ASan runtime is not installed")
    lib = os.path.join(ROOT, "oracle", "liboracle_asan.so")
    out = _run({"LD_PRELOAD": rt, "LOOM_ORACLE_LIB": lib}, ["tests/test_oracle.py"])
    assert " passed" in out
