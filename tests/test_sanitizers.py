"""The oracle's C restatement and the library's host code under
AddressSanitizer + UndefinedBehaviorSanitizer (CPU only, no GPU touched):
the oracle's own test file runs against oracle/_san/liboracle.so (gcc's
sanitizers, `make -C oracle sanitize`) and the weight-manifest reader's tests
against _san/libqwen_kernels.so (the host side of every unit built with
clang's sanitizers, build_lib.py --sanitize).  Each run is a child process with
the sanitizer runtime preloaded; any report fails it (UBSan does not
recover)."""
import glob
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "qwen35-ax7020-edge-llm_amd"
SAN_ENV = {"ASAN_OPTIONS": "detect_leaks=0:abort_on_error=0:halt_on_error=1",
           "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"}


def _run_pytest(preload, extra_env, *args):
    env = dict(os.environ, LD_PRELOAD=preload, PYTHONPATH=os.pathsep.join([str(PKG), str(ROOT / "tests")]),
               **SAN_ENV, **extra_env)
    # --noconftest: the suite's conftest imports torch, which is not under test here
    cmd = [sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "--noconftest", *args]
    res = subprocess.run(cmd, cwd=str(ROOT), env=env, capture_output=True, text=True, timeout=900)
    out = res.stdout + res.stderr
    assert res.returncode == 0, out[-4000:]
    assert "runtime error:" not in out and "ERROR: AddressSanitizer" not in out, out[-4000:]
    return out


def test_oracle_under_asan_ubsan():
    libasan = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    if not os.path.isabs(libasan):
        pytest.skip("gcc's libasan is not installed")
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "sanitize"], check=True, capture_output=True)
    out = _run_pytest(libasan, {"ORACLE_LIB_UNDER_TEST": str(ROOT / "oracle" / "_san" / "liboracle.so")},
                      str(ROOT / "tests" / "test_oracle.py"), "-k", "not forward_plans_have_the_reference_layout")
    assert " passed" in out


def test_host_code_under_asan_ubsan():
    rt = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not rt:
        pytest.skip("clang's ASan runtime is not installed")
    sys.path.insert(0, str(PKG))
    import build_lib

    lib = build_lib.build_sanitized()
    out = _run_pytest(rt[-1], {"QWEN_KERNELS_LIB_UNDER_TEST": str(lib)},
                      str(ROOT / "tests" / "test_weights_manifest.py"))
    assert " passed" in out
