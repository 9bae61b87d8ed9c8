"""Host code under AddressSanitizer + UndefinedBehaviorSanitizer (CPU only).

Two builds, each made by its own Makefile target and loaded in a child
process that preloads the matching sanitizer runtime (one runtime per
process):
  * `make -C oracle san` -> oracle/_build/liboracle_san.so (gcc), driven by
    the oracle's CPU tests: formats, golden vectors, ops, the Qwen3 forward,
    greedy and speculative generation, the KV cache;
  * `make -C base-mlx_amd san` -> base-mlx_amd/lib/libbmx_san.so (the
    library with its host entry code -- the checkpoint loader and the C
    ABI's argument checks -- instrumented), driven by the loader and ABI CPU
    tests.
Both builds stop at the first report (-fno-sanitize-recover=all), so a
clean exit of the child is the result; the child also proves the
instrumented library is the one it loaded.
"""
import glob
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TESTS = os.path.join(ROOT, "tests")


def _make(path, target):
    jobs = str(min(8, os.cpu_count() or 4))
    r = subprocess.run(["make", "-C", path, "-s", "-j", jobs, target], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]


def _run_child(which, runtime, args):
    env = dict(os.environ)
    env["BMX_TEST_SANITIZED"] = which
    env["LD_PRELOAD"] = runtime
    # leaks of the interpreter and its extension modules are not this code's
    env["ASAN_OPTIONS"] = "detect_leaks=0:halt_on_error=1"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", "-m", "not gpu", *args],
                       cwd=TESTS, env=env, capture_output=True, text=True, timeout=1500)
    out = r.stdout + r.stderr
    assert "Sanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert r.returncode == 0, out[-4000:]
    return out


def test_sanitized_build_is_loaded():
    """Inside a child: the instrumented build is the one the process loaded
    (first in each child's run; skipped in the parent)."""
    which = os.environ.get("BMX_TEST_SANITIZED", "")
    if not which:
        pytest.skip("runs inside the sanitizer child processes")
    if which == "oracle":
        import oracle

        oracle.lib()
        name = "liboracle_san.so"
    else:
        import bmx

        bmx.load()
        name = "libbmx_san.so"
    assert name in open("/proc/self/maps").read()


SELF = "test_sanitizers.py::test_sanitized_build_is_loaded"


def test_oracle_under_asan_ubsan():
    _make(os.path.join(ROOT, "oracle"), "san")
    rt = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    assert os.path.isabs(rt) and os.path.exists(rt), rt
    # (the transformers comparisons are left out: torch's HIP module throws
    # C++ exceptions on a GPU-less host, which the ASan runtime's __cxa_throw
    # interceptor does not survive -- outside this code)
    _run_child("oracle", rt, [SELF, "test_oracle_format.py", "test_golden.py", "test_oracle_ops.py",
                              "test_oracle_model.py",
                              "-k", "not transformers"])


def test_library_host_code_under_asan_ubsan():
    _make(os.path.join(ROOT, "base-mlx_amd"), "san")
    rts = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not rts:
        pytest.fail("the ROCm clang ASan runtime is missing")
    _run_child("lib", rts[-1], [SELF, "test_loader.py", "test_abi.py"])
