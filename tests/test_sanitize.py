"""Host sanitizer run (CPU, no GPU): the C-ABI host layer (libtmac_attn_san.so) and the
oracle (libtmac_oracle_san.so) built with AddressSanitizer + UndefinedBehaviorSanitizer,
and the CPU test suite run against them in a child process with the sanitizer
runtimes preloaded.  That covers the ABI's argument rejection paths, the model-file
loader on truncated and foreign files, the synthetic streams and the oracle.  Any
sanitizer report aborts the child (halt_on_error), failing this test."""
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
SAN_ATTN = os.path.join(REPO, "tmac_gguf.cpp_amd", "lib", "libtmac_attn_san.so")
SAN_ORACLE = os.path.join(REPO, "oracle", "lib", "libtmac_oracle_san.so")


def _runtime(name: str) -> str:
    return subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True,
                          check=True).stdout.strip()


def _env():
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": f"{_runtime('libasan.so')} {_runtime('libubsan.so')}",
        "ASAN_OPTIONS": "detect_leaks=0:verify_asan_link_order=0:abort_on_error=1",
        "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1",
        "TMAC_ATTN_LIB": SAN_ATTN,
        "TMAC_ORACLE_LIB": SAN_ORACLE,
    })
    return env


@pytest.fixture(scope="module")
def sanitizer_builds():
    if not os.path.exists(_runtime("libasan.so")):
        pytest.skip("no libasan in this toolchain")
    for d in (os.path.join(REPO, "tmac_gguf.cpp_amd"), os.path.join(REPO, "oracle")):
        subprocess.run(["make", "-s", "-C", d, "sanitize"], check=True)
    return True


def test_sanitized_libraries_are_the_ones_loaded(sanitizer_builds):
    code = ("import ctypes, sys; sys.path[:0] = [%r, %r]; import tmac_attn, oracle; "
            "lib = tmac_attn.load_library(); print(lib._name); print(oracle.lib()._name); "
            "print(hasattr(ctypes.CDLL(None), '__asan_init'))"
            % (os.path.join(REPO, "tmac_gguf.cpp_amd"), REPO))
    out = subprocess.run([sys.executable, "-c", code], env=_env(), capture_output=True, text=True, check=True)
    lines = out.stdout.split()
    assert lines == [SAN_ATTN, SAN_ORACLE, "True"], out.stdout + out.stderr


def test_cpu_suite_under_asan_ubsan(sanitizer_builds):
    cmd = [sys.executable, "-m", "pytest", HERE, "-q", "-x", "-m", "not gpu", "-p", "no:cacheprovider",
           "--ignore", os.path.abspath(__file__)]
    res = subprocess.run(cmd, env=_env(), capture_output=True, text=True, cwd=REPO, timeout=600)
    tail = (res.stdout + res.stderr)[-4000:]
    assert res.returncode == 0, tail
    assert "passed" in res.stdout and "ERROR: AddressSanitizer" not in tail and "runtime error" not in tail, tail
