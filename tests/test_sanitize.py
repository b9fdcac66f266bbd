"""The C ABI and the N-API addon under host AddressSanitizer and
UndefinedBehaviorSanitizer (tests/sanitize/Makefile): every entry point's
argument checks and host helpers, the Node host layer's checks, and, on a
GPU box, one small call of each device entry point.  Any sanitizer report
aborts the run."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sanitize")
BUILD = os.path.join(HERE, "_build")


def _have_toolchain() -> bool:
    return os.path.exists("/opt/rocm/bin/hipcc") and os.path.exists("/opt/rocm/llvm/bin/clang++")


def _make(*targets, timeout=900):
    return subprocess.run(["make", "-s", "-C", HERE, *targets], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                          text=True, timeout=timeout)


@pytest.fixture(scope="module")
def built():
    if not _have_toolchain():
        pytest.skip("hipcc / clang++ are not installed")
    p = _make("all")
    assert p.returncode == 0, p.stdout[-3000:]


def test_c_abi_host_paths_under_asan_ubsan(built):
    p = _make("run", timeout=300)
    print(p.stdout)
    assert p.returncode == 0, p.stdout[-3000:]
    assert "[host_check] ok (0 failed expectations)" in p.stdout


def test_node_host_layer_under_asan_ubsan(built):
    if shutil.which("node") is None or not os.path.exists("/usr/include/node/node_api.h"):
        pytest.skip("node is not installed")
    p = _make("run-node", timeout=300)
    print(p.stdout)
    assert p.returncode == 0, p.stdout[-3000:]
    assert p.stdout.rstrip().endswith("all ok")


@pytest.mark.gpu
def test_c_abi_device_paths_under_asan_ubsan():
    """The driver built on the CPU side runs its device part here: one call
    of every device entry point with the library's host code instrumented."""
    exe = os.path.join(BUILD, "host_check")
    if not os.path.exists(exe):
        pytest.skip("the sanitizer build is absent (make -C tests/sanitize)")
    print("[gpu] sanitized host_check", flush=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
    p = subprocess.run([exe], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=240, env=env)
    print(p.stdout)
    assert p.returncode == 0, p.stdout[-3000:]
    assert "[host_check] device paths done" in p.stdout
    assert "[host_check] ok (0 failed expectations)" in p.stdout
