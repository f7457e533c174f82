"""AddressSanitizer + UndefinedBehaviorSanitizer builds, run on the CPU.

tests/sanitize/Makefile builds two drivers: one runs every oracle entry point (gcc, -fsanitize=address,undefined)
over exactly sized heap buffers, including the reference's error cases; the other links the library's host half
(mvr_attn_api.cpp compiled by hipcc with the sanitizers on the host side only) and runs its argument checks, planning
over many shapes with and without the host hints, the host-side table validators and every entry point's error
paths.  Neither launches a kernel.  A sanitizer report makes the driver exit non-zero
(-fno-sanitize-recover=all) and fails the test.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = os.path.join(ROOT, "tests", "sanitize")
LIB_BUILD = os.path.join(ROOT, "mini-vllm-rs_amd", "_build")
KERNEL_OBJS = ["paged_attention.o", "paged_prefill.o", "kv_gather.o", "kv_append.o"]


def _make(target):
    if not os.path.isdir(SAN):
        pytest.skip("tests/sanitize is not present")
    r = subprocess.run(["make", "-C", SAN, "-j4", target], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    return os.path.join(SAN, target)


def _run(exe, leaks):
    env = dict(os.environ)
    env["ASAN_OPTIONS"] = f"detect_leaks={1 if leaks else 0}:abort_on_error=0"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=600, env=env)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
    assert "all checks passed" in out, out[-2000:]


@pytest.mark.skipif(shutil.which("gcc") is None, reason="no gcc")
def test_oracle_under_sanitizers():
    _run(_make("_build/oracle_san"), leaks=True)


@pytest.mark.skipif(not os.path.exists("/opt/rocm/bin/hipcc"), reason="no hipcc")
def test_library_host_half_under_sanitizers():
    if not all(os.path.exists(os.path.join(LIB_BUILD, o)) for o in KERNEL_OBJS):
        pytest.skip("build the library first (python -c 'import __graft_entry__ as g; g.build()')")
    # The HIP runtime keeps allocations until exit by design, so leak checking is off for this driver.
    _run(_make("_build/api_san"), leaks=False)
