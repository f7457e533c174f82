"""The chunked-prefill kernel finds a token's page with a multiply and a shift (mvr::page_divider in
mini-vllm-rs_amd/csrc/paged_prefill.hpp), for any page size that is a multiple of 16.  The function itself is
compiled for the host with g++ and compared with integer division: every token index below 2^20 and the
indices around the multiples of the page size just below 2^31 (the largest a kernel can see), for every page
size 16, 32, ..., 4096.
"""
import os
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "mini-vllm-rs_amd", "csrc")

PROGRAM = r"""
#include "paged_prefill.hpp"
#include <cstdio>
int main() {
  long bad = 0, checks = 0;
  for (int d = 16; d <= 4096; d += 16) {
    uint64_t m; int32_t s;
    mvr::page_divider(d, m, s);
    auto q = [&](uint32_t n) { return (uint32_t)(((uint64_t)n * m) >> s); };
    for (uint32_t n = 0; n < (1u << 20); n++, checks++) bad += q(n) != n / d;
    for (uint32_t k = 1; k < 2048; k++) {
      const uint32_t base = (uint32_t)((((1ull << 31) - 1) / d - k) * d);
      for (uint32_t n = base - 1; n != base + 2; n++, checks++) bad += q(n) != n / d;
    }
    for (uint32_t n = (1u << 31) - 2048; n < (1u << 31); n++, checks++) bad += q(n) != n / d;
  }
  printf("%ld %ld\n", checks, bad);
  return 0;
}
"""


def test_page_divider_equals_integer_division():
    with tempfile.TemporaryDirectory() as tmp:
        src, exe = os.path.join(tmp, "t.cpp"), os.path.join(tmp, "t")
        with open(src, "w") as f:
            f.write(PROGRAM)
        r = subprocess.run(["g++", "-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", f"-I{CSRC}",
                            src, "-o", exe], capture_output=True, text=True)
        if r.returncode != 0:
            pytest.fail(r.stderr[-2000:])
        checks, bad = map(int, subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split())
    assert checks > 256 * (1 << 20) and bad == 0, (checks, bad)
