"""The launchers' dispatch-size arithmetic (fuselse_amd/csrc/fl_grid.hpp),
compiled alone with the host C++ compiler and run on the CPU: one launch
never carries more than 2^32 - 1 work-items, the caps are multiples of 8, and
the chunks of a launch split cover every block once, in order."""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER_DIR = os.path.join(ROOT, "fuselse_amd", "csrc")

PROGRAM = r"""
#include <stdio.h>
#include "fl_grid.hpp"
using namespace fl;
int main() {
    const int64_t threads[] = {64, 128, 256, 512, 1024};
    // totals around each cap and the shapes the launchers meet: (2^24 + 3)
    // one-block rows of 256 threads, 2^26 + 32 one-wave blocks of the flat
    // backward at 2^34 + 8192 fp32 elements
    for (int64_t t : threads) {
        const int64_t cap = max_grid_blocks(t);
        if (cap % 8 != 0 || cap * t > 0xFFFFFFFFll || (cap + 8) * t <= 0xFFFFFFFFll) {
            printf("bad cap %lld for %lld threads\n", (long long)cap, (long long)t);
            return 1;
        }
        const int64_t totals[] = {0, 1, 7, cap - 1, cap, cap + 1, 2 * cap, 2 * cap + 5, (1ll << 24) + 3,
                                  (1ll << 26) + 32, 3 * cap + 1};
        for (int64_t total : totals) {
            int64_t next = 0, calls = 0;
            bool ok = true;
            for_grid_chunks(total, t, [&](int64_t first, int64_t n) {
                ok = ok && first == next && n > 0 && n <= cap && n * t <= 0xFFFFFFFFll;
                next = first + n;
                ++calls;
            });
            const int64_t want_calls = (total + cap - 1) / cap;
            if (!ok || next != total || calls != want_calls) {
                printf("bad split of %lld blocks of %lld threads\n", (long long)total, (long long)t);
                return 1;
            }
            const int64_t g = grid_stride_blocks(total, t);
            if (g > cap || (total <= cap && g != total)) {
                printf("bad grid-stride size for %lld\n", (long long)total);
                return 1;
            }
        }
    }
    printf("ok %lld %lld\n", (long long)max_grid_blocks(64), (long long)max_grid_blocks(256));
    return 0;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="no host C++ compiler")
def test_grid_chunk_arithmetic(tmp_path):
    src = tmp_path / "grid_test.cpp"
    exe = tmp_path / "grid_test"
    src.write_text(PROGRAM)
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-I", HEADER_DIR, str(src), "-o", str(exe)], capture_output=True,
                       text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    # 2^32 - 1 work-items: 67108856 one-wave blocks, 16777208 blocks of 256
    assert r.stdout.split() == ["ok", str(((2**32 - 1) // 64) & ~7), str(((2**32 - 1) // 256) & ~7)]
