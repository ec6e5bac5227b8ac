"""Row indexing of the block-parallel mul_mat_id GEMV (k_mmid_gemv_bp), on
the CPU: the kernel's own helpers (questwend_amd/csrc/qw_bp_rows.hpp),
compiled with g++, walked over every workgroup, wave and lane of the launch
for N = 1..300 rows and 4, 8 or 16 lanes per row.  No load may touch a row
outside [0, N) (the parity tests cannot see such a read: their weight buffers
have slack past the last matrix), and every row must be loaded by the lanes
that own it.
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]

DRIVER = r"""
#include <cstdio>
#include "qw_bp_rows.hpp"
using namespace qw;
int main() {
    long bad = 0, missing = 0, cases = 0;
    const int bprs[3] = {4, 8, 16};
    for (int bi = 0; bi < 3; ++bi) {
        const int bpr = bprs[bi], rpw = bp_rows_per_wave(bpr);
        for (long N = 1; N <= 300; ++N) {
            ++cases;
            const long grid = (N + 4 * rpw - 1) / (4 * rpw);   // launch_gemv_bp's grid.x
            std::vector<char> own(N, 0);
            for (long g = 0; g < grid; ++g) {
                const long r0 = bp_wg_row0(g, bpr);
                for (int w = 0; w < 4; ++w) {
                    const long wr0 = bp_wave_row0(g, w, bpr);
                    const int wrows = bp_wave_rows(N, wr0, bpr);
                    for (int lane = 0; lane < 64; ++lane) {
                        const int rl = lane / bpr;
                        const long d = bp_direct_row(r0, wr0, wrows, rl);
                        if (d < 0 || d >= N) ++bad;
                        else if (rl < wrows && d == wr0 + rl) own[d] = 1;
                    }
                    // staged chunks: idx < wrows * nchmax, row = idx / nchmax
                    const int nchmax = 5;
                    for (int idx = 0; idx < wrows * nchmax; ++idx) {
                        const long s = bp_staged_row(wr0, wrows, idx / nchmax);
                        if (s < 0 || s >= N) ++bad;
                    }
                }
            }
            for (long r = 0; r < N; ++r) missing += !own[r];
        }
    }
    std::printf("%ld %ld %ld\n", cases, bad, missing);
    return 0;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_bp_rows_stay_inside_the_matrix(tmp_path):
    src = tmp_path / "bp_rows.cpp"
    src.write_text("#include <vector>\n" + DRIVER)
    exe = tmp_path / "bp_rows"
    subprocess.run(["g++", "-O1", "-std=c++17", "-I", str(ROOT / "questwend_amd" / "csrc"), str(src), "-o", str(exe)],
                   check=True)
    cases, bad, missing = (int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True,
                                                          text=True).stdout.split())
    assert cases == 900
    assert bad == 0, f"{bad} loads outside [0, N)"
    assert missing == 0, f"{missing} rows no lane loads as its own"
