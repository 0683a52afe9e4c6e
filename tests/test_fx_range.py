"""The range checks in front of the fixed-point accumulators (qwen-3.5_amd/csrc/fx_range.h),
compiled for the host: the boundary values on both sides, the non-finite values, and the fact
that makes the plain bound sufficient (the largest accepted value times 2^32 fits a signed 64-bit
integer), worked out here in exact integer arithmetic."""
import os
import struct
import subprocess

import numpy as np

CSRC = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "qwen-3.5_amd", "csrc")

PROG = r"""
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include "fx_range.h"
int main(int argc, char** argv) {
  for (int i = 1; i < argc; ++i) {
    unsigned u = (unsigned)strtoul(argv[i], nullptr, 16);
    float v;
    __builtin_memcpy(&v, &u, 4);
    std::printf("%d %d\n", q35::fx_addable(v) ? 1 : 0, q35::fxc_addable(v) ? 1 : 0);
  }
  return 0;
}
"""


def bits(v):
    return "%08x" % struct.unpack("<I", struct.pack("<f", v))[0]


def below(x):
    return float(np.nextafter(np.float32(x), np.float32(0)))


def test_fixed_point_range_bounds(tmp_path):
    src, exe = tmp_path / "fx.cpp", tmp_path / "fx"
    src.write_text(PROG)
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", CSRC, str(src), "-o", str(exe)], check=True)
    two31, two22 = 2.0 ** 31, 2.0 ** 22
    cases = [0.0, 1.0, -1.0, below(two22), -below(two22), two22, -two22, below(two31), -below(two31), two31, -two31,
             1e12, -1e12, float("inf"), float("-inf"), float("nan")]
    out = subprocess.run([str(exe)] + [bits(v) for v in cases], check=True, capture_output=True, text=True).stdout
    got = [tuple(int(t) for t in line.split()) for line in out.strip().splitlines()]
    exp = []
    for v in cases:
        fin = np.isfinite(v)
        exp.append((int(fin and abs(v) < two31), int(fin and abs(v) < two22)))
    assert got == exp
    # the largest accepted value converts without overflow: (2^31 - 128) * 2^32 < 2^63 - 1
    vmax = int(below(two31))
    assert vmax == 2 ** 31 - 128 and vmax * 2 ** 32 < 2 ** 63 - 1
    # and 2^31 itself would not: 2^31 * 2^32 = 2^63 is past the int64 range
    assert 2 ** 31 * 2 ** 32 > 2 ** 63 - 1
