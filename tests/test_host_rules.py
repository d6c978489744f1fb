"""Host-side addressing rules of the state step, compiled from the library's own header with g++ (no GPU).

The gathers address the previous state with one 24-bit multiply-add (row index times row bytes) into a 32-bit
buffer offset.  `fly::buffer_bytes` must therefore refuse any state whose size passes 2^31 - 1 bytes, whose row
is 2^24 bytes or more, or which holds 2^24 rows or more (the index of the row just past the buffer, which the
swept step gathers zeros from, must fit 24 bits too); the caller then takes the 64-bit path.  `state_ld`
gives every state row an odd number of 128-byte lines.
"""

import pathlib
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
CSRC = ROOT / "alpha-fly_amd" / "csrc"
HIP_INCLUDE = pathlib.Path("/opt/rocm/include")

PROGRAM = r"""
#include "common.hpp"
#include <cstdio>
int main() {
  const long long cases[][3] = {
      {166700, 1216, 2}, {166700, 1, 2}, {(1 << 24) - 1, 1, 2}, {1 << 24, 1, 2}, {(1 << 24) + 1, 64, 2},
      {1, (1 << 23) - 1, 2}, {1, 1 << 23, 2}, {4, 1 << 21, 4}, {300, 1 << 21, 4}, {16384, 32768, 4}, {16383, 32768, 4},
      {0, 64, 2}, {10, 0, 2}};
  for (const auto &c : cases) printf("b %lld %lld %lld %u\n", c[0], c[1], c[2], fly::buffer_bytes(c[0], c[1], c[2]));
  for (long long batch = 1; batch <= 4160; batch += 7)
    for (int elem = 2; elem <= 4; elem += 2) printf("s %lld %d %lld\n", batch, elem, (long long)fly::state_ld(batch, elem));
  return 0;
}
"""


@pytest.fixture(scope="module")
def rules(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None or not (HIP_INCLUDE / "hip" / "hip_runtime.h").exists():
        pytest.skip("g++ or the HIP headers are not installed")
    d = tmp_path_factory.mktemp("rules")
    (d / "rules.cpp").write_text(PROGRAM)
    exe = d / "rules"
    subprocess.run([gxx, "-std=c++17", "-D__HIP_PLATFORM_AMD__", f"-I{HIP_INCLUDE}", f"-I{CSRC}",
                    f"-I{ROOT / 'include'}", str(d / "rules.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    bb = {tuple(int(v) for v in line.split()[1:4]): int(line.split()[4]) for line in out if line.startswith("b ")}
    ld = {(int(line.split()[1]), int(line.split()[2])): int(line.split()[3]) for line in out if line.startswith("s ")}
    return bb, ld


def test_buffer_bytes_accepts_what_24_bit_offsets_can_address(rules):
    bb, _ = rules
    assert bb[(166700, 1216, 2)] == 166700 * 1216 * 2          # the full-scale half state at 1120 boards
    assert bb[(166700, 1, 2)] == 166700 * 2
    assert bb[((1 << 24) - 1, 1, 2)] == ((1 << 24) - 1) * 2    # every row index and the one past the end fit 24 bits
    assert bb[(1, (1 << 23) - 1, 2)] == (1 << 24) - 2          # the largest row below 2^24 bytes
    assert bb[(4, 1 << 21, 4)] == 1 << 25
    assert bb[(16383, 32768, 4)] == 16383 * 32768 * 4           # just below 2 GiB


def test_buffer_bytes_refuses_what_they_cannot(rules):
    bb, _ = rules
    assert bb[(1 << 24, 1, 2)] == 0            # the row past the end, 2^24, would wrap in the multiply
    assert bb[((1 << 24) + 1, 64, 2)] == 0
    assert bb[(1, 1 << 23, 2)] == 0            # a 2^24-byte row
    assert bb[(300, 1 << 21, 4)] == 0          # rows below 2^24 bytes, but 2.5 GB in all
    assert bb[(16384, 32768, 4)] == 0          # exactly 2 GiB
    assert bb[(0, 64, 2)] == 0 and bb[(10, 0, 2)] == 0


def test_state_rows_hold_an_odd_number_of_lines(rules):
    _, ld = rules
    for (batch, elem), stride in ld.items():
        line = 128 // elem
        assert stride >= batch and stride % line == 0
        assert (stride // line) % 2 == 1
        assert stride - batch < 64 + line
