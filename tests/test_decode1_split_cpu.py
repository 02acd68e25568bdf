"""The one-token decode kernel's work split (gemmainfer_amd/csrc/decode1_split.h),
compiled with g++ on the CPU: whenever the host-side check accepts a shape,
every run-time number of unique experts U in [1, umax] gives a split where
every folded output unit has an item to sum it, every item and unit has a
workgroup, and the units are covered exactly once.  Also the case that broke
the old check: more output units than workgroups (a 32-CU device, H = 1056,
top_k = 1)."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "gemmainfer_amd" / "csrc" / "decode1_split.h"

CHECK = r"""
#include <cstdio>
#include "decode1_split.h"
using namespace gi::d1;
int main() {
  const int Gs[] = {8, 32, 64, 80, 104, 120, 228, 256, 304};
  long accepted = 0;
  for (int G : Gs)
    for (int units = 1; units <= 400; ++units)
      for (int Tk = 1; Tk <= 24; ++Tk)
        for (int umax = 1; umax <= 8; ++umax) {
          if (!split_ok(G, umax, Tk, units, 8)) continue;
          ++accepted;
          for (int U = 1; U <= umax; ++U) {
            const Split s = split(G, U, Tk, units);
            if (s.n_whole < 0 || s.n_left < 0 || s.n_items + s.n_whole > G || s.n_whole + s.n_left != units ||
                s.n_left > s.n_items || s.n_left > 8) {
              std::printf("BAD G=%d units=%d Tk=%d umax=%d U=%d items=%d whole=%d left=%d\n", G, units, Tk,
                          umax, U, s.n_items, s.n_whole, s.n_left);
              return 1;
            }
          }
        }
  // more output units than workgroups: folded unit 32 would have no item
  if (split_ok(32, 1, 2, 33, 8)) { std::printf("BAD: G=32 units=33 accepted\n"); return 1; }
  // the Gemma shape on 256 CUs: 8 experts x 22 tiles, 88 units -> 80 whole, 8 folded
  const Split g = split(256, 8, 22, 88);
  if (!split_ok(256, 8, 22, 88, 8) || g.n_items != 176 || g.n_whole != 80 || g.n_left != 8) {
    std::printf("BAD: Gemma split %d %d %d\n", g.n_items, g.n_whole, g.n_left);
    return 1;
  }
  std::printf("ok %ld\n", accepted);
  return 0;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_decode1_split_covers_every_folded_unit(tmp_path):
    src = tmp_path / "split_check.cpp"
    src.write_text(CHECK)
    exe = tmp_path / "split_check"
    subprocess.run(["g++", "-std=c++17", "-O1", f"-I{HEADER.parent}", str(src), "-o", str(exe)], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.startswith("ok ") and int(res.stdout.split()[1]) > 1000, res.stdout
