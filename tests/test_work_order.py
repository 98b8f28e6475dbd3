"""The work order (common.h WorkOrder) maps the launch's blocks onto every
(row block, q head) item exactly once, for every kv-group layout and both
row-cost modes (host build of the same header, no GPU)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "vecattention_amd", "csrc")

PROG = r"""
#include "common.h"
#include <cstdio>
#include <vector>
int main() {
  const long long cfg[][4] = {{7, 1, 28, 4}, {512, 1, 28, 4}, {33, 1, 12, 12}, {5, 1, 24, 24},
                              {9, 2, 8, 2}, {3, 1, 4, 4}, {17, 1, 6, 6}, {4, 3, 20, 5},
                              {1, 1, 16, 16}, {13, 1, 32, 8}, {2, 1, 1, 1}};
  for (auto& c : cfg)
    for (int eq = 0; eq < 2; ++eq) {
      const va::WorkOrder wo{c[0], c[1], c[2], c[3], eq != 0};
      const long long n = c[0] * c[1] * c[2], grid = wo.grid_items();
      std::vector<int> seen(n, 0);
      long long mapped = 0;
      for (long long i = 0; i < grid; ++i) {
        int64_t jr, bh;
        if (!wo.map_item(i, jr, bh)) continue;
        if (jr < 0 || jr >= c[0] || bh < 0 || bh >= c[1] * c[2]) { printf("BAD range\n"); return 1; }
        // items of one kv head stay on one XCD set: (b, hk) of bh
        ++seen[jr * c[1] * c[2] + bh];
        ++mapped;
      }
      for (long long t = 0; t < n; ++t)
        if (seen[t] != 1) { printf("BAD cover %lld %lld %lld %lld eq=%d\n", c[0], c[1], c[2], c[3], eq); return 1; }
      if (grid - mapped >= 8 * (c[1] * c[3] < 8 ? 8 / (c[1] * c[3]) : 1)) { printf("BAD idle\n"); return 1; }
    }
  printf("OK\n");
  return 0;
}
"""


def test_work_order_is_a_bijection(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    src = tmp_path / "wo.hip"
    src.write_text(PROG)
    exe = tmp_path / "wo"
    r = subprocess.run([hipcc, "-std=c++17", "--offload-arch=gfx950", f"-I{CSRC}", str(src), "-o",
                        str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.stdout.strip() == "OK", out.stdout + out.stderr
