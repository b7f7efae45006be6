"""The stored-dS block layout (csrc/worklist.h): every attended (64-key group, 32-row
query tile) pair of a segment gets its own block in [0, ds_seg_blocks), with none
left over. Checked by a host program built from the header with hipcc, on edge
lengths and prefixes and on random ones; the attended predicate in it is the brute
force of the mask (the group's first key is seen by the tile's last query), not the
layout's formulas."""
import os
import shutil
import subprocess
import tempfile

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "hrm-text_amd", "csrc")

PROGRAM = r"""
#include <stdio.h>
#include <stdlib.h>
#include "worklist.h"
using namespace prefixlm;
int main() {
  int L, p;
  while (scanf("%d %d", &L, &p) == 2) {
    const int n32 = (L + 31) / 32, n64 = (L + 63) / 64, kp = ds_kp(p, L);
    const long long nb = ds_seg_blocks(p, L);
    char* seen = (char*)calloc(nb + 1, 1);
    long long cnt = 0;
    int bad = 0;
    for (int kg = 0; kg < n64; ++kg)
      for (int qt = 0; qt < n32; ++qt) {
        const int q1 = 32 * qt + 32 < L ? 32 * qt + 32 : L;
        if (!(64 * kg < p || 64 * kg <= q1 - 1)) continue;
        const long long b = (long long)ds_blk_off(kg, n32, kp) + qt;
        if (b < 0 || b >= nb || seen[b]) bad = 1; else seen[b] = 1;
        ++cnt;
      }
    printf("%lld %lld %d\n", nb, cnt, bad);
    free(seen);
  }
  return 0;
}
"""


def _hipcc():
    for c in ("/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    pytest.skip("hipcc not found")


def test_layout_is_a_bijection_onto_the_attended_blocks():
    cases = [(1, 0), (1, 1), (31, 0), (32, 32), (33, 0), (63, 63), (64, 0), (64, 64), (65, 1), (65, 64),
             (100, 0), (100, 100), (128, 127), (129, 128), (4096, 0), (4096, 4096), (4096, 1000), (8192, 7680)]
    rng = np.random.default_rng(11)
    for _ in range(300):
        L = int(rng.integers(1, 3000))
        cases.append((L, int(rng.integers(0, L + 1))))
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "layout.hip"), os.path.join(d, "layout")
        open(src, "w").write(PROGRAM)
        r = subprocess.run([_hipcc(), "--offload-arch=gfx950", "-O1", "-std=c++17", f"-I{CSRC}", src, "-o", exe],
                           capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        out = subprocess.run([exe], input="\n".join(f"{L} {p}" for L, p in cases), capture_output=True,
                             text=True, check=True).stdout.split("\n")
    for (L, p), line in zip(cases, out):
        nb, cnt, bad = map(int, line.split())
        assert bad == 0 and nb == cnt, (L, p, nb, cnt)
