"""The grid-index -> (item, head) map of the attention kernels (csrc/common.h
unit_of / unit_grid), compiled for the host with hipcc: every (item, head) is covered
exactly once, each XCD (grid index mod 8) takes units in item (cost) order, the XCDs get
equal shares, an XCD touches few heads, and for H % 8 == 0 the map is the plain
b = item * H + head order."""
import os
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "hrm-text_amd", "csrc")

PROGRAM = r'''
#include "common.h"
#include <cstdio>
int main() {
  int H, n;
  while (scanf("%d %d", &H, &n) == 2) {
    const long g = prefixlm::unit_grid(n, H);
    printf("G %d %d %ld\n", H, n, g);
    for (long b = 0; b < g; ++b) {
      int i = -1, h = -1;
      const bool ok = prefixlm::unit_of((int)b, n, H, &i, &h);
      printf("%ld %d %d %d\n", b, ok ? 1 : 0, i, h);
    }
  }
  return 0;
}
'''

CASES = [(H, n) for H in (1, 2, 3, 5, 6, 8, 10, 12, 14, 16, 20, 24) for n in (1, 2, 3, 7, 64, 135)]


@pytest.fixture(scope="module")
def table():
    from prefixlm._build import hipcc
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "u.cpp"), os.path.join(d, "u")
        open(src, "w").write(PROGRAM)
        subprocess.run([hipcc(), "-std=c++17", f"-I{CSRC}", src, "-o", exe], check=True, capture_output=True)
        inp = "".join(f"{H} {n}\n" for H, n in CASES)
        out = subprocess.run([exe], input=inp, capture_output=True, text=True, check=True).stdout
    res, cur = {}, None
    for line in out.splitlines():
        f = line.split()
        if f[0] == "G":
            cur = (int(f[1]), int(f[2]))
            res[cur] = []
        else:
            res[cur].append(tuple(int(x) for x in f))
    return res


@pytest.mark.parametrize("H,n", CASES)
def test_every_unit_once_in_cost_order_and_balanced(table, H, n):
    rows = table[(H, n)]
    seen = {}
    per_xcd = {x: [] for x in range(8)}
    for b, ok, i, h in rows:
        if ok:
            assert 0 <= i < n and 0 <= h < H
            assert (i, h) not in seen, (i, h)
            seen[(i, h)] = b
            per_xcd[b % 8].append((b // 8, i, h))
    assert len(seen) == n * H
    counts = []
    for x, units in per_xcd.items():
        units.sort()
        # the valid units of an XCD are a prefix of its sequence, in item order
        assert [j for j, _, _ in units] == list(range(len(units)))
        items = [i for _, i, _ in units]
        assert items == sorted(items)
        counts.append(len(units))
        # heads this XCD touches: its own F = H // 8 plus at most the remainder parts
        r = H % 8
        extra = 0 if r == 0 else r // {1: 1, 2: 2, 3: 1, 4: 4, 5: 1, 6: 2, 7: 1}[r]
        assert len({h for _, _, h in units}) <= H // 8 + extra
    # equal shares up to one block of items
    assert max(counts) - min(counts) <= max(1, (H % 8) and 8)
    if H % 8 == 0:
        assert all(b == i * H + h for b, ok, i, h in rows if ok)
