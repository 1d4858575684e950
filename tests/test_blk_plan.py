"""CPU checks of the register-storage forward's work plan (csrc/sinkhorn_blk_plan.h).

The plan runs inside the kernel (every workgroup computes it from the valid lengths
of the groups on its XCD), so a mistake there would show up as a workgroup owning a
block that does not fit its register tiles or LDS.  A probe built with g++ from the
same header checks, for many (B*H, N) the host accepts and random valid lengths
n <= N of every group:

* every group with tokens gets a member grid that fits (R, C <= 8, each wave's
  sub-block within 3 x 8 tiles), and no more members than its XCD has;
* the blocks of a grid partition the n_tiles x n_tiles tile square exactly;
* the iteration-phase LDS of every block is within the bound the host sizes LDS by;
* at the headline workload (B2 H8 N768, n = 501 / 759 on each XCD, 32 workgroups
  per XCD) every wave sweeps 2 x 8 tiles (a member 128 at most), against the 3 x 48
  tiles of a member's row stripe in the resident forward.
"""

import os
import subprocess
import tempfile

from conftest import PKG_ROOT

PLAN = os.path.join(PKG_ROOT, "csrc", "sinkhorn_blk_plan.h")

PROBE = r"""
#include <stdio.h>
#include <stdlib.h>
#include "PLAN"
using namespace dfl;

static unsigned rng = 12345u;
static int rnd(int n) { rng = rng * 1664525u + 1013904223u; return (int)((rng >> 8) % (unsigned)n); }

int main() {
  int checked = 0, fails = 0;
  const int L = 32;
  for (int BH = 1; BH <= 256; BH = BH < 16 ? BH + 1 : BH * 2) {
    for (int N = 16; N <= 1536; N += 16) {
      if (!blk_fits(1, BH, N, L)) continue;
      const int Tmax = cdiv(N, 16);
      const size_t bound = blk_iter_lds_bound(Tmax);
      for (int trial = 0; trial < 6; ++trial) {
        for (int x = 0; x < 8; ++x) {
          const int S = (BH - x + 7) / 8;
          if (S <= 0) continue;
          int T[BLK_MAXS], cost[BLK_MAXS * BLK_MAXL], Gs[BLK_MAXS];
          for (int s = 0; s < S; ++s) {
            const int n = trial == 0 ? N : (trial == 1 ? 0 : rnd(N + 1));
            T[s] = cdiv(n, 16);
          }
          for (int e = 0; e < S * L; ++e) cost[e] = blk_grid(T[e / L], e % L + 1).pairs;
          if (!blk_allocate(cost, S, L, Gs)) { printf("alloc refused BH=%d N=%d\n", BH, N); ++fails; continue; }
          int tot = 0;
          for (int s = 0; s < S; ++s) {
            tot += Gs[s];
            const BlkGrid g = blk_grid(T[s], Gs[s]);
            ++checked;
            if (T[s] == 0) continue;
            if (g.pairs == BLK_NONE || g.R < 1 || g.C < 1 || g.R > BLK_MAXRC || g.C > BLK_MAXRC ||
                g.R * g.C > Gs[s] || g.sr * g.sc != 8) {
              printf("bad grid BH=%d N=%d T=%d G=%d R=%d C=%d\n", BH, N, T[s], Gs[s], g.R, g.C); ++fails; continue;
            }
            long area = 0;
            for (int r = 0; r < g.R; ++r)
              for (int c = 0; c < g.C; ++c) {
                const int TR = T[s] * (r + 1) / g.R - T[s] * r / g.R, TC = T[s] * (c + 1) / g.C - T[s] * c / g.C;
                area += (long)TR * TC;
                if (TR < 1 || TC < 1) { printf("empty block\n"); ++fails; }
                if (blk_iter_lds(TR, TC, g.sr, g.sc) > bound) {
                  printf("lds %zu > %zu BH=%d N=%d T=%d\n", blk_iter_lds(TR, TC, g.sr, g.sc), bound, BH, N, T[s]); ++fails;
                }
                for (int w = 0; w < 8; ++w) {
                  const int wi = w / g.sc, wj = w % g.sc;
                  const int wr = TR * (wi + 1) / g.sr - TR * wi / g.sr, wc = TC * (wj + 1) / g.sc - TC * wj / g.sc;
                  if (wr > BLK_WR || wc > BLK_WC || wr * BLK_WC > g.pairs) { printf("wave block %dx%d\n", wr, wc); ++fails; }
                }
              }
            if (area != (long)T[s] * T[s]) { printf("area %ld != %d^2\n", area, T[s]); ++fails; }
          }
          if (tot > L) { printf("members %d > %d\n", tot, L); ++fails; }
        }
      }
    }
  }
  // headline: one n = 501 and one n = 759 group per XCD
  int T[2] = {cdiv(501, 16), cdiv(759, 16)}, cost[2 * 32], Gs[2];
  for (int e = 0; e < 64; ++e) cost[e] = blk_grid(T[e / 32], e % 32 + 1).pairs;
  blk_allocate(cost, 2, 32, Gs);
  const BlkGrid g0 = blk_grid(T[0], Gs[0]), g1 = blk_grid(T[1], Gs[1]);
  printf("headline %d %d %d %d %dx%d %dx%d\n", Gs[0], Gs[1], g0.pairs, g1.pairs, g0.R, g0.C, g1.R, g1.C);
  printf("checked %d fails %d\n", checked, fails);
  return fails != 0;
}
"""


def test_register_storage_plan():
    with tempfile.TemporaryDirectory() as td:
        src, exe = os.path.join(td, "plan.cpp"), os.path.join(td, "plan")
        open(src, "w").write(PROBE.replace("PLAN", PLAN))
        subprocess.run(["g++", "-std=c++17", "-O2", "-o", exe, src], check=True)
        out = subprocess.run([exe], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout[-2000:]
    lines = out.stdout.splitlines()
    head = [l for l in lines if l.startswith("headline")][0].split()
    assert int(head[1]) + int(head[2]) <= 32 and head[3:5] == ["16", "16"], head
    assert int(lines[-1].split()[1]) > 1000
