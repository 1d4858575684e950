// Work plan of the register-storage flash-Sinkhorn forward (sinkhorn_fwd_blk.h):
// member grids, members per group and LDS sizes.  Plain C++ shared by the kernel, the
// host launch code and a host-side check of the plan (tests/test_blk_plan.py builds
// it with g++).
#pragma once
#include <stddef.h>

#ifndef __HIPCC__
#define __host__
#define __device__
#endif

namespace dfl {

constexpr int BLK_NT = 512;  // 8 waves, two per SIMD
constexpr int BLK_NW = 8;     // waves per workgroup
constexpr int BLK_WR = 3;     // row tiles of a wave's sub-block, at most
constexpr int BLK_WC = 8;     // column tiles of a wave's sub-block (a wave always sweeps this many:
                              // columns past its block carry logits of NEG_BIG, which add 0)
constexpr int BLK_MAXRC = 8;  // rows / columns of a member grid, at most
constexpr int BLK_MAXS = 32;  // groups per XCD, at most
constexpr int BLK_MAXL = 64;  // workgroups per XCD, at most
// Exchange vectors of Np words per (b,h): C row partials and R column partials, each in
// two slots used by alternate iterations, then the final v.
constexpr int BLK_XCH_VECS = 4 * BLK_MAXRC + 1;

__host__ __device__ inline int cdiv(int a, int b) { return (a + b - 1) / b; }

// Member grid of a group: R x C blocks and the wave split sr x sc (sr * sc = 8) of a
// block.  pairs = the tiles one wave sweeps (its row tiles, at most, times BLK_WC, the
// columns every wave sweeps): the sweep time of a member.
struct BlkGrid {
  int R, C, sr, sc;
  int pairs;  // 0x7fffffff when no grid fits
};
constexpr int BLK_NONE = 0x7fffffff;

// Best grid for T tiles and at most G members: fewest tiles swept per wave; ties go to
// fewer exchange words per member (C rows + R columns per tile), then fewer members.
__host__ __device__ inline BlkGrid blk_grid(int T, int G) {
  BlkGrid best{0, 0, 1, 8, BLK_NONE};
  if (T <= 0) {
    best.pairs = 0;
    return best;
  }
  int best_words = 0x7fffffff;
  for (int R = 1; R <= BLK_MAXRC && R <= T && R <= G; ++R) {
    int C = G / R;
    if (C > BLK_MAXRC) C = BLK_MAXRC;
    if (C > T) C = T;
    const int TR = cdiv(T, R), TC = cdiv(T, C);
    int bsr = 0, bw = 0x7fffffff;
    for (int sr = 1; sr <= 8; sr *= 2) {
      const int wr = cdiv(TR, sr), wc = cdiv(TC, 8 / sr);
      if (wr <= BLK_WR && wc <= BLK_WC && wr < bw) {
        bw = wr;
        bsr = sr;
      }
    }
    if (!bsr) continue;
    const int pairs = bw * BLK_WC, words = C * TR + R * TC;
    if (pairs < best.pairs || (pairs == best.pairs && (words < best_words ||
                                                       (words == best_words && R * C < best.R * best.C)))) {
      best = BlkGrid{R, C, bsr, 8 / bsr, pairs};
      best_words = words;
    }
  }
  return best;
}

// Members per group for S groups of T[s] tiles sharing L workgroups (one XCD): each
// group starts with one member, then every further workgroup goes to the group whose
// members carry the most tiles (cost[s * L + G - 1] = blk_grid(T[s], G).pairs).  If
// that leaves a group without a grid, the even split is taken (the host checks that
// it fits every group at T = ceil(N / 16)).  Returns false if S > L.
__host__ __device__ inline bool blk_allocate(const int* cost, int S, int L, int* Gs) {
  if (S > L) return false;
  for (int s = 0; s < S; ++s) Gs[s] = 1;
  for (int left = L - S; left > 0; --left) {
    int arg = 0, worst = -1;
    for (int s = 0; s < S; ++s) {
      const int c = cost[s * L + Gs[s] - 1];
      if (c > worst) {
        worst = c;
        arg = s;
      }
    }
    if (worst <= 0) break;  // every group is empty
    ++Gs[arg];
  }
  bool ok = true;
  for (int s = 0; s < S; ++s) ok = ok && cost[s * L + Gs[s] - 1] != BLK_NONE;
  if (!ok)
    for (int s = 0; s < S; ++s) Gs[s] = L / S + (s < L % S ? 1 : 0);
  return true;
}

// LDS of the iteration phase for a block of TR x TC tiles split sr x sc over the waves:
// row / column partials of the waves, operand parts of the potentials, potentials,
// shifts and marginals.
__host__ __device__ inline size_t blk_iter_lds(int TR, int TC, int sr, int sc) {
  size_t b = (size_t)sc * TR * 64 * 4;  // row partials   [sc][TR][64]
  b += (size_t)sr * TC * 256 * 4;       // column partials [sr][TC][64][4]
  b += (size_t)2 * TR * 16 * 8;         // row operand parts: -shift, u
  b += (size_t)2 * TC * 16 * 8;         // column operand parts: v, -shift
  b += (size_t)3 * TR * 16 * 4;         // u, row shift, log mu
  b += (size_t)3 * TC * 16 * 4;         // v, column shift, log nu
  return b;
}
// Upper bound of blk_iter_lds over the grids blk_grid can return for T tiles.
__host__ __device__ inline size_t blk_iter_lds_bound(int T) {
  const int tr = T < 8 * BLK_WR ? T : 8 * BLK_WR;  // block rows
  const int tc = T < 8 * BLK_WC ? T : 8 * BLK_WC;  // block columns
  // sc * TR <= 8 * min(WR, T) and sr * TC <= 8 * min(WC, T) for any split that fits
  const int scr = 8 * (T < BLK_WR ? T : BLK_WR), src = 8 * (T < BLK_WC ? T : BLK_WC);
  size_t b = (size_t)scr * 64 * 4 + (size_t)src * 256 * 4;
  b += (size_t)2 * tr * 16 * 8 + (size_t)2 * tc * 16 * 8 + (size_t)3 * tr * 16 * 4 + (size_t)3 * tc * 16 * 4;
  return b;
}
// Whether every XCD's groups get a member grid that fits the register tiles when each
// (b,h) has all N tokens valid (the most tiles the device-side allocation can see):
// with L workgroups per XCD the most loaded XCD hosts ceil(B*H / 8) groups, and the
// even split must fit each of them (blk_allocate falls back to it).
__host__ __device__ inline bool blk_fits(int B, int H, int N, int L) {
  const int S = (B * H + 7) / 8;
  if (L > BLK_MAXL || S > BLK_MAXS || S > L) return false;
  return blk_grid(cdiv(N, 16), L / S).pairs != BLK_NONE;
}

}  // namespace dfl
