// Launch-shape rules that decide a kernel's work split on the host.  Plain C++
// (no HIP types) so that the host test suite compiles them with g++ and checks
// them over many device sizes.
#pragma once

#if defined(__HIPCC__)
#define MKD_RULE __host__ __device__ __forceinline__
#else
#define MKD_RULE inline
#endif

namespace mkd {

// QKV projection + norm at one block per CU (qkv_norm.hip): N / 16 row tiles of
// a K-long contraction over 8 waves (nf = K / 256 fragments per wave).  With
// more tiles than CUs, the tiles past the CU count are split into K quarters
// taken by two extra waves of the blocks on the first CUs, and the head
// preparation adds the four quarter partials of every head at or past the
// split row.  Returns that number of extra tiles, or 0 (no split) when:
//   * the tiles fit the CUs, the CU count is unknown, or nf > 8;
//   * more than one extra tile per four CUs would be needed;
//   * the split row (main tiles * 16) is not a multiple of the head size d, so
//     that one head would straddle it (its rows before the split have a single
//     partial, the rest four; the head preparation reads a head as one or the
//     other).
inline int qkv_extra_tiles_rule(int N, int K, int d, int cus) {
  const int tiles = N / 16, nf = K / 32 / 8;
  if (cus <= 0 || tiles <= cus || nf > 8 || d <= 0) return 0;
  const int extra = tiles - cus;
  if (extra * 4 > cus) return 0;
  return ((tiles - extra) * 16) % d == 0 ? extra : 0;
}

// The LDS-tiled GEMM (gemm_tile.hip) deals its `live` logical tiles to the 8
// XCDs (workgroups go round-robin to the XCDs by linear id L): XCD x = L % 8 owns
// the contiguous run starting at x * q + min(x, r) of q or q + 1 tiles (live =
// 8q + r), and its k-th block (k = L / 8) takes tile k of the run.  Returns
// whether block L has a tile (then *lt); with a grid of at least `live` blocks
// every tile is taken exactly once.
MKD_RULE bool tile_deal_rule(int live, int L, int* lt) {
  const int xcd = L % 8, k = L / 8, q = live / 8, r = live % 8;
  *lt = xcd * q + (xcd < r ? xcd : r) + k;
  return k < q + (xcd < r ? 1 : 0);
}

// K slices for a dense tiled GEMM (256 x 256 output tiles, 32-wide stages) whose
// tiles leave CUs idle: the largest of 2, 4, 8 that divides the stage count,
// keeps at least 16 stages per slice and tiles x slices within the CU count
// (cus <= 0: taken as 256).
MKD_RULE int tile_kgrid_rule(int N, int K, int T, int cus) {
  if (cus <= 0) cus = 256;
  if (K <= 0 || K % 32 != 0 || N <= 0 || T <= 0) return 1;
  const long long tiles = (long long)((N + 255) / 256) * ((T + 255) / 256);
  const int KB = K / 32;
  int kg = 1;
  for (int c = 2; c <= 8; c *= 2)
    if (KB % c == 0 && KB / c >= 16 && tiles * c <= cus) kg = c;
  return kg;
}

// Prefill attention work units, longest query tiles first (unit u = tile
// nqt - 1 - u / sets of set u % sets).  Where the grid of `total` blocks is
// resident at two blocks per CU (cus < total <= 2 cus, pair_cus = cus, else 0),
// block L >= cus -- on the CU of block L - cus -- takes unit total - 1 - (L -
// cus), so the two tiles of a CU have complementary lengths; a bijection of
// [0, total) either way.
MKD_RULE int prefill_unit_rule(int L, int total, int pair_cus) {
  return (pair_cus > 0 && L >= pair_cus) ? total - 1 - (L - pair_cus) : L;
}
MKD_RULE int prefill_pair_rule(long long total, int cus, int heads_per_block) {
  return (heads_per_block == 8 && cus > 0 && total > cus && total <= 2LL * cus) ? cus : 0;
}

// Split routing of tk slots over e experts: slots per placing block (a multiple
// of 256, at least min_chunk), such that the chunks number at most max_chunks
// and chunks x e counts fit max_counts; 0 when one block places them all (tk
// <= min_chunk, or fewer than two chunks fit).
MKD_RULE int route_chunk_rule(int tk, int e, int min_chunk, int max_chunks, int max_counts) {
  if (tk <= min_chunk || e <= 0) return 0;
  const int by_counts = max_counts / e;
  const int max_nc = max_chunks < by_counts ? max_chunks : by_counts;
  if (max_nc < 2) return 0;
  int cs = (tk + max_nc - 1) / max_nc;
  cs = (cs + 255) / 256 * 256;
  return cs > min_chunk ? cs : min_chunk;
}

}  // namespace mkd
