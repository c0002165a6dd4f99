// Launch-shape rules that decide a kernel's work split on the host.  Plain C++
// (no HIP types) so that the host test suite compiles them with g++ and checks
// them over many device sizes.
#pragma once

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

}  // namespace mkd
