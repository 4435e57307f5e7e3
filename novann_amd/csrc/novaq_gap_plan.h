// Host-side plan of numpy's pairwise float32 summation on a plane of at most
// 8192 elements (one block of numpy's ufunc buffer), used by the wave-parallel
// GlobalAvgPool2d kernel in pool.hip.  Plain C++ (no HIP types) so that a host
// compiler can build it on its own.
//
// numpy's pairwise sum of n elements: n <= 128 is one leaf (8 interleaved
// partial sums, combined ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)), then the
// remainder in order; below 8 elements a plain in-order sum); otherwise the
// run splits at n2 = n/2 - (n/2) % 8 and the two halves' sums are added.  For
// n <= 8192 this gives at most 65 leaves (every n in [7689, 8191] does) and a
// tree at most 7 levels deep, whose postfix evaluation needs a stack of 8.
#ifndef NOVAQ_GAP_PLAN_H
#define NOVAQ_GAP_PLAN_H

#include <stdint.h>

namespace novaq {

constexpr int GAP_MAX_LEAVES = 80;                   // 65 are needed at n <= 8192
constexpr int GAP_PROG_WORDS = (2 * GAP_MAX_LEAVES + 31) / 32;  // 2L - 1 postfix bits
constexpr int GAP_MAX_STACK = 8;

struct GapLeaf {
  int off, len;
};

// The leaves in order and the combining tree as a postfix program: bit k of
// prog is 1 for "push the next leaf's sum", 0 for "add the two top values".
// balanced: the tree is complete (L = 2^d <= 8 leaves, all at depth d), so
// adding neighbouring leaf sums pairwise, then neighbouring pairs, and so on,
// associates exactly as the program does.
struct GapPlan {
  int L, nops, balanced;
  uint32_t prog[GAP_PROG_WORDS];
  GapLeaf leaf[GAP_MAX_LEAVES];
};

namespace gap_detail {
inline bool plan_rec(int n, int off, int depth, GapPlan& p) {
  if (depth >= GAP_MAX_STACK) return false;
  if (n <= 128) {
    if (p.L >= GAP_MAX_LEAVES || p.nops >= 32 * GAP_PROG_WORDS) return false;
    p.leaf[p.L].off = off;
    p.leaf[p.L].len = n;
    ++p.L;
    p.prog[p.nops >> 5] |= 1u << (p.nops & 31);
    ++p.nops;
    return true;
  }
  int n2 = n / 2;
  n2 -= n2 % 8;
  if (!plan_rec(n2, off, depth + 1, p) || !plan_rec(n - n2, off + n2, depth + 1, p))
    return false;
  if (p.nops >= 32 * GAP_PROG_WORDS) return false;
  ++p.nops;  // bit 0: add
  return true;
}
inline void depth_range(int n, int depth, int& lo, int& hi) {
  if (n <= 128) {
    lo = depth < lo ? depth : lo;
    hi = depth > hi ? depth : hi;
    return;
  }
  int n2 = n / 2;
  n2 -= n2 % 8;
  depth_range(n2, depth + 1, lo, hi);
  depth_range(n - n2, depth + 1, lo, hi);
}
// the length of the longest (longest = true) or shortest leaf
inline int leaf_len(int n, bool longest) {
  if (n <= 128) return n;
  int n2 = n / 2;
  n2 -= n2 % 8;
  const int a = leaf_len(n2, longest), b = leaf_len(n - n2, longest);
  return (a > b) == longest ? a : b;
}
}  // namespace gap_detail

// Fills p for a plane of n elements (1 <= n).  Returns false, leaving p
// unusable, when the plan does not fit GapPlan's capacity (the caller then
// takes a path without a plan); that does not happen for n <= 8192.
inline bool gap_plan(int n, GapPlan& p) {
  p = GapPlan{};
  if (n < 1) return false;
  if (!gap_detail::plan_rec(n, 0, 0, p)) return false;
  int lo = 1 << 30, hi = -1;
  gap_detail::depth_range(n, 0, lo, hi);
  p.balanced = (lo == hi && p.L == (1 << lo) && p.L <= 8) ? 1 : 0;
  return true;
}

}  // namespace novaq

#endif  // NOVAQ_GAP_PLAN_H
