// numpy's pairwise float32 summation of one block (at most 8192 elements, its
// ufunc buffer) as the GlobalAvgPool2d kernels in pool.hip walk it.  Plain
// C++ (no HIP types) so that a host compiler can build it on its own; under
// hipcc the descent is also a device function, the one the kernels run.
//
// numpy's pairwise sum of n elements: n <= 128 is one leaf (8 interleaved
// partial sums, combined ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)), then the
// remainder in order; below 8 elements a plain in-order sum); otherwise the
// run splits at n2 = n/2 - (n/2) % 8 and the two halves' sums are added.
//
// The kernels make that tree complete: with D its deepest level, virtual
// leaf v (0 <= v < 2^D) walks down D levels taking the bits of v from the top;
// where a real leaf is reached at a level d < D, the virtual leaf whose
// remaining bits are all 0 owns it and the others are idle (they hold -0.0f,
// the exact additive identity).  Adding virtual leaves neighbours first, level
// by level, then associates exactly as numpy's recursion.
#ifndef NOVAQ_GAP_PLAN_H
#define NOVAQ_GAP_PLAN_H

#ifdef __HIPCC__
#define NOVAQ_GAP_HD __host__ __device__
#else
#define NOVAQ_GAP_HD
#endif

namespace novaq {
namespace gap_detail {

// deepest leaf level of the tree over n elements (0: one leaf)
inline int tree_depth(int n) {
  if (n <= 128) return 0;
  int n2 = n / 2;
  n2 -= n2 % 8;
  const int a = tree_depth(n2), b = tree_depth(n - n2);
  return 1 + (a > b ? a : b);
}

// the length of the longest (longest = true) or shortest leaf
inline int leaf_len(int n, bool longest) {
  if (n <= 128) return n;
  int n2 = n / 2;
  n2 -= n2 % 8;
  const int a = leaf_len(n2, longest), b = leaf_len(n - n2, longest);
  return (a > b) == longest ? a : b;
}

// Virtual leaf vi of the depth-D tree over n elements: whether it owns a real
// leaf, and that leaf's first element and length.
NOVAQ_GAP_HD inline bool virtual_leaf(int n, int D, int vi, int& off, int& len) {
  bool owner = (vi >> D) == 0;
  off = 0;
  len = n;
  for (int lvl = D - 1; lvl >= 0; --lvl) {
    const int bit = (vi >> lvl) & 1;
    if (len > 128) {
      const int n2 = (len >> 1) & ~7;
      off = bit ? off + n2 : off;
      len = bit ? len - n2 : n2;
    } else if (bit) {
      owner = false;
    }
  }
  return owner;
}

}  // namespace gap_detail
}  // namespace novaq

#endif  // NOVAQ_GAP_PLAN_H
