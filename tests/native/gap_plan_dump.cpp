// Test helper: prints the complete-tree walk of numpy's pairwise summation
// that the GlobalAvgPool2d kernels follow (novaq_gap_plan.h), for n = 1 ..
// argv[1]: one line per n, "n D longest shortest" then "vi,off,len" for every
// virtual leaf that owns a real leaf.  Built with g++ by tests/test_gap_plan.py.
#include <cstdio>
#include <cstdlib>

#include "../../novann_amd/csrc/novaq_gap_plan.h"

int main(int argc, char** argv) {
  using namespace novaq::gap_detail;
  const int nmax = argc > 1 ? std::atoi(argv[1]) : 8192;
  for (int n = 1; n <= nmax; ++n) {
    const int D = tree_depth(n);
    std::printf("%d %d %d %d", n, D, leaf_len(n, true), leaf_len(n, false));
    // one virtual leaf past the tree too: it must own nothing
    for (int vi = 0; vi <= (1 << D); ++vi) {
      int off = -1, len = -1;
      if (virtual_leaf(n, D, vi, off, len)) std::printf(" %d,%d,%d", vi, off, len);
    }
    std::printf("\n");
  }
  return 0;
}
