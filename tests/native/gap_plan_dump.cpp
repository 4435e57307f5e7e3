// Test helper: prints novaq::gap_plan for n = 1 .. argv[1] (the host-side
// plan of numpy's pairwise summation used by the GlobalAvgPool2d kernel), one
// line per n: "n ok L nops balanced prog-words... off,len ...".  Built with g++ by
// tests/test_gap_plan.py.
#include <cstdio>
#include <cstdlib>

#include "../../novann_amd/csrc/novaq_gap_plan.h"

int main(int argc, char** argv) {
  const int nmax = argc > 1 ? std::atoi(argv[1]) : 8192;
  for (int n = 1; n <= nmax; ++n) {
    novaq::GapPlan p;
    const bool ok = novaq::gap_plan(n, p);
    std::printf("%d %d %d %d %d", n, ok ? 1 : 0, ok ? p.L : 0, ok ? p.nops : 0,
                ok ? p.balanced : 0);
    if (ok) {
      for (int w = 0; w < novaq::GAP_PROG_WORDS; ++w) std::printf(" %u", p.prog[w]);
      for (int i = 0; i < p.L; ++i) std::printf(" %d,%d", p.leaf[i].off, p.leaf[i].len);
    }
    std::printf("\n");
  }
  return 0;
}
