// Prints branchcraft::auto_splits (the reference-compatible C++ wrapper,
// default cap 16), the same with a BC_MAX_SPLITS cap, and bc_auto_splits for
// a sweep of shapes, one line per shape: "batch max_length cus wrapper
// wrapper_uncapped c_abi".  Host-only: no HIP call reaches a device.
#include <cstdio>

#include "branchcraft.hpp"

int main() {
  const int batches[] = {1, 2, 4, 8, 16, 32, 64, 128, 256, 512};
  const int lengths[] = {0, 100, 511, 512, 1024, 1025, 4096, 8192, 32768, 1 << 20};
  const int cus[] = {1, 80, 256, 304};
  for (int b : batches)
    for (int len : lengths)
      for (int cu : cus) {
        const branchcraft::Shape s{b, 32, 8, 128, (len + 15) / 16 + 1, 1};
        std::printf("%d %d %d %d %d %d\n", b, len, cu, branchcraft::auto_splits(s, len, cu),
                    branchcraft::auto_splits(s, len, cu, BC_MAX_SPLITS),
                    bc_auto_splits(s, len, cu));
      }
  return 0;
}
