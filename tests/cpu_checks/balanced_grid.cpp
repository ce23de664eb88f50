// balanced_grid.cpp -- host check of mxk::balanced_grid (mx_kernels.hpp), the
// block count the persistent GEMMs run on. TEST PROGRAM.
//
// For every tile count 1..20000 and resident-block counts that are whole
// multiples of the 8 XCDs, the balanced count g must:
//   - lie in [1, grid];
//   - walk the tiles in as many rounds as `grid` blocks: ceil(n / g) ==
//     ceil(n / grid), so the makespan in tiles is unchanged;
//   - be a multiple of 8 from 16 blocks up (the kernel's XCD-chunked order);
//   - be the fewest such blocks: one step fewer (8 blocks from 16 up, else 1)
//     needs another round.
// Prints "ok <cases>" and exits 0, or names the first failure and exits 1.
#include <cstdio>

#include "mx_kernels.hpp"

static int rounds(int n, int g) { return (n + g - 1) / g; }

int main() {
  const int grids[] = {64, 104, 256, 304};
  long cases = 0;
  for (int grid : grids) {
    for (int n = 1; n <= 20000; ++n) {
      const int g = mxk::balanced_grid(n, grid);
      // the next smaller valid count: 8 fewer above 16 blocks, else one fewer
      const int step = g > 16 ? 8 : 1;
      const bool fewer_needs_more = g == 1 || rounds(n, g - step) > rounds(n, grid);
      if (g < 1 || g > grid || rounds(n, g) != rounds(n, grid) || (g >= 16 && g % 8 != 0) ||
          !fewer_needs_more) {
        std::printf("FAIL: balanced_grid(%d, %d) = %d\n", n, grid, g);
        return 1;
      }
      ++cases;
    }
  }
  // The packed bge-base GEMMs (M 17,455 on 256 x 256 tiles): QKV, FFN-up and
  // the N = 768 sites all on 208 of 256 blocks.
  if (mxk::balanced_grid(621, 256) != 208 || mxk::balanced_grid(828, 256) != 208 ||
      mxk::balanced_grid(207, 256) != 208) {
    std::printf("FAIL: bge-base sites\n");
    return 1;
  }
  std::printf("ok %ld\n", cases);
  return 0;
}
