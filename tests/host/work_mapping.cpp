// Host check of the attention kernels' workgroup -> work item mappings
// (kerneldev_amd/csrc/kd_work.h) over many (items per head m, heads H)
// shapes, with n = H m workgroups:
//   xcd_remap: a bijection of [0, n); the workgroups of one XCD (wg = x,
//              x + 8, ...) take one contiguous range of items, in order;
//   fwd_work:  the workgroups of XCD x take exactly the items xcd_remap gives
//              that XCD; where those ranges are whole heads it is xcd_remap
//              itself, and where they split a head the ranks never decrease
//              from one slot to the next (rank-major within the range).
// Prints "shapes S failures F" and each failing shape.
#define KD_WORK_FN inline
#include "../../kerneldev_amd/csrc/kd_work.h"

#include <algorithm>
#include <cstdio>
#include <vector>

int main() {
  const int ms[] = {1, 2, 3, 7, 8, 16, 64, 96, 128, 129, 192, 256};
  const int hs[] = {1, 2, 3, 5, 8, 12, 16, 32, 64};
  int shapes = 0, failures = 0;
  for (int m : ms)
    for (int H : hs) {
      const int n = H * m;
      ++shapes;
      bool ok = true;
      std::vector<int> seen(n, 0);
      for (int x = 0; x < 8; ++x) {
        std::vector<int> range, got;
        int prev_w = -1, prev_r = -1;
        for (int wg = x; wg < n; wg += 8) {
          const int w = kd::xcd_remap(wg, n);
          if (w < 0 || w >= n || (prev_w >= 0 && w != prev_w + 1)) ok = false;
          if (w >= 0 && w < n) seen[w]++;
          prev_w = w;
          range.push_back(w);
          int h = -1, r = -1;
          kd::fwd_work(wg, n, m, &h, &r);
          if (h < 0 || h >= H || r < 0 || r >= m) {
            ok = false;
            continue;
          }
          got.push_back(h * m + r);
          const bool whole = n % 8 == 0 && (n / 8) % m == 0;
          if (whole && h * m + r != w) ok = false;
          if (!whole && r < prev_r) ok = false;
          prev_r = r;
        }
        std::sort(range.begin(), range.end());
        std::sort(got.begin(), got.end());
        if (range != got) ok = false;
      }
      for (int i = 0; i < n; ++i)
        if (seen[i] != 1) ok = false;
      if (!ok) {
        ++failures;
        std::printf("FAIL m=%d H=%d\n", m, H);
      }
    }
  std::printf("shapes %d failures %d\n", shapes, failures);
  return failures != 0;
}
