// Workgroup -> work item mappings of the attention kernels.  Plain integer
// code: the including file defines KD_WORK_FN (the library:
// __host__ __device__ inline; a host test program: inline).
#pragma once

namespace kd {

KD_WORK_FN int work_imin(int a, int b) { return a < b ? a : b; }
KD_WORK_FN int work_imax(int a, int b) { return a > b ? a : b; }

// Linear workgroup id -> work index so that each XCD (workgroups are dealt
// round-robin over the 8 XCDs) receives one contiguous range of work items,
// i.e. the blocks of the same head share that XCD's L2.  The kernels order
// work head-major (so every XCD gets the same mix of batch rows) and take
// each head's (b, block) items in the plan's longest-first work order.
KD_WORK_FN int xcd_remap(int wg, int n) {
  constexpr int NX = 8;
  const int per = n / NX;
  const int rem = n % NX;
  const int x = wg % NX, slot = wg / NX;
  // the first `rem` XCDs take per+1 items each
  const int base = x * per + work_imin(x, rem);
  const int cap = per + (x < rem ? 1 : 0);
  if (slot < cap) return base + slot;
  return wg;  // unreachable when gridDim.x == n
}

// The forward's work: head h and rank r in the plan's order (m = B n items
// per head, n_items = H m = gridDim.x).  XCD x = wg % 8 holds the contiguous
// item range [base, base + cap) of xcd_remap (items g = h m + r).  When every
// range is whole heads, its slots take them head by head, each head's items
// longest first (the range of xcd_remap as it is).  When the ranges split a
// head, slot s = wg / 8 takes the s-th item of the range in rank-major order
// (ascending r, then h): otherwise an XCD would start with the short tail of
// the head it shares with the previous XCD, and take the long items of its
// next head last.
KD_WORK_FN void fwd_work(int wg, int n_items, int m, int* h_out, int* r_out) {
  constexpr int NX = 8;
  const int per = n_items / NX, rem = n_items % NX;
  if (rem == 0 && per % m == 0) {
    const int work = xcd_remap(wg, n_items);
    *h_out = work / m;
    *r_out = work - *h_out * m;
    return;
  }
  const int x = wg % NX, s = wg / NX;
  const int base = x * per + work_imin(x, rem);
  const int cap = per + (x < rem ? 1 : 0);
  const int h0 = base / m, h1 = (base + cap - 1) / m;
  auto count_below = [&](int r) {  // items of the range with rank < r
    int c = 0;
    for (int h = h0; h <= h1; ++h) {
      const int lo = work_imax(0, base - h * m), hi = work_imin(m, base + cap - h * m);
      c += work_imax(0, work_imin(r, hi) - lo);
    }
    return c;
  };
  int lo = 0, hi = m;  // count_below(lo) <= s < count_below(hi) (count_below(m) = cap)
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (count_below(mid) <= s) lo = mid;
    else hi = mid;
  }
  int j = s - count_below(lo);  // the j-th head (ascending) of the range holding rank lo
  *h_out = h0;
  *r_out = lo;
  for (int h = h0; h <= h1; ++h) {
    const int lo_h = work_imax(0, base - h * m), hi_h = work_imin(m, base + cap - h * m);
    if (lo >= lo_h && lo < hi_h) {
      if (j == 0) {
        *h_out = h;
        return;
      }
      --j;
    }
  }
}

}  // namespace kd
