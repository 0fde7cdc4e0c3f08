// Grid arithmetic of the prefill and backward kernels, as pure functions of
// the device's shape (compute units, XCDs) so that it can be checked on the
// host for any shape. Workgroups are dispatched round-robin over the XCDs
// (block L goes to XCD L % xcds), each with its own L2; the mappings below
// keep the workgroups that read the same chunks on one XCD.
#pragma once

namespace pbgdn {

// Block L of a grid of ngroups * gsize workgroups -> (group, member). When
// ngroups is a multiple of xcds, every member of a group is on XCD
// group % xcds; otherwise groups are consecutive blocks. A bijection either way.
__host__ __device__ inline void xcd_group(int L, int ngroups, int gsize, int xcds, int &group, int &member) {
  if (xcds > 1 && ngroups % xcds == 0) {
    const int slot = L / xcds;
    group = (slot / gsize) * xcds + L % xcds;
    member = slot % gsize;
  } else {
    group = L / gsize;
    member = L % gsize;
  }
}

// The prep kernel's items: the grid is resident from the start with tiers =
// grid / cus workgroups per CU (1 to 3), and the k-th workgroup dispatched to
// a CU (block / cus) runs slower than the ones before it (the oldest waves
// win issue arbitration). The items are split into one contiguous segment
// per tier in proportion to paces of 1, 0.80 and 0.66: the best of the splits
// timed on MI355X at T = 32K (c1 prefill 0.6735-0.6750 ms, against
// 0.6755-0.6769 with 0.85 and 0.74, 0.6750-0.6765 with 0.74 and 0.58,
// 0.678 with equal shares, 0.680 with 0.68 and 0.50); within a
// segment the tier's workgroups take every `stride`-th item from `first`,
// numbered so that consecutive items (the value heads of one key head) share
// an XCD. Every item of [0, items) belongs to exactly one workgroup.
struct PrepShare {
  int first, stride, end;
};
__host__ __device__ inline PrepShare prep_share(int items, int grid, int block, int cus, int xcds) {
  const int pace[3] = {100, 80, 66};
  const int tiers = (cus > 0 && grid % cus == 0 && grid / cus >= 1 && grid / cus <= 3) ? grid / cus : 1;
  PrepShare s;
  s.stride = grid / tiers;
  const int tier = block / s.stride;
  const int j = block % s.stride;
  int total = 0, before = 0;
  for (int t = 0; t < tiers; ++t) {
    total += pace[t];
    if (t < tier) before += pace[t];
  }
  const int begin = static_cast<int>(static_cast<long long>(items) * before / total);
  s.end = static_cast<int>(static_cast<long long>(items) * (before + pace[tier]) / total);
  const bool spread = xcds > 1 && s.stride % xcds == 0;
  s.first = begin + (spread ? (j % xcds) * (s.stride / xcds) + j / xcds : j);
  return s;
}

// Prep grid: wg_per_cu workgroups per CU, fewer (a multiple of the XCDs)
// when the items do not fill them.
__host__ __device__ inline long prep_grid(long items, int cus, int wg_per_cu, int xcds) {
  long grid = static_cast<long>(cus) * wg_per_cu;
  const int x = xcds > 0 ? xcds : 1;
  if (items < grid) grid = (items + x - 1) / x * x;
  return grid;
}

// Sequence groups of the narrow scan (one workgroup per CU): sequences of
// 2,048 tokens or more on average get a workgroup each; shorter ones run back
// to back in groups, one group when the (value head, column tile) pairs fill
// the CUs, else enough groups to.
__host__ __device__ inline int scan_groups(long tokens, int num_seqs, int pairs, int cus) {
  if (tokens >= 2048L * num_seqs) return num_seqs;
  int g = cus / (pairs > 0 ? pairs : 1);
  if (g > num_seqs) g = num_seqs;
  return g < 1 ? 1 : g;
}

}  // namespace pbgdn
