// Host check of the kernels' grid arithmetic (pseudobrain_amd/csrc/schedule.hpp)
// for device shapes other than the full MI355X: every block maps to a distinct
// (group, member) and every prep item to exactly one workgroup. Built and run by
// tests/test_schedule.py with the host compiler (__host__/__device__ defined away).
#include <cstdio>
#include <vector>

#include "schedule.hpp"

using namespace pbgdn;

static int failures = 0;
#define CHECK(cond, ...)                  \
  do {                                    \
    if (!(cond)) {                        \
      if (failures++ < 20) {              \
        std::printf("FAIL %s: ", #cond);  \
        std::printf(__VA_ARGS__);         \
        std::printf("\n");                \
      }                                   \
    }                                     \
  } while (0)

static void check_xcd_group() {
  for (int xcds : {1, 2, 4, 8})
    for (int ngroups = 1; ngroups <= 48; ++ngroups)
      for (int gsize = 1; gsize <= 16; ++gsize) {
        std::vector<int> seen(ngroups * gsize, 0);
        for (int L = 0; L < ngroups * gsize; ++L) {
          int g, m;
          xcd_group(L, ngroups, gsize, xcds, g, m);
          CHECK(g >= 0 && g < ngroups && m >= 0 && m < gsize, "xcds %d ngroups %d gsize %d L %d", xcds, ngroups,
                gsize, L);
          if (g < 0 || g >= ngroups || m < 0 || m >= gsize) continue;
          seen[g * gsize + m]++;
          if (xcds > 1 && ngroups % xcds == 0)
            CHECK(L % xcds == g % xcds, "group %d member %d on XCD %d (xcds %d)", g, m, L % xcds, xcds);
        }
        for (int i = 0; i < ngroups * gsize; ++i)
          CHECK(seen[i] == 1, "xcds %d ngroups %d gsize %d: pair %d seen %d times", xcds, ngroups, gsize, i, seen[i]);
      }
}

static void check_prep_share() {
  for (int cus : {32, 64, 80, 128, 256})
    for (int xcds : {1, 2, 4, 8})
      for (int wgpc : {1, 2, 3})
        for (long items : {0L, 1L, 7L, 100L, 257L, 1000L, 16448L, 65539L}) {
          const long grid = prep_grid(items, cus, wgpc, xcds);
          CHECK(grid >= 1 || items == 0, "grid %ld", grid);
          std::vector<int> owner(items, -1);
          for (int b = 0; b < grid; ++b) {
            const PrepShare s = prep_share(static_cast<int>(items), static_cast<int>(grid), b, cus, xcds);
            CHECK(s.stride >= 1, "stride %d", s.stride);
            for (long i = s.first; i < s.end; i += s.stride) {
              CHECK(i >= 0 && i < items, "cus %d xcds %d grid %ld block %d item %ld of %ld", cus, xcds, grid, b, i,
                    items);
              if (i < 0 || i >= items) break;
              CHECK(owner[i] < 0, "item %ld owned twice (blocks %d, %d)", i, owner[i], b);
              owner[i] = b;
            }
          }
          for (long i = 0; i < items; ++i) {
            CHECK(owner[i] >= 0, "cus %d xcds %d wgpc %d items %ld: item %ld unowned", cus, xcds, wgpc, items, i);
          }
          // Item i of a tier's segment [begin, end) is on XCD ((i - begin) % stride) / (stride / xcds)
          // when the stride divides over the XCDs: runs of stride / xcds consecutive items share one.
          for (long i = 0; i < items; ++i) {
            const PrepShare s = prep_share(static_cast<int>(items), static_cast<int>(grid), owner[i], cus, xcds);
            if (xcds < 2 || s.stride % xcds != 0) continue;
            const int tier_first_block = owner[i] / s.stride * s.stride;
            const long begin = prep_share(static_cast<int>(items), static_cast<int>(grid), tier_first_block, cus, xcds).first;
            CHECK(owner[i] % xcds == ((i - begin) % s.stride) / (s.stride / xcds), "item %ld on XCD %d", i,
                  owner[i] % xcds);
          }
        }
}

static void check_scan_groups() {
  for (int cus : {32, 64, 128, 256})
    for (int seqs : {1, 2, 8, 100, 1024})
      for (int pairs : {8, 64, 256, 512})
        for (long tokens : {64L, 32768L, 262144L}) {
          const int g = scan_groups(tokens, seqs, pairs, cus);
          CHECK(g >= 1 && g <= seqs, "groups %d of %d sequences", g, seqs);
          if (tokens >= 2048L * seqs) CHECK(g == seqs, "long sequences get a workgroup each");
          if (tokens < 2048L * seqs && pairs * g > cus) CHECK(g == 1, "groups %d overfill %d CUs", g, cus);
        }
}

int main() {
  check_xcd_group();
  check_prep_share();
  check_scan_groups();
  std::printf("%s (%d failures)\n", failures ? "FAILED" : "ok", failures);
  return failures ? 1 : 0;
}
