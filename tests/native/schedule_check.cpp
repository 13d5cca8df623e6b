// Host check of the TP kernels' row schedules (o2mi_tp.hpp row_schedule):
// over many (rows, rows per iteration, blocks), in forward and reverse order,
// every row is visited by exactly one (block, iteration) and every iteration
// a kernel may address, including one past the last (iteration `iters`), has a
// descriptor inside [0, n_rows) or covers no rows.  Prints "<cases> cases,
// <bad> bad" and exits non-zero on the first violation.
#include <cstdio>
#include <vector>

#include "o2mi_tp.hpp"

template <bool kReverse>
static int check(int64_t n, int rows_per_iter, int64_t groups) {
  o2mi::TPGeom g{};
  g.n_rows = n;
  g.rows_per_iter = rows_per_iter;
  g.groups = groups;
  std::vector<int> seen(n, 0);
  for (int64_t b = 0; b < groups; ++b) {
    const o2mi::RowSchedule s = o2mi::row_schedule<kReverse>(g, b);
    for (int it = -1; it <= s.iters + 1; ++it) {
      const int r = s.rows(it);
      if (r == 0) continue;
      const int64_t r0 = s.row0(it);
      if (it < 0 || it >= s.iters || r0 < 0 || r0 + r > n) {
        std::printf("out of range: reverse=%d n=%lld rows/iter=%d G=%lld b=%lld it=%d row0=%lld rows=%d\n",
                    (int)kReverse, (long long)n, rows_per_iter, (long long)groups, (long long)b, it,
                    (long long)r0, r);
        return 1;
      }
      for (int k = 0; k < r; ++k) seen[r0 + k]++;
    }
  }
  for (int64_t i = 0; i < n; ++i) {
    if (seen[i] != 1) {
      std::printf("row %lld visited %d times: reverse=%d n=%lld rows/iter=%d G=%lld\n",
                  (long long)i, seen[i], (int)kReverse, (long long)n, rows_per_iter,
                  (long long)groups);
      return 1;
    }
  }
  return 0;
}

int main() {
  int bad = 0, cases = 0;
  for (int64_t n : {1, 2, 3, 7, 127, 128, 129, 300, 1000, 4096, 20000, 131072})
    for (int rows_per_iter : {1, 2, 3, 4, 8, 16})
      for (int64_t groups : {1, 2, 3, 255, 256, 512, 768, 1024}) {
        bad += check<false>(n, rows_per_iter, groups);
        bad += check<true>(n, rows_per_iter, groups);
        cases += 2;
      }
  std::printf("%d cases, %d bad\n", cases, bad);
  return bad != 0;
}
