// Host check of the per-row-weight (V = 1) streamed kernels' work mapping
// (o2mi_radial_streamed.hpp row_wave, o2mi_radial_launch.hpp row_grid): over
// many (edges, channels, channel span), every (edge, channel) is covered by
// exactly one wave of one block, every covered 16-channel range lies inside
// its block's span, and no wave starts at a negative edge.  Prints
// "<cases> cases, <bad> bad" and exits non-zero on the first violation.
#include <algorithm>
#include <cstdio>
#include <vector>

#include "o2mi_radial_launch.hpp"

using namespace o2mi::radial;

static int check(int64_t n, int C, int span) {
  Args a{};
  a.n = n;
  a.C = C;
  a.tile_span = span;
  const dim3 grid = row_grid(a);
  const int waves = kSFwdWaves;
  std::vector<int> seen(n * C, 0);
  for (unsigned by = 0; by < grid.y; ++by) {
    const int u_begin = (int)by * span;
    const int u_end = std::min(u_begin + span, C);
    for (unsigned bx = 0; bx < grid.x; ++bx) {
      for (int wave = 0; wave < waves; ++wave) {
        const RowWave w = row_wave(C, bx, wave, waves);
        if (w.e0 < 0) {
          std::printf("negative edge: n=%lld C=%d span=%d block=%u wave=%d\n", (long long)n, C,
                      span, bx, wave);
          return 1;
        }
        const int64_t rows = std::min<int64_t>(std::max<int64_t>(n - w.e0, 0), kEdgesPerWave);
        for (int u0 = u_begin; u0 < u_end; u0 += 32 * w.pairs) {
          const int c0 = u0 + 32 * w.sub + 16 * w.half;
          if (c0 >= u_end) continue;
          if (c0 < u_begin || c0 + 16 > u_end) {
            std::printf("channels [%d, %d) outside span [%d, %d): n=%lld C=%d wave=%d\n", c0,
                        c0 + 16, u_begin, u_end, (long long)n, C, wave);
            return 1;
          }
          for (int64_t e = w.e0; e < w.e0 + rows; ++e)
            for (int c = c0; c < c0 + 16; ++c) seen[e * C + c]++;
        }
      }
    }
  }
  for (int64_t i = 0; i < n * C; ++i) {
    if (seen[i] != 1) {
      std::printf("edge %lld channel %lld covered %d times: n=%lld C=%d span=%d\n",
                  (long long)(i / C), (long long)(i % C), seen[i], (long long)n, C, span);
      return 1;
    }
  }
  return 0;
}

int main() {
  const int64_t edges[] = {1, 5, 15, 16, 17, 31, 32, 33, 47, 63, 64, 65, 100, 129, 1000};
  int cases = 0, bad = 0;
  for (int64_t n : edges) {
    for (int C = 16; C <= 256; C += 16) {
      for (int span = 16; span <= C; span += 16) {
        ++cases;
        if (check(n, C, span)) {
          ++bad;
          std::printf("%d cases, %d bad\n", cases, bad);
          return 1;
        }
      }
    }
  }
  std::printf("%d cases, %d bad\n", cases, bad);
  return 0;
}
