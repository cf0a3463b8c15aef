// Brute-force check of the stream-K split shared by the decode kernel and its
// merge (velokv_params.h): ranges cover [0, W) in order, none is empty, they
// differ in length by at most one block, and sk_worker_of inverts sk_begin for
// every block.
#include <cstdio>
#include <random>

#include "velokv_params.h"

using namespace velokv;

static int check(int64_t W, int32_t nw) {
  const SkSplit s = sk_split(W, nw);
  if (s.nw < 1 || s.nw > nw || s.nw > W) { printf("bad nw %d for W=%lld nw=%d\n", s.nw, (long long)W, nw); return 1; }
  if (sk_begin(s, 0) != 0 || sk_begin(s, s.nw) != W) { printf("ends W=%lld nw=%d\n", (long long)W, nw); return 1; }
  for (int32_t w = 0; w < s.nw; ++w) {
    const int64_t b0 = sk_begin(s, w), b1 = sk_begin(s, w + 1);
    if (b1 - b0 < W / s.nw || b1 - b0 > (W + s.nw - 1) / s.nw) {
      printf("range %lld of worker %d (W=%lld nw=%d)\n", (long long)(b1 - b0), w, (long long)W, nw);
      return 1;
    }
    const int64_t step = W <= 300000 ? 1 : (b1 - b0 > 2 ? b1 - b0 - 1 : 1);  // every block, or the ends
    for (int64_t x = b0; x < b1; x += step)
      if (sk_worker_of(s, x) != w) {
        printf("worker_of(%lld)=%d, want %d (W=%lld nw=%d)\n", (long long)x, sk_worker_of(s, x), w, (long long)W, nw);
        return 1;
      }
  }
  return 0;
}

int main() {
  int bad = 0;
  bad |= check(262144, 2048);  // 64 x 8192, Hkv 8
  bad |= check(141600, 2048);  // a ragged batch
  bad |= check(100, 2048);     // W < nw: 100 workers of one block
  bad |= check(1, 2048);
  bad |= check((int64_t)1 << 26, 65536);
  std::mt19937_64 rng(5);
  for (int i = 0; i < 400 && !bad; ++i) {
    const int32_t nw = 1 + (int32_t)(rng() % 5000);
    bad |= check(1 + (int64_t)(rng() % (300LL * nw)), nw);
  }
  printf(bad ? "FAILED\n" : "ok\n");
  return bad;
}
