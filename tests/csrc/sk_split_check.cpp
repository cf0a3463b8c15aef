// Brute-force check of the stream-K split shared by the decode kernel and its
// merge (velokv_params.h): ranges cover [0, W) in order, none is empty, none
// exceeds the 256 block ids a worker holds, the weighted ranges follow the
// weights, and sk_worker_of inverts sk_begin for every block.
#include <cstdio>
#include <cstdlib>
#include <random>

#include "velokv_params.h"

using namespace velokv;

static int check(int64_t W, int32_t nw, int32_t nf, int32_t wf, int32_t ws) {
  const SkSplit s = sk_split(W, nw, nf, wf, ws);
  const bool weighted = s.nf > 0;
  if (s.nw < 1 || s.nw > nw) { printf("bad nw %d for W=%lld nw=%d\n", s.nw, (long long)W, nw); return 1; }
  if (sk_begin(s, 0) != 0 || sk_begin(s, s.nw) != W) { printf("ends W=%lld nw=%d\n", (long long)W, nw); return 1; }
  int64_t max_fast = 0, min_fast = W, max_slow = 0, min_slow = W;
  for (int32_t w = 0; w < s.nw; ++w) {
    const int64_t b0 = sk_begin(s, w), b1 = sk_begin(s, w + 1);
    const int64_t len = b1 - b0;
    if (len < 1) { printf("empty range w=%d W=%lld nw=%d nf=%d\n", w, (long long)W, nw, nf); return 1; }
    if (weighted && len > 255) { printf("range %lld > 255 w=%d W=%lld\n", (long long)len, w, (long long)W); return 1; }
    if (!weighted && len > (W + s.nw - 1) / s.nw) { printf("uneven w=%d\n", w); return 1; }
    if (w < s.nf) { max_fast = len > max_fast ? len : max_fast; min_fast = len < min_fast ? len : min_fast; }
    else { max_slow = len > max_slow ? len : max_slow; min_slow = len < min_slow ? len : min_slow; }
    // every block of the range maps back to w (all blocks for small W, the ends otherwise)
    if (W <= 200000) {
      for (int64_t x = b0; x < b1; ++x)
        if (sk_worker_of(s, x) != w) { printf("worker_of(%lld)=%d, want %d (W=%lld nw=%d nf=%d wf=%d ws=%d)\n", (long long)x, sk_worker_of(s, x), w, (long long)W, nw, nf, wf, ws); return 1; }
    } else if (sk_worker_of(s, b0) != w || sk_worker_of(s, b1 - 1) != w) {
      printf("worker_of ends w=%d W=%lld\n", w, (long long)W);
      return 1;
    }
  }
  if (weighted) {
    // fast ranges are wf/ws times the slow ones, up to the rounding of both ends
    const double r_lo = (double)(min_fast) / (double)(max_slow), r_hi = (double)(max_fast) / (double)(min_slow);
    const double want = (double)wf / ws;
    const double tol = 2.0 / (double)min_slow;
    if (want < r_lo * (1 - tol) - 1e-9 || want > r_hi * (1 + tol) + 1e-9) {
      printf("weights %d/%d give ranges fast [%lld,%lld] slow [%lld,%lld]\n", wf, ws, (long long)min_fast,
             (long long)max_fast, (long long)min_slow, (long long)max_slow);
      return 1;
    }
  }
  return 0;
}

int main() {
  int bad = 0;
  // the configurations the decode runs at on one MI355X (2048 workers, 1024 fast)
  bad |= check(262144, 2048, 1024, 117, 100);  // 64 x 8192, Hkv 8
  bad |= check(141600, 2048, 1024, 117, 100);  // ragged
  bad |= check(524288, 2048, 1024, 117, 100);  // 64 x 16k: 256 per worker, weights off
  bad |= check(8191, 2048, 1024, 117, 100);    // W < 4 nw: even split
  bad |= check(100, 2048, 1024, 117, 100);     // W < nw: 100 workers of one block
  bad |= check(1, 2048, 1024, 117, 100);
  bad |= check(262144, 2048, 0, 1, 1);         // unweighted
  std::mt19937_64 rng(5);
  for (int i = 0; i < 400 && !bad; ++i) {
    const int32_t nw = 1 + (int32_t)(rng() % 3000);
    const int64_t W = 1 + (int64_t)(rng() % (300LL * nw));
    const int32_t nf = (int32_t)(rng() % (nw + 1));
    const int32_t wf = 1 + (int32_t)(rng() % 200), ws = 1 + (int32_t)(rng() % 200);
    bad |= check(W, nw, nf, wf, ws);
  }
  printf(bad ? "FAILED\n" : "ok\n");
  return bad;
}
