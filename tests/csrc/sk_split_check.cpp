// Brute-force check of the stream-K split shared by the decode kernel and its
// merge (velokv_params.h): ranges cover [0, W) in order, none is empty, they
// differ in length by at most one block, and sk_worker_of inverts sk_begin for
// every block.
#include <cstdio>
#include <map>
#include <random>
#include <utility>
#include <vector>

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

// The kernel's walk over a worker's unit range and the merge's choice of
// workers per segment, on segments of nbs[i] blocks (0 = empty) with pen units
// ahead of each non-empty one: every block is run by exactly one worker, every
// (worker, slot) partial is written at most once, and the merge finds, for each
// split segment, exactly the partials that cover it (slot 1 of w_lo at block 0,
// slot 0 of the others, contiguous), and a direct write for the others.
static int check_pieces(const std::vector<int>& nbs, int32_t nw, int32_t pen) {
  std::vector<int64_t> seg0(nbs.size());
  int64_t C = 0;
  for (size_t i = 0; i < nbs.size(); ++i) { seg0[i] = C; C += nbs[i] > 0 ? pen + nbs[i] : 0; }
  if (C == 0) return 0;
  const SkSplit sp = sk_split(C, nw);
  struct Part { int seg, lo, hi; };
  std::map<std::pair<int, int>, Part> parts;
  std::vector<int> direct(nbs.size(), 0);
  std::vector<int> covered(nbs.size(), 0);
  for (int32_t w = 0; w < sp.nw; ++w) {
    const int64_t c0 = sk_begin(sp, w), c1 = sk_begin(sp, w + 1);
    // the kernel's loop: from the segment holding c0, one segment at a time
    size_t i = 0;
    while (i < nbs.size() && (nbs[i] == 0 || seg0[i] + pen + nbs[i] <= c0)) ++i;
    for (int64_t x = c0; x < c1 && i < nbs.size(); ++i) {
      if (nbs[i] == 0) continue;
      int32_t lo, hi;
      sk_piece(seg0[i], nbs[i], pen, x, c1, &lo, &hi);
      if (lo < hi) {
        covered[i] += hi - lo;
        if (lo == 0 && hi == nbs[i]) { direct[i] = 1; }
        else {
          const int slot = lo > 0 ? 0 : 1;
          if (!parts.emplace(std::make_pair(w, slot), Part{(int)i, lo, hi}).second) {
            printf("pieces: slot (%d,%d) written twice (nw=%d pen=%d)\n", w, slot, nw, pen);
            return 1;
          }
        }
      }
      x = seg0[i] + pen + nbs[i];
    }
  }
  for (size_t i = 0; i < nbs.size(); ++i) {
    if (nbs[i] == 0) continue;
    if (covered[i] != nbs[i]) { printf("pieces: segment %zu covered %d of %d\n", i, covered[i], nbs[i]); return 1; }
    int32_t wl, wh;
    sk_segment_workers(sp, seg0[i], nbs[i], pen, &wl, &wh);
    if (wl == wh) {
      if (!direct[i]) { printf("pieces: segment %zu not written directly (nw=%d pen=%d)\n", i, nw, pen); return 1; }
      continue;
    }
    int next = 0;
    for (int32_t w = wl; w <= wh; ++w) {
      auto it = parts.find(std::make_pair(w, w == wl ? 1 : 0));
      if (it == parts.end() || it->second.seg != (int)i || it->second.lo != next) {
        printf("pieces: segment %zu worker %d partial missing or out of order (nw=%d pen=%d)\n", i, w, nw, pen);
        return 1;
      }
      next = it->second.hi;
    }
    if (next != nbs[i]) { printf("pieces: segment %zu partials end at %d of %d\n", i, next, nbs[i]); return 1; }
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
  for (int i = 0; i < 2000 && !bad; ++i) {
    const int n = 1 + (int)(rng() % 70);
    std::vector<int> nbs(n);
    for (auto& v : nbs) {
      const int k = (int)(rng() % 6);
      v = k == 0 ? 0 : k == 1 ? 1 : k == 2 ? 2 : k == 3 ? 17 : (int)(rng() % 700);
    }
    const int32_t nws[] = {1, 3, 64, 300, 2048};
    const int32_t pens[] = {0, 1, 4, 8, 50};
    bad |= check_pieces(nbs, nws[rng() % 5], pens[rng() % 5]);
  }
  bad |= check_pieces(std::vector<int>(512, 276), 2048, 4);  // config-3-like
  printf(bad ? "FAILED\n" : "ok\n");
  return bad;
}
