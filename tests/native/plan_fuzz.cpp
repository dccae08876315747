// Randomised driver for aegkv_transfer_entries (aegaeon_amd/csrc/plan.cpp),
// built with AddressSanitizer and UndefinedBehaviorSanitizer by
// tests/test_native_sanitized.py. Checks every call stays inside its
// arrays, that rows reference live columns in table / group / column order,
// that extents stay inside the page, and that a too-small row buffer is
// rejected with AEGKV_ENOMEM and the exact row count.

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#include "aegkv.h"

// The library's error helpers live in aegkv.hip; this host-only build
// provides its own.
int aegkv_set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  va_end(ap);
  return code;
}
void aegkv_clear_error() {}

#define CHECK(c)                                                         \
  do {                                                                   \
    if (!(c)) {                                                          \
      std::fprintf(stderr, "check failed at line %d: %s\n", __LINE__, #c); \
      return 1;                                                          \
    }                                                                    \
  } while (0)

int main(int argc, char** argv) {
  const int iters = argc > 1 ? std::atoi(argv[1]) : 20000;
  std::mt19937_64 rng(12345);
  auto rnd = [&](int64_t lo, int64_t hi) {  // inclusive
    return std::uniform_int_distribution<int64_t>(lo, hi)(rng);
  };
  for (int it = 0; it < iters; ++it) {
    const int32_t G = static_cast<int32_t>(rnd(1, 4));
    std::vector<int32_t> kind(G);
    std::vector<int64_t> bs(G), kbs(G), win(G);
    for (int g = 0; g < G; ++g) {
      kind[g] = rnd(0, 3) == 0 ? 1 : 0;
      kbs[g] = rnd(1, 32);
      bs[g] = kind[g] ? kbs[g] : kbs[g] * rnd(1, 8);
      win[g] = kind[g] ? 0 : (rnd(0, 2) ? rnd(1, 300) : 0);
    }
    const int64_t T = rnd(0, 6);
    std::vector<int64_t> tokens(T), offsets(T * G + 1, 0), ids;
    for (int64_t t = 0; t < T; ++t) {
      tokens[t] = rnd(0, 2000);
      for (int g = 0; g < G; ++g) {
        const int64_t n = kind[g] ? 1 : (tokens[t] + bs[g] - 1) / bs[g] + rnd(0, 1);
        for (int64_t c = 0; c < n; ++c) ids.push_back(rnd(0, 4) == 0 ? -1 : rnd(0, 1 << 20));
        offsets[t * G + g + 1] = static_cast<int64_t>(ids.size());
      }
    }
    if (ids.empty()) ids.push_back(0);  // keep the pointer valid
    const int64_t cap = static_cast<int64_t>(ids.size());
    std::vector<int64_t> o_tab(cap), o_col(cap), o_blk(cap), o_first(cap), o_cnt(cap);
    std::vector<int32_t> o_grp(cap);
    int64_t rows = -1;
    int rc = aegkv_transfer_entries(G, kind.data(), bs.data(), kbs.data(), win.data(), T,
                                    tokens.data(), offsets.data(), ids.data(), cap, o_tab.data(),
                                    o_grp.data(), o_col.data(), o_blk.data(), o_first.data(),
                                    o_cnt.data(), &rows);
    CHECK(rc == AEGKV_OK);
    CHECK(rows >= 0 && rows <= cap);
    int64_t prev = -1;
    for (int64_t r = 0; r < rows; ++r) {
      const int64_t t = o_tab[r], g = o_grp[r], c = o_col[r];
      CHECK(t >= 0 && t < T && g >= 0 && g < G);
      const int64_t lo = offsets[t * G + g], hi = offsets[t * G + g + 1];
      CHECK(c >= 0 && c < hi - lo);
      CHECK(ids[lo + c] == o_blk[r] && o_blk[r] != -1);
      const int64_t key = (t * G + g) * (int64_t(1) << 32) + c;
      CHECK(key > prev);
      prev = key;
      const int64_t kpp = bs[g] / kbs[g];
      CHECK(o_first[r] >= 0 && o_cnt[r] >= 0 && o_first[r] + o_cnt[r] <= kpp);
    }
    if (rows > 0) {  // one row short of what is needed
      int64_t rows2 = -1;
      std::vector<int64_t> s_tab(rows), s_col(rows), s_blk(rows), s_first(rows), s_cnt(rows);
      std::vector<int32_t> s_grp(rows);
      rc = aegkv_transfer_entries(G, kind.data(), bs.data(), kbs.data(), win.data(), T,
                                  tokens.data(), offsets.data(), ids.data(), rows - 1,
                                  s_tab.data(), s_grp.data(), s_col.data(), s_blk.data(),
                                  s_first.data(), s_cnt.data(), &rows2);
      CHECK(rc == AEGKV_ENOMEM);
    }
  }
  std::printf("plan_fuzz: %d iterations clean\n", iters);
  return 0;
}
