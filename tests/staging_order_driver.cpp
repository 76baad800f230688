// Host-side check of the staged kernel's A staging order
// (StagedGemm::a_item in tensorforge_amd/csrc/staged_gemm.hpp), compiled with
// hipcc for the host only by tests/test_staging_order.py.  For each
// configuration: every (row, column vector) of the BM x BK slab is staged by
// exactly one index q; every 8 consecutive indices (one 8-lane pass of a
// 128-bit LDS write) hit 8 distinct 4-bank groups of the padded A tile; and
// the 64 indices of one wave instruction cover whole rows of the slab, so the
// global loads read whole row segments.  Prints one line per configuration
// and "ok" when all pass; exits 1 on the first failure.
#include <cstdio>
#include <set>
#include <utility>

#include "staged_gemm.hpp"

template <int BM, int BN, int TM, int TN, int BK>
static bool check() {
  using G = tfk::StagedGemm<BM, BN, TM, TN, BK, 1, 1>;
  constexpr int CPR = BK / 4, N = G::A_VECS;
  std::set<std::pair<int, int>> seen;
  int conflicts = 0;
  for (int q = 0; q < N; ++q) {
    int r, c;
    G::a_item(q, r, c);
    if (r < 0 || r >= BM || c < 0 || c >= BK || c % 4 != 0 || !seen.insert({r, c}).second) {
      std::printf("b%dx%d t%dx%d k%d: index %d -> (%d, %d) out of the slab or repeated\n", BM, BN, TM, TN, BK, q, r, c);
      return false;
    }
  }
  for (int p0 = 0; p0 < N; p0 += 8) {
    std::set<int> groups;
    for (int q = p0; q < p0 + 8; ++q) {
      int r, c;
      G::a_item(q, r, c);
      groups.insert(((r * G::LDA + c) / 4) % 8);
    }
    conflicts += 8 - (int)groups.size();
  }
  for (int w0 = 0; w0 < N; w0 += 64) {
    std::set<int> rows;
    std::set<std::pair<int, int>> items;
    for (int q = w0; q < w0 + 64 && q < N; ++q) {
      int r, c;
      G::a_item(q, r, c);
      rows.insert(r);
      items.insert({r, c});
    }
    if (CPR <= 64 && items.size() != rows.size() * CPR) {
      std::printf("b%dx%d t%dx%d k%d: wave at %d covers partial rows\n", BM, BN, TM, TN, BK, w0);
      return false;
    }
  }
  std::printf("b%dx%d t%dx%d k%d (LDA %d): %d staging vectors, %d bank-group collisions\n", BM, BN, TM, TN, BK,
              G::LDA, N, conflicts);
  return conflicts == 0;
}

int main() {
  const bool ok = check<128, 128, 8, 8, 16>() && check<128, 128, 8, 4, 16>() && check<128, 64, 8, 4, 16>() &&
                  check<64, 64, 4, 4, 16>() && check<64, 64, 2, 2, 16>() && check<64, 128, 4, 4, 16>() &&
                  check<128, 128, 8, 4, 8>() && check<64, 64, 4, 4, 8>() && check<32, 32, 4, 4, 8>() &&
                  check<128, 128, 8, 4, 32>() && check<64, 64, 2, 2, 32>() && check<256, 128, 8, 8, 32>() &&
                  check<128, 128, 4, 4, 64>() && check<64, 64, 2, 2, 64>() && check<128, 256, 8, 4, 32>();
  std::printf(ok ? "ok\n" : "FAILED\n");
  return ok ? 0 : 1;
}
