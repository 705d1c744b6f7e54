// Host-side check of the balanced decode's step split (StreamSplit in
// decode_stream.hip), compiled from the kernel source itself and run on the
// CPU (no GPU call): over random group counts, step counts, dispatch-slot
// counts 1-4 and slot weights 0.5-2, every group owns a non-empty span, the
// spans are consecutive and cover [0, N), and owner() inverts start(). The
// merge locates each segment's partials through owner(), and the partial
// slots are distinct only while every group owns at least one step. The
// 32-bit form of the split's arithmetic (W * N below 2^32) agrees with the
// 64-bit one.
#include "decode_stream.hip"

#include <algorithm>
#include <cstdio>
#include <random>

// The file's host launchers reference this; nothing here launches.
namespace clv {
bool decode_mfma_supported(DType, int, int) { return false; }
}  // namespace clv

int main() {
  std::mt19937_64 rng(1);
  long cases = 0, bad = 0;
  for (int it = 0; it < 200000; ++it) {
    clv::DecodeParams p{};
    const int cus = 1 + (int)(rng() % 300);
    const int hg = 1 << (rng() % 3);
    const int slots = 1 + (int)(rng() % 4);
    p.slot_count = slots;
    p.slot_groups = 4 * cus / hg;
    for (int k = 0; k < 4; ++k) p.slot_q8[k] = 128 + (int)(rng() % 385);
    const int64_t w_full = (int64_t)slots * p.slot_groups;
    // Step counts past 2^32 / W take the split's 64-bit arithmetic, the
    // others its 32-bit form, which must give the same spans.
    const int64_t n_range = it % 3 == 0 ? 4 * w_full + 2 : it % 3 == 1 ? 200000 : 0x7fffffff;
    const int64_t n = 1 + (int64_t)(rng() % n_range);
    const int64_t w_all = std::min(w_full, n);
    const clv::StreamSplit sp(p, w_all, n);
    clv::StreamSplit wide = sp;
    wide.narrow = false;
    ++cases;
    bool ok = sp.start(0) == 0 && sp.start((int)w_all) == n;
    for (int64_t w = 0; w < w_all && ok; ++w) {
      const int a = sp.start((int)w), b = sp.start((int)w + 1);
      if (!(a < b) || sp.owner(a) != w || sp.owner(b - 1) != w) ok = false;
      if (a != wide.start((int)w) || sp.owner(a) != wide.owner(a) ||
          sp.owner(b - 1) != wide.owner(b - 1))
        ok = false;
      for (int x = a + 1; ok && x < std::min(b - 1, a + 3); ++x)
        if (sp.owner(x) != w || wide.owner(x) != w) ok = false;
    }
    if (!ok) {
      if (bad < 5)
        printf("bad: cus %d hg %d slots %d W %ld N %ld\n", cus, hg, slots, (long)w_all, (long)n);
      ++bad;
    }
  }
  printf("cases %ld bad %ld\n", cases, bad);
  return bad != 0;
}
