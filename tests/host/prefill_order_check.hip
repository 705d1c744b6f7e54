// Host-side check of the chunked prefill's dispatch order (dispatch_slot in
// prefill_mfma.hip), compiled from the kernel source and run on the CPU (no
// GPU call). Over random XCD sizes, query-tile counts and CU counts: the
// order is a permutation of the XCD's positions that keeps every item in its
// round of one workgroup per CU (so each round reads the same kv heads as in
// the natural order) and maps positions past the valid items to themselves;
// where it reorders, a round dispatches its query tiles heaviest first.
#include "prefill_mfma.hip"

#include <cstdio>
#include <random>
#include <vector>

// The file's host launcher references this; nothing here launches.
namespace clv {
hipError_t launch_prefill_valu(const PrefillParams &, DType, hipStream_t) {
  return hipErrorInvalidValue;
}
}  // namespace clv

int main() {
  std::mt19937_64 rng(7);
  long cases = 0, reordered = 0, bad = 0;
  for (int it = 0; it < 100000; ++it) {
    const int n_q = 1 + (int)(rng() % 24);
    const int cus = (it % 4 == 0) ? 0 : 1 + (int)(rng() % 40);
    const int per_xcd = (it % 2 ? n_q * (1 + (int)(rng() % 12)) : 1 + (int)(rng() % 300));
    const int valid = (int)(rng() % (per_xcd + 3));
    std::vector<int> seen(per_xcd, 0);
    bool ok = true, moved = false;
    for (int i = 0; i < per_xcd && ok; ++i) {
      const int j = clv::dispatch_slot(i, per_xcd, valid, n_q, cus);
      if (j < 0 || j >= per_xcd || seen[j]++) ok = false;
      else if (i >= valid && j != i) ok = false;
      else if (cus > 0 && j / cus != i / cus) ok = false;
      if (j != i) moved = true;
    }
    if (ok && moved) {
      // In a reordered round, weights (n_q - 1 - item % n_q: the query tile)
      // never rise along the dispatch order.
      const int nv = valid < per_xcd ? valid : per_xcd;
      for (int r0 = cus; r0 < nv && ok; r0 += cus) {
        const int r1 = r0 + cus < nv ? r0 + cus : nv;
        bool round_moved = false;
        for (int i = r0; i < r1; ++i)
          if (clv::dispatch_slot(i, per_xcd, valid, n_q, cus) != i) round_moved = true;
        if (!round_moved) continue;
        int prev = n_q;
        for (int i = r0; i < r1; ++i) {
          const int qt = n_q - 1 - clv::dispatch_slot(i, per_xcd, valid, n_q, cus) % n_q;
          if (qt > prev) ok = false;
          prev = qt;
        }
      }
      ++reordered;
    }
    ++cases;
    if (!ok) {
      if (bad < 5) printf("bad: n_q %d cus %d per_xcd %d valid %d\n", n_q, cus, per_xcd, valid);
      ++bad;
    }
  }
  // The 8 x (4096 + 512) shape on 32 CUs per XCD: 64 items per XCD, 8 tiles
  // per kv head; the second round goes 7,7,7,7,6,6,6,6,...
  for (int i = 32; i < 64; ++i) {
    const int qt = 7 - clv::dispatch_slot(i, 64, 64, 8, 32) % 8;
    if (qt != 7 - (i - 32) / 4) ++bad;
  }
  printf("cases %ld reordered %ld bad %ld\n", cases, reordered, bad);
  return bad != 0;
}
