// Instantiations of one band-pass kernel family for one gradient type, in a translation unit of
// its own so the families compile in parallel.  Built once per combination with
//   -DCAME8_BAND_TYPE=F32|BF16|F16  -DCAME8_BAND_PASS=1|2
// and linked into libcame8.so beside came8.hip, which calls the selector defined here.
#include "came8_dispatch.h"
#include "came8_kernels.h"

#if !defined(CAME8_BAND_TYPE) || !defined(CAME8_BAND_PASS)
#error "build with -DCAME8_BAND_TYPE=<F32|BF16|F16> -DCAME8_BAND_PASS=<1|2>"
#endif

namespace came8 {

namespace {
using TG = CAME8_BAND_TYPE;
constexpr int kVW = 16 / int(sizeof(TG::storage));  // elements per 16-byte chunk

// st: pass 2 with fp32 states; pass 1 without the column sums of g^2/R_i (k_fact_pass1n, which also
// has the MS variants)
template <int V, int K, int TPB, bool UA = false, bool MS = false>
BandFn pick(int st) {
  if constexpr (CAME8_BAND_PASS == 2)
    return st ? k_fact_pass2<TG, V, K, TPB, true, UA, MS> : k_fact_pass2<TG, V, K, TPB, false, UA, MS>;
  else if constexpr (MS) return st ? k_fact_pass1n<TG, V, K, TPB, UA, true> : nullptr;
  else return st ? k_fact_pass1n<TG, V, K, TPB, UA> : k_fact_pass1<TG, V, K, TPB, UA>;
}
template <int V, int K, int TPB>
BandFn pick_ua(int st, int ua) {
  return ua ? pick<V, K, TPB, true>(st) : pick<V, K, TPB, false>(st);
}
}  // namespace

// the (V, K, TPB) variants the host's band_variant() can choose; st selects fp32 states (pass 2) or the
// default clip mode's pass 1, ua the variants for rows of any length and alignment, ms the variants for
// rows wider than their sweep (pass 2, and pass 1 with st)
BandFn CAME8_BAND_SELECTOR(CAME8_BAND_TYPE, CAME8_BAND_PASS)(int V, int K, int TPB, int st, int ua, int ms) {
  if (ms) {
    if (V == 1 && K == 32 && TPB == 256 && !ua) return pick<1, 32, 256, false, true>(st);
    if (V == kVW && K == 3 && TPB == 256 && !ua) return pick<kVW, 3, 256, false, true>(st);
    return nullptr;
  }
  if (V == 1 && TPB == 256 && !ua) {
    switch (K) {
      case 1: return pick<1, 1, 256>(st);
      case 2: return pick<1, 2, 256>(st);
      case 4: return pick<1, 4, 256>(st);
      case 8: return pick<1, 8, 256>(st);
      case 16: return pick<1, 16, 256>(st);
      case 32: return pick<1, 32, 256>(st);
      default: return nullptr;
    }
  }
  if (V == kVW) {
    if (TPB == 128 && K == 1) return pick_ua<kVW, 1, 128>(st, ua);
    if (TPB == 128 && K == 2) return pick_ua<kVW, 2, 128>(st, ua);
    if (TPB == 256 && K == 1) return pick_ua<kVW, 1, 256>(st, ua);
    if (TPB == 256 && K == 2) return pick_ua<kVW, 2, 256>(st, ua);
    if (TPB == 256 && K == 3) return pick_ua<kVW, 3, 256>(st, ua);
    if (TPB == 512 && K == 2) return pick_ua<kVW, 2, 512>(st, ua);
    if (TPB == 512 && K == 3) return pick_ua<kVW, 3, 512>(st, ua);
    if (TPB == 512 && K == 4) return pick_ua<kVW, 4, 512>(st, ua);
  }
  return nullptr;
}

}  // namespace came8
