// Band-pass kernel selectors shared by came8.hip and the per-family translation units
// (came8_band.hip, one build per gradient type and pass).
#pragma once

#include "came8_kernels.h"

namespace came8 {

using BandFn = void (*)(const DevTensor*, const int32_t*, const int64_t*, int, Hp);

#define CAME8_BAND_SELECTOR_(T, P) band_fn_##T##_p##P
#define CAME8_BAND_SELECTOR(T, P) CAME8_BAND_SELECTOR_(T, P)

// kernel for (V, K, TPB), for pass 2 the state kind (st: fp32 states), and ua (rows of any length and
// alignment, V > 1 only), or nullptr for a combination that is not built
BandFn band_fn_F32_p1(int V, int K, int TPB, int st, int ua, int ms);
BandFn band_fn_F32_p2(int V, int K, int TPB, int st, int ua, int ms);
BandFn band_fn_BF16_p1(int V, int K, int TPB, int st, int ua, int ms);
BandFn band_fn_BF16_p2(int V, int K, int TPB, int st, int ua, int ms);
BandFn band_fn_F16_p1(int V, int K, int TPB, int st, int ua, int ms);
BandFn band_fn_F16_p2(int V, int K, int TPB, int st, int ua, int ms);

}  // namespace came8
