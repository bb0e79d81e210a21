// Twiddle factors exp(+2 pi i k / N).
#pragma once

#include "fno_common.h"

namespace fno {

// exp(+2 pi i k / 1024), k < 1024, evaluated at compile time in double
// precision (octant reduction + Taylor series to x^23, error << 1e-16) and
// rounded once to float, so every twiddle is within half an ulp.
namespace twd {
constexpr double kPi = 3.14159265358979323846264338327950288;
constexpr double sin_series(double x) {  // |x| <= pi/4
  double x2 = x * x, term = x, sum = x;
  for (int n = 1; n < 12; ++n) {
    term *= -x2 / ((2.0 * n) * (2.0 * n + 1.0));
    sum += term;
  }
  return sum;
}
constexpr double cos_series(double x) {
  double x2 = x * x, term = 1.0, sum = 1.0;
  for (int n = 1; n < 12; ++n) {
    term *= -x2 / ((2.0 * n - 1.0) * (2.0 * n));
    sum += term;
  }
  return sum;
}
constexpr int kN = 1024;
struct Table {
  float re[kN], im[kN];
};
constexpr Table make_table() {
  Table t{};
  for (int k = 0; k < kN; ++k) {
    const int q = k / (kN / 4), m = k % (kN / 4);   // quadrant, position in it
    double c = 0, sn = 0;
    if (m <= kN / 8) {
      c = cos_series(2.0 * kPi * m / kN);
      sn = sin_series(2.0 * kPi * m / kN);
    } else {
      c = sin_series(2.0 * kPi * (kN / 4 - m) / kN);
      sn = cos_series(2.0 * kPi * (kN / 4 - m) / kN);
    }
    double cr = c, sr = sn;
    if (q == 1) { cr = -sn; sr = c; }
    else if (q == 2) { cr = -c; sr = -sn; }
    else if (q == 3) { cr = sn; sr = -c; }
    t.re[k] = (float)cr;
    t.im[k] = (float)sr;
  }
  return t;
}
}  // namespace twd
// one copy per translation unit (internal linkage): device code is not
// relocatable across units
static __constant__ const twd::Table kTw = twd::make_table();

// LDS table of exp(+2 pi i t / N), t < N, for N dividing 1024
template <int N>
__device__ __forceinline__ void fill_twiddles(float2* tw) {
  static_assert(twd::kN % N == 0, "N must divide 1024");
  for (int i = threadIdx.x; i < N; i += blockDim.x)
    tw[i] = make_float2(kTw.re[i * (twd::kN / N)], kTw.im[i * (twd::kN / N)]);
}

// exp(+2 pi i t / n) for 0 <= t < n: the table entry when n divides 1024 (the
// same correctly rounded value), else evaluated in double precision.
__device__ __forceinline__ float2 twiddle_any(int t, int n) {
  if (twd::kN % n == 0) {
    const int i = t * (twd::kN / n);
    return make_float2(kTw.re[i], kTw.im[i]);
  }
  return twiddle_pos(t, n);
}

}  // namespace fno
