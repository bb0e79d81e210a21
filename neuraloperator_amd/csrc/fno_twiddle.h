// Twiddle factors exp(+2 pi i k / N).
#pragma once

#include "fno_common.h"

namespace fno {

// exp(+2 pi i k / 256), k < 256, evaluated at compile time in double
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
struct Table256 {
  float re[256], im[256];
};
constexpr Table256 make_table() {
  Table256 t{};
  for (int k = 0; k < 256; ++k) {
    const int q = k / 64, m = k % 64;   // quadrant, position in it
    double c = 0, sn = 0;
    if (m <= 32) {
      c = cos_series(2.0 * kPi * m / 256.0);
      sn = sin_series(2.0 * kPi * m / 256.0);
    } else {
      c = sin_series(2.0 * kPi * (64 - m) / 256.0);
      sn = cos_series(2.0 * kPi * (64 - m) / 256.0);
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
static __constant__ const twd::Table256 kTw256 = twd::make_table();

// LDS table of exp(+2 pi i t / N), t < N, for N dividing 256
template <int N>
__device__ __forceinline__ void fill_twiddles(float2* tw) {
  static_assert(256 % N == 0, "N must divide 256");
  for (int i = threadIdx.x; i < N; i += blockDim.x)
    tw[i] = make_float2(kTw256.re[i * (256 / N)], kTw256.im[i * (256 / N)]);
}

// exp(+2 pi i t / n) for 0 <= t < n: the table entry when n divides 256 (the
// same correctly rounded value), else evaluated in double precision.
__device__ __forceinline__ float2 twiddle_any(int t, int n) {
  if (256 % n == 0) {
    const int i = t * (256 / n);
    return make_float2(kTw256.re[i], kTw256.im[i]);
  }
  return twiddle_pos(t, n);
}

}  // namespace fno
