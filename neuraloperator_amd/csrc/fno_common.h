// Shared device helpers and host-side error plumbing for the FNO spectral
// library (gfx950).  Complex numbers are interleaved float pairs (float2),
// the same memory layout as torch.complex64.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/fno_hip.h"

namespace fno {

// ---------------------------------------------------------------- device math
__device__ __forceinline__ float2 cadd(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
__device__ __forceinline__ float2 csub(float2 a, float2 b) { return make_float2(a.x - b.x, a.y - b.y); }
__device__ __forceinline__ float2 cmul(float2 a, float2 b) {
  return make_float2(fmaf(a.x, b.x, -a.y * b.y), fmaf(a.x, b.y, a.y * b.x));
}
// a * conj(b)
__device__ __forceinline__ float2 cmulc(float2 a, float2 b) {
  return make_float2(fmaf(a.x, b.x, a.y * b.y), fmaf(a.y, b.x, -a.x * b.y));
}
// acc += a * b
__device__ __forceinline__ void cfma(float2& acc, float2 a, float2 b) {
  acc.x = fmaf(a.x, b.x, acc.x);
  acc.x = fmaf(-a.y, b.y, acc.x);
  acc.y = fmaf(a.x, b.y, acc.y);
  acc.y = fmaf(a.y, b.x, acc.y);
}
__device__ __forceinline__ float2 cscale(float2 a, float s) { return make_float2(a.x * s, a.y * s); }

// exp(+2 pi i t / n) computed in double precision and rounded once, so every
// twiddle is within half an ulp of the true value.
__device__ __forceinline__ float2 twiddle_pos(long long t, long long n) {
  long long r = t % n;
  if (r < 0) r += n;
  double s, c;
  sincospi(2.0 * (double)r / (double)n, &s, &c);
  return make_float2((float)c, (float)s);
}

// Exact erf GELU: 0.5 x (1 + erf(x / sqrt 2)), the torch.nn.functional.gelu
// default.  erff is the device libm erf.
__device__ __forceinline__ float gelu_erf(float x) {
  return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f));
}

// ------------------------------------------------------------------ host side
void set_error(const char* fmt, ...);
int hip_status(hipError_t e, const char* what);
int launch_status(const char* what);

// FFT scaling for a transform direction given torch's norm= convention.
double forward_scale(int norm, const int32_t* in_sizes, int ndim);
double inverse_scale(int norm, const int32_t* out_sizes, int ndim);

}  // namespace fno

#define FNO_CHECK_ARG(cond, ...)         \
  do {                                   \
    if (!(cond)) {                       \
      fno::set_error(__VA_ARGS__);       \
      return FNO_ERR_INVALID;            \
    }                                    \
  } while (0)
