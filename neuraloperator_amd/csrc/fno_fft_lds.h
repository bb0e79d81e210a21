// In-register / LDS-exchanged line FFTs for power-of-two lines of 64, 128 and
// 256 complex points, used by the fused 2D kernels.
//
// A line of N points is owned by a group of T consecutive lanes of one
// wavefront (T = 16 for N = 256, else 8).  Lane t holds v[s] = x[t + T*s],
// s < R = N/T.  The transform is the four-step split N = T*R:
//   1. R-point DFT over s in registers               -> F[k1], k1 < R
//   2. twiddle F[k1] *= w_N^(t*k1)
//   3. exchange through the group's LDS slice (XOR swizzle, no padding,
//      bank-conflict free) so that a lane holds, for its k1, all t
//   4. T-point DFT over t in registers              -> X[k1 + R*k2], k2 < T
// Each lane ends with Q = R/T second-pass results: out[q][k2] = X[k1 + R*k2]
// for k1 = lane + T*q.
//
// The group's lanes exchange data through LDS without a block barrier: they
// sit in one wavefront, LDS instructions of a wavefront execute in order, and
// wave_sync() keeps the compiler from moving LDS accesses across it.
#pragma once

#include "fno_common.h"

namespace fno {

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int N>
struct LinePlan {
  static_assert(N == 64 || N == 128 || N == 256, "line length must be 64, 128 or 256");
  static constexpr int T = (N >= 256) ? 16 : 8;  // lanes per line
  static constexpr int R = N / T;                 // points per lane, first pass
  static constexpr int Q = R / T;                 // second-pass DFTs per lane
};

// exp(SIGN * 2 pi i k / 16), k in [0, 16)
template <int SIGN>
__device__ __forceinline__ float2 w16(int k) {
  constexpr float c1 = 0.92387953251128675613f;  // cos(pi/8)
  constexpr float s1 = 0.38268343236508977173f;  // sin(pi/8)
  constexpr float r2 = 0.70710678118654752440f;  // cos(pi/4)
  float c, s;
  switch (k & 15) {
    case 0: c = 1.f; s = 0.f; break;
    case 1: c = c1; s = s1; break;
    case 2: c = r2; s = r2; break;
    case 3: c = s1; s = c1; break;
    case 4: c = 0.f; s = 1.f; break;
    case 5: c = -s1; s = c1; break;
    case 6: c = -r2; s = r2; break;
    case 7: c = -c1; s = s1; break;
    case 8: c = -1.f; s = 0.f; break;
    case 9: c = -c1; s = -s1; break;
    case 10: c = -r2; s = -r2; break;
    case 11: c = -s1; s = -c1; break;
    case 12: c = 0.f; s = -1.f; break;
    case 13: c = s1; s = -c1; break;
    case 14: c = r2; s = -r2; break;
    default: c = c1; s = -s1; break;
  }
  return make_float2(c, SIGN > 0 ? s : -s);
}

// multiply by SIGN*i
template <int SIGN>
__device__ __forceinline__ float2 mul_i(float2 a) {
  return SIGN > 0 ? make_float2(-a.y, a.x) : make_float2(a.y, -a.x);
}

template <int SIGN>
__device__ __forceinline__ void dft4(float2& a, float2& b, float2& c, float2& d) {
  const float2 t0 = cadd(a, c), t1 = csub(a, c), t2 = cadd(b, d), t3 = mul_i<SIGN>(csub(b, d));
  a = cadd(t0, t2);
  c = csub(t0, t2);
  b = cadd(t1, t3);
  d = csub(t1, t3);
}

// In-place 8-point DFT, natural order in and out.
template <int SIGN>
__device__ __forceinline__ void dft8(float2 (&v)[8]) {
  // n = n1 + 2 n2: 4-point DFTs over n2 for n1 = 0, 1
  float2 e0 = v[0], e1 = v[2], e2 = v[4], e3 = v[6];
  float2 o0 = v[1], o1 = v[3], o2 = v[5], o3 = v[7];
  dft4<SIGN>(e0, e1, e2, e3);
  dft4<SIGN>(o0, o1, o2, o3);
  // twiddle w8^(k1) on the odd branch
  o1 = cmul(o1, w16<SIGN>(2));
  o2 = mul_i<SIGN>(o2);
  o3 = cmul(o3, w16<SIGN>(6));
  v[0] = cadd(e0, o0);
  v[4] = csub(e0, o0);
  v[1] = cadd(e1, o1);
  v[5] = csub(e1, o1);
  v[2] = cadd(e2, o2);
  v[6] = csub(e2, o2);
  v[3] = cadd(e3, o3);
  v[7] = csub(e3, o3);
}

// In-place 16-point DFT, natural order in and out (4 x 4 four-step).
template <int SIGN>
__device__ __forceinline__ void dft16(float2 (&v)[16]) {
  float2 f[4][4];
#pragma unroll
  for (int n1 = 0; n1 < 4; ++n1) {
    float2 a = v[n1], b = v[n1 + 4], c = v[n1 + 8], d = v[n1 + 12];
    dft4<SIGN>(a, b, c, d);
    f[n1][0] = a;
    f[n1][1] = (n1 == 0) ? b : cmul(b, w16<SIGN>(n1));
    f[n1][2] = (n1 == 0) ? c : cmul(c, w16<SIGN>(2 * n1));
    f[n1][3] = (n1 == 0) ? d : cmul(d, w16<SIGN>(3 * n1));
  }
#pragma unroll
  for (int k1 = 0; k1 < 4; ++k1) {
    float2 a = f[0][k1], b = f[1][k1], c = f[2][k1], d = f[3][k1];
    dft4<SIGN>(a, b, c, d);
    v[k1] = a;
    v[k1 + 4] = b;
    v[k1 + 8] = c;
    v[k1 + 12] = d;
  }
}

template <int M, int SIGN>
__device__ __forceinline__ void dft_small(float2 (&v)[M]) {
  if constexpr (M == 16) dft16<SIGN>(v);
  else dft8<SIGN>(v);
}

// Line FFT.  tw[i] = exp(+2 pi i i / N) for i < N (LDS table); ex is the
// group's exchange slice of N float2 at a stride of exs float2 (1: a
// contiguous slice).  t = lane index within the group.
template <int N, int SIGN>
__device__ __forceinline__ void line_fft_strided(float2 (&v)[LinePlan<N>::R], float2* ex, int exs,
                                                 const float2* tw, int t,
                                                 float2 (&out)[LinePlan<N>::Q][LinePlan<N>::T]) {
  constexpr int T = LinePlan<N>::T, R = LinePlan<N>::R, Q = LinePlan<N>::Q;
  dft_small<R, SIGN>(v);
#pragma unroll
  for (int k1 = 1; k1 < R; ++k1) {
    const float2 w = tw[t * k1];
    v[k1] = SIGN > 0 ? cmul(v[k1], w) : cmulc(v[k1], w);
  }
  wave_sync();
#pragma unroll
  for (int k1 = 0; k1 < R; ++k1) ex[(k1 * T + (t ^ (k1 & (T - 1)))) * exs] = v[k1];
  wave_sync();
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int k1 = t + T * q;
    float2 u[T];
#pragma unroll
    for (int s = 0; s < T; ++s) u[s] = ex[(k1 * T + (s ^ t)) * exs];
    dft_small<T, SIGN>(u);
#pragma unroll
    for (int s = 0; s < T; ++s) out[q][s] = u[s];
  }
  wave_sync();
}

template <int N, int SIGN>
__device__ __forceinline__ void line_fft(float2 (&v)[LinePlan<N>::R], float2* ex, const float2* tw,
                                         int t,
                                         float2 (&out)[LinePlan<N>::Q][LinePlan<N>::T]) {
  line_fft_strided<N, SIGN>(v, ex, 1, tw, t, out);
}

}  // namespace fno
