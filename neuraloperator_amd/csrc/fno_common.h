// Shared device helpers and host-side error plumbing for the FNO spectral
// library (gfx950).  Complex numbers are interleaved float pairs (float2),
// the same memory layout as torch.complex64.
#pragma once

#include <initializer_list>
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

// erf GELU, 0.5 v (1 + erf(v / sqrt 2)) -- the torch.nn.functional.gelu
// default (not the tanh form) -- branch-free.  erf comes from Abramowitz &
// Stegun 7.1.28: for u >= 0, erf u = 1 - T(u) with
//   T(u) = (1 + a1 u + a2 u^2 + ... + a6 u^6)^-16,  |error| <= 3e-7.
// Then GELU(v) = max(v, 0) - |v| T / 2 (v - v T / 2 for v >= 0, v T / 2 for
// v < 0, as one fused multiply-add and no compare / select), so the tail for
// large negative v keeps its relative accuracy.  In float32 the result is
// within 1e-6 absolute of the exact GELU (about the rounding of a value of
// magnitude 4) at ~17 VALU slots, against ~36 for the two-branch libm erff.
__device__ __forceinline__ float gelu_erf(float v) {
  const float a = fabsf(v);
  const float u = a * 0.70710678118654752440f;
  float p = 0.0000430638f;
  p = fmaf(p, u, 0.0002765672f);
  p = fmaf(p, u, 0.0001520143f);
  p = fmaf(p, u, 0.0092705272f);
  p = fmaf(p, u, 0.0422820123f);
  p = fmaf(p, u, 0.0705230784f);
  p = fmaf(p, u, 1.0f);
  p = p * p;  // ^2
  p = p * p;  // ^4
  p = p * p;  // ^8
  p = p * p;  // ^16
  return fmaf(-0.5f * a, __builtin_amdgcn_rcpf(p), fmaxf(v, 0.f));
}

// Activation on/off without a branch: the compiler turns `on ? gelu(v) : v`
// into a uniform branch around every element's GELU, so the choice is a
// bit-select (v_bfi_b32) against a mask it cannot see through.
__device__ __forceinline__ uint32_t act_mask(bool on) {
  uint32_t m = (uint32_t)__builtin_amdgcn_readfirstlane(on ? -1 : 0);
  asm volatile("" : "+s"(m));
  return m;
}
__device__ __forceinline__ float act_select(float g, float v, uint32_t m) {
  return __builtin_bit_cast(float, (__builtin_bit_cast(uint32_t, g) & m) |
                                       (__builtin_bit_cast(uint32_t, v) & ~m));
}

// 16-byte loads / stores with the non-temporal (streaming) cache policy, for
// activations a kernel touches once (16-byte aligned addresses).
typedef float nt_v4f __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 load_nt(const float* p) {
  const nt_v4f v = __builtin_nontemporal_load(reinterpret_cast<const nt_v4f*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void store_nt(float* p, float4 v) {
  const nt_v4f w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<nt_v4f*>(p));
}

// Raw buffer resource over [base, base + bytes): loads past the end return
// zero, and offsets are 32-bit, so address arithmetic stays in 32-bit VGPRs.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// The channel MLP of an FNO layer folded into the fused 2D block's row
// epilogue (64 channels, 32 hidden):
//   y = act(W2 gelu(W1 y1 + b1) + b2 + gate(x)),  y1 = act(spectral + skip)
// gate: soft-gating g * x + gb, the identity x, or nothing.
struct LayerMlp {
  const float* w1 = nullptr;       // [32, 64]
  const float* b1 = nullptr;       // [32] or NULL
  const float* w2 = nullptr;       // [64, 32]
  const float* b2 = nullptr;       // [64] or NULL
  const float* gate_w = nullptr;   // [64] (soft-gating)
  const float* gate_b = nullptr;   // [64] or NULL
  int gate_kind = 0;               // FNO_SKIP_NONE / SOFT_GATING / IDENTITY
};

// ------------------------------------------------------------------ host side
void set_error(const char* fmt, ...);
int hip_status(hipError_t e, const char* what);
int launch_status(const char* what);

// FFT scaling for a transform direction given torch's norm= convention.
double forward_scale(int norm, const int32_t* in_sizes, int ndim);
double inverse_scale(int norm, const int32_t* out_sizes, int ndim);

// Largest element count of any operand or intermediate the entry points
// accept (2^40: 8 TiB of complex64, beyond any device), so that every byte
// and offset computed from a validated shape fits int64 and size_t.
constexpr int64_t kMaxElems = (int64_t)1 << 40;

// True when every factor is positive and their product stays within
// kMaxElems.
inline bool extent_ok(std::initializer_list<int64_t> factors) {
  int64_t e = 1;
  for (int64_t v : factors)
    if (v < 1 || __builtin_mul_overflow(e, v, &e) || e > kMaxElems) return false;
  return true;
}

// planes * prod(max(a[d], b[d])) for d < n (b may be NULL), or -1 when a
// factor is not positive or the product passes kMaxElems.
inline int64_t bounded_elems(int64_t planes, int n, const int32_t* a, const int32_t* b = nullptr) {
  if (planes < 1 || planes > kMaxElems) return -1;
  int64_t e = planes;
  for (int d = 0; d < n; ++d) {
    const int64_t f = b && b[d] > a[d] ? b[d] : a[d];
    if (f < 1 || __builtin_mul_overflow(e, f, &e) || e > kMaxElems) return -1;
  }
  return e;
}

}  // namespace fno

#define FNO_CHECK_ARG(cond, ...)         \
  do {                                   \
    if (!(cond)) {                       \
      fno::set_error(__VA_ARGS__);       \
      return FNO_ERR_INVALID;            \
    }                                    \
  } while (0)
