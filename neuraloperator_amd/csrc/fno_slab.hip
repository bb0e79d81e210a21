// Forward window transform of the last two axes of 64 x 64 slabs in one pass:
//
//   X[k1, k2] = s sum_{d1, d2} x[d1, d2] e^{-2 pi i ((k1 - m1/2) d1 + k2 d2) / 64},
//               k1 < m1 <= 16 (window rows of the next-to-last axis, centred),
//               k2 < m2h <= 16 (rfft bins of the last axis),
//
// the first two stages of the window transform (torch.fft.rfftn + fftshift +
// window slice over those two axes, neuralop/layers/spectral_convolution.py
// :443-449, :500-521), so the last-axis spectrum of the whole field never
// goes through memory.  One wave per slab, two products on
// v_mfma_f32_16x16x32_bf16 (three-term bf16 splits, fp32 accumulation):
//   1. A1[d1, c] = sum_d2 x[d1, d2] F[d2, c]: columns c < 16 the real parts
//      (cos) of bins c, columns 16 + c the imaginary parts (-sin), so a
//      lane's two column tiles hold Re and Im of the same bin;
//   2. [Xr; Xi][k1, k2] = sum over (d1, part) of A2 . A1: the accumulators
//      of step 1 are the B operand as they stand, K slot (G, i) of k-step ks
//      being row d1 = 16 ks + 4 G + i % 4 of part i / 4 (Re / Im), and A2 the
//      window's twiddles (cos / sin) in that slot order, scaled by s.
// The twiddle fragments of both products are built once per workgroup in LDS.
#include "fno_common.h"
#include "fno_fft_lds.h"
#include "fno_twiddle.h"

namespace fno {

namespace sl {
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kN = 64, kWaves = 4, kThreads = 64 * kWaves;
struct bf2 {
  __bf16 hi, lo;
};
__device__ __forceinline__ bf2 split(float v) {
  const __bf16 h = (__bf16)v;
  return {h, (__bf16)(v - (float)h)};
}
__device__ __forceinline__ v4f mma3(v8bf ah, v8bf al, v8bf bh, v8bf bl, v4f acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc, 0, 0, 0);
}
}  // namespace sl

__global__ void __launch_bounds__(sl::kThreads)
k_slab_fwd64(const float* __restrict__ x, float2* __restrict__ out, int64_t slabs, int m1,
             int m2h, float scale) {
  using namespace sl;
  // F fragments [ks 2][nt 2][hi|lo][64]; A2 fragments [rt 2][ks 4][hi|lo][64]
  __shared__ v8bf ff[2 * 2 * 2 * 64];
  __shared__ v8bf af[2 * 4 * 2 * 64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int G = lane >> 4, n = lane & 15;
  for (int f = tid; f < 2 * 2 * 64; f += kThreads) {
    const int ln = f & 63, nt = (f >> 6) & 1, ks = f >> 7;
    const int c = ln & 15, g = ln >> 4;
    v8bf h, l;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int d2 = 32 * ks + 8 * g + i;
      float v = 0.f;
      if (c < m2h) {
        const float2 t = twiddle_any((c * d2) & (kN - 1), kN);
        v = nt ? -t.y : t.x;
      }
      const bf2 q = split(v);
      h[i] = q.hi;
      l[i] = q.lo;
    }
    ff[((ks * 2 + nt) * 2) * 64 + ln] = h;
    ff[((ks * 2 + nt) * 2 + 1) * 64 + ln] = l;
  }
  for (int f = tid; f < 2 * 4 * 64; f += kThreads) {
    const int ln = f & 63, ks = (f >> 6) & 3, rt = f >> 8;
    const int k1 = ln & 15, g = ln >> 4;
    v8bf h, l;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int d1 = 16 * ks + 4 * g + (i & 3), part = i >> 2;
      float v = 0.f;
      if (k1 < m1) {
        // e^{-i theta} (a + i b): Re = cos a + sin b, Im = cos b - sin a
        const int f1 = k1 - m1 / 2;
        const float2 t = twiddle_any(((f1 * d1) % kN + kN) % kN, kN);
        v = rt == 0 ? (part == 0 ? t.x : t.y) : (part == 0 ? -t.y : t.x);
        v *= scale;
      }
      const bf2 q = split(v);
      h[i] = q.hi;
      l[i] = q.lo;
    }
    af[((rt * 4 + ks) * 2) * 64 + ln] = h;
    af[((rt * 4 + ks) * 2 + 1) * 64 + ln] = l;
  }
  __syncthreads();

  const int64_t nwaves = (int64_t)gridDim.x * kWaves;
  // rows 16 mt + m of a slab, columns 32 ks + 8 G .. + 7.  Rolling
  // prefetch: as soon as step 1 has issued the products of row tile mt, that
  // tile's registers are loaded with the next slab's rows, so those loads are
  // in flight during the rest of step 1, step 2 and the store
  float4 xv[4][2][2];
  auto load = [&](int64_t sl, int mt) __attribute__((always_inline)) {
    const float* xs = x + sl * (kN * kN);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const float* p = xs + (16 * mt + n) * kN + 32 * ks + 8 * G;
      xv[mt][ks][0] = load_nt(p);
      xv[mt][ks][1] = load_nt(p + 4);
    }
  };
  int64_t s = (int64_t)blockIdx.x * kWaves + (tid >> 6);
  if (s < slabs) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) load(s, mt);
  }
#pragma unroll 1
  for (; s < slabs; s += nwaves) {
    const bool more = s + nwaves < slabs;
    v4f a1[4][2];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      a1[mt][0] = (v4f)0.f;
      a1[mt][1] = (v4f)0.f;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const float v[8] = {xv[mt][ks][0].x, xv[mt][ks][0].y, xv[mt][ks][0].z, xv[mt][ks][0].w,
                            xv[mt][ks][1].x, xv[mt][ks][1].y, xv[mt][ks][1].z, xv[mt][ks][1].w};
        v8bf ah, al;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const bf2 q = split(v[i]);
          ah[i] = q.hi;
          al[i] = q.lo;
        }
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
          a1[mt][nt] = mma3(ah, al, ff[((ks * 2 + nt) * 2) * 64 + lane],
                            ff[((ks * 2 + nt) * 2 + 1) * 64 + lane], a1[mt][nt]);
      }
      if (more) load(s + nwaves, mt);
    }
    // step 2: k-step ks of the window product is row tile ks of step 1
    v4f a2[2] = {(v4f)0.f, (v4f)0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      v8bf bh, bl;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const bf2 q = split(a1[ks][i >> 2][i & 3]);
        bh[i] = q.hi;
        bl[i] = q.lo;
      }
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
        a2[rt] = mma3(af[((rt * 4 + ks) * 2) * 64 + lane], af[((rt * 4 + ks) * 2 + 1) * 64 + lane],
                      bh, bl, a2[rt]);
    }
    // row k1 = 4 G + r, column k2 = n of both tiles
    float2* os = out + s * m1 * m2h;
    if (n < m2h) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int k1 = 4 * G + r;
        if (k1 < m1) os[k1 * m2h + n] = make_float2(a2[0][r], a2[1][r]);
      }
    }
  }
}

// ----------------------------------------------------------------------------
// Inverse along one 64-point axis from a window of m <= 16 rows (frequency
// j - m/2 at window row j), for inner <= 16 columns:
//
//   Z[s, d, c] = t sum_{j < m} U[s, j, c] e^{2 pi i (j - m/2) d / 64}
//
// (an ifftn axis of SpectralConv.forward's inverse, spectral_convolution.py
// :547-548, zero-padded window to the full axis).  One wave per slab s as one
// product on the matrix cores: rows (d, Re | Im) in row tiles (16 d, part),
// K = (j, Re | Im of U) against the constant twiddle fragments, columns c.
// Three-term bf16 splits, fp32 accumulation.
__global__ void __launch_bounds__(sl::kThreads)
k_axis_inv64(const float2* __restrict__ src, float2* __restrict__ dst, int64_t slabs, int m,
             int inner, float scale) {
  using namespace sl;
  // A fragments [row tile 8][hi|lo][64]: row tile rt = 2 t + part, rows
  // d = 16 t + lane % 16; K slot (G, i) = window row 4 G + i / 2, Re / Im of U
  __shared__ v8bf af[8 * 2 * 64];
  // per wave: the slab's [64][inner] output, staged so it leaves as whole
  // 16-byte words of one contiguous run (64 inner 8 bytes per slab)
  extern __shared__ float4 stage[];   // [kWaves][32 inner]
  const int tid = threadIdx.x, lane = tid & 63;
  const int G = lane >> 4, n = lane & 15;
  float4* st4 = stage + (tid >> 6) * 32 * inner;
  float2* stw = reinterpret_cast<float2*>(st4);
  for (int f = tid; f < 8 * 64; f += kThreads) {
    const int ln = f & 63, rt = f >> 6;
    const int d = 16 * (rt >> 1) + (ln & 15), part = rt & 1, g = ln >> 4;
    v8bf h, l;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int j = 4 * g + (i >> 1), cu = i & 1;
      float v = 0.f;
      if (j < m) {
        const float2 t = twiddle_any((((j - m / 2) * d) % kN + kN) % kN, kN);
        // Re Z = cos Ur - sin Ui, Im Z = sin Ur + cos Ui
        v = part == 0 ? (cu == 0 ? t.x : -t.y) : (cu == 0 ? t.y : t.x);
        v *= scale;
      }
      const bf2 q = split(v);
      h[i] = q.hi;
      l[i] = q.lo;
    }
    af[(rt * 2) * 64 + ln] = h;
    af[(rt * 2 + 1) * 64 + ln] = l;
  }
  __syncthreads();
  const int64_t nwaves = (int64_t)gridDim.x * kWaves;
#pragma unroll 1
  for (int64_t s = (int64_t)blockIdx.x * kWaves + (tid >> 6); s < slabs; s += nwaves) {
    // B: lane (G, n) holds U[s, 4 G + i / 2, n] (Re, Im) for i < 8
    const float2* us = src + s * m * inner;
    v8bf bh, bl;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int j = 4 * G + q;
      const float2 uv = (j < m && n < inner) ? us[j * inner + n] : make_float2(0.f, 0.f);
      const bf2 a = split(uv.x), c = split(uv.y);
      bh[2 * q] = a.hi;
      bl[2 * q] = a.lo;
      bh[2 * q + 1] = c.hi;
      bl[2 * q + 1] = c.lo;
    }
    float2* zs = dst + s * kN * inner;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      v4f re = (v4f)0.f, im = (v4f)0.f;
      re = mma3(af[((2 * t) * 2) * 64 + lane], af[((2 * t) * 2 + 1) * 64 + lane], bh, bl, re);
      im = mma3(af[((2 * t + 1) * 2) * 64 + lane], af[((2 * t + 1) * 2 + 1) * 64 + lane], bh, bl, im);
      if (n < inner) {
#pragma unroll
        for (int r = 0; r < 4; ++r) stw[(16 * t + 4 * G + r) * inner + n] = make_float2(re[r], im[r]);
      }
    }
    wave_sync();
    // 32 inner float4 words: the slab's output run (16-byte aligned: 512 inner bytes per slab)
    float4* z4 = reinterpret_cast<float4*>(zs);
    for (int q = lane; q < 32 * inner; q += 64) z4[q] = st4[q];
    wave_sync();
  }
}

// ----------------------------------------------------------------------------
// Inverse along the first two 64-point axes of a plane's window of m0 x m1
// centred rows (m0, m1 <= 16) and inner <= 16 columns:
//
//   U[d0, j1, c] = sum_{j0 < m0} Y[j0, j1, c] e^{2 pi i (j0 - m0/2) d0 / 64}
//   Z[d0, d1, c] = t sum_{j1 < m1} U[d0, j1, c] e^{2 pi i (j1 - m1/2) d1 / 64}
//
// (the first two ifftn axes of a 3D SpectralConv.forward inverse,
// spectral_convolution.py:547-548).  A workgroup takes 16 values of d0 of one
// plane: it loads the plane's window into LDS, forms U for its 16 d0 there as
// a product on the matrix cores (the window expanded along the first axis
// never goes through memory), and each wave runs k_axis_inv64's product on 4
// of the 16 slabs.  Both products: three-term bf16 splits, fp32 accumulation.  The four
// workgroups of a plane run on one XCD, so the window is fetched into one L2.
constexpr int kInv2D0 = 16;   // values of d0 per workgroup

__global__ void __launch_bounds__(sl::kThreads)
k_axis_inv64x2(const float2* __restrict__ src, float2* __restrict__ dst, int64_t planes, int m0,
               int m1, int inner, float scale) {
  using namespace sl;
  __shared__ float2 tw[kN];
  // [ybig] the plane's window [m0][m1][inner], later the waves' output
  // stages [kWaves][64 inner]; then U [kInv2D0][m1][inner]
  extern __shared__ float4 dyn[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = lane >> 4, n = lane & 15;
  // workgroup i -> plane 8 (i / 32) + i % 8, quarter (i / 8) % 4: consecutive
  // workgroups go to consecutive XCDs, so the quarters of a plane share one
  const int i = (int)blockIdx.x, k = i >> 3;
  const int64_t p = (int64_t)(k >> 2) * 8 + (i & 7);
  const int d0b = kInv2D0 * (k & 3);
  if (p >= planes) return;
  const int ul = m1 * inner, yl = m0 * ul;
  const int ybig = yl > kWaves * 64 * inner ? yl : kWaves * 64 * inner;
  float2* yb = reinterpret_cast<float2*>(dyn);
  float2* ub = yb + ybig;
  const float2* ys = src + p * yl;
  for (int f = tid; f < yl; f += kThreads) yb[f] = ys[f];
  if (tid < kN) tw[tid] = twiddle_any(tid, kN);
  __syncthreads();
  // U for d0 = d0b + dl as a product on the matrix cores: rows (dl, Re | Im)
  // in two row tiles, K slot (G, e) = window row j0 = 4 G + e / 2 and Re / Im
  // of Y (as in the second product), columns (j1, c) in tiles of 16
  {
    v8bf ah[2], al[2];
#pragma unroll
    for (int part = 0; part < 2; ++part) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int j = 4 * G + (e >> 1), cu = e & 1;
        float v = 0.f;
        if (j < m0) {
          const float2 t = tw[((j - m0 / 2) * (d0b + n)) & (kN - 1)];
          v = part == 0 ? (cu == 0 ? t.x : -t.y) : (cu == 0 ? t.y : t.x);
        }
        const bf2 q = split(v);
        ah[part][e] = q.hi;
        al[part][e] = q.lo;
      }
    }
    const int ctiles = (ul + 15) / 16;
#pragma unroll 1
    for (int ct = wave; ct < ctiles; ct += kWaves) {
      const int col = 16 * ct + n;
      v8bf bh, bl;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int j = 4 * G + q;
        const float2 yv = (j < m0 && col < ul) ? yb[j * ul + col] : make_float2(0.f, 0.f);
        const bf2 a = split(yv.x), c = split(yv.y);
        bh[2 * q] = a.hi;
        bl[2 * q] = a.lo;
        bh[2 * q + 1] = c.hi;
        bl[2 * q + 1] = c.lo;
      }
      const v4f re = mma3(ah[0], al[0], bh, bl, (v4f)0.f);
      const v4f im = mma3(ah[1], al[1], bh, bl, (v4f)0.f);
      if (col < ul) {
#pragma unroll
        for (int r = 0; r < 4; ++r) ub[(4 * G + r) * ul + col] = make_float2(re[r], im[r]);
      }
    }
  }
  __syncthreads();
  // the second product's A fragments (as in k_axis_inv64, window rows j1) in
  // registers: row tile rt = 2 t + part, rows d1 = 16 t + lane % 16
  v8bf fh[8], fl[8];
#pragma unroll
  for (int rt = 0; rt < 8; ++rt) {
    const int d = 16 * (rt >> 1) + n, part = rt & 1;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int j = 4 * G + (e >> 1), cu = e & 1;
      float v = 0.f;
      if (j < m1) {
        const float2 t = tw[((j - m1 / 2) * d) & (kN - 1)];
        v = part == 0 ? (cu == 0 ? t.x : -t.y) : (cu == 0 ? t.y : t.x);
        v *= scale;
      }
      const bf2 q = split(v);
      fh[rt][e] = q.hi;
      fl[rt][e] = q.lo;
    }
  }
  // the window is no longer read: its space holds the waves' output stages
  float4* st4 = dyn + wave * 32 * inner;
  float2* stw = reinterpret_cast<float2*>(st4);
#pragma unroll 1
  for (int dl = wave; dl < kInv2D0; dl += kWaves) {
    const float2* us = ub + dl * ul;
    v8bf bh, bl;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int j = 4 * G + q;
      const float2 uv = (j < m1 && n < inner) ? us[j * inner + n] : make_float2(0.f, 0.f);
      const bf2 a = split(uv.x), c = split(uv.y);
      bh[2 * q] = a.hi;
      bl[2 * q] = a.lo;
      bh[2 * q + 1] = c.hi;
      bl[2 * q + 1] = c.lo;
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      v4f re = (v4f)0.f, im = (v4f)0.f;
      re = mma3(fh[2 * t], fl[2 * t], bh, bl, re);
      im = mma3(fh[2 * t + 1], fl[2 * t + 1], bh, bl, im);
      if (n < inner) {
#pragma unroll
        for (int r = 0; r < 4; ++r) stw[(16 * t + 4 * G + r) * inner + n] = make_float2(re[r], im[r]);
      }
    }
    wave_sync();
    float4* z4 = reinterpret_cast<float4*>(dst + ((p * kN) + d0b + dl) * kN * inner);
    for (int q = lane; q < 32 * inner; q += 64) z4[q] = st4[q];
    wave_sync();
  }
}

// ============================================================== host side
bool slab_fwd64_supported(int N1, int N2, int m1, int m2h) {
  return N1 == sl::kN && N2 == sl::kN && m1 >= 1 && m1 <= 16 && m2h >= 1 && m2h <= 16;
}

// slabs of 64 x 64 floats at x (16-byte aligned) -> [slabs][m1][m2h] window
static int slab_cus() {
  static int cus = 0;
  if (!cus) {
    int dev = 0, n = 0;
    cus = (hipGetDevice(&dev) == hipSuccess &&
           hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
           n > 0)
              ? n
              : 256;
  }
  return cus;
}

int slab_fwd64(const float* x, float2* out, int64_t slabs, int m1, int m2h, float scale,
               hipStream_t st) {
  // as many workgroups as are resident at once (two per CU by registers);
  // the waves loop over the slabs, so each workgroup builds its twiddle
  // fragments once
  int64_t grid = (slabs + sl::kWaves - 1) / sl::kWaves;
  if (grid > 2 * slab_cus()) grid = 2 * slab_cus();
  hipLaunchKernelGGL(k_slab_fwd64, dim3((unsigned)grid), dim3(sl::kThreads), 0, st, x, out, slabs,
                     m1, m2h, scale);
  return launch_status("k_slab_fwd64");
}

bool axis_inv64_supported(int N, int Np, int m, int64_t inner) {
  return N == sl::kN && Np == sl::kN && m >= 1 && m <= 16 && inner >= 1 && inner <= 16;
}

// [slabs][m][inner] window -> [slabs][64][inner], scaled by scale
int axis_inv64(const float2* src, float2* dst, int64_t slabs, int m, int inner, float scale,
               hipStream_t st) {
  int64_t grid = (slabs + sl::kWaves - 1) / sl::kWaves;
  if (grid > 4 * slab_cus()) grid = 4 * slab_cus();
  hipLaunchKernelGGL(k_axis_inv64, dim3((unsigned)grid), dim3(sl::kThreads),
                     (size_t)sl::kWaves * 32 * inner * sizeof(float4), st, src, dst, slabs,
                     m, inner, scale);
  return launch_status("k_axis_inv64");
}

bool axis_inv64x2_supported(int N0, int Np0, int m0, int N1, int Np1, int m1, int64_t inner) {
  return N0 == sl::kN && Np0 == sl::kN && m0 >= 1 && m0 <= 16 &&
         axis_inv64_supported(N1, Np1, m1, inner);
}

// [planes][m0][m1][inner] window -> [planes][64][64][inner], scaled by scale
int axis_inv64x2(const float2* src, float2* dst, int64_t planes, int m0, int m1, int inner,
                 float scale, hipStream_t st) {
  const int64_t yl = (int64_t)m0 * m1 * inner, stg = (int64_t)sl::kWaves * 64 * inner;
  const size_t lds = (size_t)((yl > stg ? yl : stg) + (int64_t)kInv2D0 * m1 * inner) * 8;
  if (lds > 64 * 1024) {
    int rc = hip_status(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_axis_inv64x2),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                        "hipFuncSetAttribute(MaxDynamicSharedMemorySize)");
    if (rc) return rc;
  }
  // planes rounded up to groups of 8 (one per XCD), four workgroups each
  const int64_t grid = (planes + 7) / 8 * 8 * (sl::kN / kInv2D0);
  hipLaunchKernelGGL(k_axis_inv64x2, dim3((unsigned)grid), dim3(sl::kThreads), lds, st, src, dst,
                     planes, m0, m1, inner, scale);
  return launch_status("k_axis_inv64x2");
}

}  // namespace fno
