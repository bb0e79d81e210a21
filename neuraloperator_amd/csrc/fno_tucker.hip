// Tucker-factorized spectral contraction in two launches (instead of a chain
// of one launch per factor):
//
//   K[g, h, k] = sum_a core[g, h, a_1..a_n] prod_d U_d[k_d, a_d]        (k_tucker_core)
//   y[b, o, k] = sum_h U_out[o, h] sum_g K[g, h, k] sum_i x[b, i, k] U_in[i, g]
//                                                                       (k_tucker_contract)
//
// which is _contract_tucker's einsum (neuralop/layers/spectral_convolution.py
// :76-103, non-separable) evaluated factor by factor: the mode factors are
// folded into the core once per call (K has rank_in x rank_out x modes
// entries), then each mode's three small products run in LDS.  Complex fp32
// arithmetic on VALU: the operands are a few MB, the work a few hundred
// MFLOP, so both kernels are bound by their loads.
#include "fno_common.h"

namespace fno {

namespace tk {
// threads per workgroup: both kernels are bound by per-thread latency chains
// (few waves per SIMD at 256 threads), so each thread takes fewer outputs
// (C4 shape: core 13.9 -> 11.0 us at 1024, contraction 23.0 -> 21.9 at 512)
constexpr int kCoreThreads = 1024, kContractThreads = 512;
constexpr size_t kMaxLds = 64 * 1024;
}  // namespace tk

// One workgroup per (g, h): the core's [r1, r2(, r3)] block is multiplied
// along its last axis first, then the middle one, then the first, each stage
// in LDS; the last stage writes K[g][h][k1][k2](k3) to memory.  ND = 2 or 3.
template <int ND>
__global__ void __launch_bounds__(tk::kCoreThreads)
k_tucker_core(const float2* __restrict__ core, const float2* __restrict__ U1,
              const float2* __restrict__ U2, const float2* __restrict__ U3,
              float2* __restrict__ K, int r1, int r2, int r3, int m1, int m2, int m3) {
  extern __shared__ float2 lds[];
  const int tid = threadIdx.x;
  const int R3 = ND == 3 ? r3 : 1, M3 = ND == 3 ? m3 : 1;
  const int nc = r1 * r2 * R3;
  float2* c = lds;                        // [r1][r2][R3]
  float2* t1 = c + nc;                    // [r1][r2][M3]
  float2* t2 = t1 + r1 * r2 * M3;         // [r1][m2][M3]
  float2* u1 = t2 + r1 * m2 * M3;         // [m1][r1]
  float2* u2 = u1 + m1 * r1;              // [m2][r2]
  float2* u3 = u2 + m2 * r2;              // [M3][R3]
  const float2* src = core + (int64_t)blockIdx.x * nc;
  for (int i = tid; i < nc; i += tk::kCoreThreads) c[i] = src[i];
  for (int i = tid; i < m1 * r1; i += tk::kCoreThreads) u1[i] = U1[i];
  for (int i = tid; i < m2 * r2; i += tk::kCoreThreads) u2[i] = U2[i];
  if (ND == 3)
    for (int i = tid; i < m3 * r3; i += tk::kCoreThreads) u3[i] = U3[i];
  __syncthreads();
  const float2* s1 = c;
  if (ND == 3) {
    // t1[a1][a2][k3] = sum_a3 c[a1][a2][a3] U3[k3][a3]
    for (int e = tid; e < r1 * r2 * m3; e += tk::kCoreThreads) {
      const int k3 = e % m3, a12 = e / m3;
      float2 acc = make_float2(0.f, 0.f);
      for (int a3 = 0; a3 < r3; ++a3) cfma(acc, c[a12 * r3 + a3], u3[k3 * r3 + a3]);
      t1[e] = acc;
    }
    __syncthreads();
    s1 = t1;
  }
  // t2[a1][k2][k3] = sum_a2 s1[a1][a2][k3] U2[k2][a2]
  for (int e = tid; e < r1 * m2 * M3; e += tk::kCoreThreads) {
    const int k3 = e % M3, k2 = (e / M3) % m2, a1 = e / (M3 * m2);
    float2 acc = make_float2(0.f, 0.f);
    for (int a2 = 0; a2 < r2; ++a2) cfma(acc, s1[(a1 * r2 + a2) * M3 + k3], u2[k2 * r2 + a2]);
    t2[e] = acc;
  }
  __syncthreads();
  // K[k1][k2][k3] = sum_a1 t2[a1][k2][k3] U1[k1][a1]
  float2* dst = K + (int64_t)blockIdx.x * m1 * m2 * M3;
  for (int e = tid; e < m1 * m2 * M3; e += tk::kCoreThreads) {
    const int k23 = e % (m2 * M3), k1 = e / (m2 * M3);
    float2 acc = make_float2(0.f, 0.f);
    for (int a1 = 0; a1 < r1; ++a1) cfma(acc, t2[a1 * m2 * M3 + k23], u1[k1 * r1 + a1]);
    dst[e] = acc;
  }
}

// A workgroup per tile of KT modes: x, K, U_in and U_out of the tile into
// LDS, then t1 = x U_in, t2 = t1 K, y = t2 U_out^T, each a loop over the
// workgroup's outputs with the modes fastest (coalesced loads and stores).
__global__ void __launch_bounds__(tk::kContractThreads)
k_tucker_contract(const float2* __restrict__ X, const float2* __restrict__ K,
                  const float2* __restrict__ Uin, const float2* __restrict__ Uout,
                  float2* __restrict__ Y, int B, int Ci, int Co, int rin, int rout, int64_t M,
                  int KT) {
  extern __shared__ float2 lds[];
  const int tid = threadIdx.x;
  const int64_t k0 = (int64_t)blockIdx.x * KT;
  const int kt = (int)(M - k0 < KT ? M - k0 : KT);
  float2* uin = lds;                          // [Ci][rin]
  float2* uout = uin + Ci * rin;              // [Co][rout]
  float2* kk = uout + Co * rout;              // [rin][rout][KT]
  float2* xt = kk + rin * rout * KT;          // [B][Ci][KT]
  float2* t1 = xt + B * Ci * KT;              // [B][rin][KT]
  float2* t2 = t1 + B * rin * KT;             // [B][rout][KT]
  for (int i = tid; i < Ci * rin; i += tk::kContractThreads) uin[i] = Uin[i];
  for (int i = tid; i < Co * rout; i += tk::kContractThreads) uout[i] = Uout[i];
  for (int e = tid; e < rin * rout * KT; e += tk::kContractThreads) {
    const int k = e % KT, gh = e / KT;
    kk[e] = k < kt ? K[(int64_t)gh * M + k0 + k] : make_float2(0.f, 0.f);
  }
  for (int e = tid; e < B * Ci * KT; e += tk::kContractThreads) {
    const int k = e % KT, bi = e / KT;
    xt[e] = k < kt ? X[(int64_t)bi * M + k0 + k] : make_float2(0.f, 0.f);
  }
  __syncthreads();
  for (int e = tid; e < B * rin * KT; e += tk::kContractThreads) {
    const int k = e % KT, g = (e / KT) % rin, b = e / (KT * rin);
    float2 acc = make_float2(0.f, 0.f);
    for (int i = 0; i < Ci; ++i) cfma(acc, xt[(b * Ci + i) * KT + k], uin[i * rin + g]);
    t1[e] = acc;
  }
  __syncthreads();
  for (int e = tid; e < B * rout * KT; e += tk::kContractThreads) {
    const int k = e % KT, h = (e / KT) % rout, b = e / (KT * rout);
    float2 acc = make_float2(0.f, 0.f);
    for (int g = 0; g < rin; ++g) cfma(acc, t1[(b * rin + g) * KT + k], kk[(g * rout + h) * KT + k]);
    t2[e] = acc;
  }
  __syncthreads();
  for (int e = tid; e < B * Co * KT; e += tk::kContractThreads) {
    const int k = e % KT, o = (e / KT) % Co, b = e / (KT * Co);
    if (k >= kt) continue;
    float2 acc = make_float2(0.f, 0.f);
    for (int h = 0; h < rout; ++h) cfma(acc, t2[(b * rout + h) * KT + k], uout[o * rout + h]);
    Y[((int64_t)b * Co + o) * M + k0 + k] = acc;
  }
}

// ============================================================== host side
static size_t tucker_core_lds(int nd, const int32_t* ranks, const int32_t* modes) {
  const int64_t r1 = ranks[2], r2 = ranks[3], r3 = nd == 3 ? ranks[4] : 1;
  const int64_t m1 = modes[0], m2 = modes[1], m3 = nd == 3 ? modes[2] : 1;
  return (size_t)(r1 * r2 * r3 + r1 * r2 * m3 + r1 * m2 * m3 + m1 * r1 + m2 * r2 + m3 * r3) * 8;
}

static size_t tucker_contract_lds(int B, int Ci, int Co, int rin, int rout, int KT) {
  return (size_t)((int64_t)Ci * rin + (int64_t)Co * rout + (int64_t)rin * rout * KT +
                  (int64_t)B * (Ci + rin + rout) * KT) * 8;
}

// Modes per contraction tile: the largest of 16, 8, 4, 2, 1 whose LDS fits.
static int tucker_tile(int B, int Ci, int Co, int rin, int rout) {
  for (int kt = 16; kt >= 1; kt /= 2)
    if (tucker_contract_lds(B, Ci, Co, rin, rout, kt) <= tk::kMaxLds) return kt;
  return 0;
}

// The two-launch path covers 2 and 3 mode axes whose per-(g, h) stages and
// contraction tiles fit in LDS; K needs rank_in x rank_out x modes entries of
// workspace (the chain's K buffer).
bool tucker_fused_supported(int B, int Ci, int Co, int ndim, const int32_t* modes,
                            const int32_t* ranks) {
  if (ndim != 2 && ndim != 3) return false;
  if (tucker_core_lds(ndim, ranks, modes) > tk::kMaxLds) return false;
  return tucker_tile(B, Ci, Co, ranks[0], ranks[1]) > 0;
}

int tucker_fused(const float2* X, const float2* core, const float2* const* factors,
                 const int32_t* ranks, float2* Y, int B, int Ci, int Co, int ndim,
                 const int32_t* modes, float2* Kbuf, hipStream_t st) {
  int64_t M = 1;
  for (int d = 0; d < ndim; ++d) M *= modes[d];
  const int rin = ranks[0], rout = ranks[1];
  const size_t lc = tucker_core_lds(ndim, ranks, modes);
  const unsigned pairs = (unsigned)(rin * rout);
  if (ndim == 3)
    hipLaunchKernelGGL(k_tucker_core<3>, dim3(pairs), dim3(tk::kCoreThreads), lc, st, core, factors[2],
                       factors[3], factors[4], Kbuf, ranks[2], ranks[3], ranks[4], modes[0],
                       modes[1], modes[2]);
  else
    hipLaunchKernelGGL(k_tucker_core<2>, dim3(pairs), dim3(tk::kCoreThreads), lc, st, core, factors[2],
                       factors[3], factors[3], Kbuf, ranks[2], ranks[3], 1, modes[0], modes[1], 1);
  int rc = launch_status("k_tucker_core");
  if (rc) return rc;
  const int KT = tucker_tile(B, Ci, Co, rin, rout);
  const unsigned tiles = (unsigned)((M + KT - 1) / KT);
  hipLaunchKernelGGL(k_tucker_contract, dim3(tiles), dim3(tk::kContractThreads),
                     tucker_contract_lds(B, Ci, Co, rin, rout, KT), st, X, Kbuf, factors[0],
                     factors[1], Y, B, Ci, Co, rin, rout, M, KT);
  return launch_status("k_tucker_contract");
}

}  // namespace fno
