// 1D spectral block for lines of N = 256 .. 1024 points (N dividing 1024) and
// at most 16 kept rfft bins, as one launch (linear skip, below) or as two
// (no / identity / soft-gating skip, the line path further down):
//
//   y[b, o, n] = act( sum_k c_k s_i Re( Y[b, o, k] e^{2 pi i k n / N} )
//                     + bias[o] + (Ws x)[b, o, n] ),
//   Y[b, o, k] = sum_c X[b, c, k] W[c, o, k],
//   X[b, c, k] = s_f sum_n x[b, c, n] e^{-2 pi i k n / N}
//
// (SpectralConv.forward for real 1D data, neuralop/layers/
// spectral_convolution.py:417-570 with order 1: rfft, the first m bins,
// _contract_dense, irfft(n = N), bias; plus the block skip and activation of
// fno_block.py:331-361.)  One workgroup per (sample, 16 output channels):
//   1. X: the truncated DFT as a matrix product x[Ci x N] . F[N x 2m] on
//      v_mfma_f32_16x16x32_bf16 with three-term bf16 splits (F = s_f cos /
//      -s_f sin, built once per workgroup as LDS fragments from a twiddle
//      table), each of the 8 waves one 16-channel tile over half the
//      points; the two halves' X land in LDS.
//   2. Y for the workgroup's 16 channels on VALU (16 x m complex sums over
//      Ci, split in two halves over all 512 threads, whose W loads are issued
//      at the start), written to LDS as the hi / lo A fragments of step 3.
//   3. y: the real synthesis as a product Yt[16 x 2m] . T[2m x N] (T = c_k
//      s_i cos / -c_k s_i sin, the Hermitian weights and the inverse scale
//      folded in, the imaginary part of the DC bin meeting sin 0 = 0) plus
//      the skip Ws[16 x Ci] . x[Ci x N] (the 1x1 conv; diag(g) for
//      soft-gating, the identity), seeded with the bias; activation; store.
// The spectrum never leaves the chip.
// Products as three-term bf16 splits with fp32 accumulation, as in the 2D
// row epilogue (each within 3 * 2^-16 of |a b|).
#include "fno_twiddle.h"

namespace fno {

namespace f1 {
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kWaves = 8, kThreads = 64 * kWaves;
constexpr int kMaxN = 1024, kMaxM = 16;
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
}  // namespace f1

// CI input channels (32 or 64); N, m, Co runtime (N % 256 == 0, N | 1024,
// m <= 16, Co % 16 == 0).  MFMA 16x16x32 bf16 operand layout: A[m = lane % 16]
// [k = 8 (lane / 16) + i], B[k = 8 (lane / 16) + i][n = lane % 16], D[4 (lane
// / 16) + r][lane % 16].
template <int CI, bool XSKIP>
__global__ void __launch_bounds__(f1::kThreads)
k_conv1d_fused(const float* __restrict__ x, const float2* __restrict__ w,
               const float* __restrict__ bias, const float* __restrict__ skip_w,
               float* __restrict__ y, int N, int m, int Co, int skip_kind, int act, float fs,
               float is) {
  using namespace f1;
  constexpr int CT = CI / 16;                  // channel tiles of the forward product
  static_assert(CT * 2 <= kWaves, "one forward tile per wave");
  __shared__ float2 tw[kMaxN];                 // e^{+2 pi i t / N}
  __shared__ float2 Yp[2][16][kMaxM];          // two halves of the channel sums of Y
  __shared__ v8bf yf[2][64];                   // Yt fragments (hi, lo) of the 16 channels
  __shared__ v8bf wfr[CI / 32 > 0 ? CI / 32 : 1][2][64];  // skip-weight fragments
  // F fragments of the forward product, [k-step][column tile][hi | lo][lane];
  // once it is done the region holds X[half][c][2k + (0 re | 1 im)], the two
  // point halves' partial spectra (rows padded to an odd stride, so the
  // contraction's two channel parities read different banks)
  extern __shared__ v8bf ffr[];
  constexpr int XS = 2 * kMaxM + 1;
  float (*Xs)[CI][XS] = reinterpret_cast<float (*)[CI][XS]>(ffr);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = lane >> 4, nl = lane & 15;
  const int OT = Co / 16;
  const int b = blockIdx.x / OT, o0 = 16 * (blockIdx.x % OT);
  const float* xb = x + (int64_t)b * CI * N;
  const uint32_t gmask = act_mask(act == FNO_ACT_GELU);
  // forward roles: wave (ct, kh) takes channel tile ct over points
  // [kh N/2, (kh + 1) N/2), both column tiles; its first 256 points' loads go
  // out before the set-up below
  // (with 32 channels waves 4..7 have no tile; they load wave - 4's rows,
  // unused, to keep every load outside a branch)
  const int fct = wave % CT, fkh = (wave / CT) & 1;
  const bool fwd_on = 2 * CT == kWaves || wave < 2 * CT;
  // Every global load of the set-up is unconditional (indices clamped into
  // range) so that none of them sits behind a branch: the twiddles (at most
  // two per thread) first, then the x batch, then W.
  const int tstep = twd::kN / N;
  float tre[2], tim[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int t = (tid + kThreads * u) & (N - 1);
    tre[u] = kTw.re[t * tstep];
    tim[u] = kTw.im[t * tstep];
  }
  // (a batch is 8 k-steps of 32 points, 4 when the half line has only 128;
  // the 4 spare loads then re-read the first ones)
  const int qn = N >= 512 ? 8 : 4;
  const float* xr = xb + (int64_t)(16 * fct + nl) * N + (N / 2) * fkh + 8 * G;
  float4 a[8][2];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int qq = q < qn ? q : 0;
    a[q][0] = *reinterpret_cast<const float4*>(xr + 32 * qq);
    a[q][1] = *reinterpret_cast<const float4*>(xr + 32 * qq + 4);
  }
  // W of the contraction, used after the forward product: thread (ol, k,
  // half) sums the channels c = 2 i + half of Y[o0 + ol][k].  A bin
  // k >= m reads bin m - 1's weights: its X is zero (the F columns of such
  // bins are zero) and its T rows are zero, so those products never reach y.
  const int yo = tid >> 5, yk = (tid >> 1) & 15, yh = tid & 1;
  float2 wv[CI / 2];
  {
    const float2* wp = w + (int64_t)(o0 + yo) * m + (yk < m ? yk : m - 1);   // w[c][o][k]
    const int64_t cs = (int64_t)Co * m;
#pragma unroll
    for (int c = 0; c < CI / 2; ++c) wv[c] = wp[(int64_t)(2 * c + yh) * cs];
  }
  // (entries N .. 1023 get wrapped copies, never read)
#pragma unroll
  for (int u = 0; u < 2; ++u) tw[tid + kThreads * u] = make_float2(tre[u], tim[u]);
  if constexpr (XSKIP) {
    // A[m = o0 + lane % 16][k = c = 32 ks + 8 G + i]
    for (int f = tid; f < (CI / 32) * 64; f += kThreads) {
      const int ln = f & 63, ks = f >> 6, o = o0 + (ln & 15);
      v8bf h, l;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int c = 32 * ks + 8 * (ln >> 4) + i;
        float v;
        if (skip_kind == FNO_SKIP_LINEAR) v = skip_w[o * CI + c];
        else if (skip_kind == FNO_SKIP_SOFT_GATING) v = (c == o) ? skip_w[o] : 0.f;
        else v = (c == o) ? 1.f : 0.f;
        const bf2 p = split(v);
        h[i] = p.hi;
        l[i] = p.lo;
      }
      wfr[ks][0][ln] = h;
      wfr[ks][1][ln] = l;
    }
  }
  __syncthreads();
  // F[n][col] = s_f cos (even col) / -s_f sin (odd col) of 2 pi (col / 2) n / N
  // for bins col / 2 < m, as B fragments: element i of lane l in k-step ks,
  // column tile nt is F[32 ks + 8 (l / 16) + i][16 nt + l % 16]
  const int NKS = N / 32;
  for (int f = tid; f < NKS * 2 * 64; f += kThreads) {
    const int ln = f & 63, nt = (f >> 6) & 1, ks = f >> 7;
    const int col = 16 * nt + (ln & 15), kb = col >> 1;
    v8bf h, l;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int n = 32 * ks + 8 * (ln >> 4) + i;
      const float2 t = tw[(kb * n) & (N - 1)];
      const float v = kb < m ? fs * ((col & 1) ? -t.y : t.x) : 0.f;
      const bf2 p = split(v);
      h[i] = p.hi;
      l[i] = p.lo;
    }
    ffr[((ks * 2 + nt) * 2) * 64 + ln] = h;
    ffr[((ks * 2 + nt) * 2 + 1) * 64 + ln] = l;
  }
  __syncthreads();

  // ---- 1. X tiles: wave (ct, kh) accumulates X[16 ct + row][col] over its
  //      half of the points for both column tiles (col = 16 nt + lane % 16)
  v4f acc[2] = {(v4f)0.f, (v4f)0.f};
  if (fwd_on) {
    const int ks0 = (N / 64) * fkh;            // first k-step of this half
#pragma unroll 1
    for (int nc = 0; nc < N / 2; nc += 256) {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        if (q < qn) {
          const float av[8] = {a[q][0].x, a[q][0].y, a[q][0].z, a[q][0].w,
                               a[q][1].x, a[q][1].y, a[q][1].z, a[q][1].w};
          v8bf ah, al;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const bf2 pa = split(av[i]);
            ah[i] = pa.hi;
            al[i] = pa.lo;
          }
          const int ks = ks0 + (nc >> 5) + q;
#pragma unroll
          for (int nt = 0; nt < 2; ++nt)
            acc[nt] = mma3(ah, al, ffr[((ks * 2 + nt) * 2) * 64 + lane],
                           ffr[((ks * 2 + nt) * 2 + 1) * 64 + lane], acc[nt]);
        }
      }
      if (nc + 256 < N / 2) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          a[q][0] = *reinterpret_cast<const float4*>(xr + nc + 256 + 32 * q);
          a[q][1] = *reinterpret_cast<const float4*>(xr + nc + 256 + 32 * q + 4);
        }
      }
    }
  }
  __syncthreads();                             // every wave is done with F
  if (fwd_on) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) Xs[fkh][16 * fct + 4 * G + r][16 * nt + nl] = acc[nt][r];
  }
  __syncthreads();

  // ---- 2. Y[o0 + ol][k] on VALU: the two channel halves from the W loads
  //      issued at the start, summed, then written as the A fragments
  //      Yt[ol][j = 2k + (0 | 1)]: lane ol + 16 (j / 8), element j % 8
  {
    float2 acc = make_float2(0.f, 0.f);
#pragma unroll
    for (int c = 0; c < CI / 2; ++c) {
      const int cc = 2 * c + yh;
      const float2 xv = make_float2(Xs[0][cc][2 * yk] + Xs[1][cc][2 * yk],
                                    Xs[0][cc][2 * yk + 1] + Xs[1][cc][2 * yk + 1]);
      cfma(acc, xv, wv[c]);
    }
    Yp[yh][yo][yk] = acc;
  }
  __syncthreads();
  if (tid < 256) {
    const int ol = tid >> 4, k = tid & 15;
    const float2 a = Yp[0][ol][k], c2 = Yp[1][ol][k];
    const float2 acc = make_float2(a.x + c2.x, a.y + c2.y);
    const int j = 2 * k, ln = ol + 16 * (j >> 3), el = j & 7;
    const bf2 pr = split(acc.x), pi = split(acc.y);
    __bf16* fh = reinterpret_cast<__bf16*>(&yf[0][ln]) + el;
    __bf16* fl = reinterpret_cast<__bf16*>(&yf[1][ln]) + el;
    fh[0] = pr.hi;
    fh[1] = pi.hi;
    fl[0] = pr.lo;
    fl[1] = pi.lo;
  }
  __syncthreads();

  // ---- 3. y tiles: 16 output channels x 16 points per tile, the line's
  //      N / 16 tiles dealt out over the 8 waves
  const v8bf zh = yf[0][lane], zl = yf[1][lane];
  float bch[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) bch[r] = bias ? bias[o0 + 4 * G + r] : 0.f;
  float* yb = y + ((int64_t)b * Co + o0) * N;
  for (int nt = wave; nt < N / 16; nt += kWaves) {
    const int n = 16 * nt + nl;
    v4f acc;
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = bch[r];
    if constexpr (XSKIP) {
      // the tile's skip operand: all CI channel loads in flight first
      float xv[CI / 32][8];
#pragma unroll
      for (int ks = 0; ks < CI / 32; ++ks)
#pragma unroll
        for (int i = 0; i < 8; ++i) xv[ks][i] = xb[(int64_t)(32 * ks + 8 * G + i) * N + n];
#pragma unroll
      for (int ks = 0; ks < CI / 32; ++ks) {
        v8bf bh, bl;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const bf2 p = split(xv[ks][i]);
          bh[i] = p.hi;
          bl[i] = p.lo;
        }
        acc = mma3(wfr[ks][0][lane], wfr[ks][1][lane], bh, bl, acc);
      }
    }
    v8bf th, tl;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int j = 8 * G + i, k = j >> 1;
      float v = 0.f;
      if (k < m) {
        const float2 t = tw[(k * n) & (N - 1)];
        const float c = (k == 0) ? is : 2.f * is;
        v = (j & 1) ? -c * t.y : c * t.x;
      }
      const bf2 p = split(v);
      th[i] = p.hi;
      tl[i] = p.lo;
    }
    acc = mma3(zh, zl, th, tl, acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = acc[r];
      v = act_select(gelu_erf(v), v, gmask);
      yb[(int64_t)(4 * G + r) * N + n] = v;
    }
  }
}

// ============================================================== host side
// Shapes the one-launch 1D block covers: N a power of two in [256, 1024], at
// most 16 kept bins (never the Nyquist bin then), 32 or 64 input channels
// (the forward product and the skip tile them by 16 and 32), output channels
// a multiple of 16.
// ---------------------------------------------------------------------------
// Two-kernel 1D path for blocks without a linear skip (the plain SpectralConv
// of a 1D FNO): the one-launch kernel above runs one workgroup per (sample, 16
// output channels), each loading its sample's whole x and computing its full
// truncated DFT, so a batch of 16 samples keeps 64 CUs busy, bound by their
// loads.  Here the DFT is spread over one wave per line and the synthesis over
// one workgroup per (sample, 4 output channels), and only the m-bin spectra
// pass between the two through the workspace.
namespace l1 {
constexpr int kThreads = 256, kLines = 4;   // lines (waves) per DFT workgroup
constexpr int kOut = 4;                      // output channels per synthesis workgroup
constexpr int kSynThreads = 512;             // two waves (point halves) per output channel
constexpr int kMaxM = 16;
constexpr int kChunk = 8;                    // contraction loads in flight per thread
}  // namespace l1

// X[line][k] = s sum_n x[line][n] e^{-2 pi i k n / N}, k < m.  Lane l of the
// line's wave holds n = l + 64 j (j < J = N / 64):
//   X[k] = sum_l e^{-2 pi i k l / N} S_{k mod J}(l),
//   S_r(l) = sum_j x[l + 64 j] e^{-2 pi i r j / J}
// (a J-point DFT per lane with constant twiddles, S_{J - r} = conj(S_r) for
// real x, one twiddle per bin, then the sum over the wave's lanes as a
// butterfly reduce-scatter of the 32 floats: 32 lane exchanges instead of
// 6 x 32).
template <int N>
__global__ void __launch_bounds__(l1::kThreads)
k_line_dft(const float* __restrict__ x, float2* __restrict__ xhat, int64_t lines, int m,
           float scale) {
  constexpr int J = N / 64;
  const int lane = threadIdx.x & 63;
  const int64_t line = (int64_t)blockIdx.x * l1::kLines + (threadIdx.x >> 6);
  if (line >= lines) return;   // whole waves; the kernel has no barrier
  const float* xl = x + line * N;
  float xv[J];
#pragma unroll
  for (int j = 0; j < J; ++j) xv[j] = xl[lane + 64 * j];
  float2 S[J / 2 + 1];
#pragma unroll
  for (int r = 0; r <= J / 2; ++r) {
    float2 sr = make_float2(0.f, 0.f);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const float2 t = twiddle_any((r * j) % J, J);
      sr.x = fmaf(xv[j], t.x, sr.x);
      sr.y = fmaf(-xv[j], t.y, sr.y);
    }
    S[r] = sr;
  }
  const float2 wl = twiddle_any(lane, N);         // e^{+2 pi i l / N}
  const float2 step = make_float2(wl.x, -wl.y);   // e^{-2 pi i l / N}
  float2 p = make_float2(1.f, 0.f);               // e^{-2 pi i k l / N}
  float v[2 * l1::kMaxM];
#pragma unroll
  for (int k = 0; k < l1::kMaxM; ++k) {
    const int r = k % J;
    const float2 sk = r <= J / 2 ? S[r] : make_float2(S[J - r].x, -S[J - r].y);
    const float2 a = cmul(p, sk);
    v[2 * k] = a.x;
    v[2 * k + 1] = a.y;
    p = cmul(p, step);
  }
  // reduce-scatter: after the exchange over lane bit b the lane keeps the half
  // of its values selected by that bit; the last exchange (bit 0) completes
  // the sum of value 16 b5 + 8 b4 + 4 b3 + 2 b2 + b1
#pragma unroll
  for (int h = 16, bit = 32; h >= 1; h >>= 1, bit >>= 1) {
    const bool up = (lane & bit) != 0;
#pragma unroll
    for (int i = 0; i < h; ++i) {
      // the empty asm keeps the two selects on values: folded into one select
      // of the array index they become a lane-varying index into v[], which
      // lowers to compare-and-select chains over the whole array
      float lo = v[i], hi = v[h + i];
      asm volatile("" : "+v"(lo), "+v"(hi));
      const float send = up ? lo : hi;
      const float keep = up ? hi : lo;
      v[i] = keep + __shfl_xor(send, bit, 64);
    }
  }
  float t = v[0] + __shfl_xor(v[0], 1, 64);
  const int idx = lane >> 1;   // 2 k + (0 re | 1 im)
  if (!(lane & 1) && idx < 2 * m)
    reinterpret_cast<float*>(xhat)[line * 2 * m + idx] = t * scale;
}

// v[jj] = bo + sum_k Re(q_k e^{2 pi i k j / J}), j = H J / 2 + jj: the table
// index k j mod J is a compile-time constant
template <int J, int H>
__device__ __forceinline__ void line_synth_half(const float2 (&q)[l1::kMaxM], float bo,
                                                float (&v)[J / 2]) {
#pragma unroll
  for (int jj = 0; jj < J / 2; ++jj) {
    float a = bo;
#pragma unroll
    for (int k = 0; k < l1::kMaxM; ++k) {
      const float2 t = twiddle_any((k * (jj + H * J / 2)) % J, J);
      a = fmaf(q[k].x, t.x, a);
      a = fmaf(-q[k].y, t.y, a);
    }
    v[jj] = a;
  }
}

// y[b, o, n] for kOut output channels o of sample b:
//   Y[o][k] = sum_c X[b][c][k] W[c][o][k]
//   y = act( bias[o] + s sum_k c_k Re(Y[o][k] e^{2 pi i k n / N}) + skip(x)[b, o, n] )
// (c_0 = 1, c_k = 2: m <= N / 2 - 1 keeps the Nyquist bin out; the imaginary
// part of the DC bin meets sin 0).  Skip: none, identity or soft-gating.
// Wave w: output channel o0 + w % 4, points n = l + 64 j with j in the
// half w / 4 of 0 .. J - 1.
template <int N>
__global__ void __launch_bounds__(l1::kSynThreads)
k_line_synth(const float2* __restrict__ xhat, const float2* __restrict__ w,
             const float* __restrict__ bias, const float* __restrict__ x,
             const float* __restrict__ skip_w, float* __restrict__ y, int Ci, int Co, int m,
             int skip_kind, int act, float s) {
  constexpr int J = N / 64, JH = J / 2;
  __shared__ float2 yp[2][l1::kOut][l1::kMaxM];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ow = wave & 3, half = wave >> 2;
  const int groups = Co / l1::kOut;
  const int b = blockIdx.x / groups, o0 = l1::kOut * (blockIdx.x % groups);
  const int o = o0 + ow;
  // contraction: thread (o, k = lane % 16, part = 4 half + lane / 16) sums
  // the channels c = part + 8 i in chunks whose loads are all issued first;
  // then the sum over lane / 16 by exchanges and over the halves in LDS
  {
    const int k = lane & 15, part = 4 * half + (lane >> 4);
    float2 acc = make_float2(0.f, 0.f);
    if (k < m) {
      const float2* xb = xhat + (int64_t)b * Ci * m + k;
      const float2* wo = w + (int64_t)o * m + k;
      const int64_t ws = (int64_t)Co * m;
      for (int c0 = part; c0 < Ci; c0 += 8 * l1::kChunk) {
        float2 xv[l1::kChunk], wv[l1::kChunk];
#pragma unroll
        for (int u = 0; u < l1::kChunk; ++u) {
          const int c = c0 + 8 * u;
          xv[u] = c < Ci ? xb[(int64_t)c * m] : make_float2(0.f, 0.f);
          wv[u] = c < Ci ? wo[(int64_t)c * ws] : make_float2(0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < l1::kChunk; ++u) cfma(acc, xv[u], wv[u]);
      }
    }
    acc.x += __shfl_xor(acc.x, 16, 64);
    acc.y += __shfl_xor(acc.y, 16, 64);
    acc.x += __shfl_xor(acc.x, 32, 64);
    acc.y += __shfl_xor(acc.y, 32, 64);
    if (lane < 16) yp[half][ow][k] = acc;   // k >= m: zero
  }
  __syncthreads();
  // synthesis: q_k = c_k s Y_k e^{2 pi i k l / N}
  const float2 wl = twiddle_any(lane, N);
  float2 p = make_float2(1.f, 0.f);
  float2 q[l1::kMaxM];
#pragma unroll
  for (int k = 0; k < l1::kMaxM; ++k) {
    const float ck = (k == 0 ? 1.f : 2.f) * s;
    const float2 a = yp[0][ow][k], c = yp[1][ow][k];
    q[k] = cmul(make_float2(ck * (a.x + c.x), ck * (a.y + c.y)), p);
    p = cmul(p, wl);
  }
  const float bo = bias ? bias[o] : 0.f;
  const float g = skip_kind == FNO_SKIP_SOFT_GATING ? skip_w[o] : 1.f;
  const bool skip = skip_kind != FNO_SKIP_NONE;
  const uint32_t gmask = act_mask(act == FNO_ACT_GELU);
  // x rows exist for o < Ci only: the skips that read them have Ci == Co
  const float* xo = skip ? x + ((int64_t)b * Ci + o) * N + 64 * JH * half + lane : x;
  float* yo = y + ((int64_t)b * Co + o) * N + 64 * JH * half + lane;
  float xs[JH];
  if (skip) {
#pragma unroll
    for (int j = 0; j < JH; ++j) xs[j] = xo[64 * j];
  }
  float vo[JH];
  if (half == 0)
    line_synth_half<J, 0>(q, bo, vo);
  else
    line_synth_half<J, 1>(q, bo, vo);
#pragma unroll
  for (int j = 0; j < JH; ++j) {
    float v = vo[j];
    if (skip) v = fmaf(g, xs[j], v);
    yo[64 * j] = act_select(gelu_erf(v), v, gmask);
  }
}

bool line1d_supported(int Ci, int Co, int N, int m, int skip_kind) {
  if (!(N == 256 || N == 512 || N == 1024)) return false;
  if (m < 1 || m > l1::kMaxM || m > N / 2 - 1) return false;
  if (Ci < 1 || Co < l1::kOut || Co % l1::kOut != 0) return false;
  if (skip_kind == FNO_SKIP_LINEAR) return false;
  return skip_kind == FNO_SKIP_NONE || Ci == Co;
}

size_t line1d_workspace(int B, int Ci, int m) { return (size_t)B * Ci * m * sizeof(float2); }

int line1d_block(const float* x, const float2* w, const float* bias, const float* skip_w, float* y,
                 int B, int Ci, int Co, int N, int m, int norm, int skip_kind, int act, void* ws,
                 size_t ws_bytes, hipStream_t st) {
  if (ws_bytes < line1d_workspace(B, Ci, m)) {
    set_error("1D block: workspace %zu < %zu bytes", ws_bytes, line1d_workspace(B, Ci, m));
    return FNO_ERR_WORKSPACE;
  }
  const int32_t sz[1] = {N};
  const float fs = (float)forward_scale(norm, sz, 1);
  const float is = (float)inverse_scale(norm, sz, 1);
  float2* xhat = reinterpret_cast<float2*>(ws);
  const int64_t lines = (int64_t)B * Ci;
  const unsigned g1 = (unsigned)((lines + l1::kLines - 1) / l1::kLines);
  const unsigned g2 = (unsigned)((int64_t)B * (Co / l1::kOut));
#define FNO_L1(n)                                                                                  \
  if (N == n) {                                                                                    \
    hipLaunchKernelGGL(k_line_dft<n>, dim3(g1), dim3(l1::kThreads), 0, st, x, xhat, lines, m, fs); \
    int rc = launch_status("k_line_dft");                                                          \
    if (rc) return rc;                                                                             \
    hipLaunchKernelGGL(k_line_synth<n>, dim3(g2), dim3(l1::kSynThreads), 0, st, xhat, w, bias, x,  \
                       skip_w, y, Ci, Co, m, skip_kind, act, is);                                  \
    return launch_status("k_line_synth");                                                          \
  }
  FNO_L1(256) FNO_L1(512) FNO_L1(1024)
#undef FNO_L1
  set_error("1D block: unsupported N=%d", N);
  return FNO_ERR_UNSUPPORTED;
}

bool fast1d_supported(int Ci, int Co, int N, int m) {
  if (!(N == 256 || N == 512 || N == 1024)) return false;
  if (m < 1 || m > f1::kMaxM || 2 * m > N) return false;
  if (!(Ci == 32 || Ci == 64)) return false;
  return Co >= 16 && Co % 16 == 0;
}

int fast1d_block(const float* x, const float2* w, const float* bias, const float* skip_w, float* y,
                 int B, int Ci, int Co, int N, int m, int norm, int skip_kind, int act,
                 hipStream_t st) {
  const int32_t sz[1] = {N};
  const float fs = (float)forward_scale(norm, sz, 1);
  const float is = (float)inverse_scale(norm, sz, 1);
  const dim3 grid((unsigned)((int64_t)B * (Co / 16)));
  const bool xs = skip_kind != FNO_SKIP_NONE;
  // F fragments, later the two partial spectra (2 x Ci x 32 floats)
  const size_t lds = std::max((size_t)(N / 32) * 2 * 2 * 64 * 16, (size_t)2 * Ci * 33 * 4);
#define FNO_1D(ci, skip)                                                                           \
  if (Ci == ci && xs == skip) {                                                                    \
    if (lds > 64 * 1024) {                                                                         \
      int rc = hip_status(                                                                         \
          hipFuncSetAttribute(reinterpret_cast<const void*>(k_conv1d_fused<ci, skip>),             \
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),               \
          "hipFuncSetAttribute(MaxDynamicSharedMemorySize)");                                      \
      if (rc) return rc;                                                                           \
    }                                                                                              \
    hipLaunchKernelGGL((k_conv1d_fused<ci, skip>), grid, dim3(f1::kThreads), lds, st, x, w, bias, \
                       skip_w, y, N, m, Co, skip_kind, act, fs, is);                               \
    return launch_status("k_conv1d_fused");                                                        \
  }
  FNO_1D(32, false) FNO_1D(32, true) FNO_1D(64, false) FNO_1D(64, true)
#undef FNO_1D
  set_error("fused 1D block: unsupported Ci=%d", Ci);
  return FNO_ERR_UNSUPPORTED;
}

}  // namespace fno
