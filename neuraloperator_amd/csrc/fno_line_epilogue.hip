// Last-axis epilogue of an N-D spectral block for lines of 64 points: the
// inverse real DFT of each line, the bias, the skip and the activation as one
// matrix product per line on the matrix cores,
//
//   y[o, p] = act( sum_s Zt[o, s] T[s, p]  +  sum_c Ws[o, c] x[c, p] ),
//
// where Z is the block's spectrum after the inverse transforms of every axis
// but the last (window bins kw < m2h of the line, unscaled), so the full
// spectral field never goes through memory.  The K slots s of Zt / T:
//   s < 28:  bin kw = 1 + s / 2, Re (s even) / Im (s odd) of Z, against
//            c_kw t cos(2 pi kw p / 64) / -c_kw t sin(..) (c_kw = 2 for bins
//            that stand for a conjugate pair, 1 at the Nyquist bin 32; t the
//            inverse norm scale),
//   s = 28:  Re Z[kw = 0] against t (the DC bin; its imaginary part meets
//            sin 0 = 0),
//   s = 29:  bias[o] against 1,
// all in one k-step of 32; the skip is Ws (the 1x1 conv), diag(g)
// (soft-gating) or the identity, in k-steps of 32 input channels.
//
// Semantics: the last-axis irfft + bias of SpectralConv.forward
// (neuralop/layers/spectral_convolution.py:547-568) and the skip add and
// activation of FNOBlocks.forward_with_postactivation (neuralop/layers/
// fno_block.py:331-361, skips of skip_connections.py:88-130).
//
// Arithmetic: three-term bf16 splits on v_mfma_f32_16x16x32_bf16 with fp32
// accumulation, as in the fused 2D row epilogue (each product within
// 3 * 2^-16 of |a b|).  Work: each wave takes lines of one sample in turn, all
// output channels of a line: tiles of 16 channels x 16 pixels, where column n
// of pixel tile pt is pixel 4 n + pt, so a lane loads and stores four
// consecutive pixels of a channel as one 16-byte access.  No LDS, no barriers.
#include "fno_common.h"
#include "fno_twiddle.h"

namespace fno {

namespace le {
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kW = 64;                 // line length
constexpr int kWaves = 4, kThreads = 64 * kWaves;
constexpr int kMaxBins = 15;           // kw < 15: 28 slots of bins 1..14
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
}  // namespace le

// CO output channels (2 or 4 tiles of 16), CI input channels of the skip (k-
// steps of 32; CI == CO for soft-gating / identity), XSKIP: a skip at all.
// Lines: B samples x L lines per channel plane; wave v of the grid takes the
// lines [v * LPW, (v + 1) * LPW) of the flattened (b, line) order.
template <int CO, int CI, bool XSKIP>
__global__ void __launch_bounds__(le::kThreads)
k_line_epilogue(const float2* __restrict__ z, const float* __restrict__ x,
                const float* __restrict__ skip_w, const float* __restrict__ bias,
                float* __restrict__ y, int B, int64_t L, int m2h, int skip_kind, int act,
                float scale, int LPW) {
  using namespace le;
  constexpr int OT = CO / 16, KS = CI / 32;
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  const int G = lane >> 4, n = lane & 15;
  const int64_t total = (int64_t)B * L;
  int64_t l0 = wave * LPW;
  if (l0 >= total) return;
  const int64_t l1 = l0 + LPW < total ? l0 + LPW : total;
  const uint32_t gmask = act_mask(act == FNO_ACT_GELU);

  // synthesis table fragments (B operand of pixel tile pt): slot s = 8 G + i
  // against pixel p = 4 n + pt
  v8bf th[4], tl[4];
#pragma unroll
  for (int pt = 0; pt < 4; ++pt) {
    const int p = 4 * n + pt;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int s = 8 * G + i;
      float v = 0.f;
      if (s < 28) {
        const int kw = 1 + (s >> 1);
        if (kw < m2h) {
          const float c = (2 * kw == kW) ? scale : 2.f * scale;
          const float2 t = twiddle_any((kw * p) & (kW - 1), kW);
          v = (s & 1) ? -c * t.y : c * t.x;
        }
      } else if (s == 28) {
        v = scale;
      } else if (s == 29) {
        v = 1.f;
      }
      const bf2 q = split(v);
      th[pt][i] = q.hi;
      tl[pt][i] = q.lo;
    }
  }
  // skip operand A[o = 16 ot + m][c = 32 ks + 8 G + i]
  v8bf wh[OT][KS > 0 ? KS : 1], wl[OT][KS > 0 ? KS : 1];
  if constexpr (XSKIP) {
#pragma unroll
    for (int ot = 0; ot < OT; ++ot)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int o = 16 * ot + n, c = 32 * ks + 8 * G + i;
          float v;
          if (skip_kind == FNO_SKIP_LINEAR) v = skip_w[o * CI + c];
          else if (skip_kind == FNO_SKIP_SOFT_GATING) v = (c == o) ? skip_w[o] : 0.f;
          else v = (c == o) ? 1.f : 0.f;
          const bf2 q = split(v);
          wh[ot][ks][i] = q.hi;
          wl[ot][ks][i] = q.lo;
        }
  }
  float bo[OT];
#pragma unroll
  for (int ot = 0; ot < OT; ++ot) bo[ot] = bias ? bias[16 * ot + n] : 0.f;

  // Z of line l: lane (G, m) of tile ot holds channel 16 ot + m, bins
  // 1 + 4 G .. 4 + 4 G (slots 8 G .. 8 G + 7), and at G == 3 also the DC bin
  // and the bias in slots 28, 29.  Bins at or past m2h read as zero.
#pragma unroll 1
  for (int64_t l = l0; l < l1; ++l) {
    const int b = (int)(l / L);
    const int64_t line = l - (int64_t)b * L;
    v4f acc[OT][4];
#pragma unroll
    for (int ot = 0; ot < OT; ++ot)
#pragma unroll
      for (int pt = 0; pt < 4; ++pt) acc[ot][pt] = (v4f)0.f;
    // x operand loads first (the skip): channel 32 ks + 8 G + i, pixels 4n..4n+3
    float4 xv[KS > 0 ? KS : 1][8];
    if constexpr (XSKIP) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int i = 0; i < 8; ++i)
          xv[ks][i] = load_nt(x + (((int64_t)b * CI + 32 * ks + 8 * G + i) * L + line) * kW + 4 * n);
    }
#pragma unroll
    for (int ot = 0; ot < OT; ++ot) {
      const int o = 16 * ot + n;
      const float2* zl = z + (((int64_t)b * CO + o) * L + line) * m2h;
      float2 zv[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int kw = 1 + 4 * G + q;
        zv[q] = kw < m2h ? zl[kw] : make_float2(0.f, 0.f);
      }
      const float dc = zl[0].x;
      v8bf ah, al;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float v = (i & 1) ? zv[i >> 1].y : zv[i >> 1].x;
        if (G == 3) v = (i < 4) ? v : (i == 4) ? dc : (i == 5) ? bo[ot] : 0.f;
        const bf2 q = split(v);
        ah[i] = q.hi;
        al[i] = q.lo;
      }
#pragma unroll
      for (int pt = 0; pt < 4; ++pt) acc[ot][pt] = mma3(ah, al, th[pt], tl[pt], acc[ot][pt]);
    }
    if constexpr (XSKIP) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int pt = 0; pt < 4; ++pt) {
          v8bf bh, bl;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float v = pt == 0 ? xv[ks][i].x : pt == 1 ? xv[ks][i].y
                          : pt == 2 ? xv[ks][i].z : xv[ks][i].w;
            const bf2 q = split(v);
            bh[i] = q.hi;
            bl[i] = q.lo;
          }
#pragma unroll
          for (int ot = 0; ot < OT; ++ot)
            acc[ot][pt] = mma3(wh[ot][ks], wl[ot][ks], bh, bl, acc[ot][pt]);
        }
    }
    // D[o = 16 ot + 4 G + r][column n] of pixel tile pt is pixel 4 n + pt
#pragma unroll
    for (int ot = 0; ot < OT; ++ot)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float4 v;
        v.x = act_select(gelu_erf(acc[ot][0][r]), acc[ot][0][r], gmask);
        v.y = act_select(gelu_erf(acc[ot][1][r]), acc[ot][1][r], gmask);
        v.z = act_select(gelu_erf(acc[ot][2][r]), acc[ot][2][r], gmask);
        v.w = act_select(gelu_erf(acc[ot][3][r]), acc[ot][3][r], gmask);
        store_nt(y + (((int64_t)b * CO + 16 * ot + 4 * G + r) * L + line) * kW + 4 * n, v);
      }
  }
}

// ============================================================== host side
// Lines of 64 points, 32 or 64 output channels, a 1x1-conv skip over 32 or
// 64 input channels (or a gating / identity skip with CI == CO), at most
// 15 kept bins of the line.
bool line_epilogue_supported(int W, int Ci, int Co, int m2h, int skip_kind) {
  if (W != le::kW || m2h < 1 || m2h > le::kMaxBins) return false;
  if (!(Co == 32 || Co == 64)) return false;
  if (skip_kind == FNO_SKIP_LINEAR) return Ci == 32 || Ci == 64;
  if (skip_kind == FNO_SKIP_SOFT_GATING || skip_kind == FNO_SKIP_IDENTITY) return Ci == Co;
  return skip_kind == FNO_SKIP_NONE;
}

int line_epilogue(const float2* z, const float* x, const float* skip_w, const float* bias,
                  float* y, int B, int Ci, int Co, int64_t L, int m2h, int skip_kind, int act,
                  float scale, hipStream_t st) {
  const int64_t lines = (int64_t)B * L;
  // about 8 waves per CU in flight, a handful of lines each
  int LPW = (int)((lines + 8 * 256 * 2 - 1) / (8 * 256 * 2));
  if (LPW < 1) LPW = 1;
  const int64_t waves = (lines + LPW - 1) / LPW;
  const unsigned grid = (unsigned)((waves + le::kWaves - 1) / le::kWaves);
  const int ci = skip_kind == FNO_SKIP_LINEAR ? Ci : Co;
#define FNO_LE(co, cin, xs)                                                                       \
  if (Co == co && ci == cin && (skip_kind != FNO_SKIP_NONE) == xs) {                             \
    hipLaunchKernelGGL((k_line_epilogue<co, cin, xs>), dim3(grid), dim3(le::kThreads), 0, st, z,  \
                       x, skip_w, bias, y, B, L, m2h, skip_kind, act, scale, LPW);               \
    return launch_status("k_line_epilogue");                                                      \
  }
  FNO_LE(32, 32, true) FNO_LE(32, 64, true) FNO_LE(64, 32, true) FNO_LE(64, 64, true)
  FNO_LE(32, 32, false) FNO_LE(64, 64, false)
#undef FNO_LE
  set_error("line epilogue: unsupported Ci=%d Co=%d skip=%d", Ci, Co, skip_kind);
  return FNO_ERR_UNSUPPORTED;
}

}  // namespace fno
