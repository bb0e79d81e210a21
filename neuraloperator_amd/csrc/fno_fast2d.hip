// Fused 2D spectral block for power-of-two planes (H in {64,128,256},
// W in {128,256}):
//
//   y = act( irfft2_window( contract( rfft2_window(x) ) ) + bias + skip(x) )
//
// K1  k_fwd_plane      one workgroup per (b, c) plane: row real FFTs (two real
//                      rows packed as one complex line) keep m2h bins in an LDS
//                      plane buffer; column FFTs then emit only the m1 kept rows,
//                      already in window (fftshift-ed) order, scaled.
// K2  contraction      fno_generic.hip (mode-wise complex GEMM).
// K3  k_inv_cols       one workgroup per (b, o) plane: inverse column FFTs of
//                      the m2h kept columns from the m1 window rows, staged in
//                      LDS and written as Z[b,o,h,kw] with coalesced stores.
// K4  k_row_epilogue   one workgroup per (b, h) output row: inverse row real
//                      FFTs of Z for every output channel (two channels packed
//                      per complex line), the 1x1-conv skip on fp32 MFMA
//                      (v_mfma_f32_32x32x2f32, accumulators = skip result),
//                      bias and exact erf GELU, one write of y.
//
// Semantics follow SpectralConv.forward (neuralop/layers/spectral_convolution.py
// :429-568) with output size == input size, and the post-activation block of
// FNOBlocks (neuralop/layers/fno_block.py:331-361).
#include "fno_fft_lds.h"

namespace fno {

typedef float v16f __attribute__((ext_vector_type(16)));

template <int N>
__device__ __forceinline__ void fill_twiddles(float2* tw) {
  for (int i = threadIdx.x; i < N; i += blockDim.x) tw[i] = twiddle_pos(i, N);
}

// ------------------------------------------------------------------------ K1
template <int H, int W, int BLOCK>
__global__ void __launch_bounds__(BLOCK)
k_fwd_plane(const float* __restrict__ x, float2* __restrict__ xhat, int m1, int m2h, int TS,
            float scale) {
  using PW = LinePlan<W>;
  using PH = LinePlan<H>;
  extern __shared__ float4 smem4[];
  float2* twW = reinterpret_cast<float2*>(smem4);
  float2* twH = twW + W;
  float2* plane = twH + H;                 // [H][TS]
  float2* exall = plane + H * TS;          // per-group exchange slices
  fill_twiddles<W>(twW);
  fill_twiddles<H>(twH);
  __syncthreads();

  const float* xp = x + (int64_t)blockIdx.x * H * W;
  // ---- rows: pairs (2r, 2r+1) packed as one complex line
  {
    constexpr int T = PW::T, R = PW::R, Q = PW::Q;
    constexpr int G = BLOCK / T;
    const int g = threadIdx.x / T, t = threadIdx.x % T;
    float2* ex = exall + g * W;
    for (int pr = g; pr < H / 2; pr += G) {
      const float* ra = xp + (2 * pr) * W;
      const float* rb = ra + W;
      float2 v[R];
#pragma unroll
      for (int s = 0; s < R; ++s) v[s] = make_float2(ra[t + T * s], rb[t + T * s]);
      float2 out[Q][T];
      line_fft<W, -1>(v, ex, twW, t, out);
      // Z[k] in natural order for the bins the split needs
#pragma unroll
      for (int q = 0; q < Q; ++q)
#pragma unroll
        for (int s = 0; s < T; ++s) {
          const int k = t + T * q + R * s;
          if (k < m2h || k > W - m2h) ex[k] = out[q][s];
        }
      wave_sync();
      // X_a[k] = (Z[k] + conj Z[W-k]) / 2,  X_b[k] = -i (Z[k] - conj Z[W-k]) / 2
      for (int k = t; k < m2h; k += T) {
        const float2 zk = ex[k];
        const float2 zn = ex[(W - k) & (W - 1)];
        const float2 xa = make_float2(0.5f * (zk.x + zn.x), 0.5f * (zk.y - zn.y));
        const float2 xb = make_float2(0.5f * (zk.y + zn.y), 0.5f * (zn.x - zk.x));
        plane[(2 * pr) * TS + k] = xa;
        plane[(2 * pr + 1) * TS + k] = xb;
      }
      wave_sync();
    }
  }
  __syncthreads();
  // ---- columns: kept bins only, emit kept rows in window order
  {
    constexpr int T = PH::T, R = PH::R, Q = PH::Q;
    constexpr int G = BLOCK / T;
    const int g = threadIdx.x / T, t = threadIdx.x % T;
    float2* ex = exall + g * H;
    float2* op = xhat + (int64_t)blockIdx.x * m1 * m2h;
    const int pos = m1 - m1 / 2;  // kept non-negative frequencies 0..pos-1
    const int neg = m1 / 2;       // kept negative frequencies -neg..-1
    for (int kw = g; kw < m2h; kw += G) {
      float2 v[R];
#pragma unroll
      for (int s = 0; s < R; ++s) v[s] = plane[(t + T * s) * TS + kw];
      float2 out[Q][T];
      line_fft<H, -1>(v, ex, twH, t, out);
#pragma unroll
      for (int q = 0; q < Q; ++q)
#pragma unroll
        for (int s = 0; s < T; ++s) {
          const int k = t + T * q + R * s;
          int j = -1;
          if (k < pos) j = k + neg;
          else if (k >= H - neg) j = k - H + neg;
          if (j >= 0) op[j * m2h + kw] = cscale(out[q][s], scale);
        }
    }
  }
}

// ------------------------------------------------------------------------ K3
template <int H, int BLOCK>
__global__ void __launch_bounds__(BLOCK)
k_inv_cols(const float2* __restrict__ yhat, float2* __restrict__ z, int m1, int m2h, int TS) {
  using PH = LinePlan<H>;
  extern __shared__ float4 smem4[];
  float2* twH = reinterpret_cast<float2*>(smem4);
  float2* zs = twH + H;                   // [H][TS]
  float2* exall = zs + H * TS;            // groups x H
  fill_twiddles<H>(twH);
  const float2* win = yhat + (int64_t)blockIdx.x * m1 * m2h;   // [m1][m2h] window
  __syncthreads();
  {
    constexpr int T = PH::T, R = PH::R, Q = PH::Q;
    constexpr int G = BLOCK / T;
    const int g = threadIdx.x / T, t = threadIdx.x % T;
    float2* ex = exall + g * H;
    const int pos = m1 - m1 / 2, neg = m1 / 2;
    for (int kw = g; kw < m2h; kw += G) {
      float2 v[R];
#pragma unroll
      for (int s = 0; s < R; ++s) {
        const int k = t + T * s;  // frequency index mod H
        int j = -1;
        if (k < pos) j = k + neg;
        else if (k >= H - neg) j = k - H + neg;
        v[s] = (j >= 0) ? win[j * m2h + kw] : make_float2(0.f, 0.f);
      }
      float2 out[Q][T];
      line_fft<H, +1>(v, ex, twH, t, out);
#pragma unroll
      for (int q = 0; q < Q; ++q)
#pragma unroll
        for (int s = 0; s < T; ++s) zs[(t + T * q + R * s) * TS + kw] = out[q][s];
    }
  }
  __syncthreads();
  float2* zp = z + (int64_t)blockIdx.x * H * m2h;
  for (int i = threadIdx.x; i < H * m2h; i += BLOCK) {
    const int h = i / m2h, kw = i - h * m2h;
    zp[i] = zs[h * TS + kw];
  }
}

// ------------------------------------------------------------------------ K4
// MFMA 32x32x2 f32 operand/result layout (wave64):
//   A (32 x 2):  lane l supplies A[l % 32][l / 32]
//   B (2 x 32):  lane l supplies B[l / 32][l % 32]
//   D (32 x 32): lane l, register r holds D[8*(r/4) + 4*(l/32) + r%4][l % 32]
// Here M = output pixels of the row, N = output channels, K = input channels.
template <int W, int CO>
__global__ void __launch_bounds__(256)
k_row_epilogue(const float* __restrict__ x, const float2* __restrict__ z,
               const float* __restrict__ skip_w, const float* __restrict__ bias,
               float* __restrict__ y, int H, int Ci, int m2h, int skip_kind, int act,
               float inv_scale) {
  using PW = LinePlan<W>;
  constexpr int MT = W / 4 / 32;       // 32-pixel tiles per wave
  constexpr int NT = CO / 32;          // 32-channel tiles
  constexpr int AST = W + 4;           // LDS row stride of the irfft chunk
  static_assert(MT >= 1, "row too short for the wave tiling");
  extern __shared__ float4 smem4[];
  float2* twW = reinterpret_cast<float2*>(smem4);
  float* wsk = reinterpret_cast<float*>(twW + W);          // [CO][Ci] skip weight
  float* achunk = wsk + (skip_kind == FNO_SKIP_LINEAR ? CO * Ci : 0);  // [32][AST]

  const int b = blockIdx.x / H, h = blockIdx.x % H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int p_wave = wave * (W / 4);
  fill_twiddles<W>(twW);
  if (skip_kind == FNO_SKIP_LINEAR)
    for (int i = threadIdx.x; i < CO * Ci; i += 256) wsk[i] = skip_w[i];
  __syncthreads();

  v16f acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mt][nt][r] = 0.f;

  const int64_t HW = (int64_t)H * W;
  const float* xb = x + (int64_t)b * Ci * HW + (int64_t)h * W;
  if (skip_kind == FNO_SKIP_LINEAR) {
    const int kk = lane >> 5, mm = lane & 31;
    for (int i0 = 0; i0 < Ci; i0 += 2) {
      float a[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) a[mt] = xb[(int64_t)(i0 + kk) * HW + p_wave + 32 * mt + mm];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const float bv = wsk[(32 * nt + mm) * Ci + i0 + kk];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[mt], bv, acc[mt][nt], 0, 0, 0);
      }
    }
  } else if (skip_kind == FNO_SKIP_SOFT_GATING || skip_kind == FNO_SKIP_IDENTITY) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int o = 32 * nt + (lane & 31);
      const float gate = (skip_kind == FNO_SKIP_SOFT_GATING) ? skip_w[o] : 1.f;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int p = p_wave + 32 * mt + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          acc[mt][nt][r] = gate * xb[(int64_t)o * HW + p];
        }
    }
  }

  // ---- inverse row FFTs, 32 output channels (16 packed pairs) per chunk
  constexpr int T = PW::T, R = PW::R, Q = PW::Q;
  constexpr int G = 256 / T;
  const int g = threadIdx.x / T, t = threadIdx.x % T;
  const float2* zb = z + ((int64_t)b * CO * H + h) * m2h;   // + o*H*m2h
  const int64_t zo = (int64_t)H * m2h;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    if (g < 16) {
      const int oa = 32 * nt + 2 * g;
      float* slot = achunk + (2 * g) * AST;
      float2* ex = reinterpret_cast<float2*>(slot);
      const float2* za = zb + oa * zo;
      const float2* zbb = za + zo;
      // Z2[k] = Ya[k] + i Yb[k] extended with Hermitian symmetry; imaginary
      // parts of bin 0 and bin W/2 are dropped (irfft semantics)
      float2 v[R];
#pragma unroll
      for (int s = 0; s < R; ++s) {
        const int k = t + T * s;
        float2 val = make_float2(0.f, 0.f);
        if (k < m2h) {
          float2 ya = za[k], yb = zbb[k];
          if (k == 0 || 2 * k == W) {
            ya.y = 0.f;
            yb.y = 0.f;
          }
          val = make_float2(ya.x - yb.y, ya.y + yb.x);
        } else if (k > W / 2 && W - k < m2h) {
          const float2 ya = za[W - k], yb = zbb[W - k];
          // conj(ya) + i conj(yb)
          val = make_float2(ya.x + yb.y, yb.x - ya.y);
        }
        v[s] = val;
      }
      float2 out[Q][T];
      line_fft<W, +1>(v, ex, twW, t, out);
#pragma unroll
      for (int q = 0; q < Q; ++q)
#pragma unroll
        for (int s = 0; s < T; ++s) {
          const int p = t + T * q + R * s;
          slot[p] = out[q][s].x * inv_scale;
          slot[AST + p] = out[q][s].y * inv_scale;
        }
    }
    __syncthreads();
    {
      const int o = 32 * nt + (lane & 31);
      const float bo = bias ? bias[o] : 0.f;
      const float* arow = achunk + (lane & 31) * AST;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int p = p_wave + 32 * mt + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          float v = acc[mt][nt][r] + arow[p] + bo;
          if (act == FNO_ACT_GELU) v = gelu_erf(v);
          acc[mt][nt][r] = v;
        }
    }
    __syncthreads();
  }
  // ---- store y[b, o, h, p]: four consecutive pixels per register group
  float* yb = y + (int64_t)b * CO * HW + (int64_t)h * W;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int o = 32 * nt + (lane & 31);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int p = p_wave + 32 * mt + 8 * r4 + 4 * (lane >> 5);
        float4 v = make_float4(acc[mt][nt][4 * r4], acc[mt][nt][4 * r4 + 1], acc[mt][nt][4 * r4 + 2],
                               acc[mt][nt][4 * r4 + 3]);
        *reinterpret_cast<float4*>(yb + (int64_t)o * HW + p) = v;
      }
  }
}

// ============================================================== host side
int contract_dense(const float2* X, const float2* W, float2* Y, int B, int Ci, int Co, int64_t M,
                   int64_t sWi, int64_t sWo, int64_t sWk, hipStream_t st);

static constexpr size_t kMaxLds = 160 * 1024;

static int line_lanes(int n) { return n >= 256 ? 16 : 8; }
static int fwd_block(int H, int W) { return (H >= 256 || W >= 256) ? 512 : 256; }
static int inv_block(int H) { return H >= 256 ? 512 : 256; }

static size_t fwd_lds_bytes(int H, int W, int m2h) {
  const int blk = fwd_block(H, W);
  const int exW = blk / line_lanes(W) * W, exH = blk / line_lanes(H) * H;
  const int TS = m2h | 1;
  return (size_t)(W + H + H * TS + (exW > exH ? exW : exH)) * sizeof(float2);
}
static size_t inv_lds_bytes(int H, int m2h) {
  const int TS = m2h | 1;
  return (size_t)(H + H * TS + inv_block(H) / line_lanes(H) * H) * sizeof(float2);
}
static size_t epi_lds_bytes(int W, int Co, int Ci, int skip_kind) {
  return (size_t)W * sizeof(float2) +
         (size_t)(skip_kind == FNO_SKIP_LINEAR ? Co * Ci : 0) * sizeof(float) +
         (size_t)32 * (W + 4) * sizeof(float);
}

bool fast2d_supported(int B, int Ci, int Co, int ndim, const int32_t* sizes, const int32_t* modes,
                      int skip_kind) {
  if (ndim != 2 || B < 1) return false;
  const int H = sizes[0], W = sizes[1];
  if (!(H == 64 || H == 128 || H == 256)) return false;
  if (!(W == 128 || W == 256)) return false;
  if (!(Co == 32 || Co == 64 || Co == 96 || Co == 128)) return false;
  if (skip_kind == FNO_SKIP_LINEAR && (Ci % 2 != 0 || Ci < 2)) return false;
  if ((skip_kind == FNO_SKIP_IDENTITY || skip_kind == FNO_SKIP_SOFT_GATING) && Ci != Co)
    return false;
  if (modes[0] < 1 || modes[0] > H || modes[1] < 1 || modes[1] > W / 2 + 1) return false;
  if (fwd_lds_bytes(H, W, modes[1]) > kMaxLds) return false;
  if (inv_lds_bytes(H, modes[1]) > kMaxLds) return false;
  if (epi_lds_bytes(W, Co, Ci, skip_kind) > kMaxLds) return false;
  return true;
}

size_t fast2d_workspace(int B, int Ci, int Co, const int32_t* sizes, const int32_t* modes) {
  const int64_t M = (int64_t)modes[0] * modes[1];
  const int64_t e = (int64_t)B * Ci * M + (int64_t)B * Co * M + (int64_t)B * Co * sizes[0] * modes[1];
  return (size_t)e * sizeof(float2);
}

// Kernels taking more than 64 KB of dynamic LDS get the limit raised once.
template <typename K>
static int allow_lds(K kernel, size_t bytes) {
  if (bytes <= 64 * 1024) return FNO_OK;
  return hip_status(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes),
                    "hipFuncSetAttribute(MaxDynamicSharedMemorySize)");
}

template <int H, int W>
static int launch_fwd(const float* x, float2* xhat, int64_t planes, int m1, int m2h, float scale,
                      hipStream_t st) {
  constexpr int BLOCK = (H >= 256 || W >= 256) ? 512 : 256;
  const int TS = m2h | 1;
  const size_t lds = fwd_lds_bytes(H, W, m2h);
  int rc = allow_lds(k_fwd_plane<H, W, BLOCK>, lds);
  if (rc) return rc;
  hipLaunchKernelGGL((k_fwd_plane<H, W, BLOCK>), dim3((unsigned)planes), dim3(BLOCK), lds, st, x,
                     xhat, m1, m2h, TS, scale);
  return launch_status("k_fwd_plane");
}

template <int H>
static int launch_inv(const float2* yhat, float2* zbuf, int64_t planes, int m1, int m2h,
                      hipStream_t st) {
  constexpr int BLOCK = (H >= 256) ? 512 : 256;
  const int TS = m2h | 1;
  const size_t lds = inv_lds_bytes(H, m2h);
  int rc = allow_lds(k_inv_cols<H, BLOCK>, lds);
  if (rc) return rc;
  hipLaunchKernelGGL((k_inv_cols<H, BLOCK>), dim3((unsigned)planes), dim3(BLOCK), lds, st, yhat,
                     zbuf, m1, m2h, TS);
  return launch_status("k_inv_cols");
}

template <int W, int CO>
static int launch_epi(const float* x, const float2* zbuf, const float* skip_w, const float* bias,
                      float* y, int B, int H, int Ci, int m2h, int skip_kind, int act,
                      float inv_scale, hipStream_t st) {
  const size_t lds = epi_lds_bytes(W, CO, Ci, skip_kind);
  int rc = allow_lds(k_row_epilogue<W, CO>, lds);
  if (rc) return rc;
  hipLaunchKernelGGL((k_row_epilogue<W, CO>), dim3((unsigned)(B * H)), dim3(256), lds, st, x, zbuf,
                     skip_w, bias, y, H, Ci, m2h, skip_kind, act, inv_scale);
  return launch_status("k_row_epilogue");
}

static int dispatch_fwd(int H, int W, const float* x, float2* xhat, int64_t planes, int m1, int m2h,
                        float scale, hipStream_t st) {
#define FNO_FWD(h, w) \
  if (H == h && W == w) return launch_fwd<h, w>(x, xhat, planes, m1, m2h, scale, st);
  FNO_FWD(64, 128) FNO_FWD(128, 128) FNO_FWD(256, 128)
  FNO_FWD(64, 256) FNO_FWD(128, 256) FNO_FWD(256, 256)
#undef FNO_FWD
  set_error("fused 2D forward: unsupported plane %dx%d", H, W);
  return FNO_ERR_UNSUPPORTED;
}

static int dispatch_inv(int H, const float2* yhat, float2* zbuf, int64_t planes, int m1, int m2h,
                        hipStream_t st) {
  if (H == 64) return launch_inv<64>(yhat, zbuf, planes, m1, m2h, st);
  if (H == 128) return launch_inv<128>(yhat, zbuf, planes, m1, m2h, st);
  if (H == 256) return launch_inv<256>(yhat, zbuf, planes, m1, m2h, st);
  set_error("fused 2D inverse: unsupported H=%d", H);
  return FNO_ERR_UNSUPPORTED;
}

static int dispatch_epi(int W, int Co, const float* x, const float2* zbuf, const float* skip_w,
                        const float* bias, float* y, int B, int H, int Ci, int m2h, int skip_kind,
                        int act, float inv_scale, hipStream_t st) {
#define FNO_EPI(w, co)                                                                        \
  if (W == w && Co == co)                                                                     \
    return launch_epi<w, co>(x, zbuf, skip_w, bias, y, B, H, Ci, m2h, skip_kind, act, inv_scale, \
                             st);
  FNO_EPI(128, 32) FNO_EPI(128, 64) FNO_EPI(128, 96) FNO_EPI(128, 128)
  FNO_EPI(256, 32) FNO_EPI(256, 64) FNO_EPI(256, 96) FNO_EPI(256, 128)
#undef FNO_EPI
  set_error("fused 2D epilogue: unsupported W=%d Co=%d", W, Co);
  return FNO_ERR_UNSUPPORTED;
}

int fast2d_block(const float* x, const float2* w, const float* bias, const float* skip_w, float* y,
                 int B, int Ci, int Co, const int32_t* sizes, const int32_t* modes, int norm,
                 int skip_kind, int act, void* ws, size_t ws_bytes, hipStream_t st) {
  const int H = sizes[0], W = sizes[1], m1 = modes[0], m2h = modes[1];
  const int64_t M = (int64_t)m1 * m2h;
  const size_t need = fast2d_workspace(B, Ci, Co, sizes, modes);
  if (ws_bytes < need) {
    set_error("fused 2D block: workspace %zu < %zu bytes", ws_bytes, need);
    return FNO_ERR_WORKSPACE;
  }
  float2* xhat = reinterpret_cast<float2*>(ws);
  float2* yhat = xhat + (int64_t)B * Ci * M;
  float2* zbuf = yhat + (int64_t)B * Co * M;
  const int32_t sz[2] = {H, W};
  const float fscale = (float)forward_scale(norm, sz, 2);
  const float iscale = (float)inverse_scale(norm, sz, 2);
  int rc = dispatch_fwd(H, W, x, xhat, (int64_t)B * Ci, m1, m2h, fscale, st);
  if (rc) return rc;
  rc = contract_dense(xhat, w, yhat, B, Ci, Co, M, (int64_t)Co * M, M, 1, st);
  if (rc) return rc;
  rc = dispatch_inv(H, yhat, zbuf, (int64_t)B * Co, m1, m2h, st);
  if (rc) return rc;
  return dispatch_epi(W, Co, x, zbuf, skip_w, bias, y, B, H, Ci, m2h, skip_kind, act, iscale, st);
}

}  // namespace fno
