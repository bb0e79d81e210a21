// Generic kernels of the FNO spectral path: any spatial size (up to 4096 per
// axis), 1-3 spatial dims, any mode window.  Each spatial axis is handled by a
// direct pruned DFT (only the kept frequencies are computed, O(N*m) per line),
// which is the right tool when m << N or N is not a power of two; the last
// axis of 64-, 128- and 256-point lines goes through line FFTs instead
// (fno_generic_fft.hip), and the fused 2D kernels in fno_fast2d.hip take over
// for large power-of-two planes.
//
// Frequency bookkeeping follows SpectralConv.forward
// (neuralop/layers/spectral_convolution.py:429-568):
//   forward  window index j on a non-last axis holds frequency j - m/2
//            (rfftn + fftshift + centred slice, :443-449, :500-519);
//            on the last axis it holds frequency j (rfft half spectrum)
//   inverse  ifftshift + ifftn(s = N') puts frequency f at index t = f mod N of
//            the length-N spectrum and then zero-pads / truncates at the end,
//            so the entry contributes exp(+2 pi i t n / N') iff t < N' (:531-548)
//   last     irfft(n = N') with the imaginary parts of bin 0 (and of bin N/2
//            when N' is even, enforce_hermitian_symmetry) zeroed (:550-559)
#include "fno_common.h"
#include "fno_twiddle.h"

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <string>

namespace fno {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return FNO_OK;
  set_error("%s: %s", what, hipGetErrorString(e));
  return FNO_ERR_HIP;
}

int launch_status(const char* what) { return hip_status(hipGetLastError(), what); }

const char* last_error_cstr() { return g_last_error.c_str(); }
void clear_error() { g_last_error.clear(); }

static double prod_sizes(const int32_t* s, int n) {
  double p = 1.0;
  for (int i = 0; i < n; ++i) p *= (double)s[i];
  return p;
}

double forward_scale(int norm, const int32_t* in_sizes, int ndim) {
  double p = prod_sizes(in_sizes, ndim);
  if (norm == FNO_NORM_FORWARD) return 1.0 / p;
  if (norm == FNO_NORM_ORTHO) return 1.0 / std::sqrt(p);
  return 1.0;
}

double inverse_scale(int norm, const int32_t* out_sizes, int ndim) {
  double p = prod_sizes(out_sizes, ndim);
  if (norm == FNO_NORM_BACKWARD) return 1.0 / p;
  if (norm == FNO_NORM_ORTHO) return 1.0 / std::sqrt(p);
  return 1.0;
}

static constexpr int kMaxAxis = 4096;
static constexpr int kThreads = 256;

// --------------------------------------------------------------- forward axes
// Last axis, real -> complex:  out[r, j] = s * sum_n x[r, n] exp(-2 pi i j n / N)
__global__ void __launch_bounds__(kThreads)
k_r2c_direct(const float* __restrict__ x, float2* __restrict__ out, int64_t rows, int N, int m,
             int rows_per_block, float scale) {
  // a (row, bin) task is summed by 16 lanes over n = lane, lane + 16, ...
  // and reduced across them
  constexpr int L = 16;
  extern __shared__ float smem[];
  float2* tw = reinterpret_cast<float2*>(smem);
  float* xs = reinterpret_cast<float*>(tw + N);
  for (int t = threadIdx.x; t < N; t += blockDim.x) tw[t] = twiddle_any(t, N);
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  const int nr = (int)min((int64_t)rows_per_block, rows - r0);
  const float* xg = x + r0 * N;
  for (int t = threadIdx.x; t < nr * N; t += blockDim.x) xs[t] = xg[t];
  __syncthreads();
  const int sub = threadIdx.x % L;
  // every lane runs the same number of passes so the shuffles stay converged
  const int passes = (nr * m + kThreads / L - 1) / (kThreads / L);
  for (int pass = 0; pass < passes; ++pass) {
    const int task = pass * (kThreads / L) + threadIdx.x / L;
    const bool live = task < nr * m;
    const int rr = live ? task / m : 0, j = live ? task % m : 0;
    const float* xr = xs + rr * N;
    float re = 0.f, im = 0.f;
    if (live) {
      int idx = (int)(((int64_t)j * sub) % N);
      const int step = (int)(((int64_t)j * L) % N);
      for (int n = sub; n < N; n += L) {
        const float2 w = tw[idx];
        const float v = xr[n];
        re = fmaf(v, w.x, re);
        im = fmaf(-v, w.y, im);
        idx += step;
        if (idx >= N) idx -= N;
      }
    }
#pragma unroll
    for (int off = L / 2; off > 0; off >>= 1) {
      re += __shfl_xor(re, off, L);
      im += __shfl_xor(im, off, L);
    }
    if (live && sub == 0) out[(r0 + rr) * m + j] = make_float2(re * scale, im * scale);
  }
}

// Last axis, real -> window, on the matrix cores.  For rows of N points and m
// kept bins the pruned DFT is the product [rows x N] . [N x 2m] with
//   T[n][2j] = cos(2 pi j n / N),  T[n][2j+1] = -sin(2 pi j n / N),
// run on v_mfma_f32_16x16x4f32 (fp32 products and accumulation); the output
// columns 2j, 2j+1 are the float2 bins of the window.  A wave owns 16 rows
// and all NT = ceil(2m / 16) column tiles.  The k order is permuted so the x
// loads stay row-contiguous: in k-step (c, i) lane group G supplies point
// n = 16c + 4G + i, so lane (G, r) holds points 16c + 4G .. +3 of row r.  The
// B entries come from the LDS twiddle table at index j n mod N, kept per
// (tile, i) as a running index that steps by 16 j mod N per chunk.
typedef float v4f_g __attribute__((ext_vector_type(4)));

template <int NT>
__global__ void __launch_bounds__(kThreads)
k_r2c_mfma(const float* __restrict__ x, float* __restrict__ out, int64_t rows, int N, int m,
           float scale) {
  extern __shared__ float smem[];
  float2* tw = reinterpret_cast<float2*>(smem);
  for (int t = threadIdx.x; t < N; t += blockDim.x) tw[t] = twiddle_any(t, N);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int G = lane >> 4, col = lane & 15;
  const int64_t r0 = ((int64_t)blockIdx.x * (kThreads / 64) + wave) * 16;
  if (r0 >= rows) return;   // no barrier follows
  const int64_t row = r0 + col;                    // this lane's A row
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)(rows * N * 4));
  int step[NT], idx[NT][4];
  bool on[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int j = (16 * t + col) >> 1;
    on[t] = j < m;
    step[t] = (16 * j) % N;
#pragma unroll
    for (int i = 0; i < 4; ++i) idx[t][i] = (j * (4 * G + i)) % N;
  }
  v4f_g acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = (v4f_g)0.f;
  // points 16c + 4G + i of the row; past the row or the last row: zero
  auto load = [&](int c, float (&dst)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = 16 * c + 4 * G + i;
      const uint32_t off = (row < rows && n < N) ? (uint32_t)((row * N + n) * 4) : 0x80000000u;
      dst[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, (int)off, 0, 0));
    }
  };
  const int nc = (N + 15) / 16;
  float a[4], an[4];
  load(0, a);
  for (int c = 0; c < nc; ++c) {
    if (c + 1 < nc) load(c + 1, an);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const float2 w = tw[idx[t][i]];
        const float bv = on[t] ? ((col & 1) ? -w.y : w.x) : 0.f;
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], bv, acc[t], 0, 0, 0);
        idx[t][i] += step[t];
        if (idx[t][i] >= N) idx[t][i] -= N;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = an[i];
  }
  // D: lane (G, col) register r is row r0 + 4G + r, column 16t + col
  const int w2 = 2 * m;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int q = 16 * t + col;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t ro = r0 + 4 * G + r;
      if (ro < rows && q < w2) out[ro * w2 + q] = acc[t][r] * scale;
    }
  }
}

// Non-last axis (or the last axis of complex data), complex -> complex: window
// entry j is frequency j + off (off = -m/2: the centred window):
//   out[o, j, q] = s * sum_n in[o, n, q] exp(-2 pi i (j + off) n / N)
__global__ void __launch_bounds__(kThreads)
k_c2c_fwd_direct(const float2* __restrict__ in, float2* __restrict__ out, int64_t outer, int N,
                 int64_t inner, int m, int off, float scale) {
  extern __shared__ float smem[];
  float2* tw = reinterpret_cast<float2*>(smem);
  for (int t = threadIdx.x; t < N; t += blockDim.x) tw[t] = twiddle_any(t, N);
  __syncthreads();
  const int64_t total = outer * m * inner;
  for (int64_t task = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; task < total;
       task += (int64_t)gridDim.x * blockDim.x) {
    const int64_t q = task % inner;
    const int64_t t2 = task / inner;
    const int j = (int)(t2 % m);
    const int64_t o = t2 / m;
    int step = (j + off) % N;
    if (step < 0) step += N;
    const float2* src = in + o * (int64_t)N * inner + q;
    float2 acc = make_float2(0.f, 0.f);
    int idx = 0;
    for (int n = 0; n < N; ++n) {
      const float2 v = src[(int64_t)n * inner];
      const float2 w = tw[idx];
      acc.x = fmaf(v.x, w.x, fmaf(v.y, w.y, acc.x));
      acc.y = fmaf(v.y, w.x, fmaf(-v.x, w.y, acc.y));
      idx += step;
      if (idx >= N) idx -= N;
    }
    out[task] = cscale(acc, scale);
  }
}

// ---------------------------------------------------------------- inverse axes
// Window -> length N' (ifftshift + ifftn(s = N') semantics):
//   out[o, n, q] = s * sum_{j : t_j < N'} in[o, j, q] exp(+2 pi i t_j n / N'),
//   t_j = (j + off) mod N (off = -m/2: the centred window)
__global__ void __launch_bounds__(kThreads)
k_c2c_inv_direct(const float2* __restrict__ in, float2* __restrict__ out, int64_t outer, int N,
                 int Np, int64_t inner, int m, int off, float scale) {
  extern __shared__ float smem[];
  float2* tw = reinterpret_cast<float2*>(smem);
  for (int t = threadIdx.x; t < Np; t += blockDim.x) tw[t] = twiddle_any(t, Np);
  __syncthreads();
  const int64_t total = outer * Np * inner;
  for (int64_t task = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; task < total;
       task += (int64_t)gridDim.x * blockDim.x) {
    const int64_t q = task % inner;
    const int64_t t2 = task / inner;
    const int n = (int)(t2 % Np);
    const int64_t o = t2 / Np;
    const float2* src = in + o * (int64_t)m * inner + q;
    float2 acc = make_float2(0.f, 0.f);
    // window entry j is frequency t = (j + off) mod N, at twiddle t n mod Np:
    // both indices advance by one step per entry (t wraps at N to 0)
    int t = off % N;
    if (t < 0) t += N;
    int idx = (int)(((int64_t)t * n) % Np);
    for (int j = 0; j < m; ++j) {
      if (t < Np) cfma(acc, src[(int64_t)j * inner], tw[idx]);
      ++t;
      idx += n;
      if (idx >= Np) idx -= Np;
      if (t == N) {
        t = 0;
        idx = 0;
      }
    }
    out[task] = cscale(acc, scale);
  }
}

// Non-last axis (or the last axis of complex data), complex -> complex, on the
// matrix cores: Out[o, r, q] = s sum_{j<S} W(r, j) In[o, j, q] over the C =
// outer * inner columns (o, q), as the real product
//   D[2r + po][c] = sum_{2j + pi} A[2r + po][2j + pi] B[2j + pi][c]
// with A the real form of the twiddle w = W(r, j) (re: w.re, -w.im; im: w.im,
// w.re) and B the real and imaginary parts of In.
//   DIR = -1 (analysis):  R = m rows, S = N points,  W = exp(-2 pi i f n / N),
//                         f = (r + off) mod N
//   DIR = +1 (synthesis): R = Np points, S = m entries, W = exp(2 pi i r t / Np),
//                         t = (j + off) mod N, zero where t >= Np
// A wave owns MT row tiles of 16 and one column tile of 16.  In k-step ks lane
// group G supplies k = 4 ks + G, i.e. j = 2 ks + G/2 and part G & 1, so j steps
// by 2 per k-step and the twiddle index j f mod N (analysis) or r t mod Np
// (synthesis) is a running sum per row tile.
template <int DIR, int MT>
__global__ void __launch_bounds__(kThreads)
k_c2c_axis_mfma(const float2* __restrict__ in, float2* __restrict__ out, int64_t outer,
                int64_t inner, int N, int Np, int m, int off, int mgroups, float scale) {
  extern __shared__ float smem[];
  float2* tw = reinterpret_cast<float2*>(smem);
  const int L = DIR < 0 ? N : Np;
  for (int t = threadIdx.x; t < L; t += blockDim.x) tw[t] = twiddle_any(t, L);
  __syncthreads();
  const int R = DIR < 0 ? m : Np, S = DIR < 0 ? N : m;
  const int64_t C = outer * inner;
  const int lane = threadIdx.x & 63, G = lane >> 4, col = lane & 15;
  const int64_t wid = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  const int mt0 = (int)(wid % mgroups) * MT;
  const int64_t c0 = (wid / mgroups) * 16;
  const int mtiles = (2 * R + 15) / 16;
  if (c0 >= C || mt0 >= mtiles) return;   // no barrier follows
  const int pi = G & 1;
  // B column of this lane
  const int64_t cb = c0 + col;
  const bool cl = cb < C;
  const int64_t ob = cl ? cb / inner : 0, qb = cl ? cb % inner : 0;
  const float* inf = reinterpret_cast<const float*>(in);
  const __amdgpu_buffer_rsrc_t rin = make_rsrc(inf, (uint32_t)(outer * S * inner * 8));
  // A rows of this lane: row r of tile t, its running twiddle index
  int rr[MT], idx[MT], step[MT];
  int t = 0;   // synthesis: frequency of entry j = G / 2 (+ 2 per k-step)
  if (DIR > 0) {
    t = (G >> 1) + off;
    t %= N;
    if (t < 0) t += N;
  }
#pragma unroll
  for (int u = 0; u < MT; ++u) {
    const int rho = 16 * (mt0 + u) + col;
    rr[u] = rho >> 1;
    if (DIR < 0) {
      int f = (rr[u] + off) % N;
      if (f < 0) f += N;
      idx[u] = (int)(((int64_t)f * (G >> 1)) % N);
      step[u] = (int)((2LL * f) % N);
    } else {
      idx[u] = (int)(((int64_t)rr[u] * t) % Np);
      step[u] = (int)((2LL * rr[u]) % Np);
    }
  }
  v4f_g acc[MT];
#pragma unroll
  for (int u = 0; u < MT; ++u) acc[u] = (v4f_g)0.f;
  const int ksteps = (2 * S + 3) / 4;
  auto load_b = [&](int ks) __attribute__((always_inline)) {
    const int j = 2 * ks + (G >> 1);
    const uint32_t off_b = (cl && j < S) ? (uint32_t)((((ob * S + j) * inner + qb) * 2 + pi) * 4)
                                         : 0x80000000u;
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rin, (int)off_b, 0, 0));
  };
  // B values in blocks of KB k-steps, the next block in flight; k-steps past
  // the last read zero (j >= S), so a partial last block adds nothing
  constexpr int KB = 8;
  float bc[KB], bn[KB];
#pragma unroll
  for (int i = 0; i < KB; ++i) bc[i] = load_b(i);
  for (int k0 = 0; k0 < ksteps; k0 += KB) {
#pragma unroll
    for (int i = 0; i < KB; ++i) bn[i] = k0 + KB < ksteps ? load_b(k0 + KB + i) : 0.f;
#pragma unroll
    for (int i = 0; i < KB; ++i) {
      const bool live = DIR < 0 || t < Np;
#pragma unroll
      for (int u = 0; u < MT; ++u) {
        const float2 w = tw[idx[u]];
        const float wi = DIR < 0 ? -w.y : w.y;   // imaginary part of W
        const int po = col & 1;                   // A row 2r + po of this lane
        float av = (po == pi) ? w.x : (po ? wi : -wi);
        av = live && rr[u] < R ? av : 0.f;
        acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bc[i], acc[u], 0, 0, 0);
        idx[u] += step[u];
        if (idx[u] >= L) idx[u] -= L;
      }
      if (DIR > 0) {   // the entries two further on: t + 2, wrapping at N
        t += 2;
        if (t >= N) {
          while (t >= N) t -= N;
#pragma unroll
          for (int u = 0; u < MT; ++u) idx[u] = (int)(((int64_t)rr[u] * t) % Np);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < KB; ++i) bc[i] = bn[i];
  }
  // D: lane (G, col) register v is row 16 (mt0 + u) + 4G + v, column c0 + col
  const int64_t cd = c0 + col;
  if (cd >= C) return;
  const int64_t od = cd / inner, qd = cd % inner;
  float* outf = reinterpret_cast<float*>(out);
#pragma unroll
  for (int u = 0; u < MT; ++u)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int rho = 16 * (mt0 + u) + 4 * G + v, r = rho >> 1;
      if (r < R) outf[((od * R + r) * inner + qd) * 2 + (rho & 1)] = acc[u][v] * scale;
    }
}

// Last axis, window -> real length N' (irfft semantics) + bias:
//   y[r, n] = s * sum_{j < N'/2+1} c_j Re(Z_j exp(2 pi i j n / N')) + bias[channel(r)]
__global__ void __launch_bounds__(kThreads)
k_c2r_direct(const float2* __restrict__ in, float* __restrict__ out, const float* __restrict__ bias,
             int64_t rows, int64_t rows_per_plane, int channels, int N, int Np, int m, int enforce,
             int rows_per_block, float scale) {
  extern __shared__ float smem[];
  float2* tw = reinterpret_cast<float2*>(smem);
  float2* zs = tw + Np;
  for (int t = threadIdx.x; t < Np; t += blockDim.x) tw[t] = twiddle_any(t, Np);
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  const int nr = (int)min((int64_t)rows_per_block, rows - r0);
  const int K = min(m, Np / 2 + 1);
  for (int t = threadIdx.x; t < nr * K; t += blockDim.x) {
    const int rr = t / K, j = t - (t / K) * K;
    float2 z = in[(r0 + rr) * m + j];
    float c = 2.f;
    if (j == 0) {
      z.y = 0.f;
      c = 1.f;
    }
    if (enforce && (Np % 2 == 0) && j == N / 2) z.y = 0.f;
    if ((Np % 2 == 0) && j == Np / 2) c = 1.f;
    zs[rr * K + j] = cscale(z, c);
  }
  __syncthreads();
  for (int task = threadIdx.x; task < nr * Np; task += blockDim.x) {
    const int rr = task / Np, n = task - (task / Np) * Np;
    const float2* z = zs + rr * K;
    float acc = 0.f;
    int idx = 0;
    for (int j = 0; j < K; ++j) {
      const float2 w = tw[idx];
      acc = fmaf(z[j].x, w.x, fmaf(-z[j].y, w.y, acc));
      idx += n;
      if (idx >= Np) idx -= Np;
    }
    float v = acc * scale;
    if (bias) v += bias[((r0 + rr) / rows_per_plane) % channels];
    out[(r0 + rr) * Np + n] = v;
  }
}

// Last axis, window -> real length Np on the matrix cores (the irfft of
// k_c2r_direct as a product): y[r, n] = s sum_k A[r, k] T[k, n] + bias with
//   A[r, 2j] = c_j Re Z_j,  A[r, 2j+1] = c_j Im Z_j   (Hermitian fix-ups as in
//   k_c2r_direct), T[2j, n] = cos(2 pi j n / Np), T[2j+1, n] = -sin(...).
// A wave owns 16 rows and CT column tiles of 16 points; a workgroup's four
// waves take consecutive column tiles of the same rows.  In k-step (c, i)
// lane group G supplies k = 16c + 4G + i (four consecutive floats of a Z row
// per lane), and the B entry of lane (G, col) in tile t is the twiddle at
// j n mod Np with j = 8c + 2G + i/2, kept as a running index per (t, i/2).
template <int CT>
__global__ void __launch_bounds__(kThreads)
k_c2r_mfma(const float2* __restrict__ in, float* __restrict__ out, const float* __restrict__ bias,
           int64_t rows, int64_t rows_per_plane, int channels, int N, int Np, int m, int enforce,
           int col_groups, float scale) {
  extern __shared__ float smem[];
  float2* tw = reinterpret_cast<float2*>(smem);
  for (int t = threadIdx.x; t < Np; t += blockDim.x) tw[t] = twiddle_any(t, Np);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int G = lane >> 4, col = lane & 15;
  const int64_t r0 = (int64_t)(blockIdx.x / col_groups) * 16;
  const int tile0 = ((int)(blockIdx.x % col_groups) * (kThreads / 64) + wave) * CT;
  const int ntiles = (Np + 15) / 16;
  if (tile0 >= ntiles) return;   // no barrier follows
  const int K = m < Np / 2 + 1 ? m : Np / 2 + 1;   // bins used
  const int64_t row = r0 + col;                      // this lane's A row
  const float* zf = reinterpret_cast<const float*>(in);
  const __amdgpu_buffer_rsrc_t rz = make_rsrc(zf, (uint32_t)(rows * m * 8));
  int idx[CT][2], step[CT];
#pragma unroll
  for (int t = 0; t < CT; ++t) {
    const int n = 16 * (tile0 + t) + col;
    step[t] = (int)((8LL * n) % Np);
#pragma unroll
    for (int h = 0; h < 2; ++h) idx[t][h] = (int)(((int64_t)(2 * G + h) * n) % Np);
  }
  v4f_g acc[CT];
#pragma unroll
  for (int t = 0; t < CT; ++t) acc[t] = (v4f_g)0.f;
  // A entries k = 16c + 4G + i of the row, Hermitian weights applied
  auto load = [&](int c, float (&dst)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = 16 * c + 4 * G + i, j = k >> 1;
      const bool live = row < rows && j < K;
      const uint32_t off = live ? (uint32_t)((row * m * 2 + k) * 4) : 0x80000000u;
      float v = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rz, (int)off, 0, 0));
      if (k & 1) {   // imaginary part
        if (j == 0 || (enforce && (Np % 2 == 0) && j == N / 2)) v = 0.f;
      }
      const float cw = (j == 0 || ((Np % 2 == 0) && j == Np / 2)) ? 1.f : 2.f;
      dst[i] = v * cw;
    }
  };
  const int nc = (2 * K + 15) / 16;
  float a[4], an[4];
  load(0, a);
  for (int c = 0; c < nc; ++c) {
    if (c + 1 < nc) load(c + 1, an);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int t = 0; t < CT; ++t) {
        const float2 w = tw[idx[t][i >> 1]];
        const float bv = (i & 1) ? -w.y : w.x;
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], bv, acc[t], 0, 0, 0);
      }
    }
#pragma unroll
    for (int t = 0; t < CT; ++t)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        idx[t][h] += step[t];
        if (idx[t][h] >= Np) idx[t][h] -= Np;
      }
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = an[i];
  }
  // D: lane (G, col) register r is row r0 + 4G + r, point 16 (tile0 + t) + col
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t ro = r0 + 4 * G + r;
    if (ro >= rows) continue;
    const float bb = bias ? bias[(ro / rows_per_plane) % channels] : 0.f;
#pragma unroll
    for (int t = 0; t < CT; ++t) {
      const int n = 16 * (tile0 + t) + col;
      if (n < Np) out[ro * Np + n] = acc[t][r] * scale + bb;
    }
  }
}

// ----------------------------------------------------------------- contraction
// y[b, o, k] = sum_i x[b, i, k] * w[i*sWi + o*sWo + k*sWk]     (complex)
// Output mode index of mode k = j W' + kw of an m1 x W' window when the
// consumer wants each row's AC bins as one run (ymap_w = W'): AC bins of all
// rows first (entry j (W' - 1) + kw - 1), then the DC column (m1 (W' - 1) + j).
// ymap_w = 0 keeps the window order.
__device__ __forceinline__ int64_t ymap_index(int64_t k, int64_t M, int ymap_w) {
  if (!ymap_w) return k;
  const int64_t j = k / ymap_w, kw = k - j * ymap_w;
  return kw ? j * (ymap_w - 1) + kw - 1 : (M / ymap_w) * (ymap_w - 1) + j;
}

// One lane per mode k; each thread owns a TB x TO tile of (b, o).
template <int TB, int TO>
__global__ void __launch_bounds__(kThreads)
k_contract_dense(const float2* __restrict__ X, const float2* __restrict__ W, float2* __restrict__ Y,
                 int B, int Ci, int Co, int64_t M, int64_t sWi, int64_t sWo, int64_t sWk,
                 int ymap_w) {
  const int64_t k = (int64_t)blockIdx.x * 64 + (threadIdx.x & 63);
  const int nOt = (Co + TO - 1) / TO;
  const int nBt = (B + TB - 1) / TB;
  const int tile = blockIdx.y * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (tile >= nOt * nBt || k >= M) return;
  const int b0 = (tile / nOt) * TB;
  const int o0 = (tile % nOt) * TO;
  float2 acc[TB][TO];
#pragma unroll
  for (int a = 0; a < TB; ++a)
#pragma unroll
    for (int c = 0; c < TO; ++c) acc[a][c] = make_float2(0.f, 0.f);
  for (int i = 0; i < Ci; ++i) {
    float2 xv[TB], wv[TO];
#pragma unroll
    for (int a = 0; a < TB; ++a)
      xv[a] = (b0 + a < B) ? X[((int64_t)(b0 + a) * Ci + i) * M + k] : make_float2(0.f, 0.f);
#pragma unroll
    for (int c = 0; c < TO; ++c)
      wv[c] = (o0 + c < Co) ? W[(int64_t)i * sWi + (int64_t)(o0 + c) * sWo + k * sWk]
                            : make_float2(0.f, 0.f);
#pragma unroll
    for (int a = 0; a < TB; ++a)
#pragma unroll
      for (int c = 0; c < TO; ++c) cfma(acc[a][c], xv[a], wv[c]);
  }
#pragma unroll
  for (int a = 0; a < TB; ++a)
#pragma unroll
    for (int c = 0; c < TO; ++c)
      if (b0 + a < B && o0 + c < Co)
        Y[((int64_t)(b0 + a) * Co + o0 + c) * M + ymap_index(k, M, ymap_w)] = acc[a][c];
}

// Small contractions (few modes): 16 lanes per output y[b, o, k], each
// summing every 16th input channel, reduced across the lanes; outputs are
// ordered k fastest, then o, then b.
__global__ void __launch_bounds__(kThreads)
k_contract_small(const float2* __restrict__ X, const float2* __restrict__ W, float2* __restrict__ Y,
                 int B, int Ci, int Co, int64_t M, int64_t sWi, int64_t sWo, int64_t sWk,
                 int ymap_w) {
  constexpr int L = 16;
  const int64_t out = ((int64_t)blockIdx.x * kThreads + threadIdx.x) / L;
  const int sub = threadIdx.x % L;
  const bool live = out < (int64_t)B * Co * M;
  const int64_t k = live ? out % M : 0;
  const int o = live ? (int)((out / M) % Co) : 0;
  const int b = live ? (int)(out / (M * Co)) : 0;
  float2 acc = make_float2(0.f, 0.f);
  if (live) {
    for (int i = sub; i < Ci; i += L)
      cfma(acc, X[((int64_t)b * Ci + i) * M + k], W[(int64_t)i * sWi + (int64_t)o * sWo + k * sWk]);
  }
#pragma unroll
  for (int off = L / 2; off > 0; off >>= 1) {
    acc.x += __shfl_xor(acc.x, off, L);
    acc.y += __shfl_xor(acc.y, off, L);
  }
  if (live && sub == 0) Y[((int64_t)b * Co + o) * M + ymap_index(k, M, ymap_w)] = acc;
}

// y[b, i, k] = x[b, i, k] * w[i, k]
__global__ void __launch_bounds__(kThreads)
k_contract_separable(const float2* __restrict__ X, const float2* __restrict__ W,
                     float2* __restrict__ Y, int64_t CM, int64_t total) {
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x)
    Y[t] = cmul(X[t], W[t % CM]);
}

// out[o, j, q] = sum_a in[o, a, q] * mat[j, a]   (complex matrix along an axis)
__global__ void __launch_bounds__(kThreads)
k_axis_matmul(const float2* __restrict__ in, const float2* __restrict__ mat, float2* __restrict__ out,
              int64_t outer, int A, int J, int64_t inner) {
  const int64_t total = outer * J * inner;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t q = t % inner;
    const int64_t t2 = t / inner;
    const int j = (int)(t2 % J);
    const int64_t o = t2 / J;
    const float2* src = in + o * (int64_t)A * inner + q;
    float2 acc = make_float2(0.f, 0.f);
    for (int a = 0; a < A; ++a) cfma(acc, src[(int64_t)a * inner], mat[(int64_t)j * A + a]);
    out[t] = acc;
  }
}

// ------------------------------------------------------------------- epilogue
// y[b, o, p] = act(spec[b, o, p] + skip(x)[b, o, p]); spec may alias y (each
// thread reads its spec entries before writing the same entries).
// A thread owns PP consecutive points and OT output channels, so x is read once
// per OT output channels; the linear skip's weights sit transposed in LDS
// (wT[i][o]) and are read as broadcast float4s.
template <int OT, int PP>
__global__ void __launch_bounds__(kThreads)
k_epilogue(const float* spec, const float* __restrict__ x, const float* __restrict__ ws, float* y,
           int B, int Ci, int Co, int64_t P, int skip_kind, int act) {
  typedef float vpp __attribute__((ext_vector_type(PP)));
  extern __shared__ float4 smem4[];
  float* wT = reinterpret_cast<float*>(smem4);   // [Ci][OT], linear skip only
  const int o0 = blockIdx.y * OT;
  const int b = blockIdx.z;
  const int on = min(OT, Co - o0);
  const bool linear = skip_kind == FNO_SKIP_LINEAR;
  constexpr int KB = 8;   // input channels per batch of x loads
  const int CiP = (Ci + KB - 1) / KB * KB;
  if (linear) {
    // rows Ci .. CiP-1 are zero so whole batches need no guard
    for (int e = threadIdx.x; e < CiP * OT; e += kThreads) {
      const int i = e / OT, c = e % OT;
      wT[e] = (c < on && i < Ci) ? ws[(int64_t)(o0 + c) * Ci + i] : 0.f;
    }
    __syncthreads();
  }
  const int64_t p = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * PP;
  if (p >= P) return;
  vpp acc[OT];
#pragma unroll
  for (int c = 0; c < OT; ++c) acc[c] = (vpp)0.f;
  if (linear) {
    const float* xb = x + (int64_t)b * Ci * P + p;
    // batches of KB input channels; the next batch is in flight while this
    // one is used
    vpp cur[KB], nxt[KB];
    auto load = [&](int i0, vpp (&d)[KB]) __attribute__((always_inline)) {
#pragma unroll
      for (int k = 0; k < KB; ++k)
        d[k] = i0 + k < Ci ? *reinterpret_cast<const vpp*>(xb + (int64_t)(i0 + k) * P) : (vpp)0.f;
    };
    load(0, cur);
    for (int i0 = 0; i0 < Ci; i0 += KB) {
      if (i0 + KB < Ci) load(i0 + KB, nxt);
#pragma unroll
      for (int k = 0; k < KB; ++k) {
        const float4* w4 = reinterpret_cast<const float4*>(wT + (i0 + k) * OT);
#pragma unroll
        for (int c4 = 0; c4 < OT / 4; ++c4) {
          const float4 w = w4[c4];
          acc[4 * c4 + 0] += w.x * cur[k];
          acc[4 * c4 + 1] += w.y * cur[k];
          acc[4 * c4 + 2] += w.z * cur[k];
          acc[4 * c4 + 3] += w.w * cur[k];
        }
      }
#pragma unroll
      for (int k = 0; k < KB; ++k) cur[k] = nxt[k];
    }
  } else if (skip_kind == FNO_SKIP_SOFT_GATING || skip_kind == FNO_SKIP_IDENTITY) {
#pragma unroll
    for (int c = 0; c < OT; ++c)
      if (c < on) {
        const vpp v = *reinterpret_cast<const vpp*>(x + ((int64_t)b * Ci + o0 + c) * P + p);
        acc[c] = (skip_kind == FNO_SKIP_SOFT_GATING) ? ws[o0 + c] * v : v;
      }
  }
#pragma unroll
  for (int c = 0; c < OT; ++c) {
    if (c >= on) break;
    const int64_t idx = ((int64_t)b * Co + o0 + c) * P + p;
    vpp v = *reinterpret_cast<const vpp*>(spec + idx) + acc[c];
    if (act == FNO_ACT_GELU) {
#pragma unroll
      for (int k = 0; k < PP; ++k) v[k] = gelu_erf(v[k]);
    }
    *reinterpret_cast<vpp*>(y + idx) = v;
  }
}

// ============================================================== host helpers
static int grid_for(int64_t total) {
  int64_t g = (total + kThreads - 1) / kThreads;
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return (int)g;
}

// grid-stride kernels that first build an N-entry twiddle table: at most
// 2048 workgroups (8 per CU), so each table serves many tasks
static int grid_for_table(int64_t total) {
  const int g = grid_for(total);
  return g > 2048 ? 2048 : g;
}

static int c2c_axis_fwd(const float2* src, float2* dst, int64_t outer, int N, int64_t inner, int m,
                        int off, float sc, hipStream_t st);
static int c2c_axis_inv(const float2* src, float2* dst, int64_t outer, int N, int Np, int64_t inner,
                        int m, int off, float sc, hipStream_t st);

static int validate_axes(int32_t ndim, const int32_t* sizes, const int32_t* modes) {
  FNO_CHECK_ARG(ndim >= 1 && ndim <= 4, "ndim must be 1..4 (got %d)", ndim);
  FNO_CHECK_ARG(sizes && modes, "sizes/modes must not be NULL");
  for (int d = 0; d < ndim; ++d) {
    FNO_CHECK_ARG(sizes[d] >= 1, "size[%d]=%d must be positive", d, sizes[d]);
    const int cap = (d == ndim - 1) ? sizes[d] / 2 + 1 : sizes[d];
    FNO_CHECK_ARG(modes[d] >= 1 && modes[d] <= cap, "modes[%d]=%d outside [1, %d]", d, modes[d],
                  cap);
  }
  for (int d = 0; d < ndim; ++d) {
    if (sizes[d] > kMaxAxis) {
      set_error("axis %d has size %d > %d supported by the generic kernels", d, sizes[d], kMaxAxis);
      return FNO_ERR_UNSUPPORTED;
    }
  }
  return FNO_OK;
}

// elements of the intermediate after the forward transform of axes d..ndim-1
// (axes before d still full size)
static int64_t fwd_stage_elems(int64_t planes, int32_t ndim, const int32_t* sizes,
                               const int32_t* modes, int first_done) {
  int64_t e = planes;
  for (int d = 0; d < ndim; ++d) e *= (d >= first_done) ? modes[d] : sizes[d];
  return e;
}

// Intermediate stages of a window transform alternate between two workspace
// buffers (one for 2 axes, none for 1), each as large as the largest of them.
static int stage_buffers(int32_t ndim) { return ndim >= 3 ? 2 : ndim - 1; }

static int64_t fwd_buffer_elems(int64_t planes, int32_t ndim, const int32_t* sizes,
                                const int32_t* modes) {
  int64_t e = 0;
  for (int d = 1; d < ndim; ++d) {   // axis d done (stages before the last)
    const int64_t s = fwd_stage_elems(planes, ndim, sizes, modes, d);
    if (s > e) e = s;
  }
  return e;
}

// the inverse stage that has expanded axes 0..d to their output lengths
static int64_t inv_stage_elems(int64_t planes, int32_t ndim, const int32_t* out_sizes,
                               const int32_t* modes, int d) {
  int64_t e = planes;
  for (int a = 0; a < ndim; ++a) e *= (a <= d) ? out_sizes[a] : modes[a];
  return e;
}

static int64_t inv_buffer_elems(int64_t planes, int32_t ndim, const int32_t* out_sizes,
                                const int32_t* modes) {
  int64_t e = 0;
  for (int d = 0; d + 1 < ndim; ++d) {
    const int64_t s = inv_stage_elems(planes, ndim, out_sizes, modes, d);
    if (s > e) e = s;
  }
  return e;
}

// line-FFT last-axis transforms (fno_generic_fft.hip)
bool r2c_fft_supported(int N, int m, int64_t rows);
int r2c_fft(const float* x, float2* out, int64_t rows, int N, int m, float scale, hipStream_t st);
bool c2r_fft_supported(int Np, int64_t rows);
int c2r_fft(const float2* in, float* out, const float* bias, int64_t rows, int64_t rows_per_plane,
            int channels, int N, int Np, int m, int enforce, float scale, hipStream_t st);
bool c2c_fft_supported(int L, int64_t outer, int64_t inner);
int c2c_fft_fwd(const float2* in, float2* out, int64_t outer, int64_t inner, int N, int m, int off,
                float scale, hipStream_t st);
int c2c_fft_inv(const float2* in, float2* out, int64_t outer, int64_t inner, int N, int Np, int m,
                int off, float scale, hipStream_t st);

bool slab_fwd64_supported(int N1, int N2, int m1, int m2h);
int slab_fwd64(const float* x, float2* out, int64_t slabs, int m1, int m2h, float scale,
               hipStream_t st);

int rfft_window(const float* x, float2* xhat, int64_t planes, int32_t ndim, const int32_t* sizes,
                const int32_t* modes, int32_t norm, void* ws, size_t ws_bytes, hipStream_t st) {
  // stage s transforms axis (ndim-1-s); stage outputs go to the workspace
  // (two alternating buffers), the last one to xhat.
  const double scale = forward_scale(norm, sizes, ndim);
  const int64_t eb = fwd_buffer_elems(planes, ndim, sizes, modes);
  const size_t need = (size_t)stage_buffers(ndim) * eb * sizeof(float2);
  if (ws_bytes < need) {
    set_error("rfft_window: workspace %zu < %zu bytes", ws_bytes, need);
    return FNO_ERR_WORKSPACE;
  }
  float2* bufs[2] = {reinterpret_cast<float2*>(ws), reinterpret_cast<float2*>(ws) + eb};
  float2* bufA = bufs[0];
  // 64 x 64 trailing slabs: the last two axes in one pass (stages 0 and 1,
  // written where stage 1 writes), then the remaining axes as below
  if (ndim >= 2 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
      slab_fwd64_supported(sizes[ndim - 2], sizes[ndim - 1], modes[ndim - 2], modes[ndim - 1])) {
    int64_t slabs = planes;
    for (int d = 0; d + 2 < ndim; ++d) slabs *= sizes[d];
    float2* dst = ndim == 2 ? xhat : bufs[1];
    int rc = slab_fwd64(x, dst, slabs, modes[ndim - 2], modes[ndim - 1],
                        ndim == 2 ? (float)scale : 1.f, st);
    if (rc) return rc;
    const float2* src = dst;
    for (int d = ndim - 3; d >= 0; --d) {
      int64_t outer = planes;
      for (int a = 0; a < d; ++a) outer *= sizes[a];
      int64_t inner = 1;
      for (int a = d + 1; a < ndim; ++a) inner *= modes[a];
      float2* out = (d == 0) ? xhat : bufs[(ndim - 1 - d) % 2];
      rc = c2c_axis_fwd(src, out, outer, sizes[d], inner, modes[d], -(modes[d] / 2),
                        d == 0 ? (float)scale : 1.f, st);
      if (rc) return rc;
      src = out;
    }
    return FNO_OK;
  }
  // last axis
  {
    const int N = sizes[ndim - 1], m = modes[ndim - 1];
    int64_t rows = planes;
    for (int d = 0; d < ndim - 1; ++d) rows *= sizes[d];
    float2* dst = ndim == 1 ? xhat : bufA;
    // only the last stage of the chain carries the scale
    const float sc = (ndim == 1) ? (float)scale : 1.f;
    if (r2c_fft_supported(N, m, rows)) {
      int rc = r2c_fft(x, dst, rows, N, m, sc, st);
      if (rc) return rc;
    } else if (m <= 64 && rows >= 16384 && rows * (int64_t)N * 4 < (int64_t(1) << 31)) {
      // many rows: the DFT product on the matrix cores, 64 rows per workgroup
      const unsigned blocks = (unsigned)((rows + 63) / 64);
      const size_t lds = (size_t)N * 8;
      float* o = reinterpret_cast<float*>(dst);
#define FNO_R2C_MFMA(nt)                                                                          \
  case nt:                                                                                        \
    hipLaunchKernelGGL(k_r2c_mfma<nt>, dim3(blocks), dim3(kThreads), lds, st, x, o, rows, N, m, sc); \
    break;
      switch ((2 * m + 15) / 16) {
        FNO_R2C_MFMA(1) FNO_R2C_MFMA(2) FNO_R2C_MFMA(3) FNO_R2C_MFMA(4)
        FNO_R2C_MFMA(5) FNO_R2C_MFMA(6) FNO_R2C_MFMA(7) FNO_R2C_MFMA(8)
        default: break;
      }
#undef FNO_R2C_MFMA
      int rc = launch_status("k_r2c_mfma");
      if (rc) return rc;
    } else {
      int rpb = (int)((48 * 1024 - 8 * N) / (4 * N));
      if (rpb < 1) rpb = 1;
      if (rpb > 64) rpb = 64;
      // one pass of 16 tasks per workgroup: more workgroups for few bins,
      // unless there are rows enough for 2048 workgroups of more rows each
      // (every workgroup builds the N-entry twiddle table first)
      int rfill = (16 + m - 1) / m;
      if (rows / 2048 > rfill) rfill = (int)(rows / 2048 < 64 ? rows / 2048 : 64);
      if (rpb > rfill) rpb = rfill;
      const size_t lds = (size_t)N * 8 + (size_t)rpb * N * 4;
      const int64_t blocks = (rows + rpb - 1) / rpb;
      hipLaunchKernelGGL(k_r2c_direct, dim3((unsigned)blocks), dim3(kThreads), lds, st, x, dst,
                         rows, N, m, rpb, sc);
      int rc = launch_status("k_r2c_direct");
      if (rc) return rc;
    }
  }
  // the other axes, innermost first; stage s = ndim - 1 - d writes bufs[s % 2]
  const float2* src = bufA;
  for (int d = ndim - 2; d >= 0; --d) {
    int64_t outer = planes;
    for (int a = 0; a < d; ++a) outer *= sizes[a];
    int64_t inner = 1;
    for (int a = d + 1; a < ndim; ++a) inner *= modes[a];
    const int N = sizes[d], m = modes[d];
    float2* dst = (d == 0) ? xhat : bufs[(ndim - 1 - d) % 2];
    const float sc = (d == 0) ? (float)scale : 1.f;
    const int rc = c2c_axis_fwd(src, dst, outer, N, inner, m, -(m / 2), sc, st);
    if (rc) return rc;
    src = dst;
  }
  return FNO_OK;
}

// ------------------------------------------------- complex-data windows
// One axis of a complex window transform: line FFTs for 64/128/256 points,
// direct sums otherwise.  Window entry j is frequency j + off.
// the matrix-core form when there are columns enough for 64+ waves and the
// buffer offsets fit 31 bits
static bool c2c_mfma_ok(int64_t outer, int64_t inner, int S, int R) {
  const int64_t C = outer * inner;
  return C >= 1024 && C * (S > R ? S : R) * 8 < (int64_t(1) << 31);
}

template <int DIR, int MT>
static int launch_c2c_mfma(const float2* src, float2* dst, int64_t outer, int64_t inner, int N,
                           int Np, int m, int off, float sc, hipStream_t st) {
  const int R = DIR < 0 ? m : Np;
  const int mgroups = ((2 * R + 15) / 16 + MT - 1) / MT;
  const int64_t waves = (outer * inner + 15) / 16 * mgroups;
  const unsigned blocks = (unsigned)((waves + kThreads / 64 - 1) / (kThreads / 64));
  hipLaunchKernelGGL((k_c2c_axis_mfma<DIR, MT>), dim3(blocks), dim3(kThreads),
                     (size_t)(DIR < 0 ? N : Np) * 8, st, src, dst, outer, inner, N, Np, m, off,
                     mgroups, sc);
  return launch_status("k_c2c_axis_mfma");
}

static int c2c_axis_fwd(const float2* src, float2* dst, int64_t outer, int N, int64_t inner, int m,
                        int off, float sc, hipStream_t st) {
  // lines fewer than a 16-line tile apart: the product form reads them whole
  if (inner < 16 && c2c_mfma_ok(outer, inner, N, m))
    return launch_c2c_mfma<-1, 1>(src, dst, outer, inner, N, N, m, off, sc, st);
  if (c2c_fft_supported(N, outer, inner)) return c2c_fft_fwd(src, dst, outer, inner, N, m, off, sc, st);
  if (c2c_mfma_ok(outer, inner, N, m))
    return launch_c2c_mfma<-1, 1>(src, dst, outer, inner, N, N, m, off, sc, st);
  hipLaunchKernelGGL(k_c2c_fwd_direct, dim3(grid_for_table(outer * m * inner)), dim3(kThreads),
                     (size_t)N * 8, st, src, dst, outer, N, inner, m, off, sc);
  return launch_status("k_c2c_fwd_direct");
}

bool axis_inv64_supported(int N, int Np, int m, int64_t inner);
int axis_inv64(const float2* src, float2* dst, int64_t slabs, int m, int inner, float scale,
               hipStream_t st);
bool axis_inv64x2_supported(int N0, int Np0, int m0, int N1, int Np1, int m1, int64_t inner);
int axis_inv64x2(const float2* src, float2* dst, int64_t planes, int m0, int m1, int inner,
                 float scale, hipStream_t st);

static int c2c_axis_inv(const float2* src, float2* dst, int64_t outer, int N, int Np, int64_t inner,
                        int m, int off, float sc, hipStream_t st) {
  // 64-point axis, a window of at most 16 rows (centred: off = -(m / 2)) and
  // at most 16 columns: one matrix-core product per slab
  if (off == -(m / 2) && axis_inv64_supported(N, Np, m, inner))
    return axis_inv64(src, dst, outer, m, (int)inner, sc, st);
  if (inner < 16 && c2c_mfma_ok(outer, inner, m, Np))
    return launch_c2c_mfma<1, 4>(src, dst, outer, inner, N, Np, m, off, sc, st);
  if (c2c_fft_supported(Np, outer, inner))
    return c2c_fft_inv(src, dst, outer, inner, N, Np, m, off, sc, st);
  if (c2c_mfma_ok(outer, inner, m, Np))
    return launch_c2c_mfma<1, 4>(src, dst, outer, inner, N, Np, m, off, sc, st);
  hipLaunchKernelGGL(k_c2c_inv_direct, dim3(grid_for_table(outer * Np * inner)), dim3(kThreads),
                     (size_t)Np * 8, st, src, dst, outer, N, Np, inner, m, off, sc);
  return launch_status("k_c2c_inv_direct");
}

// y[plane, p] += bias[plane % channels] on the real part
__global__ void __launch_bounds__(kThreads)
k_add_bias_re(float2* __restrict__ y, const float* __restrict__ bias, int64_t per_plane,
              int channels, int64_t total) {
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x)
    y[t].x += bias[(t / per_plane) % channels];
}

// Window offsets of complex data (spectral_convolution.py:436-449, :500-517,
// :531-538): the non-last axes are fftshift-ed and keep the centred window;
// the last axis keeps the first m entries of its fftshift-ed order (the
// first m frequencies when the field is 1D, which is not shifted), and the
// inverse places window entry j at index j of that axis (no ifftshift there).
static int complex_fwd_off(int d, int ndim, int N, int m) {
  if (d < ndim - 1) return -(m / 2);
  return ndim > 1 ? -(N / 2) : 0;
}

int fft_window_c2c(const float2* x, float2* xhat, int64_t planes, int32_t ndim,
                   const int32_t* sizes, const int32_t* modes, int32_t norm, void* ws,
                   size_t ws_bytes, hipStream_t st) {
  const double scale = forward_scale(norm, sizes, ndim);
  const int64_t eb = fwd_buffer_elems(planes, ndim, sizes, modes);
  const size_t need = (size_t)stage_buffers(ndim) * eb * sizeof(float2);
  if (ws_bytes < need) {
    set_error("fft_window: workspace %zu < %zu bytes", ws_bytes, need);
    return FNO_ERR_WORKSPACE;
  }
  float2* bufs[2] = {reinterpret_cast<float2*>(ws), reinterpret_cast<float2*>(ws) + eb};
  const float2* src = x;
  for (int d = ndim - 1, stage = 0; d >= 0; --d, ++stage) {
    int64_t outer = planes;
    for (int a = 0; a < d; ++a) outer *= sizes[a];
    int64_t inner = 1;
    for (int a = d + 1; a < ndim; ++a) inner *= modes[a];
    float2* dst = (d == 0) ? xhat : bufs[stage % 2];
    const int rc = c2c_axis_fwd(src, dst, outer, sizes[d], inner, modes[d],
                                complex_fwd_off(d, ndim, sizes[d], modes[d]),
                                d == 0 ? (float)scale : 1.f, st);
    if (rc) return rc;
    src = dst;
  }
  return FNO_OK;
}

size_t fft_window_c2c_ws(int64_t planes, int32_t ndim, const int32_t* sizes, const int32_t* modes) {
  return (size_t)stage_buffers(ndim) * fwd_buffer_elems(planes, ndim, sizes, modes) * sizeof(float2);
}

int ifft_window_c2c(const float2* yhat, const float* bias, float2* y, int64_t batch,
                    int32_t channels, int32_t ndim, const int32_t* in_sizes,
                    const int32_t* out_sizes, const int32_t* modes, int32_t norm, void* ws,
                    size_t ws_bytes, hipStream_t st) {
  const int64_t planes = batch * channels;
  const double scale = inverse_scale(norm, out_sizes, ndim);
  const int64_t eb = inv_buffer_elems(planes, ndim, out_sizes, modes);
  const size_t need = (size_t)stage_buffers(ndim) * eb * sizeof(float2);
  if (ws_bytes < need) {
    set_error("ifft_window: workspace %zu < %zu bytes", ws_bytes, need);
    return FNO_ERR_WORKSPACE;
  }
  float2* bufs[2] = {reinterpret_cast<float2*>(ws), reinterpret_cast<float2*>(ws) + eb};
  const float2* src = yhat;
  for (int d = 0; d < ndim; ++d) {
    int64_t outer = planes;
    for (int a = 0; a < d; ++a) outer *= out_sizes[a];
    int64_t inner = 1;
    for (int a = d + 1; a < ndim; ++a) inner *= modes[a];
    const bool last = d == ndim - 1;
    float2* dst = last ? y : bufs[d % 2];
    const int off = last ? 0 : -(modes[d] / 2);
    const int rc = c2c_axis_inv(src, dst, outer, in_sizes[d], out_sizes[d], inner, modes[d], off,
                                last ? (float)scale : 1.f, st);
    if (rc) return rc;
    src = dst;
  }
  if (bias) {
    int64_t per_plane = 1;
    for (int a = 0; a < ndim; ++a) per_plane *= out_sizes[a];
    hipLaunchKernelGGL(k_add_bias_re, dim3(grid_for(planes * per_plane)), dim3(kThreads), 0, st, y,
                       bias, per_plane, channels, planes * per_plane);
    return launch_status("k_add_bias_re");
  }
  return FNO_OK;
}

size_t ifft_window_c2c_ws(int64_t planes, int32_t ndim, const int32_t* out_sizes,
                          const int32_t* modes) {
  return (size_t)stage_buffers(ndim) * inv_buffer_elems(planes, ndim, out_sizes, modes) *
         sizeof(float2);
}

// The inverse transforms of every axis but the last (unscaled), from the
// window spectrum into the workspace's stage buffers (eb elements each):
// *out ends as [planes][out_0 .. out_{ndim-2}][m_last] (yhat itself in 1D).
static int inverse_nonlast(const float2* yhat, int64_t planes, int32_t ndim,
                           const int32_t* in_sizes, const int32_t* out_sizes,
                           const int32_t* modes, void* ws, int64_t eb, const float2** out,
                           hipStream_t st) {
  float2* bufs[2] = {reinterpret_cast<float2*>(ws), reinterpret_cast<float2*>(ws) + eb};
  const float2* src = yhat;
  // 3D, 64 x 64 leading axes: both in one pass, written where stage 1 writes
  if (ndim == 3 && axis_inv64x2_supported(in_sizes[0], out_sizes[0], modes[0], in_sizes[1],
                                          out_sizes[1], modes[1], modes[2])) {
    const int rc = axis_inv64x2(yhat, bufs[1], planes, modes[0], modes[1], modes[2], 1.f, st);
    if (rc) return rc;
    *out = bufs[1];
    return FNO_OK;
  }
  for (int d = 0; d < ndim - 1; ++d) {
    int64_t outer = planes;
    for (int a = 0; a < d; ++a) outer *= out_sizes[a];
    int64_t inner = 1;
    for (int a = d + 1; a < ndim; ++a) inner *= modes[a];
    float2* dst = bufs[d % 2];
    const int N = in_sizes[d], Np = out_sizes[d], m = modes[d];
    const int rc = c2c_axis_inv(src, dst, outer, N, Np, inner, m, -(m / 2), 1.f, st);
    if (rc) return rc;
    src = dst;
  }
  *out = src;
  return FNO_OK;
}

int irfft_window(const float2* yhat, const float* bias, float* y, int64_t batch, int32_t channels,
                 int32_t ndim, const int32_t* in_sizes, const int32_t* out_sizes,
                 const int32_t* modes, int32_t norm, int32_t enforce, void* ws, size_t ws_bytes,
                 hipStream_t st) {
  const int64_t planes = batch * channels;
  const double scale = inverse_scale(norm, out_sizes, ndim);
  // stage d (d < ndim-1) expands axis d to out_sizes[d] into bufs[d % 2]
  const int64_t eb = inv_buffer_elems(planes, ndim, out_sizes, modes);
  const size_t need = (size_t)stage_buffers(ndim) * eb * sizeof(float2);
  if (ws_bytes < need) {
    set_error("irfft_window: workspace %zu < %zu bytes", ws_bytes, need);
    return FNO_ERR_WORKSPACE;
  }
  const float2* src = yhat;
  int rc0 = inverse_nonlast(yhat, planes, ndim, in_sizes, out_sizes, modes, ws, eb, &src, st);
  if (rc0) return rc0;
  {
    int64_t rows = planes;
    for (int a = 0; a < ndim - 1; ++a) rows *= out_sizes[a];
    const int N = in_sizes[ndim - 1], Np = out_sizes[ndim - 1], m = modes[ndim - 1];
    // rows run over (b, c, outer spatial...): the channel of a row is
    // (row / rows_per_plane) mod channels
    const int64_t rows_per_plane = rows / planes;
    if (c2r_fft_supported(Np, rows)) {
      int rc = c2r_fft(src, y, bias, rows, rows_per_plane, channels, N, Np, m, enforce,
                       (float)scale, st);
      if (rc) return rc;
    } else if (m <= 64 && rows >= 16384 && rows * (int64_t)(Np > 2 * m ? Np : 2 * m) * 4 <
                                                  (int64_t(1) << 31)) {
      // many rows: the synthesis product on the matrix cores; a workgroup's
      // four waves take 8 column tiles each of the same 16 rows
      constexpr int CT = 8;
      const int col_groups = ((Np + 15) / 16 + 4 * CT - 1) / (4 * CT);
      const unsigned blocks = (unsigned)(((rows + 15) / 16) * col_groups);
      hipLaunchKernelGGL(k_c2r_mfma<CT>, dim3(blocks), dim3(kThreads), (size_t)Np * 8, st, src, y,
                         bias, rows, rows_per_plane, channels, N, Np, m, enforce, col_groups,
                         (float)scale);
      int rc = launch_status("k_c2r_mfma");
      if (rc) return rc;
    } else {
      const int K = m < Np / 2 + 1 ? m : Np / 2 + 1;
      int rpb = kThreads / (Np < kThreads ? Np : kThreads);
      // rows enough for 2048 workgroups: more rows per workgroup, so the
      // Np-entry twiddle table each one builds is shared, within 48 KB of LDS
      if (rows / 2048 > rpb) {
        const int64_t lds_rows = (48 * 1024 - (int64_t)Np * 8) / ((int64_t)K * 8);
        rpb = (int)(rows / 2048 < lds_rows ? rows / 2048 : lds_rows);
      }
      if (rpb < 1) rpb = 1;
      if (rpb > 32) rpb = 32;
      const size_t lds = (size_t)Np * 8 + (size_t)rpb * K * 8;
      hipLaunchKernelGGL(k_c2r_direct, dim3((unsigned)((rows + rpb - 1) / rpb)), dim3(kThreads),
                         lds, st, src, y, bias, rows, rows_per_plane, channels, N, Np, m, enforce,
                         rpb, (float)scale);
      int rc = launch_status("k_c2r_direct");
      if (rc) return rc;
    }
  }
  return FNO_OK;
}

bool line_epilogue_supported(int W, int Ci, int Co, int m2h, int skip_kind);
int line_epilogue(const float2* z, const float* x, const float* skip_w, const float* bias,
                  float* y, int B, int Ci, int Co, int64_t L, int m2h, int skip_kind, int act,
                  float scale, hipStream_t st);
int block_epilogue(const float* spec, const float* x, const float* ws, float* y, int B, int Ci,
                   int Co, int64_t P, int skip_kind, int act, hipStream_t st);

// The inverse window transform (output on the input grid) with the bias, the
// skip and the activation: y = act(irfft(yhat) + bias + skip(x)).  Lines the
// line epilogue covers take the last axis, bias, skip and activation in one
// kernel from the non-last stages' output (no spectral field in memory);
// otherwise the inverse transform writes y and the block epilogue finishes it
// in place.  Workspace: irfft_window_ws(batch * out_channels, ...).
int irfft_epilogue(const float2* yhat, const float* bias, const float* x, const float* skip_w,
                   float* y, int B, int Ci, int Co, int32_t ndim, const int32_t* sizes,
                   const int32_t* modes, int32_t norm, int32_t skip_kind, int32_t act, void* ws,
                   size_t ws_bytes, hipStream_t st) {
  const int64_t planes = (int64_t)B * Co;
  const int W = sizes[ndim - 1], m2h = modes[ndim - 1];
  const bool aligned = (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) % 16 == 0;
  if (aligned && line_epilogue_supported(W, Ci, Co, m2h, skip_kind)) {
    const int64_t eb = inv_buffer_elems(planes, ndim, sizes, modes);
    const size_t need = (size_t)stage_buffers(ndim) * eb * sizeof(float2);
    if (ws_bytes < need) {
      set_error("inverse + epilogue: workspace %zu < %zu bytes", ws_bytes, need);
      return FNO_ERR_WORKSPACE;
    }
    const float2* z = yhat;
    int rc = inverse_nonlast(yhat, planes, ndim, sizes, sizes, modes, ws, eb, &z, st);
    if (rc) return rc;
    int64_t L = 1;
    for (int d = 0; d + 1 < ndim; ++d) L *= sizes[d];
    return line_epilogue(z, x, skip_w, bias, y, B, Ci, Co, L, m2h, skip_kind, act,
                         (float)inverse_scale(norm, sizes, ndim), st);
  }
  int rc = irfft_window(yhat, bias, y, B, Co, ndim, sizes, sizes, modes, norm, 1, ws, ws_bytes, st);
  if (rc) return rc;
  if (skip_kind == FNO_SKIP_NONE && act == FNO_ACT_NONE) return FNO_OK;
  int64_t P = 1;
  for (int d = 0; d < ndim; ++d) P *= sizes[d];
  return block_epilogue(y, x, skip_w, y, B, Ci, Co, P, skip_kind, act, st);
}

bool contract_mfma_supported(int B, int Ci, int Co, int64_t M, int64_t sWi, int64_t sWo,
                             int64_t sWk);
int contract_mfma(const float2* X, const float2* W, float2* Y, int B, int Ci, int Co, int64_t M,
                  hipStream_t st, int ymap_w);

// ymap_w: the output mode order (ymap_index); 0 for the window order.
int contract_dense(const float2* X, const float2* W, float2* Y, int B, int Ci, int Co, int64_t M,
                   int64_t sWi, int64_t sWo, int64_t sWk, hipStream_t st, int ymap_w) {
  // few modes: the MFMA kernel's grid (a workgroup per 8+ modes and 32
  // output channels) would leave most CUs idle; spread the outputs instead
  const int64_t outs = (int64_t)B * Co * M;
  if (M <= 64 && outs <= (int64_t(1) << 20)) {
    const int64_t blocks = (outs * 16 + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(k_contract_small, dim3((unsigned)blocks), dim3(kThreads), 0, st, X, W, Y, B,
                       Ci, Co, M, sWi, sWo, sWk, ymap_w);
    return launch_status("k_contract_small");
  }
  if (contract_mfma_supported(B, Ci, Co, M, sWi, sWo, sWk))
    return contract_mfma(X, W, Y, B, Ci, Co, M, st, ymap_w);
  constexpr int TB = 4, TO = 8;
  const int nTiles = ((B + TB - 1) / TB) * ((Co + TO - 1) / TO);
  const int wavesPerBlock = kThreads / 64;
  dim3 grid((unsigned)((M + 63) / 64), (unsigned)((nTiles + wavesPerBlock - 1) / wavesPerBlock));
  hipLaunchKernelGGL((k_contract_dense<TB, TO>), grid, dim3(kThreads), 0, st, X, W, Y, B, Ci, Co, M,
                     sWi, sWo, sWk, ymap_w);
  return launch_status("k_contract_dense");
}

int contract_separable(const float2* X, const float2* W, float2* Y, int B, int C, int64_t M,
                       hipStream_t st) {
  const int64_t total = (int64_t)B * C * M;
  hipLaunchKernelGGL(k_contract_separable, dim3(grid_for(total)), dim3(kThreads), 0, st, X, W, Y,
                     (int64_t)C * M, total);
  return launch_status("k_contract_separable");
}

int axis_matmul(const float2* in, const float2* mat, float2* out, int64_t outer, int A, int J,
                int64_t inner, hipStream_t st) {
  hipLaunchKernelGGL(k_axis_matmul, dim3(grid_for(outer * J * inner)), dim3(kThreads), 0, st, in,
                     mat, out, outer, A, J, inner);
  return launch_status("k_axis_matmul");
}

template <int OT, int PP>
static int launch_epilogue(const float* spec, const float* x, const float* ws, float* y, int B,
                           int Ci, int Co, int64_t P, int skip_kind, int act, hipStream_t st) {
  const int64_t per = (int64_t)kThreads * PP;
  dim3 grid((unsigned)((P + per - 1) / per), (unsigned)((Co + OT - 1) / OT), (unsigned)B);
  const size_t lds = skip_kind == FNO_SKIP_LINEAR ? (size_t)((Ci + 7) / 8 * 8) * OT * sizeof(float) : 0;
  if (lds > 160 * 1024) {
    set_error("block epilogue: %d input channels exceed the staged skip weights", Ci);
    return FNO_ERR_UNSUPPORTED;
  }
  if (lds > 48 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_epilogue<OT, PP>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
      set_error("block epilogue: %s", hipGetErrorString(e));
      return FNO_ERR_HIP;
    }
  }
  hipLaunchKernelGGL((k_epilogue<OT, PP>), grid, dim3(kThreads), lds, st, spec, x, ws, y, B, Ci, Co,
                     P, skip_kind, act);
  return launch_status("k_epilogue");
}

bool skip_gemm_supported(int Ci, int Co, int64_t P, const void* x, const void* spec,
                         const void* y);
int skip_gemm(const float* x, const float* ws, const float* spec, float* y, int64_t B, int Ci,
              int Co, int64_t P, int act, hipStream_t st);

int block_epilogue(const float* spec, const float* x, const float* ws, float* y, int B, int Ci,
                   int Co, int64_t P, int skip_kind, int act, hipStream_t st) {
  // the linear skip as an MFMA GEMM with the spectral term added in its epilogue
  if (skip_kind == FNO_SKIP_LINEAR && skip_gemm_supported(Ci, Co, P, x, spec, y))
    return skip_gemm(x, ws, spec, y, B, Ci, Co, P, act, st);
  // vector access needs every (b, c) row to start on the vector boundary
  const uintptr_t addr = reinterpret_cast<uintptr_t>(spec) | reinterpret_cast<uintptr_t>(x) |
                         reinterpret_cast<uintptr_t>(y);
  const bool v4 = P % 4 == 0 && addr % 16 == 0, v2 = P % 2 == 0 && addr % 8 == 0;
  // wide output blocks while their staged weights stay small
  const bool wide_ok = skip_kind != FNO_SKIP_LINEAR || (size_t)Ci * 64 * sizeof(float) <= 64 * 1024;
  // OT x PP = 64 accumulators per thread
  if (Co <= 16 || !wide_ok)
    return v4 ? launch_epilogue<16, 4>(spec, x, ws, y, B, Ci, Co, P, skip_kind, act, st)
              : launch_epilogue<16, 1>(spec, x, ws, y, B, Ci, Co, P, skip_kind, act, st);
  if (Co <= 32)
    return v2 ? launch_epilogue<32, 2>(spec, x, ws, y, B, Ci, Co, P, skip_kind, act, st)
              : launch_epilogue<32, 1>(spec, x, ws, y, B, Ci, Co, P, skip_kind, act, st);
  return launch_epilogue<64, 1>(spec, x, ws, y, B, Ci, Co, P, skip_kind, act, st);
}

int validate_window(int32_t ndim, const int32_t* sizes, const int32_t* modes) {
  return validate_axes(ndim, sizes, modes);
}

size_t rfft_window_ws(int64_t planes, int32_t ndim, const int32_t* sizes, const int32_t* modes) {
  return (size_t)stage_buffers(ndim) * fwd_buffer_elems(planes, ndim, sizes, modes) * sizeof(float2);
}

size_t irfft_window_ws(int64_t planes, int32_t ndim, const int32_t* out_sizes,
                       const int32_t* modes) {
  return (size_t)stage_buffers(ndim) * inv_buffer_elems(planes, ndim, out_sizes, modes) *
         sizeof(float2);
}

}  // namespace fno
