// Last-axis transforms of the generic path for power-of-two lines of 64, 128
// and 256 points, by LDS-exchanged line FFTs instead of direct sums:
//
//   k_r2c_fft   rows of N reals -> the first m rfft bins, scaled
//   k_c2r_fft   rows of m half-spectrum bins -> Np reals (irfft(n = Np)),
//               scaled, + per-channel bias
//
// Two rows share one complex line (real parts one row, imaginary parts the
// other).  A 256-thread workgroup runs 256 / T lines; the rows of a workgroup
// are contiguous in memory and move through LDS with 16-byte accesses.
// Semantics are those of the direct kernels in fno_generic.hip (the rfft half
// spectrum, and for the inverse the Hermitian extension with the imaginary
// part of bin 0 -- and of bin N/2 under enforce_hermitian_symmetry --
// dropped; spectral_convolution.py:443, :547-559).
#include "fno_fft_lds.h"
#include "fno_twiddle.h"

namespace fno {

namespace {
constexpr int kFftThreads = 256;
template <int N>
struct RowPlan {
  static constexpr int T = LinePlan<N>::T, R = LinePlan<N>::R, Q = LinePlan<N>::Q;
  static constexpr int LINES = kFftThreads / T;    // lines (row pairs) per workgroup
  static constexpr int ROWS = 2 * LINES;
  static constexpr int EXS = N + 4;                // line slice (float2); 16-byte multiple
};
}  // namespace

template <int N>
__global__ void __launch_bounds__(kFftThreads)
k_r2c_fft(const float* __restrict__ x, float2* __restrict__ out, int64_t rows, int m, float scale) {
  using P = RowPlan<N>;
  constexpr int T = P::T, R = P::R, Q = P::Q, EXS = P::EXS;
  extern __shared__ float4 smem4[];
  float2* tw = reinterpret_cast<float2*>(smem4);
  float2* exall = tw + N;
  fill_twiddles<N>(tw);
  const int64_t r0 = (int64_t)blockIdx.x * P::ROWS;
  const int nr = (int)min((int64_t)P::ROWS, rows - r0);
  // rows r0 .. r0 + nr into the slices: row r at slice r / 2, floats
  // [(r % 2) N, (r % 2 + 1) N); missing rows read as zero
  {
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + r0 * N, (uint32_t)(nr * N * 4));
    for (int q = threadIdx.x; q < P::ROWS * N / 4; q += kFftThreads) {
      const int r = q / (N / 4), c4 = q % (N / 4);
      const float4 v = __builtin_bit_cast(
          float4, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)((uint32_t)q * 16u), 0, 0));
      *reinterpret_cast<float4*>(reinterpret_cast<float*>(exall + (r >> 1) * EXS) + (r & 1) * N +
                                 4 * c4) = v;
    }
  }
  __syncthreads();
  const int L = threadIdx.x / T, t = threadIdx.x % T;
  float2* ex = exall + L * EXS;
  const float* exf = reinterpret_cast<const float*>(ex);
  float2 v[R];
#pragma unroll
  for (int s = 0; s < R; ++s) v[s] = make_float2(exf[t + T * s], exf[N + t + T * s]);
  wave_sync();
  float2 o[Q][T];
  line_fft<N, -1>(v, ex, tw, t, o);
#pragma unroll
  for (int q = 0; q < Q; ++q)
#pragma unroll
    for (int s = 0; s < T; ++s) {
      const int k = t + T * q + R * s;
      if (k < m || k > N - m) ex[k] = o[q][s];
    }
  wave_sync();
  // X_a[k] = (Z[k] + conj Z[N-k]) / 2,  X_b[k] = -i (Z[k] - conj Z[N-k]) / 2
  const int64_t ra = r0 + 2 * L;
  for (int k = t; k < m; k += T) {
    const float2 zk = ex[k];
    const float2 zn = ex[(N - k) & (N - 1)];
    const float2 a = make_float2(0.5f * (zk.x + zn.x), 0.5f * (zk.y - zn.y));
    const float2 b = make_float2(0.5f * (zk.y + zn.y), 0.5f * (zn.x - zk.x));
    if (2 * L < nr) out[ra * m + k] = cscale(a, scale);
    if (2 * L + 1 < nr) out[(ra + 1) * m + k] = cscale(b, scale);
  }
}

template <int NP>
__global__ void __launch_bounds__(kFftThreads)
k_c2r_fft(const float2* __restrict__ in, float* __restrict__ out, const float* __restrict__ bias,
          int64_t rows, int64_t rows_per_plane, int channels, int N, int m, int enforce,
          float scale) {
  using P = RowPlan<NP>;
  constexpr int T = P::T, R = P::R, Q = P::Q, EXS = P::EXS;
  extern __shared__ float4 smem4[];
  float2* tw = reinterpret_cast<float2*>(smem4);
  float2* exall = tw + NP;
  fill_twiddles<NP>(tw);
  const int64_t r0 = (int64_t)blockIdx.x * P::ROWS;
  const int nr = (int)min((int64_t)P::ROWS, rows - r0);
  const int K = min(m, NP / 2 + 1);
  const int L = threadIdx.x / T, t = threadIdx.x % T;
  float2* ex = exall + L * EXS;
  const int64_t ra = r0 + 2 * L;
  const bool has_a = 2 * L < nr, has_b = 2 * L + 1 < nr;
  // packed spectrum Z = A + i B of the line's two rows, Hermitian-extended
  for (int k = t; k < NP; k += T) ex[k] = make_float2(0.f, 0.f);
  wave_sync();
  for (int k = t; k < K; k += T) {
    float2 a = has_a ? in[ra * m + k] : make_float2(0.f, 0.f);
    float2 b = has_b ? in[(ra + 1) * m + k] : make_float2(0.f, 0.f);
    // bin 0, the Nyquist bin of the output length and (enforce) of the input
    // length are taken as real
    if (k == 0 || 2 * k == NP || (enforce && k == N / 2)) {
      a.y = 0.f;
      b.y = 0.f;
    }
    ex[k] = make_float2(a.x - b.y, a.y + b.x);                  // A + i B
    if (k > 0 && 2 * k < NP) ex[NP - k] = make_float2(a.x + b.y, b.x - a.y);   // conj A + i conj B
  }
  wave_sync();
  float2 v[R];
#pragma unroll
  for (int s = 0; s < R; ++s) v[s] = ex[t + T * s];
  wave_sync();
  float2 o[Q][T];
  line_fft<NP, +1>(v, ex, tw, t, o);
  const float ba = (bias && has_a) ? bias[(ra / rows_per_plane) % channels] : 0.f;
  const float bb = (bias && has_b) ? bias[((ra + 1) / rows_per_plane) % channels] : 0.f;
  // rows back through the slice as floats [row a | row b], then out with
  // 16-byte stores
  float* exf = reinterpret_cast<float*>(ex);
#pragma unroll
  for (int q = 0; q < Q; ++q)
#pragma unroll
    for (int s = 0; s < T; ++s) {
      const int n = t + T * q + R * s;
      exf[n] = fmaf(o[q][s].x, scale, ba);
      exf[NP + n] = fmaf(o[q][s].y, scale, bb);
    }
  __syncthreads();
  float4* og = reinterpret_cast<float4*>(out + r0 * NP);
  for (int q = threadIdx.x; q < nr * NP / 4; q += kFftThreads) {
    const int r = q / (NP / 4), c4 = q % (NP / 4);
    og[q] = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(exall + (r >> 1) * EXS) +
                                             (r & 1) * NP + 4 * c4);
  }
}

// Non-last axis, complex <-> complex, one line per (outer o, inner q) at a
// stride of `inner` entries.  A workgroup takes QB consecutive q of one o:
// the [L][QB] tile moves through LDS with coalesced row accesses and each line
// FFTs in its own tile column.  Row stride TS: with 8 lanes per line, 2 TS = 8
// mod 64 dwords puts a line's 8 lanes on 8 distinct bank groups in every pass
// of the strided FFT (TS = 40 put lanes t and t + 4 on the same banks).
//   forward (SIGN -1): L = N input points; out[o][j][q] = s X[(j + off) mod N]
//   inverse (SIGN +1): L = Np; window entry j goes to index (j + off) mod N
//                      when that is < Np (zero-padding / truncation of the
//                      length-N spectrum), out[o][n][q] for n < Np
// (off = -m/2 for the centred window of fftshift-ed axes)
template <int L, int SIGN>
__global__ void __launch_bounds__(kFftThreads)
k_c2c_fft_axis(const float2* __restrict__ in, float2* __restrict__ out, int64_t inner, int N,
               int m, int off, float scale) {
  using PL = LinePlan<L>;
  constexpr int T = PL::T, R = PL::R, Q = PL::Q;
  constexpr int QB = kFftThreads / T;
  constexpr int TS = (QB == 32) ? 36 : QB + 1;
  extern __shared__ float4 smem4[];
  float2* tw = reinterpret_cast<float2*>(smem4);
  float2* tile = tw + L;   // [L][TS]
  fill_twiddles<L>(tw);
  const int64_t nqb = (inner + QB - 1) / QB;
  const int64_t o = blockIdx.x / nqb;
  const int64_t q0 = (blockIdx.x % nqb) * QB;
  const int qn = (int)min((int64_t)QB, inner - q0);
  const int nin = (SIGN < 0) ? L : m;                 // entries per input line
  const int nout = (SIGN < 0) ? m : L;                // entries per output line
  const float2* src = in + o * (int64_t)nin * inner + q0;
  float2* dst = out + o * (int64_t)nout * inner + q0;
  if (SIGN < 0) {
    for (int i = threadIdx.x; i < L * QB; i += kFftThreads) {
      const int n = i / QB, g = i % QB;
      tile[n * TS + g] = g < qn ? src[(int64_t)n * inner + g] : make_float2(0.f, 0.f);
    }
  } else {
    for (int i = threadIdx.x; i < L * QB; i += kFftThreads) tile[(i / QB) * TS + i % QB] =
        make_float2(0.f, 0.f);
    __syncthreads();
    for (int i = threadIdx.x; i < m * QB; i += kFftThreads) {
      const int j = i / QB, g = i % QB;
      int t = (j + off) % N;
      if (t < 0) t += N;
      if (t < L && g < qn) tile[t * TS + g] = src[(int64_t)j * inner + g];
    }
  }
  __syncthreads();
  {
    const int g = threadIdx.x / T, t = threadIdx.x % T;
    float2* col = tile + g;
    float2 v[R];
#pragma unroll
    for (int s = 0; s < R; ++s) v[s] = col[(t + T * s) * TS];
    wave_sync();
    float2 o[Q][T];
    line_fft_strided<L, SIGN>(v, col, TS, tw, t, o);
#pragma unroll
    for (int q = 0; q < Q; ++q)
#pragma unroll
      for (int s = 0; s < T; ++s) col[(t + T * q + R * s) * TS] = o[q][s];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < nout * QB; i += kFftThreads) {
    const int j = i / QB, g = i % QB;
    int k = j;
    if (SIGN < 0) {
      k = (j + off) % L;
      if (k < 0) k += L;
    }
    if (g < qn) dst[(int64_t)j * inner + g] = cscale(tile[k * TS + g], scale);
  }
}

// ------------------------------------------------------------------- host
static bool pow2_line(int n) { return n == 64 || n == 128 || n == 256; }

template <int N>
static size_t row_fft_lds() {
  return (size_t)(N + RowPlan<N>::LINES * RowPlan<N>::EXS) * sizeof(float2);
}

bool r2c_fft_supported(int N, int m, int64_t rows) {
  return pow2_line(N) && m >= 1 && m <= N / 2 + 1 && rows * N * 4 < (int64_t(1) << 31);
}

template <int N>
static int launch_r2c(const float* x, float2* out, int64_t rows, int m, float scale,
                      hipStream_t st) {
  const int64_t blocks = (rows + RowPlan<N>::ROWS - 1) / RowPlan<N>::ROWS;
  hipLaunchKernelGGL(k_r2c_fft<N>, dim3((unsigned)blocks), dim3(kFftThreads), row_fft_lds<N>(), st,
                     x, out, rows, m, scale);
  return launch_status("k_r2c_fft");
}

int r2c_fft(const float* x, float2* out, int64_t rows, int N, int m, float scale, hipStream_t st) {
  if (N == 64) return launch_r2c<64>(x, out, rows, m, scale, st);
  if (N == 128) return launch_r2c<128>(x, out, rows, m, scale, st);
  return launch_r2c<256>(x, out, rows, m, scale, st);
}

bool c2r_fft_supported(int Np, int64_t rows) { return pow2_line(Np) && rows >= 1; }

template <int NP>
static int launch_c2r(const float2* in, float* out, const float* bias, int64_t rows,
                      int64_t rows_per_plane, int channels, int N, int m, int enforce, float scale,
                      hipStream_t st) {
  const int64_t blocks = (rows + RowPlan<NP>::ROWS - 1) / RowPlan<NP>::ROWS;
  hipLaunchKernelGGL(k_c2r_fft<NP>, dim3((unsigned)blocks), dim3(kFftThreads), row_fft_lds<NP>(),
                     st, in, out, bias, rows, rows_per_plane, channels, N, m, enforce, scale);
  return launch_status("k_c2r_fft");
}

int c2r_fft(const float2* in, float* out, const float* bias, int64_t rows, int64_t rows_per_plane,
            int channels, int N, int Np, int m, int enforce, float scale, hipStream_t st) {
  if (Np == 64)
    return launch_c2r<64>(in, out, bias, rows, rows_per_plane, channels, N, m, enforce, scale, st);
  if (Np == 128)
    return launch_c2r<128>(in, out, bias, rows, rows_per_plane, channels, N, m, enforce, scale, st);
  return launch_c2r<256>(in, out, bias, rows, rows_per_plane, channels, N, m, enforce, scale, st);
}

// the grid is one workgroup per (outer, QB inner entries)
bool c2c_fft_supported(int L, int64_t outer, int64_t inner) {
  if (!pow2_line(L)) return false;
  const int QB = kFftThreads / (L >= 256 ? 16 : 8);
  return outer * ((inner + QB - 1) / QB) <= 0x7fffffff;
}

template <int L, int SIGN>
static int launch_c2c(const float2* in, float2* out, int64_t outer, int64_t inner, int N, int m,
                      int off, float scale, hipStream_t st) {
  constexpr int QB = kFftThreads / LinePlan<L>::T;
  constexpr int TS = (QB == 32) ? 36 : QB + 1;
  const size_t lds = (size_t)(L + L * TS) * sizeof(float2);
  const int64_t blocks = outer * ((inner + QB - 1) / QB);
  hipLaunchKernelGGL((k_c2c_fft_axis<L, SIGN>), dim3((unsigned)blocks), dim3(kFftThreads), lds,
                     st, in, out, inner, N, m, off, scale);
  return launch_status("k_c2c_fft_axis");
}

// forward: lines of N points -> m window modes (entry j = frequency j + off)
int c2c_fft_fwd(const float2* in, float2* out, int64_t outer, int64_t inner, int N, int m, int off,
                float scale, hipStream_t st) {
  if (N == 64) return launch_c2c<64, -1>(in, out, outer, inner, N, m, off, scale, st);
  if (N == 128) return launch_c2c<128, -1>(in, out, outer, inner, N, m, off, scale, st);
  return launch_c2c<256, -1>(in, out, outer, inner, N, m, off, scale, st);
}

// inverse: m window modes of a length-N spectrum -> lines of Np points
int c2c_fft_inv(const float2* in, float2* out, int64_t outer, int64_t inner, int N, int Np, int m,
                int off, float scale, hipStream_t st) {
  if (Np == 64) return launch_c2c<64, +1>(in, out, outer, inner, N, m, off, scale, st);
  if (Np == 128) return launch_c2c<128, +1>(in, out, outer, inner, N, m, off, scale, st);
  return launch_c2c<256, +1>(in, out, outer, inner, N, m, off, scale, st);
}

}  // namespace fno
