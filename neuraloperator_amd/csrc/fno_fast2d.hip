// Fused 2D spectral block for power-of-two planes (H in {64,128,256},
// W in {128,256}):
//
//   y = act( irfft2_window( contract( rfft2_window(x) ) ) + bias + skip(x) )
//
// K1  k_fwd_stream     one workgroup per (b, c) plane, streaming the plane in
//                      D = H/32 chunks of 32 rows h = c + D*h2 (h2 < 32):
//                        * row real FFTs (two rows packed as one complex line,
//                          LDS-exchanged four-step) keep the m2h kept bins;
//                        * a 32-point DFT down each kept column of the chunk
//                          (4 lanes x 8 points) gives the chunk's spectrum at
//                          every frequency mod 32;
//                        * the twiddle w_H^(-kh c) folds it into register
//                          accumulators of the m1 kept rows.
//                      x is read once, 16-byte loads, the next chunk's rows in
//                      flight; 39 KB of LDS and <= 128 VGPRs let 4 workgroups
//                      share a CU.
// K2  contraction      fno_contract.hip (mode-wise complex GEMM on bf16-split MFMA).
// K3  k_inv_cols       one workgroup per (b, o) plane: inverse FFT along H of
//                      the m2h kept columns (zero-padded window rows), written
//                      as one contiguous block Z[b][o][h][kw].
// K4  k_row_epilogue_r one workgroup per (b, TR consecutive rows); per row:
//                        * inverse row real FFTs of all output channels (two
//                          channels per complex line) straight into the
//                          accumulators of the skip GEMM (v_mfma_f32_16x16x4f32
//                          output layout = line FFT output layout);
//                        * the 1x1-conv skip on fp32 MFMA, x streamed through
//                          an LDS ring with the next row's loads in flight;
//                        * bias, gated skip add and erf GELU in registers, one
//                          write of y.
//                      At W = 128 a step is two adjacent rows, one per 8-lane
//                      half of each 16-lane group.
//                      (k_row_epilogue: the LDS-staged variant for the
//                      channel counts K4 does not cover.)
//
// Semantics follow SpectralConv.forward (neuralop/layers/spectral_convolution.py
// :429-568) with output size == input size, and the post-activation block of
// FNOBlocks (neuralop/layers/fno_block.py:331-361).
#include "fno_fft_lds.h"
#include "fno_twiddle.h"

#include <type_traits>

namespace fno {

typedef float v16f __attribute__((ext_vector_type(16)));

// ------------------------------------------------------------------------ K1

// Kept window of a plane: rows kh in [kmin, kmin + m1), kmin = -(m1/2), stored
// at window row kh - kmin; columns kw < m2h.  A kept row kh is reached from its
// residue k' = kh mod 32 as kh = k0(k') + 32 e, k0 = kmin + ((k' - kmin) & 31).
//
// LDS: twW [W] | twH [H] | 16 line slices of EXS float2.  The 4 (W = 256) or
// 8 (W = 128) slices of one wavefront form its region; the chunk spectrum rows
// of the wavefront's lines (2 per line, stride SP) sit at the end of that
// region, so a wavefront writes them without waiting for the others.  The
// column stage exchanges its partial DFTs through the spectrum entries it has
// just read.
// BF: x is bfloat16 (the activation storage of the bf16 FNO forward), widened
// to fp32 as it is staged; everything after that is the same.
template <int H, int W, int KPR, bool BF = false>
__global__ void __launch_bounds__(16 * LinePlan<W>::T)
k_fwd_stream(const void* __restrict__ x, float2* __restrict__ xhat, int m1, int m2h, float scale) {
  using PW = LinePlan<W>;
  constexpr int T = PW::T, R = PW::R, Q = PW::Q;
  constexpr int D = H / 32;
  static_assert(H % 32 == 0 && D >= 1, "H must be a multiple of 32");
  constexpr int EXS = W + 16;                 // padded line slice (float2)
  constexpr int LPW = 64 / T;                 // lines per wavefront
  constexpr int WREG = LPW * EXS;             // wavefront region (float2)
  constexpr int NS = 4;                       // m2h <= 4T: split passes per lane
  extern __shared__ float4 smem4[];
  float2* twW = reinterpret_cast<float2*>(smem4);  // w_W^t, t < W
  float2* twH = twW + W;                             // w_H^t, t < H
  float2* exall = twH + H;
  // spectrum row r = 2 * line + (0 | 1), stride SP float2: >= m2h (<= 64),
  // = 8 (mod 32) so the 4 rows a half-wave reads in the column stage sit 16
  // banks apart, and a compile-time constant so row addresses fold into
  // instruction offsets
  constexpr int SP = 72;
  constexpr int sbase = WREG - 2 * LPW * SP;
  static_assert(sbase >= 0, "spectrum rows fit the wavefront region");
  auto srow = [&](int r) __attribute__((always_inline)) {
    return exall + (__mul24(r / (2 * LPW), WREG) + sbase + __mul24(r % (2 * LPW), SP));
  };
  fill_twiddles<W>(twW);
  fill_twiddles<H>(twH);

  const int tid = threadIdx.x;
  const int L = tid / T, t = tid % T;     // line of the chunk, lane in the line
  constexpr int ES = BF ? 2 : 4;              // bytes per element of x
  const char* xp = static_cast<const char*>(x) + (int64_t)blockIdx.x * H * W * ES;

  // column stage roles: 4 lanes per kept column
  const int col = tid >> 2, j = tid & 3;
  const bool col_on = col < m2h;
  const int kmin = -(m1 / 2);
  float2 acc[2][4][KPR];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int e = 0; e < KPR; ++e) acc[a][b][e] = make_float2(0.f, 0.f);

  // rows of line L in chunk c: h = c + D*(2L), c + D*(2L+1).  Each lane
  // loads 4 float4 of each row (16 lanes x 16 B = 256 contiguous bytes per
  // load instruction) one chunk ahead; at the chunk they are staged in the
  // line's own LDS slice and read back in the FFT's stride-T layout.
  constexpr int EPL = 16 / ES;        // elements per 16-byte load
  constexpr int NF4 = W / (EPL * T);  // 16-byte loads per lane and row
  static_assert(NF4 * EPL * T == W, "row split");
  const __amdgpu_buffer_rsrc_t rxp = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(xp), (short)0, H * W * ES, 0x00020000);
  // cache policy 2 = non-temporal (nt): x streams through once here, and
  // keeping it out of the caches' recent set measured 17 us faster at
  // B32 C64 256^2 (the caches keep what the following kernels reuse)
  constexpr int kNT = 2;
  auto load_rows = [&](uint32_t row, int lt, float4 (&dst)[2 * NF4]) __attribute__((always_inline)) {
    const uint32_t off = (row * W + EPL * lt) * (uint32_t)ES;
#pragma unroll
    for (int k = 0; k < NF4; ++k) {
      dst[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                              rxp, (int)(off + 16u * T * k), 0, kNT));
      dst[NF4 + k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                    rxp, (int)(off + 16u * T * k), D * W * ES, kNT));
    }
  };
  // Chunk order: workgroups that share an XCD (ids 8 apart) start at
  // different residues, which spreads the concurrent row reads (D rows apart
  // within a chunk) over the HBM channels: ~4.5 -> ~5.8 TB/s for this pattern.
  const int rot = (int)(blockIdx.x >> 3) & (D - 1);
  float4 xs4[2 * NF4];
  load_rows((uint32_t)(rot + D * (2 * L)), t, xs4);
  __syncthreads();

#pragma unroll 1
  for (int cs = 0; cs < D; ++cs) {
    const int c = (cs + rot) & (D - 1);
    // thread index laundered through an empty asm so per-lane addresses are
    // recomputed in the loop rather than hoisted into live registers
    int tl = tid;
    asm volatile("" : "+v"(tl));
    const int Ll = tl / T, tt = tl % T;
    float2* exl = exall + Ll * EXS;
    float2 v[R];
    {
      float* exf = reinterpret_cast<float*>(exl);   // rows a | b
#pragma unroll
      for (int k = 0; k < NF4; ++k) {
        if constexpr (BF) {
          // 8 bf16 of pixels 8 (tt + T k) .. + 7: widen (bits << 16)
          auto widen = [](float4 p, float4* d) __attribute__((always_inline)) {
            const uint4 u = __builtin_bit_cast(uint4, p);
            d[0] = make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                               __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
            d[1] = make_float4(__uint_as_float(u.z << 16), __uint_as_float(u.z & 0xffff0000u),
                               __uint_as_float(u.w << 16), __uint_as_float(u.w & 0xffff0000u));
          };
          widen(xs4[k], reinterpret_cast<float4*>(exf) + 2 * (tt + T * k));
          widen(xs4[NF4 + k], reinterpret_cast<float4*>(exf + W) + 2 * (tt + T * k));
        } else {
          reinterpret_cast<float4*>(exf)[tt + T * k] = xs4[k];
          reinterpret_cast<float4*>(exf + W)[tt + T * k] = xs4[NF4 + k];
        }
      }
      if (cs + 1 < D)  // next chunk's rows in flight during this chunk
        load_rows((uint32_t)(((c + 1) & (D - 1)) + D * (2 * Ll)), tt, xs4);
      wave_sync();
#pragma unroll
      for (int s = 0; s < R; ++s) v[s] = make_float2(exf[tt + T * s], exf[W + tt + T * s]);
    }
    // ---- row pair FFT; bins k < 4T and k > W - 4T (a superset of the kept
    // k < m2h and their mirrors) go back to the slice
    {
      float2 out[Q][T];
      line_fft<W, -1>(v, exl, twW, tt, out);
#pragma unroll
      for (int q = 0; q < Q; ++q)
#pragma unroll
        for (int s = 0; s < T; ++s) {
          if (T * q + R * s < 4 * T || T * q + R * s + T - 1 > W - 4 * T)
            exl[tt + T * q + R * s] = out[q][s];
        }
      wave_sync();
      // X_a[k] = (Z[k] + conj Z[W-k]) / 2,  X_b[k] = -i (Z[k] - conj Z[W-k]) / 2
      float2 xa[NS], xb[NS];
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        const int k = tt + T * i;
        const float2 zk = exl[k];
        const float2 zn = exl[(W - k) & (W - 1)];
        xa[i] = make_float2(0.5f * (zk.x + zn.x), 0.5f * (zk.y - zn.y));
        xb[i] = make_float2(0.5f * (zk.y + zn.y), 0.5f * (zn.x - zk.x));
      }
      wave_sync();
      float2* sa = srow(2 * Ll);
      float2* sb = srow(2 * Ll + 1);
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        const int k = tt + T * i;
        if (k < m2h) {
          sa[k] = xa[i];
          sb[k] = xb[i];
        }
      }
    }
    __syncthreads();
    // ---- 32-point column DFTs of the chunk, folded into the kept rows
    if (col_on) {
      const int col = tl >> 2, j = tl & 3;
      float2 f[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) f[u] = srow(j + 4 * u)[col];
      dft8<-1>(f);
#pragma unroll
      for (int k1 = 1; k1 < 8; ++k1) f[k1] = cmulc(f[k1], twH[((j * k1) & 31) * D]);
      // exchange among the column's 4 lanes through the column's own 32
      // spectrum entries (all read above): slot (lane jj, k1) is row
      // ((jj + k1/2) & 3) + 4 k1, so both the writes (fixed k1) and the reads
      // (fixed jj, k1 = 2j + e2) of a half-wave touch 4 distinct rows mod 4
#pragma unroll
      for (int k1 = 0; k1 < 8; ++k1) srow(((j + (k1 >> 1)) & 3) + 4 * k1)[col] = f[k1];
      wave_sync();
      // w_H^(-kh c) for kh = k0 + 32 e is w_H^(-k0 c) * u^e, u = w_H^(-32 c)
      const float2 u = twH[(H - 32 * c) & (H - 1)];
#pragma unroll
      for (int e2 = 0; e2 < 2; ++e2) {
        const int k1 = 2 * j + e2;
        float2 g0 = srow(((0 + j) & 3) + 4 * k1)[col], g1 = srow(((1 + j) & 3) + 4 * k1)[col];
        float2 g2 = srow(((2 + j) & 3) + 4 * k1)[col], g3 = srow(((3 + j) & 3) + 4 * k1)[col];
        dft4<-1>(g0, g1, g2, g3);
        const float2 P[4] = {g0, g1, g2, g3};
#pragma unroll
        for (int k2 = 0; k2 < 4; ++k2) {
          const int kr = k1 + 8 * k2;  // frequency mod 32
          const int k0 = kmin + ((kr - kmin) & 31);
          // rows kh >= kmin + m1 accumulate too; they are never written
          // (-k0 c) mod H with a 24-bit multiply (|k0| <= 64, c < 8)
          float2 q = cmul(P[k2], twH[__mul24(-k0, c) & (H - 1)]);
          acc[e2][k2][0] = cadd(acc[e2][k2][0], q);
#pragma unroll
          for (int e = 1; e < KPR; ++e) {
            q = cmul(q, u);
            acc[e2][k2][e] = cadd(acc[e2][k2][e], q);
          }
        }
      }
    }
    __syncthreads();
  }
  if (col_on) {
    float2* op = xhat + (int64_t)blockIdx.x * m1 * m2h;
#pragma unroll
    for (int e2 = 0; e2 < 2; ++e2)
#pragma unroll
      for (int k2 = 0; k2 < 4; ++k2) {
        const int kr = 2 * j + e2 + 8 * k2;
        const int k0 = kmin + ((kr - kmin) & 31);
#pragma unroll
        for (int e = 0; e < KPR; ++e) {
          const int kh = k0 + 32 * e;
          if (kh < kmin + m1) op[(kh - kmin) * m2h + col] = cscale(acc[e2][k2][e], scale);
        }
      }
  }
}

// ------------------------------------------------------------------------ K3
// Inverse column transform of one (b, o) plane: the m2h kept columns of the
// window spectrum, zero-padded to H rows at their frequencies, inverse
// FFT-ed along H and written as Z[b][o][h][kw]: one contiguous block per
// plane, so the stores stream; K4 reads a 8*m2h-byte row per channel.  One
// group of T lanes per column; each group exchanges through its own column of
// the LDS result tile (odd row stride), so the tile is the only LDS (~70 KB at
// H = 256, m2h = 33) and two 512-thread workgroups share a CU.
template <int H>
__global__ void __launch_bounds__(1024)
k_inv_cols(const float2* __restrict__ yhat, float2* __restrict__ z, int Co, int m1, int m2h) {
  using PH = LinePlan<H>;
  constexpr int T = PH::T, R = PH::R, Q = PH::Q;
  extern __shared__ float4 smem4[];
  float2* twH = reinterpret_cast<float2*>(smem4);
  const int TS = m2h | 1;
  float2* zs = twH + H;          // [H][TS]
  fill_twiddles<H>(twH);
  const int plane = blockIdx.x;  // b * Co + o
  const int b = plane / Co, o = plane - b * Co;
  const float2* win = yhat + (int64_t)plane * m1 * m2h;   // [m1][m2h] window
  const int nthreads = blockDim.x;
  __syncthreads();
  {
    const int g = threadIdx.x / T, t = threadIdx.x % T;
    const int G = nthreads / T;
    const int pos = m1 - m1 / 2, neg = m1 / 2;
    // rows outside the window read past the end of the buffer: zero
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(win, (uint32_t)(m1 * m2h * 8));
    for (int kw = g; kw < m2h; kw += G) {
      float2 v[R];
#pragma unroll
      for (int s = 0; s < R; ++s) {
        const int k = t + T * s;  // frequency index mod H
        int j = -1;
        if (k < pos) j = k + neg;
        else if (k >= H - neg) j = k - H + neg;
        const uint32_t off = j >= 0 ? (uint32_t)(j * m2h + kw) * 8u : 0x80000000u;
        v[s] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rw, (int)off, 0, 0));
      }
      // the four-step line FFT of fno_fft_lds.h, exchanging through the
      // column itself and storing the second pass straight back into it
      float2* col = zs + kw;
      dft_small<R, +1>(v);
#pragma unroll
      for (int k1 = 1; k1 < R; ++k1) v[k1] = cmul(v[k1], twH[t * k1]);
      wave_sync();
#pragma unroll
      for (int k1 = 0; k1 < R; ++k1) col[(k1 * T + (t ^ (k1 & (T - 1)))) * TS] = v[k1];
      wave_sync();
      float2 u[Q][T];
#pragma unroll
      for (int q = 0; q < Q; ++q)
#pragma unroll
        for (int s = 0; s < T; ++s) u[q][s] = col[((t + T * q) * T + (s ^ t)) * TS];
#pragma unroll
      for (int q = 0; q < Q; ++q) dft_small<T, +1>(u[q]);
      wave_sync();
#pragma unroll
      for (int q = 0; q < Q; ++q)
#pragma unroll
        for (int s = 0; s < T; ++s) col[(t + T * q + R * s) * TS] = u[q][s];
    }
  }
  __syncthreads();
  // the plane's H x m2h block is contiguous in Z: 16-byte stores of bin pairs
  float4* zp = reinterpret_cast<float4*>(z + (int64_t)plane * H * m2h);
  for (int i = threadIdx.x; i < H * m2h / 2; i += nthreads) {
    const int i0 = 2 * i, h0 = i0 / m2h, k0 = i0 - h0 * m2h;
    const int i1 = i0 + 1, h1 = i1 / m2h, k1 = i1 - h1 * m2h;
    const float2 a = zs[h0 * TS + k0], c = zs[h1 * TS + k1];
    zp[i] = make_float4(a.x, a.y, c.x, c.y);
  }
}

// ------------------------------------------------------------------------ K4
// MFMA 32x32x2 f32 operand/result layout (wave64):
//   A (32 x 2):  lane l supplies A[l % 32][l / 32]
//   B (2 x 32):  lane l supplies B[l / 32][l % 32]
//   D (32 x 32): lane l, register r holds D[8*(r/4) + 4*(l/32) + r%4][l % 32]
// Here M = output channels, N = pixels of the row, K = input channels.
//
// One workgroup runs TR (even) consecutive rows of one sample as a software
// pipeline.  Step s, between two barriers:
//   1. issue the loads of row s+1 (x operand, Z bins) into the idle buffers
//   2. the MFMA skip of row s, each k-step interleaved (sched_barrier) with
//      bias + GELU + store of EPK elements of row s-1, so the matrix cores and
//      the VALU work at the same time
//   3. inverse row FFTs of row s into spec buffer s & 1
// Accumulators, operands and spec buffers are double-buffered by row parity.
//
// LDS (floats): twW [2W] | wsT [CI*CO] | bias [CO] | spec [2][CO][W+8]
template <int W>
__host__ __device__ constexpr int spec_stride() { return W + 8; }

// Raw buffer resource over [base, base + bytes): loads and stores take a
// 32-bit VGPR byte offset plus an SGPR byte offset, so per-element address
// arithmetic stays 32-bit and mostly scalar.  Reads past the end return 0.
// soff must be wave-uniform; readfirstlane states that to the compiler so it
// stays in an SGPR.  The b32/b64 builtins move raw bits: values are bit-cast.
__device__ __forceinline__ float ld_f32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff,
                                                  __builtin_amdgcn_readfirstlane((int)soff), 0));
}
__device__ __forceinline__ float2 ld_f64(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(
      float2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff,
                                                   __builtin_amdgcn_readfirstlane((int)soff), 0));
}
__device__ __forceinline__ void st_f32(float v, __amdgpu_buffer_rsrc_t r, uint32_t voff,
                                       uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, (int)voff,
                                        __builtin_amdgcn_readfirstlane((int)soff), 0);
}

template <int H, int W, int CO, int CI, int NB>
__global__ void __launch_bounds__(CO / 2 * LinePlan<W>::T)
k_row_epilogue(const float* __restrict__ x, const float2* __restrict__ z,
               const float* __restrict__ skip_w, const float* __restrict__ bias,
               float* __restrict__ y, int TR, int m2h, int skip_kind, int act, float inv_scale) {
  using PW = LinePlan<W>;
  constexpr int T = PW::T, R = PW::R, Q = PW::Q;
  constexpr int BLOCK = CO / 2 * T;
  constexpr int SS = spec_stride<W>();
  constexpr int NPX = W / 32;                  // 32-pixel tiles of a row
  constexpr int MT_PER = (CO >= 64) ? 2 : 1;   // channel tiles per wave
  constexpr int NT_PER = 2 / MT_PER;           // pixel tiles per wave
  constexpr int KS = CI / 2;                   // MFMA k-steps
  constexpr int NEL = MT_PER * NT_PER * 16;    // epilogue elements per lane and row
  constexpr int EPK = NEL / KS;                // ... per k-step
  constexpr uint32_t HW = (uint32_t)H * W;
  static_assert(CO % 32 == 0 && CI % 2 == 0, "channel counts");
  static_assert((CO / 32) * NPX == 2 * (BLOCK / 64), "two MFMA tiles per wave");
  static_assert(NEL % KS == 0, "epilogue elements must spread evenly over the k-steps");
  extern __shared__ float4 smem4[];
  float2* twW = reinterpret_cast<float2*>(smem4);
  float* wsT = reinterpret_cast<float*>(twW + W);
  float* bS = wsT + (skip_kind == FNO_SKIP_LINEAR ? CI * CO : 0);
  float* spec = bS + CO + (CO & 1);   // [2][CO][SS]: irfft * scale + bias

  const int RB = H / TR;
  const int b = blockIdx.x / RB, h0 = (blockIdx.x % RB) * TR;
  const int tid = threadIdx.x, wave = tid >> 6;
  const bool linear = (skip_kind == FNO_SKIP_LINEAR);
  const bool gated = (skip_kind == FNO_SKIP_SOFT_GATING || skip_kind == FNO_SKIP_IDENTITY);
  const bool gelu_on = (act == FNO_ACT_GELU);
  const uint32_t gmask = act_mask(gelu_on);
  const int pxt0 = (CO >= 64) ? (wave % NPX) : 2 * wave;
  const int mt0 = (CO >= 64) ? 2 * (wave / NPX) : 0;
  // per-sample bases (uniform); buffer descriptors are built where used so
  // they stay in scalar registers
  const float* xs = x + (size_t)b * CI * HW;
  const float2* zs = z + (size_t)b * H * CO * m2h;
  float* ys = y + (size_t)b * CO * HW;
  constexpr uint32_t xbytes = CI * HW * 4u, ybytes = CO * HW * 4u;
  const uint32_t zbytes = (uint32_t)H * CO * m2h * 8u;

  fill_twiddles<W>(twW);
  if (linear)
    for (int i = tid; i < CI * CO; i += BLOCK) {
      const int ci = i / CO, o = i - ci * CO;
      wsT[i] = skip_w[o * CI + ci];
    }
  for (int i = tid; i < CO; i += BLOCK) bS[i] = bias ? bias[i] : 0.f;

  float xr[2][NT_PER][KS];
  float2 za[2][NB], zc[2][NB];   // bins k = t + T*n of channels 2g and 2g+1
  v16f acc[2][MT_PER][NT_PER];

  // ---- loads of row h into buffer BUF (tv: laundered thread index)
  auto load_row = [&](int h, int tv, auto buf_c) __attribute__((always_inline)) {
    constexpr int buf = decltype(buf_c)::value;
    const int ln = tv & 63;
    if (linear) {
      const __amdgpu_buffer_rsrc_t rx = make_rsrc(xs, xbytes);
      const uint32_t xo = ((uint32_t)(ln >> 5) * HW + (uint32_t)h * W + 32 * pxt0 + (ln & 31)) * 4u;
#pragma unroll
      for (int n = 0; n < NT_PER; ++n)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          xr[buf][n][ks] = __builtin_bit_cast(
              float, __builtin_amdgcn_raw_buffer_load_b32(rx, (int)(xo + 128u * n),
                                                          (int)((uint32_t)(2 * ks) * HW * 4u), 0));
    }
    const __amdgpu_buffer_rsrc_t rz = make_rsrc(zs, zbytes);
    const int tl = tv % T;
    // Z[b][o][h][kw]; bins past m2h read past the buffer end: zero
    const uint32_t zo = (((uint32_t)(2 * (tv / T)) * H + h) * m2h + tl) * 8u;
    const int m2o = __builtin_amdgcn_readfirstlane(H * m2h * 8);
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      const uint32_t off = (tl + T * n < m2h) ? zo + 8u * T * n : 0x80000000u;
      za[buf][n] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rz, (int)off, 0, 0));
      zc[buf][n] = __builtin_bit_cast(float2,
                                      __builtin_amdgcn_raw_buffer_load_b64(rz, (int)off, m2o, 0));
    }
  };

  // ---- inverse row FFTs of the Z bins in buffer BUF into spec buffer BUF,
  //      written as irfft * inv_scale + bias
  auto irfft_row = [&](int tv, auto buf_c) __attribute__((always_inline)) {
    constexpr int buf = decltype(buf_c)::value;
    const int gl = tv / T, tt = tv % T;
    float* rowa = spec + (buf * CO + 2 * gl) * SS;
    float2* ex = reinterpret_cast<float2*>(rowa);
    // stage the line's bins (Za[k], Zb[k] interleaved) to gather the mirrors
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int k = tt + T * u;
      if (k < m2h) {
        ex[2 * k] = za[buf][u];
        ex[2 * k + 1] = zc[buf][u];
      }
    }
    wave_sync();
    float2 v[R];
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const int k = tt + T * u;
      float2 val = make_float2(0.f, 0.f);
      if (u < NB && k < m2h) {
        float2 a = za[buf][u < NB ? u : 0], c = zc[buf][u < NB ? u : 0];
        if (k == 0 || 2 * k == W) {  // Hermitian fix-up of the irfft input
          a.y = 0.f;
          c.y = 0.f;
        }
        val = make_float2(a.x - c.y, a.y + c.x);           // Za + i Zb
      } else if (k > W / 2 && W - k < m2h) {
        const float2 a = ex[2 * (W - k)], c = ex[2 * (W - k) + 1];
        val = make_float2(a.x + c.y, c.x - a.y);           // conj Za + i conj Zb
      }
      v[u] = val;
    }
    const float ba = bS[2 * gl], bb = bS[2 * gl + 1];
    wave_sync();
    float2 out[Q][T];
    line_fft<W, +1>(v, ex, twW, tt, out);
#pragma unroll
    for (int q = 0; q < Q; ++q)
#pragma unroll
      for (int u = 0; u < T; ++u) {
        const int p = tt + T * q + R * u;
        rowa[p] = fmaf(out[q][u].x, inv_scale, ba);
        rowa[SS + p] = fmaf(out[q][u].y, inv_scale, bb);
      }
  };

  // element e of the lane's NEL: tile (m, n), register r
  auto el_m = [](int e) { return e / (NT_PER * 16); };
  auto el_n = [](int e) { return (e / 16) % NT_PER; };
  // spec address of element e (o = channel, px = pixel) for lane ln
  auto spec_idx = [&](int e, int ln, int buf) __attribute__((always_inline)) {
    const int r = e % 16;
    const int o = 32 * (mt0 + el_m(e)) + 8 * (r >> 2) + 4 * (ln >> 5) + (r & 3);
    const int px = 32 * (pxt0 + el_n(e)) + (ln & 31);
    return (buf * CO + o) * SS + px;
  };
  // final value and store of element e of row h from (acc, spec value)
  auto epi_store = [&](int e, float accv, float specv, uint32_t yo) __attribute__((always_inline)) {
    const int r = e % 16;
    const uint32_t oc = 32 * (mt0 + el_m(e)) + 8 * (r >> 2) + (r & 3);   // o minus the lane part
    float v = accv + specv;
    v = act_select(gelu_erf(v), v, gmask);
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), make_rsrc(ys, ybytes),
                                          (int)(yo + 128u * el_n(e)), (int)(oc * HW * 4u), 0);
  };

  // ---- the skip accumulators of row h (gated / identity / none)
  auto skip_direct = [&](int h, int ln, auto buf_c) __attribute__((always_inline)) {
    constexpr int buf = decltype(buf_c)::value;
#pragma unroll
    for (int m = 0; m < MT_PER; ++m)
#pragma unroll
      for (int n = 0; n < NT_PER; ++n)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float v = 0.f;
          if (gated) {
            const int o = 32 * (mt0 + m) + 8 * (r >> 2) + 4 * (ln >> 5) + (r & 3);
            const int px = 32 * (pxt0 + n) + (ln & 31);
            const float gate = (skip_kind == FNO_SKIP_SOFT_GATING) ? skip_w[o] : 1.f;
            v = gate * xs[(size_t)o * HW + (size_t)h * W + px];
          }
          acc[buf][m][n][r] = v;
        }
  };

  // ---- pipeline step s: MFMA (row s) with EPI of row s-1, then irfft (row s)
  auto step = [&](int s, auto cur_c, auto mf_c, auto ep_c) __attribute__((always_inline)) {
    constexpr int cur = decltype(cur_c)::value, prv = cur ^ 1;
    constexpr bool MF = decltype(mf_c)::value, EP = decltype(ep_c)::value;
    // Thread index laundered through an empty asm: the addresses derived from
    // it are recomputed in the step instead of hoisted into live registers.
    int tv = tid;
    asm volatile("" : "+v"(tv));
    const int ln = tv & 63;
    const int h = h0 + s;
    if constexpr (MF) {
      if (s + 1 < TR) load_row(h + 1, tv, std::integral_constant<int, prv>());
      if (!linear) skip_direct(h, ln, cur_c);
    }
    const uint32_t yo = ((uint32_t)(4 * (ln >> 5)) * HW + (uint32_t)(h - 1) * W +
                         32 * pxt0 + (ln & 31)) * 4u;
    if (MF && linear) {
#pragma unroll
      for (int m = 0; m < MT_PER; ++m)
#pragma unroll
        for (int n = 0; n < NT_PER; ++n)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[cur][m][n][r] = 0.f;
      const float* arow = wsT + (ln >> 5) * CO + 32 * mt0 + (ln & 31);
      // LDS operands one k-step ahead: A (weights) and the spec values of
      // the elements stored in the next step
      float a_c[MT_PER], a_n[MT_PER], sp_c[EPK], sp_n[EPK];
#pragma unroll
      for (int m = 0; m < MT_PER; ++m) a_c[m] = arow[32 * m];
      if constexpr (EP) {
#pragma unroll
        for (int i = 0; i < EPK; ++i) sp_c[i] = spec[spec_idx(i, ln, prv)];
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if (ks + 1 < KS) {
#pragma unroll
          for (int m = 0; m < MT_PER; ++m) a_n[m] = arow[2 * (ks + 1) * CO + 32 * m];
          if constexpr (EP) {
#pragma unroll
            for (int i = 0; i < EPK; ++i) sp_n[i] = spec[spec_idx((ks + 1) * EPK + i, ln, prv)];
          }
        }
#pragma unroll
        for (int m = 0; m < MT_PER; ++m)
#pragma unroll
          for (int n = 0; n < NT_PER; ++n)
            acc[cur][m][n] =
                __builtin_amdgcn_mfma_f32_32x32x2f32(a_c[m], xr[cur][n][ks], acc[cur][m][n], 0, 0, 0);
        if constexpr (EP) {
#pragma unroll
          for (int i = 0; i < EPK; ++i) {
            const int e = ks * EPK + i;
            epi_store(e, acc[prv][el_m(e)][el_n(e)][e % 16], sp_c[i], yo);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int m = 0; m < MT_PER; ++m) a_c[m] = a_n[m];
#pragma unroll
        for (int i = 0; i < EPK; ++i) sp_c[i] = sp_n[i];
      }
    } else if constexpr (EP) {
#pragma unroll
      for (int e = 0; e < NEL; ++e)
        epi_store(e, acc[prv][el_m(e)][el_n(e)][e % 16], spec[spec_idx(e, ln, prv)], yo);
    }
    if constexpr (MF) irfft_row(tv, cur_c);
    __syncthreads();
  };

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using BT = std::integral_constant<bool, true>;
  using BF = std::integral_constant<bool, false>;
  load_row(h0, tid, I0());
  __syncthreads();
  step(0, I0(), BT(), BF());
#pragma unroll 1
  for (int s = 1; s < TR; s += 2) {
    step(s, I1(), BT(), BT());
    if (s + 1 < TR) step(s + 1, I0(), BT(), BT());
  }
  step(TR, I0(), BF(), BT());   // TR even: row TR-1 sits in buffer 1
}

// ----------------------------------------------------------------------- K4R
// Register-resident row epilogue for W = 256 (16-lane line FFTs).
// MFMA 16x16x4 f32 operand/result layout (wave64):
//   A (16 x 4):  lane l supplies A[l % 16][l / 16]
//   B (4 x 16):  lane l supplies B[l / 16][l % 16]
//   D (16 x 16): lane l, register r holds D[4*(l/16) + r][l % 16]
// M = the wave's 16 output channels, N = 16 pixels of a tile, K = 4 input
// channels.  Group G = l/16 of wave w runs the inverse row FFTs of channels
// 16w+4G .. 16w+4G+3 (two lines, two channels packed per line); lane
// t = l % 16 ends holding pixels t + 16u (u < 16), which is D of tile u.  So
// the accumulators start as spec * scale + bias straight from the FFT
// registers, the skip MFMAs add W_s x on top, and GELU + store read them
// back: the spectral term never goes through LDS.  The x operand streams
// through a double-buffered LDS ring of 16-channel chunks (loaded a row ahead
// into registers), so a workgroup needs ~36 KB of LDS and two share a CU.
typedef float v4f __attribute__((ext_vector_type(4)));

template <int W, int CO, int CI, int NB>
__global__ void __launch_bounds__(CO * 4) __attribute__((amdgpu_waves_per_eu(2, 2)))
k_row_epilogue_r(const float* __restrict__ x, const float2* __restrict__ z,
                 const float* __restrict__ skip_w, const float* __restrict__ bias,
                 float* __restrict__ y, int H, int TR, int m2h, int skip_kind, int act,
                 float inv_scale) {
  // A step covers PW = 256 pixels of every channel: one row at W = 256, two
  // adjacent rows at W = 128 (the two 8-lane halves of each 16-lane group run
  // one row each).  Lane t of a group holds pixel p(u, t) = (t / T) W + t % T
  // + T u of tile u, which is column t of MFMA tile u.
  using PL = LinePlan<W>;
  constexpr int T = PL::T, R = PL::R, Q = PL::Q;
  constexpr int PW = 256, ROWS = PW / W;
  static_assert(R == 16 && T * ROWS == 16, "16 tiles of 16 pixels per step");
  constexpr int NWAVE = CO / 16, BLOCK = 64 * NWAVE;
  constexpr int KC = 16;                 // input channels per LDS chunk
  constexpr int NCH = CI / KC;           // chunks per step
  constexpr int XS = PW + 16;            // LDS row stride of a chunk (floats)
  constexpr int KS = CI / 4;             // MFMA k-steps per step
  constexpr int LPT = KC * PW / 4 / BLOCK; // float4 loads per thread per chunk
  constexpr int EXS = PW + 8;            // exchange slice per 16-lane group (float2)
  constexpr int HS = EXS / ROWS;         // ... per line (one per half at W = 128)
  static_assert(CO % 16 == 0 && CI % KC == 0 && LPT >= 1 && KC * PW / 4 % BLOCK == 0, "shape");
  extern __shared__ float4 smem4[];
  float2* twW = reinterpret_cast<float2*>(smem4);
  float* region = reinterpret_cast<float*>(twW + W);   // exchange slices / x ring

  const int RB = H / TR;
  const int b = blockIdx.x / RB, h0 = (blockIdx.x % RB) * TR;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = lane >> 4, t = lane & 15;
  const int half = t / T, tl = t % T;  // row of the step, lane within the line
  const uint32_t HW = (uint32_t)H * W;
  const bool linear = (skip_kind == FNO_SKIP_LINEAR);
  const bool gated = (skip_kind == FNO_SKIP_SOFT_GATING || skip_kind == FNO_SKIP_IDENTITY);
  const bool gelu_on = (act == FNO_ACT_GELU);
  const uint32_t gmask = act_mask(gelu_on);
  const int o0 = 16 * wave + 4 * G;    // first of the lane's 4 output channels
  const float* xs = x + (size_t)b * CI * HW;
  const float2* zs = z + (size_t)b * H * CO * m2h;
  float* ys = y + (size_t)b * CO * HW;
  const uint32_t xbytes = CI * HW * 4u, ybytes = CO * HW * 4u;
  const uint32_t zbytes = (uint32_t)H * CO * m2h * 8u;

  fill_twiddles<W>(twW);
  float aW[KS];
  if (linear) {
#pragma unroll
    for (int k = 0; k < KS; ++k) aW[k] = skip_w[(16 * wave + (lane & 15)) * CI + 4 * k + (lane >> 4)];
  }
  float bch[4], gch[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    bch[r] = bias ? bias[o0 + r] : 0.f;
    gch[r] = (skip_kind == FNO_SKIP_SOFT_GATING) ? skip_w[o0 + r] : 1.f;
  }

  float4 xst[2][LPT];
  float2 za[2][NB], zc[2][NB];   // bins k = t + 16n of the two lines' channel pairs
  v4f acc[R];

  // x chunk c of row h into staging buffer sb: float4 q = tid + BLOCK*j is
  // channel (q / 64) of the chunk, pixels 4*(q % 64) .. +3
  auto load_chunk = [&](int h, int c, float4 (&dst)[LPT]) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(xs, xbytes);
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      const int q = tid + BLOCK * j;
      const uint32_t off = ((uint32_t)(c * KC + (q >> 6)) * HW + (uint32_t)h * W + 4 * (q & 63)) * 4u;
      dst[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)off, 0, 0));
    }
  };
  auto store_chunk = [&](int buf, const float4 (&src)[LPT]) __attribute__((always_inline)) {
    float* ring = region + buf * KC * XS;
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      const int q = tid + BLOCK * j;
      *reinterpret_cast<float4*>(ring + (q >> 6) * XS + 4 * (q & 63)) = src[j];
    }
  };
  // Z[b][o][h][kw]: bins of channel o0 + 2L (za) and the next channel (zc,
  // one H x m2h plane further) in the lane's row; bins past m2h read past the
  // buffer end: zero
  const int zplane = __builtin_amdgcn_readfirstlane(H * m2h * 8);
  auto load_z = [&](int h) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rz = make_rsrc(zs, zbytes);
#pragma unroll
    for (int L = 0; L < 2; ++L) {
      const uint32_t zo = (((uint32_t)(o0 + 2 * L) * H + h + half) * m2h + tl) * 8u;
#pragma unroll
      for (int n = 0; n < NB; ++n) {
        const uint32_t off = (tl + T * n < m2h) ? zo + 8u * T * n : 0x80000000u;
        za[L][n] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rz, (int)off, 0, 0));
        zc[L][n] = __builtin_bit_cast(float2,
                                      __builtin_amdgcn_raw_buffer_load_b64(rz, (int)off, zplane, 0));
      }
    }
  };

  // Row order: workgroups that share an XCD (ids 8 apart) start at different
  // rows of their block, so concurrent x reads spread over the HBM channels.
  const int NS = TR / ROWS;              // steps per workgroup
  const int rot = (int)(blockIdx.x >> 3) % NS;
  auto row_at = [&](int s) __attribute__((always_inline)) { return h0 + ROWS * ((s + rot) % NS); };

  // first row's operands
  if (linear) {
    load_chunk(row_at(0), 0, xst[0]);
    if (NCH > 1) load_chunk(row_at(0), 1, xst[1]);
  }
  load_z(row_at(0));
  __syncthreads();

#pragma unroll 1
  for (int s = 0; s < NS; ++s) {
    const int h = row_at(s);
    // ---- inverse row FFTs: line L packs channels o0+2L (re) and o0+2L+1 (im)
    {
      float2* ex = reinterpret_cast<float2*>(region) + (4 * wave + G) * EXS + half * HS;
#pragma unroll
      for (int L = 0; L < 2; ++L) {
#pragma unroll
        for (int u = 0; u < NB; ++u) {
          const int k = tl + T * u;
          if (k < m2h) {
            ex[2 * k] = za[L][u];
            ex[2 * k + 1] = zc[L][u];
          }
        }
        wave_sync();
        float2 v[R];
#pragma unroll
        for (int u = 0; u < R; ++u) {
          const int k = tl + T * u;
          float2 val = make_float2(0.f, 0.f);
          if (u < NB && k < m2h) {
            float2 a = za[L][u < NB ? u : 0], c = zc[L][u < NB ? u : 0];
            if (k == 0 || 2 * k == W) {  // Hermitian fix-up of the irfft input
              a.y = 0.f;
              c.y = 0.f;
            }
            val = make_float2(a.x - c.y, a.y + c.x);           // Za + i Zb
          } else if (u >= R - NB && k > W / 2 && W - k < m2h) {
            // mirrors of bins < m2h <= 16 NB sit at u >= R - NB: the lanes'
            // other inputs are compile-time zeros, which prunes the first pass
            const float2 a = ex[2 * (W - k)], c = ex[2 * (W - k) + 1];
            val = make_float2(a.x + c.y, c.x - a.y);           // conj Za + i conj Zb
          }
          v[u] = val;
        }
        wave_sync();
        float2 out[Q][T];
        line_fft<W, +1>(v, ex, twW, tl, out);
        // out[q][s] is pixel tl + T (q + Q s) of the line: tile u = q + Q s
#pragma unroll
        for (int u = 0; u < R; ++u) {
          acc[u][2 * L] = fmaf(out[u % Q][u / Q].x, inv_scale, bch[2 * L]);
          acc[u][2 * L + 1] = fmaf(out[u % Q][u / Q].y, inv_scale, bch[2 * L + 1]);
        }
      }
    }
    if (gated) {
#pragma unroll
      for (int u = 0; u < R; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          acc[u][r] += gch[r] * xs[(size_t)(o0 + r) * HW + (size_t)(h + half) * W + T * u + tl];
    }
    __syncthreads();   // exchange slices free: the region becomes the x ring
    if (linear) {
      store_chunk(0, xst[0]);
      if (NCH > 2) load_chunk(h, 2, xst[0]);
      __syncthreads();
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const float* ring = region + (c & 1) * KC * XS + (lane >> 4) * XS + half * W + tl;
        // B operands in groups of 4 tiles: group g + 1 is read while the 4
        // MFMAs of group g run, so the LDS latency hides under them
        constexpr int GT = 4, NG = KC / 4 * R / GT;
        float bq[2][GT];
#pragma unroll
        for (int u = 0; u < GT; ++u) bq[0][u] = ring[T * u];
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          if (g + 1 < NG) {
            const int kn = (g + 1) * GT / R, un = (g + 1) * GT % R;
#pragma unroll
            for (int u = 0; u < GT; ++u) bq[(g + 1) & 1][u] = ring[4 * kn * XS + T * (un + u)];
          }
          __builtin_amdgcn_sched_barrier(0);
          const int kk = g * GT / R, u0 = g * GT % R;
#pragma unroll
          for (int u = 0; u < GT; ++u)
            acc[u0 + u] = __builtin_amdgcn_mfma_f32_16x16x4f32(aW[c * (KC / 4) + kk], bq[g & 1][u],
                                                               acc[u0 + u], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
        if (c + 1 < NCH) {
          store_chunk((c + 1) & 1, xst[(c + 1) & 1]);
          if (c + 3 < NCH) load_chunk(h, c + 3, xst[(c + 1) & 1]);
        }
        __syncthreads();
      }
    }
    // ---- next row's operands in flight during GELU + store and its FFTs
    if (s + 1 < NS) {
      if (linear) {
        load_chunk(row_at(s + 1), 0, xst[0]);
        if (NCH > 1) load_chunk(row_at(s + 1), 1, xst[1]);
      }
      load_z(row_at(s + 1));
    }
    // ---- activation and store: channel o0 + r, pixel p(u, t)
    {
      const __amdgpu_buffer_rsrc_t ry = make_rsrc(ys, ybytes);
      const uint32_t yo = ((uint32_t)o0 * HW + (uint32_t)(h + half) * W + tl) * 4u;
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int u = 0; u < R; ++u) {
          float v = acc[u][r];
          v = act_select(gelu_erf(v), v, gmask);
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), ry,
                                                (int)(yo + 4u * T * u),
                                                __builtin_amdgcn_readfirstlane((int)(r * HW * 4u)), 0);
        }
    }
  }
}

// ============================================================== host side
bool rowsynth_covers(int H, int W, int Ci, int Co, int m1, int m2h);
int rowsynth_epilogue(const float* x, const float2* yhat, const float* skip_w, const float* bias,
                      float* y, int B, int Ci, int H, int W, int m1, int m2h, int skip_kind,
                      int act, float s, hipStream_t st);
bool rowsynth_mlp_covers(int H, int W, int Ci, int Co, int m1, int m2h, int hidden,
                         int skip_kind);
int rowsynth_mlp_epilogue(const void* x, const float2* yhat, const float* skip_w,
                          const float* bias, void* y, int B, int H, int W, int m1, int m2h,
                          int skip_kind, int act, float s, const LayerMlp& mlp, bool bf,
                          hipStream_t st);
int contract_dense(const float2* X, const float2* W, float2* Y, int B, int Ci, int Co, int64_t M,
                   int64_t sWi, int64_t sWo, int64_t sWk, hipStream_t st, int ymap_w);
int rfft_window(const float* x, float2* xhat, int64_t planes, int32_t ndim, const int32_t* sizes,
                const int32_t* modes, int32_t norm, void* ws, size_t ws_bytes, hipStream_t st);
size_t rfft_window_ws(int64_t planes, int32_t ndim, const int32_t* sizes, const int32_t* modes);

static constexpr size_t kMaxLds = 160 * 1024;

static int line_lanes(int n) { return n >= 256 ? 16 : 8; }

static size_t fwd_lds_bytes(int H, int W, int m2h) {
  (void)m2h;   // the chunk spectrum lives inside the line slices
  return (size_t)(W + H + 16 * (W + 16)) * sizeof(float2);
}

static int fwd_kpr(int m1) { return m1 <= 32 ? 1 : (m1 <= 64 ? 2 : 4); }

// K1 covers the plane when the kept columns fit one pass of the column stage
// (4 lanes per column) and the kept rows fit the register accumulators.
static bool fwd_supported(int H, int W, int m1, int m2h) {
  if (!(H == 64 || H == 128 || H == 256)) return false;
  if (!(W == 128 || W == 256)) return false;
  if (m1 < 1 || m1 > 128 || m1 > H) return false;
  if (m2h < 1 || m2h > 16 * line_lanes(W) / 4) return false;
  return fwd_lds_bytes(H, W, m2h) <= kMaxLds;
}

// one group of line_lanes(H) lanes per kept column, whole waves, <= 512
// threads: with the ~70 KB tile two workgroups then share a CU, which pays for
// an extra pass when more than 512 / T columns are kept
static int inv_block(int H, int m2h) {
  const int t = line_lanes(H);
  const int g = m2h < 512 / t ? m2h : 512 / t;
  return (g * t + 63) / 64 * 64;
}

static size_t inv_lds_bytes(int H, int m2h) {
  const int TS = m2h | 1;
  return (size_t)(H + H * TS) * sizeof(float2);
}

static size_t epi_lds_bytes(int W, int Co, int Ci, int skip_kind) {
  size_t f = 2 * (size_t)W + (skip_kind == FNO_SKIP_LINEAR ? (size_t)Ci * Co : 0) + (size_t)Co +
             (Co & 1);
  f += 2 * (size_t)Co * (W + 8);
  return f * sizeof(float);
}

// bin slots per lane of the row irfft: ceil(m2h / lanes per line)
static int epi_bins(int W, int m2h) {
  const int T = line_lanes(W);
  const int nb = (m2h + T - 1) / T;
  return nb <= 2 ? 2 : (nb <= 3 ? 3 : (nb <= 5 ? 5 : 9));
}

static int epi_rows_per_block(int H) { return H >= 64 ? 16 : H; }

static bool epi_r_supported(int H, int W, int Ci, int Co, int m2h, int skip_kind);

// K3 has instances for H in {64, 128, 256} only: every epilogue variant needs
// it, so the fused path covers no other column count.
static bool inv_supported(int H, int m1, int m2h) {
  if (!(H == 64 || H == 128 || H == 256)) return false;
  if (m1 < 1 || m1 > H || m2h < 1) return false;
  return inv_lds_bytes(H, m2h) <= kMaxLds;
}

static bool epi_supported(int H, int W, int Ci, int Co, int m1, int m2h, int skip_kind) {
  if (!inv_supported(H, m1, m2h)) return false;
  if (epi_r_supported(H, W, Ci, Co, m2h, skip_kind)) return true;
  if (!(W == 128 || W == 256)) return false;
  if (!(Co == 32 || Co == 64)) return false;
  if (skip_kind == FNO_SKIP_LINEAR && !(Ci == 32 || Ci == 64)) return false;
  if ((skip_kind == FNO_SKIP_IDENTITY || skip_kind == FNO_SKIP_SOFT_GATING) && Ci != Co)
    return false;
  if (m2h > W / 2 + 1) return false;
  if (2 * m2h > W + 8) return false;  // mirror staging fits the line's LDS rows
  return epi_lds_bytes(W, Co, Ci, skip_kind) <= kMaxLds;
}

// The fused path is taken when the epilogue kernel covers the shape; the
// forward window transform is K1 when it covers the plane and the generic
// direct-DFT kernels otherwise.
bool fast2d_supported(int B, int Ci, int Co, int ndim, const int32_t* sizes, const int32_t* modes,
                      int skip_kind) {
  if (ndim != 2 || B < 1) return false;
  const int H = sizes[0], W = sizes[1];
  if (rowsynth_covers(H, W, Ci, Co, modes[0], modes[1])) return true;
  return epi_supported(H, W, Ci, Co, modes[0], modes[1], skip_kind);
}

// bfloat16 activation storage (the one-pass layer only) needs the streamed
// forward, which reads x as stored.
bool fast2d_bf16_supported(const int32_t* sizes, const int32_t* modes) {
  return fwd_supported(sizes[0], sizes[1], modes[0], modes[1]);
}

// The inverse column transform Z [B][Co][H][m2h] lives in the workspace only
// when the epilogue reads it; the row-synthesis epilogue builds it on chip.
static bool uses_z(int Ci, int Co, const int32_t* sizes, const int32_t* modes) {
  return !rowsynth_covers(sizes[0], sizes[1], Ci, Co, modes[0], modes[1]);
}

size_t fast2d_workspace(int B, int Ci, int Co, const int32_t* sizes, const int32_t* modes) {
  const int64_t M = (int64_t)modes[0] * modes[1];
  const int64_t zel = uses_z(Ci, Co, sizes, modes) ? (int64_t)B * sizes[0] * Co * modes[1] : 0;
  size_t e = (size_t)((int64_t)B * Ci * M + (int64_t)B * Co * M + zel) * sizeof(float2);
  if (!fwd_supported(sizes[0], sizes[1], modes[0], modes[1]))
    e += rfft_window_ws((int64_t)B * Ci, 2, sizes, modes);
  return e;
}

// Kernels taking more than 64 KB of dynamic LDS get the limit raised.
template <typename K>
static int allow_lds(K kernel, size_t bytes) {
  if (bytes <= 64 * 1024) return FNO_OK;
  return hip_status(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes),
                    "hipFuncSetAttribute(MaxDynamicSharedMemorySize)");
}

template <int H, int W, int KPR, bool BF>
static int launch_fwd(const void* x, float2* xhat, int64_t planes, int m1, int m2h, float scale,
                      hipStream_t st) {
  constexpr int BLOCK = 16 * (W >= 256 ? 16 : 8);
  const size_t lds = fwd_lds_bytes(H, W, m2h);
  int rc = allow_lds(k_fwd_stream<H, W, KPR, BF>, lds);
  if (rc) return rc;
  hipLaunchKernelGGL((k_fwd_stream<H, W, KPR, BF>), dim3((unsigned)planes), dim3(BLOCK), lds, st,
                     x, xhat, m1, m2h, scale);
  return launch_status("k_fwd_stream");
}

template <int H, int W, bool BF>
static int launch_fwd_k(const void* x, float2* xhat, int64_t planes, int m1, int m2h, float scale,
                        hipStream_t st) {
  switch (fwd_kpr(m1)) {
    case 1: return launch_fwd<H, W, 1, BF>(x, xhat, planes, m1, m2h, scale, st);
    case 2: return launch_fwd<H, W, 2, BF>(x, xhat, planes, m1, m2h, scale, st);
    default: return launch_fwd<H, W, 4, BF>(x, xhat, planes, m1, m2h, scale, st);
  }
}

// bf: x bfloat16 (else float32)
static int dispatch_fwd(int H, int W, const void* x, float2* xhat, int64_t planes, int m1, int m2h,
                        float scale, hipStream_t st, bool bf = false) {
#define FNO_FWD(h, w)                                                                     \
  if (H == h && W == w)                                                                   \
    return bf ? launch_fwd_k<h, w, true>(x, xhat, planes, m1, m2h, scale, st)             \
              : launch_fwd_k<h, w, false>(x, xhat, planes, m1, m2h, scale, st);
  FNO_FWD(64, 128) FNO_FWD(128, 128) FNO_FWD(256, 128)
  FNO_FWD(64, 256) FNO_FWD(128, 256) FNO_FWD(256, 256)
#undef FNO_FWD
  set_error("fused 2D forward: unsupported plane %dx%d", H, W);
  return FNO_ERR_UNSUPPORTED;
}

template <int H>
static int launch_inv(const float2* yhat, float2* zbuf, int B, int Co, int m1, int m2h,
                      hipStream_t st) {
  const int block = inv_block(H, m2h);
  const size_t lds = inv_lds_bytes(H, m2h);
  int rc = allow_lds(k_inv_cols<H>, lds);
  if (rc) return rc;
  hipLaunchKernelGGL((k_inv_cols<H>), dim3((unsigned)(B * Co)), dim3(block), lds, st, yhat,
                     zbuf, Co, m1, m2h);
  return launch_status("k_inv_cols");
}

static int dispatch_inv(int H, const float2* yhat, float2* zbuf, int B, int Co, int m1, int m2h,
                        hipStream_t st) {
  if (H == 64) return launch_inv<64>(yhat, zbuf, B, Co, m1, m2h, st);
  if (H == 128) return launch_inv<128>(yhat, zbuf, B, Co, m1, m2h, st);
  if (H == 256) return launch_inv<256>(yhat, zbuf, B, Co, m1, m2h, st);
  set_error("fused 2D inverse: unsupported H=%d", H);
  return FNO_ERR_UNSUPPORTED;
}

template <int H, int W, int CO, int CI, int NB>
static int launch_epi(const float* x, const float2* z, const float* skip_w, const float* bias,
                      float* y, int B, int m2h, int skip_kind, int act, float inv_scale,
                      hipStream_t st) {
  constexpr int BLOCK = CO / 2 * (W >= 256 ? 16 : 8);
  const size_t lds = epi_lds_bytes(W, CO, CI, skip_kind);
  int rc = allow_lds(k_row_epilogue<H, W, CO, CI, NB>, lds);
  if (rc) return rc;
  const int TR = epi_rows_per_block(H);
  const int64_t grid = (int64_t)B * (H / TR);
  hipLaunchKernelGGL((k_row_epilogue<H, W, CO, CI, NB>), dim3((unsigned)grid), dim3(BLOCK), lds,
                     st, x, z, skip_w, bias, y, TR, m2h, skip_kind, act, inv_scale);
  return launch_status("k_row_epilogue");
}

template <int W, int CO, int CI>
static int launch_epi_h(const float* x, const float2* z, const float* skip_w, const float* bias,
                        float* y, int B, int H, int m2h, int skip_kind, int act, float inv_scale,
                        hipStream_t st) {
  const bool few = epi_bins(W, m2h) <= 3;
#define FNO_EPI_H(h)                                                                          \
  if (H == h)                                                                                 \
    return few ? launch_epi<h, W, CO, CI, 3>(x, z, skip_w, bias, y, B, m2h, skip_kind, act,   \
                                             inv_scale, st)                                   \
               : launch_epi<h, W, CO, CI, 9>(x, z, skip_w, bias, y, B, m2h, skip_kind, act,   \
                                             inv_scale, st);
  FNO_EPI_H(64) FNO_EPI_H(128) FNO_EPI_H(256)
#undef FNO_EPI_H
  set_error("fused 2D epilogue: unsupported H=%d", H);
  return FNO_ERR_UNSUPPORTED;
}

// ---- register-resident epilogue (W = 256)
static size_t epi_r_lds_bytes(int Co) {
  const size_t ex = (size_t)4 * (Co / 16) * (256 + 8) * 2;   // exchange slices (floats)
  const size_t ring = (size_t)2 * 16 * (256 + 16);            // x ring (floats)
  return (2 * 256 + (ex > ring ? ex : ring)) * sizeof(float);
}

static bool epi_r_supported(int H, int W, int Ci, int Co, int m2h, int skip_kind) {
  if (!(W == 128 || W == 256) || H % 16 != 0) return false;
  if (!(Co == 64 || Co == 128)) return false;
  const int ci = (skip_kind == FNO_SKIP_LINEAR) ? Ci : Co;
  if (!(ci == 32 || ci == 64 || ci == 128)) return false;
  if ((skip_kind == FNO_SKIP_IDENTITY || skip_kind == FNO_SKIP_SOFT_GATING) && Ci != Co)
    return false;
  // 8 bins per lane at most (NB = 8, T = W / 16 lanes per line); the mirror
  // staging (2 m2h entries) fits the line's 264 / (256 / W) entry slice
  if (m2h < 1 || m2h > W / 2) return false;
  return epi_r_lds_bytes(Co) <= kMaxLds;
}

template <int W, int CO, int CI, int NB>
static int launch_epi_r(const float* x, const float2* z, const float* skip_w, const float* bias,
                        float* y, int B, int H, int m2h, int skip_kind, int act, float inv_scale,
                        hipStream_t st) {
  const size_t lds = epi_r_lds_bytes(CO);
  int rc = allow_lds(k_row_epilogue_r<W, CO, CI, NB>, lds);
  if (rc) return rc;
  // 16 rows per workgroup, or 8 when that leaves fewer than two workgroups
  // per CU (two share a CU by LDS and registers)
  const int TR = ((int64_t)B * (H / 16) >= 512) ? 16 : 8;
  const int64_t grid = (int64_t)B * (H / TR);
  hipLaunchKernelGGL((k_row_epilogue_r<W, CO, CI, NB>), dim3((unsigned)grid), dim3(CO * 4), lds,
                     st, x, z, skip_w, bias, y, H, TR, m2h, skip_kind, act, inv_scale);
  return launch_status("k_row_epilogue_r");
}

template <int W>
static int dispatch_epi_r_w(int Co, int Ci, const float* x, const float2* z, const float* skip_w,
                            const float* bias, float* y, int B, int H, int m2h, int skip_kind,
                            int act, float inv_scale, hipStream_t st) {
  const int ci = (skip_kind == FNO_SKIP_LINEAR) ? Ci : Co;
  const bool few = m2h <= 3 * (W / 16);   // 3 bins per lane
#define FNO_EPI_R(co, cin)                                                                      \
  if (Co == co && ci == cin)                                                                    \
    return few ? launch_epi_r<W, co, cin, 3>(x, z, skip_w, bias, y, B, H, m2h, skip_kind, act,  \
                                             inv_scale, st)                                     \
               : launch_epi_r<W, co, cin, 8>(x, z, skip_w, bias, y, B, H, m2h, skip_kind, act,  \
                                             inv_scale, st);
  FNO_EPI_R(64, 32) FNO_EPI_R(64, 64) FNO_EPI_R(64, 128)
  FNO_EPI_R(128, 32) FNO_EPI_R(128, 64) FNO_EPI_R(128, 128)
#undef FNO_EPI_R
  set_error("fused 2D epilogue: unsupported Co=%d Ci=%d", Co, Ci);
  return FNO_ERR_UNSUPPORTED;
}

static int dispatch_epi_r(int W, int Co, int Ci, const float* x, const float2* z,
                          const float* skip_w, const float* bias, float* y, int B, int H, int m2h,
                          int skip_kind, int act, float inv_scale, hipStream_t st) {
  if (W == 128)
    return dispatch_epi_r_w<128>(Co, Ci, x, z, skip_w, bias, y, B, H, m2h, skip_kind, act,
                                 inv_scale, st);
  return dispatch_epi_r_w<256>(Co, Ci, x, z, skip_w, bias, y, B, H, m2h, skip_kind, act,
                               inv_scale, st);
}

static int dispatch_epi(int W, int Co, int Ci, const float* x, const float2* z,
                        const float* skip_w, const float* bias, float* y, int B, int H, int m2h,
                        int skip_kind, int act, float inv_scale, hipStream_t st) {
  // the x operand width only matters for the linear skip
  const int ci = (skip_kind == FNO_SKIP_LINEAR) ? Ci : Co;
#define FNO_EPI(w, co, cin)                                                                     \
  if (W == w && Co == co && ci == cin)                                                          \
    return launch_epi_h<w, co, cin>(x, z, skip_w, bias, y, B, H, m2h, skip_kind, act, inv_scale, \
                                    st);
  FNO_EPI(128, 32, 32) FNO_EPI(128, 32, 64) FNO_EPI(128, 64, 32) FNO_EPI(128, 64, 64)
  FNO_EPI(256, 32, 32) FNO_EPI(256, 32, 64) FNO_EPI(256, 64, 32) FNO_EPI(256, 64, 64)
#undef FNO_EPI
  set_error("fused 2D epilogue: unsupported W=%d Co=%d Ci=%d", W, Co, Ci);
  return FNO_ERR_UNSUPPORTED;
}

// bf (with a channel MLP only): x and y are bfloat16.
int fast2d_block(const void* x, const float2* w, const float* bias, const float* skip_w, void* y,
                 int B, int Ci, int Co, const int32_t* sizes, const int32_t* modes, int norm,
                 int skip_kind, int act, void* ws, size_t ws_bytes, hipStream_t st,
                 const LayerMlp* mlp, bool bf) {
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
  int rc;
  if (bf && (!mlp || !fwd_supported(H, W, m1, m2h))) {
    set_error("fused 2D block: bfloat16 activations need the one-pass layer's shapes");
    return FNO_ERR_UNSUPPORTED;
  }
  if (fwd_supported(H, W, m1, m2h)) {
    rc = dispatch_fwd(H, W, x, xhat, (int64_t)B * Ci, m1, m2h, fscale, st, bf);
  } else {
    // the generic forward's scratch goes where Z lives later
    void* rest = zbuf;
    rc = rfft_window(static_cast<const float*>(x), xhat, (int64_t)B * Ci, 2, sizes, modes, norm, rest,
                     ws_bytes - (size_t)((int64_t)B * (Ci + Co) * M) * sizeof(float2), st);
  }
  if (rc) return rc;
  // The row synthesis reads each window row's AC bins as one run, so for it
  // the contraction writes every (b, o) plane as the rows' AC bins (m2h - 1
  // entries each, 128-byte aligned at 17 and 33 bins) followed by the DC
  // column, instead of in the weight's mode order.
  const bool rsyn = mlp || !uses_z(Ci, Co, sizes, modes);
  rc = contract_dense(xhat, w, yhat, B, Ci, Co, M, (int64_t)Co * M, M, 1, st, rsyn ? m2h : 0);
  if (rc) return rc;
  if (mlp)
    return rowsynth_mlp_epilogue(x, yhat, skip_w, bias, y, B, H, W, m1, m2h, skip_kind, act,
                                 iscale, *mlp, bf, st);
  const float* xf = static_cast<const float*>(x);
  float* yf = static_cast<float*>(y);
  if (rsyn)
    return rowsynth_epilogue(xf, yhat, skip_w, bias, yf, B, Ci, H, W, m1, m2h, skip_kind, act,
                             iscale, st);
  rc = dispatch_inv(H, yhat, zbuf, B, Co, m1, m2h, st);
  if (rc) return rc;
  if (epi_r_supported(H, W, Ci, Co, m2h, skip_kind))
    return dispatch_epi_r(W, Co, Ci, xf, zbuf, skip_w, bias, yf, B, H, m2h, skip_kind, act, iscale,
                          st);
  return dispatch_epi(W, Co, Ci, xf, zbuf, skip_w, bias, yf, B, H, m2h, skip_kind, act, iscale, st);
}

}  // namespace fno
