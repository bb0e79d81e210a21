// Row epilogue of the fused 2D block: the inverse column transform, the
// inverse real FFT along the rows, bias, skip and activation, as one matrix
// product per row on the matrix cores:
//
//   y[o, p] = act( sum_i Ws[o, i] x[i, p]  +  sum_j Zt[o, j] T[j, p]  +  c[o] )
//
// Zt holds the row's inverse-column-transformed bins kw = 1 .. m2h-1 (Re, Im
// interleaved), synthesised here from the window spectrum (below); T is the
// real synthesis table of the inverse real FFT along the row with the
// Hermitian weights (2 below the Nyquist bin, 1 at it) and the inverse norm
// scale s folded in:
//   T[2(kw-1)][p] = c_kw s cos(2 pi kw p / W),  T[2(kw-1)+1][p] = -c_kw s sin(..)
// so Re(Z e^{i theta}) needs no Hermitian fix-up (the imaginary parts of the
// DC and Nyquist bins meet sin = 0).  The DC bin is constant along the row:
// c[o] = bias[o] + s Re Z[o, h, 0] seeds the accumulators.  The skip is the
// matrix Ws: the 1x1 conv (linear), diag(g) (soft-gating) or the identity.
//
// Arithmetic: the products run on v_mfma_f32_16x16x32_bf16 as three-term
// bf16 splits, a = a_hi + a_lo with a_hi = bf16(a), a_lo = bf16(a - a_hi)
// (round to nearest even each), a b ~ a_hi b_lo + a_lo b_hi + a_hi b_hi with
// fp32 accumulation.  a_hi + a_lo carries 16 significant bits of a, so each
// product is within 3 * 2^-16 of |a b| (the dropped a_lo b_lo and the two
// representation errors); the terms' rounding errors are independent, and a
// row sum lands within ~1e-5 of its magnitude of the fp32 result.
//
// Work split: 8 waves (two per SIMD, so one wave's matrix work overlaps the
// other's vector work), each owning 32 pixels of a step of 256 (one row of
// W = 256, two rows of W = 128) and all 64 output channels: 4 x 2 tiles of
// 16 channels x 16 pixels.  Lane l = 16 G + n of wave w holds pixels
// p = 32 w' + 2 n + u (u = tile column 0/1, w' = w mod the waves per row) of
// its row, so the x operand of both tiles comes from one 8-byte load per
// input channel and the output goes out as one 8-byte store per channel.  T
// operand fragments stay in registers for the whole kernel, Ws fragments in
// LDS; the Zt fragments of a row are staged in LDS (bf16 hi / lo, in lane
// order) and read by all waves.
//
// Semantics: SpectralConv.forward's inverse (neuralop/layers/
// spectral_convolution.py:547-568: ifftn over the non-last axes, imaginary
// parts of the DC / Nyquist columns dropped, irfft, bias) and the block
// epilogue of FNOBlocks.forward_with_postactivation (neuralop/layers/
// fno_block.py:331-361: skip add, erf GELU).
#include "fno_fft_lds.h"
#include "fno_twiddle.h"

namespace fno {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

namespace rg {
constexpr int kWaves = 8, kThreads = 64 * kWaves;
// cache policy of the x loads and y stores: non-temporal (streaming).  Each
// x and y byte is touched once here, and streaming them keeps the caches for
// the spectrum every block re-reads; measured 482 -> 465 us per block call at
// B32 C64 256^2 (calls back to back: less of y left to write back in the
// next call).
constexpr int kNT = 2;
constexpr int kCo = 64;                 // output channels (4 tiles of 16)
constexpr int kStepPx = 256;            // pixels per step
}  // namespace rg

struct bf16x2 {
  __bf16 hi, lo;
};
__device__ __forceinline__ bf16x2 split_bf16(float v) {
  const __bf16 hi = (__bf16)v;
  return {hi, (__bf16)(v - (float)hi)};
}

// Synthesis table entry T[j][col] (see the top of the file).
__device__ __forceinline__ float synth_entry(int j, int col, int W, int m2h, float s) {
  const int kw = 1 + (j >> 1);
  if (kw >= m2h) return 0.f;
  const float c = (2 * kw == W) ? s : 2.f * s;
  const float2 t = twiddle_any((kw * col) % W, W);
  return (j & 1) ? -c * t.y : c * t.x;
}

// ------------------------------------------------------------------------
// The inverse column transform is done here, from the window spectrum
// yhat[b][o] (j < m1 window rows, frequency j - m1/2; per channel the rows'
// AC bins kw >= 1 as runs of m2h - 1 entries, then the m1 DC entries), so no
// H x m2h intermediate goes through memory.  A workgroup takes blocks
// of R = 8 rows of one sample, h_t = r + (H / R) t (one residue class r of
// H / R), for which
//   Z[o, h_t, kw] = sum_j yhat[o, j, kw] w_H^(f_j h_t)
//                 = sum_{c < R} w_R^(c t) P_c,   P_c = sum_{f_j = c mod R} yhat[o, j, kw] w_H^(f_j r)
// (w_N = e^{2 pi i / N}): m1 twiddled sums into R residues, then one R-point
// DFT gives all R rows.  Thread (o, q) of the 512 owns channel o and the
// bins 1 + 4q .. 4 + 4q, exactly one 8-entry fragment group of Zt per row,
// and writes the rows' hi / lo fragments to LDS; the 8 threads of a channel
// also split the DC bin's sum (residue classes of j) and exchange the
// partial sums by lane shuffles.  Then the block's rows run as row products,
// a step of 256 pixels being one row (W = 256) or two rows t, t + 1 of the
// block (W = 128).  The next step's x is in flight during each step, across
// block boundaries too.  Two barriers per block.
//
// Workgroup -> blocks: when the batch is a multiple of the 8 XCDs and the
// CU count is a multiple of 8 x (H / R), the grid is one workgroup per CU and
// workgroup g (placed on XCD g mod 8) takes residue i mod (H / R), i = g / 8,
// of samples g mod 8 + 8 (i / (H / R)) + 8 S k, k = 0, 1, ... (S = CUs /
// (8 H / R) samples per XCD at a time): the workgroups of one XCD work on S
// samples at a time, so their spectra stay in the XCD's L2.  Otherwise blocks
// are dealt out in a stride.
namespace rs {
constexpr int R = 8;                     // rows per block
constexpr int kHidden = 32;              // hidden units of a folded channel MLP
}  // namespace rs
static constexpr int kSynthMaxM1 = 128;   // window rows of the LDS twiddle table
// window rows whose loads are issued together: 4 keeps the 256-pixel row
// kernels free of spills (8: 15 VGPRs spilled) and measured 1-3% faster at
// B32 C64 128^2 and 256^2 than 8 or 16, on a par with 2
#ifndef SYN_BATCH
#define SYN_BATCH 4
#endif

// BF: x and y are bfloat16 (activation storage of the bf16 FNO forward); x
// is then exact in one bf16 term, so the skip and gate products take two
// matrix products instead of three, and y is rounded to bf16 (nearest even)
// at the store.
template <bool BF> struct RowIO;
template <> struct RowIO<false> {
  typedef float T;        // element
  typedef float2 Pair;    // the two pixels of a lane
};
template <> struct RowIO<true> {
  typedef __bf16 T;
  typedef uint32_t Pair;  // two bf16, pixel col0 in the low half
};

template <int W, int CI, int KSZ, bool XSKIP, bool MLP, bool BF>
__global__ void __launch_bounds__(rg::kThreads)
k_row_synth(const typename RowIO<BF>::T* __restrict__ x, const float2* __restrict__ yhat,
            const float* __restrict__ skip_w, const float* __restrict__ bias,
            typename RowIO<BF>::T* __restrict__ y, int B, int H, int m1, int m2h, int skip_kind,
            int act, float s, int xcd_map, LayerMlp mlp) {
  using XPair = typename RowIO<BF>::Pair;
  constexpr uint32_t ES = sizeof(typename RowIO<BF>::T);   // bytes per element
  constexpr int R = rs::R;
  constexpr int ROWS = rg::kStepPx / W;          // rows per step
  constexpr int WPR = rg::kWaves / ROWS;         // waves per row
  constexpr int KSX = XSKIP ? CI / 32 : 0;
  constexpr int KX = KSX > 0 ? KSX : 1;
  constexpr int ZROW = KSZ * 4 * 2 * 64;         // 16-byte fragments per row
  constexpr int WFRAG = 4 * KX * 2 * 64;
  static_assert(R % ROWS == 0, "steps pair rows of a block");
  static_assert(CI % 32 == 0, "input channels in k-steps of 32");
  extern __shared__ float4 smem4[];
  v8bf* zf = reinterpret_cast<v8bf*>(smem4);                   // [R][ZROW]
  v8bf* wf = zf + R * ZROW;                                    // [WFRAG]
  float* cinit = reinterpret_cast<float*>(wf + WFRAG);         // [R][64]
  float2* twl = reinterpret_cast<float2*>(cinit + R * rg::kCo);  // [m1] block twiddles
  // channel MLP (MLP only): W1 / W2 as bf16 A fragments, b1, b2 (+ gate
  // bias) and the gate weights
  v8bf* w1f = reinterpret_cast<v8bf*>(twl + kSynthMaxM1);    // [2 ht][2 ks][64]
  v8bf* w2f = w1f + 2 * 2 * 64;                              // [4 ot][64]
  float* mb1 = reinterpret_cast<float*>(w2f + 4 * 64);       // [32]
  float* mseed = mb1 + rs::kHidden;                          // [64] b2 + gate bias
  float* mgate = mseed + rg::kCo;                            // [64] gate weight (0: none)

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = lane >> 4, n = lane & 15;
  const int wrow = wave / WPR;                   // row of the step (0 or 1)
  const int col0 = 32 * (wave % WPR) + 2 * n;
  const uint32_t HW = (uint32_t)H * W;
  const int NR = H / R;                          // residue classes per sample
  const int64_t nblocks = (int64_t)B * NR;
  const uint32_t gmask = act_mask(act == FNO_ACT_GELU);

  // block index k of this workgroup -> (sample, residue), or -1 past the end
  auto block_of = [&](int k, int& b, int& r) __attribute__((always_inline)) -> bool {
    if (xcd_map) {
      // xcd_map = S samples per XCD at a time: workgroup g takes residue
      // (g / 8) % NR of the XCD's sample slot (g / 8) / NR
      const int i = (int)(blockIdx.x >> 3), sl = i / NR;
      b = (int)(blockIdx.x & 7) + 8 * (sl + xcd_map * k);
      r = i - sl * NR;
      return b < B;
    }
    const int64_t e = (int64_t)blockIdx.x + (int64_t)gridDim.x * k;
    b = (int)(e / NR);
    r = (int)(e % NR);
    return e < nblocks;
  };

  // ---- skip-weight fragments (LDS) and synthesis-table fragments (registers)
  if constexpr (XSKIP) {
    for (int f = tid; f < 4 * KSX * 64; f += rg::kThreads) {
      const int ln = f & 63, ks = (f >> 6) % KSX, ot = (f >> 6) / KSX;
      v8bf hi, lo;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int o = 16 * ot + (ln & 15), ci = 32 * ks + 8 * (ln >> 4) + i;
        float v;
        if (skip_kind == FNO_SKIP_LINEAR) v = skip_w[o * CI + ci];
        else if (skip_kind == FNO_SKIP_SOFT_GATING) v = (ci == o) ? skip_w[o] : 0.f;
        else v = (ci == o) ? 1.f : 0.f;
        const bf16x2 p = split_bf16(v);
        hi[i] = p.hi;
        lo[i] = p.lo;
      }
      wf[((ot * KSX + ks) * 2) * 64 + ln] = hi;
      wf[((ot * KSX + ks) * 2 + 1) * 64 + ln] = lo;
    }
  }
  if constexpr (MLP) {
    // The accumulators of a 16-row tile hold rows 4G + r (r < 4) in lane
    // group G, so the bf16 B operand of the next product, 8 rows per lane
    // group, takes rows 4G + r of two consecutive tiles: K slot (G, i) of
    // k-step ks is channel 32 ks + 16 (i / 4) + 4 G + i % 4 of y1 (W1
    // product) and hidden unit 16 (i / 4) + 4 G + i % 4 of h (W2 product).
    // The A fragments take their columns in the same order.
    for (int f = tid; f < 2 * 2 * 64 + 4 * 64; f += rg::kThreads) {
      const int ln = f & 63, m = ln & 15, g = ln >> 4;
      v8bf a;
      if (f < 2 * 2 * 64) {
        const int ks = (f >> 6) & 1, ht = f >> 7;
#pragma unroll
        for (int i = 0; i < 8; ++i)
          a[i] = (__bf16)mlp.w1[(16 * ht + m) * rg::kCo + 32 * ks + 16 * (i >> 2) + 4 * g + (i & 3)];
        w1f[f] = a;
      } else {
        const int ot = (f - 2 * 2 * 64) >> 6;
#pragma unroll
        for (int i = 0; i < 8; ++i)
          a[i] = (__bf16)mlp.w2[(16 * ot + m) * rs::kHidden + 16 * (i >> 2) + 4 * g + (i & 3)];
        w2f[f - 2 * 2 * 64] = a;
      }
    }
    for (int o = tid; o < rg::kCo; o += rg::kThreads) {
      if (o < rs::kHidden) mb1[o] = mlp.b1 ? mlp.b1[o] : 0.f;
      mseed[o] = (mlp.b2 ? mlp.b2[o] : 0.f) + (mlp.gate_b ? mlp.gate_b[o] : 0.f);
      mgate[o] = mlp.gate_kind == FNO_SKIP_SOFT_GATING ? mlp.gate_w[o]
                 : mlp.gate_kind == FNO_SKIP_IDENTITY  ? 1.f
                                                       : 0.f;
    }
  }
  v8bf th[2][KSZ], tl[2][KSZ];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int ks = 0; ks < KSZ; ++ks)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const bf16x2 p = split_bf16(synth_entry(32 * ks + 8 * G + i, col0 + u, W, m2h, s));
        th[u][ks][i] = p.hi;
        tl[u][ks][i] = p.lo;
      }

  // ---- x operand of rows (h, h + 1 at W = 128): channel 32 ks + 8 G + i,
  //      pixels col0, col0 + 1 of row h + wrow
  const uint32_t xbytes = (uint32_t)CI * HW * ES;
  const uint32_t xvoff = ((uint32_t)(8 * G) * HW + (uint32_t)(wrow * NR * W + col0)) * ES;
  XPair xa[KX][8], xb[KX][8];
  // row of step t of a block: steps pair rows t, t + 1 of the block at W = 128
  auto step_row = [&](int r, int t) __attribute__((always_inline)) { return r + NR * t; };
  auto load_x = [&](int b, int h, XPair (&dst)[KX][8]) __attribute__((always_inline)) {
    if constexpr (XSKIP) {
      const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + (int64_t)b * CI * HW, xbytes);
      // rows h (waves of row 0) and h + NR (row 1 of the step at W = 128)
#pragma unroll
      for (int ks = 0; ks < KSX; ++ks)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int soff = __builtin_amdgcn_readfirstlane(
              (int)(((uint32_t)(32 * ks + i) * HW + (uint32_t)h * W) * ES));
          if constexpr (BF)
            dst[ks][i] = __builtin_amdgcn_raw_buffer_load_b32(rx, (int)xvoff, soff, rg::kNT);
          else
            dst[ks][i] = __builtin_bit_cast(
                float2, __builtin_amdgcn_raw_buffer_load_b64(rx, (int)xvoff, soff, rg::kNT));
        }
    }
  };

  // ---- one step: rows t0 (+1) of the block in zf / cinit
  // bf16 hi / lo parts of pixel u of an x pair (lo = 0 for bf16 x)
  auto split_x = [&](const XPair& p, int u) __attribute__((always_inline)) -> bf16x2 {
    if constexpr (BF)
      return {__builtin_bit_cast(__bf16, (unsigned short)(u ? (p >> 16) : (p & 0xffffu))),
              (__bf16)0.f};
    else
      return split_bf16(u ? p.y : p.x);
  };
  auto compute_store = [&](int b, int h, int t0, const XPair (&xc)[KX][8])
      __attribute__((always_inline)) {
    const int t = t0 + wrow;
    v4f acc[4][2];
    const float* ci0 = cinit + t * rg::kCo + 4 * G;
#pragma unroll
    for (int ot = 0; ot < 4; ++ot) {
      const v4f c = *reinterpret_cast<const v4f*>(ci0 + 16 * ot);
      acc[ot][0] = c;
      acc[ot][1] = c;
    }
    if constexpr (XSKIP) {
#pragma unroll
      for (int ks = 0; ks < KSX; ++ks)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          v8bf bh, bl;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const bf16x2 q = split_x(xc[ks][i], u);
            bh[i] = q.hi;
            bl[i] = q.lo;
          }
#pragma unroll
          for (int ot = 0; ot < 4; ++ot) {
            const v8bf wh = wf[((ot * KSX + ks) * 2) * 64 + lane];
            const v8bf wl = wf[((ot * KSX + ks) * 2 + 1) * 64 + lane];
            if constexpr (!BF)
              acc[ot][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wh, bl, acc[ot][u], 0, 0, 0);
            acc[ot][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wl, bh, acc[ot][u], 0, 0, 0);
            acc[ot][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wh, bh, acc[ot][u], 0, 0, 0);
          }
        }
    }
    const v8bf* fz = zf + t * ZROW + lane;
#pragma unroll
    for (int ks = 0; ks < KSZ; ++ks)
#pragma unroll
      for (int ot = 0; ot < 4; ++ot) {
        const v8bf ah = fz[((ks * 4 + ot) * 2) * 64];
        const v8bf al = fz[((ks * 4 + ot) * 2 + 1) * 64];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          acc[ot][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, tl[u][ks], acc[ot][u], 0, 0, 0);
          acc[ot][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, th[u][ks], acc[ot][u], 0, 0, 0);
          acc[ot][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, th[u][ks], acc[ot][u], 0, 0, 0);
        }
      }
    if constexpr (MLP) {
      // compiler barrier: the MLP's LDS operands are read again in every
      // step rather than kept in registers across the unrolled steps
      __asm__ volatile("" ::: "memory");
      // y1 = act(acc), rounded to bf16, as the B fragments of the W1 product
      // (K slot (G, i) of k-step ks: channel 32 ks + 16 (i / 4) + 4 G + i % 4)
      v8bf yb[2][2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            float v = acc[2 * ks + (i >> 2)][u][i & 3];
            v = act_select(gelu_erf(v), v, gmask);
            yb[ks][u][i] = (__bf16)v;
          }
      // h = gelu(W1 y1 + b1), 2 tiles of 16 hidden units
      v4f hacc[2][2];
#pragma unroll
      for (int ht = 0; ht < 2; ++ht)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int r = 0; r < 4; ++r) hacc[ht][u][r] = mb1[16 * ht + 4 * G + r];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int ht = 0; ht < 2; ++ht) {
          const v8bf a = w1f[(ht * 2 + ks) * 64 + lane];
#pragma unroll
          for (int u = 0; u < 2; ++u)
            hacc[ht][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, yb[ks][u], hacc[ht][u], 0, 0, 0);
        }
      v8bf hb[2];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i) hb[u][i] = (__bf16)gelu_erf(hacc[i >> 2][u][i & 3]);
      // y = act(W2 h + b2 + g x): the accumulators seeded with b2 (+ gate
      // bias); g x as the product diag(g) . x on the x fragments of the skip
      // (three-term splits, like the skip); the store applies the activation
#pragma unroll
      for (int ot = 0; ot < 4; ++ot)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[ot][u][r] = mseed[16 * ot + 4 * G + r];
      // diag(g) fragment of tile ot in k-step ks = ot / 2: lane (G, m) holds
      // g[16 ot + m] in slot m % 8 when 8 G + m % 8 == 16 (ot % 2) + m
      const int m16 = lane & 15;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          v8bf bh, bl;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const bf16x2 q = split_x(xc[ks][i], u);
            bh[i] = q.hi;
            bl[i] = q.lo;
          }
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const int ot = 2 * ks + t;
            const bool mine = G == 2 * t + (m16 >> 3);
            const bf16x2 g = split_bf16(mine ? mgate[16 * ot + m16] : 0.f);
            v8bf gh, gl;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              gh[i] = (i == (m16 & 7)) ? g.hi : (__bf16)0.f;
              gl[i] = (i == (m16 & 7)) ? g.lo : (__bf16)0.f;
            }
            if constexpr (!BF)
              acc[ot][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(gh, bl, acc[ot][u], 0, 0, 0);
            acc[ot][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(gl, bh, acc[ot][u], 0, 0, 0);
            acc[ot][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(gh, bh, acc[ot][u], 0, 0, 0);
          }
        }
#pragma unroll
      for (int ot = 0; ot < 4; ++ot) {
        const v8bf a = w2f[ot * 64 + lane];
#pragma unroll
        for (int u = 0; u < 2; ++u)
          acc[ot][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, hb[u], acc[ot][u], 0, 0, 0);
      }
    }
    const __amdgpu_buffer_rsrc_t ry = make_rsrc(y + (int64_t)b * rg::kCo * HW,
                                                (uint32_t)rg::kCo * HW * ES);
    const uint32_t yvoff =
        ((uint32_t)(4 * G) * HW + (uint32_t)(wrow * NR * W + col0)) * ES;
#pragma unroll
    for (int ot = 0; ot < 4; ++ot)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v0 = acc[ot][0][r], v1 = acc[ot][1][r];
        v0 = act_select(gelu_erf(v0), v0, gmask);
        v1 = act_select(gelu_erf(v1), v1, gmask);
        const int soff = __builtin_amdgcn_readfirstlane(
            (int)(((uint32_t)(16 * ot + r) * HW + (uint32_t)h * W) * ES));
        if constexpr (BF) {
          const uint32_t lo = __builtin_bit_cast(unsigned short, (__bf16)v0);
          const uint32_t hi = __builtin_bit_cast(unsigned short, (__bf16)v1);
          __builtin_amdgcn_raw_buffer_store_b32(lo | (hi << 16), ry, (int)yvoff, soff, rg::kNT);
        } else {
          __builtin_amdgcn_raw_buffer_store_b64(
              __builtin_bit_cast(__attribute__((ext_vector_type(2))) int, make_float2(v0, v1)),
              ry, (int)yvoff, soff, rg::kNT);
        }
      }
  };

  // ---- column synthesis of block (b, r) into zf / cinit.  Window row j =
  //      j0 + cc (j0 a multiple of R) has frequency f = j - m1/2, so its
  //      residue is c = (cc - m1/2) mod R: sums are kept by cc and the offset
  //      becomes the factor w_R^(-(m1/2) t) of output row t.
  //      Bins 1..32: thread tid owns bin kw = 1 + tid % 32 of the channels
  //      o = tid / 32 + 16 i (i < 4), so 32 consecutive lanes read one
  //      channel's 256 contiguous bytes of a window row.  DC: thread (so, sq)
  //      = (tid / 8, tid % 8) sums the window rows j = sq (mod R) of channel so.
  const int kwt = 1 + (tid & 31), ot0 = tid >> 5;
  const int so = tid >> 3, sq = tid & 7;
  const int jlo = m1 / 2;
  auto synthesize = [&](int b, int r) __attribute__((always_inline)) {
    // the block's twiddles w_H^((j - m1/2) r), j < m1, into LDS
    for (int j = tid; j < m1; j += rg::kThreads)
      twl[j] = twiddle_any((((j - jlo) * r) % H + H) % H, H);
    // one descriptor per sample (a per-lane base would serialise every load
    // over the distinct channels of the wave); the channel goes in the offset
    const __amdgpu_buffer_rsrc_t ryh = make_rsrc(yhat + (int64_t)b * rg::kCo * m1 * m2h,
                                                 (uint32_t)(rg::kCo * m1 * m2h * 8));
    // a channel's plane (m1 x m2h entries) holds the window rows' AC bins
    // kw = 1 .. m2h-1 first (row j at j (m2h - 1) + kw - 1), then the DC
    // column (row j at m1 (m2h - 1) + j)
    const int ac = m2h - 1;
    const uint32_t cstride = (uint32_t)(16 * m1 * m2h) * 8u;   // 16 channels
    const uint32_t boff = kwt < m2h ? (uint32_t)(ot0 * m1 * m2h + kwt - 1) * 8u : 0x80000000u;
    const uint32_t dbase = (uint32_t)(so * m1 * m2h + m1 * ac) * 8u;
    float2 P[R][4];
#pragma unroll
    for (int c = 0; c < R; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) P[c][i] = make_float2(0.f, 0.f);
    float2 pdc = make_float2(0.f, 0.f);
    __syncthreads();
    // chunks of R window rows; rows past m1 read past the end (zero).  Each
    // half chunk's loads are all issued before its products.
#pragma unroll 1
    for (int j0 = 0; j0 < m1; j0 += R) {
      // DC: row j0 + sq of channel so
      const int jd = j0 + sq;
      const float2 vd = __builtin_bit_cast(
          float2, __builtin_amdgcn_raw_buffer_load_b64(
                      ryh, (int)(jd < m1 ? dbase + (uint32_t)jd * 8u : 0x80000000u), 0, 0));
#pragma unroll
      for (int hc = 0; hc < R; hc += SYN_BATCH) {
        float2 v[SYN_BATCH][4];
#pragma unroll
        for (int cc = 0; cc < SYN_BATCH; ++cc) {
          const int j = j0 + hc + cc;
          const uint32_t bo = j < m1 ? boff : 0x80000000u;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int soff = __builtin_amdgcn_readfirstlane((int)(i * cstride + j * ac * 8));
            v[cc][i] = __builtin_bit_cast(
                float2, __builtin_amdgcn_raw_buffer_load_b64(ryh, (int)bo, soff, 0));
          }
        }
#pragma unroll
        for (int cc = 0; cc < SYN_BATCH; ++cc) {
          const float2 w = twl[min(j0 + hc + cc, m1 - 1)];
#pragma unroll
          for (int i = 0; i < 4; ++i) cfma(P[hc + cc][i], v[cc][i], w);
        }
      }
      cfma(pdc, vd, twl[min(jd, m1 - 1)]);
    }
    // DC bin: thread (so, sq) has summed the window rows j = sq (mod R);
    // it gathers the channel's 8 sums and keeps row t = sq
    float2 zdc = make_float2(0.f, 0.f);
#pragma unroll
    for (int cc = 0; cc < R; ++cc) {
      const int src = (lane & ~(R - 1)) | cc;
      const float2 pc = make_float2(__shfl(pdc.x, src, 64), __shfl(pdc.y, src, 64));
      cfma(zdc, pc, twiddle_any((cc * sq) % R, R));
    }
    const float2 rot = twiddle_any(((-jlo * sq) % R + R) % R, R);
    cinit[sq * rg::kCo + so] = (bias ? bias[so] : 0.f) + s * (zdc.x * rot.x - zdc.y * rot.y);
    // R-point DFT over the residues for each channel, the row factor, and
    // the hi / lo parts into the fragment slots of (o, kw): entry
    // j' = 2 (kw - 1) (+1 for Im) of k-step j' / 32, lane group (j' % 32) / 8
    const int jp = 2 * (kwt - 1), ks = jp >> 5, g = (jp & 31) >> 3, el = jp & 7;
    const bool on = kwt < m2h && ks < KSZ;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float2 v[R];
#pragma unroll
      for (int c = 0; c < R; ++c) v[c] = P[c][i];
      dft8<+1>(v);
      const int o = ot0 + 16 * i;
      if (on) {
        // 16-byte fragment (ks, ot = i, hi | lo) of lane (o % 16) + 16 g; the
        // pair (Re, Im) is bf16 elements el, el + 1 of it
        __bf16* fb = reinterpret_cast<__bf16*>(zf + ((ks * 4 + i) * 2) * 64 + (o & 15) + 16 * g) + el;
#pragma unroll
        for (int t = 0; t < R; ++t) {
          const float2 zt = cmul(v[t], twiddle_any(((-jlo * t) % R + R) % R, R));
          const bf16x2 pr = split_bf16(zt.x), pi = split_bf16(zt.y);
          typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
          v2bf h2, l2;
          h2[0] = pr.hi;
          h2[1] = pi.hi;
          l2[0] = pr.lo;
          l2[1] = pi.lo;
          *reinterpret_cast<v2bf*>(fb + t * ZROW * 8) = h2;
          *reinterpret_cast<v2bf*>(fb + (t * ZROW + 64) * 8) = l2;
        }
      }
    }
    // fragment entries of bins at or past m2h (and of unowned slots) stay
    // zero: written once at the start, since every block leaves them alone
  };

  int b, r;
  if (!block_of(0, b, r)) return;   // no barrier is reached by this workgroup
  for (int i = tid; i < R * ZROW; i += rg::kThreads) zf[i] = (v8bf)0;
  __syncthreads();
  load_x(b, step_row(r, 0), xa);
  constexpr int NSTEP = R / ROWS;
#pragma unroll 1
  for (int k = 0;; ++k) {
    synthesize(b, r);
    __syncthreads();
    int nb, nr;
    const bool more = block_of(k + 1, nb, nr);
#pragma unroll
    for (int st = 0; st < NSTEP; st += 2) {
      // step st from xa, step st + 1 from xb; the following step's x in flight
      load_x(b, step_row(r, ROWS * (st + 1)), xb);
      compute_store(b, step_row(r, ROWS * st), ROWS * st, xa);
      if (st + 2 < NSTEP) load_x(b, step_row(r, ROWS * (st + 2)), xa);
      else if (more) load_x(nb, step_row(nr, 0), xa);
      compute_store(b, step_row(r, ROWS * (st + 1)), ROWS * (st + 1), xb);
    }
    __syncthreads();
    if (!more) break;
    b = nb;
    r = nr;
  }
}

// ============================================================== host side
static int rowgemm_ksz(int m2h) { return (2 * (m2h - 1) + 31) / 32; }

static int device_cus() {
  static int cus = 0;
  if (!cus) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cus = n;
    else
      cus = 256;
  }
  return cus;
}

// ---- row products with the column synthesis from yhat

static size_t rowsynth_lds_bytes(int ksz, int ksx, bool mlp = false) {
  return (size_t)rs::R * ksz * 4 * 2 * 64 * 16 + (size_t)4 * (ksx > 0 ? ksx : 1) * 2 * 64 * 16 +
         (size_t)rs::R * rg::kCo * sizeof(float) + (size_t)kSynthMaxM1 * 8 +
         (mlp ? (size_t)(2 * 2 * 64 + 4 * 64) * 16 + (size_t)(rs::kHidden + 2 * rg::kCo) * 4 : 0);
}

// Shapes k_row_synth covers for every skip kind: 64 output channels, 32 or
// 64 input channels, rows of 128 or 256 pixels, H a multiple of the block's
// 8 rows, at most 32 bins past DC (two k-steps of Zt).
bool rowsynth_covers(int H, int W, int Ci, int Co, int m1, int m2h) {
  if (!(W == 128 || W == 256) || Co != rg::kCo || !(Ci == 32 || Ci == 64)) return false;
  if (H % rs::R != 0 || H < rs::R || m1 < 1 || m1 > H || m1 > kSynthMaxM1) return false;
  if (m2h < 2 || m2h > 33) return false;
  return rowsynth_lds_bytes(rowgemm_ksz(m2h), 2) <= 160 * 1024;
}

template <int W, int CI, int KSZ, bool XSKIP, bool MLP = false, bool BF = false>
static int launch_rowsynth(const typename RowIO<BF>::T* x, const float2* yhat, const float* skip_w,
                           const float* bias, typename RowIO<BF>::T* y, int B, int H, int m1, int m2h,
                           int skip_kind, int act, float s, hipStream_t st,
                           const LayerMlp& mlp = LayerMlp{}) {
  const size_t lds = rowsynth_lds_bytes(KSZ, XSKIP ? CI / 32 : 0, MLP);
  auto kern = k_row_synth<W, CI, KSZ, XSKIP, MLP, BF>;
  if (lds > 64 * 1024) {
    int rc = hip_status(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                        "hipFuncSetAttribute(MaxDynamicSharedMemorySize)");
    if (rc) return rc;
  }
  const int NR = H / rs::R;
  const int64_t nblocks = (int64_t)B * NR;
  const int cus = device_cus();
  // XCD-grouped blocks when every XCD gets whole samples and one workgroup
  // per CU covers S whole samples' residues per XCD (S = 1 at 256 rows, 2 at
  // 128); otherwise a stride over all blocks
  const int S = (B % 8 == 0 && cus % (8 * NR) == 0) ? cus / (8 * NR) : 0;
  const int64_t grid = S ? cus : (nblocks < cus ? nblocks : cus);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(rg::kThreads), lds, st, x, yhat, skip_w,
                     bias, y, B, H, m1, m2h, skip_kind, act, s, S, mlp);
  return launch_status("k_row_synth");
}

template <int W>
static int dispatch_rowsynth_w(const float* x, const float2* yhat, const float* skip_w,
                               const float* bias, float* y, int B, int Ci, int H, int m1, int m2h,
                               int skip_kind, int act, float s, hipStream_t st) {
  const int ksz = rowgemm_ksz(m2h);
  const bool xs = skip_kind != FNO_SKIP_NONE;
  const int ci = skip_kind == FNO_SKIP_LINEAR ? Ci : rg::kCo;
#define FNO_RS(cin, k)                                                                           \
  if (xs && ci == cin && ksz == k)                                                               \
    return launch_rowsynth<W, cin, k, true>(x, yhat, skip_w, bias, y, B, H, m1, m2h, skip_kind, \
                                            act, s, st);
  FNO_RS(32, 1) FNO_RS(32, 2) FNO_RS(64, 1) FNO_RS(64, 2)
#undef FNO_RS
  if (!xs && ksz == 1)
    return launch_rowsynth<W, 64, 1, false>(x, yhat, skip_w, bias, y, B, H, m1, m2h, skip_kind,
                                            act, s, st);
  if (!xs && ksz == 2)
    return launch_rowsynth<W, 64, 2, false>(x, yhat, skip_w, bias, y, B, H, m1, m2h, skip_kind,
                                            act, s, st);
  set_error("row synthesis epilogue: unsupported Ci=%d m2h=%d", Ci, m2h);
  return FNO_ERR_UNSUPPORTED;
}

// Shapes the row epilogue can also fold a layer's channel MLP into: 64
// input channels (the gate adds the layer input), 64 hidden-row bins at most
// two k-steps, a skip, and room in LDS for the MLP's weights.
bool rowsynth_mlp_covers(int H, int W, int Ci, int Co, int m1, int m2h, int hidden,
                         int skip_kind) {
  if (!rowsynth_covers(H, W, Ci, Co, m1, m2h) || Ci != rg::kCo || hidden != rs::kHidden)
    return false;
  if (skip_kind == FNO_SKIP_NONE) return false;
  return rowsynth_lds_bytes(rowgemm_ksz(m2h), 2, true) <= 160 * 1024;
}

// bf: x and y bfloat16 (else float32).
int rowsynth_mlp_epilogue(const void* x, const float2* yhat, const float* skip_w,
                          const float* bias, void* y, int B, int H, int W, int m1, int m2h,
                          int skip_kind, int act, float s, const LayerMlp& mlp, bool bf,
                          hipStream_t st) {
  const int ksz = rowgemm_ksz(m2h);
#define FNO_RSM(w, k, b)                                                                           \
  if (W == w && ksz == k && bf == b)                                                               \
    return launch_rowsynth<w, 64, k, true, true, b>(                                               \
        static_cast<const typename RowIO<b>::T*>(x), yhat, skip_w, bias,                           \
        static_cast<typename RowIO<b>::T*>(y), B, H, m1, m2h, skip_kind, act, s, st, mlp);
  FNO_RSM(128, 1, false) FNO_RSM(128, 2, false) FNO_RSM(256, 1, false) FNO_RSM(256, 2, false)
  FNO_RSM(128, 1, true) FNO_RSM(128, 2, true) FNO_RSM(256, 1, true) FNO_RSM(256, 2, true)
#undef FNO_RSM
  set_error("row epilogue with channel MLP: unsupported W=%d m2h=%d", W, m2h);
  return FNO_ERR_UNSUPPORTED;
}

int rowsynth_epilogue(const float* x, const float2* yhat, const float* skip_w, const float* bias,
                      float* y, int B, int Ci, int H, int W, int m1, int m2h, int skip_kind,
                      int act, float s, hipStream_t st) {
  if (W == 128)
    return dispatch_rowsynth_w<128>(x, yhat, skip_w, bias, y, B, Ci, H, m1, m2h, skip_kind, act,
                                    s, st);
  return dispatch_rowsynth_w<256>(x, yhat, skip_w, bias, y, B, Ci, H, m1, m2h, skip_kind, act, s,
                                  st);
}

}  // namespace fno
