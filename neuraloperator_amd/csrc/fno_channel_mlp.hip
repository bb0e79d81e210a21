// Fused channel MLP of an FNO layer:
//
//   y = act( W2 gelu(W1 x + b1) + b2 + skip(xs) )
//
// the two pointwise 1x1 convolutions of ChannelMLP.forward
// (neuralop/layers/channel_mlp.py:82-119, n_layers = 2, GELU between), the
// channel-MLP skip (SoftGating.forward, neuralop/layers/skip_connections.py
// :88-93, or identity) and the block's second activation
// (neuralop/layers/fno_block.py:363-379), in one pass over the field: x and xs
// are read once, y written once, the hidden activation never leaves the CU.
//
// k_channel_mlp<CI, CH, CO>: persistent workgroups of 4 waves stride over
// tiles of TP = 128 points of one sample.  Per tile:
//   * the [CI][TP] slab of x moves through LDS (the next tile's slab is in
//     flight in registers while this one is computed);
//   * GEMM 1 on v_mfma_f32_16x16x4f32: each wave owns 32 points (2 column
//     tiles) and all CH hidden rows; A (W1) comes from LDS in lane order, B
//     (x) from the slab;
//   * bias + GELU in the accumulators;
//   * GEMM 2 takes its B operand straight from GEMM 1's accumulators: lane
//     group G holds hidden rows 16m + 4G + r (register r) of its point column,
//     so k-step (m, r) contracts hidden row 16m + 4G + r in lane group G, and
//     W2 is staged in that order;
//   * bias, skip, activation and the store of y from GEMM 2's accumulators.
// BF = false: fp32 operands and accumulation throughout.  BF = true: the two
// GEMMs take bf16-rounded operands (round to nearest even) on
// v_mfma_f32_16x16x32_bf16 with fp32 accumulation, the arithmetic of a 1x1
// convolution under torch.autocast(dtype=torch.bfloat16); bias, skip and
// activations stay fp32.  Its k order is permuted the same way: element j of
// lane group G is input row 32 kb + 16 (j / 4) + 4 (j % 4) + G in GEMM 1 (so
// the slab swizzle still separates the groups) and hidden row
// 16 (2 kb + j / 4) + 4 G + j % 4 in GEMM 2 (two of GEMM 1's accumulator
// tiles per k-step).
#include <type_traits>

#include "fno_common.h"

namespace fno {

namespace {
constexpr int kMlpWaves = 4;
constexpr int kMlpThreads = 64 * kMlpWaves;
constexpr int kMlpTP = 32 * kMlpWaves;   // points per tile
constexpr int kMlpXS = kMlpTP;           // slab row stride (floats)
// slab column of point c in row `row`: XOR-swizzled by 16 (row % 4) so the
// four lane groups of an MFMA operand read (rows 4k + G) hit distinct banks
__device__ __forceinline__ int slab_col(int row, int c) { return c ^ ((row & 3) << 4); }
// output tile column: rows 16 mo + 4 G + r are written by lane group G, so
// the swizzle follows G = (row / 4) % 4
__device__ __forceinline__ int out_col(int row, int c) { return c ^ (((row >> 2) & 3) << 4); }
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// LDS bytes of the staged weights: fp32 lane-order operands, or bf16 ones as
// 64 lanes x 8 elements (1 KB) per (M tile, k-step)
template <int CI, int CH, int CO, bool TWO, bool BF>
struct MlpLds {
  static constexpr int MT1 = CH / 16, MT2 = CO / 16, KB1 = (CI + 31) / 32, KB2 = (MT1 + 1) / 2;
  static constexpr size_t w1 = BF ? (size_t)MT1 * KB1 * 1024 : (size_t)CH * CI * 4;
  static constexpr size_t w2 = !TWO ? 0 : BF ? (size_t)MT2 * KB2 * 1024 : (size_t)CO * CH * 4;
  // output tile [CO][TP] for 16-byte stores: the input slab when it is at
  // least as tall, else a region of its own
  static constexpr size_t ot = CO <= CI ? 0 : (size_t)CO * kMlpXS * 4;
  static constexpr size_t total = w1 + w2 + (size_t)(CI * kMlpXS + 2 * CO) * 4 + ot;
};
}  // namespace

// TWO = false: a single 1x1 layer y = act(W1 x + b2 + skip) (CH == CO), the
// linear skip of the block epilogue with the spectral term as identity skip.
// IO: storage of x (bit 0) and y (bit 1), bfloat16 where set (the lifting's
// output and the projection's input in the bf16 FNO forward), else float32;
// x is widened to fp32 in the slab, y rounded to bf16 (nearest even) at the
// store.
template <int CI, int CH, int CO, bool TWO, bool BF, int IO = 0>
__global__ void __launch_bounds__(kMlpThreads) __attribute__((amdgpu_waves_per_eu(CI <= 64 ? 2 : 1)))
k_channel_mlp(const void* xv, const float* __restrict__ w1, const float* __restrict__ b1,
              const float* __restrict__ w2, const float* __restrict__ b2, const float* xs,
              const float* __restrict__ sw, const float* __restrict__ sb, void* yv, int64_t P,
              int64_t tiles_per_sample, int64_t tiles, int ci, int co, int skip_kind, int act) {
  constexpr bool XBF = IO & 1, YBF = IO & 2;
  using XT = std::conditional_t<XBF, __bf16, float>;
  using YT = std::conditional_t<YBF, __bf16, float>;
  using XQ = std::conditional_t<XBF, uint2, float4>;   // 4 points of x as loaded
  const XT* x = static_cast<const XT*>(xv);
  YT* y = static_cast<YT*>(yv);
  static_assert(CI % 4 == 0 && CH % 16 == 0 && CO % 16 == 0, "channel multiples");
  static_assert(TWO || CH == CO, "one layer: CH == CO");
  // outputs go back through LDS as a [CO][TP] tile (the slab, or a region of
  // their own when CO > CI) for 16-byte stores
  constexpr int NQO = CO * kMlpTP / 4;                // float4s per output tile
  constexpr int LPO = (NQO + kMlpThreads - 1) / kMlpThreads;
  constexpr int KS1 = CI / 4, MT1 = CH / 16, MT2 = CO / 16;
  constexpr int NQ = CI * kMlpTP / 4;                  // float4s per slab
  constexpr int LPT = (NQ + kMlpThreads - 1) / kMlpThreads;   // ... per thread
  static_assert(NQ % kMlpThreads == 0 || NQ < kMlpThreads, "slab split");
  using LD = MlpLds<CI, CH, CO, TWO, BF>;
  constexpr int KB1 = LD::KB1, KB2 = LD::KB2;
  extern __shared__ float4 smem4[];
  char* lds = reinterpret_cast<char*>(smem4);
  float* w1s = reinterpret_cast<float*>(lds);          // [MT1][KS1][64] lane order
  float* w2s = reinterpret_cast<float*>(lds + LD::w1);  // [MT2][MT1][4][64] lane order
  __bf16* w1b = reinterpret_cast<__bf16*>(lds);         // [MT1][KB1][64][8]
  __bf16* w2b = reinterpret_cast<__bf16*>(lds + LD::w1);  // [MT2][KB2][64][8]
  float* slab = reinterpret_cast<float*>(lds + LD::w1 + LD::w2);   // [CI][kMlpXS]
  float* bos = slab + CI * kMlpXS;                // [CO] output bias (+ gate bias)
  float* gws = bos + CO;                          // [CO] gate weight
  float* otile = CO <= CI ? slab : gws + CO;      // [CO][kMlpXS] output tile
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = lane >> 4, t = lane & 15;

  if constexpr (BF) {
    for (int e = tid; e < MT1 * KB1 * 512; e += kMlpThreads) {
      const int j = e & 7, l = (e >> 3) & 63, kb = (e >> 9) % KB1, m = (e >> 9) / KB1;
      const int k = 32 * kb + 16 * (j >> 2) + 4 * (j & 3) + (l >> 4);
      w1b[e] = (__bf16)(k < ci ? w1[(16 * m + (l & 15)) * ci + k] : 0.f);
    }
    for (int e = tid; TWO && e < MT2 * KB2 * 512; e += kMlpThreads) {
      const int j = e & 7, l = (e >> 3) & 63, kb = (e >> 9) % KB2, mo = (e >> 9) / KB2;
      const int m = 2 * kb + (j >> 2), oc = 16 * mo + (l & 15);
      w2b[e] = (__bf16)(oc < co && m < MT1 ? w2[oc * CH + 16 * m + 4 * (l >> 4) + (j & 3)] : 0.f);
    }
  } else {
    for (int e = tid; e < CH * CI; e += kMlpThreads) {
      const int l = e & 63, ks = (e >> 6) % KS1, m = (e >> 6) / KS1;
      const int k = 4 * ks + (l >> 4);
      w1s[e] = k < ci ? w1[(16 * m + (l & 15)) * ci + k] : 0.f;
    }
    for (int e = tid; TWO && e < CO * CH; e += kMlpThreads) {
      const int l = e & 63, r = (e >> 6) & 3, m = ((e >> 8) % MT1), mo = (e >> 8) / MT1;
      const int oc = 16 * mo + (l & 15);
      w2s[e] = oc < co ? w2[oc * CH + 16 * m + 4 * (l >> 4) + r] : 0.f;
    }
  }
  for (int o = tid; o < CO; o += kMlpThreads) {
    bos[o] = o >= co ? 0.f
                     : (b2 ? b2[o] : 0.f) + (skip_kind == FNO_SKIP_SOFT_GATING && sb ? sb[o] : 0.f);
    gws[o] = o < co && skip_kind == FNO_SKIP_SOFT_GATING ? sw[o] : 1.f;
  }
  float bh[MT1][4];
#pragma unroll
  for (int m = 0; m < MT1; ++m)
#pragma unroll
    for (int r = 0; r < 4; ++r) bh[m][r] = b1 ? b1[16 * m + 4 * G + r] : 0.f;
  const bool has_skip = skip_kind != FNO_SKIP_NONE;
  const bool gelu_out = act == FNO_ACT_GELU;

  // slab of tile `tile` into registers: float4 q = tid + kMlpThreads j is row
  // q / (TP/4), points 4 (q % (TP/4)) .. +3; points past P read as zero
  XQ pre[LPT];
  auto load_slab = [&](int64_t tile) __attribute__((always_inline)) {
    const int64_t b = tile / tiles_per_sample;
    const int64_t p0 = (tile % tiles_per_sample) * kMlpTP;
    const XT* xb = x + b * ci * P;
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      const int q = tid + kMlpThreads * j;
      const int c = q / (kMlpTP / 4);
      const int64_t p = p0 + 4 * (q % (kMlpTP / 4));
      // a branch, not `cond ? *ptr : zero`: with two lvalue operands that
      // selects between the addresses, putting zero in scratch memory and
      // turning the load into a flat one
      XQ v;
      if constexpr (XBF) v = make_uint2(0u, 0u);
      else v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (q < NQ && p < P && c < ci) v = *reinterpret_cast<const XQ*>(xb + c * P + p);
      pre[j] = v;
    }
  };
  auto widen = [](const XQ& v) __attribute__((always_inline)) -> float4 {
    if constexpr (XBF)
      return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                         __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u));
    else
      return v;
  };

  int64_t tile = blockIdx.x;
  if (tile < tiles) load_slab(tile);
  for (; tile < tiles; tile += gridDim.x) {
    __syncthreads();   // previous tile's slab reads done (and the weights staged)
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      const int q = tid + kMlpThreads * j;
      const int row = q / (kMlpTP / 4);
      if (q < NQ)
        *reinterpret_cast<float4*>(slab + row * kMlpXS + slab_col(row, 4 * (q % (kMlpTP / 4)))) = widen(pre[j]);
    }
    __syncthreads();
    const int64_t b = tile / tiles_per_sample;
    const int64_t p0 = (tile % tiles_per_sample) * kMlpTP;
    if (tile + gridDim.x < tiles) load_slab(tile + gridDim.x);
    // the skip input of this tile's outputs, in flight during the GEMMs
    float4 svq[LPO];
#pragma unroll
    for (int j = 0; j < LPO; ++j) {
      const int q = tid + kMlpThreads * j;
      const int c = q / (kMlpTP / 4);
      const int64_t p = p0 + 4 * (q % (kMlpTP / 4));
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (has_skip && q < NQO && c < co && p < P)
        v = *reinterpret_cast<const float4*>(xs + (b * co + c) * P + p);
      svq[j] = v;
    }

    // GEMM 1: h[16m + row][point] over the wave's 2 column tiles
    v4f h[MT1][2];
#pragma unroll
    for (int m = 0; m < MT1; ++m) h[m][0] = h[m][1] = (v4f)0.f;
    // rows 4 ks + G: the swizzle is 16 G for every ks
    const float* bcol0 = slab + G * kMlpXS + slab_col(G, 32 * wave + t);
    const float* bcol1 = slab + G * kMlpXS + slab_col(G, 32 * wave + 16 + t);
    if constexpr (BF) {
#pragma unroll
      for (int kb = 0; kb < KB1; ++kb) {
        v8bf xb0, xb1;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          // input row r0 + G; rows at or past CI (a multiple of 4) are zero
          const int r0 = 32 * kb + 16 * (j >> 2) + 4 * (j & 3);
          xb0[j] = (__bf16)(r0 < CI ? bcol0[r0 * kMlpXS] : 0.f);
          xb1[j] = (__bf16)(r0 < CI ? bcol1[r0 * kMlpXS] : 0.f);
        }
#pragma unroll
        for (int m = 0; m < MT1; ++m) {
          const v8bf a = *reinterpret_cast<const v8bf*>(w1b + ((m * KB1 + kb) * 64 + lane) * 8);
          h[m][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, xb0, h[m][0], 0, 0, 0);
          h[m][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, xb1, h[m][1], 0, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < KS1; ++ks) {
        const float xb0 = bcol0[4 * ks * kMlpXS], xb1 = bcol1[4 * ks * kMlpXS];
#pragma unroll
        for (int m = 0; m < MT1; ++m) {
          const float a = w1s[(m * KS1 + ks) * 64 + lane];
          h[m][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, xb0, h[m][0], 0, 0, 0);
          h[m][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, xb1, h[m][1], 0, 0, 0);
        }
      }
    }
    v4f o[MT2][2];
    if constexpr (TWO) {
#pragma unroll
      for (int m = 0; m < MT1; ++m)
#pragma unroll
        for (int n = 0; n < 2; ++n)
#pragma unroll
          for (int r = 0; r < 4; ++r) h[m][n][r] = gelu_erf(h[m][n][r] + bh[m][r]);

      // GEMM 2: k-step (m, r) contracts hidden row 16m + 4G + r of lane group G
#pragma unroll
      for (int mo = 0; mo < MT2; ++mo) o[mo][0] = o[mo][1] = (v4f)0.f;
      if constexpr (BF) {
#pragma unroll
        for (int kb = 0; kb < KB2; ++kb) {
          v8bf hb0, hb1;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int m = 2 * kb + (j >> 2), mc = m < MT1 ? m : 0;
            hb0[j] = (__bf16)(m < MT1 ? h[mc][0][j & 3] : 0.f);
            hb1[j] = (__bf16)(m < MT1 ? h[mc][1][j & 3] : 0.f);
          }
#pragma unroll
          for (int mo = 0; mo < MT2; ++mo) {
            const v8bf a = *reinterpret_cast<const v8bf*>(w2b + ((mo * KB2 + kb) * 64 + lane) * 8);
            o[mo][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, hb0, o[mo][0], 0, 0, 0);
            o[mo][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, hb1, o[mo][1], 0, 0, 0);
          }
        }
      } else {
#pragma unroll
        for (int m = 0; m < MT1; ++m)
#pragma unroll
          for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int mo = 0; mo < MT2; ++mo) {
              const float a = w2s[((mo * MT1 + m) * 4 + r) * 64 + lane];
              o[mo][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, h[m][0][r], o[mo][0], 0, 0, 0);
              o[mo][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, h[m][1][r], o[mo][1], 0, 0, 0);
            }
      }
    } else {
#pragma unroll
      for (int mo = 0; mo < MT2; ++mo) {
        o[mo][0] = h[mo][0];
        o[mo][1] = h[mo][1];
      }
    }

    // every wave is past GEMM 1 (the slab may be the output tile)
    __syncthreads();
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int mo = 0; mo < MT2; ++mo)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 16 * mo + 4 * G + r;
          otile[row * kMlpXS + out_col(row, 32 * wave + 16 * n + t)] = o[mo][n][r];
        }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < LPO; ++j) {
      const int q = tid + kMlpThreads * j;
      const int c = q / (kMlpTP / 4);
      const int64_t p = p0 + 4 * (q % (kMlpTP / 4));
      if (q >= NQO || c >= co || p >= P) continue;
      float4 v = *reinterpret_cast<const float4*>(otile + c * kMlpXS + out_col(c, 4 * (q % (kMlpTP / 4))));
      const float bb = bos[c], gg = gws[c];
      v.x += bb; v.y += bb; v.z += bb; v.w += bb;
      if (has_skip) {
        v.x = fmaf(gg, svq[j].x, v.x);
        v.y = fmaf(gg, svq[j].y, v.y);
        v.z = fmaf(gg, svq[j].z, v.z);
        v.w = fmaf(gg, svq[j].w, v.w);
      }
      if (gelu_out) {
        v.x = gelu_erf(v.x);
        v.y = gelu_erf(v.y);
        v.z = gelu_erf(v.z);
        v.w = gelu_erf(v.w);
      }
      if constexpr (YBF) {
        auto pk = [](float a, float b) __attribute__((always_inline)) {
          return (uint32_t)__builtin_bit_cast(unsigned short, (__bf16)a) |
                 ((uint32_t)__builtin_bit_cast(unsigned short, (__bf16)b) << 16);
        };
        *reinterpret_cast<uint2*>(y + (b * co + c) * P + p) = make_uint2(pk(v.x, v.y), pk(v.z, v.w));
      } else {
        *reinterpret_cast<float4*>(y + (b * co + c) * P + p) = v;
      }
    }
  }
}

// --------------------------------------------------------------------- host

// (Ci, Ch, Co) -> kernel widths: Ci <= 4 runs padded to 4 input channels and
// Co <= 16 padded to 16 outputs (the lifting 3 -> 2H -> H and projection
// H -> 2H -> 1 MLPs of FNO); the block MLPs C -> C/2 -> C run at their widths
static int mlp_variant(int Ci, int Ch, int Co) {
  if (Ci == 64 && Ch == 32 && Co == 64) return 0;
  if (Ci == 32 && Ch == 16 && Co == 32) return 1;
  if (Ci == 128 && Ch == 64 && Co == 128) return 2;
  if (Ci <= 4 && Ch == 128 && Co == 64) return 3;
  if (Ci <= 4 && Ch == 64 && Co == 32) return 4;
  if (Ci == 64 && Ch == 128 && Co <= 16) return 5;
  if (Ci == 32 && Ch == 64 && Co <= 16) return 6;
  return -1;
}

bool channel_mlp_supported(int Ci, int Ch, int Co, int64_t P) {
  return P % 4 == 0 && mlp_variant(Ci, Ch, Co) >= 0;
}

template <int CI, int CH, int CO, bool TWO, bool BF, int IO = 0>
static int launch_mlp(const void* x, const float* w1, const float* b1, const float* w2,
                      const float* b2, const float* xs, const float* sw, const float* sb, void* y,
                      int64_t B, int64_t P, int ci, int co, int skip_kind, int act, hipStream_t st) {
  const size_t lds = MlpLds<CI, CH, CO, TWO, BF>::total;
  if (lds > 48 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_channel_mlp<CI, CH, CO, TWO, BF, IO>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
      set_error("channel MLP: %s", hipGetErrorString(e));
      return FNO_ERR_HIP;
    }
  }
  const int64_t tps = (P + kMlpTP - 1) / kMlpTP;
  const int64_t tiles = B * tps;
  // persistent grid: exactly as many workgroups as are resident at once (a
  // second round of workgroups would each carry a full share of the tiles)
  static int per_cu = 0;
  if (per_cu == 0) {
    int n = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &n, reinterpret_cast<const void*>(&k_channel_mlp<CI, CH, CO, TWO, BF, IO>), kMlpThreads, lds);
    per_cu = (e == hipSuccess && n > 0) ? n : 1;
  }
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
    cus = 256;
  int64_t grid = (int64_t)cus * per_cu;
  if (grid > tiles) grid = tiles;
  hipLaunchKernelGGL((k_channel_mlp<CI, CH, CO, TWO, BF, IO>), dim3((unsigned)grid), dim3(kMlpThreads), lds, st,
                     x, w1, b1, w2, b2, xs, sw, sb, y, P, tps, tiles, ci, co, skip_kind, act);
  return launch_status("k_channel_mlp");
}

int channel_mlp(const float* x, const float* w1, const float* b1, const float* w2, const float* b2,
                const float* xs, const float* sw, const float* sb, float* y, int64_t B, int Ci,
                int Ch, int Co, int64_t P, int skip_kind, int act, bool bf16_products,
                hipStream_t st) {
#define FNO_MLP(ci_, ch_, co_)                                                                     \
  (bf16_products                                                                                   \
       ? launch_mlp<ci_, ch_, co_, true, true>(x, w1, b1, w2, b2, xs, sw, sb, y, B, P, Ci, Co,     \
                                               skip_kind, act, st)                                 \
       : launch_mlp<ci_, ch_, co_, true, false>(x, w1, b1, w2, b2, xs, sw, sb, y, B, P, Ci, Co,    \
                                                skip_kind, act, st))
  switch (mlp_variant(Ci, Ch, Co)) {
    case 0: return FNO_MLP(64, 32, 64);
    case 1: return FNO_MLP(32, 16, 32);
    case 2: return FNO_MLP(128, 64, 128);
    case 3: return FNO_MLP(4, 128, 64);
    case 4: return FNO_MLP(4, 64, 32);
    case 5: return FNO_MLP(64, 128, 16);
    case 6: return FNO_MLP(32, 64, 16);
    default: break;
  }
#undef FNO_MLP
  set_error("channel MLP %d -> %d -> %d is not covered by the kernel", Ci, Ch, Co);
  return FNO_ERR_UNSUPPORTED;
}

// bfloat16 storage of x (x_bf16) or y (y_bf16), with bf16 products: the
// lifting widths (Ci <= 4, y bf16) and the projection widths (Co <= 16, x
// bf16) of the bf16 FNO forward.
bool channel_mlp_io_supported(int Ci, int Ch, int Co, int64_t P, bool x_bf16, bool y_bf16) {
  if (!channel_mlp_supported(Ci, Ch, Co, P)) return false;
  const int v = mlp_variant(Ci, Ch, Co);
  if (x_bf16 && y_bf16) return false;
  if (y_bf16) return v == 3 || v == 4;
  if (x_bf16) return v == 5 || v == 6;
  return true;
}

int channel_mlp_io(const void* x, const float* w1, const float* b1, const float* w2,
                   const float* b2, void* y, int64_t B, int Ci, int Ch, int Co, int64_t P, int act,
                   bool x_bf16, bool y_bf16, hipStream_t st) {
#define FNO_MLPIO(ci_, ch_, co_, io)                                                             \
  launch_mlp<ci_, ch_, co_, true, true, io>(x, w1, b1, w2, b2, nullptr, nullptr, nullptr, y, B, P, \
                                            Ci, Co, FNO_SKIP_NONE, act, st)
  const int v = mlp_variant(Ci, Ch, Co);
  if (y_bf16 && !x_bf16 && v == 3) return FNO_MLPIO(4, 128, 64, 2);
  if (y_bf16 && !x_bf16 && v == 4) return FNO_MLPIO(4, 64, 32, 2);
  if (x_bf16 && !y_bf16 && v == 5) return FNO_MLPIO(64, 128, 16, 1);
  if (x_bf16 && !y_bf16 && v == 6) return FNO_MLPIO(32, 64, 16, 1);
#undef FNO_MLPIO
  set_error("channel MLP %d -> %d -> %d with bfloat16 %s is not covered by the kernel", Ci, Ch, Co,
            x_bf16 ? "input" : "output");
  return FNO_ERR_UNSUPPORTED;
}

// Linear block skip on MFMA: y = act(Ws x + spec); spec may alias y.  The
// slab loads of x and the staged rows of spec and y are 16-byte accesses.
bool skip_gemm_supported(int Ci, int Co, int64_t P, const void* x, const void* spec,
                         const void* y) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(spec) |
                      reinterpret_cast<uintptr_t>(y);
  return P % 4 == 0 && Ci == Co && (Ci == 32 || Ci == 64 || Ci == 128) && a % 16 == 0;
}

int skip_gemm(const float* x, const float* ws, const float* spec, float* y, int64_t B, int Ci,
              int Co, int64_t P, int act, hipStream_t st) {
#define FNO_SKIPG(c)                                                                               \
  launch_mlp<c, c, c, false, false>(x, ws, nullptr, nullptr, nullptr, spec, nullptr, nullptr, y, B, \
                                    P, Ci, Co, FNO_SKIP_IDENTITY, act, st)
  if (Ci == 32) return FNO_SKIPG(32);
  if (Ci == 64) return FNO_SKIPG(64);
  return FNO_SKIPG(128);
#undef FNO_SKIPG
}

}  // namespace fno
