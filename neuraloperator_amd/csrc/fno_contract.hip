// Mode-wise complex contraction on the matrix cores:
//
//   Y[b, o, k] = sum_i X[b, i, k] W[i, o, k]      X [B][Ci][M], W [Ci][Co][M], Y [B][Co][M]
//
// (spectral_convolution.py:21-46, _contract_dense: einsum 'bixy,ioxy->boxy').
// Per mode k this is the real GEMM
//
//   [Yr; Yi] (2Co x B) = A (2Co x 2Ci) * Bm (2Ci x B)
//   A[o][2i]    =  Wr[i][o]     A[o][2i+1]    = -Wi[i][o]
//   A[Co+o][2i] =  Wi[i][o]     A[Co+o][2i+1] =  Wr[i][o]
//   Bm[2i][b]   =  Xr[b][i]     Bm[2i+1][b]   =  Xi[b][i]
//
// Arithmetic: v_mfma_f32_16x16x16_bf16 with three-term bf16 splits, a =
// a_hi + a_lo with a_hi = bf16(a), a_lo = bf16(a - a_hi) (round to nearest
// even each), a b ~ a_hi b_lo + a_lo b_hi + a_hi b_hi with fp32 accumulation:
// each product within 3 * 2^-16 of |a b| (the row epilogue's arithmetic).
// Against fp32 products this takes a fifth of the matrix-core cycles
// (v_mfma_f32_32x32x2f32: 64 cycles per 4,096 flop); the kernel is then
// bound by its loads (fp32 products: 50 us at B32 C64 64x33 modes, bf16
// splits 40 us).
//
// A workgroup owns KB = 16 consecutive modes (a 128-byte run of every X and W
// row in their reference layouts), 32 batch entries and one half of the
// output channels; wave w owns modes k0 + 2w and k0 + 2w + 1, i.e. 8 16x16
// tiles per mode (Yr and Yi rows of its 32 channels x 32 batch entries).
// Input channels stream through LDS in chunks of IC, split and transposed on
// the way in, double-buffered, with the next chunk loaded into registers
// meanwhile.  The two channel halves of a mode block are placed on one XCD,
// next to each other, so the second read of the block's X rows hits that
// XCD's L2.
#include "fno_common.h"

namespace fno {

namespace {
constexpr int MPW = 2;            // modes per wave
constexpr int IC = 8;             // input channels per LDS chunk
constexpr int OH = 32;            // output channels per workgroup
constexpr int WF4 = 4;            // W float4 per thread per chunk (IC*OH*KB/2/THREADS)
constexpr int XF4 = 4;            // X float4 per thread per chunk (IC*32*KB/2/THREADS)
__host__ __device__ constexpr int contract_threads(int kb) { return 64 * kb / MPW; }
}  // namespace

// KB modes per workgroup (KB/2 waves): 16 normally (one workgroup per CU),
// 18 when that keeps the grid within one round, 8 when even 16 leaves most
// CUs idle.  The chunk's operands are split once as they go into LDS, as
// (hi, lo) pairs of bf16x2 words:
//   Wl[i][mode][o] = (Wr, -Wi)    Xl[i][mode][b] = (Xr, Xi)
// (33 pairs per row, one of padding).  One k-step of 16 is the chunk's 8
// input channels: lane (r = l % 16, g = l / 16) holds k = 4 g .. 4 g + 3,
// i.e. channels 2 g and 2 g + 1, so A[o][k] of the Yr rows is one pair from
// each of those channels' rows, and A of the Yi rows (Wi, Wr) is the same
// word with its halves swapped and the low half negated.
namespace cb3 {
typedef short v4s __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
constexpr int RS = 33;            // uint2 per (channel, mode) row: 32 + 1 padding
__host__ __device__ constexpr size_t lds_bytes(int kb) {
  return 2 * (size_t)2 * IC * kb * RS * sizeof(uint2);   // two buffers of W and X
}
// (hi, lo) bf16x2 words of the pair (a, b)
__device__ __forceinline__ uint2 split2(float a, float b) {
  const v2bf h = {(__bf16)a, (__bf16)b};
  const v2bf l = {(__bf16)(a - (float)h[0]), (__bf16)(b - (float)h[1])};
  return make_uint2(__builtin_bit_cast(uint32_t, h), __builtin_bit_cast(uint32_t, l));
}
// (re, -im) -> (im, re): swap the halves, negate the new low half
__device__ __forceinline__ uint32_t rot_conj(uint32_t w) {
  return __builtin_amdgcn_alignbit(w, w, 16) ^ 0x8000u;
}
__device__ __forceinline__ v4s frag(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(v4s, make_uint2(a, b));
}
}  // namespace cb3

template <int KB>
__global__ void __launch_bounds__(contract_threads(KB))
__attribute__((amdgpu_waves_per_eu(2, 4)))
k_contract_mfma(const float2* __restrict__ X, const float2* __restrict__ W, float2* __restrict__ Y,
               int B, int Ci, int Co, int64_t M, int nblocks, int ymap_w) {
  using namespace cb3;
  constexpr int THREADS = contract_threads(KB);
  constexpr int NP = KB / 2;
  static_assert(KB % 2 == 0 && IC * OH * KB / 2 == WF4 * THREADS && IC * 32 * KB / 2 == XF4 * THREADS,
                "tile split");
  static_assert(IC == 8, "one k-step of 16 per chunk");
  extern __shared__ float4 smem4[];
  uint2* lds2 = reinterpret_cast<uint2*>(smem4);
  float* smem = reinterpret_cast<float*>(smem4);
  constexpr int BUF = 2 * IC * KB * RS;   // uint2 per buffer: W rows, then X rows
  auto Wl = [&](int d) __attribute__((always_inline)) { return lds2 + d * BUF; };
  auto Xl = [&](int d) __attribute__((always_inline)) { return lds2 + d * BUF + IC * KB * RS; };
  const int bid = blockIdx.x;
  const int p = (bid % 8) * ((nblocks + 7) / 8) + bid / 16;
  const int half = (bid / 8) % 2;
  if (p >= nblocks) return;
  const int64_t k0 = (int64_t)p * KB;
  const int o0 = half * OH;
  const int b0 = blockIdx.y * 32;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const uint32_t xbytes = (uint32_t)((int64_t)B * Ci * M * 8);
  const uint32_t wbytes = (uint32_t)((int64_t)Ci * Co * M * 8);
  const int Mi = (int)M;

  float4 wr[WF4], xr[XF4];
  constexpr uint32_t kOut = 0x80000000u;
  auto load = [&](int i0) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(W, wbytes), rx = make_rsrc(X, xbytes);
#pragma unroll
    for (int j = 0; j < WF4; ++j) {
      const int q = tid + THREADS * j, part = q % NP, row = q / NP;
      const int o = o0 + row % OH, i = i0 + row / OH;
      const int k = (int)k0 + 2 * part;
      const uint32_t off = (k < Mi && o < Co)
                               ? ((uint32_t)(i * Co + o) * (uint32_t)Mi + (uint32_t)k) * 8u
                               : kOut;
      wr[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rw, (int)off, 0, 0));
    }
#pragma unroll
    for (int j = 0; j < XF4; ++j) {
      const int q = tid + THREADS * j, part = q % NP, row = q / NP;
      const int b = b0 + (row & 31), i = i0 + (row >> 5);
      const int k = (int)k0 + 2 * part;
      const uint32_t off = (k < Mi && b < B)
                               ? ((uint32_t)(b * Ci + i) * (uint32_t)Mi + (uint32_t)k) * 8u
                               : kOut;
      xr[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)off, 0, 0));
    }
  };
  auto stash = [&](int buf) __attribute__((always_inline)) {
    uint2* Ws = Wl(buf);
    uint2* Xs = Xl(buf);
#pragma unroll
    for (int j = 0; j < WF4; ++j) {
      const int q = tid + THREADS * j, part = q % NP, row = q / NP;
      const int o = row % OH, ii = row / OH, m = 2 * part;
      uint2* d = Ws + (ii * KB + m) * RS + o;
      d[0] = split2(wr[j].x, -wr[j].y);
      d[RS] = split2(wr[j].z, -wr[j].w);
    }
#pragma unroll
    for (int j = 0; j < XF4; ++j) {
      const int q = tid + THREADS * j, part = q % NP, row = q / NP;
      const int b = row & 31, ii = row >> 5, m = 2 * part;
      uint2* d = Xs + (ii * KB + m) * RS + b;
      d[0] = split2(xr[j].x, xr[j].y);
      d[RS] = split2(xr[j].z, xr[j].w);
    }
  };

  // acc[mode][row tile: Yr o 0-15, Yr o 16-31, Yi o 0-15, Yi o 16-31][batch tile]
  v4f acc[MPW][4][2];
#pragma unroll
  for (int mm = 0; mm < MPW; ++mm)
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int c = 0; c < 2; ++c) acc[mm][t][c] = v4f{0.f, 0.f, 0.f, 0.f};
  const int r16 = lane & 15, g = lane >> 4;

  load(0);
  stash(0);
  if (IC < Ci) load(IC);
  __syncthreads();
#pragma unroll 1
  for (int i0 = 0, cb = 0; i0 < Ci; i0 += IC, cb ^= 1) {
    if (i0 + IC < Ci) {
      stash(cb ^ 1);
      if (i0 + 2 * IC < Ci) load(i0 + 2 * IC);
    }
    const uint2* Ws = Wl(cb);
    const uint2* Xs = Xl(cb);
#pragma unroll
    for (int mm = 0; mm < MPW; ++mm) {
      const int m = MPW * w + mm;
      const uint2* w0 = Ws + ((2 * g) * KB + m) * RS + r16;
      const uint2* x0 = Xs + ((2 * g) * KB + m) * RS + r16;
      v4s ah[4], al[4], bh[2], bl[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint2 u0 = w0[16 * t], u1 = w0[KB * RS + 16 * t];
        ah[t] = frag(u0.x, u1.x);
        al[t] = frag(u0.y, u1.y);
        ah[2 + t] = frag(rot_conj(u0.x), rot_conj(u1.x));
        al[2 + t] = frag(rot_conj(u0.y), rot_conj(u1.y));
        const uint2 v0 = x0[16 * t], v1 = x0[KB * RS + 16 * t];
        bh[t] = frag(v0.x, v1.x);
        bl[t] = frag(v0.y, v1.y);
      }
      // the small terms first, over all tiles, then the main term
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int c = 0; c < 2; ++c)
          acc[mm][t][c] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ah[t], bl[c], acc[mm][t][c], 0, 0, 0);
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int c = 0; c < 2; ++c)
          acc[mm][t][c] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(al[t], bh[c], acc[mm][t][c], 0, 0, 0);
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int c = 0; c < 2; ++c)
          acc[mm][t][c] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ah[t], bh[c], acc[mm][t][c], 0, 0, 0);
    }
    __syncthreads();
  }
  // D[row][col]: lane l, register r holds row 4 (l / 16) + r, column l % 16.
  // Batch tile hb at a time through LDS into [b][o][mode][re/im], then the
  // rows [b][o][k0 .. k0+KB) as whole runs.
  constexpr int YB = 32 * KB * 2 + 8;
  static_assert(16 * YB * sizeof(float) <= lds_bytes(KB), "transpose tile fits the chunk buffers");
  // unrolled: acc[..][hb] with a run-time hb would put acc in scratch memory
#pragma unroll
  for (int hb = 0; hb < 2; ++hb) {
    __syncthreads();
#pragma unroll
    for (int mm = 0; mm < MPW; ++mm) {
      float* d = smem + r16 * YB + (MPW * w + mm) * 2;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          d[(16 * (t & 1) + 4 * g + r) * KB * 2 + (t >> 1)] = acc[mm][t][hb][r];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 16 * 32 * KB * 2 / 4 / THREADS; ++j) {
      const int q = tid + THREADS * j, part = q % NP, row = q / NP;
      const int bl = row >> 5, o = row & 31;
      const int b = b0 + 16 * hb + bl;
      const int64_t k = k0 + 2 * part;
      const float4 v = *reinterpret_cast<const float4*>(smem + bl * YB + o * KB * 2 + part * 4);
      if (b < B && o0 + o < Co && k < M) {
        float2* yp = Y + ((int64_t)b * Co + o0 + o) * M;
        if (ymap_w) {
          const int m1 = Mi / ymap_w;
          auto map = [&](int kk) {
            const int j = kk / ymap_w, kw = kk - j * ymap_w;
            return kw ? j * (ymap_w - 1) + kw - 1 : m1 * (ymap_w - 1) + j;
          };
          yp[map((int)k)] = make_float2(v.x, v.y);
          yp[map((int)k + 1)] = make_float2(v.z, v.w);
        } else {
          reinterpret_cast<float4*>(yp)[k >> 1] = v;
        }
      }
    }
  }
}

// Host: covers the reference layouts (W [Ci][Co][M]) with Ci a multiple of
// IC, at most two channel halves, an even mode count (16-byte aligned float4
// rows) and operands under 2 GiB.
bool contract_mfma_supported(int B, int Ci, int Co, int64_t M, int64_t sWi, int64_t sWo,
                             int64_t sWk) {
  // 32-bit buffer offsets: both operands under 2 GiB
  return B >= 1 && Ci % IC == 0 && Co >= 1 && Co <= 2 * OH && M % 2 == 0 && sWk == 1 &&
         sWo == M && sWi == (int64_t)Co * M && (int64_t)B * Ci * M * 8 < (int64_t(1) << 31) &&
         (int64_t)Ci * Co * M * 8 < (int64_t(1) << 31);
}

template <int KB>
static int launch_contract(const float2* X, const float2* W, float2* Y, int B, int Ci, int Co,
                           int64_t M, int ymap_w, hipStream_t st) {
  const int nblocks = (int)((M + KB - 1) / KB);
  const int pairs16 = (nblocks + 7) / 8;              // groups of 8 blocks
  dim3 grid((unsigned)(pairs16 * 16), (unsigned)((B + 31) / 32));
  auto kern = k_contract_mfma<KB>;
  const size_t lds = cb3::lds_bytes(KB);
  if (lds > 64 * 1024) {
    int rc = hip_status(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                        "hipFuncSetAttribute(MaxDynamicSharedMemorySize)");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(kern, grid, dim3(contract_threads(KB)), lds, st, X, W, Y, B, Ci, Co, M,
                     nblocks, ymap_w);
  return launch_status("k_contract_mfma");
}

// One workgroup per CU (the double-buffered tile takes 135-152 KB of LDS at
// 16-18 modes); a grid just over the CU count would leave a few CUs a second
// round, so such grids take the smallest wider block that fits one round.
// ymap_w = 0: Y [B][Co][M] in the mode order of X and W.  ymap_w = W' > 0
// (modes = m1 rows of W' bins): each (b, o) plane of Y holds the rows' bins
// 1 .. W'-1 first, row after row (entry j (W'-1) + kw - 1), then the m1 DC
// bins (entry m1 (W'-1) + j), so the AC part of every row starts at a
// multiple of 8 (W'-1) bytes from the plane.
int contract_mfma(const float2* X, const float2* W, float2* Y, int B, int Ci, int Co, int64_t M,
                  hipStream_t st, int ymap_w) {
  const int64_t bt = (B + 31) / 32, cus = 256;
  auto wgs = [&](int kb) { return 2 * ((M + kb - 1) / kb) * bt; };
  if (wgs(16) > cus && wgs(16) <= 2 * cus) {
    if (wgs(18) <= cus) return launch_contract<18>(X, W, Y, B, Ci, Co, M, ymap_w, st);
  }
  // few modes (e.g. 32 x 17): halve the block so twice the CUs take part
  if (2 * wgs(16) <= cus) return launch_contract<8>(X, W, Y, B, Ci, Co, M, ymap_w, st);
  return launch_contract<16>(X, W, Y, B, Ci, Co, M, ymap_w, st);
}

}  // namespace fno
