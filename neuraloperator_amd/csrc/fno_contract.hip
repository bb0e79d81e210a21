// Mode-wise complex contraction on fp32 MFMA (v_mfma_f32_32x32x2f32):
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
// A workgroup owns KB = 16 consecutive modes (a 128-byte run of every X and W
// row in their reference layouts), 32 batch entries and one half of the
// output channels; wave w owns modes k0 + 2w and k0 + 2w + 1, i.e. four 32x32
// tiles (the Yr and Yi rows of its 32 channels for both modes).  Eight waves
// and <= 128 VGPRs per workgroup let two workgroups share a CU, so the 2 x 132
// workgroups of a 64x33-mode layer run in one wave of the grid.  Input channels stream through LDS in chunks
// of IC, transposed on the way in so each MFMA operand read is a run of
// consecutive words, with the next chunk loaded into registers meanwhile.
// The two channel halves of a mode block are placed on one XCD, next to each
// other, so the second read of the block's X rows hits that XCD's L2.
#include "fno_common.h"

namespace fno {

typedef float v16f_c __attribute__((ext_vector_type(16)));

namespace {
constexpr int MPW = 2;            // modes per wave
constexpr int IC = 8;             // input channels per LDS chunk
constexpr int OH = 32;            // output channels per workgroup
constexpr int PS = OH;            // plane stride of a W tile row (re, im planes)
constexpr int MS = 2 * PS + 4;    // (i, mode) block stride of the W tile
constexpr int XM = 64 + 4;        // (i, mode) block stride of the X tile: [c][b]
constexpr int WF4 = 4;            // W float4 per thread per chunk (IC*OH*KB/2/THREADS)
constexpr int XF4 = 4;            // X float4 per thread per chunk (IC*32*KB/2/THREADS)
__host__ __device__ constexpr int contract_threads(int kb) { return 64 * kb / MPW; }
__host__ __device__ constexpr size_t contract_lds(int kb) {
  return 2 * (size_t)IC * kb * (MS + XM) * sizeof(float);   // two chunk buffers
}
}  // namespace

// KB modes per workgroup (KB/2 waves): 16 normally (one workgroup per CU), 18
// when that keeps the grid within one round, 8 when even 16 leaves most CUs
// idle.
template <int KB>
__global__ void __launch_bounds__(contract_threads(KB))
__attribute__((amdgpu_waves_per_eu(2, 4)))
k_contract_mfma(const float2* __restrict__ X, const float2* __restrict__ W, float2* __restrict__ Y,
                int B, int Ci, int Co, int64_t M, int nblocks, int ymap_w) {
  constexpr int THREADS = contract_threads(KB);
  constexpr int NP = KB / 2;          // float4 (mode pairs) per operand row
  static_assert(KB % 2 == 0 && IC * OH * KB / 2 == WF4 * THREADS && IC * 32 * KB / 2 == XF4 * THREADS,
                "tile split");
  extern __shared__ float4 smem4[];
  float* smem = reinterpret_cast<float*>(smem4);
  // two chunk buffers, each W chunk [i][mode][re/im plane][o] then
  // X chunk [i][mode][re/im][b]
  constexpr int BUF = IC * KB * (MS + XM);
  auto Wbuf = [&](int d) __attribute__((always_inline)) { return smem + d * BUF; };
  auto Xbuf = [&](int d) __attribute__((always_inline)) { return smem + d * BUF + IC * KB * MS; };
  // pair (mode block, channel half) placement: the halves of block p run on
  // one XCD (workgroup id mod 8), 8 ids apart, and each XCD takes a
  // contiguous range of mode blocks, so the 128-byte lines that two adjacent
  // blocks' mode runs share are fetched into one L2
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

  // float4 q of a chunk: part = q % NP (modes 2*part, 2*part+1), row = q / NP.
  // W rows: o = row % OH fastest, then the chunk's input channel.
  // X rows: b = row % 32 fastest, then the chunk's input channel.
  float4 wr[WF4], xr[XF4];
  // Entries outside the operands (mode >= M, channel >= Co, batch >= B) get
  // an offset past the buffer end, which the buffer load returns as zero: no
  // select on the loaded value, so every load of a chunk stays in flight.
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
    float* Ws = Wbuf(buf);
    float* Xs = Xbuf(buf);
#pragma unroll
    for (int j = 0; j < WF4; ++j) {
      const int q = tid + THREADS * j, part = q % NP, row = q / NP;
      const int o = row % OH, ii = row / OH, m = 2 * part;
      float* d = Ws + (ii * KB + m) * MS + o;
      d[0] = wr[j].x;
      d[PS] = wr[j].y;
      d[MS] = wr[j].z;
      d[MS + PS] = wr[j].w;
    }
#pragma unroll
    for (int j = 0; j < XF4; ++j) {
      const int q = tid + THREADS * j, part = q % NP, row = q / NP;
      const int b = row & 31, ii = row >> 5, m = 2 * part;
      float* d = Xs + (ii * KB + m) * XM + b;
      d[0] = xr[j].x;
      d[32] = xr[j].y;
      d[XM] = xr[j].z;
      d[XM + 32] = xr[j].w;
    }
  };

  v16f_c acc[MPW][2];
#pragma unroll
  for (int mm = 0; mm < MPW; ++mm)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mm][t][r] = 0.f;
  const int c = lane >> 5, oo = lane & 31;
  const float sgn = c ? -1.f : 1.f;   // A[o][2i+1] = -Wi

  // Double-buffered chunks: chunk n+1 is transposed into the other buffer
  // while the MFMAs of chunk n run, and chunk n+2 is in flight meanwhile, so
  // one barrier per chunk separates the phases.
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
    const float* Ws = Wbuf(cb);
    const float* Xs = Xbuf(cb);
    // operands of input channel s + 1 are read while the MFMAs of s run
    float bv[2][MPW], ar[2][MPW], ai[2][MPW];
    auto operands = [&](int s, int d) __attribute__((always_inline)) {
#pragma unroll
      for (int mm = 0; mm < MPW; ++mm) {
        const int m = MPW * w + mm;
        bv[d][mm] = Xs[(s * KB + m) * XM + c * 32 + oo];
        const float* wrow = Ws + (s * KB + m) * MS + oo;
        ar[d][mm] = wrow[c * PS];         // Yr rows: Wr (c=0), Wi (c=1, negated below)
        ai[d][mm] = wrow[(1 - c) * PS];   // Yi rows: Wi (c=0), Wr (c=1)
      }
    };
    operands(0, 0);
#pragma unroll
    for (int s = 0; s < IC; ++s) {
      if (s + 1 < IC) operands(s + 1, (s + 1) & 1);
      __builtin_amdgcn_sched_barrier(0);   // keep the reads ahead of the MFMAs
#pragma unroll
      for (int mm = 0; mm < MPW; ++mm) {
        acc[mm][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(sgn * ar[s & 1][mm], bv[s & 1][mm],
                                                          acc[mm][0], 0, 0, 0);
        acc[mm][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(ai[s & 1][mm], bv[s & 1][mm],
                                                          acc[mm][1], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();   // chunk n+1 is in place; chunk n's buffer is free
  }
  // D[m][n]: lane l, register r holds row 8(r/4) + 4(l/32) + r%4 (channel),
  // column l%32 (batch entry).  Y rows [b][o][k0 .. k0+KB) are 8*KB-byte runs:
  // transpose through LDS, 16 batch entries at a time, and store whole runs.
  constexpr int YB = 32 * KB * 2 + 8;   // LDS stride of one batch entry: [o][mode][re/im]
  static_assert(16 * YB <= 2 * IC * KB * (MS + XM), "transpose tile fits the chunk buffers");
#pragma unroll 1
  for (int hb = 0; hb < 2; ++hb) {
    __syncthreads();
    if ((oo >> 4) == hb) {
#pragma unroll
      for (int mm = 0; mm < MPW; ++mm) {
        float* d = smem + (oo & 15) * YB + (MPW * w + mm) * 2;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            d[(8 * (r >> 2) + 4 * c + (r & 3)) * KB * 2 + t] = acc[mm][t][r];
      }
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
          // rows of AC bins first, the DC column after them (see contract_mfma)
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
  const size_t lds = contract_lds(KB);
  if (lds > 64 * 1024) {
    int rc = hip_status(hipFuncSetAttribute(reinterpret_cast<const void*>(k_contract_mfma<KB>),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                        "hipFuncSetAttribute(MaxDynamicSharedMemorySize)");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(k_contract_mfma<KB>, grid, dim3(contract_threads(KB)), lds, st, X, W, Y, B,
                     Ci, Co, M, nblocks, ymap_w);
  return launch_status("k_contract_mfma");
}

// One workgroup per CU (the double-buffered tile takes 136-157 KB of LDS at
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
