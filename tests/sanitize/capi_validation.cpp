// Host-side validation of the C-ABI (include/fno_hip.h) under AddressSanitizer
// and UndefinedBehaviorSanitizer, without a GPU: every entry point is called
// with arguments it must reject before touching the HIP runtime (bad ranks,
// sizes, modes, kinds, NULLs, overlapping or misaligned buffers, workspaces
// that are too small, shapes whose byte counts overflow), and the workspace
// queries with valid, invalid and overflowing shapes.  The buffers are host
// arrays standing in for device pointers: a call that got past its checks and
// launched a kernel would fail with a HIP error, which counts as a failure.
// Exit status 0 when every call returned what it must.
#include "fno_hip.h"

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <thread>

static int failures = 0, checks = 0;

static void expect_rc(int rc, int want, const char* what, int line) {
  ++checks;
  const char* msg = fno_last_error();
  const bool msg_ok = want == FNO_OK || (msg && msg[0] != '\0');
  if (rc != want || !msg_ok) {
    std::fprintf(stderr, "FAIL line %d: %s returned %d (want %d), message '%s'\n", line, what, rc,
                 want, msg ? msg : "(null)");
    ++failures;
  }
}
#define EXPECT(call, want) expect_rc((call), (want), #call, __LINE__)

static void expect_true(bool ok, const char* what, int line) {
  ++checks;
  if (!ok) {
    std::fprintf(stderr, "FAIL line %d: %s\n", line, what);
    ++failures;
  }
}
#define CHECK(cond) expect_true((cond), #cond, __LINE__)

alignas(256) static float bufA[4096], bufB[4096], bufC[4096], bufD[4096];

int main() {
  float *x = bufA, *y = bufB, *w = bufC, *ws = bufD;
  void* st = nullptr;
  const size_t big_ws = sizeof(bufD);
  CHECK(fno_version() != nullptr && std::strlen(fno_version()) > 0);

  // ---------------------------------------------------------------- rfft window
  {
    const int32_t s2[2] = {16, 16}, m2[2] = {8, 9}, m2bad[2] = {8, 10}, m2zero[2] = {0, 4};
    const int32_t s0[2] = {0, 16}, sneg[2] = {-4, 16};
    EXPECT(fno_rfft_window_f32(x, y, 1, 0, s2, m2, FNO_NORM_FORWARD, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_rfft_window_f32(x, y, 1, 5, s2, m2, FNO_NORM_FORWARD, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_rfft_window_f32(x, y, 1, 2, nullptr, m2, FNO_NORM_FORWARD, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_rfft_window_f32(x, y, 1, 2, s2, nullptr, FNO_NORM_FORWARD, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_rfft_window_f32(x, y, 1, 2, s2, m2bad, FNO_NORM_FORWARD, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_rfft_window_f32(x, y, 1, 2, s2, m2zero, FNO_NORM_FORWARD, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_rfft_window_f32(x, y, 1, 2, s0, m2, FNO_NORM_FORWARD, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_rfft_window_f32(x, y, 1, 2, sneg, m2, FNO_NORM_FORWARD, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_rfft_window_f32(x, y, 0, 2, s2, m2, FNO_NORM_FORWARD, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_rfft_window_f32(x, y, -3, 2, s2, m2, FNO_NORM_FORWARD, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_rfft_window_f32(nullptr, y, 1, 2, s2, m2, FNO_NORM_FORWARD, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_rfft_window_f32(x, nullptr, 1, 2, s2, m2, FNO_NORM_FORWARD, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_rfft_window_f32(x, y, 1, 2, s2, m2, 7, ws, big_ws, st), FNO_ERR_INVALID);
    const size_t need = fno_rfft_window_workspace_bytes(4, 2, s2, m2);
    CHECK(need > 0);
    EXPECT(fno_rfft_window_f32(x, y, 4, 2, s2, m2, FNO_NORM_FORWARD, ws, need - 1, st),
           FNO_ERR_WORKSPACE);
    CHECK(fno_rfft_window_workspace_bytes(4, 0, s2, m2) == 0);
    CHECK(fno_rfft_window_workspace_bytes(4, 2, nullptr, m2) == 0);
    CHECK(fno_rfft_window_workspace_bytes(4, 2, s2, m2bad) == 0);
    // byte counts beyond size_t: rejected, not wrapped
    const int32_t huge[4] = {1 << 30, 1 << 30, 1 << 30, 1 << 30}, hm[4] = {4, 4, 4, 4};
    CHECK(fno_rfft_window_workspace_bytes(INT64_MAX / 2, 4, huge, hm) == 0);
    const int rc = fno_rfft_window_f32(x, y, INT64_MAX / 2, 4, huge, hm, FNO_NORM_FORWARD, ws, big_ws,
                                       st);
    CHECK(rc == FNO_ERR_INVALID || rc == FNO_ERR_UNSUPPORTED);
  }
  // ------------------------------------------------------------ irfft window
  {
    const int32_t s2[2] = {16, 16}, o2[2] = {32, 24}, m2[2] = {8, 9}, m2bad[2] = {17, 9};
    const int32_t obad[2] = {0, 24};
    EXPECT(fno_irfft_window_f32(y, nullptr, x, 1, 0, 2, s2, o2, m2, 0, 1, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_irfft_window_f32(y, nullptr, x, 0, 3, 2, s2, o2, m2, 0, 1, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_irfft_window_f32(y, nullptr, x, 1, 3, 2, s2, obad, m2, 0, 1, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_irfft_window_f32(y, nullptr, x, 1, 3, 2, s2, o2, m2bad, 0, 1, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_irfft_window_f32(y, nullptr, x, 1, 3, 2, nullptr, o2, m2, 0, 1, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_irfft_window_f32(y, nullptr, x, 1, 3, 2, s2, nullptr, m2, 0, 1, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_irfft_window_f32(nullptr, nullptr, x, 1, 3, 2, s2, o2, m2, 0, 1, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_irfft_window_f32(y, nullptr, nullptr, 1, 3, 2, s2, o2, m2, 0, 1, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_irfft_window_f32(y, nullptr, x, 1, 3, 2, s2, o2, m2, -1, 1, ws, big_ws, st), FNO_ERR_INVALID);
    const size_t need = fno_irfft_window_workspace_bytes(3, 2, o2, m2);
    CHECK(need > 0);
    EXPECT(fno_irfft_window_f32(y, nullptr, x, 1, 3, 2, s2, o2, m2, 0, 1, ws, need - 1, st),
           FNO_ERR_WORKSPACE);
    CHECK(fno_irfft_window_workspace_bytes(3, 2, obad, m2) == 0);
  }
  // ------------------------------------------------ complex-data window pair
  {
    const int32_t s2[2] = {16, 12}, m2[2] = {8, 12}, m2bad[2] = {8, 13};
    EXPECT(fno_fft_window_c64(x, y, 1, 2, s2, m2bad, 0, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_fft_window_c64(x, y, 1, 5, s2, m2, 0, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_fft_window_c64(nullptr, y, 1, 2, s2, m2, 0, ws, big_ws, st), FNO_ERR_INVALID);
    const size_t need = fno_fft_window_workspace_bytes(2, 2, s2, m2);
    CHECK(need > 0);
    EXPECT(fno_fft_window_c64(x, y, 2, 2, s2, m2, 0, ws, need - 1, st), FNO_ERR_WORKSPACE);
    EXPECT(fno_ifft_window_c64(y, nullptr, x, 1, 2, 2, s2, s2, m2bad, 0, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_ifft_window_c64(y, nullptr, x, 1, -2, 2, s2, s2, m2, 0, ws, big_ws, st), FNO_ERR_INVALID);
    const size_t ineed = fno_ifft_window_workspace_bytes(2, 2, s2, m2);
    CHECK(ineed > 0);
    EXPECT(fno_ifft_window_c64(y, nullptr, x, 1, 2, 2, s2, s2, m2, 0, ws, ineed - 1, st),
           FNO_ERR_WORKSPACE);
  }
  // ------------------------------------------------------------ contractions
  {
    EXPECT(fno_contract_dense_c64(x, w, y, 0, 3, 4, 10, 0, st), FNO_ERR_INVALID);
    EXPECT(fno_contract_dense_c64(x, w, y, 2, 0, 4, 10, 0, st), FNO_ERR_INVALID);
    EXPECT(fno_contract_dense_c64(x, w, y, 2, 3, 4, 0, 0, st), FNO_ERR_INVALID);
    EXPECT(fno_contract_dense_c64(x, w, y, 2, 3, 4, 10, 1, st), FNO_ERR_INVALID);   // separable Ci != Co
    EXPECT(fno_contract_dense_c64(nullptr, w, y, 2, 3, 4, 10, 0, st), FNO_ERR_INVALID);
    EXPECT(fno_contract_dense_c64(x, nullptr, y, 2, 3, 4, 10, 0, st), FNO_ERR_INVALID);
    EXPECT(fno_contract_dense_c64(x, w, nullptr, 2, 3, 4, 10, 0, st), FNO_ERR_INVALID);
    const int32_t m3[3] = {4, 4, 3}, r5[5] = {2, 2, 2, 2, 2}, r5bad[5] = {2, 0, 2, 2, 2};
    const void* fac[5] = {w, w, w, w, w};
    const void* facnull[5] = {w, nullptr, w, w, w};
    const size_t need = fno_contract_tucker_workspace_bytes(2, 3, m3, r5);
    CHECK(need > 0);
    CHECK(fno_contract_tucker_workspace_bytes(2, 0, m3, r5) == 0);
    CHECK(fno_contract_tucker_workspace_bytes(2, 3, nullptr, r5) == 0);
    EXPECT(fno_contract_tucker_c64(x, w, fac, r5bad, y, 2, 3, 4, 3, m3, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_contract_tucker_c64(x, w, facnull, r5, y, 2, 3, 4, 3, m3, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_contract_tucker_c64(x, w, nullptr, r5, y, 2, 3, 4, 3, m3, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_contract_tucker_c64(x, w, fac, nullptr, y, 2, 3, 4, 3, m3, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_contract_tucker_c64(x, w, fac, r5, y, 2, 3, 4, 5, m3, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_contract_tucker_c64(x, w, fac, r5, y, 2, 3, 4, 3, m3, ws, need - 1, st), FNO_ERR_WORKSPACE);
  }
  // ---------------------------------------------------------- block epilogue
  {
    EXPECT(fno_block_epilogue_f32(y, x, w, y, 2, 3, 4, 64, 9, FNO_ACT_GELU, st), FNO_ERR_INVALID);
    EXPECT(fno_block_epilogue_f32(y, x, w, y, 2, 3, 4, 64, FNO_SKIP_LINEAR, 5, st), FNO_ERR_INVALID);
    EXPECT(fno_block_epilogue_f32(y, x, w, y, 2, 3, 4, 64, FNO_SKIP_SOFT_GATING, 0, st), FNO_ERR_INVALID);
    EXPECT(fno_block_epilogue_f32(y, x, nullptr, y, 2, 3, 4, 64, FNO_SKIP_IDENTITY, 0, st), FNO_ERR_INVALID);
    EXPECT(fno_block_epilogue_f32(y, x, nullptr, y, 2, 4, 4, 64, FNO_SKIP_LINEAR, 0, st), FNO_ERR_INVALID);
    EXPECT(fno_block_epilogue_f32(y, nullptr, w, y, 2, 4, 4, 64, FNO_SKIP_LINEAR, 0, st), FNO_ERR_INVALID);
    EXPECT(fno_block_epilogue_f32(y, x, w, y, 2, 4, 4, 0, FNO_SKIP_LINEAR, 0, st), FNO_ERR_INVALID);
  }
  // ------------------------------------------------------------- channel MLP
  {
    CHECK(fno_channel_mlp_is_supported(64, 32, 64, 1024) == 1);
    CHECK(fno_channel_mlp_is_supported(64, 32, 64, 1022) == 0);   // points % 4
    CHECK(fno_channel_mlp_is_supported(48, 32, 64, 1024) == 0);
    CHECK(fno_channel_mlp_is_supported(-1, 32, 64, 1024) == 0);
    EXPECT(fno_channel_mlp_f32(x, w, nullptr, w, nullptr, nullptr, nullptr, nullptr, y, 1, 48, 32, 64, 1024,
                               FNO_SKIP_NONE, 0, 0, st), FNO_ERR_UNSUPPORTED);
    EXPECT(fno_channel_mlp_f32(x, w, nullptr, w, nullptr, nullptr, nullptr, nullptr, y, 1, 64, 32, 64, 1024,
                               7, 0, 0, st), FNO_ERR_INVALID);
    EXPECT(fno_channel_mlp_f32(x, w, nullptr, w, nullptr, nullptr, nullptr, nullptr, y, 1, 64, 32, 64, 1024,
                               FNO_SKIP_SOFT_GATING, 0, 0, st), FNO_ERR_INVALID);   // no skip_x
    EXPECT(fno_channel_mlp_f32(x, w, nullptr, w, nullptr, nullptr, nullptr, nullptr, x + 4, 1, 64, 32, 64, 8,
                               FNO_SKIP_NONE, 0, 0, st), FNO_ERR_INVALID);          // y overlaps x, shifted
    EXPECT(fno_channel_mlp_f32(x + 1, w, nullptr, w, nullptr, nullptr, nullptr, nullptr, y, 1, 64, 32, 64, 8,
                               FNO_SKIP_NONE, 0, 0, st), FNO_ERR_UNSUPPORTED);      // misaligned x
    EXPECT(fno_channel_mlp_f32(nullptr, w, nullptr, w, nullptr, nullptr, nullptr, nullptr, y, 1, 64, 32, 64,
                               8, FNO_SKIP_NONE, 0, 0, st), FNO_ERR_INVALID);
    EXPECT(fno_channel_mlp_f32(x, w, nullptr, w, nullptr, nullptr, nullptr, nullptr, y, 0, 64, 32, 64, 8,
                               FNO_SKIP_NONE, 0, 0, st), FNO_ERR_INVALID);
  }
  // ---------------------------------------------------------- spectral block
  {
    // shapes of hundreds of MB: far-apart stand-in addresses, never dereferenced
    float* const x = reinterpret_cast<float*>((uintptr_t)1 << 44);
    float* const y = reinterpret_cast<float*>((uintptr_t)2 << 44);
    const int32_t s2[2] = {256, 256}, m2[2] = {64, 33}, m2bad[2] = {64, 130};
    const int32_t s1[1] = {1024}, m1[1] = {16};
    CHECK(fno_spectral_block_is_fused(32, 64, 64, 2, s2, m2, FNO_SKIP_LINEAR) == 1);
    CHECK(fno_spectral_block_is_fused(32, 64, 64, 1, s1, m1, FNO_SKIP_LINEAR) == 0);
    CHECK(fno_spectral_block_is_fused(32, 64, 64, 2, s2, m2bad, FNO_SKIP_LINEAR) == 0);
    const size_t need = fno_spectral_block_workspace_bytes(32, 64, 64, 2, s2, m2);
    CHECK(need == (size_t)32 * 64 * 64 * 33 * 2 * 8);
    CHECK(fno_spectral_block_workspace_bytes(32, 64, 64, 2, s2, m2bad) == 0);
    CHECK(fno_spectral_block_workspace_bytes(0, 64, 64, 2, s2, m2) == 0);
    EXPECT(fno_spectral_block_f32(x, w, nullptr, w, y, 32, 64, 64, 2, s2, m2, 0, FNO_SKIP_LINEAR,
                                  FNO_ACT_GELU, ws, need - 1, st), FNO_ERR_WORKSPACE);
    EXPECT(fno_spectral_block_f32(x, w, nullptr, w, y, 32, 64, 64, 2, s2, m2bad, 0, FNO_SKIP_LINEAR,
                                  FNO_ACT_GELU, ws, big_ws, st), FNO_ERR_INVALID);
    EXPECT(fno_spectral_block_f32(x, w, nullptr, nullptr, y, 32, 64, 64, 2, s2, m2, 0, FNO_SKIP_LINEAR,
                                  FNO_ACT_GELU, ws, need, st), FNO_ERR_INVALID);     // no skip weight
    EXPECT(fno_spectral_block_f32(x, w, nullptr, nullptr, y, 32, 64, 32, 2, s2, m2, 0,
                                  FNO_SKIP_IDENTITY, FNO_ACT_GELU, ws, need, st), FNO_ERR_INVALID);
    EXPECT(fno_spectral_block_f32(x, w, nullptr, w, y, 32, 64, 64, 2, s2, m2, 0, FNO_SKIP_LINEAR, 3, ws,
                                  need, st), FNO_ERR_INVALID);
    EXPECT(fno_spectral_block_f32(x, w, nullptr, w, x, 32, 64, 64, 2, s2, m2, 0, FNO_SKIP_LINEAR,
                                  FNO_ACT_GELU, ws, need, st), FNO_ERR_INVALID);     // y aliases x
    EXPECT(fno_spectral_block_f32(nullptr, w, nullptr, w, y, 32, 64, 64, 2, s2, m2, 0, FNO_SKIP_LINEAR,
                                  FNO_ACT_GELU, ws, need, st), FNO_ERR_INVALID);
    // no-allocation variant: rejected before any HIP call
    EXPECT(fno_spectral_block_f32_noalloc(x, w, nullptr, w, y, 32, 64, 64, 2, s2, m2bad, 0,
                                          FNO_SKIP_LINEAR, FNO_ACT_GELU, st), FNO_ERR_INVALID);
    const int32_t s3[3] = {512, 512, 512}, m3[3] = {64, 64, 64};
    EXPECT(fno_spectral_block_f32_noalloc(x, w, nullptr, nullptr, y, 1, 64, 64, 3, s3, m3, 0,
                                          FNO_SKIP_NONE, FNO_ACT_NONE, st), FNO_ERR_UNSUPPORTED);
  }
  // ------------------------------------------- one-pass FNO layer (fp32 / bf16)
  {
    float* const x = reinterpret_cast<float*>((uintptr_t)1 << 44);
    float* const y = reinterpret_cast<float*>((uintptr_t)2 << 44);
    const int32_t s2[2] = {256, 256}, m2[2] = {64, 33}, s48[2] = {48, 256}, m48[2] = {20, 12};
    CHECK(fno_layer_is_fused(2, 64, 32, 2, s2, m2, FNO_SKIP_LINEAR, FNO_SKIP_SOFT_GATING) == 1);
    CHECK(fno_layer_bf16_is_fused(2, 64, 32, 2, s2, m2, FNO_SKIP_LINEAR, FNO_SKIP_SOFT_GATING) == 1);
    CHECK(fno_layer_is_fused(2, 64, 32, 2, s48, m48, FNO_SKIP_LINEAR, FNO_SKIP_IDENTITY) == 1);
    CHECK(fno_layer_bf16_is_fused(2, 64, 32, 2, s48, m48, FNO_SKIP_LINEAR, FNO_SKIP_IDENTITY) == 0);
    CHECK(fno_layer_is_fused(2, 64, 48, 2, s2, m2, FNO_SKIP_LINEAR, FNO_SKIP_SOFT_GATING) == 0);
    CHECK(fno_layer_is_fused(2, 64, 32, 2, s2, m2, FNO_SKIP_NONE, FNO_SKIP_SOFT_GATING) == 0);
    CHECK(fno_layer_is_fused(2, 64, 32, 2, s2, m2, FNO_SKIP_LINEAR, 7) == 0);
    const size_t need = fno_spectral_block_workspace_bytes(2, 64, 64, 2, s2, m2);
    EXPECT(fno_layer_f32(x, w, nullptr, w, w, nullptr, w, nullptr, w, nullptr, y, 2, 64, 32, 2, s2,
                         m2, 0, FNO_SKIP_LINEAR, FNO_SKIP_SOFT_GATING, FNO_ACT_GELU, ws, need - 1, st),
           FNO_ERR_WORKSPACE);
    EXPECT(fno_layer_bf16(x, w, nullptr, w, w, nullptr, w, nullptr, w, nullptr, y, 2, 64, 32, 2, s2,
                          m2, 0, FNO_SKIP_LINEAR, FNO_SKIP_SOFT_GATING, FNO_ACT_GELU, ws, need - 1,
                          st), FNO_ERR_WORKSPACE);
    EXPECT(fno_layer_f32(x, w, nullptr, w, nullptr, nullptr, w, nullptr, w, nullptr, y, 2, 64, 32, 2,
                         s2, m2, 0, FNO_SKIP_LINEAR, FNO_SKIP_SOFT_GATING, FNO_ACT_GELU, ws, need,
                         st), FNO_ERR_INVALID);                                  // no W1
    EXPECT(fno_layer_f32(x, w, nullptr, w, w, nullptr, w, nullptr, nullptr, nullptr, y, 2, 64, 32, 2,
                         s2, m2, 0, FNO_SKIP_LINEAR, FNO_SKIP_SOFT_GATING, FNO_ACT_GELU, ws, need,
                         st), FNO_ERR_INVALID);                                  // no gate weight
    EXPECT(fno_layer_f32(x, w, nullptr, w, w, nullptr, w, nullptr, w, nullptr, y, 2, 64, 48, 2, s2,
                         m2, 0, FNO_SKIP_LINEAR, FNO_SKIP_SOFT_GATING, FNO_ACT_GELU, ws, need, st),
           FNO_ERR_UNSUPPORTED);                                                 // 48 hidden
    EXPECT(fno_layer_bf16(x, w, nullptr, w, w, nullptr, w, nullptr, w, nullptr, y, 2, 64, 32, 2, s48,
                          m48, 0, FNO_SKIP_LINEAR, FNO_SKIP_IDENTITY, FNO_ACT_GELU, ws, big_ws, st),
           FNO_ERR_UNSUPPORTED);                                                 // 48-row planes
    // bf16 x and y: 2 bytes per element, so y one fp32 plane-half past x overlaps
    EXPECT(fno_layer_bf16(x, w, nullptr, w, w, nullptr, w, nullptr, w, nullptr,
                          reinterpret_cast<char*>(x) + 2 * 64 * 256 * 256, 2, 64, 32, 2, s2, m2, 0,
                          FNO_SKIP_LINEAR, FNO_SKIP_SOFT_GATING, FNO_ACT_GELU, ws, need, st),
           FNO_ERR_INVALID);
  }
  // ----------------------------- lifting / projection with bf16 storage
  {
    CHECK(fno_channel_mlp_io_is_supported(3, 128, 64, 1024, 0, 1) == 1);
    CHECK(fno_channel_mlp_io_is_supported(64, 128, 1, 1024, 1, 0) == 1);
    CHECK(fno_channel_mlp_io_is_supported(3, 128, 64, 1024, 1, 0) == 0);
    CHECK(fno_channel_mlp_io_is_supported(64, 128, 1, 1024, 0, 1) == 0);
    CHECK(fno_channel_mlp_io_is_supported(64, 32, 64, 1024, 1, 1) == 0);
    CHECK(fno_channel_mlp_io_is_supported(64, 32, 64, 1022, 0, 0) == 0);
    EXPECT(fno_channel_mlp_io(x, w, nullptr, w, nullptr, y, 1, 64, 128, 1, 1024, 0, 0, 1, st),
           FNO_ERR_UNSUPPORTED);
    EXPECT(fno_channel_mlp_io(x, w, nullptr, w, nullptr, y, 1, 3, 128, 64, 1024, 0, 2, 0, st),
           FNO_ERR_INVALID);
    EXPECT(fno_channel_mlp_io(x, w, nullptr, w, nullptr, y, 1, 3, 128, 64, 1024, 5, 0, 1, st),
           FNO_ERR_INVALID);
    EXPECT(fno_channel_mlp_io(x + 1, w, nullptr, w, nullptr, y, 1, 3, 128, 64, 8, 0, 0, 1, st),
           FNO_ERR_UNSUPPORTED);                                                 // misaligned
    EXPECT(fno_channel_mlp_io(x, w, nullptr, w, nullptr, x + 4, 1, 3, 128, 64, 8, 0, 0, 1, st),
           FNO_ERR_INVALID);                                                     // overlap
    EXPECT(fno_channel_mlp_io(nullptr, w, nullptr, w, nullptr, y, 1, 3, 128, 64, 8, 0, 0, 1, st),
           FNO_ERR_INVALID);
  }
  // ------------------------------------------------ inverse + epilogue
  {
    float* const x = reinterpret_cast<float*>((uintptr_t)1 << 44);
    float* const y = reinterpret_cast<float*>((uintptr_t)2 << 44);
    const int32_t s3[3] = {16, 16, 64}, m3[3] = {8, 8, 9}, m3bad[3] = {8, 8, 40};
    const size_t need = fno_irfft_window_workspace_bytes(2 * 32, 3, s3, m3);
    EXPECT(fno_irfft_window_epilogue_f32(x, nullptr, x, w, y, 2, 32, 32, 3, s3, m3bad, 0,
                                         FNO_SKIP_LINEAR, FNO_ACT_GELU, ws, big_ws, st),
           FNO_ERR_INVALID);
    EXPECT(fno_irfft_window_epilogue_f32(x, nullptr, x, nullptr, y, 2, 32, 32, 3, s3, m3, 0,
                                         FNO_SKIP_LINEAR, FNO_ACT_GELU, ws, big_ws, st),
           FNO_ERR_INVALID);                                                     // no skip weight
    EXPECT(fno_irfft_window_epilogue_f32(x, nullptr, x, w, y, 2, 32, 32, 3, s3, m3, 0, 9,
                                         FNO_ACT_GELU, ws, big_ws, st), FNO_ERR_INVALID);
    if (need > 0)
      EXPECT(fno_irfft_window_epilogue_f32(x, nullptr, x, w, y, 2, 32, 32, 3, s3, m3, 0,
                                           FNO_SKIP_LINEAR, FNO_ACT_GELU, ws, need - 1, st),
             FNO_ERR_WORKSPACE);
  }
  // ------------------------------------ the error message is per host thread
  {
    EXPECT(fno_contract_dense_c64(x, w, y, 0, 3, 4, 10, 0, st), FNO_ERR_INVALID);
    char other[512] = {0};
    std::thread t([&] { std::snprintf(other, sizeof other, "%s", fno_last_error()); });
    t.join();
    CHECK(other[0] == '\0');
    CHECK(fno_last_error()[0] != '\0');
  }
  std::printf("%d checks, %d failures\n", checks, failures);
  return failures == 0 ? 0 : 1;
}
