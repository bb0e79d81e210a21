// extern "C" entry points of libfnohip.so: host-side validation, workspace
// accounting and dispatch to the generic and fused kernels.  Declarations and
// the reference interfaces each entry point replaces are in include/fno_hip.h.
#include "fno_common.h"

namespace fno {
const char* last_error_cstr();
void clear_error();
int validate_window(int32_t ndim, const int32_t* sizes, const int32_t* modes);
size_t rfft_window_ws(int64_t planes, int32_t ndim, const int32_t* sizes, const int32_t* modes);
size_t irfft_window_ws(int64_t planes, int32_t ndim, const int32_t* out_sizes,
                       const int32_t* modes);
int fft_window_c2c(const float2* x, float2* xhat, int64_t planes, int32_t ndim,
                   const int32_t* sizes, const int32_t* modes, int32_t norm, void* ws,
                   size_t ws_bytes, hipStream_t st);
size_t fft_window_c2c_ws(int64_t planes, int32_t ndim, const int32_t* sizes, const int32_t* modes);
int ifft_window_c2c(const float2* yhat, const float* bias, float2* y, int64_t batch,
                    int32_t channels, int32_t ndim, const int32_t* in_sizes,
                    const int32_t* out_sizes, const int32_t* modes, int32_t norm, void* ws,
                    size_t ws_bytes, hipStream_t st);
size_t ifft_window_c2c_ws(int64_t planes, int32_t ndim, const int32_t* out_sizes,
                          const int32_t* modes);
int rfft_window(const float* x, float2* xhat, int64_t planes, int32_t ndim, const int32_t* sizes,
                const int32_t* modes, int32_t norm, void* ws, size_t ws_bytes, hipStream_t st);
int irfft_window(const float2* yhat, const float* bias, float* y, int64_t batch, int32_t channels,
                 int32_t ndim, const int32_t* in_sizes, const int32_t* out_sizes,
                 const int32_t* modes, int32_t norm, int32_t enforce, void* ws, size_t ws_bytes,
                 hipStream_t st);
int contract_dense(const float2* X, const float2* W, float2* Y, int B, int Ci, int Co, int64_t M,
                   int64_t sWi, int64_t sWo, int64_t sWk, hipStream_t st, int ymap_w = 0);
int contract_separable(const float2* X, const float2* W, float2* Y, int B, int C, int64_t M,
                       hipStream_t st);
int axis_matmul(const float2* in, const float2* mat, float2* out, int64_t outer, int A, int J,
                int64_t inner, hipStream_t st);
int irfft_epilogue(const float2* yhat, const float* bias, const float* x, const float* skip_w,
                   float* y, int B, int Ci, int Co, int32_t ndim, const int32_t* sizes,
                   const int32_t* modes, int32_t norm, int32_t skip_kind, int32_t act, void* ws,
                   size_t ws_bytes, hipStream_t st);
int block_epilogue(const float* spec, const float* x, const float* ws, float* y, int B, int Ci,
                   int Co, int64_t P, int skip_kind, int act, hipStream_t st);
bool channel_mlp_supported(int Ci, int Ch, int Co, int64_t P);
int channel_mlp(const float* x, const float* w1, const float* b1, const float* w2, const float* b2,
                const float* xs, const float* sw, const float* sb, float* y, int64_t B, int Ci,
                int Ch, int Co, int64_t P, int skip_kind, int act, bool bf16_products,
                hipStream_t st);
bool channel_mlp_io_supported(int Ci, int Ch, int Co, int64_t P, bool x_bf16, bool y_bf16);
int channel_mlp_io(const void* x, const float* w1, const float* b1, const float* w2,
                   const float* b2, void* y, int64_t B, int Ci, int Ch, int Co, int64_t P, int act,
                   bool x_bf16, bool y_bf16, hipStream_t st);
bool fast2d_supported(int B, int Ci, int Co, int ndim, const int32_t* sizes, const int32_t* modes,
                      int skip_kind);
bool fast2d_bf16_supported(const int32_t* sizes, const int32_t* modes);
size_t fast2d_workspace(int B, int Ci, int Co, const int32_t* sizes, const int32_t* modes);
bool rowsynth_covers(int H, int W, int Ci, int Co, int m1, int m2h);
bool fast1d_supported(int Ci, int Co, int N, int m);
bool line1d_supported(int Ci, int Co, int N, int m, int skip_kind);
int line1d_block(const float* x, const float2* w, const float* bias, const float* skip_w, float* y,
                 int B, int Ci, int Co, int N, int m, int norm, int skip_kind, int act, void* ws,
                 size_t ws_bytes, hipStream_t st);
int fast1d_block(const float* x, const float2* w, const float* bias, const float* skip_w, float* y,
                 int B, int Ci, int Co, int N, int m, int norm, int skip_kind, int act,
                 hipStream_t st);
int fast2d_block(const void* x, const float2* w, const float* bias, const float* skip_w, void* y,
                 int B, int Ci, int Co, const int32_t* sizes, const int32_t* modes, int norm,
                 int skip_kind, int act, void* ws, size_t ws_bytes, hipStream_t st,
                 const LayerMlp* mlp = nullptr, bool bf = false);
bool rowsynth_mlp_covers(int H, int W, int Ci, int Co, int m1, int m2h, int hidden,
                         int skip_kind);
bool tucker_fused_supported(int B, int Ci, int Co, int ndim, const int32_t* modes,
                            const int32_t* ranks);
int tucker_fused(const float2* X, const float2* core, const float2* const* factors,
                 const int32_t* ranks, float2* Y, int B, int Ci, int Co, int ndim,
                 const int32_t* modes, float2* Kbuf, hipStream_t st);
}  // namespace fno

using namespace fno;

static int64_t mode_count(int32_t ndim, const int32_t* modes) {
  int64_t m = 1;
  for (int d = 0; d < ndim; ++d) m *= modes[d];
  return m;
}

static bool ranges_overlap(const void* a, size_t na, const void* b, size_t nb) {
  const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
  return pa < pb + nb && pb < pa + na;
}

static int check_norm(int32_t norm) {
  FNO_CHECK_ARG(norm == FNO_NORM_BACKWARD || norm == FNO_NORM_FORWARD || norm == FNO_NORM_ORTHO,
                "norm must be FNO_NORM_BACKWARD/FORWARD/ORTHO (got %d)", norm);
  return FNO_OK;
}

static int check_skip(int32_t skip_kind, int32_t act, int32_t ci, int32_t co, const void* skip_w) {
  FNO_CHECK_ARG(skip_kind >= FNO_SKIP_NONE && skip_kind <= FNO_SKIP_IDENTITY,
                "unknown skip kind %d", skip_kind);
  FNO_CHECK_ARG(act == FNO_ACT_NONE || act == FNO_ACT_GELU, "unknown activation %d", act);
  FNO_CHECK_ARG(!(skip_kind == FNO_SKIP_LINEAR || skip_kind == FNO_SKIP_SOFT_GATING) || skip_w,
                "skip kind %d needs a skip weight", skip_kind);
  FNO_CHECK_ARG(!(skip_kind == FNO_SKIP_SOFT_GATING || skip_kind == FNO_SKIP_IDENTITY) || ci == co,
                "soft-gating / identity skips need in_channels == out_channels (%d vs %d)", ci,
                co);
  return FNO_OK;
}

extern "C" {

const char* fno_version(void) { return "fnohip 0.1 gfx950"; }

const char* fno_last_error(void) { return last_error_cstr(); }

size_t fno_rfft_window_workspace_bytes(int64_t planes, int32_t ndim, const int32_t* sizes,
                                       const int32_t* modes) {
  if (validate_window(ndim, sizes, modes) != FNO_OK || bounded_elems(planes, ndim, sizes) < 0)
    return 0;
  return rfft_window_ws(planes, ndim, sizes, modes);
}

int fno_rfft_window_f32(const float* x, void* xhat, int64_t planes, int32_t ndim,
                        const int32_t* sizes, const int32_t* modes, int32_t norm, void* workspace,
                        size_t workspace_bytes, void* stream) {
  clear_error();
  FNO_CHECK_ARG(x && xhat, "x/xhat must not be NULL");
  FNO_CHECK_ARG(planes >= 1, "planes must be positive");
  int rc = validate_window(ndim, sizes, modes);
  if (rc) return rc;
  FNO_CHECK_ARG(bounded_elems(planes, ndim, sizes) > 0, "planes x sizes exceeds %lld elements",
                (long long)kMaxElems);
  rc = check_norm(norm);
  if (rc) return rc;
  return rfft_window(x, reinterpret_cast<float2*>(xhat), planes, ndim, sizes, modes, norm, workspace,
                     workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

int fno_contract_dense_c64(const void* xhat, const void* w, void* yhat, int32_t batch,
                           int32_t in_channels, int32_t out_channels, int64_t n_modes,
                           int32_t separable, void* stream) {
  clear_error();
  FNO_CHECK_ARG(xhat && w && yhat, "xhat/w/yhat must not be NULL");
  FNO_CHECK_ARG(batch >= 1 && in_channels >= 1 && out_channels >= 1 && n_modes >= 1,
                "batch/channels/modes must be positive");
  FNO_CHECK_ARG(extent_ok({batch, in_channels > out_channels ? in_channels : out_channels, n_modes}) &&
                    extent_ok({in_channels, out_channels, n_modes}),
                "contraction operands exceed %lld elements", (long long)kMaxElems);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const float2* X = reinterpret_cast<const float2*>(xhat);
  const float2* W = reinterpret_cast<const float2*>(w);
  float2* Y = reinterpret_cast<float2*>(yhat);
  if (separable) {
    FNO_CHECK_ARG(in_channels == out_channels, "separable contraction needs Ci == Co");
    return contract_separable(X, W, Y, batch, in_channels, n_modes, st);
  }
  return contract_dense(X, W, Y, batch, in_channels, out_channels, n_modes,
                        (int64_t)out_channels * n_modes, n_modes, 1, st);
}

size_t fno_contract_tucker_workspace_bytes(int32_t batch, int32_t ndim, const int32_t* modes,
                                           const int32_t* ranks) {
  if (!modes || !ranks || ndim < 1 || ndim > 4 || batch < 1) return 0;
  for (int d = 0; d < ndim + 2; ++d)
    if (ranks[d] < 1) return 0;
  if (bounded_elems((int64_t)batch * (ranks[0] > ranks[1] ? ranks[0] : ranks[1]), ndim, modes) < 0 ||
      bounded_elems((int64_t)ranks[0] * ranks[1], ndim, modes, ranks + 2) < 0)
    return 0;
  const int64_t M = mode_count(ndim, modes);
  int64_t big = (int64_t)ranks[0] * ranks[1];
  for (int d = 0; d < ndim; ++d) big *= (modes[d] > ranks[2 + d] ? modes[d] : ranks[2 + d]);
  const int64_t K = (int64_t)ranks[0] * ranks[1] * M;
  const int64_t e = K + 2 * big + (int64_t)batch * ranks[0] * M + (int64_t)batch * ranks[1] * M;
  return (size_t)e * sizeof(float2);
}

int fno_contract_tucker_c64(const void* xhat, const void* core, const void* const* factors,
                            const int32_t* ranks, void* yhat, int32_t batch, int32_t in_channels,
                            int32_t out_channels, int32_t ndim, const int32_t* modes,
                            void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  FNO_CHECK_ARG(xhat && core && factors && ranks && yhat && modes, "NULL argument");
  FNO_CHECK_ARG(ndim >= 1 && ndim <= 4, "ndim must be 1..4");
  for (int d = 0; d < ndim + 2; ++d) {
    FNO_CHECK_ARG(factors[d], "factor %d is NULL", d);
    FNO_CHECK_ARG(ranks[d] >= 1, "rank %d must be positive", d);
  }
  FNO_CHECK_ARG(batch >= 1 && in_channels >= 1 && out_channels >= 1, "bad batch/channels");
  for (int d = 0; d < ndim; ++d) FNO_CHECK_ARG(modes[d] >= 1, "modes[%d] must be positive", d);
  FNO_CHECK_ARG(bounded_elems((int64_t)batch * (in_channels > out_channels ? in_channels : out_channels),
                              ndim, modes) > 0 &&
                    fno_contract_tucker_workspace_bytes(batch, ndim, modes, ranks) > 0,
                "tucker contraction operands exceed %lld elements", (long long)kMaxElems);
  const size_t need = fno_contract_tucker_workspace_bytes(batch, ndim, modes, ranks);
  if (workspace_bytes < need || !workspace) {
    set_error("tucker contraction: workspace %zu < %zu bytes", workspace_bytes, need);
    return FNO_ERR_WORKSPACE;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t M = mode_count(ndim, modes);
  const int rin = ranks[0], rout = ranks[1];
  int64_t big = (int64_t)rin * rout;
  for (int d = 0; d < ndim; ++d) big *= (modes[d] > ranks[2 + d] ? modes[d] : ranks[2 + d]);
  float2* Kt = reinterpret_cast<float2*>(workspace);
  // two launches (mode factors into the core, then the mode-wise products)
  // where their LDS stages fit; the chain of one launch per factor otherwise
  if (tucker_fused_supported(batch, in_channels, out_channels, ndim, modes, ranks))
    return tucker_fused(reinterpret_cast<const float2*>(xhat), reinterpret_cast<const float2*>(core),
                        reinterpret_cast<const float2* const*>(factors), ranks,
                        reinterpret_cast<float2*>(yhat), batch, in_channels, out_channels, ndim,
                        modes, Kt, st);
  float2* e1 = Kt + (int64_t)rin * rout * M;
  float2* e2 = e1 + big;
  float2* t1 = e2 + big;
  float2* t2 = t1 + (int64_t)batch * rin * M;
  // K[g,h,k] = core x_d U_d over the mode axes
  const float2* src = reinterpret_cast<const float2*>(core);
  for (int a = 0; a < ndim; ++a) {
    int64_t outer = (int64_t)rin * rout;
    for (int b = 0; b < a; ++b) outer *= modes[b];
    int64_t inner = 1;
    for (int b = a + 1; b < ndim; ++b) inner *= ranks[2 + b];
    float2* dst = (a == ndim - 1) ? Kt : ((a % 2 == 0) ? e1 : e2);
    int rc = axis_matmul(src, reinterpret_cast<const float2*>(factors[2 + a]), dst, outer,
                         ranks[2 + a], modes[a], inner, st);
    if (rc) return rc;
    src = dst;
  }
  const float2* X = reinterpret_cast<const float2*>(xhat);
  const float2* Uin = reinterpret_cast<const float2*>(factors[0]);
  const float2* Uout = reinterpret_cast<const float2*>(factors[1]);
  // t1[b,g,k] = sum_i x[b,i,k] U_in[i,g]
  int rc = contract_dense(X, Uin, t1, batch, in_channels, rin, M, rin, 1, 0, st);
  if (rc) return rc;
  // t2[b,h,k] = sum_g t1[b,g,k] K[g,h,k]
  rc = contract_dense(t1, Kt, t2, batch, rin, rout, M, (int64_t)rout * M, M, 1, st);
  if (rc) return rc;
  // y[b,o,k] = sum_h t2[b,h,k] U_out[o,h]
  return contract_dense(t2, Uout, reinterpret_cast<float2*>(yhat), batch, rout, out_channels, M, 1,
                        rout, 0, st);
}

size_t fno_irfft_window_workspace_bytes(int64_t planes, int32_t ndim, const int32_t* out_sizes,
                                        const int32_t* modes) {
  if (!out_sizes || !modes || ndim < 1 || ndim > 4) return 0;
  for (int d = 0; d < ndim; ++d)
    if (out_sizes[d] < 1 || out_sizes[d] > 4096 || modes[d] < 1) return 0;
  if (bounded_elems(planes, ndim, out_sizes, modes) < 0) return 0;
  return irfft_window_ws(planes, ndim, out_sizes, modes);
}

int fno_irfft_window_f32(const void* yhat, const float* bias, float* y, int64_t batch,
                         int32_t channels, int32_t ndim, const int32_t* in_sizes,
                         const int32_t* out_sizes, const int32_t* modes, int32_t norm,
                         int32_t enforce_hermitian, void* workspace, size_t workspace_bytes,
                         void* stream) {
  clear_error();
  FNO_CHECK_ARG(yhat && y, "yhat/y must not be NULL");
  FNO_CHECK_ARG(batch >= 1 && channels >= 1, "batch/channels must be positive");
  int rc = validate_window(ndim, in_sizes, modes);
  if (rc) return rc;
  FNO_CHECK_ARG(out_sizes, "out_sizes must not be NULL");
  for (int d = 0; d < ndim; ++d) {
    FNO_CHECK_ARG(out_sizes[d] >= 1 && out_sizes[d] <= 4096, "out size %d outside [1, 4096]",
                  out_sizes[d]);
  }
  FNO_CHECK_ARG(extent_ok({batch, channels}) &&
                    bounded_elems(batch * channels, ndim, out_sizes, in_sizes) > 0,
                "batch x channels x sizes exceeds %lld elements", (long long)kMaxElems);
  rc = check_norm(norm);
  if (rc) return rc;
  return irfft_window(reinterpret_cast<const float2*>(yhat), bias, y, batch, channels, ndim,
                      in_sizes, out_sizes, modes, norm, enforce_hermitian, workspace,
                      workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

// complex data: every axis keeps at most its own length in modes
static int validate_complex_window(int32_t ndim, const int32_t* sizes, const int32_t* modes) {
  FNO_CHECK_ARG(ndim >= 1 && ndim <= 4, "ndim must be 1..4 (got %d)", ndim);
  FNO_CHECK_ARG(sizes && modes, "sizes/modes must not be NULL");
  for (int d = 0; d < ndim; ++d) {
    FNO_CHECK_ARG(sizes[d] >= 1 && sizes[d] <= 4096, "size[%d]=%d outside [1, 4096]", d, sizes[d]);
    FNO_CHECK_ARG(modes[d] >= 1 && modes[d] <= sizes[d], "modes[%d]=%d outside [1, %d]", d,
                  modes[d], sizes[d]);
  }
  return FNO_OK;
}

size_t fno_fft_window_workspace_bytes(int64_t planes, int32_t ndim, const int32_t* sizes,
                                      const int32_t* modes) {
  if (validate_complex_window(ndim, sizes, modes) != FNO_OK ||
      bounded_elems(planes, ndim, sizes) < 0)
    return 0;
  return fft_window_c2c_ws(planes, ndim, sizes, modes);
}

int fno_fft_window_c64(const void* x, void* xhat, int64_t planes, int32_t ndim,
                       const int32_t* sizes, const int32_t* modes, int32_t norm, void* workspace,
                       size_t workspace_bytes, void* stream) {
  clear_error();
  FNO_CHECK_ARG(x && xhat, "x/xhat must not be NULL");
  FNO_CHECK_ARG(planes >= 1, "planes must be positive");
  int rc = validate_complex_window(ndim, sizes, modes);
  if (rc) return rc;
  FNO_CHECK_ARG(bounded_elems(planes, ndim, sizes) > 0, "planes x sizes exceeds %lld elements",
                (long long)kMaxElems);
  rc = check_norm(norm);
  if (rc) return rc;
  return fft_window_c2c(reinterpret_cast<const float2*>(x), reinterpret_cast<float2*>(xhat), planes,
                        ndim, sizes, modes, norm, workspace, workspace_bytes,
                        reinterpret_cast<hipStream_t>(stream));
}

size_t fno_ifft_window_workspace_bytes(int64_t planes, int32_t ndim, const int32_t* out_sizes,
                                       const int32_t* modes) {
  if (!out_sizes || !modes || ndim < 1 || ndim > 4) return 0;
  for (int d = 0; d < ndim; ++d)
    if (out_sizes[d] < 1 || out_sizes[d] > 4096 || modes[d] < 1) return 0;
  if (bounded_elems(planes, ndim, out_sizes, modes) < 0) return 0;
  return ifft_window_c2c_ws(planes, ndim, out_sizes, modes);
}

int fno_ifft_window_c64(const void* yhat, const float* bias, void* y, int64_t batch,
                        int32_t channels, int32_t ndim, const int32_t* in_sizes,
                        const int32_t* out_sizes, const int32_t* modes, int32_t norm,
                        void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  FNO_CHECK_ARG(yhat && y, "yhat/y must not be NULL");
  FNO_CHECK_ARG(batch >= 1 && channels >= 1, "batch/channels must be positive");
  int rc = validate_complex_window(ndim, in_sizes, modes);
  if (rc) return rc;
  FNO_CHECK_ARG(out_sizes, "out_sizes must not be NULL");
  for (int d = 0; d < ndim; ++d) {
    FNO_CHECK_ARG(out_sizes[d] >= 1 && out_sizes[d] <= 4096, "out size %d outside [1, 4096]",
                  out_sizes[d]);
  }
  FNO_CHECK_ARG(extent_ok({batch, channels}) &&
                    bounded_elems(batch * channels, ndim, out_sizes, in_sizes) > 0,
                "batch x channels x sizes exceeds %lld elements", (long long)kMaxElems);
  rc = check_norm(norm);
  if (rc) return rc;
  return ifft_window_c2c(reinterpret_cast<const float2*>(yhat), bias, reinterpret_cast<float2*>(y),
                         batch, channels, ndim, in_sizes, out_sizes, modes, norm, workspace,
                         workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

int fno_irfft_window_epilogue_f32(const void* yhat, const float* bias, const float* x,
                                  const float* skip_weight, float* y, int32_t batch,
                                  int32_t in_channels, int32_t out_channels, int32_t ndim,
                                  const int32_t* sizes, const int32_t* modes, int32_t norm,
                                  int32_t skip_kind, int32_t act, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  clear_error();
  FNO_CHECK_ARG(yhat && y, "yhat/y must not be NULL");
  FNO_CHECK_ARG(skip_kind == FNO_SKIP_NONE || x, "x must not be NULL with a skip");
  FNO_CHECK_ARG(batch >= 1 && in_channels >= 1 && out_channels >= 1, "bad batch/channels");
  int rc = validate_window(ndim, sizes, modes);
  if (rc) return rc;
  const int64_t cmax = in_channels > out_channels ? in_channels : out_channels;
  const int64_t elems = bounded_elems((int64_t)batch * cmax, ndim, sizes);
  FNO_CHECK_ARG(elems > 0, "batch x channels x sizes exceeds %lld elements", (long long)kMaxElems);
  const int64_t points = elems / ((int64_t)batch * cmax);
  FNO_CHECK_ARG(skip_kind == FNO_SKIP_NONE ||
                    !ranges_overlap(x, (size_t)batch * in_channels * points * sizeof(float), y,
                                    (size_t)batch * out_channels * points * sizeof(float)),
                "inverse + epilogue: y must not overlap x");
  rc = check_norm(norm);
  if (rc) return rc;
  rc = check_skip(skip_kind, act, in_channels, out_channels, skip_weight);
  if (rc) return rc;
  return irfft_epilogue(reinterpret_cast<const float2*>(yhat), bias, x, skip_weight, y, batch,
                        in_channels, out_channels, ndim, sizes, modes, norm, skip_kind, act,
                        workspace, workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

int fno_block_epilogue_f32(const float* spec, const float* x, const float* skip_weight, float* y,
                           int32_t batch, int32_t in_channels, int32_t out_channels,
                           int64_t points, int32_t skip_kind, int32_t act, void* stream) {
  clear_error();
  FNO_CHECK_ARG(spec && y, "spec/y must not be NULL");
  FNO_CHECK_ARG(skip_kind == FNO_SKIP_NONE || x, "x must not be NULL with a skip");
  FNO_CHECK_ARG(batch >= 1 && in_channels >= 1 && out_channels >= 1 && points >= 1,
                "bad batch/channels/points");
  FNO_CHECK_ARG(extent_ok({batch, in_channels > out_channels ? in_channels : out_channels, points}),
                "batch x channels x points exceeds %lld elements", (long long)kMaxElems);
  int rc = check_skip(skip_kind, act, in_channels, out_channels, skip_weight);
  if (rc) return rc;
  return block_epilogue(spec, x, skip_weight, y, batch, in_channels, out_channels, points,
                        skip_kind, act, reinterpret_cast<hipStream_t>(stream));
}

int fno_channel_mlp_is_supported(int32_t in_channels, int32_t hidden_channels,
                                 int32_t out_channels, int64_t points) {
  return channel_mlp_supported(in_channels, hidden_channels, out_channels, points) ? 1 : 0;
}

int fno_channel_mlp_f32(const float* x, const float* w1, const float* b1, const float* w2,
                        const float* b2, const float* skip_x, const float* skip_weight,
                        const float* skip_bias, float* y, int64_t batch, int32_t in_channels,
                        int32_t hidden_channels, int32_t out_channels, int64_t points,
                        int32_t skip_kind, int32_t act, int32_t bf16_products, void* stream) {
  clear_error();
  FNO_CHECK_ARG(x && w1 && w2 && y, "x/w1/w2/y must not be NULL");
  FNO_CHECK_ARG(bf16_products == 0 || bf16_products == 1, "bf16_products must be 0 or 1 (got %d)",
                bf16_products);
  FNO_CHECK_ARG(batch >= 1 && in_channels >= 1 && hidden_channels >= 1 && out_channels >= 1 &&
                    points >= 1,
                "bad batch/channels/points");
  FNO_CHECK_ARG(extent_ok({batch, in_channels > out_channels ? in_channels : out_channels, points}),
                "batch x channels x points exceeds %lld elements", (long long)kMaxElems);
  FNO_CHECK_ARG(skip_kind == FNO_SKIP_NONE || skip_kind == FNO_SKIP_SOFT_GATING ||
                    skip_kind == FNO_SKIP_IDENTITY,
                "channel MLP skip must be none, soft-gating or identity (got %d)", skip_kind);
  FNO_CHECK_ARG(skip_kind == FNO_SKIP_NONE || skip_x, "skip_x must not be NULL with a skip");
  FNO_CHECK_ARG(skip_kind != FNO_SKIP_SOFT_GATING || skip_weight,
                "soft-gating needs a skip weight");
  FNO_CHECK_ARG(act == FNO_ACT_NONE || act == FNO_ACT_GELU, "unknown activation %d", act);
  if (!channel_mlp_supported(in_channels, hidden_channels, out_channels, points)) {
    set_error("channel MLP %d -> %d -> %d over %lld points is not covered by the kernel",
              in_channels, hidden_channels, out_channels, (long long)points);
    return FNO_ERR_UNSUPPORTED;
  }
  // 16-byte slab loads of x, staged 16-byte rows of skip_x and y
  const uintptr_t addr = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(skip_x) |
                         reinterpret_cast<uintptr_t>(y);
  if (addr % 16 != 0) {
    set_error("channel MLP: x, skip_x and y must be 16-byte aligned");
    return FNO_ERR_UNSUPPORTED;
  }
  // In place is safe only element for element: y over x when both have the
  // same layout (Ci == Co), y over skip_x (always [B, Co, P]).  Any other
  // overlap lets a workgroup overwrite rows another one has not read yet.
  const size_t ybytes = (size_t)batch * out_channels * points * sizeof(float);
  const size_t xbytes = (size_t)batch * in_channels * points * sizeof(float);
  FNO_CHECK_ARG(!ranges_overlap(x, xbytes, y, ybytes) || (x == y && in_channels == out_channels),
                "channel MLP: y may alias x only exactly and with in_channels == out_channels "
                "(%d vs %d)", in_channels, out_channels);
  FNO_CHECK_ARG(skip_kind == FNO_SKIP_NONE || !ranges_overlap(skip_x, ybytes, y, ybytes) ||
                    skip_x == y,
                "channel MLP: y may alias skip_x only exactly");
  return channel_mlp(x, w1, b1, w2, b2, skip_x, skip_weight, skip_bias, y, batch, in_channels,
                     hidden_channels, out_channels, points, skip_kind, act, bf16_products != 0,
                     reinterpret_cast<hipStream_t>(stream));
}

int fno_channel_mlp_io_is_supported(int32_t in_channels, int32_t hidden_channels,
                                    int32_t out_channels, int64_t points, int32_t x_bf16,
                                    int32_t y_bf16) {
  return channel_mlp_io_supported(in_channels, hidden_channels, out_channels, points, x_bf16 != 0,
                                  y_bf16 != 0)
             ? 1
             : 0;
}

int fno_channel_mlp_io(const void* x, const float* w1, const float* b1, const float* w2,
                       const float* b2, void* y, int64_t batch, int32_t in_channels,
                       int32_t hidden_channels, int32_t out_channels, int64_t points, int32_t act,
                       int32_t x_bf16, int32_t y_bf16, void* stream) {
  clear_error();
  FNO_CHECK_ARG(x && w1 && w2 && y, "x/w1/w2/y must not be NULL");
  FNO_CHECK_ARG((x_bf16 == 0 || x_bf16 == 1) && (y_bf16 == 0 || y_bf16 == 1),
                "x_bf16 / y_bf16 must be 0 or 1 (got %d, %d)", x_bf16, y_bf16);
  FNO_CHECK_ARG(batch >= 1 && in_channels >= 1 && hidden_channels >= 1 && out_channels >= 1 &&
                    points >= 1,
                "bad batch/channels/points");
  FNO_CHECK_ARG(extent_ok({batch, in_channels > out_channels ? in_channels : out_channels, points}),
                "batch x channels x points exceeds %lld elements", (long long)kMaxElems);
  FNO_CHECK_ARG(act == FNO_ACT_NONE || act == FNO_ACT_GELU, "unknown activation %d", act);
  if (!channel_mlp_io_supported(in_channels, hidden_channels, out_channels, points, x_bf16 != 0,
                                y_bf16 != 0)) {
    set_error("channel MLP %d -> %d -> %d over %lld points with %s storage is not covered by the "
              "kernel", in_channels, hidden_channels, out_channels, (long long)points,
              x_bf16 ? (y_bf16 ? "bf16 in / bf16 out" : "bf16 in") : (y_bf16 ? "bf16 out" : "fp32"));
    return FNO_ERR_UNSUPPORTED;
  }
  const uintptr_t addr = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y);
  if (addr % 16 != 0) {
    set_error("channel MLP: x and y must be 16-byte aligned");
    return FNO_ERR_UNSUPPORTED;
  }
  const size_t ybytes = (size_t)batch * out_channels * points * (y_bf16 ? 2 : 4);
  const size_t xbytes = (size_t)batch * in_channels * points * (x_bf16 ? 2 : 4);
  FNO_CHECK_ARG(!ranges_overlap(x, xbytes, y, ybytes), "channel MLP: y must not overlap x");
  if (!x_bf16 && !y_bf16)
    return channel_mlp(static_cast<const float*>(x), w1, b1, w2, b2, nullptr, nullptr, nullptr,
                       static_cast<float*>(y), batch, in_channels, hidden_channels, out_channels,
                       points, FNO_SKIP_NONE, act, true, reinterpret_cast<hipStream_t>(stream));
  return channel_mlp_io(x, w1, b1, w2, b2, y, batch, in_channels, hidden_channels, out_channels,
                        points, act, x_bf16 != 0, y_bf16 != 0,
                        reinterpret_cast<hipStream_t>(stream));
}

int fno_spectral_block_is_fused(int32_t batch, int32_t in_channels, int32_t out_channels,
                                int32_t ndim, const int32_t* sizes, const int32_t* modes,
                                int32_t skip_kind) {
  if (!sizes || !modes) return 0;
  return fast2d_supported(batch, in_channels, out_channels, ndim, sizes, modes, skip_kind) ? 1 : 0;
}

size_t fno_spectral_block_workspace_bytes(int32_t batch, int32_t in_channels,
                                          int32_t out_channels, int32_t ndim,
                                          const int32_t* sizes, const int32_t* modes) {
  if (batch < 1 || in_channels < 1 || out_channels < 1 ||
      validate_window(ndim, sizes, modes) != FNO_OK ||
      bounded_elems((int64_t)batch * (in_channels > out_channels ? in_channels : out_channels), ndim,
                    sizes) < 0)
    return 0;
  size_t fused = 0;
  if (ndim == 2) fused = fast2d_workspace(batch, in_channels, out_channels, sizes, modes);
  // shapes the row-synthesis epilogue covers take the fused path for every skip kind
  if (ndim == 2 && rowsynth_covers(sizes[0], sizes[1], in_channels, out_channels, modes[0],
                                   modes[1]))
    return fused;
  const int64_t M = mode_count(ndim, modes);
  const size_t spectra = (size_t)((int64_t)batch * in_channels * M +
                                  (int64_t)batch * out_channels * M) * sizeof(float2);
  size_t a = rfft_window_ws((int64_t)batch * in_channels, ndim, sizes, modes);
  size_t b = irfft_window_ws((int64_t)batch * out_channels, ndim, sizes, modes);
  const size_t generic = spectra + (a > b ? a : b);
  return fused > generic ? fused : generic;
}

}  // extern "C"

namespace fno {

// es: bytes per element of x and y (4: float32, 2: bfloat16)
int spectral_block_check(const void* x, const void* w, void* y, int32_t batch,
                         int32_t in_channels, int32_t out_channels, int32_t ndim,
                         const int32_t* sizes, const int32_t* modes, int32_t norm,
                         int32_t skip_kind, int32_t act, const float* skip_weight,
                         size_t es = sizeof(float)) {
  FNO_CHECK_ARG(x && w && y, "x/w/y must not be NULL");
  FNO_CHECK_ARG(batch >= 1 && in_channels >= 1 && out_channels >= 1, "bad batch/channels");
  int rc = validate_window(ndim, sizes, modes);
  if (rc) return rc;
  const int64_t cmax = in_channels > out_channels ? in_channels : out_channels;
  const int64_t elems = bounded_elems((int64_t)batch * cmax, ndim, sizes);
  FNO_CHECK_ARG(elems > 0, "batch x channels x sizes exceeds %lld elements", (long long)kMaxElems);
  const int64_t points = elems / ((int64_t)batch * cmax);
  FNO_CHECK_ARG(!ranges_overlap(x, (size_t)batch * in_channels * points * es, y,
                                (size_t)batch * out_channels * points * es),
                "spectral block: y must not overlap x");
  rc = check_norm(norm);
  if (rc) return rc;
  return check_skip(skip_kind, act, in_channels, out_channels, skip_weight);
}

// The block on validated arguments and a workspace of at least
// fno_spectral_block_workspace_bytes(batch, ...) bytes.
int spectral_block_run(const float* x, const void* w, const float* bias, const float* skip_weight,
                       float* y, int32_t batch, int32_t in_channels, int32_t out_channels,
                       int32_t ndim, const int32_t* sizes, const int32_t* modes, int32_t norm,
                       int32_t skip_kind, int32_t act, void* workspace, size_t workspace_bytes,
                       hipStream_t st) {
  int rc;
  if (ndim == 1 && line1d_supported(in_channels, out_channels, sizes[0], modes[0], skip_kind))
    return line1d_block(x, reinterpret_cast<const float2*>(w), bias, skip_weight, y, batch,
                        in_channels, out_channels, sizes[0], modes[0], norm, skip_kind, act,
                        workspace, workspace_bytes, st);
  if (ndim == 1 && fast1d_supported(in_channels, out_channels, sizes[0], modes[0]))
    return fast1d_block(x, reinterpret_cast<const float2*>(w), bias, skip_weight, y, batch,
                        in_channels, out_channels, sizes[0], modes[0], norm, skip_kind, act, st);
  if (fast2d_supported(batch, in_channels, out_channels, ndim, sizes, modes, skip_kind))
    return fast2d_block(x, reinterpret_cast<const float2*>(w), bias, skip_weight, y, batch,
                        in_channels, out_channels, sizes, modes, norm, skip_kind, act, workspace,
                        workspace_bytes, st);
  // generic composition
  const int64_t M = mode_count(ndim, modes);
  float2* xhat = reinterpret_cast<float2*>(workspace);
  float2* yhat = xhat + (int64_t)batch * in_channels * M;
  void* rest = yhat + (int64_t)batch * out_channels * M;
  const size_t rest_bytes = workspace_bytes - (size_t)((int64_t)batch * (in_channels + out_channels) *
                                                       M * sizeof(float2));
  rc = rfft_window(x, xhat, (int64_t)batch * in_channels, ndim, sizes, modes, norm, rest,
                   rest_bytes, st);
  if (rc) return rc;
  rc = contract_dense(xhat, reinterpret_cast<const float2*>(w), yhat, batch, in_channels,
                      out_channels, M, (int64_t)out_channels * M, M, 1, st);
  if (rc) return rc;
  // inverse + bias + skip + activation (one pass over the last axis where
  // the line epilogue covers it)
  return irfft_epilogue(yhat, bias, x, skip_weight, y, batch, in_channels, out_channels, ndim,
                        sizes, modes, norm, skip_kind, act, rest, rest_bytes, st);
}

}  // namespace fno

extern "C" {

int fno_spectral_block_f32(const float* x, const void* w, const float* bias,
                           const float* skip_weight, float* y, int32_t batch, int32_t in_channels,
                           int32_t out_channels, int32_t ndim, const int32_t* sizes,
                           const int32_t* modes, int32_t norm, int32_t skip_kind, int32_t act,
                           void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  int rc = spectral_block_check(x, w, y, batch, in_channels, out_channels, ndim, sizes, modes, norm,
                                skip_kind, act, skip_weight);
  if (rc) return rc;
  const size_t need = fno_spectral_block_workspace_bytes(batch, in_channels, out_channels, ndim,
                                                         sizes, modes);
  if (!workspace || workspace_bytes < need) {
    set_error("spectral block: workspace %zu < %zu bytes", workspace_bytes, need);
    return FNO_ERR_WORKSPACE;
  }
  return spectral_block_run(x, w, bias, skip_weight, y, batch, in_channels, out_channels, ndim,
                            sizes, modes, norm, skip_kind, act, workspace, workspace_bytes,
                            reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"

// ---------------------------------------------------------------- FNO layer
// bf16: bfloat16 activation storage (fno_layer_bf16)
static bool layer_fused(int32_t batch, int32_t channels, int32_t hidden, int32_t ndim,
                        const int32_t* sizes, const int32_t* modes, int32_t skip_kind,
                        int32_t mlp_skip_kind, bool bf16 = false) {
  if (!sizes || !modes || ndim != 2 || batch < 1) return false;
  if (!(mlp_skip_kind == FNO_SKIP_NONE || mlp_skip_kind == FNO_SKIP_SOFT_GATING ||
        mlp_skip_kind == FNO_SKIP_IDENTITY))
    return false;
  if (!fast2d_supported(batch, channels, channels, ndim, sizes, modes, skip_kind) ||
      !rowsynth_mlp_covers(sizes[0], sizes[1], channels, channels, modes[0], modes[1], hidden,
                           skip_kind))
    return false;
  return !bf16 || fast2d_bf16_supported(sizes, modes);
}

extern "C" {

int fno_layer_is_fused(int32_t batch, int32_t channels, int32_t hidden_channels, int32_t ndim,
                       const int32_t* sizes, const int32_t* modes, int32_t skip_kind,
                       int32_t mlp_skip_kind) {
  return layer_fused(batch, channels, hidden_channels, ndim, sizes, modes, skip_kind,
                     mlp_skip_kind)
             ? 1
             : 0;
}

int fno_layer_bf16_is_fused(int32_t batch, int32_t channels, int32_t hidden_channels,
                            int32_t ndim, const int32_t* sizes, const int32_t* modes,
                            int32_t skip_kind, int32_t mlp_skip_kind) {
  return layer_fused(batch, channels, hidden_channels, ndim, sizes, modes, skip_kind,
                     mlp_skip_kind, true)
             ? 1
             : 0;
}

// Both layer entry points: es = bytes per element of x and y.
static int layer_run(const void* x, const void* w, const float* bias, const float* skip_weight,
                     const float* mlp_w1, const float* mlp_b1, const float* mlp_w2,
                     const float* mlp_b2, const float* gate_weight, const float* gate_bias, void* y,
                     int32_t batch, int32_t channels, int32_t hidden_channels, int32_t ndim,
                     const int32_t* sizes, const int32_t* modes, int32_t norm, int32_t skip_kind,
                     int32_t mlp_skip_kind, int32_t act, void* workspace, size_t workspace_bytes,
                     void* stream, size_t es) {
  clear_error();
  int rc = spectral_block_check(x, w, y, batch, channels, channels, ndim, sizes, modes, norm,
                                skip_kind, act, skip_weight, es);
  if (rc) return rc;
  FNO_CHECK_ARG(mlp_w1 && mlp_w2, "mlp_w1/mlp_w2 must not be NULL");
  FNO_CHECK_ARG(hidden_channels >= 1, "hidden_channels must be positive");
  FNO_CHECK_ARG(mlp_skip_kind == FNO_SKIP_NONE || mlp_skip_kind == FNO_SKIP_SOFT_GATING ||
                    mlp_skip_kind == FNO_SKIP_IDENTITY,
                "channel MLP skip must be none, soft-gating or identity (got %d)", mlp_skip_kind);
  FNO_CHECK_ARG(mlp_skip_kind != FNO_SKIP_SOFT_GATING || gate_weight,
                "soft-gating needs a gate weight");
  if (!layer_fused(batch, channels, hidden_channels, ndim, sizes, modes, skip_kind,
                   mlp_skip_kind, es == 2)) {
    set_error(es == 2 ? "FNO layer: this shape has no one-pass bfloat16 kernel "
                        "(fno_layer_bf16_is_fused)"
                      : "FNO layer: this shape has no one-pass kernel (compose "
                        "fno_spectral_block_f32 and fno_channel_mlp_f32)");
    return FNO_ERR_UNSUPPORTED;
  }
  const size_t need = fno_spectral_block_workspace_bytes(batch, channels, channels, ndim, sizes,
                                                         modes);
  if (!workspace || workspace_bytes < need) {
    set_error("FNO layer: workspace %zu < %zu bytes", workspace_bytes, need);
    return FNO_ERR_WORKSPACE;
  }
  LayerMlp mlp;
  mlp.w1 = mlp_w1;
  mlp.b1 = mlp_b1;
  mlp.w2 = mlp_w2;
  mlp.b2 = mlp_b2;
  mlp.gate_w = gate_weight;
  mlp.gate_b = mlp_skip_kind == FNO_SKIP_SOFT_GATING ? gate_bias : nullptr;
  mlp.gate_kind = mlp_skip_kind;
  return fast2d_block(x, reinterpret_cast<const float2*>(w), bias, skip_weight, y, batch, channels,
                      channels, sizes, modes, norm, skip_kind, act, workspace, workspace_bytes,
                      reinterpret_cast<hipStream_t>(stream), &mlp, es == 2);
}

int fno_layer_f32(const float* x, const void* w, const float* bias, const float* skip_weight,
                  const float* mlp_w1, const float* mlp_b1, const float* mlp_w2,
                  const float* mlp_b2, const float* gate_weight, const float* gate_bias, float* y,
                  int32_t batch, int32_t channels, int32_t hidden_channels, int32_t ndim,
                  const int32_t* sizes, const int32_t* modes, int32_t norm, int32_t skip_kind,
                  int32_t mlp_skip_kind, int32_t act, void* workspace, size_t workspace_bytes,
                  void* stream) {
  return layer_run(x, w, bias, skip_weight, mlp_w1, mlp_b1, mlp_w2, mlp_b2, gate_weight, gate_bias,
                   y, batch, channels, hidden_channels, ndim, sizes, modes, norm, skip_kind,
                   mlp_skip_kind, act, workspace, workspace_bytes, stream, sizeof(float));
}

int fno_layer_bf16(const void* x, const void* w, const float* bias, const float* skip_weight,
                   const float* mlp_w1, const float* mlp_b1, const float* mlp_w2,
                   const float* mlp_b2, const float* gate_weight, const float* gate_bias, void* y,
                   int32_t batch, int32_t channels, int32_t hidden_channels, int32_t ndim,
                   const int32_t* sizes, const int32_t* modes, int32_t norm, int32_t skip_kind,
                   int32_t mlp_skip_kind, int32_t act, void* workspace, size_t workspace_bytes,
                   void* stream) {
  return layer_run(x, w, bias, skip_weight, mlp_w1, mlp_b1, mlp_w2, mlp_b2, gate_weight, gate_bias,
                   y, batch, channels, hidden_channels, ndim, sizes, modes, norm, skip_kind,
                   mlp_skip_kind, act, workspace, workspace_bytes, stream, 2);
}

}  // extern "C"
