/*
 * fno_hip.h -- C ABI of the MI355X (gfx950) FNO spectral-block library
 * (libfnohip.so).
 *
 * Conventions
 *   - Every pointer is a device pointer to contiguous memory allocated by the
 *     caller (in practice torch's caching allocator).  Real fields are float32
 *     N C D1..Dn; complex spectra are complex64 (interleaved float pairs).
 *   - Returns 0 (FNO_OK) on success, otherwise an FNO_ERR_* code; the message
 *     is available from fno_last_error() (thread-local).
 *   - Shapes are validated on the host before any launch.  Work is enqueued on
 *     `stream` (a hipStream_t passed as void*); nothing synchronizes.
 *   - The library allocates no device memory: scratch space is the caller's
 *     `workspace` of at least the size the matching *_workspace_bytes() call
 *     reports.
 *   - ndim (spatial axes) is 1..4, each axis 1..4096 points.
 *   - Spectrum window layout ("window order"): along every axis but the last,
 *     window index j holds frequency j - m/2 (integer division), which is the
 *     fftshift-ed order the reference's weights use; along the last (rfft)
 *     axis index j holds frequency j.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   neuralop/layers/spectral_convolution.py  SpectralConv.forward :417-570
 *   neuralop/layers/fno_block.py             FNOBlocks.forward_with_postactivation :327-381
 *   neuralop/layers/skip_connections.py      Flattened1dConv.forward :122-130,
 *                                            SoftGating.forward :88-93
 */
#ifndef FNO_HIP_H
#define FNO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FNO_OK 0
#define FNO_ERR_INVALID 1     /* bad argument or shape */
#define FNO_ERR_UNSUPPORTED 2 /* valid request the kernels do not cover */
#define FNO_ERR_HIP 3         /* HIP runtime error */
#define FNO_ERR_WORKSPACE 4   /* workspace smaller than required */

/* torch.fft norm= values */
#define FNO_NORM_BACKWARD 0
#define FNO_NORM_FORWARD 1
#define FNO_NORM_ORTHO 2

/* skip connection applied by the block entry points */
#define FNO_SKIP_NONE 0
#define FNO_SKIP_LINEAR 1      /* 1x1 conv, weight [Co, Ci], no bias */
#define FNO_SKIP_SOFT_GATING 2 /* per-channel scale, weight [C] (Ci == Co) */
#define FNO_SKIP_IDENTITY 3    /* Ci == Co */

/* activation applied by the block entry points */
#define FNO_ACT_NONE 0
#define FNO_ACT_GELU 1 /* exact erf GELU, torch.nn.functional.gelu default */

/* Library version string. */
const char* fno_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* fno_last_error(void);

/*
 * Forward truncated real FFT.  Replaces torch.fft.rfftn(norm=...) + fftshift
 * + window slice, spectral_convolution.py:443-449 and :500-521.
 *   x     float32 [planes, N_1..N_ndim]
 *   xhat  complex64 [planes, m_1..m_ndim] in window order
 *   modes m_d = kept count per axis (m_last <= N_last/2+1, m_d <= N_d)
 */
int fno_rfft_window_f32(const float* x, void* xhat, int64_t planes, int32_t ndim,
                        const int32_t* sizes, const int32_t* modes, int32_t norm,
                        void* workspace, size_t workspace_bytes, void* stream);
size_t fno_rfft_window_workspace_bytes(int64_t planes, int32_t ndim, const int32_t* sizes,
                                       const int32_t* modes);

/*
 * Dense mode-wise complex contraction.  Replaces _contract_dense and
 * _contract_dense_separable, spectral_convolution.py:21-52.
 *   separable == 0: y[b,o,k] = sum_i x[b,i,k] w[i,o,k]   (w [Ci,Co,M])
 *   separable != 0: y[b,i,k] = x[b,i,k] w[i,k]           (w [Ci,M], Co == Ci)
 * M = prod(m_d) modes, all complex64.
 */
int fno_contract_dense_c64(const void* xhat, const void* w, void* yhat, int32_t batch,
                           int32_t in_channels, int32_t out_channels, int64_t n_modes,
                           int32_t separable, void* stream);

/*
 * Tucker-factorized contraction with the factors, never forming the dense
 * weight.  Replaces _contract_tucker (non-separable),
 * spectral_convolution.py:76-103.
 *   core     complex64 [r_in, r_out, r_1..r_ndim]
 *   factors  ndim+2 complex64 matrices: U_in [Ci, r_in], U_out [Co, r_out],
 *            U_d [m_d, r_d] (already cut to the window rows)
 *   y[b,o,k] = sum x[b,i,k] core[g,h,a..] U_in[i,g] U_out[o,h] prod_d U_d[k_d,a_d]
 */
int fno_contract_tucker_c64(const void* xhat, const void* core, const void* const* factors,
                            const int32_t* ranks, void* yhat, int32_t batch,
                            int32_t in_channels, int32_t out_channels, int32_t ndim,
                            const int32_t* modes, void* workspace, size_t workspace_bytes,
                            void* stream);
size_t fno_contract_tucker_workspace_bytes(int32_t batch, int32_t ndim, const int32_t* modes,
                                           const int32_t* ranks);

/*
 * Inverse of the window transform plus bias.  Replaces ifftshift + ifftn
 * (s = out sizes) + Hermitian fix-up + irfft + bias,
 * spectral_convolution.py:524-568 (enforce_hermitian_symmetry selects the
 * :547-559 or the :564 branch; out sizes differ from in sizes under
 * output_shape / resolution_scaling_factor).
 *   yhat  complex64 [batch*channels, m_1..m_ndim] window order
 *   bias  float32 [channels] or NULL
 *   y     float32 [batch*channels, N'_1..N'_ndim]
 */
int fno_irfft_window_f32(const void* yhat, const float* bias, float* y, int64_t batch,
                         int32_t channels, int32_t ndim, const int32_t* in_sizes,
                         const int32_t* out_sizes, const int32_t* modes, int32_t norm,
                         int32_t enforce_hermitian, void* workspace, size_t workspace_bytes,
                         void* stream);
size_t fno_irfft_window_workspace_bytes(int64_t planes, int32_t ndim, const int32_t* out_sizes,
                                        const int32_t* modes);

/*
 * Complex-data window transforms (SpectralConv(complex_data=True)).  Replace
 * torch.fft.fftn + fftshift + window slice and the inverse scatter +
 * ifftshift + ifftn of spectral_convolution.py:436-449, :500-538.
 *   x     complex64 [planes, N_1..N_ndim]
 *   xhat  complex64 [planes, m_1..m_ndim], m_d <= N_d: on every axis but the
 *         last, window index j holds frequency j - m/2; on the last axis it
 *         holds frequency j - N/2 (j of the fftshift-ed order) when ndim > 1
 *         and frequency j when ndim == 1
 *   fno_ifft_window_c64: window -> complex64 y [batch, channels, out sizes];
 *         on the last axis window entry j is frequency j (no ifftshift
 *         there); bias (float32 [channels] or NULL) is added to the real part
 */
int fno_fft_window_c64(const void* x, void* xhat, int64_t planes, int32_t ndim,
                       const int32_t* sizes, const int32_t* modes, int32_t norm, void* workspace,
                       size_t workspace_bytes, void* stream);
size_t fno_fft_window_workspace_bytes(int64_t planes, int32_t ndim, const int32_t* sizes,
                                      const int32_t* modes);
int fno_ifft_window_c64(const void* yhat, const float* bias, void* y, int64_t batch,
                        int32_t channels, int32_t ndim, const int32_t* in_sizes,
                        const int32_t* out_sizes, const int32_t* modes, int32_t norm,
                        void* workspace, size_t workspace_bytes, void* stream);
size_t fno_ifft_window_workspace_bytes(int64_t planes, int32_t ndim, const int32_t* out_sizes,
                                       const int32_t* modes);

/*
 * Inverse window transform with the bias, skip and activation, output on the
 * input grid:  y = act(irfft(yhat) + bias + skip(x)).  Replaces the inverse
 * of SpectralConv.forward (ifftshift, ifftn over the non-last axes, Hermitian
 * fix-up, irfft, bias: spectral_convolution.py:531-568) followed by the skip
 * add and first activation of FNOBlocks.forward_with_postactivation
 * (fno_block.py:331-361, skips of skip_connections.py:88-130).
 *   yhat  complex64 [batch, out_channels, m_1..m_ndim] window order
 *   x     float32 [batch, in_channels, N_1..N_ndim] (NULL without a skip);
 *         y float32 [batch, out_channels, N_1..N_ndim], not overlapping x
 * Lines of 64 points with at most 15 kept bins and 32 / 64 channels take the
 * last axis, bias, skip and activation in one pass over the non-last
 * transforms' output (the spectral field never reaches memory); other shapes
 * run fno_irfft_window_f32 then fno_block_epilogue_f32.  Workspace:
 * fno_irfft_window_workspace_bytes(batch * out_channels, ndim, sizes, modes).
 */
int fno_irfft_window_epilogue_f32(const void* yhat, const float* bias, const float* x,
                                  const float* skip_weight, float* y, int32_t batch,
                                  int32_t in_channels, int32_t out_channels, int32_t ndim,
                                  const int32_t* sizes, const int32_t* modes, int32_t norm,
                                  int32_t skip_kind, int32_t act, void* workspace,
                                  size_t workspace_bytes, void* stream);

/*
 * Block epilogue: y = act(spec + skip(x)).  Replaces the skip, add and first
 * activation of FNOBlocks.forward_with_postactivation, fno_block.py:331-361,
 * with the skips of skip_connections.py:88-130.  spec may alias y.
 *   spec, y  float32 [B, Co, P];  x float32 [B, Ci, P]
 */
int fno_block_epilogue_f32(const float* spec, const float* x, const float* skip_weight,
                           float* y, int32_t batch, int32_t in_channels, int32_t out_channels,
                           int64_t points, int32_t skip_kind, int32_t act, void* stream);

/*
 * Fused channel MLP of an FNO layer: y = act(W2 gelu(W1 x + b1) + b2 + skip).
 * Replaces ChannelMLP.forward with n_layers = 2 (neuralop/layers/channel_mlp.py
 * :82-119: two 1x1 Conv1d with GELU between), the channel-MLP skip
 * (SoftGating.forward, skip_connections.py:88-93, or identity) and the second
 * activation of FNOBlocks.forward_with_postactivation (fno_block.py:363-379).
 *   x       float32 [B, Ci, P]; y float32 [B, Co, P]; x, y and skip_x
 *           16-byte aligned.  y may be the same buffer as skip_x, or as x
 *           when Ci == Co; any other overlap of y with x or skip_x returns
 *           FNO_ERR_INVALID
 *   w1 [Ch, Ci], b1 [Ch] (may be NULL), w2 [Co, Ch], b2 [Co] (may be NULL)
 *   skip_kind FNO_SKIP_NONE, FNO_SKIP_SOFT_GATING (skip_x [B, Co, P] scaled
 *           by skip_weight [Co] plus skip_bias [Co] or NULL) or
 *           FNO_SKIP_IDENTITY (skip_x added)
 *   bf16_products 0: fp32 products; 1: the two 1x1 layers take x, W1, the
 *           hidden activation and W2 rounded to bf16 (nearest even) with fp32
 *           accumulation, as Conv1d runs under torch.autocast(dtype=bfloat16);
 *           biases, skip and activations stay fp32, y is fp32 either way
 * Covered: (Ci, Ch, Co) in {(32,16,32), (64,32,64), (128,64,128)} (block
 * MLPs), Ci <= 4 with (Ch, Co) in {(128,64), (64,32)} (lifting) and
 * (Ci, Ch) in {(64,128), (32,64)} with Co <= 16 (projection), P % 4 == 0;
 * otherwise FNO_ERR_UNSUPPORTED (fno_channel_mlp_is_supported tells which).
 */
int fno_channel_mlp_f32(const float* x, const float* w1, const float* b1, const float* w2,
                        const float* b2, const float* skip_x, const float* skip_weight,
                        const float* skip_bias, float* y, int64_t batch, int32_t in_channels,
                        int32_t hidden_channels, int32_t out_channels, int64_t points,
                        int32_t skip_kind, int32_t act, int32_t bf16_products, void* stream);
int fno_channel_mlp_is_supported(int32_t in_channels, int32_t hidden_channels,
                                 int32_t out_channels, int64_t points);

/*
 * The lifting and projection MLPs of the bf16 FNO forward, with bfloat16
 * activation storage on one side: y = act(W2 gelu(W1 x + b1) + b2), both 1x1
 * layers on bf16 operands with fp32 accumulation (as fno_channel_mlp_f32 with
 * bf16_products = 1; ChannelMLP.forward, neuralop/layers/channel_mlp.py
 * :82-119, under torch.autocast(dtype=bfloat16)), no skip.
 *   x_bf16 = 1: x is bfloat16 [B, Ci, P] (the projection's input);
 *   y_bf16 = 1: y is bfloat16 [B, Co, P], rounded to nearest even (the
 *   lifting's output); the other side is float32.  x and y 16-byte aligned,
 *   not overlapping.
 * Covered: Ci <= 4 -> (128, 64) or (64, 32) with y_bf16 (lifting),
 * (64, 128) or (32, 64) -> Co <= 16 with x_bf16 (projection), P % 4 == 0;
 * with neither flag every fno_channel_mlp_f32 width.  Otherwise
 * FNO_ERR_UNSUPPORTED (fno_channel_mlp_io_is_supported tells which).
 */
int fno_channel_mlp_io(const void* x, const float* w1, const float* b1, const float* w2,
                       const float* b2, void* y, int64_t batch, int32_t in_channels,
                       int32_t hidden_channels, int32_t out_channels, int64_t points, int32_t act,
                       int32_t x_bf16, int32_t y_bf16, void* stream);
int fno_channel_mlp_io_is_supported(int32_t in_channels, int32_t hidden_channels,
                                    int32_t out_channels, int64_t points, int32_t x_bf16,
                                    int32_t y_bf16);

/*
 * One call for the whole spectral block
 *     y = act(SpectralConv(x) + skip(x))
 * with a dense weight (w [Ci, Co, m_1..m_ndim] window, complex64) and bias
 * [Co] (or NULL).  Output size equals input size.  Picks the fused 2D path
 * (LDS FFTs + MFMA skip epilogue) when the shape allows it and composes the
 * generic kernels otherwise.
 */
int fno_spectral_block_f32(const float* x, const void* w, const float* bias,
                           const float* skip_weight, float* y, int32_t batch,
                           int32_t in_channels, int32_t out_channels, int32_t ndim,
                           const int32_t* sizes, const int32_t* modes, int32_t norm,
                           int32_t skip_kind, int32_t act, void* workspace,
                           size_t workspace_bytes, void* stream);
size_t fno_spectral_block_workspace_bytes(int32_t batch, int32_t in_channels,
                                          int32_t out_channels, int32_t ndim,
                                          const int32_t* sizes, const int32_t* modes);

/* 1 if fno_spectral_block_f32 takes the fused 2D path for this shape. */
int fno_spectral_block_is_fused(int32_t batch, int32_t in_channels, int32_t out_channels,
                                int32_t ndim, const int32_t* sizes, const int32_t* modes,
                                int32_t skip_kind);

/*
 * One FNO layer in post-activation form, for the autocast (bfloat16)
 * forward.  Replaces FNOBlocks.forward_with_postactivation with a two-layer
 * channel MLP, neuralop/layers/fno_block.py:331-379 (SpectralConv, the fno
 * skip, activation, ChannelMLP.forward of channel_mlp.py:82-119, the
 * channel-MLP skip of skip_connections.py:88-93, activation):
 *     y1 = act(SpectralConv(x) + skip(x))                 (as fno_spectral_block_f32)
 *     y  = act(W2 gelu(W1 y1 + b1) + b2 + mlp_skip(x))
 *   channels in == out; mlp_w1 [hidden, C], mlp_b1 [hidden] or NULL,
 *   mlp_w2 [C, hidden], mlp_b2 [C] or NULL; mlp_skip_kind FNO_SKIP_NONE,
 *   FNO_SKIP_SOFT_GATING (gate_weight [C], gate_bias [C] or NULL) or
 *   FNO_SKIP_IDENTITY.  The two MLP products take y1, W1, h and W2 rounded to
 *   bfloat16 (nearest even) with fp32 accumulation, as the Conv1d layers run
 *   under torch.autocast(dtype=torch.bfloat16); everything else is fp32.
 *   One pass: the MLP runs in the spectral block's row epilogue, so y1 never
 *   reaches memory.  Covered where fno_layer_is_fused says so (2D, 64
 *   channels, 32 hidden, a skip, the fused block's shapes); otherwise
 *   FNO_ERR_UNSUPPORTED, nothing enqueued (compose fno_spectral_block_f32 and
 *   fno_channel_mlp_f32).  Workspace: fno_spectral_block_workspace_bytes.
 */
int fno_layer_f32(const float* x, const void* w, const float* bias, const float* skip_weight,
                  const float* mlp_w1, const float* mlp_b1, const float* mlp_w2,
                  const float* mlp_b2, const float* gate_weight, const float* gate_bias, float* y,
                  int32_t batch, int32_t channels, int32_t hidden_channels, int32_t ndim,
                  const int32_t* sizes, const int32_t* modes, int32_t norm, int32_t skip_kind,
                  int32_t mlp_skip_kind, int32_t act, void* workspace, size_t workspace_bytes,
                  void* stream);
int fno_layer_is_fused(int32_t batch, int32_t channels, int32_t hidden_channels, int32_t ndim,
                       const int32_t* sizes, const int32_t* modes, int32_t skip_kind,
                       int32_t mlp_skip_kind);

/*
 * fno_layer_f32 with bfloat16 activation storage: x and y are bfloat16
 * [batch, channels, N_1, N_2] (16-byte aligned, not overlapping); the
 * arithmetic is fno_layer_f32's, on x widened exactly to fp32, and y is
 * rounded to bfloat16 (nearest even) at the store.  Replaces the same
 * reference layer (fno_block.py:331-379) in the bf16 FNO forward, where the
 * activations between layers are kept in bfloat16 (half the bytes of every
 * layer's reads and writes of the field).  Covered where
 * fno_layer_bf16_is_fused says so: fno_layer_is_fused's shapes with planes of
 * 64, 128 or 256 rows by 128 or 256 columns; otherwise FNO_ERR_UNSUPPORTED,
 * nothing enqueued.  Workspace and errors as fno_layer_f32.
 */
int fno_layer_bf16(const void* x, const void* w, const float* bias, const float* skip_weight,
                   const float* mlp_w1, const float* mlp_b1, const float* mlp_w2,
                   const float* mlp_b2, const float* gate_weight, const float* gate_bias, void* y,
                   int32_t batch, int32_t channels, int32_t hidden_channels, int32_t ndim,
                   const int32_t* sizes, const int32_t* modes, int32_t norm, int32_t skip_kind,
                   int32_t mlp_skip_kind, int32_t act, void* workspace, size_t workspace_bytes,
                   void* stream);
int fno_layer_bf16_is_fused(int32_t batch, int32_t channels, int32_t hidden_channels,
                            int32_t ndim, const int32_t* sizes, const int32_t* modes,
                            int32_t skip_kind, int32_t mlp_skip_kind);

/*
 * fno_spectral_block_f32 without a workspace argument and without any device
 * allocation.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, kernels and results as
 * fno_spectral_block_f32.
 *   - The scratch is a fixed device array of FNO_NOALLOC_SCRATCH_BYTES owned
 *     by the library; each GPU that runs this call holds its own copy until
 *     the process ends.
 *   - The batch runs in consecutive chunks whose workspace
 *     (fno_spectral_block_workspace_bytes) fits that array.  A shape whose
 *     single sample needs more returns FNO_ERR_UNSUPPORTED, nothing enqueued.
 *   - Calls on one GPU share the array.  Calls that overlap in time on one
 *     GPU (different streams or host threads) race; the caller serialises
 *     them.  Every scratch byte the kernels read is written earlier in the
 *     same call, so nothing needs clearing between calls.
 */
#define FNO_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int fno_spectral_block_f32_noalloc(const float* x, const void* w, const float* bias,
                                   const float* skip_weight, float* y, int32_t batch,
                                   int32_t in_channels, int32_t out_channels, int32_t ndim,
                                   const int32_t* sizes, const int32_t* modes, int32_t norm,
                                   int32_t skip_kind, int32_t act, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FNO_HIP_H */
