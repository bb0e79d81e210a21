// fno_spectral_block_f32_noalloc: the spectral block without a caller
// workspace and without any device allocation, for callers that cannot
// allocate (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc).  No counterpart in the reference.
//
// The scratch the block's kernels need (window spectra, the inverse column
// transform, the generic path's stage buffers) lives in one file-scope device
// array of FNO_NOALLOC_SCRATCH_BYTES.  Each GPU that runs this entry point
// holds its own copy of the array until the process ends.  In host code the
// array's name is only a host-side stand-in; its device address on the
// stream's device comes from hipGetSymbolAddress, taken once per device with
// that device current, and only that address is handed to the kernels.
//
// The batch runs in consecutive chunks whose workspace fits the array, so any
// batch size works; a shape whose single sample needs more than the array
// returns FNO_ERR_UNSUPPORTED before anything is enqueued.  Every scratch byte
// a kernel reads is written earlier in the same chunk, so the array needs no
// clearing between calls.  Calls on one GPU share the array: calls that
// overlap in time on one GPU (two streams, two host threads) race on it and
// must be serialised by the caller.
#include "fno_common.h"

#include <mutex>

namespace fno {
void clear_error();
int spectral_block_check(const void* x, const void* w, void* y, int32_t batch,
                         int32_t in_channels, int32_t out_channels, int32_t ndim,
                         const int32_t* sizes, const int32_t* modes, int32_t norm,
                         int32_t skip_kind, int32_t act, const float* skip_weight, size_t es);
int spectral_block_run(const float* x, const void* w, const float* bias, const float* skip_weight,
                       float* y, int32_t batch, int32_t in_channels, int32_t out_channels,
                       int32_t ndim, const int32_t* sizes, const int32_t* modes, int32_t norm,
                       int32_t skip_kind, int32_t act, void* workspace, size_t workspace_bytes,
                       hipStream_t st);
}  // namespace fno

extern "C" size_t fno_spectral_block_workspace_bytes(int32_t batch, int32_t in_channels,
                                                     int32_t out_channels, int32_t ndim,
                                                     const int32_t* sizes, const int32_t* modes);

using namespace fno;

static __device__ __align__(256) unsigned char scratch[FNO_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the device `stream` belongs to.
int scratch_address(hipStream_t stream, void** out) {
  int dev = -1;
  if (stream) {
    int rc = hip_status(hipStreamGetDevice(stream, &dev), "hipStreamGetDevice");
    if (rc) return rc;
  } else {
    int rc = hip_status(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("no-alloc spectral block: device index %d outside [0, %d)", dev, kMaxDevices);
    return FNO_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    int rc = hip_status(hipGetDevice(&cur), "hipGetDevice");
    if (rc) return rc;
    if (cur != dev) {
      rc = hip_status(hipSetDevice(dev), "hipSetDevice");
      if (rc) return rc;
    }
    void* p = nullptr;
    rc = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (cur != dev) {
      const int rc2 = hip_status(hipSetDevice(cur), "hipSetDevice");
      if (!rc) rc = rc2;
    }
    if (rc) return rc;
    if (!p) {
      set_error("no-alloc spectral block: hipGetSymbolAddress returned NULL");
      return FNO_ERR_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return FNO_OK;
}

}  // namespace

extern "C" {

int fno_spectral_block_f32_noalloc(const float* x, const void* w, const float* bias,
                                   const float* skip_weight, float* y, int32_t batch,
                                   int32_t in_channels, int32_t out_channels, int32_t ndim,
                                   const int32_t* sizes, const int32_t* modes, int32_t norm,
                                   int32_t skip_kind, int32_t act, void* stream) {
  clear_error();
  int rc = spectral_block_check(x, w, y, batch, in_channels, out_channels, ndim, sizes, modes, norm,
                                skip_kind, act, skip_weight, sizeof(float));
  if (rc) return rc;
  constexpr size_t cap = FNO_NOALLOC_SCRATCH_BYTES;
  const size_t one = fno_spectral_block_workspace_bytes(1, in_channels, out_channels, ndim, sizes,
                                                        modes);
  if (one == 0 || one > cap) {
    set_error("no-alloc spectral block: one sample needs %zu bytes of scratch, the fixed array "
              "holds %zu", one, cap);
    return FNO_ERR_UNSUPPORTED;
  }
  // largest chunk of samples whose workspace fits the array
  int32_t chunk = (int32_t)(cap / one < (size_t)batch ? cap / one : (size_t)batch);
  while (chunk > 1 && fno_spectral_block_workspace_bytes(chunk, in_channels, out_channels, ndim,
                                                         sizes, modes) > cap)
    --chunk;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  void* ws = nullptr;
  rc = scratch_address(st, &ws);
  if (rc) return rc;
  int64_t points = 1;
  for (int d = 0; d < ndim; ++d) points *= sizes[d];
  for (int32_t b0 = 0; b0 < batch; b0 += chunk) {
    const int32_t nb = batch - b0 < chunk ? batch - b0 : chunk;
    const size_t need = fno_spectral_block_workspace_bytes(nb, in_channels, out_channels, ndim,
                                                           sizes, modes);
    rc = spectral_block_run(x + (int64_t)b0 * in_channels * points, w, bias, skip_weight,
                            y + (int64_t)b0 * out_channels * points, nb, in_channels,
                            out_channels, ndim, sizes, modes, norm, skip_kind, act, ws, need, st);
    if (rc) return rc;
  }
  return FNO_OK;
}

}  // extern "C"
