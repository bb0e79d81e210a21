"""Tensor-level wrappers over the C ABI of libfnohip.so.

Every function takes CUDA (HIP) tensors, enqueues work on torch's current
stream and returns new tensors allocated by torch.  Inputs are made
contiguous float32 / complex64 first.  Nothing here computes on the CPU:
a CPU tensor or a missing library raises.
"""
from __future__ import annotations

import ctypes
import functools
from typing import Optional, Sequence

import torch

from . import _native as nat


def _require_gpu(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "neuraloperator_amd runs the FNO spectral path only on the GPU (HIP); "
                f"got a tensor on {t.device}")


def _ptr(t: Optional[torch.Tensor]):
    """Device address of a tensor's data for the C-ABI (an int, which the
    c_void_p arguments take as it is).  The kernels read the storage as it is,
    so a lazily conjugated or negated view (torch's conj / neg bits, which
    leave the storage untouched) must have been resolved."""
    if t is None:
        return None
    if t.is_conj() or t.is_neg():
        raise RuntimeError("internal: a conjugate / negative view reached the C-ABI unresolved")
    return t.data_ptr()


# torch's current stream of a device as the raw hipStream_t, without building
# a torch.cuda.Stream object per call (the public route below otherwise)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device):
    if _raw_stream is not None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(idx)
    return torch.cuda.current_stream(device).cuda_stream


def _workspace(nbytes: int, device):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def _f32(t):
    t = t if t.dtype == torch.float32 else t.float()
    return t.resolve_neg().contiguous()


def _c64(t):
    # resolve_conj: w.conj() is a view with the conjugate bit set over the
    # same storage, and .contiguous() keeps it so when the view is contiguous
    t = t if t.dtype == torch.complex64 else t.to(torch.complex64)
    return t.resolve_conj().resolve_neg().contiguous()


def rfft_window(x: torch.Tensor, modes: Sequence[int], fft_norm: str = "forward") -> torch.Tensor:
    """Kept-mode window of rfftn(x) in fftshift-ed window order.
    x [B, C, *S] -> complex64 [B, C, *modes]."""
    _require_gpu(x)
    lib = nat.load()
    x = _f32(x)
    B, C, *S = x.shape
    nd = len(S)
    planes = B * C
    out = torch.empty((B, C, *modes), dtype=torch.complex64, device=x.device)
    sz, md = nat.i32_array(S), nat.i32_array(modes)
    wsb = lib.fno_rfft_window_workspace_bytes(planes, nd, sz, md)
    ws = _workspace(wsb, x.device)
    nat.check(lib.fno_rfft_window_f32(_ptr(x), _ptr(out), planes, nd, sz, md, nat.NORMS[fft_norm],
                                      _ptr(ws), wsb, _stream(x.device)), "fno_rfft_window_f32")
    return out


def contract_dense(xhat: torch.Tensor, weight: torch.Tensor, separable: bool = False) -> torch.Tensor:
    """Mode-wise contraction of the window spectrum with a dense weight window."""
    _require_gpu(xhat, weight)
    lib = nat.load()
    xhat, weight = _c64(xhat), _c64(weight)
    B, Ci, *modes = xhat.shape
    Co = Ci if separable else weight.shape[1]
    M = 1
    for m in modes:
        M *= m
    out = torch.empty((B, Co, *modes), dtype=torch.complex64, device=xhat.device)
    nat.check(lib.fno_contract_dense_c64(_ptr(xhat), _ptr(weight), _ptr(out), B, Ci, Co, M,
                                         int(bool(separable)), _stream(xhat.device)),
              "fno_contract_dense_c64")
    return out


def contract_tucker(xhat: torch.Tensor, core: torch.Tensor, factors: Sequence[torch.Tensor]) -> torch.Tensor:
    """Tucker-factorized contraction; factors = [U_in, U_out, U_1..U_d] with
    the mode factors already cut to the window rows."""
    _require_gpu(xhat, core, *factors)
    lib = nat.load()
    xhat = _c64(xhat)
    core = _c64(core)
    factors = [_c64(f) for f in factors]
    B, Ci, *modes = xhat.shape
    nd = len(modes)
    Co = factors[1].shape[0]
    ranks = list(core.shape)
    out = torch.empty((B, Co, *modes), dtype=torch.complex64, device=xhat.device)
    fp = (ctypes.c_void_p * len(factors))(*[f.data_ptr() for f in factors])
    md, rk = nat.i32_array(modes), nat.i32_array(ranks)
    wsb = lib.fno_contract_tucker_workspace_bytes(B, nd, md, rk)
    ws = _workspace(wsb, xhat.device)
    nat.check(lib.fno_contract_tucker_c64(_ptr(xhat), _ptr(core), fp, rk, _ptr(out), B, Ci, Co, nd,
                                          md, _ptr(ws), wsb, _stream(xhat.device)),
              "fno_contract_tucker_c64")
    return out


def irfft_window(yhat: torch.Tensor, in_sizes: Sequence[int], out_sizes: Sequence[int],
                 bias: Optional[torch.Tensor] = None, fft_norm: str = "forward",
                 enforce_hermitian_symmetry: bool = True) -> torch.Tensor:
    """Real field of size out_sizes from a window spectrum (+ bias)."""
    _require_gpu(yhat, bias)
    lib = nat.load()
    yhat = _c64(yhat)
    B, C, *modes = yhat.shape
    nd = len(modes)
    y = torch.empty((B, C, *out_sizes), dtype=torch.float32, device=yhat.device)
    b = _f32(bias.reshape(-1)) if bias is not None else None
    isz, osz, md = nat.i32_array(in_sizes), nat.i32_array(out_sizes), nat.i32_array(modes)
    wsb = lib.fno_irfft_window_workspace_bytes(B * C, nd, osz, md)
    ws = _workspace(wsb, yhat.device)
    nat.check(lib.fno_irfft_window_f32(_ptr(yhat), _ptr(b), _ptr(y), B, C, nd, isz, osz, md,
                                       nat.NORMS[fft_norm], int(bool(enforce_hermitian_symmetry)),
                                       _ptr(ws), wsb, _stream(yhat.device)),
              "fno_irfft_window_f32")
    return y


def irfft_window_epilogue(yhat: torch.Tensor, sizes: Sequence[int], bias: Optional[torch.Tensor],
                          x: Optional[torch.Tensor], skip_kind: int,
                          skip_weight: Optional[torch.Tensor], act: int,
                          fft_norm: str = "forward") -> torch.Tensor:
    """act(irfft(yhat) + bias + skip(x)) on the input grid (see
    fno_irfft_window_epilogue_f32)."""
    _require_gpu(yhat, bias, x, skip_weight)
    lib = nat.load()
    yhat = _c64(yhat)
    B, Co, *modes = yhat.shape
    nd = len(modes)
    xx = _f32(x) if x is not None else None
    Ci = xx.shape[1] if xx is not None else Co
    y = torch.empty((B, Co, *sizes), dtype=torch.float32, device=yhat.device)
    b = _f32(bias.reshape(-1)) if bias is not None else None
    w = _f32(skip_weight.reshape(-1)) if skip_weight is not None else None
    sz, md = nat.i32_array(sizes), nat.i32_array(modes)
    wsb = lib.fno_irfft_window_workspace_bytes(B * Co, nd, sz, md)
    ws = _workspace(wsb, yhat.device)
    nat.check(lib.fno_irfft_window_epilogue_f32(_ptr(yhat), _ptr(b), _ptr(xx), _ptr(w), _ptr(y), B,
                                                Ci, Co, nd, sz, md, nat.NORMS[fft_norm], skip_kind,
                                                act, _ptr(ws), wsb, _stream(yhat.device)),
              "fno_irfft_window_epilogue_f32")
    return y


def fft_window(x: torch.Tensor, modes: Sequence[int], fft_norm: str = "forward") -> torch.Tensor:
    """Kept-mode window of fftn(x) for complex data (see fno_fft_window_c64).
    x complex [B, C, *S] -> complex64 [B, C, *modes]."""
    _require_gpu(x)
    lib = nat.load()
    x = _c64(x)
    B, C, *S = x.shape
    nd = len(S)
    out = torch.empty((B, C, *modes), dtype=torch.complex64, device=x.device)
    sz, md = nat.i32_array(S), nat.i32_array(modes)
    wsb = lib.fno_fft_window_workspace_bytes(B * C, nd, sz, md)
    ws = _workspace(wsb, x.device)
    nat.check(lib.fno_fft_window_c64(_ptr(x), _ptr(out), B * C, nd, sz, md, nat.NORMS[fft_norm],
                                     _ptr(ws), wsb, _stream(x.device)), "fno_fft_window_c64")
    return out


def ifft_window(yhat: torch.Tensor, in_sizes: Sequence[int], out_sizes: Sequence[int],
                bias: Optional[torch.Tensor] = None, fft_norm: str = "forward") -> torch.Tensor:
    """Complex field of size out_sizes from a complex-data window (+ bias on
    the real part)."""
    _require_gpu(yhat, bias)
    lib = nat.load()
    yhat = _c64(yhat)
    B, C, *modes = yhat.shape
    nd = len(modes)
    y = torch.empty((B, C, *out_sizes), dtype=torch.complex64, device=yhat.device)
    b = _f32(bias.reshape(-1)) if bias is not None else None
    isz, osz, md = nat.i32_array(in_sizes), nat.i32_array(out_sizes), nat.i32_array(modes)
    wsb = lib.fno_ifft_window_workspace_bytes(B * C, nd, osz, md)
    ws = _workspace(wsb, yhat.device)
    nat.check(lib.fno_ifft_window_c64(_ptr(yhat), _ptr(b), _ptr(y), B, C, nd, isz, osz, md,
                                      nat.NORMS[fft_norm], _ptr(ws), wsb, _stream(yhat.device)),
              "fno_ifft_window_c64")
    return y


def block_epilogue(spec: torch.Tensor, x: Optional[torch.Tensor], skip_kind: int,
                   skip_weight: Optional[torch.Tensor], act: int, out: Optional[torch.Tensor] = None):
    """act(spec + skip(x)); writes into ``out`` (default: spec itself)."""
    _require_gpu(spec, x, skip_weight)
    lib = nat.load()
    spec = _f32(spec)
    y = spec if out is None else out
    B, Co, *S = spec.shape
    Ci = x.shape[1] if x is not None else Co
    P = 1
    for s in S:
        P *= s
    xx = _f32(x) if x is not None else None
    w = _f32(skip_weight.reshape(-1)) if skip_weight is not None else None
    nat.check(lib.fno_block_epilogue_f32(_ptr(spec), _ptr(xx), _ptr(w), _ptr(y), B, Ci, Co, P,
                                         skip_kind, act, _stream(spec.device)),
              "fno_block_epilogue_f32")
    return y


def channel_mlp_is_supported(Ci: int, Ch: int, Co: int, P: int, *tensors) -> bool:
    """Widths and point count the kernel covers; tensors passed here must
    also start on a 16-byte boundary (its vector accesses)."""
    if any(t is not None and t.data_ptr() % 16 for t in tensors):
        return False
    return bool(nat.load().fno_channel_mlp_is_supported(Ci, Ch, Co, P))


def autocast_bf16(device_type: str = "cuda") -> bool:
    """True inside torch.autocast(device_type, dtype=torch.bfloat16), where
    torch runs Conv1d on bf16 operands with fp32 accumulation."""
    return (torch.is_autocast_enabled(device_type)
            and torch.get_autocast_dtype(device_type) == torch.bfloat16)


def channel_mlp(x: torch.Tensor, w1: torch.Tensor, b1: Optional[torch.Tensor], w2: torch.Tensor,
                b2: Optional[torch.Tensor], skip_kind: int = nat.SKIP_NONE,
                skip_x: Optional[torch.Tensor] = None, skip_weight: Optional[torch.Tensor] = None,
                skip_bias: Optional[torch.Tensor] = None, act: int = nat.ACT_NONE,
                out: Optional[torch.Tensor] = None, bf16_products: bool = False) -> torch.Tensor:
    """act(W2 gelu(W1 x + b1) + b2 + skip(skip_x)) over x [B, Ci, *S]
    (ChannelMLP.forward with two layers, channel_mlp.py:82-119, plus the
    channel-MLP skip and second activation of fno_block.py:363-379).
    bf16_products: both 1x1 layers on bf16-rounded operands with fp32
    accumulation (Conv1d under a bf16 autocast); the output stays fp32."""
    _require_gpu(x, w1, w2, skip_x)
    lib = nat.load()
    B, Ci, *S = x.shape
    P = 1
    for s in S:
        P *= s
    Ch, Co = w1.shape[0], w2.shape[0]
    xx = _f32(x)
    y = torch.empty((B, Co, *S), dtype=torch.float32, device=x.device) if out is None else out
    sx = _f32(skip_x) if skip_x is not None else None
    # flattened operands held in locals until the launch is enqueued
    w1f, b1f, w2f, b2f, swf, sbf = (_f32(t.reshape(-1)) if t is not None else None
                                    for t in (w1, b1, w2, b2, skip_weight, skip_bias))
    nat.check(lib.fno_channel_mlp_f32(_ptr(xx), _ptr(w1f), _ptr(b1f), _ptr(w2f), _ptr(b2f), _ptr(sx),
                                      _ptr(swf), _ptr(sbf), _ptr(y), B, Ci, Ch, Co, P, skip_kind,
                                      act, int(bool(bf16_products)), _stream(x.device)),
              "fno_channel_mlp_f32")
    return y


def spectral_block_is_fused(B, Ci, Co, sizes, modes, skip_kind) -> bool:
    lib = nat.load()
    return bool(lib.fno_spectral_block_is_fused(B, Ci, Co, len(sizes), nat.i32_array(sizes),
                                                nat.i32_array(modes), skip_kind))


@functools.lru_cache(maxsize=256)
def _block_shape(B, Ci, Co, sizes, modes):
    """The C-ABI size / mode arrays and the workspace size of a block shape
    (read-only arrays, so one copy serves every call of that shape)."""
    sz, md = nat.i32_array(sizes), nat.i32_array(modes)
    return sz, md, nat.load().fno_spectral_block_workspace_bytes(B, Ci, Co, len(sizes), sz, md)


def spectral_block(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
                   modes: Sequence[int], skip_kind: int = nat.SKIP_NONE,
                   skip_weight: Optional[torch.Tensor] = None, act: int = nat.ACT_NONE,
                   fft_norm: str = "forward", out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = act(SpectralConv(x) + skip(x)), output size == input size, dense
    weight window [Ci, Co, *modes]."""
    _require_gpu(x, weight, bias, skip_weight)
    lib = nat.load()
    x = _f32(x)
    weight = _c64(weight)
    B, Ci, *S = x.shape
    Co = weight.shape[1]
    nd = len(S)
    y = out if out is not None else torch.empty((B, Co, *S), dtype=torch.float32, device=x.device)
    b = _f32(bias.reshape(-1)) if bias is not None else None
    w = _f32(skip_weight.reshape(-1)) if skip_weight is not None else None
    sz, md, wsb = _block_shape(B, Ci, Co, tuple(S), tuple(int(m) for m in modes))
    ws = _workspace(wsb, x.device)
    nat.check(lib.fno_spectral_block_f32(_ptr(x), _ptr(weight), _ptr(b), _ptr(w), _ptr(y), B, Ci, Co,
                                         nd, sz, md, nat.NORMS[fft_norm], skip_kind, act, _ptr(ws),
                                         wsb, _stream(x.device)),
              "fno_spectral_block_f32")
    return y


def channel_mlp_io_is_supported(Ci, Ch, Co, P, x_bf16: bool, y_bf16: bool) -> bool:
    lib = nat.load()
    return bool(lib.fno_channel_mlp_io_is_supported(Ci, Ch, Co, P, int(x_bf16), int(y_bf16)))


def channel_mlp_io(x: torch.Tensor, w1: torch.Tensor, b1: Optional[torch.Tensor], w2: torch.Tensor,
                   b2: Optional[torch.Tensor], act: int, y_bf16: bool) -> torch.Tensor:
    """act(W2 gelu(W1 x + b1) + b2) with bf16 products (fno_channel_mlp_io):
    x is read as stored (bfloat16 or float32), y is bfloat16 when y_bf16 —
    the lifting and projection of the bf16 FNO forward."""
    _require_gpu(x, w1, w2)
    lib = nat.load()
    x_bf16 = x.dtype == torch.bfloat16
    x = x.contiguous() if x_bf16 else _f32(x)
    B, Ci, *S = x.shape
    P = 1
    for s_ in S:
        P *= s_
    Ch, Co = w1.shape[0], w2.shape[0]
    y = torch.empty((B, Co, *S), dtype=torch.bfloat16 if y_bf16 else torch.float32,
                    device=x.device)
    w1f, b1f, w2f, b2f = (_f32(t.reshape(-1)) if t is not None else None for t in (w1, b1, w2, b2))
    nat.check(lib.fno_channel_mlp_io(_ptr(x), _ptr(w1f), _ptr(b1f), _ptr(w2f), _ptr(b2f), _ptr(y), B,
                                     Ci, Ch, Co, P, act, int(x_bf16), int(bool(y_bf16)),
                                     _stream(x.device)),
              "fno_channel_mlp_io")
    return y


def layer_is_fused(B, C, hidden, sizes, modes, skip_kind, mlp_skip_kind, bf16=False) -> bool:
    """Shapes fno_layer_f32 (bf16: fno_layer_bf16) covers."""
    lib = nat.load()
    fn = lib.fno_layer_bf16_is_fused if bf16 else lib.fno_layer_is_fused
    return bool(fn(B, C, hidden, len(sizes), nat.i32_array(sizes), nat.i32_array(modes), skip_kind,
                   mlp_skip_kind))


def fno_layer(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
              modes: Sequence[int], skip_kind: int, skip_weight: Optional[torch.Tensor],
              w1: torch.Tensor, b1: Optional[torch.Tensor], w2: torch.Tensor,
              b2: Optional[torch.Tensor], mlp_skip_kind: int, gate_weight: Optional[torch.Tensor],
              gate_bias: Optional[torch.Tensor], act: int, fft_norm: str = "forward") -> torch.Tensor:
    """One FNO layer in one pass (fno_layer_f32): act(W2 gelu(W1 y1 + b1) +
    b2 + mlp_skip(x)) with y1 = act(SpectralConv(x) + skip(x)); the MLP
    products on bf16-rounded operands (the autocast forward).  A bfloat16 x
    runs fno_layer_bf16 and gives a bfloat16 y (activation storage of the
    bf16 FNO forward)."""
    _require_gpu(x, weight, bias, skip_weight, w1, w2, gate_weight)
    lib = nat.load()
    bf = x.dtype == torch.bfloat16
    x = x.contiguous() if bf else _f32(x)
    weight = _c64(weight)
    B, C, *S = x.shape
    nd = len(S)
    hidden = w1.shape[0]
    y = torch.empty((B, C, *S), dtype=x.dtype, device=x.device)
    flat = [(_f32(t.reshape(-1)) if t is not None else None)
            for t in (bias, skip_weight, w1, b1, w2, b2, gate_weight, gate_bias)]
    b, sw, w1f, b1f, w2f, b2f, gw, gb = flat
    sz, md = nat.i32_array(S), nat.i32_array(modes)
    wsb = lib.fno_spectral_block_workspace_bytes(B, C, C, nd, sz, md)
    ws = _workspace(wsb, x.device)
    fn = lib.fno_layer_bf16 if bf else lib.fno_layer_f32
    nat.check(fn(_ptr(x), _ptr(weight), _ptr(b), _ptr(sw), _ptr(w1f), _ptr(b1f), _ptr(w2f),
                 _ptr(b2f), _ptr(gw), _ptr(gb), _ptr(y), B, C, hidden, nd, sz, md,
                 nat.NORMS[fft_norm], skip_kind, mlp_skip_kind, act, _ptr(ws), wsb,
                 _stream(x.device)),
              "fno_layer_bf16" if bf else "fno_layer_f32")
    return y
