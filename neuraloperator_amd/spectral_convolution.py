"""SpectralConv on MI355X: same module API as neuralop's SpectralConv
(neuralop/layers/spectral_convolution.py:183-570), forward computed by the
HIP kernels of libfnohip.so.

Forward dispatch (all on the GPU, nothing in torch.fft):
  * dense / reconstructed weight, output size == input size
        -> fno_spectral_block_f32 (fused 2D FFT path when the plane allows it,
           generic window transforms otherwise)
  * output_shape / resolution_scaling_factor, separable, or a Tucker weight
    contracted through its factors ('factorized')
        -> fno_rfft_window_f32 -> contraction -> fno_irfft_window_f32
CP / TT weights are reconstructed (torch ops on the weight only) and then
contracted densely; the result is the same mathematics as the reference's
factor-wise einsums (spectral_convolution.py:55-73, :106-132).

complex_data=True runs fno_fft_window_c64 -> contraction -> fno_ifft_window_c64.

Autograd: when gradients are required (training), the forward runs as
_SpectralConvFn, whose backward is built from the same library calls (window
transforms under the dual norm and the mode-wise contraction), for dense and
separable weights and for outputs on the input grid or resized; a factorized
weight gets its gradient through the torch reconstruction of its dense
window; complex_data=True likewise.
"""
from __future__ import annotations

import math

from typing import List, Optional, Tuple, Union

import torch
from torch import nn

from . import _native as nat
from . import functional as Fh
from .factorized_tensors import DenseTensor, FactorizedTensor, TuckerTensor, _TuckerView
from .resample import resample
from .utils import get_active_profiler, maybe_profile, validate_scaling_factor

Number = Union[int, float]


class BaseSpectralConv(nn.Module):
    """Abstract base (neuralop/layers/base_spectral_conv.py:4-27)."""

    def __init__(self, device=None, dtype=None):
        super().__init__()
        self.dtype = dtype
        self.device = device

    def transform(self, x):
        return x


def get_contract_fun(weight, implementation="reconstructed", separable=False):
    """Validates the implementation / factorization pair the way
    spectral_convolution.py:135-177 does and names the contraction used."""
    if implementation == "reconstructed":
        return "dense_separable" if separable else "dense"
    if implementation == "factorized":
        if torch.is_tensor(weight):
            return "dense"
        if isinstance(weight, FactorizedTensor):
            name = weight.name.lower()
            if name.endswith("dense"):
                return "dense"
            if name.endswith("tucker"):
                return "tucker"
            if name.endswith("tt"):
                return "tt"
            if name.endswith("cp"):
                return "cp"
            raise ValueError(f"Got unexpected factorized weight type {weight.name}")
        raise ValueError(f"Got unexpected weight type of class {weight.__class__.__name__}")
    raise ValueError(
        f'Got implementation={implementation}, expected "reconstructed" or "factorized"')


class _NoGradThroughHip(torch.autograd.Function):
    """Attaches the result of a forward-only fused kernel (spectral block with
    skip / activation, fused channel MLP) to the graph with a backward that
    raises.  The modules take those kernels only when no gradient is needed;
    with gradients they run their autograd paths."""

    @staticmethod
    def forward(ctx, y, *inputs):
        return y

    @staticmethod
    def backward(ctx, *grads):
        raise NotImplementedError(
            "this fused forward kernel has no backward; call the module with gradients "
            "enabled so that it takes its autograd path")


_DUAL_NORM = {"forward": "backward", "backward": "forward", "ortho": "ortho"}


def _hermitian_weights(m_last: int, n_last: int, ndim: int, device) -> torch.Tensor:
    """c_k of the real inverse transform along the last axis: 1 for bin 0 and
    the Nyquist bin, 2 for the bins that stand for a conjugate pair."""
    c = torch.full((m_last,), 2.0, device=device)
    c[0] = 1.0
    if n_last % 2 == 0 and n_last // 2 < m_last:
        c[n_last // 2] = 1.0
    return c.view(*([1] * (ndim + 1)), m_last)


def _landing_index(kept: List[int], in_sizes: List[int], out_sizes: List[int], device):
    """Where each kept window mode lands in the output grid's rfft layout.

    The reference's inverse (spectral_convolution.py:531-564) places the
    window in the input grid's spectrum (non-last axes centred, frequency
    q - m//2 at window position q; last axis bins 0..m-1), ifftshifts, and
    lets ifftn(s=out) / irfft(n=out) trim or zero-pad every axis at its end:
    a mode at standard index i of axis d survives when i < N'_d (last axis:
    i < N'_last//2 + 1) and then meets the output basis e^{2 pi i i n / N'_d}.
    Returns, per axis, the position of that index in the output grid's full
    window (non-last axes in the same centred order) and a mask of the modes
    that survive."""
    nd = len(kept)
    pos, mask = [], []
    for d in range(nd):
        q = torch.arange(kept[d], device=device)
        if d < nd - 1:
            i = (q - kept[d] // 2) % in_sizes[d]
            ok = i < out_sizes[d]
            p = (i + out_sizes[d] // 2) % out_sizes[d]
        else:
            ok = q < out_sizes[d] // 2 + 1
            p = torch.where(ok, q, torch.zeros_like(q))
        pos.append(torch.where(ok, p, torch.zeros_like(p)))
        mask.append(ok)
    return pos, mask


def _inverse_adjoint(gy: torch.Tensor, kept: List[int], in_sizes: List[int],
                     out_sizes: List[int], dual: str, enforce: bool = True) -> torch.Tensor:
    """Adjoint of the window inverse (window spectrum [B, C, *kept] ->
    real field [B, C, *out_sizes]): the output grid's forward transform of gy
    under the dual norm (so it carries the inverse's scaling), read at the
    output index of every surviving mode, times the output grid's Hermitian
    weight of its last-axis bin; modes that do not survive get zero.

    With enforce_hermitian_symmetry and an even output length the reference
    zeroes the imaginary part of the input grid's last rfft bin N//2 after
    the non-last inverse transforms (spectral_convolution.py:555-556).  On a
    resized grid that bin is not the output Nyquist bin, so the output sees
    only the real part of that column: its adjoint keeps the Hermitian-even
    part over the non-last output frequencies, (G[j] + conj(G[-j])) / 2 (the
    real part in 1D).  On the input grid it is the Nyquist bin, whose
    imaginary part the real inverse ignores anyway."""
    nd = len(kept)
    if list(out_sizes) == list(in_sizes):
        c = _hermitian_weights(kept[-1], out_sizes[-1], nd, gy.device)
        return Fh.rfft_window(gy, kept, dual) * c
    full = list(out_sizes[:-1]) + [out_sizes[-1] // 2 + 1]
    G = Fh.rfft_window(gy, full, dual)                      # [B, C, *full]
    bz = in_sizes[-1] // 2
    if enforce and out_sizes[-1] % 2 == 0 and bz < kept[-1] and bz < full[-1]:
        col = G[..., bz]
        neg = []
        for d in range(nd - 1):
            n = out_sizes[d]
            p = torch.arange(n, device=gy.device)
            j = (p - n // 2) % n                             # standard index at position p
            neg.append(((-j) % n + n // 2) % n)              # position of -j
        flipped = col[(slice(None), slice(None)) + tuple(torch.meshgrid(*neg, indexing="ij"))] \
            if nd > 1 else col
        G = G.clone()
        G[..., bz] = 0.5 * (col + flipped.conj())
    pos, mask = _landing_index(kept, in_sizes, out_sizes, gy.device)
    idx = torch.meshgrid(*pos, indexing="ij")
    ok = torch.ones((), dtype=torch.bool, device=gy.device)
    for d, m in enumerate(mask):
        ok = ok & m.view(*([1] * d), -1, *([1] * (nd - d - 1)))
    gY = G[(slice(None), slice(None)) + tuple(idx)]
    c = _hermitian_weights(kept[-1], out_sizes[-1], nd, gy.device)
    return torch.where(ok, gY * c, torch.zeros((), dtype=gY.dtype, device=gy.device))


class _SpectralConvFn(torch.autograd.Function):
    """Spectral convolution y = s_i I(W . s_f F(x)) + bias with the gradients
    of SpectralConv.forward (spectral_convolution.py:417-570), dense or
    separable (_contract_dense / _contract_dense_separable, :25-52), output on
    the input grid or resized (output_shape / resolution_scaling_factor,
    :524-528).  With F the window of the forward transform (bins e^{-i
    phi_k(n)}) and I the real inverse onto the output grid (y = sum_k c'_k
    Re(Y_k e^{i phi'_k(n')}), c' = 2 for bins that stand for a conjugate pair
    of the output grid, modes the output grid trims away dropped):

        gY = I^H gy  (_inverse_adjoint)      gX = gY . conj(W)^T   (gY * conj(W))
        gW = conj(X)^T . gY  (sum_b conj(X) gY)
        gx = s_f Re(sum_k gX_k e^{i phi_k}) = s_f I_unscaled(gX / c_k)

    (separable forms in brackets), so both transforms are the library's own
    window transforms under the dual norm (forward <-> backward scaling) and
    the dense contractions its mode-wise contraction; the separable weight
    gradient is a batch sum of window-sized products."""

    @staticmethod
    def forward(ctx, x, w, bias, kept, fft_norm, out_sizes=None, separable=False, enforce=True):
        sizes = list(x.shape[2:])
        out_sizes = sizes if out_sizes is None else list(out_sizes)
        b = bias.reshape(-1) if bias is not None else None
        if out_sizes == sizes and not separable:
            y = Fh.spectral_block(x, w, b, kept, nat.SKIP_NONE, None, nat.ACT_NONE, fft_norm)
        else:
            xhat = Fh.rfft_window(x, kept, fft_norm)
            yhat = Fh.contract_dense(xhat, w, separable=separable)
            y = Fh.irfft_window(yhat, sizes, out_sizes, b, fft_norm, enforce)
        ctx.save_for_backward(x, w)
        ctx.kept, ctx.fft_norm, ctx.sizes, ctx.out_sizes = list(kept), fft_norm, sizes, out_sizes
        ctx.separable, ctx.enforce = bool(separable), bool(enforce)
        ctx.bias_shape = None if bias is None else bias.shape
        return y

    @staticmethod
    def backward(ctx, gy):
        x, w = ctx.saved_tensors
        kept, norm, sizes = ctx.kept, ctx.fft_norm, ctx.sizes
        gy = gy.contiguous().float()
        dual = _DUAL_NORM[norm]
        same_dense = ctx.out_sizes == sizes and not ctx.separable
        gY = None
        if ctx.needs_input_grad[1] or (ctx.needs_input_grad[0] and not same_dense):
            gY = _inverse_adjoint(gy, kept, sizes, ctx.out_sizes, dual, ctx.enforce)
        gx = gw = gb = None
        if ctx.needs_input_grad[0] and same_dense:
            # on the input grid the Hermitian weights cancel (gX / c with gY =
            # c . F_dual gy), so gx = I_dual(conj(W)^T . F_dual gy) is the
            # spectral block itself with the transposed conjugate weight and the
            # dual norm: one call of the fused forward kernels
            wt = w.conj().transpose(0, 1).contiguous()              # [Co, Ci, *m]
            gx = Fh.spectral_block(gy, wt, None, kept, nat.SKIP_NONE, None, nat.ACT_NONE, dual)
        elif ctx.needs_input_grad[0]:
            if ctx.separable:
                gX = Fh.contract_dense(gY.contiguous(), w.conj().contiguous(), separable=True)
            else:
                wt = w.conj().transpose(0, 1).contiguous()          # [Co, Ci, *m]
                gX = Fh.contract_dense(gY.contiguous(), wt)         # [B, Ci, *m]
            c = _hermitian_weights(kept[-1], sizes[-1], len(sizes), gy.device)
            gx = Fh.irfft_window(gX / c, sizes, sizes, None, dual, False)
        if ctx.needs_input_grad[1]:
            X = Fh.rfft_window(x, kept, norm)                       # [B, Ci, *m]
            if ctx.separable:
                gw = (X.conj() * gY).sum(dim=0)                     # [C, *m]
            else:
                xt = X.conj().transpose(0, 1).contiguous()          # [Ci, B, *m]
                gw = Fh.contract_dense(xt, gY.contiguous())         # [Ci, Co, *m]
        if ctx.bias_shape is not None and ctx.needs_input_grad[2]:
            dims = [0] + list(range(2, gy.ndim))
            gb = gy.sum(dim=dims).reshape(ctx.bias_shape)
        return gx, gw, gb, None, None, None, None, None


def _last_axis_phase(n: int, ndim: int, device) -> torch.Tensor:
    """psi_t = exp(-2 pi i (n//2) t / n) along the last axis (1 in 1D): the
    complex-data forward window takes last-axis frequencies j - n//2 and the
    inverse puts them back at j (spectral_convolution.py:448-449, :531-538),
    so each transform's adjoint is the other library transform times psi."""
    if ndim == 1:
        return torch.ones(n, dtype=torch.complex64, device=device)
    t = torch.arange(n, dtype=torch.float64, device=device)
    return torch.polar(torch.ones_like(t), -2.0 * math.pi * (n // 2) * t / n).to(torch.complex64)


def _complex_inverse_adjoint(gy: torch.Tensor, kept: List[int], in_sizes: List[int],
                             out_sizes: List[int], dual: str) -> torch.Tensor:
    """Adjoint of the complex-data window inverse onto a resized grid
    (spectral_convolution.py:531-538: ifftshift of the non-last axes when
    there are several, then ifftn(s=out), which trims or zero-pads each axis
    at its end).  On a non-last axis the window's position q sits at shifted
    position N//2 - m//2 + q, i.e. at standard index i = (q - m//2) mod N; on
    the last axis (sliced [:m] and never shifted back) at i = q.  A mode
    survives when i < N'_d and meets the output basis e^{2 pi i i n / N'_d}.
    The adjoint reads the output grid's full forward window of gy under the
    dual norm (every axis centred when there are several, none in 1D) at
    those indices; modes that do not survive get zero."""
    nd = len(kept)
    G = Fh.fft_window(gy, list(out_sizes), dual)            # [B, C, *out_sizes]
    pos, oks = [], []
    for d in range(nd):
        n, n2, m = in_sizes[d], out_sizes[d], kept[d]
        q = torch.arange(m, device=gy.device)
        i = (q - m // 2) % n if d < nd - 1 else q
        p = (i + n2 // 2) % n2 if nd > 1 else i
        ok = i < n2
        pos.append(torch.where(ok, p, torch.zeros_like(p)))
        oks.append(ok)
    ok = torch.ones((), dtype=torch.bool, device=gy.device)
    for d, m in enumerate(oks):
        ok = ok & m.view(*([1] * d), -1, *([1] * (nd - d - 1)))
    gY = G[(slice(None), slice(None)) + tuple(torch.meshgrid(*pos, indexing="ij"))]
    return torch.where(ok, gY, torch.zeros((), dtype=gY.dtype, device=gy.device))


class _SpectralConvComplexFn(torch.autograd.Function):
    """complex_data=True spectral convolution y = I(W . F(x)) + bias with
    its gradients, dense or separable, output on the input grid or resized.
    F (windowed fftn) and I (zero-filled ifftn) are C-linear, so with psi from
    _last_axis_phase and the dual norm:

        gY = I^H gy = F_dual(gy . psi)  (resized: _complex_inverse_adjoint)
        gX = gY . conj(W)^T  (gY * conj(W))      gW = conj(X)^T . gY  (sum_b conj(X) gY)
        gx = F^H gX = I_dual(gX) . psi           gbias = sum Re(gy)
    (separable forms in brackets; the real bias is added to the real part)"""

    @staticmethod
    def forward(ctx, x, w, bias, kept, fft_norm, out_sizes=None, separable=False):
        sizes = list(x.shape[2:])
        out_sizes = sizes if out_sizes is None else list(out_sizes)
        xhat = Fh.fft_window(x, kept, fft_norm)
        yhat = Fh.contract_dense(xhat, w, separable=separable)
        b = bias.reshape(-1) if bias is not None else None
        y = Fh.ifft_window(yhat, sizes, out_sizes, b, fft_norm)
        ctx.save_for_backward(xhat, w)
        ctx.kept, ctx.fft_norm, ctx.sizes, ctx.out_sizes = list(kept), fft_norm, sizes, out_sizes
        ctx.separable = bool(separable)
        ctx.bias_shape = None if bias is None else bias.shape
        return y

    @staticmethod
    def backward(ctx, gy):
        xhat, w = ctx.saved_tensors
        kept, sizes = ctx.kept, ctx.sizes
        dual = _DUAL_NORM[ctx.fft_norm]
        gy = gy.contiguous().to(torch.complex64)
        psi = _last_axis_phase(sizes[-1], len(sizes), gy.device)
        if ctx.out_sizes == sizes:
            gY = Fh.fft_window((gy * psi).contiguous(), kept, dual)      # [B, Co, *m]
        else:
            gY = _complex_inverse_adjoint(gy, kept, sizes, ctx.out_sizes, dual)
        gx = gw = gb = None
        if ctx.needs_input_grad[0]:
            if ctx.separable:
                gX = Fh.contract_dense(gY.contiguous(), w.conj().contiguous(), separable=True)
            else:
                wt = w.conj().transpose(0, 1).contiguous()               # [Co, Ci, *m]
                gX = Fh.contract_dense(gY.contiguous(), wt)              # [B, Ci, *m]
            gx = Fh.ifft_window(gX, sizes, sizes, None, dual) * psi
        if ctx.needs_input_grad[1]:
            if ctx.separable:
                gw = (xhat.conj() * gY).sum(dim=0)                       # [C, *m]
            else:
                xt = xhat.conj().transpose(0, 1).contiguous()            # [Ci, B, *m]
                gw = Fh.contract_dense(xt, gY.contiguous())              # [Ci, Co, *m]
        if ctx.bias_shape is not None and ctx.needs_input_grad[2]:
            dims = [0] + list(range(2, gy.ndim))
            gb = gy.real.sum(dim=dims).reshape(ctx.bias_shape)
        return gx, gw, gb, None, None, None, None


def _fp16_round(t: torch.Tensor) -> torch.Tensor:
    """Round to float16 (nearest even) and widen back; complex part by part."""
    if t.is_complex():
        return torch.complex(_fp16_round(t.real), _fp16_round(t.imag))
    return t.half().float()


def _attach(y, *params):
    if torch.is_grad_enabled() and any(p is not None and p.requires_grad for p in params):
        return _NoGradThroughHip.apply(y, *[p for p in params if p is not None])
    return y


class SpectralConv(BaseSpectralConv):
    """Spectral convolution of an FNO layer; constructor and attributes as in
    neuralop/layers/spectral_convolution.py:285-381."""

    def __init__(
        self,
        in_channels,
        out_channels,
        n_modes,
        complex_data=False,
        max_n_modes=None,
        bias=True,
        separable=False,
        resolution_scaling_factor: Optional[Union[Number, List[Number]]] = None,
        fno_block_precision="full",
        rank=1.0,
        factorization=None,
        implementation="reconstructed",
        enforce_hermitian_symmetry=True,
        fixed_rank_modes=False,
        decomposition_kwargs: Optional[dict] = None,
        init_std="auto",
        fft_norm="forward",
        device=None,
    ):
        super().__init__(device=device)
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.complex_data = complex_data
        self.n_modes = n_modes
        self.order = len(self.n_modes)
        if max_n_modes is None:
            max_n_modes = self.n_modes
        elif isinstance(max_n_modes, int):
            max_n_modes = [max_n_modes]
        self.max_n_modes = max_n_modes
        self.fno_block_precision = fno_block_precision
        self.rank = rank
        self.factorization = factorization
        self.implementation = implementation
        self.enforce_hermitian_symmetry = enforce_hermitian_symmetry
        self.resolution_scaling_factor = validate_scaling_factor(resolution_scaling_factor, self.order)
        if init_std == "auto":
            init_std = (2 / (in_channels + out_channels)) ** 0.5
        if isinstance(fixed_rank_modes, bool):
            fixed_rank_modes = [0] if fixed_rank_modes else None
        if fft_norm not in nat.NORMS:
            raise ValueError(f"fft_norm must be one of {sorted(nat.NORMS)}, got {fft_norm}")
        self.fft_norm = fft_norm
        if factorization is None:
            factorization = "Dense"
        if separable:
            if in_channels != out_channels:
                raise ValueError(
                    "To use separable Fourier Conv, in_channels must be equal "
                    f"to out_channels, but got in_channels={in_channels} and "
                    f"out_channels={out_channels}")
            weight_shape = (in_channels, *max_n_modes)
        else:
            weight_shape = (in_channels, out_channels, *max_n_modes)
        self.separable = separable
        tensor_kwargs = decomposition_kwargs if decomposition_kwargs is not None else {}
        self.weight = FactorizedTensor.new(weight_shape, rank=self.rank, factorization=factorization,
                                           fixed_rank_modes=fixed_rank_modes, dtype=torch.cfloat,
                                           **tensor_kwargs)
        self.weight.normal_(0, init_std)
        self._contract = get_contract_fun(self.weight, implementation=implementation,
                                          separable=separable)
        if bias:
            self.bias = nn.Parameter(init_std * torch.randn(*((self.out_channels,) + (1,) * self.order)))
        else:
            self.bias = None
        if device is not None:
            self.to(device)

    # ---------------------------------------------------------------- API
    def transform(self, x, output_shape=None):
        """Resample the skip input to the output resolution (:383-398)."""
        in_shape = list(x.shape[2:])
        if self.resolution_scaling_factor is not None and output_shape is None:
            out_shape = [round(s * r) for s, r in zip(in_shape, self.resolution_scaling_factor)]
        elif output_shape is not None:
            out_shape = list(output_shape)
        else:
            out_shape = in_shape
        if in_shape == out_shape:
            return x
        return resample(x, 1.0, list(range(2, x.ndim)), output_shape=out_shape)

    @property
    def n_modes(self):
        return self._n_modes

    @n_modes.setter
    def n_modes(self, n_modes):
        """Last entry becomes n//2+1 for real data (:404-415)."""
        if isinstance(n_modes, int):
            n_modes = [n_modes]
        else:
            n_modes = list(n_modes)
        if not self.complex_data:
            n_modes[-1] = n_modes[-1] // 2 + 1
        self._n_modes = n_modes

    # ------------------------------------------------------ window bookkeeping
    def window(self, spatial_sizes) -> Tuple[List[int], tuple]:
        """Kept mode counts and the weight slice for an input of the given
        spatial size (:464-489): kept_d = min(fft_size_d, n_modes_d); on every
        axis but the last the weight window starts (max_d - kept_d) // 2 in."""
        fft_size = list(spatial_sizes)
        if not self.complex_data:
            fft_size[-1] = fft_size[-1] // 2 + 1
        starts = [mx - min(s, n) for s, n, mx in zip(fft_size, self.n_modes, self.max_n_modes)]
        sl = [slice(None)] if self.separable else [slice(None), slice(None)]
        if self.complex_data:   # every axis centred (:475-479)
            sl += [slice(s // 2, -s // 2) if s else slice(s, None) for s in starts]
        else:
            sl += [slice(s // 2, -s // 2) if s else slice(s, None) for s in starts[:-1]]
            sl += [slice(None, -starts[-1]) if starts[-1] else slice(None)]
        kept = [mx - s for mx, s in zip(self.max_n_modes, starts)]
        return kept, tuple(sl)

    def output_sizes(self, spatial_sizes, output_shape=None) -> List[int]:
        sizes = list(spatial_sizes)
        if self.resolution_scaling_factor is not None and output_shape is None:
            sizes = [round(s * r) for s, r in zip(sizes, self.resolution_scaling_factor)]
        if output_shape is not None:
            sizes = list(output_shape)
        return [int(s) for s in sizes]

    def dense_window_weight(self, sl) -> torch.Tensor:
        """The weight window as a dense complex tensor (reconstructing a
        factorized weight when needed)."""
        if type(self.weight) is DenseTensor:   # a view of the parameter, no window module
            return self.weight.tensor[sl]
        w = self.weight[sl]
        return w.to_tensor() if isinstance(w, FactorizedTensor) else w

    # ---------------------------------------------------------------- forward
    def forward(self, x: torch.Tensor, output_shape: Optional[Tuple[int]] = None):
        if not x.is_cuda:
            raise RuntimeError(
                "SpectralConv (neuraloperator_amd) runs on the GPU only; move the module and "
                "input to a HIP device")
        profiler = get_active_profiler()
        name = getattr(self, "profile_prefix", "spectral_conv")
        with maybe_profile(profiler, name, x.device):
            if self.complex_data:
                return self._forward_complex(x, output_shape)
            if torch.is_grad_enabled() and (x.requires_grad or
                                            any(p.requires_grad for p in self.parameters())):
                y = self._forward_autograd(x, output_shape)
            elif self._half_arithmetic():
                return self._forward_half(x, output_shape)
            else:
                y = self._forward_hip(x, output_shape)
            # fno_block_precision 'half' / 'mixed' (:436-459): the reference's
            # inverse returns float16, promoted to float32 by the float32 bias
            # when there is one (with gradients and for factorized contractions
            # the values are the fp32 ones)
            if self.fno_block_precision in ("half", "mixed") and self.bias is None:
                y = y.half()
            return y

    def _half_arithmetic(self) -> bool:
        """fno_block_precision 'half' / 'mixed' with a contraction whose
        complex-half arithmetic _forward_half restates: a dense window weight
        (dense, or factorized and reconstructed), real data."""
        return (self.fno_block_precision in ("half", "mixed") and not self.complex_data and
                self._contract in ("dense", "dense_separable"))

    def _forward_half(self, x, output_shape=None):
        """fno_block_precision 'half' / 'mixed' (spectral_convolution.py
        :436-462, :520-568 with _contract_dense on complex32, einsum_utils.py
        :10-34), rounded where the reference holds half precision: x ('half'
        only), the kept spectrum (complex32), the weight and each of the four
        real partial contractions of the complex-half einsum, their
        combination Re = t00 - t11, Im = t10 + t01, and the inverse's output.
        The library's transforms and contraction run in fp32 between those
        roundings; the complex32 intermediate between the reference's split
        inverse transforms (ifftn over the leading axes, then irfft) is not
        rounded here (its effect on y is below one float16 step of the output).
        Returns float16, or float32 after the float32 bias."""
        sizes = list(x.shape[2:])
        kept, sl = self.window(sizes)
        out_sizes = self.output_sizes(sizes, output_shape)
        xin = x.detach()
        if self.fno_block_precision == "half":
            xin = _fp16_round(xin)
        X = _fp16_round(Fh.rfft_window(xin, kept, self.fft_norm))
        W = self.dense_window_weight(sl).detach()
        if self.separable:
            # complex32 x times the complex64 weight, rounded by the store
            Y = _fp16_round(X * W)
        else:
            z = torch.zeros_like(W.real)
            A = Fh.contract_dense(X, torch.complex(_fp16_round(W.real), z))    # t00 + i t10
            Bq = Fh.contract_dense(X, torch.complex(_fp16_round(W.imag), z))   # t01 + i t11
            t00, t10 = _fp16_round(A.real), _fp16_round(A.imag)
            t01, t11 = _fp16_round(Bq.real), _fp16_round(Bq.imag)
            Y = torch.complex(_fp16_round(t00 - t11), _fp16_round(t10 + t01))
        y = Fh.irfft_window(Y.contiguous(), sizes, out_sizes, None, self.fft_norm,
                            self.enforce_hermitian_symmetry)
        y = y.half()
        if self.bias is not None:
            y = y + self.bias.detach()
        return y

    def _forward_complex(self, x, output_shape=None):
        """complex_data=True: fftn / window / contraction / ifftn on complex
        fields (spectral_convolution.py:436-449, :500-538), output complex.
        With gradients through _SpectralConvComplexFn on the dense window
        weight."""
        sizes = list(x.shape[2:])
        kept, sl = self.window(sizes)
        out_sizes = self.output_sizes(sizes, output_shape)
        if (torch.is_grad_enabled() and
                (x.requires_grad or any(p.requires_grad for p in self.parameters()))):
            return _SpectralConvComplexFn.apply(x, self.dense_window_weight(sl), self.bias, kept,
                                                self.fft_norm, out_sizes, self.separable)
        xhat = Fh.fft_window(x.detach(), kept, self.fft_norm)
        if self._contract == "tucker" and not self.separable:
            wv = self.weight[sl]
            yhat = Fh.contract_tucker(xhat, wv.core.detach(), [f.detach() for f in wv.factors])
        else:
            yhat = Fh.contract_dense(xhat, self.dense_window_weight(sl).detach(),
                                     separable=self.separable)
        bias = self.bias.reshape(-1).detach() if self.bias is not None else None
        y = Fh.ifft_window(yhat, sizes, out_sizes, bias, self.fft_norm)
        return _attach(y, x, self.bias, *self.weight.parameters())

    def _forward_autograd(self, x, output_shape=None):
        """Forward with gradients for x, the weight (through its dense window,
        so factorized weights get theirs through the reconstruction) and the
        bias, on the input grid or resized, dense or separable."""
        sizes = list(x.shape[2:])
        out_sizes = self.output_sizes(sizes, output_shape)
        kept, sl = self.window(sizes)
        w = self.dense_window_weight(sl)
        return _SpectralConvFn.apply(x, w, self.bias, kept, self.fft_norm, out_sizes,
                                     self.separable, self.enforce_hermitian_symmetry)

    def _forward_hip(self, x, output_shape=None, skip_kind=nat.SKIP_NONE, skip_weight=None,
                     act=nat.ACT_NONE):
        sizes = list(x.shape[2:])
        kept, sl = self.window(sizes)
        out_sizes = self.output_sizes(sizes, output_shape)
        bias = self.bias.reshape(-1) if self.bias is not None else None
        same_size = out_sizes == sizes
        kind = self._contract
        # the parameters only matter to _attach with gradients enabled
        params = ([self.bias] + list(self.weight.parameters()) + [skip_weight]
                  if torch.is_grad_enabled() else [])
        if kind in ("dense", "cp", "tt") and same_size and not self.separable:
            w = self.dense_window_weight(sl).detach()
            y = Fh.spectral_block(x.detach(), w, None if bias is None else bias.detach(), kept,
                                  skip_kind, None if skip_weight is None else skip_weight.detach(),
                                  act, self.fft_norm)
            return _attach(y, x, *params)
        # composed path: window transform, contraction, inverse window transform
        xhat = Fh.rfft_window(x.detach(), kept, self.fft_norm)
        if kind == "tucker" and not self.separable:
            wv = self.weight[sl]
            core = wv.core.detach()
            factors = [f.detach() for f in wv.factors]
            yhat = Fh.contract_tucker(xhat, core, factors)
        else:
            w = self.dense_window_weight(sl).detach()
            yhat = Fh.contract_dense(xhat, w, separable=self.separable)
        b = None if bias is None else bias.detach()
        if skip_kind != nat.SKIP_NONE or act != nat.ACT_NONE:
            if not same_size:
                raise RuntimeError("fused skip requires output size == input size")
            # inverse, bias, skip and activation in one call (on the input
            # grid the Hermitian fix-up is implied by the real inverse)
            y = Fh.irfft_window_epilogue(yhat, sizes, b, x.detach(), skip_kind,
                                         None if skip_weight is None else skip_weight.detach(),
                                         act, self.fft_norm)
        else:
            y = Fh.irfft_window(yhat, sizes, out_sizes, b, self.fft_norm,
                                self.enforce_hermitian_symmetry)
        return _attach(y, x, *params)
