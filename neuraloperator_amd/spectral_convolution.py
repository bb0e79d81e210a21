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
transforms under the dual norm and the dense contraction) for output size ==
input size and non-separable weights; a factorized weight gets its gradient
through the torch reconstruction of its dense window.  Other configurations
raise on backward.
"""
from __future__ import annotations

import math

from typing import List, Optional, Tuple, Union

import torch
from torch import nn

from . import _native as nat
from . import functional as Fh
from .factorized_tensors import FactorizedTensor, TuckerTensor, _TuckerView
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
    """Attaches a HIP forward result to the graph with a backward that
    raises: for the cases the gradient functions do not cover."""

    @staticmethod
    def forward(ctx, y, *inputs):
        return y

    @staticmethod
    def backward(ctx, *grads):
        raise NotImplementedError(
            "gradients of the HIP spectral path cover output size == input size and "
            "non-separable weights")


_DUAL_NORM = {"forward": "backward", "backward": "forward", "ortho": "ortho"}


def _hermitian_weights(m_last: int, n_last: int, ndim: int, device) -> torch.Tensor:
    """c_k of the real inverse transform along the last axis: 1 for bin 0 and
    the Nyquist bin, 2 for the bins that stand for a conjugate pair."""
    c = torch.full((m_last,), 2.0, device=device)
    c[0] = 1.0
    if n_last % 2 == 0 and n_last // 2 < m_last:
        c[n_last // 2] = 1.0
    return c.view(*([1] * (ndim + 1)), m_last)


class _SpectralConvFn(torch.autograd.Function):
    """Dense spectral convolution y = s_i I(W . s_f F(x)) + bias with the
    gradients of SpectralConv.forward (spectral_convolution.py:417-570), for
    output size == input size.  With F the window of the forward transform
    (bins e^{-i phi_k(n)}) and I the real inverse (y = sum_k c_k Re(Y_k
    e^{i phi_k(n)}), c_k = 2 for bins that stand for a conjugate pair):

        gY = s_i c_k . F_unscaled(gy)      gX = gY . conj(W)^T
        gW = conj(X)^T . gY               gx = s_f Re(sum_k gX_k e^{i phi_k})
                                              = s_f I_unscaled(gX / c_k)

    so both transforms are the library's own window transforms under the dual
    norm (forward <-> backward scaling), and both contractions its dense
    mode-wise contraction."""

    @staticmethod
    def forward(ctx, x, w, bias, kept, fft_norm):
        sizes = list(x.shape[2:])
        b = bias.reshape(-1) if bias is not None else None
        y = Fh.spectral_block(x, w, b, kept, nat.SKIP_NONE, None, nat.ACT_NONE, fft_norm)
        ctx.save_for_backward(x, w)
        ctx.kept, ctx.fft_norm, ctx.sizes = list(kept), fft_norm, sizes
        ctx.bias_shape = None if bias is None else bias.shape
        return y

    @staticmethod
    def backward(ctx, gy):
        x, w = ctx.saved_tensors
        kept, norm, sizes = ctx.kept, ctx.fft_norm, ctx.sizes
        gy = gy.contiguous().float()
        dual = _DUAL_NORM[norm]
        c = _hermitian_weights(kept[-1], sizes[-1], len(sizes), gy.device)
        gY = Fh.rfft_window(gy, kept, dual) * c
        gx = gw = gb = None
        if ctx.needs_input_grad[0]:
            wt = w.conj().transpose(0, 1).contiguous()              # [Co, Ci, *m]
            gX = Fh.contract_dense(gY, wt)                          # [B, Ci, *m]
            gx = Fh.irfft_window(gX / c, sizes, sizes, None, dual, False)
        if ctx.needs_input_grad[1]:
            X = Fh.rfft_window(x, kept, norm)                       # [B, Ci, *m]
            xt = X.conj().transpose(0, 1).contiguous()              # [Ci, B, *m]
            gw = Fh.contract_dense(xt, gY.contiguous())             # [Ci, Co, *m]
        if ctx.bias_shape is not None and ctx.needs_input_grad[2]:
            dims = [0] + list(range(2, gy.ndim))
            gb = gy.sum(dim=dims).reshape(ctx.bias_shape)
        return gx, gw, gb, None, None


def _last_axis_phase(n: int, ndim: int, device) -> torch.Tensor:
    """psi_t = exp(-2 pi i (n//2) t / n) along the last axis (1 in 1D): the
    complex-data forward window takes last-axis frequencies j - n//2 and the
    inverse puts them back at j (spectral_convolution.py:448-449, :531-538),
    so each transform's adjoint is the other library transform times psi."""
    if ndim == 1:
        return torch.ones(n, dtype=torch.complex64, device=device)
    t = torch.arange(n, dtype=torch.float64, device=device)
    return torch.polar(torch.ones_like(t), -2.0 * math.pi * (n // 2) * t / n).to(torch.complex64)


class _SpectralConvComplexFn(torch.autograd.Function):
    """complex_data=True spectral convolution y = I(W . F(x)) + bias with
    its gradients, output size == input size.  F (windowed fftn) and I
    (zero-filled ifftn) are C-linear, so with psi from _last_axis_phase and
    the dual norm:

        gY = I^H gy = F_dual(gy . psi)      gX = gY . conj(W)^T
        gW = conj(X)^T . gY                gx = F^H gX = I_dual(gX) . psi
        gbias = sum Re(gy)   (the real bias is added to the real part)"""

    @staticmethod
    def forward(ctx, x, w, bias, kept, fft_norm):
        sizes = list(x.shape[2:])
        xhat = Fh.fft_window(x, kept, fft_norm)
        yhat = Fh.contract_dense(xhat, w)
        b = bias.reshape(-1) if bias is not None else None
        y = Fh.ifft_window(yhat, sizes, sizes, b, fft_norm)
        ctx.save_for_backward(xhat, w)
        ctx.kept, ctx.fft_norm, ctx.sizes = list(kept), fft_norm, sizes
        ctx.bias_shape = None if bias is None else bias.shape
        return y

    @staticmethod
    def backward(ctx, gy):
        xhat, w = ctx.saved_tensors
        kept, sizes = ctx.kept, ctx.sizes
        dual = _DUAL_NORM[ctx.fft_norm]
        gy = gy.contiguous().to(torch.complex64)
        psi = _last_axis_phase(sizes[-1], len(sizes), gy.device)
        gY = Fh.fft_window((gy * psi).contiguous(), kept, dual)          # [B, Co, *m]
        gx = gw = gb = None
        if ctx.needs_input_grad[0]:
            wt = w.conj().transpose(0, 1).contiguous()                   # [Co, Ci, *m]
            gX = Fh.contract_dense(gY, wt)                               # [B, Ci, *m]
            gx = Fh.ifft_window(gX, sizes, sizes, None, dual) * psi
        if ctx.needs_input_grad[1]:
            xt = xhat.conj().transpose(0, 1).contiguous()                # [Ci, B, *m]
            gw = Fh.contract_dense(xt, gY)                               # [Ci, Co, *m]
        if ctx.bias_shape is not None and ctx.needs_input_grad[2]:
            dims = [0] + list(range(2, gy.ndim))
            gb = gy.real.sum(dim=dims).reshape(ctx.bias_shape)
        return gx, gw, gb, None, None


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
        w = self.weight[sl] if isinstance(self.weight, FactorizedTensor) else self.weight[sl]
        w = w.to_tensor() if isinstance(w, FactorizedTensor) else w
        return w

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
            else:
                y = self._forward_hip(x, output_shape)
            # fno_block_precision 'half' / 'mixed' (:436-459): the reference's
            # inverse returns float16, promoted to float32 by the float32 bias
            # when there is one; the kernels compute in fp32 either way
            if self.fno_block_precision in ("half", "mixed") and self.bias is None:
                y = y.half()
            return y

    def _forward_complex(self, x, output_shape=None):
        """complex_data=True: fftn / window / contraction / ifftn on complex
        fields (spectral_convolution.py:436-449, :500-538), output complex.
        With gradients (output size == input size, non-separable) through
        _SpectralConvComplexFn on the dense window weight; other cases run
        the same forward and raise if a backward reaches them."""
        sizes = list(x.shape[2:])
        kept, sl = self.window(sizes)
        out_sizes = self.output_sizes(sizes, output_shape)
        if (torch.is_grad_enabled() and out_sizes == sizes and not self.separable and
                (x.requires_grad or any(p.requires_grad for p in self.parameters()))):
            return _SpectralConvComplexFn.apply(x, self.dense_window_weight(sl), self.bias, kept,
                                                self.fft_norm)
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
        bias; output size == input size, non-separable.  Other cases run the
        plain forward, whose backward raises."""
        sizes = list(x.shape[2:])
        out_sizes = self.output_sizes(sizes, output_shape)
        if out_sizes != sizes or self.separable:
            return self._forward_hip(x, output_shape)
        kept, sl = self.window(sizes)
        w = self.dense_window_weight(sl)
        return _SpectralConvFn.apply(x, w, self.bias, kept, self.fft_norm)

    def _forward_hip(self, x, output_shape=None, skip_kind=nat.SKIP_NONE, skip_weight=None,
                     act=nat.ACT_NONE):
        sizes = list(x.shape[2:])
        kept, sl = self.window(sizes)
        out_sizes = self.output_sizes(sizes, output_shape)
        bias = self.bias.reshape(-1) if self.bias is not None else None
        same_size = out_sizes == sizes
        kind = self._contract
        params = [self.bias] + list(self.weight.parameters()) + [skip_weight]
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
        y = Fh.irfft_window(yhat, sizes, out_sizes, None if bias is None else bias.detach(),
                            self.fft_norm, self.enforce_hermitian_symmetry)
        if skip_kind != nat.SKIP_NONE or act != nat.ACT_NONE:
            if not same_size:
                raise RuntimeError("fused skip requires output size == input size")
            y = Fh.block_epilogue(y, x.detach(), skip_kind,
                                  None if skip_weight is None else skip_weight.detach(), act)
        return _attach(y, x, *params)
