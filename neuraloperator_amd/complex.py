"""Complex-valued spatial data around the HIP spectral layers
(neuralop/layers/complex.py): activations applied to the real and imaginary
parts separately, and a wrapper that runs a real module as a complex-linear
map (two copies: one for the real, one for the imaginary coefficients).
Torch ops; the spectral convolutions themselves run through the library."""
from __future__ import annotations

from copy import deepcopy

import torch
import torch.nn.functional as F
from torch import nn


def _split(fn, x: torch.Tensor) -> torch.Tensor:
    return torch.complex(fn(x.real), fn(x.imag))


def CGELU(x: torch.Tensor) -> torch.Tensor:
    """GELU on the real and imaginary parts (complex.py:8-27)."""
    return _split(F.gelu, x)


def cselu(x: torch.Tensor) -> torch.Tensor:
    """SELU on the real and imaginary parts (complex.py:30-39)."""
    return _split(F.selu, x)


def ctanh(x: torch.Tensor) -> torch.Tensor:
    """tanh on the real and imaginary parts (complex.py:42-51)."""
    return _split(torch.tanh, x)


def apply_complex(real_func, imag_func, x: torch.Tensor, dtype=torch.cfloat) -> torch.Tensor:
    """(fr + i fi)(xr + i xi) for real maps fr, fi (complex.py:54-63)."""
    re = real_func(x.real) - imag_func(x.imag)
    im = real_func(x.imag) + imag_func(x.real)
    return torch.complex(re, im).to(dtype)


class ComplexValued(nn.Module):
    """A real module applied as a complex-linear map (complex.py:66-80)."""

    def __init__(self, module: nn.Module):
        super().__init__()
        self.fr = deepcopy(module)
        self.fi = deepcopy(module)

    def forward(self, x):
        return apply_complex(self.fr, self.fi, x)
