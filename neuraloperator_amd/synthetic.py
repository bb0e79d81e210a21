"""Seeded synthetic inputs for the benchmark workloads (input generation is
not part of any measured path).

Gaussian random field: white noise -> FFT -> multiply by (1 + |k|^2)^-1
(power spectrum proportional to (1 + |k|^2)^-2) -> inverse FFT -> normalise
each field to zero mean and unit variance.  |k| is the integer wavenumber.
"""
from __future__ import annotations

import torch


def gaussian_random_field(shape, seed: int = 0, chunk: int = 8, device=None) -> torch.Tensor:
    """float32 GRF of ``shape`` = (B, C, *spatial).  The noise is drawn on the
    CPU from a seeded generator (device independent); the filtering runs on
    ``device`` (default CPU) and the result is returned there."""
    g = torch.Generator().manual_seed(seed)
    B, C, *spatial = shape
    dev = torch.device(device) if device is not None else torch.device("cpu")
    out = torch.empty(shape, dtype=torch.float32, device=dev)
    ks = [torch.fft.fftfreq(n, d=1.0 / n, device=dev) for n in spatial]
    grids = torch.meshgrid(*ks, indexing="ij")
    k2 = sum(k.double() ** 2 for k in grids)
    filt = (1.0 / (1.0 + k2)).to(torch.complex128)
    dims = list(range(-len(spatial), 0))
    flat = out.view(B * C, *spatial)
    for s in range(0, B * C, chunk):
        e = min(B * C, s + chunk)
        w = torch.randn((e - s, *spatial), generator=g, dtype=torch.float64).to(dev)
        f = torch.fft.ifftn(torch.fft.fftn(w, dim=dims) * filt, dim=dims).real
        f = f - f.mean(dim=dims, keepdim=True)
        f = f / f.std(dim=dims, keepdim=True)
        flat[s:e] = f.float()
    return out


def complex_normal(shape, std: float, seed: int) -> torch.Tensor:
    """complex64 tensor whose real and imaginary parts are each N(0, std^2)."""
    g = torch.Generator().manual_seed(seed)
    re = torch.randn(shape, generator=g) * std
    im = torch.randn(shape, generator=g) * std
    return torch.complex(re, im)


def real_normal(shape, std: float, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g) * std
