"""Independent float64 formulation of the FNO spectral convolution.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Written from the DFT closed form rather than from the reference's
fftshift/slice bookkeeping, so that it pins ``spectral_ref``:

* kept count per axis   m_d = min(fft_size_d, n_modes_d)
* weight window offset  (max_d - m_d) // 2 on non-last axes, 0 on the last
  axis (what spectral_convolution.py:465-489 computes with slices)
* window index j on a non-last axis carries frequency f = j - m_d // 2;
  on the last (rfft) axis it carries f = j
* forward:   X[j] = s_fwd * sum_n x[n] exp(-2 pi i sum_d f_d n_d / N_d)
* inverse on a non-last axis of output size N'_d: the entry of frequency f
  sits at index t = f mod N_d of the length-N_d spectrum; ifftn with
  s=N'_d zero-pads or truncates at the end, so it contributes
  exp(+2 pi i t n / N'_d) when t < N'_d and is dropped otherwise
* inverse on the last axis (irfft, n = N'): only bins j < N'//2 + 1 are used;
  y[n] = sum_j c_j Re(Z_j exp(2 pi i j n / N')), c_0 = 1, c_{N'/2} = 1 for even
  N', else 2 (the imaginary parts of DC and Nyquist drop out)
* with enforce_hermitian_symmetry the imaginary part of bin N//2 of the
  input-size spectrum is also zeroed when N' is even
  (spectral_convolution.py:552-556)
* scales: "forward" s_fwd = 1/prod N, s_inv = 1; "backward" s_fwd = 1,
  s_inv = 1/prod N'; "ortho" both 1/sqrt(.)
"""
from __future__ import annotations

import numpy as np


def _scales(norm, in_sizes, out_sizes):
    pin = float(np.prod(in_sizes))
    pout = float(np.prod(out_sizes))
    if norm == "forward":
        return 1.0 / pin, 1.0
    if norm == "backward":
        return 1.0, 1.0 / pout
    if norm == "ortho":
        return 1.0 / np.sqrt(pin), 1.0 / np.sqrt(pout)
    raise ValueError(norm)


def kept_counts(sizes, n_modes):
    """m_d = min(fft_size_d, n_modes_d) with fft_size_last = N//2+1."""
    fft_size = list(sizes)
    fft_size[-1] = fft_size[-1] // 2 + 1
    return [min(s, m) for s, m in zip(fft_size, n_modes)]


def weight_window(weight, sizes, n_modes, max_n_modes, separable=False):
    """Cut the used window out of the full (max_n_modes) weight by formula."""
    m = kept_counts(sizes, n_modes)
    lead = 1 if separable else 2
    idx = [slice(None)] * lead
    for d, (md, mx) in enumerate(zip(m, max_n_modes)):
        off = 0 if d == len(m) - 1 else (mx - md) // 2
        idx.append(slice(off, off + md))
    return weight[tuple(idx)]


def window_freqs(m, last):
    j = np.arange(m)
    return j if last else j - m // 2


def forward_modes(x, m, norm="forward", out_sizes=None):
    """X[b,c,j...] over the kept window, float64 complex."""
    x = np.asarray(x, dtype=np.float64)
    sizes = list(x.shape[2:])
    order = len(sizes)
    s_fwd, _ = _scales(norm, sizes, out_sizes or sizes)
    X = x.astype(np.complex128)
    for d in range(order):
        N = sizes[d]
        f = window_freqs(m[d], d == order - 1)
        E = np.exp(-2j * np.pi * np.outer(f, np.arange(N)) / N)     # [m_d, N_d]
        X = np.moveaxis(np.tensordot(X, E, axes=([2 + d], [1])), -1, 2 + d)
    return X * s_fwd


def inverse_modes(Y, in_sizes, out_sizes, norm="forward", enforce_hermitian_symmetry=True):
    """Real output field from window coefficients Y[b,o,j...]."""
    order = len(in_sizes)
    _, s_inv = _scales(norm, in_sizes, out_sizes)
    m = list(Y.shape[2:])
    Z = np.asarray(Y, dtype=np.complex128)
    for d in range(order - 1):
        N, Np = in_sizes[d], out_sizes[d]
        t = window_freqs(m[d], False) % N
        keep = (t < Np).astype(np.float64)
        E = np.exp(2j * np.pi * np.outer(np.arange(Np), t) / Np) * keep[None, :]   # [N', m]
        Z = np.moveaxis(np.tensordot(Z, E, axes=([2 + d], [1])), -1, 2 + d)
    N, Np = in_sizes[-1], out_sizes[-1]
    j = np.arange(m[-1])
    Z = Z.copy()
    Z[..., 0] = Z[..., 0].real
    if enforce_hermitian_symmetry and Np % 2 == 0 and (N // 2) < m[-1]:
        Z[..., N // 2] = Z[..., N // 2].real
    used = j < (Np // 2 + 1)
    c = np.where(j == 0, 1.0, 2.0)
    if Np % 2 == 0:
        c = np.where(j == Np // 2, 1.0, c)
    c = c * used
    E = np.exp(2j * np.pi * np.outer(np.arange(Np), j) / Np) * c[None, :]          # [N', m]
    y = np.tensordot(Z, E, axes=([Z.ndim - 1], [1])).real
    return y * s_inv


def spectral_conv(x, weight, bias, n_modes, max_n_modes=None, *, norm="forward", separable=False,
                  out_sizes=None, enforce_hermitian_symmetry=True):
    """Whole SpectralConv forward (real data), float64.

    ``n_modes``/``max_n_modes`` are the stored lists (last entry n//2+1);
    ``weight`` is the full max_n_modes complex weight."""
    x = np.asarray(x, dtype=np.float64)
    sizes = list(x.shape[2:])
    if max_n_modes is None:
        max_n_modes = list(n_modes)
    out_sizes = list(out_sizes) if out_sizes is not None else sizes
    m = kept_counts(sizes, n_modes)
    w = np.asarray(weight_window(np.asarray(weight), sizes, n_modes, max_n_modes, separable),
                   dtype=np.complex128)
    X = forward_modes(x, m, norm, out_sizes)
    if separable:
        Y = X * w[None]
    else:
        Y = np.einsum("bi...,io...->bo...", X, w)
    y = inverse_modes(Y, sizes, out_sizes, norm, enforce_hermitian_symmetry)
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64)
    return y


def gelu(x):
    """0.5 x (1 + erf(x / sqrt 2)) in float64 via math.erf."""
    from math import erf, sqrt
    v = np.vectorize(lambda t: 0.5 * t * (1.0 + erf(t / sqrt(2.0))))
    return v(np.asarray(x, dtype=np.float64))


def spectral_block(x, weight, bias, ws, n_modes, max_n_modes=None, *, norm="forward"):
    """GELU(SpectralConv(x) + Ws x), float64."""
    y = spectral_conv(x, weight, bias, n_modes, max_n_modes, norm=norm)
    y = y + np.einsum("oi,bi...->bo...", np.asarray(ws, np.float64), np.asarray(x, np.float64))
    return gelu(y)
