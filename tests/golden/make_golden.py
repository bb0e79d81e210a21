"""Writes the golden fixtures used by the parity tests.

    python tests/golden/make_golden.py

Each fixture holds seeded inputs and weights and the expected output computed
in float64 by the closed-form formulation (oracle/dft64.py); the torch
restatement (oracle/spectral_ref.py) must agree with it to ~1e-12 before a
fixture is written.  Shapes cover 1D/2D/3D, even and odd sizes, truncated
windows (n_modes < max_n_modes), resolution scaling, every fft_norm, the
Nyquist bin and the fused block (skip + bias + GELU).
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import dft64, spectral_ref  # noqa: E402

CASES = [
    # name, B, Ci, Co, sizes, n_modes (constructor), max_n_modes, out_sizes, norm, block
    ("conv1d_n12_m10", 2, 3, 4, (12,), (10,), None, None, "forward", False),
    ("conv1d_n16_m30_w16", 2, 3, 3, (32,), (30,), None, None, "forward", False),
    ("conv2d_9x10_m4x5", 2, 3, 4, (9, 10), (4, 5), None, None, "forward", False),
    ("conv2d_12x12_m6x8_max8x8", 2, 3, 4, (12, 12), (6, 8), (8, 8), None, "forward", False),
    ("conv2d_8x8_m8x8_nyquist", 2, 3, 4, (8, 8), (8, 8), None, None, "forward", False),
    ("conv2d_12x12_up24", 2, 3, 4, (12, 12), (4, 6), None, (24, 24), "forward", False),
    ("conv2d_9x9_down4_ortho", 2, 3, 4, (9, 9), (4, 7), None, (4, 4), "ortho", False),
    ("conv2d_8x10_backward", 2, 3, 4, (8, 10), (4, 4), None, None, "backward", False),
    ("conv3d_8x9x10_m4", 2, 3, 4, (8, 9, 10), (4, 4, 4), None, None, "forward", False),
    ("block2d_64x128_m8x8", 1, 32, 32, (64, 128), (8, 8), None, None, "forward", True),
    ("block2d_32x32_m8x8", 2, 4, 6, (32, 32), (8, 8), None, None, "forward", True),
]


def make(case, seed):
    name, B, Ci, Co, sizes, nm, mx, outs, norm, block = case
    g = torch.Generator().manual_seed(seed)
    nms = spectral_ref.stored_n_modes(nm)
    mxs = spectral_ref.stored_n_modes(mx) if mx else list(nms)
    x = torch.randn((B, Ci, *sizes), generator=g, dtype=torch.float64).float()
    std = (2.0 / (Ci + Co)) ** 0.5
    wr = torch.randn((Ci, Co, *mxs), generator=g, dtype=torch.float64) * std
    wi = torch.randn((Ci, Co, *mxs), generator=g, dtype=torch.float64) * std
    w = torch.complex(wr, wi).to(torch.complex64)
    bias = (torch.randn((Co,) + (1,) * len(sizes), generator=g) * std).float()
    ws = (torch.randn((Co, Ci), generator=g) / Ci ** 0.5).float() if block else None
    x64, w64, b64 = x.double(), w.to(torch.complex128), bias.double()
    ref = spectral_ref.spectral_conv_forward(x64, w64, b64, nms, mxs, fft_norm=norm, output_shape=outs)
    exp = dft64.spectral_conv(x64.numpy(), w64.numpy(), b64.numpy(), nms, mxs, norm=norm,
                              out_sizes=outs)
    err = np.abs(ref.numpy() - exp).max() / np.abs(exp).max()
    assert err < 1e-12, (name, err)
    if block:
        exp = exp + np.einsum("oi,bi...->bo...", ws.double().numpy(), x64.numpy())
        exp = dft64.gelu(exp)
    out = dict(x=x.numpy(), w=w.numpy(), bias=bias.numpy(), n_modes=np.array(nm),
               stored_n_modes=np.array(nms), max_n_modes=np.array(mxs),
               out_sizes=np.array(outs if outs else sizes), norm=np.array(norm),
               expected=exp.astype(np.float64 if exp.size < 65536 else np.float32))
    if ws is not None:
        out["skip_w"] = ws.numpy()
    return name, out


def main():
    for i, case in enumerate(CASES):
        name, arrays = make(case, seed=1000 + i)
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **arrays)
        print("wrote", name, arrays["expected"].shape)


if __name__ == "__main__":
    main()
