"""Domain padding around the Fourier layers (neuralop/layers/padding.py:9-150).

Zero padding of round(p * n) points on both sides of every spatial axis before
the FNO blocks, removed after them; the removal is scaled by the resolution
scaling factor the blocks apply.  Pads and unpad slices are cached per
resolution, as in the reference.  Plain torch data movement around the HIP
layers.
"""
from __future__ import annotations

from typing import List, Union

from torch import nn
from torch.nn import functional as F

from .utils import validate_scaling_factor


class DomainPadding(nn.Module):
    def __init__(self, domain_padding: Union[float, list],
                 resolution_scaling_factor: Union[int, List[int]] = 1):
        super().__init__()
        self.domain_padding = domain_padding
        self.resolution_scaling_factor = 1 if resolution_scaling_factor is None else resolution_scaling_factor
        self._padding = {}
        self._unpad_indices = {}

    def forward(self, x):
        return self.pad(x)

    def pad(self, x, verbose: bool = False):
        resolution = x.shape[2:]
        if isinstance(self.domain_padding, (float, int)):
            self.domain_padding = [float(self.domain_padding)] * len(resolution)
        if len(self.domain_padding) != len(resolution):
            raise ValueError("domain_padding length must match the number of spatial/time dimensions "
                             "(excluding batch, ch)")
        factor = self.resolution_scaling_factor
        if not isinstance(factor, list):
            factor = validate_scaling_factor(factor, len(resolution), n_layers=None)
        key = f"{resolution}"
        if key in self._padding:
            return F.pad(x, self._padding[key], mode="constant")
        pads = [round(p * r) for p, r in zip(self.domain_padding, resolution)]
        if verbose:
            print(f"Padding inputs of resolution={resolution} with padding={pads}, symmetric")
        out_pads = [round(f * p) for f, p in zip(factor, pads)]
        unpad = (Ellipsis,) + tuple(slice(p, -p) if p else slice(None) for p in out_pads)
        # F.pad takes (last-axis before, after, previous axis before, after, ...)
        flat = [q for p in pads[::-1] for q in (p, p)]
        self._padding[key] = flat
        padded = F.pad(x, flat, mode="constant")
        out_shape = [round(f * n) for f, n in zip(factor, padded.shape[2:])]
        self._unpad_indices[f"{out_shape}"] = unpad
        return padded

    def unpad(self, x):
        return x[self._unpad_indices[f"{list(x.shape[2:])}"]]
