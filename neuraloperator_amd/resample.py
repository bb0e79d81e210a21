"""Resampling used by SpectralConv.transform for the skip path under
resolution scaling (neuralop/layers/resample.py:7-71): linear (1D) and
bicubic (2D) interpolation with align_corners=True; for 3D and more axes the
spectral resample of resample.py:54-69 on the library's window transforms."""
from __future__ import annotations

import torch
import torch.nn.functional as F


class _NoGrad(torch.autograd.Function):
    """The spectral resample's output on the graph, with a backward that raises."""

    @staticmethod
    def forward(ctx, y, *inputs):
        return y

    @staticmethod
    def backward(ctx, *grads):
        raise NotImplementedError("gradients of the 3D+ spectral resample are not built")


def spectral_resample(x: torch.Tensor, new_size) -> torch.Tensor:
    """rfftn (norm "forward") of x over its spatial axes, the frequencies both
    grids share copied to a spectrum of the new size, irfftn (resample.py:54-69).

    Per non-last axis the reference keeps m = min(old, new) frequencies
    through the slices [:m//2] and [-m//2:]: -m/2 .. m/2-1 for even m, and for
    odd m = 2k+1 the residues of the odd grid as -k-1 .. k-1.  The library's
    windows are centred (-m/2 .. m/2-1 even, -k .. k odd), so an odd axis
    moves one row: on upsampling the old grid's +k goes to -k-1 of the new
    one, on downsampling the old grid's -k-1 goes to +k (the same residue mod
    2k+1).  The last axis keeps bins 0 .. min(old, new)//2."""
    from . import functional as Fh
    old = list(x.shape[2:])
    new = [int(s) for s in new_size]
    nd = len(old)
    kept_fwd, fixes = [], []
    for d in range(nd - 1):
        m = min(old[d], new[d])
        if m % 2 == 0 or old[d] == new[d]:
            kept_fwd.append(m)
            fixes.append(None)
        elif old[d] == m:             # odd old grid, larger new grid
            kept_fwd.append(m)
            fixes.append("up")
        else:                         # odd new grid, larger old grid
            kept_fwd.append(m + 1)
            fixes.append("down")
    kept_fwd.append(min(old[-1] // 2 + 1, new[-1] // 2 + 1))
    xh = Fh.rfft_window(x.detach(), kept_fwd, "forward")
    for d, fix in enumerate(fixes):
        ax, m = 2 + d, kept_fwd[d]
        if fix == "up":               # rows -k..k  ->  -k-1 (old +k), -k..k-1, +k (zero)
            xh = torch.cat([xh.narrow(ax, m - 1, 1), xh.narrow(ax, 0, m - 1),
                            torch.zeros_like(xh.narrow(ax, 0, 1))], dim=ax)
        elif fix == "down":           # rows -k-1..k  ->  -k..k-1, +k (old -k-1)
            xh = torch.cat([xh.narrow(ax, 1, m - 2), xh.narrow(ax, 0, 1)], dim=ax)
    y = Fh.irfft_window(xh.contiguous(), new, new, None, "forward")
    if torch.is_grad_enabled() and x.requires_grad:
        return _NoGrad.apply(y, x)
    return y


def resample(x, res_scale, axis, output_shape=None):
    if isinstance(res_scale, (float, int)):
        if axis is None:
            axis = list(range(2, x.ndim))
            res_scale = [res_scale] * len(axis)
        elif isinstance(axis, int):
            axis = [axis]
            res_scale = [res_scale]
        else:
            res_scale = [res_scale] * len(axis)
    old_size = x.shape[-len(axis):]
    if output_shape is None:
        new_size = tuple(int(round(s * r)) for s, r in zip(old_size, res_scale))
    else:
        new_size = tuple(output_shape)
    if len(axis) == 1:
        return F.interpolate(x, size=new_size[0], mode="linear", align_corners=True)
    if len(axis) == 2:
        return F.interpolate(x, size=new_size, mode="bicubic", align_corners=True)
    if sorted(a % x.ndim for a in axis) != list(range(x.ndim - len(axis), x.ndim)):
        raise NotImplementedError("the spectral resample covers the trailing spatial axes")
    return spectral_resample(x, new_size)
