"""Resampling used by SpectralConv.transform for the skip path under
resolution scaling (neuralop/layers/resample.py:7-71): linear (1D) and
bicubic (2D) interpolation with align_corners=True."""
from __future__ import annotations

import torch.nn.functional as F


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
    raise NotImplementedError(
        "spectral resampling of 3D+ skip paths (resample.py:54-69) is not built; "
        "resolution scaling is supported for 1D and 2D fields")
