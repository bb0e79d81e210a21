"""Grid positional embedding (neuralop/layers/embeddings.py:90-164, :351-383)."""
from __future__ import annotations

from typing import List

import torch
from torch import nn


def regular_grid_nd(resolutions: List[int], grid_boundaries=((0, 1), (0, 1))):
    """Per-dim coordinates linspace(start, stop, res + 1)[:-1], meshgrid 'ij'."""
    assert len(resolutions) == len(grid_boundaries), "Error: inputs must have same number of dimensions"
    dim = len(resolutions)
    inputs = [torch.linspace(a, b, r + 1)[:-1] for r, (a, b) in zip(resolutions, grid_boundaries)]
    grid = torch.meshgrid(*inputs, indexing="ij")
    return tuple(g.repeat([1] * dim) for g in grid)


class GridEmbeddingND(nn.Module):
    def __init__(self, in_channels: int, dim: int = 2, grid_boundaries=((0, 1), (0, 1))):
        super().__init__()
        self.in_channels = in_channels
        self.dim = dim
        assert self.dim == len(grid_boundaries), (
            f"Error: expected grid_boundaries to be an iterable of length {self.dim}, "
            f"received {grid_boundaries}")
        self.grid_boundaries = grid_boundaries
        self._grid = None
        self._res = None

    @property
    def out_channels(self):
        return self.in_channels + self.dim

    def grid(self, spatial_dims, device, dtype):
        if self._grid is None or self._res != spatial_dims or self._grid[0].device != device \
                or self._grid[0].dtype != dtype:
            grids = regular_grid_nd(list(spatial_dims), grid_boundaries=self.grid_boundaries)
            self._grid = [g.to(device).to(dtype).unsqueeze(0).unsqueeze(0) for g in grids]
            self._res = spatial_dims
        return self._grid

    def forward(self, data, batched=True):
        if not batched and data.ndim == self.dim + 1:
            data = data.unsqueeze(0)
        batch_size = data.shape[0]
        grids = self.grid(spatial_dims=data.shape[2:], device=data.device, dtype=data.dtype)
        grids = [g.repeat(batch_size, *[1] * (self.dim + 1)) for g in grids]
        return torch.cat((data, *grids), dim=1)
