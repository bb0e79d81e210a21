"""Skip connections of the FNO block (neuralop/layers/skip_connections.py):
1x1-conv ("linear"), soft-gating and identity.  The fused block kernel reads
their weights directly; standalone calls run as torch ops."""
from __future__ import annotations

import torch
from torch import nn


def skip_connection(in_features, out_features, n_dim=2, bias=False, skip_type="soft-gating"):
    """Factory (skip_connections.py:5-50)."""
    if skip_type.lower() == "soft-gating":
        return SoftGating(in_features=in_features, out_features=out_features, bias=bias, n_dim=n_dim)
    if skip_type.lower() == "linear":
        return Flattened1dConv(in_channels=in_features, out_channels=out_features, kernel_size=1,
                               bias=bias)
    if skip_type.lower() == "identity":
        return nn.Identity()
    raise ValueError(f"Got skip-connection type={skip_type}, expected one of"
                     f" {'soft-gating', 'linear', 'id'}.")


class SoftGating(nn.Module):
    """x * w with w of shape (1, C, 1, ...) (skip_connections.py:53-93)."""

    def __init__(self, in_features, out_features=None, n_dim=2, bias=False):
        super().__init__()
        if out_features is not None and in_features != out_features:
            raise ValueError(f"Got in_features={in_features} and out_features={out_features}, "
                             "but these two must be the same for soft-gating")
        self.in_features = in_features
        self.out_features = out_features
        self.weight = nn.Parameter(torch.ones(1, self.in_features, *(1,) * n_dim))
        self.bias = nn.Parameter(torch.ones(1, self.in_features, *(1,) * n_dim)) if bias else None

    def forward(self, x):
        return self.weight * x + self.bias if self.bias is not None else self.weight * x


class Flattened1dConv(nn.Module):
    """1x1 Conv1d over flattened spatial dims (skip_connections.py:96-130)."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size, bias=False):
        super().__init__()
        self.conv = nn.Conv1d(in_channels=in_channels, out_channels=out_channels,
                              kernel_size=kernel_size, bias=bias)

    def forward(self, x):
        size = list(x.shape)
        x = x.view(*size[:2], -1)
        x = self.conv(x)
        return x.view(size[0], self.conv.out_channels, *size[2:])
