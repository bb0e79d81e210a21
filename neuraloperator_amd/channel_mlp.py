"""Pointwise channel MLP (neuralop/layers/channel_mlp.py:82-119).

The default two-layer GELU MLP runs as one fno_channel_mlp_f32 call on the GPU
when the library covers its widths (the lifting, projection and block MLPs of
FNO); other configurations run as torch ops.  Under
torch.autocast(dtype=torch.bfloat16) the kernel takes bf16-rounded operands
with fp32 accumulation, as Conv1d does there; its output stays fp32."""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from . import _native as nat
from . import functional as Fh


class ChannelMLP(nn.Module):
    def __init__(self, in_channels, out_channels=None, hidden_channels=None, n_layers=2, n_dim=2,
                 non_linearity=F.gelu, dropout=0.0):
        super().__init__()
        self.n_layers = n_layers
        self.in_channels = in_channels
        self.out_channels = in_channels if out_channels is None else out_channels
        self.hidden_channels = in_channels if hidden_channels is None else hidden_channels
        self.non_linearity = non_linearity
        self.dropout = (nn.ModuleList([nn.Dropout(dropout) for _ in range(n_layers)])
                        if dropout > 0.0 else None)
        self.fcs = nn.ModuleList()
        for i in range(n_layers):
            if i == 0 and i == n_layers - 1:
                self.fcs.append(nn.Conv1d(self.in_channels, self.out_channels, 1))
            elif i == 0:
                self.fcs.append(nn.Conv1d(self.in_channels, self.hidden_channels, 1))
            elif i == n_layers - 1:
                self.fcs.append(nn.Conv1d(self.hidden_channels, self.out_channels, 1))
            else:
                self.fcs.append(nn.Conv1d(self.hidden_channels, self.hidden_channels, 1))

    def _fusable(self, x):
        if not x.is_cuda or x.dtype != torch.float32 or x.ndim < 3:
            return False
        if torch.is_grad_enabled() and (x.requires_grad or
                                        any(p.requires_grad for p in self.parameters())):
            return False   # torch ops carry the gradients
        if self.n_layers != 2 or self.non_linearity is not F.gelu or self.dropout is not None:
            return False
        P = 1
        for s in x.shape[2:]:
            P *= s
        return Fh.channel_mlp_is_supported(self.in_channels, self.hidden_channels,
                                           self.out_channels, P, x)

    def forward(self, x):
        if self._fusable(x):
            from .spectral_convolution import _attach
            fc0, fc1 = self.fcs
            y = Fh.channel_mlp(x.detach(), fc0.weight.detach(),
                               None if fc0.bias is None else fc0.bias.detach(), fc1.weight.detach(),
                               None if fc1.bias is None else fc1.bias.detach(), nat.SKIP_NONE, None,
                               None, None, nat.ACT_NONE,
                               bf16_products=Fh.autocast_bf16(x.device.type))
            return _attach(y, x, *self.parameters())
        reshaped = False
        size = list(x.shape)
        if x.ndim > 3:
            x = x.reshape((*size[:2], -1))
            reshaped = True
        for i, fc in enumerate(self.fcs):
            x = fc(x)
            if i < self.n_layers - 1:
                x = self.non_linearity(x)
            if self.dropout is not None:
                x = self.dropout[i](x)
        if reshaped:
            x = x.reshape((size[0], self.out_channels, *size[2:]))
        return x
