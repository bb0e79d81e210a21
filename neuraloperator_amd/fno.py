"""FNO and TFNO models (neuralop/models/fno.py:26-485) built on the MI355X
FNOBlocks.  Lifting / projection channel MLPs and the grid embedding are
torch ops; every Fourier layer runs through libfnohip.so."""
from __future__ import annotations

import warnings
from typing import List, Literal, Tuple, Union

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _native as nat
from . import functional as Fh
from .channel_mlp import ChannelMLP
from .embeddings import GridEmbeddingND
from .complex import ComplexValued
from .fno_block import FNOBlocks
from .padding import DomainPadding
from .spectral_convolution import SpectralConv
from .utils import get_active_profiler, maybe_profile

Number = Union[float, int]


class FNO(nn.Module):
    def __init__(
        self,
        n_modes: Tuple[int, ...],
        in_channels: int,
        out_channels: int,
        hidden_channels: int,
        n_layers: int = 4,
        lifting_channel_ratio: Number = 2,
        projection_channel_ratio: Number = 2,
        positional_embedding: Union[str, nn.Module] = "grid",
        non_linearity: nn.Module = F.gelu,
        norm: Literal["ada_in", "group_norm", "instance_norm"] = None,
        norm_groups: int = 1,
        complex_data: bool = False,
        use_channel_mlp: bool = True,
        channel_mlp_dropout: float = 0,
        channel_mlp_expansion: float = 0.5,
        channel_mlp_skip: Literal["linear", "identity", "soft-gating", None] = "soft-gating",
        fno_skip: Literal["linear", "identity", "soft-gating", None] = "linear",
        resolution_scaling_factor: Union[Number, List[Number]] = None,
        domain_padding: Union[Number, List[Number]] = None,
        fno_block_precision: str = "full",
        stabilizer: str = None,
        max_n_modes: Tuple[int, ...] = None,
        factorization: str = None,
        rank: float = 1.0,
        fixed_rank_modes: bool = False,
        implementation: str = "factorized",
        decomposition_kwargs: dict = None,
        separable: bool = False,
        preactivation: bool = False,
        conv_module: nn.Module = SpectralConv,
        enforce_hermitian_symmetry: bool = True,
    ):
        if decomposition_kwargs is None:
            decomposition_kwargs = {}
        super().__init__()
        self.n_dim = len(n_modes)
        self._n_modes = n_modes
        self.hidden_channels = hidden_channels
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.n_layers = n_layers
        self.lifting_channel_ratio = lifting_channel_ratio
        self.lifting_channels = int(lifting_channel_ratio * self.hidden_channels)
        self.projection_channel_ratio = projection_channel_ratio
        self.projection_channels = int(projection_channel_ratio * self.hidden_channels)
        self.non_linearity = non_linearity
        self.rank = rank
        self.factorization = factorization
        self.fixed_rank_modes = fixed_rank_modes
        self.decomposition_kwargs = decomposition_kwargs
        self.fno_skip = (fno_skip,)
        self.channel_mlp_skip = (channel_mlp_skip,)
        self.implementation = implementation
        self.separable = separable
        self.preactivation = preactivation
        self.complex_data = complex_data
        self.fno_block_precision = fno_block_precision

        if positional_embedding == "grid":
            self.positional_embedding = GridEmbeddingND(
                in_channels=self.in_channels, dim=self.n_dim,
                grid_boundaries=[[0.0, 1.0]] * self.n_dim)
        elif isinstance(positional_embedding, GridEmbeddingND):
            self.positional_embedding = positional_embedding
        elif positional_embedding is None:
            self.positional_embedding = None
        else:
            raise ValueError(
                f"Error: tried to instantiate FNO positional embedding with {positional_embedding}, "
                "expected one of 'grid', GridEmbeddingND")

        if domain_padding is not None and (
                (isinstance(domain_padding, list) and sum(domain_padding) > 0)
                or (isinstance(domain_padding, (float, int)) and domain_padding > 0)):
            self.domain_padding = DomainPadding(domain_padding=domain_padding,
                                                resolution_scaling_factor=resolution_scaling_factor)
        else:
            self.domain_padding = None

        if resolution_scaling_factor is not None and isinstance(resolution_scaling_factor, (float, int)):
            resolution_scaling_factor = [resolution_scaling_factor] * self.n_layers
        self.resolution_scaling_factor = resolution_scaling_factor

        self.fno_blocks = FNOBlocks(
            in_channels=hidden_channels, out_channels=hidden_channels, n_modes=self.n_modes,
            resolution_scaling_factor=resolution_scaling_factor, use_channel_mlp=use_channel_mlp,
            channel_mlp_dropout=channel_mlp_dropout, channel_mlp_expansion=channel_mlp_expansion,
            non_linearity=non_linearity, stabilizer=stabilizer, norm=norm, norm_groups=norm_groups,
            preactivation=preactivation, fno_skip=fno_skip, channel_mlp_skip=channel_mlp_skip,
            complex_data=complex_data, max_n_modes=max_n_modes,
            fno_block_precision=fno_block_precision, rank=rank, fixed_rank_modes=fixed_rank_modes,
            implementation=implementation, separable=separable, factorization=factorization,
            decomposition_kwargs=decomposition_kwargs, conv_module=conv_module, n_layers=n_layers,
            enforce_hermitian_symmetry=enforce_hermitian_symmetry)

        lifting_in_channels = self.in_channels + (self.n_dim if self.positional_embedding is not None else 0)
        self.lifting = ChannelMLP(in_channels=lifting_in_channels, out_channels=self.hidden_channels,
                                  hidden_channels=self.lifting_channels, n_layers=2, n_dim=self.n_dim,
                                  non_linearity=non_linearity)
        self.projection = ChannelMLP(in_channels=self.hidden_channels, out_channels=out_channels,
                                     hidden_channels=self.projection_channels, n_layers=2,
                                     n_dim=self.n_dim, non_linearity=non_linearity)
        if complex_data:   # fno.py:327-340
            self.lifting = ComplexValued(self.lifting)
            self.projection = ComplexValued(self.projection)

    def forward(self, x, output_shape=None, **kwargs):
        """fno.py:342-408."""
        if kwargs:
            warnings.warn(f"FNO.forward() received unexpected keyword arguments: {list(kwargs.keys())}. "
                          "These arguments will be ignored.", UserWarning, stacklevel=2)
        if output_shape is None:
            output_shape = [None] * self.n_layers
        elif isinstance(output_shape, tuple):
            output_shape = [None] * (self.n_layers - 1) + [output_shape]
        profiler = get_active_profiler()
        if self.positional_embedding is not None:
            with maybe_profile(profiler, "fno/positional_embedding", x.device):
                x = self.positional_embedding(x)
        bf16_io = self._bf16_storage(x, output_shape)
        with maybe_profile(profiler, "fno/lifting", x.device):
            x = self._mlp_bf16(self.lifting, x, y_bf16=True) if bf16_io else self.lifting(x)
        if self.domain_padding is not None:
            with maybe_profile(profiler, "fno/domain_padding/pad", x.device):
                x = self.domain_padding.pad(x)
        for layer_idx in range(self.n_layers):
            x = self.fno_blocks(x, layer_idx, output_shape=output_shape[layer_idx])
        if self.domain_padding is not None:
            with maybe_profile(profiler, "fno/domain_padding/unpad", x.device):
                x = self.domain_padding.unpad(x)
        with maybe_profile(profiler, "fno/projection", x.device):
            if x.dtype == torch.bfloat16 and self._mlp_io_ok(self.projection, x, x_bf16=True):
                x = self._mlp_bf16(self.projection, x, y_bf16=False)
            else:
                x = self.projection(x.float() if bf16_io else x)
        return x

    # ---- bf16 activation storage: under torch.autocast(dtype=bfloat16),
    # without gradients, when the layers run as one-pass bf16 layers
    # (fno_layer_bf16), the activations from the lifting to the projection
    # are kept in bfloat16: every layer reads and writes half the bytes.  The
    # arithmetic is that of the fp32 autocast forward, on values rounded to
    # bf16 at each layer boundary (the lifting's output is bf16 in the
    # reference's autocast forward too: a Conv1d output).
    def _mlp_io_ok(self, mlp, x, x_bf16=False, y_bf16=False) -> bool:
        if not isinstance(mlp, ChannelMLP) or mlp.n_layers != 2 or mlp.dropout is not None:
            return False
        if mlp.non_linearity is not F.gelu:
            return False
        P = 1
        for s in x.shape[2:]:
            P *= s
        return Fh.channel_mlp_io_is_supported(mlp.in_channels, mlp.hidden_channels,
                                              mlp.out_channels, P, x_bf16, y_bf16)

    def _bf16_storage(self, x, output_shape) -> bool:
        if not x.is_cuda or x.is_complex() or not Fh.autocast_bf16(x.device.type):
            return False
        if torch.is_grad_enabled() and (x.requires_grad or
                                        any(p.requires_grad for p in self.parameters())):
            return False
        if self.domain_padding is not None or any(o is not None for o in output_shape):
            return False
        if not self._mlp_io_ok(self.lifting, x, y_bf16=True):
            return False
        return self.fno_blocks.bf16_layer_ok(x.shape[0], x.shape[2:], 0)

    @staticmethod
    def _mlp_bf16(mlp, x, y_bf16):
        fc0, fc1 = mlp.fcs
        d = lambda t: None if t is None else t.detach()
        return Fh.channel_mlp_io(x.detach(), d(fc0.weight).reshape(fc0.out_channels, -1),
                                 d(fc0.bias), d(fc1.weight).reshape(fc1.out_channels, -1),
                                 d(fc1.bias), nat.ACT_NONE, y_bf16)

    @property
    def n_modes(self):
        return self._n_modes

    @n_modes.setter
    def n_modes(self, n_modes):
        self.fno_blocks.n_modes = n_modes
        self._n_modes = n_modes


class TFNO(FNO):
    """FNO with a Tucker-factorized spectral weight by default (fno.py:450-485)."""

    def __init__(self, *args, **kwargs):
        kwargs.setdefault("factorization", "Tucker")
        kwargs.setdefault("rank", 0.1)
        super().__init__(*args, **kwargs)
