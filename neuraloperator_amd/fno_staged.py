"""FNOStaged: FNO with per-layer Fourier mode counts
(neuralop/models/fno_staged.py:24-502), on the MI355X FNOBlocks.

The layers are FNOBlocks' own (so the fused spectral block and channel-MLP
calls apply per layer), with each layer's SpectralConv built at that layer's
n_modes / max_n_modes.  The module keeps the reference's top-level attribute
names (convs, fno_skips, channel_mlp, channel_mlp_skips, norm, lifting,
projection, positional_embedding).

no_br=True (fno_staged.py:110-115, :478-493): the reference runs its layers
on bit-reversed data, each SpectralConv replaced by a butterfly conv that
takes and returns bit-reversed order, so such a layer computes P B P (P the
bit reversal, B the natural-order block: every other op of the block is
pointwise or a norm over all points).  Where its butterfly conv falls back
(a dimension that is not a power of two, complex data, half precision, an
output_shape, another conv module) the natural conv sees permuted data.  The
forward here keeps the data in natural order and applies P only around the
layers of the second kind, so the common case needs no permutation at all
and the spectral work is the library's natural-order kernels either way.
"""
from __future__ import annotations

import warnings
from typing import List, Literal, Optional, Tuple, Union

import torch
import torch.nn.functional as F
from torch import nn

from .channel_mlp import ChannelMLP
from .complex import ComplexValued
from .embeddings import GridEmbeddingND
from .fno_block import FNOBlocks
from .padding import DomainPadding
from .spectral_convolution import SpectralConv
from .utils import get_active_profiler, maybe_profile

Number = Union[float, int]


class FNOStaged(FNOBlocks):
    def __init__(
        self,
        n_modes_per_layer: List[Tuple[int, ...]],
        in_channels: int,
        out_channels: int,
        hidden_channels: int,
        n_layers: Optional[int] = None,
        max_n_modes_per_layer: Optional[List[Tuple[int, ...]]] = None,
        lifting_channel_ratio: Number = 2,
        projection_channel_ratio: Number = 2,
        positional_embedding: Union[str, nn.Module] = "grid",
        non_linearity: nn.Module = F.gelu,
        norm: Literal["ada_in", "group_norm", "instance_norm", "batch_norm"] = None,
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
        factorization: str = None,
        rank: float = 1.0,
        fixed_rank_modes: bool = False,
        implementation: str = "factorized",
        decomposition_kwargs: dict = None,
        separable: bool = False,
        preactivation: bool = False,
        conv_module: nn.Module = SpectralConv,
        enforce_hermitian_symmetry: bool = True,
        no_br: bool = False,
    ):
        if decomposition_kwargs is None:
            decomposition_kwargs = {}
        # argument checks of fno_staged.py:70-86
        if n_layers is not None and n_layers != len(n_modes_per_layer):
            raise ValueError(
                f"Got n_layers={n_layers} but n_modes_per_layer has length {len(n_modes_per_layer)}")
        n_modes_per_layer = [list(m) for m in n_modes_per_layer]
        L = len(n_modes_per_layer)
        if max_n_modes_per_layer is None:
            max_n_modes_per_layer = n_modes_per_layer
        if len(max_n_modes_per_layer) != L:
            raise ValueError(
                "max_n_modes_per_layer must be None or have the same length as n_modes_per_layer")
        max_n_modes_per_layer = [list(m) for m in max_n_modes_per_layer]
        if no_br and resolution_scaling_factor is not None:
            raise NotImplementedError("no_br=True with resolution scaling is not built")
        pad_on = domain_padding is not None and (
            (isinstance(domain_padding, list) and sum(domain_padding) > 0)
            or (isinstance(domain_padding, (float, int)) and domain_padding > 0))
        # the padding takes the factor as given (fno_staged.py:143-157)
        raw_scaling = resolution_scaling_factor
        if resolution_scaling_factor is not None and isinstance(resolution_scaling_factor,
                                                                (float, int)):
            resolution_scaling_factor = [resolution_scaling_factor] * L

        super().__init__(
            in_channels=hidden_channels, out_channels=hidden_channels,
            n_modes=n_modes_per_layer[0], resolution_scaling_factor=resolution_scaling_factor,
            n_layers=L, max_n_modes=max_n_modes_per_layer[0],
            fno_block_precision=fno_block_precision, use_channel_mlp=use_channel_mlp,
            channel_mlp_dropout=channel_mlp_dropout, channel_mlp_expansion=channel_mlp_expansion,
            non_linearity=non_linearity, stabilizer=stabilizer, norm=norm, norm_groups=norm_groups,
            preactivation=preactivation, fno_skip=fno_skip, channel_mlp_skip=channel_mlp_skip,
            complex_data=complex_data, separable=separable, factorization=factorization, rank=rank,
            conv_module=conv_module, fixed_rank_modes=fixed_rank_modes,
            implementation=implementation, decomposition_kwargs=decomposition_kwargs,
            enforce_hermitian_symmetry=enforce_hermitian_symmetry)

        self.n_dim = len(n_modes_per_layer[0])
        self.n_modes_per_layer = n_modes_per_layer
        self.max_n_modes_per_layer = max_n_modes_per_layer
        self.hidden_channels = hidden_channels
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.lifting_channel_ratio = lifting_channel_ratio
        self.lifting_channels = int(lifting_channel_ratio * hidden_channels)
        self.projection_channel_ratio = projection_channel_ratio
        self.projection_channels = int(projection_channel_ratio * hidden_channels)
        self.no_br = no_br
        self._natural_convs = conv_module is SpectralConv

        # per-layer spectral convolutions (fno_staged.py:162-190)
        self.convs = nn.ModuleList([
            conv_module(
                hidden_channels, hidden_channels, n_modes=n_modes_per_layer[i],
                max_n_modes=max_n_modes_per_layer[i],
                resolution_scaling_factor=(resolution_scaling_factor[i]
                                           if resolution_scaling_factor is not None else None),
                rank=rank, fixed_rank_modes=fixed_rank_modes, implementation=implementation,
                separable=separable, factorization=factorization,
                fno_block_precision=fno_block_precision, decomposition_kwargs=decomposition_kwargs,
                complex_data=complex_data,
                **({"enforce_hermitian_symmetry": enforce_hermitian_symmetry}
                   if issubclass(conv_module, SpectralConv) else {}))
            for i in range(L)])
        for i, conv in enumerate(self.convs):
            setattr(conv, "profile_prefix", f"fno_blocks/{i}/spectral_conv")

        if positional_embedding == "grid":
            self.positional_embedding = GridEmbeddingND(
                in_channels=in_channels, dim=self.n_dim, grid_boundaries=[[0.0, 1.0]] * self.n_dim)
        elif isinstance(positional_embedding, GridEmbeddingND):
            self.positional_embedding = positional_embedding
        elif positional_embedding is None:
            self.positional_embedding = None
        else:
            raise ValueError(
                f"Error: tried to instantiate FNO positional embedding with {positional_embedding}, "
                "expected one of 'grid', GridEmbeddingND")
        self.domain_padding = (DomainPadding(domain_padding=domain_padding,
                                             resolution_scaling_factor=raw_scaling)
                               if pad_on else None)

        lifting_in = in_channels + (self.n_dim if self.positional_embedding is not None else 0)
        self.lifting = ChannelMLP(in_channels=lifting_in, out_channels=hidden_channels,
                                  hidden_channels=self.lifting_channels, n_layers=2, n_dim=self.n_dim,
                                  non_linearity=non_linearity)
        self.projection = ChannelMLP(in_channels=hidden_channels, out_channels=out_channels,
                                     hidden_channels=self.projection_channels, n_layers=2,
                                     n_dim=self.n_dim, non_linearity=non_linearity)
        if complex_data:   # fno_staged.py:349-366
            self.lifting = ComplexValued(self.lifting)
            self.projection = ComplexValued(self.projection)

    @staticmethod
    def _bitrev_spatial(x: torch.Tensor) -> torch.Tensor:
        """Each power-of-two spatial dimension permuted into bit-reversed order
        (an involution); other dimensions unchanged (fno_staged.py:325-341)."""
        for dim in range(2, x.ndim):
            n = x.shape[dim]
            if n > 1 and (n & (n - 1)) == 0:
                bits = n.bit_length() - 1
                idx = torch.arange(n, device=x.device)
                rev = torch.zeros_like(idx)
                for i in range(bits):
                    rev = (rev << 1) | ((idx >> i) & 1)
                x = torch.index_select(x, dim, rev)
        return x

    def _butterfly_layer(self, x, output_shape) -> bool:
        """Whether the reference's butterfly conv runs this layer
        (butterfly_fft.py:109-122), so that the layer is P B P."""
        return (self._natural_convs and output_shape is None and not self.complex_data
                and self.fno_block_precision == "full"
                and all(n > 0 and (n & (n - 1)) == 0 for n in x.shape[2:]))

    def forward(self, x, output_shape=None, **kwargs):
        """fno_staged.py:460-502."""
        if kwargs:
            warnings.warn(
                f"FNOStaged.forward() received unexpected keyword arguments: {list(kwargs.keys())}. "
                "These arguments will be ignored.", UserWarning, stacklevel=2)
        if output_shape is None:
            output_shape = [None] * self.n_layers
        elif isinstance(output_shape, tuple):
            output_shape = [None] * (self.n_layers - 1) + [output_shape]
        profiler = get_active_profiler()
        if self.positional_embedding is not None:
            with maybe_profile(profiler, "fno/positional_embedding", x.device):
                x = self.positional_embedding(x)
        with maybe_profile(profiler, "fno/lifting", x.device):
            x = self.lifting(x)
        if self.domain_padding is not None:
            with maybe_profile(profiler, "fno/domain_padding/pad", x.device):
                x = self.domain_padding.pad(x)
        # permuted: x holds the reference's bit-reversed data (else its
        # natural-order view)
        permuted = False
        for layer_idx in range(self.n_layers):
            if self.no_br and not self._butterfly_layer(x, output_shape[layer_idx]) and not permuted:
                x, permuted = self._bitrev_spatial(x), True
            elif self.no_br and self._butterfly_layer(x, output_shape[layer_idx]) and permuted:
                x, permuted = self._bitrev_spatial(x), False
            x = super().forward(x, layer_idx, output_shape=output_shape[layer_idx])
        if permuted:
            x = self._bitrev_spatial(x)
        if self.domain_padding is not None:
            with maybe_profile(profiler, "fno/domain_padding/unpad", x.device):
                x = self.domain_padding.unpad(x)
        with maybe_profile(profiler, "fno/projection", x.device):
            x = self.projection(x)
        return x
