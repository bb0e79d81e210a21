"""FNOBlocks on MI355X (neuralop/layers/fno_block.py:18-481).

Post-activation forward (fno_block.py:327-381).  When the layer is
  SpectralConv (this package's) + linear / soft-gating (no bias) / identity /
  no skip, no norm, no stabilizer, GELU non-linearity, output size == input
the spectral conv, bias, skip, add and first GELU run as ONE library call
(fno_spectral_block_f32: fused 2D path or generic kernels).  When the channel
MLP is the default two-layer GELU MLP (no dropout) with a soft-gating /
identity / no skip and the kernel covers its widths, the MLP, its skip and the
second GELU run as a second call (fno_channel_mlp_f32).  Every other
configuration runs as torch ops around the HIP SpectralConv.
"""
from __future__ import annotations

from typing import List, Union

import torch
import torch.nn.functional as F
from torch import nn

from . import _native as nat
from . import functional as Fh
from .channel_mlp import ChannelMLP
from .complex import CGELU, ComplexValued, ctanh
from .skip_connections import Flattened1dConv, SoftGating, skip_connection
from .spectral_convolution import SpectralConv, _attach
from .utils import get_active_profiler, maybe_profile, validate_scaling_factor

Number = Union[int, float]


def _needs_grad(module: nn.Module, x: torch.Tensor) -> bool:
    return torch.is_grad_enabled() and (x.requires_grad or
                                        any(p.requires_grad for p in module.parameters()))


class InstanceNorm(nn.Module):
    """Instance norm over all spatial dims (neuralop normalization_layers)."""

    def __init__(self, **kwargs):
        super().__init__()
        self.kwargs = kwargs

    def forward(self, x):
        size = x.shape
        x = F.instance_norm(x, **self.kwargs)
        assert x.shape == size
        return x


class AdaIN(nn.Module):
    """Adaptive instance norm (neuralop/layers/normalization_layers.py:5-56):
    each channel normalised over its spatial points, then scaled and shifted
    by the two halves of mlp(embedding); the embedding is set before the
    forward.  The default mlp is Linear(embed_dim, 512), GELU,
    Linear(512, 2 in_channels)."""

    def __init__(self, embed_dim, in_channels, mlp=None, eps=1e-5):
        super().__init__()
        self.in_channels = in_channels
        self.embed_dim = embed_dim
        self.eps = eps
        self.mlp = mlp if mlp is not None else nn.Sequential(
            nn.Linear(embed_dim, 512), nn.GELU(), nn.Linear(512, 2 * in_channels))
        self.embedding = None

    def set_embedding(self, x):
        self.embedding = x.reshape(self.embed_dim)

    def forward(self, x):
        if self.embedding is None:
            raise RuntimeError("AdaIN: set the embedding (set_ada_in_embeddings) before the forward")
        scale, shift = self.mlp(self.embedding).split(self.in_channels)
        # one group per channel: instance statistics, per-channel affine
        return F.group_norm(x, self.in_channels, scale, shift, eps=self.eps)


class BatchNorm(nn.Module):
    def __init__(self, n_dim: int, num_features: int, **kwargs):
        super().__init__()
        cls = {1: nn.BatchNorm1d, 2: nn.BatchNorm2d, 3: nn.BatchNorm3d}.get(n_dim)
        if cls is None:
            raise NotImplementedError(f"BatchNorm for {n_dim} dims")
        self.norm = cls(num_features=num_features, **kwargs)

    def forward(self, x):
        return self.norm(x)


class FNOBlocks(nn.Module):
    def __init__(
        self,
        in_channels,
        out_channels,
        n_modes,
        resolution_scaling_factor=None,
        n_layers=1,
        max_n_modes=None,
        fno_block_precision="full",
        use_channel_mlp=True,
        channel_mlp_dropout=0,
        channel_mlp_expansion=0.5,
        non_linearity=F.gelu,
        stabilizer=None,
        norm=None,
        norm_groups=1,
        ada_in_features=None,
        preactivation=False,
        fno_skip="linear",
        channel_mlp_skip="soft-gating",
        complex_data=False,
        separable=False,
        factorization=None,
        rank=1.0,
        conv_module=SpectralConv,
        fixed_rank_modes=False,
        implementation="factorized",
        decomposition_kwargs=dict(),
        enforce_hermitian_symmetry=True,
    ):
        super().__init__()
        if isinstance(n_modes, int):
            n_modes = [n_modes]
        self._n_modes = n_modes
        self.n_dim = len(n_modes)
        self.resolution_scaling_factor = validate_scaling_factor(resolution_scaling_factor, self.n_dim,
                                                                 n_layers)
        self.max_n_modes = max_n_modes
        self.fno_block_precision = fno_block_precision
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.n_layers = n_layers
        self.stabilizer = stabilizer
        self.rank = rank
        self.factorization = factorization
        self.fixed_rank_modes = fixed_rank_modes
        self.decomposition_kwargs = decomposition_kwargs
        self.fno_skip = fno_skip
        self.channel_mlp_skip = channel_mlp_skip
        self.complex_data = complex_data
        self.use_channel_mlp = use_channel_mlp
        self.channel_mlp_expansion = channel_mlp_expansion
        self.channel_mlp_dropout = channel_mlp_dropout
        self.implementation = implementation
        self.separable = separable
        self.preactivation = preactivation
        self.ada_in_features = ada_in_features
        self.enforce_hermitian_symmetry = enforce_hermitian_symmetry
        self.complex_data = complex_data
        # complex data: CGELU and complex-linear wrappers (fno_block.py:169-171, :226-302)
        self.non_linearity = CGELU if complex_data else non_linearity

        self.convs = nn.ModuleList([
            conv_module(
                self.in_channels,
                self.out_channels,
                self.n_modes,
                resolution_scaling_factor=(self.resolution_scaling_factor[i]
                                           if resolution_scaling_factor is not None else None),
                max_n_modes=max_n_modes,
                rank=rank,
                fixed_rank_modes=fixed_rank_modes,
                implementation=implementation,
                separable=separable,
                factorization=factorization,
                fno_block_precision=fno_block_precision,
                decomposition_kwargs=decomposition_kwargs,
                complex_data=complex_data,
                **({"enforce_hermitian_symmetry": enforce_hermitian_symmetry}
                   if issubclass(conv_module, SpectralConv) else {}),
            )
            for i in range(n_layers)
        ])
        for i, conv in enumerate(self.convs):
            setattr(conv, "profile_prefix", f"fno_blocks/{i}/spectral_conv")

        if fno_skip is not None:
            self.fno_skips = nn.ModuleList([
                skip_connection(self.in_channels, self.out_channels, skip_type=fno_skip,
                                n_dim=self.n_dim) for _ in range(n_layers)])
        else:
            self.fno_skips = None

        if self.use_channel_mlp:
            self.channel_mlp = nn.ModuleList([
                ChannelMLP(in_channels=self.out_channels,
                           hidden_channels=round(self.out_channels * channel_mlp_expansion),
                           dropout=channel_mlp_dropout, n_dim=self.n_dim)
                for _ in range(n_layers)])
            if channel_mlp_skip is not None:
                self.channel_mlp_skips = nn.ModuleList([
                    skip_connection(self.in_channels, self.out_channels, skip_type=channel_mlp_skip,
                                    n_dim=self.n_dim) for _ in range(n_layers)])
            else:
                self.channel_mlp_skips = None

        self.n_norms = 2
        if norm is None:
            self.norm = None
        elif norm == "instance_norm":
            self.norm = nn.ModuleList([InstanceNorm() for _ in range(n_layers * self.n_norms)])
        elif norm == "group_norm":
            self.norm = nn.ModuleList([nn.GroupNorm(num_groups=norm_groups, num_channels=self.out_channels)
                                       for _ in range(n_layers * self.n_norms)])
        elif norm == "batch_norm":
            self.norm = nn.ModuleList([BatchNorm(n_dim=self.n_dim, num_features=self.out_channels)
                                       for _ in range(n_layers * self.n_norms)])
        elif norm == "ada_in":
            self.norm = nn.ModuleList([AdaIN(ada_in_features, self.out_channels)
                                       for _ in range(n_layers * self.n_norms)])
        else:
            raise ValueError(f"Got norm={norm} but expected None or one of "
                             "[instance_norm, group_norm, batch_norm, ada_in]")

        if complex_data:
            wrap = lambda ms: nn.ModuleList([ComplexValued(m) for m in ms]) if ms is not None else None
            self.fno_skips = wrap(self.fno_skips)
            if self.use_channel_mlp:
                self.channel_mlp = wrap(self.channel_mlp)
                self.channel_mlp_skips = wrap(self.channel_mlp_skips)
            self.norm = wrap(self.norm)

    # ------------------------------------------------------------------ fused
    def _fused_skip(self, index):
        """(skip_kind, skip_weight) if the fno skip can run inside the kernel."""
        if self.fno_skips is None:
            return nat.SKIP_NONE, None
        s = self.fno_skips[index]
        if isinstance(s, Flattened1dConv) and s.conv.bias is None:
            return nat.SKIP_LINEAR, s.conv.weight.reshape(s.conv.out_channels, -1)
        if isinstance(s, SoftGating) and s.bias is None:
            return nat.SKIP_SOFT_GATING, s.weight.reshape(-1)
        if isinstance(s, nn.Identity):
            return nat.SKIP_IDENTITY, None
        return None, None

    def _can_fuse(self, x, index, output_shape):
        conv = self.convs[index]
        if not isinstance(conv, SpectralConv) or not x.is_cuda or x.is_complex():
            return False
        if _needs_grad(self, x):
            return False   # the composed path carries the gradients
        if self.norm is not None or self.stabilizer is not None or self.preactivation:
            return False
        if conv.fno_block_precision in ("half", "mixed"):
            return False   # the conv's own forward restates the half arithmetic
        if self.non_linearity is not F.gelu:
            return False
        if output_shape is not None or conv.resolution_scaling_factor is not None:
            return False
        kind, _ = self._fused_skip(index)
        return kind is not None

    def set_ada_in_embeddings(self, *embeddings):
        """Embeddings of the Ada-IN norms (fno_block.py:304-321): one for all
        norm layers, or one per layer."""
        if self.norm is None:
            return
        if len(embeddings) == 1:
            embeddings = embeddings * len(self.norm)
        for n, e in zip(self.norm, embeddings):
            # a complex-data norm holds a real copy for each part
            for part in ((n.fr, n.fi) if isinstance(n, ComplexValued) else (n,)):
                part.set_embedding(e)

    def forward(self, x, index=0, output_shape=None):
        if self.preactivation:
            return self.forward_with_preactivation(x, index, output_shape)
        return self.forward_with_postactivation(x, index, output_shape)

    def _fused_mlp(self, x, index, output_shape):
        """(skip_kind, gate) when the channel MLP, its skip and the second
        activation of this layer can run as one fno_channel_mlp_f32 call, else
        None."""
        if not self.use_channel_mlp or not x.is_cuda or x.dtype not in (torch.float32,
                                                                        torch.bfloat16):
            return None
        if _needs_grad(self, x):
            return None
        if self.norm is not None or self.non_linearity is not F.gelu:
            return None
        conv = self.convs[index]
        if output_shape is not None or getattr(conv, "resolution_scaling_factor", None) is not None:
            return None
        mlp = self.channel_mlp[index]
        if (mlp.n_layers != 2 or mlp.non_linearity is not F.gelu or mlp.dropout is not None
                or mlp.in_channels != conv.out_channels):
            return None
        P = 1
        for s in x.shape[2:]:
            P *= s
        # x here is the block input (the skip input); the MLP input is the
        # spectral block's fresh output, allocated aligned
        if not Fh.channel_mlp_is_supported(mlp.in_channels, mlp.hidden_channels, mlp.out_channels, P,
                                           x):
            return None
        return self._mlp_skip(index)

    def _mlp_skip(self, index):
        """(skip_kind, gate) of the channel-MLP skip if a kernel can apply it."""
        conv = self.convs[index]
        if self.channel_mlp_skips is None:
            return nat.SKIP_NONE, None
        sk = self.channel_mlp_skips[index]
        if isinstance(sk, SoftGating):
            return nat.SKIP_SOFT_GATING, sk
        if isinstance(sk, nn.Identity) and conv.in_channels == conv.out_channels:
            return nat.SKIP_IDENTITY, None
        return None

    def bf16_layer_ok(self, batch, sizes, index=0) -> bool:
        """True if layer `index` runs as one fno_layer_bf16 call for a
        bfloat16 input [batch, C, *sizes] (under a bf16 autocast, without
        gradients): the structure _fused_layer needs, checked without a
        tensor, so FNO can choose bf16 activation storage up front."""
        if not self.use_channel_mlp or self.norm is not None or self.non_linearity is not F.gelu:
            return False
        if self.stabilizer is not None or self.preactivation:
            return False
        conv = self.convs[index]
        if not isinstance(conv, SpectralConv) or conv.resolution_scaling_factor is not None:
            return False
        if (conv.separable or conv.complex_data or conv._contract not in ("dense", "cp", "tt")
                or conv.in_channels != conv.out_channels):
            return False
        mlp = self.channel_mlp[index]
        if (mlp.n_layers != 2 or mlp.non_linearity is not F.gelu or mlp.dropout is not None
                or mlp.in_channels != conv.out_channels):
            return False
        kind, _ = self._fused_skip(index)
        mskip = self._mlp_skip(index)
        if kind is None or mskip is None:
            return False
        kept, _ = conv.window(list(sizes))
        return Fh.layer_is_fused(batch, conv.out_channels, mlp.hidden_channels, list(sizes), kept,
                                 kind, mskip[0], bf16=True)

    def _fused_layer(self, x, index, fused_mlp):
        """The whole layer (spectral block, its skip and activation, the
        channel MLP, its skip and the second activation) as one fno_layer_f32
        call, for the bf16-autocast forward (fno_layer_bf16, with a bfloat16
        output, for a bfloat16 x); None where that kernel does not cover the
        layer."""
        conv = self.convs[index]
        if (conv.separable or conv.complex_data or conv._contract not in ("dense", "cp", "tt")
                or conv.in_channels != conv.out_channels):
            return None
        if not Fh.autocast_bf16(x.device.type) or x.dtype not in (torch.float32, torch.bfloat16):
            return None
        kind, sw = self._fused_skip(index)
        mkind, gate = fused_mlp
        mlp = self.channel_mlp[index]
        sizes = list(x.shape[2:])
        kept, sl = conv.window(sizes)
        C, Ch = conv.out_channels, mlp.hidden_channels
        if not Fh.layer_is_fused(x.shape[0], C, Ch, sizes, kept, kind, mkind,
                                 bf16=x.dtype == torch.bfloat16):
            return None
        fc0, fc1 = mlp.fcs
        d = lambda t: None if t is None else t.detach()
        act = nat.ACT_GELU if index < (self.n_layers - 1) else nat.ACT_NONE
        y = Fh.fno_layer(x.detach(), conv.dense_window_weight(sl).detach(),
                         None if conv.bias is None else conv.bias.detach().reshape(-1), kept, kind,
                         d(sw), fc0.weight.detach().reshape(Ch, C), d(fc0.bias),
                         fc1.weight.detach().reshape(C, Ch), d(fc1.bias), mkind,
                         None if gate is None else gate.weight.detach().reshape(-1),
                         None if gate is None or gate.bias is None else gate.bias.detach().reshape(-1),
                         act, conv.fft_norm)
        params = [x] + list(conv.parameters()) + list(mlp.parameters())
        if self.fno_skips is not None:
            params += list(self.fno_skips[index].parameters())
        if gate is not None:
            params += list(gate.parameters())
        return _attach(y, *params)

    def forward_with_postactivation(self, x, index=0, output_shape=None):
        profiler = get_active_profiler()
        prefix = f"fno_blocks/{index}"
        fused_mlp = self._fused_mlp(x, index, output_shape)
        if fused_mlp is not None and self._can_fuse(x, index, output_shape):
            with maybe_profile(profiler, f"{prefix}/fno_layer", x.device):
                y = self._fused_layer(x, index, fused_mlp)
            if y is not None:
                return y
        if x.dtype == torch.bfloat16:
            # bf16 activation storage of the FNO forward, for a layer the
            # one-pass kernel does not cover: continue in fp32
            x = x.float()
            fused_mlp = self._fused_mlp(x, index, output_shape)
        x_in = x
        if self.use_channel_mlp and self.channel_mlp_skips is not None and fused_mlp is None:
            with maybe_profile(profiler, f"{prefix}/channel_mlp_skip", x.device):
                x_skip_channel_mlp = self.channel_mlp_skips[index](x)
                x_skip_channel_mlp = self.convs[index].transform(x_skip_channel_mlp,
                                                                 output_shape=output_shape)
        act0 = index < (self.n_layers - 1)
        if self._can_fuse(x, index, output_shape):
            kind, sw = self._fused_skip(index)
            with maybe_profile(profiler, f"{prefix}/spectral_block", x.device):
                x = self.convs[index]._forward_hip(x, None, kind, sw,
                                                   nat.ACT_GELU if act0 else nat.ACT_NONE)
        else:
            if self.fno_skips is not None:
                with maybe_profile(profiler, f"{prefix}/fno_skip", x.device):
                    x_skip_fno = self.fno_skips[index](x)
                    x_skip_fno = self.convs[index].transform(x_skip_fno, output_shape=output_shape)
            if self.stabilizer == "tanh":
                x = ctanh(x) if x.is_complex() else torch.tanh(x)
            x_fno = self.convs[index](x, output_shape=output_shape)
            if self.norm is not None:
                x_fno = self.norm[self.n_norms * index](x_fno)
            x = x_fno + x_skip_fno if self.fno_skips is not None else x_fno
            if act0:
                x = self.non_linearity(x)
        if fused_mlp is not None:
            # channel MLP + its skip + the second activation in one kernel
            kind, gate = fused_mlp
            mlp = self.channel_mlp[index]
            fc0, fc1 = mlp.fcs
            with maybe_profile(profiler, f"{prefix}/channel_mlp", x.device):
                y = Fh.channel_mlp(
                    x.detach(), fc0.weight.detach(), None if fc0.bias is None else fc0.bias.detach(),
                    fc1.weight.detach(), None if fc1.bias is None else fc1.bias.detach(), kind,
                    x_in.detach() if kind != nat.SKIP_NONE else None,
                    gate.weight.detach() if gate is not None else None,
                    gate.bias.detach() if gate is not None and gate.bias is not None else None,
                    nat.ACT_GELU if index < (self.n_layers - 1) else nat.ACT_NONE,
                    bf16_products=Fh.autocast_bf16(x.device.type))
            params = [x, x_in] + list(mlp.parameters())
            if gate is not None:
                params += list(gate.parameters())
            return _attach(y, *params)
        if self.use_channel_mlp:
            with maybe_profile(profiler, f"{prefix}/channel_mlp", x.device):
                x = self.channel_mlp[index](x)
            if self.channel_mlp_skips is not None:
                x = x + x_skip_channel_mlp
        if self.norm is not None:
            x = self.norm[self.n_norms * index + 1](x)
        if index < (self.n_layers - 1):
            with maybe_profile(profiler, f"{prefix}/activation_1", x.device):
                x = self.non_linearity(x)
        return x

    def forward_with_preactivation(self, x, index=0, output_shape=None):
        """fno_block.py:383-437 (torch glue around the HIP SpectralConv)."""
        x = self.non_linearity(x)
        if self.norm is not None:
            x = self.norm[self.n_norms * index](x)
        if self.fno_skips is not None:
            x_skip_fno = self.convs[index].transform(self.fno_skips[index](x), output_shape=output_shape)
        if self.use_channel_mlp and self.channel_mlp_skips is not None:
            x_skip_channel_mlp = self.convs[index].transform(self.channel_mlp_skips[index](x),
                                                             output_shape=output_shape)
        if self.stabilizer == "tanh":
            x = ctanh(x) if x.is_complex() else torch.tanh(x)
        x_fno = self.convs[index](x, output_shape=output_shape)
        x = x_fno + x_skip_fno if self.fno_skips is not None else x_fno
        if index < (self.n_layers - 1):
            x = self.non_linearity(x)
        if self.norm is not None:
            x = self.norm[self.n_norms * index + 1](x)
        if self.use_channel_mlp:
            x = self.channel_mlp[index](x)
            if self.channel_mlp_skips is not None:
                x = x + x_skip_channel_mlp
        return x

    @property
    def n_modes(self):
        return self._n_modes

    @n_modes.setter
    def n_modes(self, n_modes):
        for i in range(self.n_layers):
            self.convs[i].n_modes = n_modes
        self._n_modes = n_modes

    def get_block(self, indices):
        if self.n_layers == 1:
            raise ValueError("A single layer is parametrized, directly use the main class.")
        return SubModule(self, indices)

    def __getitem__(self, indices):
        return self.get_block(indices)


class SubModule(nn.Module):
    def __init__(self, main_module, indices):
        super().__init__()
        self.main_module = main_module
        self.indices = indices

    def forward(self, x):
        return self.main_module.forward(x, self.indices)
