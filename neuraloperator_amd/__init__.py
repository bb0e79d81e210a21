"""MI355X-native FNO spectral block: drop-in SpectralConv / FNOBlocks / FNO /
TFNO whose Fourier layers run on hand-written gfx950 HIP kernels
(libfnohip.so, C ABI in include/fno_hip.h)."""
from .spectral_convolution import BaseSpectralConv, SpectralConv, get_contract_fun
from .fno_block import FNOBlocks
from .fno import FNO, TFNO
from .fno_staged import FNOStaged
from .skip_connections import Flattened1dConv, SoftGating, skip_connection
from .channel_mlp import ChannelMLP
from .embeddings import GridEmbeddingND, regular_grid_nd
from .factorized_tensors import FactorizedTensor
from .utils import TimingProfiler, profiling, get_active_profiler, maybe_profile, validate_scaling_factor

__all__ = [
    "BaseSpectralConv", "SpectralConv", "get_contract_fun", "FNOBlocks", "FNO", "TFNO", "FNOStaged",
    "Flattened1dConv", "SoftGating", "skip_connection", "ChannelMLP", "GridEmbeddingND",
    "regular_grid_nd", "FactorizedTensor", "TimingProfiler", "profiling", "get_active_profiler",
    "maybe_profile", "validate_scaling_factor",
]
