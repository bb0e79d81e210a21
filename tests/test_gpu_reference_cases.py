"""The reference's own test cases for the FNO path, run on the HIP modules:
neuralop/layers/tests/test_spectral_convolution.py, test_fno_block.py and
neuralop/models/tests/test_fno.py.  Each keeps the reference test's
assertions (shapes, dtypes, dense == factorized, gradients reaching every
parameter); where the oracle can say more, values are checked against it."""
import pytest
import torch
import torch.nn.functional as F

import neuraloperator_amd as na
from neuraloperator_amd.factorized_tensors import FactorizedTensor
from neuraloperator_amd.resample import spectral_resample
from oracle import spectral_ref as R

pytestmark = pytest.mark.gpu

TOL = 1e-4


def rel_err(y, ref):
    y = y.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return ((y - ref).abs().max() / ref.abs().max()).item()


# ------------------------------------------------- test_spectral_convolution
@pytest.mark.parametrize("factorization", ["Dense", "CP", "Tucker", "TT"])
@pytest.mark.parametrize("implementation", ["factorized", "reconstructed"])
@pytest.mark.parametrize("separable", [False, True])
@pytest.mark.parametrize("dim", [1, 2, 3, 4])
@pytest.mark.parametrize("complex_data", [False, True])
def test_spectral_conv_factorizations(factorization, implementation, separable, dim, complex_data,
                                      cuda_device):
    """test_spectral_convolution.py:7-86: a factorized conv equals the dense
    conv holding its reconstructed weight; changing n_modes keeps the output
    shape; resolution scaling 0.5 / 2 resizes the output."""
    torch.manual_seed(40)
    modes, incremental = (10, 8, 6, 6), (6, 6, 4, 4)
    dtype = torch.cfloat if complex_data else torch.float32
    conv = na.SpectralConv(3, 3, modes[:dim], bias=False, implementation=implementation,
                           factorization=factorization, complex_data=complex_data,
                           separable=separable).to(cuda_device)
    conv_dense = na.SpectralConv(3, 3, modes[:dim], bias=False, implementation="reconstructed",
                                 factorization=None, complex_data=complex_data).to(cuda_device)
    x = torch.randn(2, 3, *(12,) * dim, dtype=dtype).to(cuda_device)
    assert torch.is_complex(conv.weight) and torch.is_complex(conv_dense.weight)
    if not separable:
        conv_dense.weight = FactorizedTensor.from_tensor(conv.weight.to_tensor(), rank=None,
                                                         factorization="ComplexDense")
    res_dense = conv_dense(x)
    res = conv(x)
    if not separable:
        torch.testing.assert_close(res_dense, res)
    shape = res.shape
    conv.n_modes = incremental[:dim]
    assert conv(x).shape == shape
    xr = torch.randn(2, 3, *(12,) * dim).to(cuda_device)
    down = na.SpectralConv(3, 4, modes[:dim], resolution_scaling_factor=0.5).to(cuda_device)
    assert list(down(xr).shape[2:]) == [6] * dim
    up = na.SpectralConv(3, 4, modes[:dim], resolution_scaling_factor=2).to(cuda_device)
    res = up(xr)
    assert res.shape[1] == 4 and list(res.shape[2:]) == [24] * dim


@pytest.mark.parametrize("enforce_hermitian_symmetry", [True, False])
@pytest.mark.parametrize("dim", [1, 2, 3])
@pytest.mark.parametrize("spatial_size", [8, 9])
@pytest.mark.parametrize("resolution_scaling_factor", [None, 0.5, 2])
@pytest.mark.parametrize("modes", [(4, 4, 4), (4, 5, 7)])
def test_spectral_conv_sizes(enforce_hermitian_symmetry, dim, spatial_size, resolution_scaling_factor,
                             modes, cuda_device):
    """test_spectral_convolution.py:89-116 (shape, dtype, real output) on
    even and odd grids, with the values checked against the oracle."""
    torch.manual_seed(41)
    modes = modes[:dim]
    size = [spatial_size] * dim
    out_size = size if resolution_scaling_factor is None else \
        [round(s * resolution_scaling_factor) for s in size]
    conv = na.SpectralConv(3, 4, modes, enforce_hermitian_symmetry=enforce_hermitian_symmetry,
                           resolution_scaling_factor=resolution_scaling_factor).to(cuda_device)
    x = torch.randn(2, 3, *size)
    res = conv(x.to(cuda_device))
    assert res.shape == (2, 4, *out_size)
    assert res.dtype == torch.float32 and not torch.is_complex(res)
    ref = R.spectral_conv_forward(x.double(), conv.weight.to_tensor().detach().cpu().to(torch.complex128),
                                  conv.bias.detach().cpu().double(), conv.n_modes, conv.max_n_modes,
                                  output_shape=out_size,
                                  enforce_hermitian_symmetry=enforce_hermitian_symmetry)
    assert rel_err(res, ref) <= TOL


# ----------------------------------------------------------- test_fno_block
@pytest.mark.parametrize("old,new", [((10, 10, 10), (5, 5, 5)), ((10, 10, 10), (20, 20, 20)),
                                     ((9, 11, 13), (12, 7, 20)), ((7, 8, 9), (7, 16, 5)),
                                     ((6, 6, 6, 8), (12, 9, 6, 4))])
def test_spectral_resample(old, new, cuda_device):
    """The 3D+ skip resample (resample.py:54-69) against the oracle, odd and
    even grids, up and down."""
    print(f"resample {old} -> {new}", flush=True)
    x = torch.randn(2, 3, *old, generator=torch.Generator().manual_seed(42))
    with torch.no_grad():
        y = spectral_resample(x.to(cuda_device), new)
    assert list(y.shape) == [2, 3, *new]
    assert rel_err(y, R.spectral_resample(x.double(), new)) <= TOL


def test_resample_reference(cuda_device):
    """test_resample.py:5-27: bicubic 2D on two axes, spectral 3D on three
    (scales 0.5, 3, 4), shapes as the reference asserts and values against
    the oracle."""
    from neuraloperator_amd.resample import resample
    g = torch.Generator().manual_seed(43)
    a = torch.randn(10, 20, 40, 50, generator=g).to(cuda_device)
    b = resample(a, [2, 3], [-2, -1])
    assert b.shape[-1] == 3 * a.shape[-1] and b.shape[-2] == 2 * a.shape[-2]
    a = torch.randn(2, 3, 40, 50, 60, generator=g)
    with torch.no_grad():
        b = resample(a.to(cuda_device), [0.5, 3, 4], [-3, -2, -1])
    assert b.shape[-1] == 4 * a.shape[-1] and b.shape[-2] == 3 * a.shape[-2] and \
        b.shape[-3] == int(0.5 * a.shape[-3])
    assert rel_err(b, R.spectral_resample(a.double(), list(b.shape[2:]))) <= TOL


def test_fno_block_resolution_scaling(cuda_device):
    """test_fno_block.py:6-68: the n_modes setter, and outputs resized by
    0.5 and 2 in 1-4 dims."""
    max_n_modes, n_modes, size = [8, 8, 8, 8], [4, 4, 4, 4], [10] * 4
    for dim in [1, 2, 3, 4]:
        block = na.FNOBlocks(3, 4, max_n_modes[:dim], max_n_modes=max_n_modes[:dim], n_layers=1,
                             channel_mlp_skip="linear").to(cuda_device)
        assert block.convs[0].n_modes[:-1] == max_n_modes[:dim - 1]
        assert block.convs[0].n_modes[-1] == max_n_modes[dim - 1] // 2 + 1
        block.n_modes = n_modes[:dim]
        assert block.convs[0].n_modes[:-1] == n_modes[:dim - 1]
        assert block.convs[0].n_modes[-1] == n_modes[dim - 1] // 2 + 1
        block.n_modes = max_n_modes[:dim]
        assert block.convs[0].n_modes[-1] == max_n_modes[dim - 1] // 2 + 1
        x = torch.randn(2, 3, *size[:dim]).to(cuda_device)
        block = na.FNOBlocks(3, 4, n_modes[:dim], n_layers=1, resolution_scaling_factor=0.5,
                             use_channel_mlp=True, channel_mlp_dropout=0, channel_mlp_expansion=0.5,
                             channel_mlp_skip="linear").to(cuda_device)
        assert list(block(x).shape[2:]) == [m // 2 for m in size[:dim]]
        block = na.FNOBlocks(3, 4, n_modes[:dim], n_layers=1, resolution_scaling_factor=2,
                             channel_mlp_dropout=0, channel_mlp_expansion=0.5,
                             channel_mlp_skip="linear").to(cuda_device)
        res = block(x)
        assert res.shape[1] == 4 and list(res.shape[2:]) == [m * 2 for m in size[:dim]]


@pytest.mark.parametrize("n_dim", [1, 2, 3, 4])
@pytest.mark.parametrize("norm", ["instance_norm", "ada_in", "group_norm", "batch_norm"])
def test_fno_block_norm(norm, n_dim, cuda_device):
    """test_fno_block.py:71-101."""
    modes, size = (8, 8, 8), [10] * 3
    block = na.FNOBlocks(3, 4, modes[:n_dim], n_layers=1, norm=norm, ada_in_features=4,
                         channel_mlp_dropout=0, channel_mlp_expansion=0.5,
                         channel_mlp_skip="linear").to(cuda_device)
    if norm == "ada_in":
        block.set_ada_in_embeddings(torch.randn(4).to(cuda_device))
    x = torch.randn(2, 3, *size[:n_dim]).to(cuda_device)
    assert list(block(x).shape[2:]) == size[:n_dim]


@pytest.mark.parametrize("norm_groups", [1, 2, 4, 8])
def test_fno_block_group_norm(norm_groups, cuda_device):
    """test_fno_block.py:104-125, plus a forward."""
    block = na.FNOBlocks(16, 16, (8, 8, 8), n_layers=1, norm="group_norm",
                         norm_groups=norm_groups).to(cuda_device)
    for layer in block.norm:
        assert isinstance(layer, torch.nn.GroupNorm)
        assert layer.num_groups == norm_groups and layer.num_channels == 16
    assert block(torch.randn(2, 16, 10, 10, 10).to(cuda_device)).shape == (2, 16, 10, 10, 10)


@pytest.mark.parametrize("n_dim", [1, 2, 3])
def test_fno_block_complex_data(n_dim, cuda_device):
    """test_fno_block.py:128-151."""
    block = na.FNOBlocks(3, 4, (8, 8, 8)[:n_dim], n_layers=1, channel_mlp_dropout=0,
                         channel_mlp_expansion=0.5, channel_mlp_skip="linear",
                         complex_data=True).to(cuda_device)
    x = torch.randn(2, 3, *[10] * n_dim, dtype=torch.cfloat).to(cuda_device)
    res = block(x)
    assert list(res.shape[2:]) == [10] * n_dim and res.is_complex()


@pytest.mark.parametrize("preactivation", [False, True])
@pytest.mark.parametrize("fno_skip", ["linear", None])
@pytest.mark.parametrize("channel_mlp_skip", ["linear", None])
def test_fno_block_skip_connections(fno_skip, channel_mlp_skip, preactivation, cuda_device):
    """test_fno_block.py:154-229, with and without the channel MLP."""
    size = [10, 10, 10]
    x = torch.randn(2, 3, *size).to(cuda_device)
    for use_mlp in (True, False):
        block = na.FNOBlocks(3, 4, (8, 8, 8), n_layers=2, fno_skip=fno_skip,
                             channel_mlp_skip=channel_mlp_skip, use_channel_mlp=use_mlp,
                             channel_mlp_expansion=0.5, channel_mlp_dropout=0.0,
                             preactivation=preactivation).to(cuda_device)
        assert block(x).shape == (2, 4, *size)


# ------------------------------------------------------------------ test_fno
@pytest.mark.parametrize("resolution_scaling_factor", [[2, 1, 1], [1, 2, 1], [1, 1, 2], [1, 2, 2],
                                                       [1, 0.5, 1]])
def test_fno_superresolution(resolution_scaling_factor, cuda_device):
    """test_fno.py:87-130 (CP weights, reconstructed)."""
    model = na.FNO(in_channels=3, out_channels=1, n_modes=(5, 5), hidden_channels=9,
                   factorization="cp", implementation="reconstructed", rank=0.2,
                   resolution_scaling_factor=resolution_scaling_factor, n_layers=3).to(cuda_device)
    out = model(torch.randn(3, 3, 12, 12).to(cuda_device))
    factor = 1
    for f in resolution_scaling_factor:
        factor *= f
    assert list(out.shape) == [3, 1] + [int(round(factor * 12))] * 2


@pytest.mark.parametrize("norm", [None, "group_norm", "instance_norm"])
@pytest.mark.parametrize("use_channel_mlp", [True, False])
@pytest.mark.parametrize("channel_mlp_skip", ["linear", "identity", "soft-gating", None])
@pytest.mark.parametrize("fno_skip", ["linear", "identity", "soft-gating", None])
@pytest.mark.parametrize("complex_data", [True, False])
def test_fno_advanced_params(norm, use_channel_mlp, channel_mlp_skip, fno_skip, complex_data,
                             cuda_device):
    """test_fno.py:133-177: forward shape and backward."""
    dtype = torch.cfloat if complex_data else torch.float32
    model = na.FNO(in_channels=3, out_channels=1, n_modes=(5, 5), hidden_channels=9, n_layers=2,
                   norm=norm, use_channel_mlp=use_channel_mlp, channel_mlp_skip=channel_mlp_skip,
                   fno_skip=fno_skip, complex_data=complex_data).to(cuda_device)
    out = model(torch.randn(3, 3, 12, 12, dtype=dtype).to(cuda_device))
    assert list(out.shape) == [3, 1, 12, 12]
    loss = out.sum()
    if complex_data:
        loss = (loss.real ** 2 + loss.imag ** 2) ** 0.5
    loss.backward()


def test_fno_group_norm(cuda_device):
    """test_fno.py:180-212."""
    model = na.FNO(in_channels=3, out_channels=1, n_modes=(5, 5), hidden_channels=16, n_layers=2,
                   norm="group_norm", norm_groups=4).to(cuda_device)
    assert list(model(torch.randn(2, 3, 12, 12).to(cuda_device)).shape) == [2, 1, 12, 12]
    for layer in model.fno_blocks.norm:
        assert isinstance(layer, torch.nn.GroupNorm) and layer.num_groups == 4


@pytest.mark.parametrize("positional_embedding", ["grid", None])
@pytest.mark.parametrize("domain_padding", [None, 0.1, [0.1, 0.2]])
def test_fno_embedding_and_padding(positional_embedding, domain_padding, cuda_device):
    """test_fno.py:215-251."""
    model = na.FNO(in_channels=3, out_channels=1, n_modes=(5, 5), hidden_channels=9, n_layers=2,
                   positional_embedding=positional_embedding, domain_padding=domain_padding,
                   projection_channel_ratio=2, lifting_channel_ratio=2).to(cuda_device)
    assert list(model(torch.randn(3, 3, 12, 12).to(cuda_device)).shape) == [3, 1, 12, 12]


@pytest.mark.parametrize("channel_mlp_dropout", [0.0, 0.1, 0.5])
@pytest.mark.parametrize("channel_mlp_expansion", [0.25, 0.5, 1.0])
@pytest.mark.parametrize("non_linearity", [F.gelu, F.relu, F.tanh])
def test_fno_channel_mlp_params(channel_mlp_dropout, channel_mlp_expansion, non_linearity, cuda_device):
    """test_fno.py:254-286."""
    model = na.FNO(in_channels=3, out_channels=1, n_modes=(5, 5), hidden_channels=9, n_layers=2,
                   channel_mlp_dropout=channel_mlp_dropout,
                   channel_mlp_expansion=channel_mlp_expansion,
                   non_linearity=non_linearity).to(cuda_device)
    assert list(model(torch.randn(3, 3, 12, 12).to(cuda_device)).shape) == [3, 1, 12, 12]
