"""GPU parity: the HIP path (through the module API and the C ABI) against
the oracle on the same seeded inputs and weights.

Tolerance (fp32 path): max |y - ref| / max |ref| <= 1e-4, ref in float64.
"""
import glob
import os

import numpy as np
import pytest
import torch

import neuraloperator_amd as na
from neuraloperator_amd import _native as nat
from neuraloperator_amd import functional as Fh
from oracle import spectral_ref as R
from neuraloperator_amd.synthetic import gaussian_random_field

pytestmark = pytest.mark.gpu

TOL = 1e-4
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def rel_err(y, ref):
    y = y.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return ((y - ref).abs().max() / ref.abs().max()).item()


def _case_id(p):
    return os.path.basename(p)[:-4]


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "*.npz"))), ids=_case_id)
def test_golden_fixtures(path, cuda_device):
    d = np.load(path)
    x = torch.from_numpy(d["x"])
    w = torch.from_numpy(d["w"])
    nm = d["n_modes"].tolist()
    mx_stored = d["max_n_modes"].tolist()
    sizes = list(x.shape[2:])
    outs = d["out_sizes"].tolist()
    norm = str(d["norm"])
    Ci, Co = w.shape[0], w.shape[1]
    print(f"golden {_case_id(path)} x{tuple(x.shape)} modes={nm} out={outs} norm={norm}", flush=True)
    conv = na.SpectralConv(Ci, Co, nm, fft_norm=norm)
    # max_n_modes as stored: rebuild the weight container at that window
    conv.max_n_modes = mx_stored
    conv.weight = na.FactorizedTensor.new((Ci, Co, *mx_stored), factorization="Dense")
    with torch.no_grad():
        conv.weight.tensor.copy_(w)
        conv.bias.copy_(torch.from_numpy(d["bias"]))
    conv = conv.to(cuda_device)
    xg = x.to(cuda_device)
    with torch.no_grad():
        if "skip_w" in d:
            ws = torch.from_numpy(d["skip_w"]).to(cuda_device)
            y = conv._forward_hip(xg, None, nat.SKIP_LINEAR, ws, nat.ACT_GELU)
        else:
            y = conv(xg, output_shape=tuple(outs) if outs != sizes else None)
    torch.cuda.synchronize()
    err = rel_err(y, torch.from_numpy(d["expected"]))
    assert err <= TOL, err


FUSED_CASES = [
    # B, Ci, Co, H, W, n_modes (constructor)
    (2, 32, 32, 64, 128, (16, 16)),
    (2, 64, 64, 128, 128, (32, 32)),
    (1, 64, 64, 256, 256, (64, 64)),
    (1, 64, 64, 256, 256, (32, 32)),
    (2, 32, 64, 256, 128, (33, 30)),
    (1, 64, 32, 128, 256, (20, 64)),
    (1, 32, 32, 64, 128, (64, 128)),    # every row and the Nyquist column kept
    (1, 64, 64, 128, 128, (48, 60)),    # 128-wide rows in pairs, 8 bins per lane
    (1, 64, 64, 64, 128, (32, 126)),    # ... with the widest window that path takes
    (1, 64, 128, 64, 128, (16, 16)),    # ... with 8 waves per workgroup
]


def _dense_conv(Ci, Co, nm, device, seed=0):
    torch.manual_seed(seed)
    conv = na.SpectralConv(Ci, Co, nm).to(device)
    return conv


@pytest.mark.parametrize("B,Ci,Co,H,W,nm", FUSED_CASES)
@pytest.mark.parametrize("skip", ["linear", "soft-gating", "identity", "none"])
def test_fused_block_matches_oracle(B, Ci, Co, H, W, nm, skip, cuda_device):
    if skip in ("soft-gating", "identity") and Ci != Co:
        pytest.skip("gating/identity skips need Ci == Co")
    print(f"fused B{B} Ci{Ci} Co{Co} {H}x{W} modes={nm} skip={skip}", flush=True)
    conv = _dense_conv(Ci, Co, nm, cuda_device)
    kept, sl = conv.window([H, W])
    g = torch.Generator().manual_seed(1)
    x = torch.randn(B, Ci, H, W, generator=g)
    kind = {"linear": nat.SKIP_LINEAR, "soft-gating": nat.SKIP_SOFT_GATING,
            "identity": nat.SKIP_IDENTITY, "none": nat.SKIP_NONE}[skip]
    ws = None
    if skip == "linear":
        ws = torch.randn(Co, Ci, generator=g) / Ci ** 0.5
    elif skip == "soft-gating":
        ws = torch.rand(Co, generator=g) + 0.5
    assert Fh.spectral_block_is_fused(B, Ci, Co, [H, W], kept, kind)
    with torch.no_grad():
        y = conv._forward_hip(x.to(cuda_device), None, kind,
                              None if ws is None else ws.to(cuda_device), nat.ACT_GELU)
    torch.cuda.synchronize()
    w = conv.weight.to_tensor().detach().cpu().to(torch.complex128)
    ref = R.spectral_conv_forward(x.double(), w, conv.bias.detach().cpu().double(), conv.n_modes,
                                  conv.max_n_modes)
    if skip == "linear":
        ref = ref + R.linear_skip(x.double(), ws.double())
    elif skip == "soft-gating":
        ref = ref + ws.double().view(1, -1, 1, 1) * x.double()
    elif skip == "identity":
        ref = ref + x.double()
    ref = R.gelu(ref)
    err = rel_err(y, ref)
    assert err <= TOL, err


def test_headline_block_per_sample_slice(cuda_device):
    """Two samples of the 256^2 headline block (C=64, n_modes (64,64), GRF
    input, N(0,1/4096) complex weights, N(0,1/64) skip, bias 0) against the
    float64 oracle."""
    print("headline slice B2 C64 256x256 modes 64x64", flush=True)
    B, C, H, W = 2, 64, 256, 256
    x = gaussian_random_field((B, C, H, W), seed=11)
    g = torch.Generator().manual_seed(12)
    w = torch.complex(torch.randn(C, C, 64, 33, generator=g), torch.randn(C, C, 64, 33, generator=g)) / 64
    ws = torch.randn(C, C, generator=g) / 8
    bias = torch.zeros(C)
    with torch.no_grad():
        y = Fh.spectral_block(x.to(cuda_device), w.to(cuda_device), bias.to(cuda_device), [64, 33],
                              nat.SKIP_LINEAR, ws.to(cuda_device), nat.ACT_GELU)
    torch.cuda.synchronize()
    ref = R.spectral_conv_forward(x.double(), w.to(torch.complex128), bias.double().view(-1, 1, 1),
                                  [64, 33], [64, 33])
    ref = R.gelu(ref + R.linear_skip(x.double(), ws.double()))
    err = rel_err(y, ref)
    print(f"headline slice max rel err {err:.3e}", flush=True)
    assert err <= TOL, err


def test_headline_full_batch_properties(cuda_device):
    """The headline block at its full size (B32 C64 256^2, n_modes (64,64),
    fused path) through properties that do not need the oracle at that size:
    every sample equals the same block run on that sample alone (batch
    indexing to the end of the buffers), the spectral part is linear, and the
    last sample matches the float64 oracle."""
    print("headline full batch B32 C64 256x256 modes 64x64", flush=True)
    B, C, H, W = 32, 64, 256, 256
    assert Fh.spectral_block_is_fused(B, C, C, [H, W], [64, 33], nat.SKIP_LINEAR)
    g = torch.Generator().manual_seed(21)
    w = (torch.complex(torch.randn(C, C, 64, 33, generator=g),
                       torch.randn(C, C, 64, 33, generator=g)) / 64).to(cuda_device)
    ws = (torch.randn(C, C, generator=g) / 8).to(cuda_device)
    bias = (torch.randn(C, generator=g) / 8).to(cuda_device)
    x = gaussian_random_field((B, C, H, W), seed=22, device=cuda_device)
    with torch.no_grad():
        y = Fh.spectral_block(x, w, bias, [64, 33], nat.SKIP_LINEAR, ws, nat.ACT_GELU)
        for b in (0, 17, B - 1):
            yb = Fh.spectral_block(x[b:b + 1].contiguous(), w, bias, [64, 33], nat.SKIP_LINEAR, ws,
                                   nat.ACT_GELU)
            assert (yb[0] - y[b]).abs().max().item() <= 1e-6 * y[b].abs().max().item(), b
        # linearity of the spectral part: no skip, no bias, no activation
        x2 = gaussian_random_field((B, C, H, W), seed=23, device=cuda_device)
        f = lambda t: Fh.spectral_block(t, w, None, [64, 33], nat.SKIP_NONE, None, nat.ACT_NONE)
        lhs = f(x + 2.0 * x2)
        rhs = f(x) + 2.0 * f(x2)
        # the row products split each operand into two bf16 terms, which
        # rounds each call separately (~1e-5 of the result): linear to the
        # parity bar, not bit for bit
        assert rel_err(lhs, rhs) <= TOL
        del x2, lhs, rhs
    torch.cuda.synchronize()
    xl = x[B - 1:].double().cpu()
    ref = R.spectral_conv_forward(xl, w.cpu().to(torch.complex128), bias.cpu().double().view(-1, 1, 1),
                                  [64, 33], [64, 33])
    ref = R.gelu(ref + R.linear_skip(xl, ws.cpu().double()))
    assert rel_err(y[B - 1:], ref) <= TOL


@pytest.mark.parametrize("dim,sizes,nm", [
    (1, (1024,), (30,)),
    (1, (37,), (12,)),
    (2, (12, 12), (6, 8)),
    (2, (9, 10), (4, 5)),
    (3, (16, 16, 16), (8, 8, 8)),
    (3, (8, 9, 10), (4, 4, 4)),
    # last axis through the line-FFT kernels (64 / 128 / 256 points)
    (1, (64,), (10,)),
    (1, (256,), (256,)),                # every bin, Nyquist included
    (2, (12, 128), (6, 40)),
    (2, (9, 256), (4, 20)),
    (3, (8, 16, 64), (4, 8, 18)),
    # non-last axes through the tiled line-FFT kernels
    (2, (64, 20), (31, 7)),             # odd window, inner run shorter than a tile
    (2, (128, 64), (64, 20)),
    (2, (256, 16), (256, 5)),           # every bin of the middle axis
    (3, (64, 128, 12), (16, 32, 5)),
])
@pytest.mark.parametrize("norm", ["forward", "backward", "ortho"])
def test_generic_spectral_conv(dim, sizes, nm, norm, cuda_device):
    print(f"generic dim{dim} {sizes} {nm} {norm}", flush=True)
    torch.manual_seed(3)
    conv = na.SpectralConv(3, 4, nm, fft_norm=norm).to(cuda_device)
    x = torch.randn(2, 3, *sizes)
    with torch.no_grad():
        y = conv(x.to(cuda_device))
    ref = R.spectral_conv_forward(x.double(), conv.weight.to_tensor().detach().cpu().to(torch.complex128),
                                  conv.bias.detach().cpu().double(), conv.n_modes, conv.max_n_modes,
                                  fft_norm=norm)
    assert rel_err(y, ref) <= TOL


@pytest.mark.parametrize("scale", [0.5, 2])
@pytest.mark.parametrize("dim", [1, 2, 3])
@pytest.mark.parametrize("size", [8, 9])
def test_resolution_scaling(scale, dim, size, cuda_device):
    """Reference test_spectral_convolution.py:89-116 shapes, plus numbers."""
    torch.manual_seed(4)
    modes = (4, 5, 7)[:dim]
    conv = na.SpectralConv(3, 4, modes, resolution_scaling_factor=scale).to(cuda_device)
    x = torch.randn(2, 3, *([size] * dim))
    with torch.no_grad():
        y = conv(x.to(cuda_device))
    out = [round(size * scale)] * dim
    assert list(y.shape) == [2, 4, *out] and y.dtype == torch.float32
    ref = R.spectral_conv_forward(x.double(), conv.weight.to_tensor().detach().cpu().to(torch.complex128),
                                  conv.bias.detach().cpu().double(), conv.n_modes, conv.max_n_modes,
                                  resolution_scaling_factor=[scale] * dim)
    assert rel_err(y, ref) <= TOL


@pytest.mark.parametrize("enforce", [True, False])
@pytest.mark.parametrize("shape_in,shape_out,nm", [
    ((16, 64), (16, 128), (8, 20)),     # line-FFT inverse onto a longer row
    ((16, 128), (16, 64), (8, 40)),     # ... onto a shorter one (bins past 33 dropped)
    ((7, 256), (7, 256), (4, 130)),     # odd number of rows, Nyquist kept
    ((64, 24), (128, 24), (20, 8)),     # middle axis onto a longer line
    ((128, 24), (64, 24), (40, 8)),     # ... onto a shorter one (bins past 32 dropped)
    ((256, 8), (256, 8), (255, 4)),     # odd window over all 256 bins
])
def test_line_fft_output_shapes(enforce, shape_in, shape_out, nm, cuda_device):
    torch.manual_seed(15)
    conv = na.SpectralConv(3, 5, nm, enforce_hermitian_symmetry=enforce).to(cuda_device)
    x = torch.randn(1, 3, *shape_in)
    with torch.no_grad():
        y = conv(x.to(cuda_device), output_shape=shape_out)
    assert list(y.shape) == [1, 5, *shape_out]
    ref = R.spectral_conv_forward(x.double(), conv.weight.to_tensor().detach().cpu().to(torch.complex128),
                                  conv.bias.detach().cpu().double(), conv.n_modes, conv.max_n_modes,
                                  output_shape=shape_out, enforce_hermitian_symmetry=enforce)
    assert rel_err(y, ref) <= TOL


@pytest.mark.parametrize("enforce", [True, False])
def test_output_shape_with_nyquist(enforce, cuda_device):
    torch.manual_seed(5)
    conv = na.SpectralConv(3, 4, (8, 8), enforce_hermitian_symmetry=enforce).to(cuda_device)
    x = torch.randn(2, 3, 8, 8)
    with torch.no_grad():
        y = conv(x.to(cuda_device), output_shape=(16, 16))
    ref = R.spectral_conv_forward(x.double(), conv.weight.to_tensor().detach().cpu().to(torch.complex128),
                                  conv.bias.detach().cpu().double(), conv.n_modes, conv.max_n_modes,
                                  output_shape=(16, 16), enforce_hermitian_symmetry=enforce)
    assert rel_err(y, ref) <= TOL


def test_incremental_modes_window(cuda_device):
    torch.manual_seed(6)
    conv = na.SpectralConv(3, 3, (10, 8), max_n_modes=(10, 8)).to(cuda_device)
    conv.n_modes = (6, 4)
    x = torch.randn(2, 3, 12, 12)
    with torch.no_grad():
        y = conv(x.to(cuda_device))
    ref = R.spectral_conv_forward(x.double(), conv.weight.to_tensor().detach().cpu().to(torch.complex128),
                                  conv.bias.detach().cpu().double(), conv.n_modes, conv.max_n_modes)
    assert rel_err(y, ref) <= TOL


@pytest.mark.parametrize("factorization", ["Tucker", "CP", "TT"])
@pytest.mark.parametrize("implementation", ["factorized", "reconstructed"])
@pytest.mark.parametrize("dim", [2, 3])
def test_factorized_weights(factorization, implementation, dim, cuda_device):
    torch.manual_seed(7)
    nm = (8, 8, 8)[:dim]
    conv = na.SpectralConv(4, 5, nm, factorization=factorization, rank=0.5,
                           implementation=implementation).to(cuda_device)
    x = torch.randn(2, 4, *([12] * dim))
    with torch.no_grad():
        y = conv(x.to(cuda_device))
    full = conv.weight.to_tensor().detach().cpu().to(torch.complex128)
    ref = R.spectral_conv_forward(x.double(), full, conv.bias.detach().cpu().double(), conv.n_modes,
                                  conv.max_n_modes)
    assert rel_err(y, ref) <= TOL


def test_separable(cuda_device):
    torch.manual_seed(8)
    conv = na.SpectralConv(4, 4, (6, 6), separable=True).to(cuda_device)
    x = torch.randn(2, 4, 10, 12)
    with torch.no_grad():
        y = conv(x.to(cuda_device))
    ref = R.spectral_conv_forward(x.double(), conv.weight.to_tensor().detach().cpu().to(torch.complex128),
                                  conv.bias.detach().cpu().double(), conv.n_modes, conv.max_n_modes,
                                  separable=True)
    assert rel_err(y, ref) <= TOL


def test_tfno3d_tucker_block(cuda_device):
    """3D Tucker-factorized block (reduced C4 shape) through the factors."""
    torch.manual_seed(9)
    B, C = 2, 32
    conv = na.SpectralConv(C, C, (16, 16, 16), factorization="Tucker", rank=0.1,
                           implementation="factorized").to(cuda_device)
    x = gaussian_random_field((B, C, 32, 32, 32), seed=13)
    with torch.no_grad():
        y = conv(x.to(cuda_device))
    core = conv.weight.core.detach().cpu().to(torch.complex128)
    factors = [f.detach().cpu().to(torch.complex128) for f in conv.weight.factors]
    ref = R.spectral_conv_forward(x.double(), {"tucker": (core, factors)},
                                  conv.bias.detach().cpu().double(), conv.n_modes, conv.max_n_modes,
                                  implementation="factorized")
    assert rel_err(y, ref) <= TOL


def _layer_params(blocks, i):
    conv = blocks.convs[i]
    layer = {"conv": dict(weight=conv.weight.to_tensor().detach().cpu().to(torch.complex128),
                          bias=conv.bias.detach().cpu().double(), n_modes=conv.n_modes,
                          max_n_modes=conv.max_n_modes)}
    s = blocks.fno_skips[i]
    layer["fno_skip"] = {"type": "linear", "w": s.conv.weight.detach().cpu().double()[:, :, 0]}
    if blocks.use_channel_mlp:
        m = blocks.channel_mlp[i]
        layer["mlp"] = {"weights": [f.weight.detach().cpu().double() for f in m.fcs],
                        "biases": [f.bias.detach().cpu().double() for f in m.fcs]}
        sk = blocks.channel_mlp_skips[i]
        layer["mlp_skip"] = {"type": "soft-gating", "w": sk.weight.detach().cpu().double()}
    return layer


def _mlp(m):
    return {"weights": [f.weight.detach().cpu().double() for f in m.fcs],
            "biases": [f.bias.detach().cpu().double() for f in m.fcs]}


@pytest.mark.parametrize("hidden,H,W,nm", [(32, 64, 128, (16, 16)), (64, 128, 128, (32, 32))])
def test_fno_forward_matches_oracle(hidden, H, W, nm, cuda_device):
    print(f"fno hidden{hidden} {H}x{W} {nm}", flush=True)
    torch.manual_seed(10)
    model = na.FNO(nm, in_channels=1, out_channels=1, hidden_channels=hidden, n_layers=4).to(cuda_device)
    with torch.no_grad():
        for sk in model.fno_blocks.channel_mlp_skips:
            sk.weight.uniform_(0.5, 1.5)
    x = gaussian_random_field((2, 1, H, W), seed=14)
    with torch.no_grad():
        y = model(x.to(cuda_device))
    params = {"lifting": _mlp(model.lifting), "projection": _mlp(model.projection),
              "layers": [_layer_params(model.fno_blocks, i) for i in range(4)]}
    ref = R.fno_forward(x.double(), params)
    assert rel_err(y, ref) <= TOL


def test_fno_c3_shape_bf16_input(cuda_device):
    """The 4-layer FNO of the bf16 configuration (hidden 64, n_modes (64,64),
    256^2, lifting 3 -> 128 -> 64, channel MLP + soft-gating, projection
    64 -> 128 -> 1) on bf16 inputs, two samples, against the float64 oracle
    on the same bf16-rounded input: within the configuration's 2e-2, and
    within the fp32 bound since every stage computes in fp32."""
    print("fno c3 shape B2 bf16 input", flush=True)
    torch.manual_seed(16)
    model = na.FNO((64, 64), in_channels=1, out_channels=1, hidden_channels=64, n_layers=4).to(cuda_device)
    with torch.no_grad():
        for sk in model.fno_blocks.channel_mlp_skips:
            sk.weight.uniform_(0.5, 1.5)
    x = gaussian_random_field((2, 1, 256, 256), seed=17).to(torch.bfloat16)
    with torch.no_grad():
        y = model(x.to(cuda_device).float())
    params = {"lifting": _mlp(model.lifting), "projection": _mlp(model.projection),
              "layers": [_layer_params(model.fno_blocks, i) for i in range(4)]}
    ref = R.fno_forward(x.double(), params)
    err = rel_err(y, ref)
    assert err <= 2e-2
    assert err <= TOL
    # the configuration as the benchmark runs it: under torch.autocast(bf16)
    # the lifting, channel and projection MLPs take bf16-rounded operands with
    # fp32 accumulation; against the oracle with the same rounding, and
    # against the full-precision oracle at the configuration's 2e-2
    print("fno c3 shape B2 under autocast(bf16)", flush=True)
    assert model._bf16_storage(x.to(cuda_device).float(), [None] * 4) is False  # gradients on
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        xin = model.positional_embedding(x.to(cuda_device).float())
        assert model._bf16_storage(xin, [None] * 4)     # bf16 activation storage
        ybf = model(x.to(cuda_device).float())
    torch.cuda.synchronize()
    assert ybf.dtype == torch.float32
    # against the oracle that rounds the operands the kernels round and stores
    # the activations between layers in bf16, and against the fp32 oracle
    ref_bf = R.fno_forward(x.double(), params, bf16_products=True, bf16_storage=True)
    ref_p = R.fno_forward(x.double(), params, bf16_products=True)
    err_bf = rel_err(ybf, ref_bf)
    print(f"autocast: vs rounded oracle {err_bf:.2e}, vs products-only oracle "
          f"{rel_err(ybf, ref_p):.2e}, vs fp32 oracle {rel_err(ybf, ref):.2e}", flush=True)
    assert err_bf <= 2e-2
    assert rel_err(ybf, ref) <= 2e-2
    # the rounded oracle is the closest: the kernels round what it rounds
    dev_of = lambda r: (ybf.double().cpu() - r).abs().mean()
    assert dev_of(ref_bf) < dev_of(ref_p) and dev_of(ref_bf) < dev_of(ref)


@pytest.mark.parametrize("N,m,Ci,Co,B", [(1024, 16, 3, 20, 2), (512, 7, 5, 4, 5), (256, 1, 1, 8, 1),
                                         (256, 16, 12, 12, 3), (1024, 13, 96, 96, 2)])
@pytest.mark.parametrize("skip", ["identity", "none"])
def test_line_1d_block_channel_counts(N, m, Ci, Co, B, skip, cuda_device):
    """The two-launch 1D line path on channel counts the one-launch kernel
    does not take (Ci not 32 / 64, Co a multiple of 4 but not of 16, batch 1,
    a single bin): the float64 oracle's SpectralConv forward plus skip and
    GELU, and without GELU for the identity skip."""
    if skip == "identity" and Ci != Co:
        pytest.skip("identity skip needs Ci == Co")
    print(f"line 1d N{N} m{m} Ci{Ci} Co{Co} B{B} {skip}", flush=True)
    g = torch.Generator().manual_seed(70 + N + m + Ci)
    x = torch.randn(B, Ci, N, generator=g)
    w = torch.complex(torch.randn(Ci, Co, m, generator=g), torch.randn(Ci, Co, m, generator=g)) / Ci
    bias = torch.randn(Co, generator=g) / 4
    kind = nat.SKIP_IDENTITY if skip == "identity" else nat.SKIP_NONE
    act = nat.ACT_NONE if skip == "identity" else nat.ACT_GELU
    d = lambda t: t.to(cuda_device)
    with torch.no_grad():
        y = Fh.spectral_block(d(x), d(w), d(bias), [m], kind, None, act)
    torch.cuda.synchronize()
    ref = R.spectral_conv_forward(x.double(), w.to(torch.complex128), bias.double().view(-1, 1),
                                  [m], [m])
    if skip == "identity":
        ref = ref + x.double()
    else:
        ref = R.gelu(ref)
    err = rel_err(y, ref)
    assert err <= TOL, err


def test_c0_workload_full_size(cuda_device):
    """The 1D workload at its full size through the call the benchmark times
    (SpectralConv.forward): x[16, 64, 1024] ~ N(0, 1), n_modes 30 -> 16 rfft
    modes, W[64, 64, 16] with re/im ~ N(0, 1/4096), a nonzero bias."""
    print("c0 full size x[16,64,1024] 16 modes", flush=True)
    B, C, N = 16, 64, 1024
    torch.manual_seed(31)
    conv = na.SpectralConv(C, C, (30,)).to(cuda_device)
    g = torch.Generator().manual_seed(32)
    w = torch.complex(torch.randn(C, C, 16, generator=g), torch.randn(C, C, 16, generator=g)) / 64
    bias = torch.randn(C, 1, generator=g) / 8
    with torch.no_grad():
        conv.weight.tensor.copy_(w.to(cuda_device))
        conv.bias.copy_(bias.to(cuda_device))
    x = torch.randn(B, C, N, generator=g)
    with torch.no_grad():
        y = conv(x.to(cuda_device))
    torch.cuda.synchronize()
    assert list(conv.n_modes) == [16]
    ref = R.spectral_conv_forward(x.double(), w.to(torch.complex128), bias.double(), conv.n_modes,
                                  conv.max_n_modes)
    err = rel_err(y, ref)
    assert err <= TOL, err


C4_TUCKER_RANK = (20, 20, 10, 10, 6)


def test_c4_workload_tucker_block(cuda_device):
    """The 3D TFNO block at its workload shape (64^3 grid, 32 channels,
    n_modes (16, 16, 16) -> 16x16x9, Tucker rank 0.1 = the recorded tuple
    (20, 20, 10, 10, 6), factors from the module's init, linear skip + erf
    GELU) through the exact call the benchmark times, on two samples of its
    batch, against the float64 oracle contracting with the factors."""
    print("c4 workload B2 C32 64^3 tucker (20,20,10,10,6) skip+gelu", flush=True)
    torch.manual_seed(34)
    B, C, S = 2, 32, 64
    conv = na.SpectralConv(C, C, (16, 16, 16), factorization="Tucker", rank=0.1,
                           implementation="factorized").to(cuda_device)
    assert tuple(conv.weight.rank) == C4_TUCKER_RANK
    with torch.no_grad():
        conv.bias.normal_(0, 0.1)
    x = gaussian_random_field((B, C, S, S, S), seed=35)
    ws = torch.randn(C, C, generator=torch.Generator().manual_seed(36)) / C ** 0.5
    with torch.no_grad():
        y = conv._forward_hip(x.to(cuda_device), None, nat.SKIP_LINEAR, ws.to(cuda_device),
                              nat.ACT_GELU)
    torch.cuda.synchronize()
    core = conv.weight.core.detach().cpu().to(torch.complex128)
    factors = [f.detach().cpu().to(torch.complex128) for f in conv.weight.factors]
    ref = R.spectral_conv_forward(x.double(), {"tucker": (core, factors)},
                                  conv.bias.detach().cpu().double(), conv.n_modes, conv.max_n_modes,
                                  implementation="factorized")
    ref = R.gelu(ref + R.linear_skip(x.double(), ws.double()))
    err = rel_err(y, ref)
    assert err <= TOL, err


@pytest.mark.parametrize("C", [32, 64])
@pytest.mark.parametrize("H,W", [(32, 128), (48, 128), (48, 256), (512, 256)])
def test_block_heights_outside_inverse_column_kernel(H, W, C, cuda_device):
    """Plane heights without an inverse-column-kernel instance (it has 64,
    128 and 256 rows): 64 output channels stay on the fused path (the row
    epilogue synthesises the columns itself), 32 take the generic
    composition; both match the oracle."""
    print(f"block heights outside the inverse column kernel {H}x{W} C{C}", flush=True)
    B = 2
    conv = _dense_conv(C, C, (16, 16), cuda_device, seed=3)
    kept, _ = conv.window([H, W])
    assert Fh.spectral_block_is_fused(B, C, C, [H, W], kept, nat.SKIP_LINEAR) == (C == 64)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(B, C, H, W, generator=g)
    ws = torch.randn(C, C, generator=g) / C ** 0.5
    with torch.no_grad():
        y = conv._forward_hip(x.to(cuda_device), None, nat.SKIP_LINEAR, ws.to(cuda_device),
                              nat.ACT_GELU)
    torch.cuda.synchronize()
    w = conv.weight.to_tensor().detach().cpu().to(torch.complex128)
    ref = R.spectral_conv_forward(x.double(), w, conv.bias.detach().cpu().double(), conv.n_modes,
                                  conv.max_n_modes)
    ref = R.gelu(ref + R.linear_skip(x.double(), ws.double()))
    assert rel_err(y, ref) <= TOL


@pytest.mark.parametrize("dim,sizes,nm,norm", [
    (2, (16, 20), (8, 10), "forward"),
    (2, (64, 128), (16, 16), "backward"),     # fused forward path
    (2, (12, 9), (6, 5), "ortho"),            # odd last axis (no Nyquist bin)
    (2, (16, 16), (16, 16), "forward"),       # every bin, Nyquist kept
    (1, (64,), (20,), "forward"),
    (3, (8, 12, 16), (4, 6, 8), "backward"),
])
def test_spectral_conv_gradients(dim, sizes, nm, norm, cuda_device):
    """x, weight and bias gradients of SpectralConv against torch autograd
    through the float64 oracle, for a random output cotangent."""
    print(f"grad dim{dim} {sizes} {nm} {norm}", flush=True)
    torch.manual_seed(18)
    Ci, Co, B = 3, 4, 2
    conv = na.SpectralConv(Ci, Co, nm, fft_norm=norm).to(cuda_device)
    with torch.no_grad():
        conv.bias.normal_()
    x = torch.randn(B, Ci, *sizes)
    g = torch.randn(B, Co, *sizes)
    xg = x.to(cuda_device).requires_grad_(True)
    (conv(xg) * g.to(cuda_device)).sum().backward()
    xd = x.double().requires_grad_(True)
    wd = conv.weight.to_tensor().detach().cpu().to(torch.complex128).requires_grad_(True)
    bd = conv.bias.detach().cpu().double().requires_grad_(True)
    yd = R.spectral_conv_forward(xd, wd, bd, conv.n_modes, conv.max_n_modes, fft_norm=norm)
    (yd * g.double()).sum().backward()
    assert rel_err(xg.grad, xd.grad) <= TOL
    assert rel_err(torch.view_as_real(conv.weight.to_tensor().grad), torch.view_as_real(wd.grad)) <= TOL
    assert rel_err(conv.bias.grad, bd.grad) <= TOL


@pytest.mark.parametrize("B,Ci,Co,sizes,nm,norm", [
    (2, 64, 64, (64, 128), (16, 16), "forward"),    # adjoint block: fused 2D path
    (2, 32, 32, (128, 256), (32, 32), "backward"),
    (3, 12, 8, (256,), (12,), "forward"),           # adjoint block: 1D line path (8 -> 12)
    (2, 64, 64, (1024,), (30,), "ortho"),
])
def test_spectral_conv_gradients_fused_adjoint(B, Ci, Co, sizes, nm, norm, cuda_device):
    """On the input grid the x gradient is the spectral block of the output
    cotangent with the transposed conjugate weight and the dual norm
    (the Hermitian weights cancel): shapes whose adjoint block takes the fused
    2D kernels or the 1D line path, against torch autograd through the
    float64 oracle."""
    print(f"fused adjoint grad B{B} {Ci}->{Co} {sizes} {nm} {norm}", flush=True)
    torch.manual_seed(19)
    conv = na.SpectralConv(Ci, Co, nm, fft_norm=norm).to(cuda_device)
    with torch.no_grad():
        conv.bias.normal_()
    x = torch.randn(B, Ci, *sizes)
    g = torch.randn(B, Co, *sizes)
    xg = x.to(cuda_device).requires_grad_(True)
    (conv(xg) * g.to(cuda_device)).sum().backward()
    xd = x.double().requires_grad_(True)
    wd = conv.weight.to_tensor().detach().cpu().to(torch.complex128).requires_grad_(True)
    bd = conv.bias.detach().cpu().double().requires_grad_(True)
    yd = R.spectral_conv_forward(xd, wd, bd, conv.n_modes, conv.max_n_modes, fft_norm=norm)
    (yd * g.double()).sum().backward()
    assert rel_err(xg.grad, xd.grad) <= TOL
    assert rel_err(torch.view_as_real(conv.weight.to_tensor().grad), torch.view_as_real(wd.grad)) <= TOL
    assert rel_err(conv.bias.grad, bd.grad) <= TOL


@pytest.mark.parametrize("sizes,nm,kw", [
    ((32,), (9,), dict(output_shape=(64,))),                 # every bin incl. N//2, upsampled
    ((30,), (8,), dict(resolution_scaling_factor=0.5)),
    ((16, 16), (8, 9), dict(output_shape=(32, 32))),         # zeroed column lands inside
    ((16, 20), (8, 10), dict(resolution_scaling_factor=[2, 1.5])),
    ((12, 9), (6, 5), dict(output_shape=(7, 10))),
    ((16, 16), (8, 8), dict(separable=True)),
    ((16, 16), (8, 9), dict(separable=True, output_shape=(24, 32))),
    ((8, 12, 16), (4, 6, 8), dict(resolution_scaling_factor=2)),
])
@pytest.mark.parametrize("enforce", [True, False])
def test_resized_and_separable_gradients(sizes, nm, kw, enforce, cuda_device):
    """Gradients through output_shape / resolution_scaling_factor and
    separable weights (spectral_convolution.py:49-52, 524-568) against torch
    autograd through the float64 oracle."""
    print(f"grad resized/separable {sizes} {nm} {kw} enforce={enforce}", flush=True)
    torch.manual_seed(21)
    C, B = 3, 2
    out_shape = kw.get("output_shape")
    conv = na.SpectralConv(C, C, nm, enforce_hermitian_symmetry=enforce,
                           **{k: v for k, v in kw.items() if k != "output_shape"}).to(cuda_device)
    with torch.no_grad():
        conv.bias.normal_()
    x = torch.randn(B, C, *sizes)
    xg = x.to(cuda_device).requires_grad_(True)
    y = conv(xg, output_shape=out_shape)
    g = torch.randn(*y.shape)
    (y * g.to(cuda_device)).sum().backward()
    xd = x.double().requires_grad_(True)
    wd = conv.weight.to_tensor().detach().cpu().to(torch.complex128).requires_grad_(True)
    bd = conv.bias.detach().cpu().double().requires_grad_(True)
    rsf = conv.resolution_scaling_factor
    yd = R.spectral_conv_forward(xd, wd, bd, conv.n_modes, conv.max_n_modes,
                                 separable=conv.separable, enforce_hermitian_symmetry=enforce,
                                 output_shape=out_shape, resolution_scaling_factor=rsf)
    assert tuple(yd.shape) == tuple(y.shape)
    (yd * g.double()).sum().backward()
    assert rel_err(xg.grad, xd.grad) <= TOL
    assert rel_err(torch.view_as_real(conv.weight.to_tensor().grad), torch.view_as_real(wd.grad)) <= TOL
    assert rel_err(conv.bias.grad, bd.grad) <= TOL


def test_tucker_spectral_conv_gradients(cuda_device):
    """A Tucker weight gets its gradients through the reconstruction of its
    dense window: compare the reconstructed-weight gradient path against the
    oracle for x and against a dense module carrying the same weight."""
    torch.manual_seed(19)
    conv = na.SpectralConv(4, 4, (8, 8), factorization="Tucker", rank=0.5,
                           implementation="factorized").to(cuda_device)
    x = torch.randn(2, 4, 16, 16)
    g = torch.randn(2, 4, 16, 16)
    xg = x.to(cuda_device).requires_grad_(True)
    (conv(xg) * g.to(cuda_device)).sum().backward()
    for p in conv.weight.parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all()
    xd = x.double().requires_grad_(True)
    wd = conv.weight.to_tensor().detach().cpu().to(torch.complex128)
    yd = R.spectral_conv_forward(xd, wd, conv.bias.detach().cpu().double(), conv.n_modes,
                                 conv.max_n_modes)
    (yd * g.double()).sum().backward()
    assert rel_err(xg.grad, xd.grad) <= TOL


def test_fno_backward_gradients(cuda_device):
    """FNO training step: every parameter gets a gradient (reference
    test_fno.py:73-84), and the lifting, spectral, skip and channel-MLP
    gradients match torch autograd through the float64 oracle."""
    torch.manual_seed(20)
    model = na.FNO((8, 8), in_channels=1, out_channels=1, hidden_channels=8, n_layers=2).to(cuda_device)
    with torch.no_grad():
        for sk in model.fno_blocks.channel_mlp_skips:
            sk.weight.uniform_(0.5, 1.5)
        for conv in model.fno_blocks.convs:
            conv.bias.normal_()
    x = gaussian_random_field((2, 1, 16, 16), seed=21)
    out = model(x.to(cuda_device))
    out.pow(2).sum().backward()
    for name, p in model.named_parameters():
        assert p.grad is not None, name
    blocks = model.fno_blocks
    d = lambda t: t.detach().cpu().double().requires_grad_(True)
    lift = {"weights": [d(f.weight) for f in model.lifting.fcs], "biases": [d(f.bias) for f in model.lifting.fcs]}
    proj = {"weights": [d(f.weight) for f in model.projection.fcs],
            "biases": [d(f.bias) for f in model.projection.fcs]}
    layers = []
    for i in range(2):
        conv = blocks.convs[i]
        layers.append({
            "conv": dict(weight=conv.weight.to_tensor().detach().cpu().to(torch.complex128).requires_grad_(True),
                         bias=d(conv.bias), n_modes=conv.n_modes, max_n_modes=conv.max_n_modes),
            "fno_skip": {"type": "linear", "w": d(blocks.fno_skips[i].conv.weight[:, :, 0])},
            "mlp": {"weights": [d(f.weight) for f in blocks.channel_mlp[i].fcs],
                    "biases": [d(f.bias) for f in blocks.channel_mlp[i].fcs]},
            "mlp_skip": {"type": "soft-gating", "w": d(blocks.channel_mlp_skips[i].weight)}})
    ref = R.fno_forward(x.double(), {"lifting": lift, "projection": proj, "layers": layers})
    ref.pow(2).sum().backward()
    assert rel_err(model.lifting.fcs[0].weight.grad, lift["weights"][0].grad) <= TOL
    assert rel_err(model.projection.fcs[1].weight.grad, proj["weights"][1].grad) <= TOL
    for i in range(2):
        assert rel_err(torch.view_as_real(blocks.convs[i].weight.to_tensor().grad),
                       torch.view_as_real(layers[i]["conv"]["weight"].grad)) <= TOL
        assert rel_err(blocks.convs[i].bias.grad, layers[i]["conv"]["bias"].grad) <= TOL
        assert rel_err(blocks.fno_skips[i].conv.weight.grad[:, :, 0], layers[i]["fno_skip"]["w"].grad) <= TOL
        assert rel_err(blocks.channel_mlp[i].fcs[0].weight.grad, layers[i]["mlp"]["weights"][0].grad) <= TOL
        assert rel_err(blocks.channel_mlp_skips[i].weight.grad, layers[i]["mlp_skip"]["w"].grad) <= TOL


@pytest.mark.parametrize("sizes,nm,out", [
    ((64,), (20,), None),                    # 1D, line FFT
    ((37,), (12,), None),                    # 1D, direct
    ((16, 64), (8, 20), None),
    ((12, 9), (6, 5), None),                 # odd last axis
    ((64, 128), (16, 32), None),             # line FFTs on both axes
    ((8, 12, 16), (4, 6, 8), None),
    ((16, 64), (8, 20), (32, 128)),          # onto a larger grid
    ((16, 64), (8, 20), (8, 32)),            # onto a smaller one
])
@pytest.mark.parametrize("norm", ["forward", "ortho"])
def test_complex_data_spectral_conv(sizes, nm, out, norm, cuda_device):
    """SpectralConv(complex_data=True) on complex fields against the float64
    oracle (fftn / window / ifftn, with the reference's last-axis window)."""
    print(f"complex {sizes} {nm} {out} {norm}", flush=True)
    torch.manual_seed(22)
    conv = na.SpectralConv(3, 4, nm, complex_data=True, fft_norm=norm).to(cuda_device)
    with torch.no_grad():
        conv.bias.normal_()
    x = torch.randn(2, 3, *sizes, dtype=torch.complex64)
    with torch.no_grad():
        y = conv(x.to(cuda_device), output_shape=out)
    assert y.dtype == torch.complex64 and list(y.shape) == [2, 4, *(out or sizes)]
    ref = R.spectral_conv_forward(x.to(torch.complex128),
                                  conv.weight.to_tensor().detach().cpu().to(torch.complex128),
                                  conv.bias.detach().cpu().double(), conv.n_modes, conv.max_n_modes,
                                  fft_norm=norm, complex_data=True, output_shape=out)
    assert rel_err(torch.view_as_real(y), torch.view_as_real(ref)) <= TOL


@pytest.mark.parametrize("sizes,nm", [((64,), (20,)), ((37,), (12,)), ((16, 20), (8, 10)),
                                      ((12, 9), (6, 5)), ((64, 128), (16, 32)), ((8, 12, 16), (4, 6, 8))])
@pytest.mark.parametrize("norm", ["forward", "backward", "ortho"])
def test_complex_spectral_conv_gradients(sizes, nm, norm, cuda_device):
    """x, weight and bias gradients of SpectralConv(complex_data=True) for
    the real loss Re(sum y * g) against torch autograd through the float64
    oracle (fftn / window / ifftn with the reference's last-axis window)."""
    print(f"complex grad {sizes} {nm} {norm}", flush=True)
    torch.manual_seed(19)
    Ci, Co, B = 3, 4, 2
    conv = na.SpectralConv(Ci, Co, nm, complex_data=True, fft_norm=norm).to(cuda_device)
    with torch.no_grad():
        conv.bias.normal_()
    x = torch.randn(B, Ci, *sizes, dtype=torch.complex64)
    g = torch.randn(B, Co, *sizes, dtype=torch.complex64)
    xg = x.to(cuda_device).requires_grad_(True)
    (conv(xg) * g.to(cuda_device)).real.sum().backward()
    xd = x.to(torch.complex128).requires_grad_(True)
    wd = conv.weight.to_tensor().detach().cpu().to(torch.complex128).requires_grad_(True)
    bd = conv.bias.detach().cpu().double().requires_grad_(True)
    yd = R.spectral_conv_forward(xd, wd, bd, conv.n_modes, conv.max_n_modes, fft_norm=norm,
                                 complex_data=True)
    (yd * g.to(torch.complex128)).real.sum().backward()
    assert rel_err(torch.view_as_real(xg.grad), torch.view_as_real(xd.grad)) <= TOL
    assert rel_err(torch.view_as_real(conv.weight.to_tensor().grad), torch.view_as_real(wd.grad)) <= TOL
    assert rel_err(conv.bias.grad, bd.grad) <= TOL


@pytest.mark.parametrize("sizes,nm,kw", [
    ((32,), (12,), dict(output_shape=(64,))),
    ((37,), (12,), dict(resolution_scaling_factor=0.5, separable=True)),
    ((16, 20), (8, 10), dict(output_shape=(32, 15))),
    ((12, 9), (12, 9), dict(resolution_scaling_factor=[2, 3])),     # every mode
    ((16, 16), (8, 8), dict(separable=True)),
    ((8, 12, 16), (4, 6, 8), dict(output_shape=(16, 6, 16), separable=True)),
])
def test_complex_resized_and_separable_gradients(sizes, nm, kw, cuda_device):
    """complex_data=True gradients through output_shape /
    resolution_scaling_factor and separable weights against torch autograd
    through the float64 oracle."""
    print(f"complex grad resized/separable {sizes} {nm} {kw}", flush=True)
    torch.manual_seed(23)
    C, B = 3, 2
    out_shape = kw.get("output_shape")
    conv = na.SpectralConv(C, C, nm, complex_data=True, fft_norm="backward",
                           **{k: v for k, v in kw.items() if k != "output_shape"}).to(cuda_device)
    with torch.no_grad():
        conv.bias.normal_()
    x = torch.randn(B, C, *sizes, dtype=torch.complex64)
    xg = x.to(cuda_device).requires_grad_(True)
    y = conv(xg, output_shape=out_shape)
    g = torch.randn(*y.shape, dtype=torch.complex64)
    (y * g.to(cuda_device)).real.sum().backward()
    xd = x.to(torch.complex128).requires_grad_(True)
    wd = conv.weight.to_tensor().detach().cpu().to(torch.complex128).requires_grad_(True)
    bd = conv.bias.detach().cpu().double().requires_grad_(True)
    yd = R.spectral_conv_forward(xd, wd, bd, conv.n_modes, conv.max_n_modes, fft_norm="backward",
                                 complex_data=True, separable=conv.separable,
                                 output_shape=out_shape,
                                 resolution_scaling_factor=conv.resolution_scaling_factor)
    assert tuple(yd.shape) == tuple(y.shape)
    (yd * g.to(torch.complex128)).real.sum().backward()
    assert rel_err(torch.view_as_real(xg.grad), torch.view_as_real(xd.grad)) <= TOL
    assert rel_err(torch.view_as_real(conv.weight.to_tensor().grad), torch.view_as_real(wd.grad)) <= TOL
    assert rel_err(conv.bias.grad, bd.grad) <= TOL


def test_fno_complex_backward_gradients(cuda_device):
    """Complex-data FNO training step: the input, lifting, spectral and
    channel-MLP gradients against torch autograd through the float64
    oracle, for the loss |sum y| of the reference's test_fno.py:73-78."""
    torch.manual_seed(34)
    model = na.FNO((8, 8), in_channels=2, out_channels=1, hidden_channels=8, n_layers=2,
                   complex_data=True).to(cuda_device)
    with torch.no_grad():
        for sk in model.fno_blocks.channel_mlp_skips:
            sk.fr.weight.uniform_(0.5, 1.5)
            sk.fi.weight.uniform_(-0.5, 0.5)
        for conv in model.fno_blocks.convs:
            conv.bias.normal_()
    x = torch.randn(2, 2, 16, 12, dtype=torch.complex64)
    xg = x.to(cuda_device).requires_grad_(True)
    out = model(xg).sum()
    ((out.real ** 2 + out.imag ** 2) ** 0.5).backward()
    for name, p in model.named_parameters():
        assert p.grad is not None, name
    blocks = model.fno_blocks
    d = lambda t: t.detach().cpu().double().requires_grad_(True)
    real_mlp = lambda m: {"weights": [d(f.weight) for f in m.fcs], "biases": [d(f.bias) for f in m.fcs]}
    layers = []
    for i in range(2):
        conv = blocks.convs[i]
        layers.append({
            "conv": dict(weight=conv.weight.to_tensor().detach().cpu().to(torch.complex128).requires_grad_(True),
                         bias=d(conv.bias), n_modes=conv.n_modes, max_n_modes=conv.max_n_modes,
                         complex_data=True),
            "fno_skip": {"type": "linear", "fr": {"w": d(blocks.fno_skips[i].fr.conv.weight[:, :, 0])},
                         "fi": {"w": d(blocks.fno_skips[i].fi.conv.weight[:, :, 0])}},
            "mlp": {"fr": real_mlp(blocks.channel_mlp[i].fr), "fi": real_mlp(blocks.channel_mlp[i].fi)},
            "mlp_skip": {"type": "soft-gating", "fr": {"w": d(blocks.channel_mlp_skips[i].fr.weight)},
                         "fi": {"w": d(blocks.channel_mlp_skips[i].fi.weight)}}})
    params = {"complex_data": True,
              "lifting": {"fr": real_mlp(model.lifting.fr), "fi": real_mlp(model.lifting.fi)},
              "projection": {"fr": real_mlp(model.projection.fr), "fi": real_mlp(model.projection.fi)},
              "layers": layers}
    xd = x.to(torch.complex128).requires_grad_(True)
    ref = R.fno_forward(xd, params).sum()
    ((ref.real ** 2 + ref.imag ** 2) ** 0.5).backward()
    assert rel_err(torch.view_as_real(xg.grad), torch.view_as_real(xd.grad)) <= TOL
    assert rel_err(model.lifting.fr.fcs[0].weight.grad, params["lifting"]["fr"]["weights"][0].grad) <= TOL
    assert rel_err(model.projection.fi.fcs[1].weight.grad,
                   params["projection"]["fi"]["weights"][1].grad) <= TOL
    for i in range(2):
        assert rel_err(torch.view_as_real(blocks.convs[i].weight.to_tensor().grad),
                       torch.view_as_real(layers[i]["conv"]["weight"].grad)) <= TOL
        assert rel_err(blocks.convs[i].bias.grad, layers[i]["conv"]["bias"].grad) <= TOL
        assert rel_err(blocks.fno_skips[i].fi.conv.weight.grad[:, :, 0],
                       layers[i]["fno_skip"]["fi"]["w"].grad) <= TOL
        assert rel_err(blocks.channel_mlp[i].fr.fcs[0].weight.grad,
                       layers[i]["mlp"]["fr"]["weights"][0].grad) <= TOL


@pytest.mark.parametrize("n_dim", [1, 2, 3, 4])
@pytest.mark.parametrize("stabilizer", [None, "tanh"])
@pytest.mark.parametrize("lifting_channel_ratio", [1, 2])
@pytest.mark.parametrize("preactivation", [False, True])
@pytest.mark.parametrize("complex_data", [True, False])
@pytest.mark.parametrize("enforce_hermitian_symmetry", [True, False])
def test_fno_reference_matrix(n_dim, stabilizer, lifting_channel_ratio, preactivation, complex_data,
                              enforce_hermitian_symmetry, cuda_device):
    """The reference's test_fno matrix (test_fno.py:13-84, its GPU sizes:
    s 12, 8 modes, width 12, batch 4, 4 layers, rank 0.2): output shape, and
    a gradient for every parameter after loss.backward()."""
    s, modes, width, batch, n_layers = 12, 8, 12, 4, 4
    model = na.FNO(in_channels=3, out_channels=1, hidden_channels=width, n_modes=(modes,) * n_dim,
                   rank=0.2, fixed_rank_modes=False, n_layers=n_layers, stabilizer=stabilizer,
                   lifting_channel_ratio=lifting_channel_ratio, preactivation=preactivation,
                   complex_data=complex_data, fno_block_precision="full",
                   enforce_hermitian_symmetry=enforce_hermitian_symmetry).to(cuda_device)
    dtype = torch.cfloat if complex_data else torch.float32
    x = torch.randn(batch, 3, *(s,) * n_dim, dtype=dtype).to(cuda_device)
    out = model(x)
    assert list(out.shape) == [batch, 1, *(s,) * n_dim]
    loss = out.sum()
    if complex_data:
        loss = (loss.real ** 2 + loss.imag ** 2) ** 0.5
    loss.backward()
    unused = [n for n, p in model.named_parameters() if p.grad is None]
    assert not unused, unused


@pytest.mark.parametrize("sizes,nm,out", [((64, 37), (16, 12), None), ((37,), (12,), None),
                                          ((40, 37), (12, 12), (64, 50)), ((9, 10, 37), (6, 6, 8), None)])
def test_complex_data_matrix_core_axes(sizes, nm, out, cuda_device):
    """Complex data with 1024+ columns per axis: the analysis and synthesis
    along every axis the line FFTs do not take run as products on the matrix
    cores, the last axis with the reference's window (frequency j - N/2
    forward, j inverse), against the float64 oracle."""
    print(f"complex mfma axes {sizes} {nm} {out}", flush=True)
    torch.manual_seed(46)
    B = 4096 if len(sizes) == 1 else 16
    conv = na.SpectralConv(8, 8, nm, complex_data=True).to(cuda_device)
    with torch.no_grad():
        conv.bias.normal_()
    x = torch.randn(B, 8, *sizes, dtype=torch.complex64)
    with torch.no_grad():
        y = conv(x.to(cuda_device), output_shape=out)
    ref = R.spectral_conv_forward(x.to(torch.complex128),
                                  conv.weight.to_tensor().detach().cpu().to(torch.complex128),
                                  conv.bias.detach().cpu().double(), conv.n_modes, conv.max_n_modes,
                                  complex_data=True, output_shape=out)
    assert rel_err(torch.view_as_real(y), torch.view_as_real(ref)) <= TOL


def test_complex_data_tucker(cuda_device):
    torch.manual_seed(23)
    conv = na.SpectralConv(4, 4, (8, 8, 8), complex_data=True, factorization="Tucker", rank=0.5,
                           implementation="factorized").to(cuda_device)
    x = torch.randn(2, 4, 16, 16, 16, dtype=torch.complex64)
    with torch.no_grad():
        y = conv(x.to(cuda_device))
    core = conv.weight.core.detach().cpu().to(torch.complex128)
    factors = [f.detach().cpu().to(torch.complex128) for f in conv.weight.factors]
    ref = R.spectral_conv_forward(x.to(torch.complex128), {"tucker": (core, factors)},
                                  conv.bias.detach().cpu().double(), conv.n_modes, conv.max_n_modes,
                                  implementation="factorized", complex_data=True)
    assert rel_err(torch.view_as_real(y), torch.view_as_real(ref)) <= TOL


@pytest.mark.parametrize("precision", ["half", "mixed"])
@pytest.mark.parametrize("bias", [True, False])
@pytest.mark.parametrize("shape,modes,separable", [((2, 3, 12, 12), (6, 6), False),
                                                   ((2, 3, 64), (10,), False),
                                                   ((2, 4, 16, 12), (8, 6), True)])
def test_block_precision_half_arithmetic(precision, bias, shape, modes, separable, cuda_device):
    """fno_block_precision 'half' / 'mixed': output dtype as the reference's
    (float16 from the inverse, float32 once the float32 bias is added) and the
    values of the oracle restating the complex-half arithmetic
    (spectral_convolution.py:436-462, einsum_utils.py:10-34).  Bound: 3e-3 of
    max |y| (a few float16 steps: the kernels round the same intermediates,
    but fp32 and float64 can land on different sides of a float16 rounding
    boundary, and the complex32 intermediate of the split inverse is not
    rounded on the GPU); 1D has no such intermediate: 2e-3.  The half result
    sits closer to the half oracle than to the full-precision one."""
    print(f"half arithmetic {precision} bias={bias} {shape} {modes} sep={separable}", flush=True)
    torch.manual_seed(24)
    C = shape[1]
    conv = na.SpectralConv(C, C if separable else 4, modes, bias=bias, separable=separable,
                           fno_block_precision=precision).to(cuda_device)
    x = torch.randn(*shape)
    with torch.no_grad():
        y = conv(x.to(cuda_device))
    assert y.dtype == (torch.float32 if bias else torch.float16)
    w = conv.weight.to_tensor().detach().cpu().to(torch.complex128)
    b = conv.bias.detach().cpu().double() if bias else None
    kw = dict(separable=separable)
    ref_h = R.spectral_conv_forward(x.double(), w, b, conv.n_modes, conv.max_n_modes,
                                    precision=precision, **kw)
    ref_f = R.spectral_conv_forward(x.double(), w, b, conv.n_modes, conv.max_n_modes, **kw)
    assert rel_err(y, ref_h) <= (2e-3 if len(shape) == 3 else 3e-3)
    dev = lambda r: (y.double().cpu() - r).abs().mean().item()
    assert dev(ref_h) < dev(ref_f)


def test_fno_staged_matches_oracle(cuda_device):
    """FNOStaged with per-layer mode counts against the oracle's FNO forward
    built from each layer's own parameters."""
    torch.manual_seed(27)
    model = na.FNOStaged([(16, 16), (12, 12), (8, 8)], in_channels=1, out_channels=1,
                         hidden_channels=32).to(cuda_device)
    with torch.no_grad():
        for sk in model.channel_mlp_skips:
            sk.weight.uniform_(0.5, 1.5)
    x = gaussian_random_field((2, 1, 64, 64), seed=28)
    with torch.no_grad():
        y = model(x.to(cuda_device))
    params = {"lifting": _mlp(model.lifting), "projection": _mlp(model.projection),
              "layers": [_layer_params(model, i) for i in range(3)]}
    ref = R.fno_forward(x.double(), params)
    assert rel_err(y, ref) <= TOL


def _staged_no_br_reference(model, x, output_shape):
    """no_br=True as the reference runs it (fno_staged.py:478-493,
    butterfly_fft.py:109-122): bit-reversed data through the layers, a
    butterfly layer computing P B P and a fallback layer B on the permuted
    data, then the inverse permutation; B is the natural-order block."""
    P = na.FNOStaged._bitrev_spatial
    r = P(model.lifting(x))
    for i in range(model.n_layers):
        shape = output_shape[i]
        pow2 = all((n & (n - 1)) == 0 for n in r.shape[2:])
        if pow2 and shape is None and not model.complex_data:
            r = P(na.FNOBlocks.forward(model, P(r), i, output_shape=shape))
        else:
            r = na.FNOBlocks.forward(model, r, i, output_shape=shape)
    return model.projection(P(r))


@pytest.mark.parametrize("spatial,n_layers,complex_data,last_shape", [
    ((16, 16), 1, False, None), ((32, 32), 4, False, None),     # test_fno_staged_no_br.py:46-54
    ((12, 12), 2, False, None),                                  # :57-66, bit reversal a no-op
    ((16, 32), 3, True, None),                                   # complex data: every layer falls back
    ((16, 16), 3, False, (16, 16)),                              # output_shape: the last layer falls back
])
def test_fno_staged_no_br(spatial, n_layers, complex_data, last_shape, cuda_device):
    """FNOStaged(no_br=True) against the reference's no_br semantics composed
    from the natural-order blocks, and against no_br=False where the bit
    reversals cancel."""
    print(f"no_br {spatial} {n_layers} {complex_data} {last_shape}", flush=True)
    torch.manual_seed(35)
    kw = dict(in_channels=1, out_channels=1, hidden_channels=8, positional_embedding=None,
              domain_padding=None, fno_skip="linear", use_channel_mlp=False, complex_data=complex_data)
    model = na.FNOStaged([[8, 8]] * n_layers, no_br=True, **kw).to(cuda_device)
    dtype = torch.cfloat if complex_data else torch.float32
    x = torch.randn(2, 1, *spatial, dtype=dtype).to(cuda_device)
    shapes = [None] * (n_layers - 1) + [last_shape]
    with torch.no_grad():
        y = model(x, output_shape=last_shape)
        ref = _staged_no_br_reference(model, x, shapes)
    assert y.shape == x.shape
    assert rel_err(torch.view_as_real(y) if complex_data else y,
                   torch.view_as_real(ref) if complex_data else ref) <= TOL
    natural = na.FNOStaged([[8, 8]] * n_layers, no_br=False, **kw).to(cuda_device)
    natural.load_state_dict(model.state_dict())
    with torch.no_grad():
        yn = natural(x, output_shape=last_shape)
    cancels = not complex_data and last_shape is None
    if cancels:
        assert rel_err(y, yn) <= TOL
    else:   # the permuted layers give another function
        assert rel_err(torch.view_as_real(y) if complex_data else y,
                       torch.view_as_real(yn) if complex_data else yn) > 1e-3


@pytest.mark.parametrize("domain_padding", [0.1, [0.1, 0.2]])
def test_fno_domain_padding(domain_padding, cuda_device):
    """FNO with domain padding (reference test_fno.py:219-253): output size kept,
    values against the oracle (pad after lifting, unpad before projection)."""
    torch.manual_seed(29)
    model = na.FNO((5, 5), in_channels=3, out_channels=1, hidden_channels=9, n_layers=2,
                   domain_padding=domain_padding).to(cuda_device)
    with torch.no_grad():
        for sk in model.fno_blocks.channel_mlp_skips:
            sk.weight.uniform_(0.5, 1.5)
    x = torch.randn(3, 3, 12, 12)
    with torch.no_grad():
        y = model(x.to(cuda_device))
    assert list(y.shape) == [3, 1, 12, 12]
    fr = domain_padding if isinstance(domain_padding, list) else [domain_padding] * 2
    params = {"lifting": _mlp(model.lifting), "projection": _mlp(model.projection),
              "layers": [_layer_params(model.fno_blocks, i) for i in range(2)],
              "domain_padding": fr}
    ref = R.fno_forward(x.double(), params)
    assert rel_err(y, ref) <= TOL


@pytest.mark.parametrize("kind", ["dense", "tucker-factorized", "cp", "separable", "complex"])
def test_spectral_conv_4d(kind, cuda_device):
    """Four spatial axes (reference test_spectral_convolution.py:10, dim 4):
    the window transforms alternate their two stage buffers over four axes."""
    print(f"4d {kind}", flush=True)
    torch.manual_seed(30)
    C, sizes, nm = 3, (6, 8, 5, 8), (4, 4, 4, 4)
    kw = {}
    if kind == "tucker-factorized":
        kw = dict(factorization="Tucker", rank=0.5, implementation="factorized")
    elif kind == "cp":
        kw = dict(factorization="CP", rank=0.5)
    elif kind == "separable":
        kw = dict(separable=True)
    elif kind == "complex":
        kw = dict(complex_data=True)
    conv = na.SpectralConv(C, C, nm, **kw).to(cuda_device)
    with torch.no_grad():
        conv.bias.normal_()
    dtype = torch.complex64 if kind == "complex" else torch.float32
    x = torch.randn(2, C, *sizes, dtype=dtype)
    with torch.no_grad():
        y = conv(x.to(cuda_device))
    if kind == "tucker-factorized":
        w = {"tucker": (conv.weight.core.detach().cpu().to(torch.complex128),
                        [f.detach().cpu().to(torch.complex128) for f in conv.weight.factors])}
        extra = dict(implementation="factorized")
    else:
        w = conv.weight.to_tensor().detach().cpu().to(torch.complex128)
        extra = {}
    ref = R.spectral_conv_forward(x.to(torch.complex128 if kind == "complex" else torch.float64), w,
                                  conv.bias.detach().cpu().double(), conv.n_modes, conv.max_n_modes,
                                  separable=(kind == "separable"), complex_data=(kind == "complex"),
                                  **extra)
    if kind == "complex":
        y, ref = torch.view_as_real(y), torch.view_as_real(ref)
    assert rel_err(y, ref) <= TOL


def _complex_layer_params(blocks, i):
    conv = blocks.convs[i]
    d = lambda t: t.detach().cpu().double()
    real_mlp = lambda m: {"weights": [d(f.weight) for f in m.fcs], "biases": [d(f.bias) for f in m.fcs]}
    return {"conv": dict(weight=conv.weight.to_tensor().detach().cpu().to(torch.complex128),
                         bias=d(conv.bias), n_modes=conv.n_modes, max_n_modes=conv.max_n_modes,
                         complex_data=True),
            "fno_skip": {"type": "linear", "fr": {"w": d(blocks.fno_skips[i].fr.conv.weight)[:, :, 0]},
                         "fi": {"w": d(blocks.fno_skips[i].fi.conv.weight)[:, :, 0]}},
            "mlp": {"fr": real_mlp(blocks.channel_mlp[i].fr), "fi": real_mlp(blocks.channel_mlp[i].fi)},
            "mlp_skip": {"type": "soft-gating", "fr": {"w": d(blocks.channel_mlp_skips[i].fr.weight)},
                         "fi": {"w": d(blocks.channel_mlp_skips[i].fi.weight)}}}


@pytest.mark.parametrize("dim,size,nm", [(1, (64,), (16,)), (2, (16, 24), (8, 8))])
def test_fno_complex_data(dim, size, nm, cuda_device):
    """FNO(complex_data=True) (reference test_fno.py:13-84 with complex data):
    complex spectral layers, ComplexValued skips / MLPs / lifting /
    projection and CGELU, against the oracle restatement."""
    torch.manual_seed(32)
    model = na.FNO(nm, in_channels=2, out_channels=1, hidden_channels=8, n_layers=2,
                   complex_data=True).to(cuda_device)
    with torch.no_grad():
        for sk in model.fno_blocks.channel_mlp_skips:
            sk.fr.weight.uniform_(0.5, 1.5)
            sk.fi.weight.uniform_(-0.5, 0.5)
    x = torch.randn(2, 2, *size, dtype=torch.complex64)
    with torch.no_grad():
        y = model(x.to(cuda_device))
    assert y.dtype == torch.complex64 and list(y.shape) == [2, 1, *size]
    d = lambda t: t.detach().cpu().double()
    real_mlp = lambda m: {"weights": [d(f.weight) for f in m.fcs], "biases": [d(f.bias) for f in m.fcs]}
    params = {"complex_data": True,
              "lifting": {"fr": real_mlp(model.lifting.fr), "fi": real_mlp(model.lifting.fi)},
              "projection": {"fr": real_mlp(model.projection.fr), "fi": real_mlp(model.projection.fi)},
              "layers": [_complex_layer_params(model.fno_blocks, i) for i in range(2)]}
    ref = R.fno_forward(x.to(torch.complex128), params)
    assert rel_err(torch.view_as_real(y), torch.view_as_real(ref)) <= TOL


@pytest.mark.parametrize("shape,modes", [((64, 256, 421), (17,)), ((64, 256, 421), (64,)),
                                         ((64, 256, 421), (9,)), ((4, 32, 128, 421), (16, 17)),
                                         ((2, 64, 130, 250), (20, 33))])
def test_rfft_window_matrix_core_dft(shape, modes, cuda_device):
    """Last-axis pruned DFTs of 16384+ rows of a size the line FFTs do not
    cover run as the DFT product on the matrix cores: the window against
    float64 numpy (rfftn with norm="forward", centred rows)."""
    print(f"rfft window mfma {shape} {modes}", flush=True)
    x = torch.randn(*shape, generator=torch.Generator().manual_seed(44))
    with torch.no_grad():
        y = Fh.rfft_window(x.to(cuda_device), list(modes), "forward")
    spatial = shape[2:]
    X = np.fft.rfftn(x.double().numpy(), axes=tuple(range(2, x.ndim)), norm="forward")
    for d, (n, m) in enumerate(zip(spatial[:-1], modes[:-1])):
        X = np.fft.fftshift(X, axes=2 + d)
        X = np.take(X, range(n // 2 - m // 2, n // 2 - m // 2 + m), axis=2 + d)
    X = X[..., :modes[-1]]
    assert rel_err(torch.view_as_real(y), torch.view_as_real(torch.from_numpy(X))) <= TOL


@pytest.mark.parametrize("shape,modes", [((2, 3, 64, 64), (16, 9)), ((2, 3, 64, 64), (5, 16)),
                                         ((1, 4, 8, 64, 64), (4, 16, 16)),
                                         ((2, 2, 64, 64, 64), (16, 16, 9)),
                                         ((3, 2, 64, 64), (1, 1)), ((2, 5, 64, 64), (16, 15))])
@pytest.mark.parametrize("norm", ["forward", "backward", "ortho"])
def test_rfft_window_slabs(shape, modes, norm, cuda_device):
    """Trailing 64 x 64 slabs with at most 16 kept rows and bins take both
    axes in one pass (the slab kernel): the window against float64 numpy
    (rfftn, centred rows of every non-last axis)."""
    print(f"rfft window slabs {shape} {modes} {norm}", flush=True)
    x = torch.randn(*shape, generator=torch.Generator().manual_seed(45))
    with torch.no_grad():
        y = Fh.rfft_window(x.to(cuda_device), list(modes), norm)
    spatial = shape[2:]
    X = np.fft.rfftn(x.double().numpy(), axes=tuple(range(2, x.ndim)), norm=norm)
    for d, (n, m) in enumerate(zip(spatial[:-1], modes[:-1])):
        X = np.fft.fftshift(X, axes=2 + d)
        X = np.take(X, range(n // 2 - m // 2, n // 2 - m // 2 + m), axis=2 + d)
    X = X[..., :modes[-1]]
    assert rel_err(torch.view_as_real(y), torch.view_as_real(torch.from_numpy(X))) <= TOL


@pytest.mark.parametrize("B,sizes,nm,out", [(4, (128, 421), (16, 32), None),
                                            (4, (128, 210), (16, 32), (128, 421)),
                                            (512, (421,), (30,), None),
                                            (4, (128, 250), (16, 40), None)])
def test_spectral_conv_matrix_core_dft(B, sizes, nm, out, cuda_device):
    """SpectralConv on grids the line FFTs do not cover, with 16384+ rows on
    the last axis: forward and inverse last-axis DFTs as products on the
    matrix cores (bias, Hermitian weights, resized output), against the
    float64 oracle."""
    print(f"spectral conv mfma dft B{B} {sizes} {nm} {out}", flush=True)
    torch.manual_seed(45)
    conv = na.SpectralConv(32, 32, nm).to(cuda_device)
    with torch.no_grad():
        conv.bias.normal_()
    x = torch.randn(B, 32, *sizes)
    with torch.no_grad():
        y = conv(x.to(cuda_device), output_shape=out)
    ref = R.spectral_conv_forward(x.double(), conv.weight.to_tensor().detach().cpu().to(torch.complex128),
                                  conv.bias.detach().cpu().double(), conv.n_modes, conv.max_n_modes,
                                  output_shape=out)
    assert list(y.shape) == list(ref.shape)
    assert rel_err(y, ref) <= TOL


def test_deterministic(cuda_device):
    torch.manual_seed(11)
    conv = na.SpectralConv(64, 64, (64, 64)).to(cuda_device)
    x = torch.randn(2, 64, 256, 256, device=cuda_device)
    ws = torch.randn(64, 64, device=cuda_device) / 8
    with torch.no_grad():
        a = conv._forward_hip(x, None, nat.SKIP_LINEAR, ws, nat.ACT_GELU)
        b = conv._forward_hip(x, None, nat.SKIP_LINEAR, ws, nat.ACT_GELU)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_errors_raise(cuda_device):
    conv = na.SpectralConv(3, 4, (4, 4)).to(cuda_device)
    with pytest.raises(RuntimeError):
        conv(torch.randn(1, 3, 8, 8))            # CPU input
    with pytest.raises(RuntimeError, match="4096"):
        conv(torch.randn(1, 3, 8, 8200, device=cuda_device))
    # the fused forward-only kernels (block with skip / activation) have no
    # backward: the modules take them only without gradients, and a direct
    # call on a tensor that needs one raises when the backward reaches it
    x = torch.randn(1, 3, 8, 8, device=cuda_device, requires_grad=True)
    sq = na.SpectralConv(3, 3, (4, 4)).to(cuda_device)
    y = sq._forward_hip(x, None, nat.SKIP_IDENTITY, None, nat.ACT_GELU)
    with pytest.raises(NotImplementedError, match="no backward"):
        y.sum().backward()


@pytest.mark.parametrize("Ci,Co,S", [(3, 4, (8, 9)), (32, 32, (16, 16, 16)), (20, 24, (37,)),
                                      (64, 48, (10, 12)), (64, 64, (33, 7)), (32, 96, (64,)),
                                      (300, 40, (16,)), (64, 64, (12, 12)), (128, 128, (10, 10)),
                                      (32, 32, (6, 10))])
@pytest.mark.parametrize("skip", ["linear", "soft-gating", "identity", "none"])
def test_block_epilogue(Ci, Co, S, skip, cuda_device):
    """Generic epilogue act(spec + skip(x)) against float64 torch: channel
    counts on and off the 16/32/64 output blocks, point counts with and without
    4- and 2-point vectors, more input channels than the wide blocks stage;
    square 32/64/128-channel linear skips over P % 4 == 0 points take the MFMA
    skip GEMM (P = 144, 100 and 60 end in a partial tile)."""
    if skip in ("soft-gating", "identity") and Ci != Co:
        Ci = Co
    g = torch.Generator().manual_seed(21)
    B = 2
    spec = torch.randn(B, Co, *S, generator=g)
    x = torch.randn(B, Ci, *S, generator=g)
    kind = {"linear": nat.SKIP_LINEAR, "soft-gating": nat.SKIP_SOFT_GATING,
            "identity": nat.SKIP_IDENTITY, "none": nat.SKIP_NONE}[skip]
    ws = {"linear": torch.randn(Co, Ci, generator=g) / Ci ** 0.5,
          "soft-gating": torch.rand(Co, generator=g) + 0.5}.get(skip)
    ref = spec.double()
    if skip == "linear":
        ref = ref + torch.einsum("oi,bi...->bo...", ws.double(), x.double())
    elif skip == "soft-gating":
        ref = ref + ws.double().view(1, -1, *([1] * len(S))) * x.double()
    elif skip == "identity":
        ref = ref + x.double()
    ref = R.gelu(ref)
    with torch.no_grad():
        y = Fh.block_epilogue(spec.to(cuda_device), x.to(cuda_device) if skip != "none" else None, kind,
                              None if ws is None else ws.to(cuda_device), nat.ACT_GELU)
    torch.cuda.synchronize()
    assert rel_err(y, ref) <= TOL


def test_block_epilogue_unaligned_views(cuda_device):
    """Tensors that start one float past a 16-byte boundary take the scalar
    path and still match."""
    g = torch.Generator().manual_seed(22)
    B, C, P = 2, 32, 64
    sbuf = torch.randn(B * C * P + 1, generator=g)
    xbuf = torch.randn(B * C * P + 1, generator=g)
    ws = torch.randn(C, C, generator=g) / C ** 0.5
    spec, x = sbuf[1:].view(B, C, P), xbuf[1:].view(B, C, P)
    ref = R.gelu(spec.double() + torch.einsum("oi,bip->bop", ws.double(), x.double()))
    sd, xd = sbuf.to(cuda_device)[1:].view(B, C, P), xbuf.to(cuda_device)[1:].view(B, C, P)
    with torch.no_grad():
        y = Fh.block_epilogue(sd, xd, nat.SKIP_LINEAR, ws.to(cuda_device), nat.ACT_GELU)
    torch.cuda.synchronize()
    assert rel_err(y, ref) <= TOL


@pytest.mark.parametrize("C,P", [(32, 64), (64, 132), (64, 4096), (128, 260)])
@pytest.mark.parametrize("skip,act", [("soft-gating", "gelu"), ("soft-gating-bias", "none"),
                                      ("identity", "gelu"), ("none", "none")])
def test_channel_mlp(C, P, skip, act, cuda_device):
    """Fused channel MLP (two 1x1 convs, GELU between) + skip + activation
    against the float64 oracle; P = 132 and 260 end in a partial tile."""
    print(f"channel mlp C{C} P{P} {skip} {act}", flush=True)
    g = torch.Generator().manual_seed(23)
    B, Ch = 3, C // 2
    x = torch.randn(B, C, P, generator=g)
    xs = torch.randn(B, C, P, generator=g)
    w1, b1 = torch.randn(Ch, C, 1, generator=g) / C ** 0.5, torch.randn(Ch, generator=g) * 0.1
    w2, b2 = torch.randn(C, Ch, 1, generator=g) / Ch ** 0.5, torch.randn(C, generator=g) * 0.1
    gw, gb = torch.rand(1, C, 1, generator=g) + 0.5, torch.randn(1, C, 1, generator=g) * 0.1
    ref = R.channel_mlp(x.double(), [w1.double(), w2.double()], [b1.double(), b2.double()])
    kind = nat.SKIP_NONE
    if skip.startswith("soft-gating"):
        kind = nat.SKIP_SOFT_GATING
        ref = ref + R.soft_gating(xs.double(), gw.double(), gb.double() if skip.endswith("bias") else None)
    elif skip == "identity":
        kind = nat.SKIP_IDENTITY
        ref = ref + xs.double()
    if act == "gelu":
        ref = R.gelu(ref)
    d = lambda t: t.to(cuda_device)
    with torch.no_grad():
        y = Fh.channel_mlp(d(x), d(w1), d(b1), d(w2), d(b2), kind,
                           d(xs) if kind != nat.SKIP_NONE else None,
                           d(gw) if kind == nat.SKIP_SOFT_GATING else None,
                           d(gb) if skip.endswith("bias") else None,
                           nat.ACT_GELU if act == "gelu" else nat.ACT_NONE)
    torch.cuda.synchronize()
    assert rel_err(y, ref) <= TOL


@pytest.mark.parametrize("Ci,Ch,Co,P", [(3, 128, 64, 512), (3, 64, 32, 132), (4, 128, 64, 64),
                                        (64, 128, 1, 260), (32, 64, 1, 1024), (64, 128, 16, 128)])
def test_channel_mlp_lifting_projection(Ci, Ch, Co, P, cuda_device):
    """The FNO lifting (3 -> 2H -> H) and projection (H -> 2H -> 1) MLPs
    through the kernel's padded input / output widths."""
    print(f"channel mlp {Ci}->{Ch}->{Co} P{P}", flush=True)
    g = torch.Generator().manual_seed(25)
    B = 2
    x = torch.randn(B, Ci, P, generator=g)
    w1, b1 = torch.randn(Ch, Ci, 1, generator=g) / Ci ** 0.5, torch.randn(Ch, generator=g) * 0.1
    w2, b2 = torch.randn(Co, Ch, 1, generator=g) / Ch ** 0.5, torch.randn(Co, generator=g) * 0.1
    ref = R.channel_mlp(x.double(), [w1.double(), w2.double()], [b1.double(), b2.double()])
    d = lambda t: t.to(cuda_device)
    assert Fh.channel_mlp_is_supported(Ci, Ch, Co, P)
    with torch.no_grad():
        y = Fh.channel_mlp(d(x), d(w1), d(b1), d(w2), d(b2))
    torch.cuda.synchronize()
    assert list(y.shape) == [B, Co, P]
    assert rel_err(y, ref) <= TOL


@pytest.mark.parametrize("Ci,Ch,Co,P,skip", [(64, 32, 64, 260, "soft-gating"), (32, 16, 32, 132, "identity"),
                                             (128, 64, 128, 256, "soft-gating"), (3, 128, 64, 512, None),
                                             (3, 64, 32, 132, None), (64, 128, 1, 260, None),
                                             (32, 64, 1, 1024, None)])
def test_channel_mlp_bf16_products(Ci, Ch, Co, P, skip, cuda_device):
    """bf16_products: both layers on bf16-rounded operands with fp32
    accumulation (Conv1d under a bf16 autocast).  Against the oracle with the
    same operand rounding, outputs agree except where a hidden value sits so
    close to a bf16 rounding boundary that the kernel's fp32 GELU and the
    float64 one round it to neighbouring values (max error <= 2e-3); the mean
    error is then < 5% of the mean error against the unrounded oracle (so the
    bf16 operands are the ones the oracle rounds), and the unrounded oracle
    stays within the bf16 configuration's 2e-2."""
    print(f"channel mlp bf16 products {Ci}->{Ch}->{Co} P{P} {skip}", flush=True)
    g = torch.Generator().manual_seed(27)
    B = 3
    x = torch.randn(B, Ci, P, generator=g)
    xs = torch.randn(B, Co, P, generator=g)
    w1, b1 = torch.randn(Ch, Ci, 1, generator=g) / Ci ** 0.5, torch.randn(Ch, generator=g) * 0.1
    w2, b2 = torch.randn(Co, Ch, 1, generator=g) / Ch ** 0.5, torch.randn(Co, generator=g) * 0.1
    gw = torch.rand(1, Co, 1, generator=g) + 0.5
    kind, act = nat.SKIP_NONE, nat.ACT_NONE
    refs = []
    for rounded in (True, False):
        r = R.channel_mlp(x.double(), [w1.double(), w2.double()], [b1.double(), b2.double()],
                          bf16_products=rounded)
        if skip == "soft-gating":
            kind, act = nat.SKIP_SOFT_GATING, nat.ACT_GELU
            r = R.gelu(r + R.soft_gating(xs.double(), gw.double()))
        elif skip == "identity":
            kind, act = nat.SKIP_IDENTITY, nat.ACT_GELU
            r = R.gelu(r + xs.double())
        refs.append(r)
    d = lambda t: t.to(cuda_device)
    with torch.no_grad():
        y = Fh.channel_mlp(d(x), d(w1), d(b1), d(w2), d(b2), kind,
                           d(xs) if kind != nat.SKIP_NONE else None,
                           d(gw) if kind == nat.SKIP_SOFT_GATING else None, None, act,
                           bf16_products=True)
    torch.cuda.synchronize()
    assert y.dtype == torch.float32
    yd = y.double().cpu()
    assert rel_err(y, refs[0]) <= 2e-3
    assert (yd - refs[0]).abs().mean() < 0.05 * (yd - refs[1]).abs().mean()
    assert rel_err(y, refs[1]) <= 2e-2


_LAYER_CASES = [
    # (B, H, W, n_modes, block skip, MLP skip, activation)
    (2, 256, 256, (64, 64), "linear", "soft-gating", True),      # a layer of the bf16 FNO
    (2, 256, 256, (64, 64), "linear", "soft-gating", False),     # its last layer
    (3, 128, 128, (32, 32), "linear", "identity", True),
    (2, 128, 128, (32, 32), "soft-gating", "none", True),
    (3, 64, 128, (16, 16), "identity", "soft-gating", True),
    (2, 64, 128, (16, 16), "linear", "none", False),
    (2, 48, 256, (20, 22), "soft-gating", "identity", True),     # one k-step of row bins
]


@pytest.mark.parametrize("B,H,W,nm,skip,gate,act", _LAYER_CASES)
def test_fused_fno_layer(B, H, W, nm, skip, gate, act, cuda_device):
    """One-pass FNO layer (fno_layer_f32: spectral block + skip + GELU +
    channel MLP 64 -> 32 -> 64 with bf16 products + MLP skip + GELU,
    fno_block.py:331-379) against the composed kernels (the block, then the
    bf16-product channel MLP) and against the bf16-rounding oracle layer."""
    print(f"fno layer B{B} {H}x{W} {nm} skip={skip} gate={gate} act={act}", flush=True)
    C, Ch = 64, 32
    torch.manual_seed(41)
    conv = na.SpectralConv(C, C, nm).to(cuda_device)
    with torch.no_grad():
        conv.bias.normal_(0, 0.1)
    kept, sl = conv.window([H, W])
    wwin = conv.dense_window_weight(sl).detach()
    g = torch.Generator().manual_seed(42)
    kinds = {"linear": nat.SKIP_LINEAR, "soft-gating": nat.SKIP_SOFT_GATING,
             "identity": nat.SKIP_IDENTITY, "none": nat.SKIP_NONE}
    ws = {"linear": torch.randn(C, C, generator=g) / 8, "soft-gating": torch.rand(C, generator=g) + 0.5,
          "identity": None}[skip]
    w1, b1 = torch.randn(Ch, C, generator=g) / 8, torch.randn(Ch, generator=g) / 4
    w2, b2 = torch.randn(C, Ch, generator=g) / 6, torch.randn(C, generator=g) / 4
    gw, gb = torch.rand(C, generator=g) + 0.5, torch.randn(C, generator=g) / 4
    x = gaussian_random_field((B, C, H, W), seed=43)
    dev = lambda t: None if t is None else t.to(cuda_device)
    a = nat.ACT_GELU if act else nat.ACT_NONE
    gkind = kinds[gate]
    gwt, gbt = (gw, gb) if gate == "soft-gating" else (None, None)
    assert Fh.layer_is_fused(B, C, Ch, [H, W], kept, kinds[skip], gkind)
    bias = conv.bias.detach().reshape(-1)
    with torch.no_grad():
        y = Fh.fno_layer(dev(x), wwin, bias, kept, kinds[skip], dev(ws), dev(w1), dev(b1), dev(w2),
                         dev(b2), gkind, dev(gwt), dev(gbt), a)
        y1 = Fh.spectral_block(dev(x), wwin, bias, kept, kinds[skip], dev(ws), a)
        yc = Fh.channel_mlp(y1, dev(w1), dev(b1), dev(w2), dev(b2), gkind,
                            dev(x) if gate != "none" else None, dev(gwt), dev(gbt), a,
                            bf16_products=True)
    torch.cuda.synchronize()
    err_c = rel_err(y, yc)
    if skip == "linear":
        skip_d = {"type": "linear", "w": ws.double()}
    elif skip == "soft-gating":
        skip_d = {"type": "soft-gating", "w": ws.double().view(1, C, 1, 1)}
    else:
        skip_d = {"type": "identity"}
    gate_d = {"soft-gating": {"type": "soft-gating", "w": gw.double().view(1, C, 1, 1),
                              "b": gb.double().view(1, C, 1, 1)},
              "identity": {"type": "identity"}, "none": None}[gate]
    convd = dict(weight=conv.weight.to_tensor().detach().cpu().to(torch.complex128),
                 bias=conv.bias.detach().cpu().double(), n_modes=conv.n_modes,
                 max_n_modes=conv.max_n_modes)
    mlpd = {"weights": [w1.double(), w2.double()], "biases": [b1.double(), b2.double()]}
    ref = R.fno_block_forward(x.double(), 0 if act else 1, 2, convd, skip_d, mlpd, gate_d,
                              bf16_products=True)
    err = rel_err(y, ref)
    print(f"  vs composed {err_c:.2e}, vs rounded oracle {err:.2e}", flush=True)
    assert err_c <= 2e-3
    assert err <= 2e-2
    # bfloat16 storage (fno_layer_bf16): a bf16 x is exact in one bf16 term,
    # so the layer on it is the fp32 layer on the widened x, rounded to bf16
    # (nearest even) at the store -- bit for bit
    xb = dev(x).to(torch.bfloat16)
    if not Fh.layer_is_fused(B, C, Ch, [H, W], kept, kinds[skip], gkind, bf16=True):
        assert H not in (64, 128, 256)    # planes without the streamed forward
        with pytest.raises(RuntimeError, match="no one-pass bfloat16 kernel"):
            Fh.fno_layer(xb, wwin, bias, kept, kinds[skip], dev(ws), dev(w1), dev(b1), dev(w2),
                         dev(b2), gkind, dev(gwt), dev(gbt), a)
        return
    with torch.no_grad():
        yb = Fh.fno_layer(xb, wwin, bias, kept, kinds[skip], dev(ws), dev(w1), dev(b1), dev(w2),
                          dev(b2), gkind, dev(gwt), dev(gbt), a)
        yw = Fh.fno_layer(xb.float(), wwin, bias, kept, kinds[skip], dev(ws), dev(w1), dev(b1),
                          dev(w2), dev(b2), gkind, dev(gwt), dev(gbt), a)
    torch.cuda.synchronize()
    assert yb.dtype == torch.bfloat16
    assert torch.equal(yb, yw.to(torch.bfloat16))


@pytest.mark.parametrize("B,ci,ch,co,P", [(2, 3, 128, 64, 4096), (3, 4, 64, 32, 1024),
                                         (2, 64, 128, 1, 4096), (2, 32, 64, 16, 512)])
def test_channel_mlp_bf16_storage(B, ci, ch, co, P, cuda_device):
    """fno_channel_mlp_io: the lifting with a bfloat16 output and the
    projection with a bfloat16 input are the bf16-product channel MLP on the
    same values, the output rounded to bf16 at the store: bit for bit against
    fno_channel_mlp_f32 (rounded / on the widened input), and within the
    rounding of the output against the oracle."""
    print(f"channel mlp bf16 storage B{B} {ci}->{ch}->{co} P{P}", flush=True)
    g = torch.Generator().manual_seed(61)
    w1, b1 = torch.randn(ch, ci, generator=g) / 2, torch.randn(ch, generator=g) / 4
    w2, b2 = torch.randn(co, ch, generator=g) / 8, torch.randn(co, generator=g) / 4
    x = torch.randn(B, ci, P, generator=g)
    d = lambda t: t.to(cuda_device)
    lifting = ci <= 4
    assert Fh.channel_mlp_io_is_supported(ci, ch, co, P, not lifting, lifting)
    assert not Fh.channel_mlp_io_is_supported(ci, ch, co, P, lifting, not lifting)
    xin = d(x) if lifting else d(x).to(torch.bfloat16)
    with torch.no_grad():
        y = Fh.channel_mlp_io(xin, d(w1), d(b1), d(w2), d(b2), nat.ACT_NONE, y_bf16=lifting)
        yf = Fh.channel_mlp(xin.float(), d(w1), d(b1), d(w2), d(b2), bf16_products=True)
    torch.cuda.synchronize()
    assert y.dtype == (torch.bfloat16 if lifting else torch.float32)
    if lifting:
        assert torch.equal(y, yf.to(torch.bfloat16))
    else:
        assert torch.equal(y, yf)
    ref = R.channel_mlp(xin.float().cpu().double(), [w1.double(), w2.double()],
                        [b1.double(), b2.double()], bf16_products=True)
    # bf16 products: the hidden activation's rounding (fp32 here, float64 in
    # the oracle) can differ by one bf16 step near ties, ~1e-4 of the output
    assert rel_err(y.float(), ref) <= (2.0 ** -8 if lifting else 0) + 1e-3


_EPI_CASES = [
    # (B, Ci, Co, sizes, window, skip, act); lines of 64 with <= 15 bins and
    # 32 / 64 channels take the one-pass line epilogue, the rest the composed path
    (2, 32, 32, (16, 16, 64), (8, 8, 9), "linear", True),
    (2, 64, 32, (32, 64), (16, 15), "linear", True),
    (2, 32, 64, (8, 12, 64), (4, 6, 12), "linear", False),
    (2, 32, 32, (24, 64), (12, 9), "soft-gating", False),
    (3, 64, 64, (64,), (9,), "identity", True),
    (2, 32, 32, (8, 64), (8, 5), "none", True),
    (2, 48, 40, (16, 64), (8, 9), "linear", True),      # 40 channels: composed
    (2, 32, 32, (16, 32), (8, 9), "linear", True),      # 32-point lines: composed
    (2, 32, 32, (16, 64), (8, 20), "linear", True),     # 20 bins: composed
    # trailing 64 x 64 slabs (the next-to-last axis' inverse on 64-point lines)
    (2, 32, 32, (4, 64, 64), (4, 16, 9), "linear", True),
    (2, 64, 32, (64, 64), (16, 9), "linear", True),
    (2, 32, 32, (64, 64), (8, 15), "soft-gating", False),
    (2, 32, 32, (3, 64, 64), (3, 12, 5), "identity", True),
    (2, 32, 32, (64, 64), (16, 9), "none", True),
    (1, 32, 32, (2, 64, 64), (2, 1, 1), "linear", True),
]


@pytest.mark.parametrize("B,Ci,Co,S,m,skip,act", _EPI_CASES)
@pytest.mark.parametrize("norm", ["forward", "ortho"])
def test_irfft_window_epilogue(B, Ci, Co, S, m, skip, act, norm, cuda_device):
    """fno_irfft_window_epilogue_f32 (inverse + bias + skip + activation in
    one call) against the same steps as separate calls: fno_irfft_window_f32
    then fno_block_epilogue_f32."""
    print(f"irfft+epilogue B{B} {Ci}->{Co} {S} {m} {skip} act={act} {norm}", flush=True)
    g = torch.Generator().manual_seed(51)
    yhat = torch.complex(torch.randn(B, Co, *m, generator=g), torch.randn(B, Co, *m, generator=g))
    x = torch.randn(B, Ci, *S, generator=g)
    kind = {"linear": nat.SKIP_LINEAR, "soft-gating": nat.SKIP_SOFT_GATING,
            "identity": nat.SKIP_IDENTITY, "none": nat.SKIP_NONE}[skip]
    ws = {"linear": torch.randn(Co, Ci, generator=g) / Ci ** 0.5,
          "soft-gating": torch.rand(Co, generator=g) + 0.5}.get(skip)
    bias = torch.randn(Co, generator=g)
    a = nat.ACT_GELU if act else nat.ACT_NONE
    dev = lambda t: None if t is None else t.to(cuda_device)
    with torch.no_grad():
        y = Fh.irfft_window_epilogue(dev(yhat), list(S), dev(bias), dev(x), kind, dev(ws), a, norm)
        ref = Fh.irfft_window(dev(yhat), list(S), list(S), dev(bias), norm)
        ref = Fh.block_epilogue(ref, dev(x), kind, dev(ws), a)
    torch.cuda.synchronize()
    assert rel_err(y, ref) <= TOL


@pytest.mark.parametrize("S,nm,skip", [((16, 16, 64), (8, 8, 16), "linear"),
                                       ((32, 64), (16, 16), "soft-gating"),
                                       ((12, 64), (12, 20), "identity")])
def test_block_with_line_epilogue_matches_oracle(S, nm, skip, cuda_device):
    """Spectral blocks whose last axis is a 64-point line (the generic path's
    one-pass line epilogue), dense weight, skip + GELU, against the float64
    oracle."""
    print(f"block with line epilogue {S} {nm} {skip}", flush=True)
    torch.manual_seed(52)
    C, B = 32, 2
    conv = na.SpectralConv(C, C, nm).to(cuda_device)
    with torch.no_grad():
        conv.bias.normal_(0, 0.1)
    g = torch.Generator().manual_seed(53)
    x = torch.randn(B, C, *S, generator=g)
    kind = {"linear": nat.SKIP_LINEAR, "soft-gating": nat.SKIP_SOFT_GATING,
            "identity": nat.SKIP_IDENTITY}[skip]
    ws = {"linear": torch.randn(C, C, generator=g) / C ** 0.5,
          "soft-gating": torch.rand(C, generator=g) + 0.5}.get(skip)
    with torch.no_grad():
        y = conv._forward_hip(x.to(cuda_device), None, kind,
                              None if ws is None else ws.to(cuda_device), nat.ACT_GELU)
    torch.cuda.synchronize()
    w = conv.weight.to_tensor().detach().cpu().to(torch.complex128)
    ref = R.spectral_conv_forward(x.double(), w, conv.bias.detach().cpu().double(), conv.n_modes,
                                  conv.max_n_modes)
    if skip == "linear":
        ref = ref + R.linear_skip(x.double(), ws.double())
    elif skip == "soft-gating":
        ref = ref + R.soft_gating(x.double(), ws.double().view(1, C, *([1] * len(S))))
    else:
        ref = ref + x.double()
    assert rel_err(y, R.gelu(ref)) <= TOL


def test_fno_autocast_bf16(cuda_device):
    """FNO forward under torch.autocast(dtype=bfloat16): lifting, block and
    projection MLPs take the bf16-product kernel, the spectral path stays
    fp32.  Within 2e-2 of the fp32 oracle, and not equal to the fp32 run."""
    torch.manual_seed(33)
    model = na.FNO((16, 16), in_channels=1, out_channels=1, hidden_channels=64, n_layers=2).to(cuda_device)
    with torch.no_grad():
        for sk in model.fno_blocks.channel_mlp_skips:
            sk.weight.uniform_(0.5, 1.5)
    x = gaussian_random_field((2, 1, 64, 128), seed=5)
    with torch.no_grad():
        y32 = model(x.to(cuda_device))
        with torch.autocast("cuda", dtype=torch.bfloat16):
            ybf = model(x.to(cuda_device))
    assert ybf.dtype == torch.float32
    params = {"lifting": _mlp(model.lifting), "projection": _mlp(model.projection),
              "layers": [_layer_params(model.fno_blocks, i) for i in range(2)]}
    ref = R.fno_forward(x.double(), params)
    assert rel_err(y32, ref) <= TOL
    assert 1e-4 < rel_err(ybf, ref) <= 2e-2


def test_channel_mlp_in_place(cuda_device):
    """y written over x (the layout FNOBlocks may use) matches the out-of-place result."""
    g = torch.Generator().manual_seed(24)
    B, C, P = 2, 64, 1024
    x = torch.randn(B, C, P, generator=g).to(cuda_device)
    xs = torch.randn(B, C, P, generator=g).to(cuda_device)
    w1 = (torch.randn(32, C, generator=g) / 8).to(cuda_device)
    w2 = (torch.randn(C, 32, generator=g) / 6).to(cuda_device)
    gw = (torch.rand(C, generator=g) + 0.5).to(cuda_device)
    with torch.no_grad():
        a = Fh.channel_mlp(x, w1, None, w2, None, nat.SKIP_SOFT_GATING, xs, gw, None, nat.ACT_GELU)
        xc = x.clone()
        b = Fh.channel_mlp(xc, w1, None, w2, None, nat.SKIP_SOFT_GATING, xs, gw, None, nat.ACT_GELU,
                           out=xc)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_block_epilogue_unaligned_spec(cuda_device):
    """An aligned x with the spectral term (and output) one float off a
    16-byte boundary: the square linear skip leaves the MFMA GEMM (its staged
    rows are 16-byte accesses) for the scalar path and still matches."""
    g = torch.Generator().manual_seed(26)
    B, C, P = 2, 32, 256
    sbuf = torch.randn(B * C * P + 1, generator=g)
    x = torch.randn(B, C, P, generator=g)
    ws = torch.randn(C, C, generator=g) / C ** 0.5
    spec = sbuf[1:].view(B, C, P)
    ref = R.gelu(spec.double() + torch.einsum("oi,bip->bop", ws.double(), x.double()))
    sd = sbuf.to(cuda_device)[1:].view(B, C, P)
    with torch.no_grad():
        y = Fh.block_epilogue(sd, x.to(cuda_device), nat.SKIP_LINEAR, ws.to(cuda_device), nat.ACT_GELU)
    torch.cuda.synchronize()
    assert rel_err(y, ref) <= TOL


def test_kernel_gelu_matches_exact_erf(cuda_device):
    """The kernels' erf GELU (Abramowitz & Stegun 7.1.28 form) against exact
    erf GELU in float64 over [-12, 12], through the C-ABI epilogue with no
    skip.  The approximation's erf error is <= 3e-7 absolute, so: absolute
    error <= 2e-6 everywhere (a float32 emulation of the formula gives 7e-7)
    and relative <= 1e-5 where |GELU| >= 0.1 (emulation: 3e-6); in the far
    negative tail only the absolute bound is meaningful."""
    v = torch.linspace(-12.0, 12.0, 1 << 20, dtype=torch.float32)
    spec = v.reshape(1, 1, -1).to(cuda_device)
    y = Fh.block_epilogue(spec.clone(), None, nat.SKIP_NONE, None, nat.ACT_GELU)
    torch.cuda.synchronize()
    vd = v.double()
    ref = 0.5 * vd * (1.0 + torch.erf(vd / 2 ** 0.5))
    err = (y.double().cpu().reshape(-1) - ref).abs()
    assert err.max().item() <= 2e-6
    big = ref.abs() >= 0.1
    assert (err[big] / ref.abs()[big]).max().item() <= 1e-5


@pytest.mark.parametrize("N,m,Ci,Co", [(1024, 16, 64, 64), (1024, 1, 32, 16), (512, 9, 64, 128),
                                       (256, 16, 32, 32), (256, 5, 64, 48)])
@pytest.mark.parametrize("skip", ["linear", "soft-gating", "identity", "none"])
@pytest.mark.parametrize("norm", ["forward", "backward", "ortho"])
def test_fused_1d_block(N, m, Ci, Co, skip, norm, cuda_device):
    """The 1D block against the float64 oracle: the SpectralConv forward
    (first m rfft bins) plus the skip and erf GELU.  A linear skip takes the
    one-launch kernel (forward DFT product, contraction and the synthesis
    product with skip, bias and GELU in one kernel), the other skips the
    two-launch line path (one wave's DFT per line, then contraction and
    synthesis per 4 output channels)."""
    if skip in ("soft-gating", "identity") and Ci != Co:
        pytest.skip("gating/identity skips need Ci == Co")
    print(f"fused 1d N{N} m{m} Ci{Ci} Co{Co} {skip} {norm}", flush=True)
    g = torch.Generator().manual_seed(40 + N + m)
    B = 3
    x = torch.randn(B, Ci, N, generator=g)
    w = torch.complex(torch.randn(Ci, Co, m, generator=g), torch.randn(Ci, Co, m, generator=g)) / Ci
    bias = torch.randn(Co, generator=g) / 4
    kind = {"linear": nat.SKIP_LINEAR, "soft-gating": nat.SKIP_SOFT_GATING,
            "identity": nat.SKIP_IDENTITY, "none": nat.SKIP_NONE}[skip]
    ws = None
    if skip == "linear":
        ws = torch.randn(Co, Ci, generator=g) / Ci ** 0.5
    elif skip == "soft-gating":
        ws = torch.rand(Co, generator=g) + 0.5
    d = lambda t: None if t is None else t.to(cuda_device)
    with torch.no_grad():
        y = Fh.spectral_block(d(x), d(w), d(bias), [m], kind, d(ws), nat.ACT_GELU, fft_norm=norm)
    torch.cuda.synchronize()
    ref = R.spectral_conv_forward(x.double(), w.to(torch.complex128), bias.double().view(-1, 1),
                                  [m], [m], fft_norm=norm)
    if skip == "linear":
        ref = ref + R.linear_skip(x.double(), ws.double())
    elif skip == "soft-gating":
        ref = ref + ws.double().view(1, -1, 1) * x.double()
    elif skip == "identity":
        ref = ref + x.double()
    ref = R.gelu(ref)
    err = rel_err(y, ref)
    assert err <= TOL, err


@pytest.mark.parametrize("B,C,S,nm", [(1, 3, (64, 64, 8), (7, 16, 4)),
                                      (2, 5, (64, 64, 64), (16, 11, 16)),
                                      (1, 8, (64, 64, 12), (1, 1, 2))])
def test_3d_leading_64x64_inverse_matches_oracle(B, C, S, nm, cuda_device):
    """3D blocks whose first two axes are 64 points: their inverse runs as one
    pass per plane (both axes expanded in LDS).  Plane counts that are not a
    multiple of 8 leave some workgroups of the XCD-grouped grid idle; odd and
    single-row windows.  Against the float64 oracle."""
    print(f"3d leading 64x64 inverse B{B} C{C} {S} {nm}", flush=True)
    torch.manual_seed(54)
    conv = na.SpectralConv(C, C, nm).to(cuda_device)
    with torch.no_grad():
        conv.bias.normal_(0, 0.1)
    g = torch.Generator().manual_seed(55)
    x = torch.randn(B, C, *S, generator=g)
    with torch.no_grad():
        y = conv(x.to(cuda_device))
    torch.cuda.synchronize()
    w = conv.weight.to_tensor().detach().cpu().to(torch.complex128)
    ref = R.spectral_conv_forward(x.double(), w, conv.bias.detach().cpu().double(), conv.n_modes,
                                  conv.max_n_modes)
    assert rel_err(y, ref) <= TOL
