"""Pins the oracle (oracle/spectral_ref.py) before the parity tests compare against it.

Each check is chosen so that a plausible mistake fails it:
  * closed-form float64 DFT (oracle/dft64.py)  -> sign, index, shift, window,
    scaling, Hermitian and output-size bookkeeping
  * plane-wave known answers                   -> amplitude / phase / row order
  * circular-shift equivariance, linearity     -> transposed operands, dropped terms
  * factorized == dense on the reconstructed weight (reference invariant,
    neuralop/layers/tests/test_spectral_convolution.py:53-65)
  * committed golden fixtures
"""
import glob
import math
import os

import numpy as np
import pytest
import torch

from oracle import dft64, spectral_ref as R

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")

CASES = [
    ((12,), (10,), None, None, "forward"),
    ((16,), (8,), (12,), None, "forward"),
    ((9, 10), (4, 5), None, None, "forward"),
    ((8, 8), (4, 4), (8, 8), None, "backward"),
    ((12, 12), (4, 6), None, (24, 24), "forward"),
    ((9, 9), (4, 7), None, (4, 4), "ortho"),
    ((8, 9, 10), (4, 4, 4), None, None, "forward"),
    ((9, 8), (4, 4), None, (18, 16), "forward"),
    ((8, 8), (8, 8), None, (16, 16), "forward"),
    ((6, 10), (6, 10), None, (12, 10), "forward"),
]


@pytest.mark.parametrize("sizes,nm,mx,outs,norm", CASES)
@pytest.mark.parametrize("enforce", [True, False])
def test_restatement_matches_closed_form(sizes, nm, mx, outs, norm, enforce):
    torch.manual_seed(0)
    nms = R.stored_n_modes(nm)
    mxs = R.stored_n_modes(mx) if mx else nms
    x = torch.randn(2, 3, *sizes, dtype=torch.float64)
    w = torch.randn(3, 4, *mxs, dtype=torch.complex128)
    b = torch.randn(4, *([1] * len(sizes)), dtype=torch.float64)
    y = R.spectral_conv_forward(x, w, b, nms, mxs, fft_norm=norm, output_shape=outs,
                                enforce_hermitian_symmetry=enforce)
    yd = dft64.spectral_conv(x.numpy(), w.numpy(), b.numpy(), nms, mxs, norm=norm, out_sizes=outs,
                             enforce_hermitian_symmetry=enforce)
    assert y.shape == yd.shape
    assert np.abs(y.numpy() - yd).max() <= 1e-12 * np.abs(yd).max()


def test_hermitian_flag_matters_only_for_kept_nyquist_with_resize():
    torch.manual_seed(1)
    nms = R.stored_n_modes((8, 8))
    x = torch.randn(1, 2, 8, 8, dtype=torch.float64)
    w = torch.randn(2, 2, *nms, dtype=torch.complex128)
    a = R.spectral_conv_forward(x, w, None, nms, nms, output_shape=(16, 16), enforce_hermitian_symmetry=True)
    b = R.spectral_conv_forward(x, w, None, nms, nms, output_shape=(16, 16), enforce_hermitian_symmetry=False)
    assert (a - b).abs().max() > 1e-3
    a = R.spectral_conv_forward(x, w, None, nms, nms, enforce_hermitian_symmetry=True)
    b = R.spectral_conv_forward(x, w, None, nms, nms, enforce_hermitian_symmetry=False)
    assert (a - b).abs().max() == 0


@pytest.mark.parametrize("kh,kw", [(0, 0), (3, 2), (-4, 5), (-2, 0), (5, 0)])
def test_plane_wave_known_answer(kh, kw):
    """x = cos(2 pi (kh h/H + kw w/W)); weight nonzero (= c) only at window
    index of (kh, kw) -> y = |c| cos(theta + arg c) for kw > 0, and half that
    amplitude per conjugate partner when kw == 0."""
    H, W, m1, m2 = 16, 16, 12, 8
    nms = R.stored_n_modes((m1, 2 * (m2 - 1)))
    assert nms == [m1, m2]
    h = torch.arange(H, dtype=torch.float64)[:, None]
    ww = torch.arange(W, dtype=torch.float64)[None, :]
    theta = 2 * math.pi * (kh * h / H + kw * ww / W)
    x = torch.cos(theta)[None, None]
    c = complex(0.7, -0.4)
    wt = torch.zeros(1, 1, m1, m2, dtype=torch.complex128)
    wt[0, 0, kh + m1 // 2, kw] = c
    y = R.spectral_conv_forward(x, wt, None, nms, nms)[0, 0]
    amp, ph = abs(c), math.atan2(c.imag, c.real)
    if kw > 0:
        expected = amp * torch.cos(theta + ph)
    else:
        # X[kh,0] = X[-kh,0] = 1/2; only the (kh,0) weight is nonzero: the
        # output is Re(c/2 e^{i theta}) from the DC column (c_0 = 1)
        expected = 0.5 * amp * torch.cos(theta + ph) if kh != 0 else amp * math.cos(ph) * torch.ones_like(theta)
    assert torch.allclose(y, expected, atol=1e-12)


@pytest.mark.parametrize("sizes,nm,f_in,j,f_out", [
    # 2D: axis 0 keeps the centred window (j = f + m/2); the last axis keeps
    # the first m entries of its fftshift-ed order (frequency j - N/2) and
    # the inverse puts entry j at frequency j (no ifftshift on the last axis,
    # spectral_convolution.py:448-449, :510-517, :531-538)
    ((8, 8), (4, 4), (1, -3), (3, 1), (1, 1)),
    ((8, 9), (4, 5), (-2, -4), (0, 0), (-2, 0)),
    # 1D: no shift at all, the first m frequencies
    ((10,), (4,), (3,), (3,), (3,)),
])
def test_complex_data_plane_wave(sizes, nm, f_in, j, f_out):
    """complex_data=True: a plane wave through a weight that is non-zero at
    one window entry comes out as the plane wave of the frequency the
    reference's shifts and slices map that entry to."""
    grids = torch.meshgrid(*[torch.arange(n, dtype=torch.float64) for n in sizes], indexing="ij")
    phase = sum(f * g / n for f, g, n in zip(f_in, grids, sizes))
    x = torch.exp(2j * math.pi * phase).reshape(1, 1, *sizes)
    w = torch.zeros(1, 1, *nm, dtype=torch.complex128)
    a = 0.7 - 0.4j
    w[(0, 0, *j)] = a
    y = R.spectral_conv_forward(x, w, None, list(nm), list(nm), complex_data=True)
    out_phase = sum(f * g / n for f, g, n in zip(f_out, grids, sizes))
    expect = a * torch.exp(2j * math.pi * out_phase).reshape(1, 1, *sizes)
    assert torch.allclose(y, expect, atol=1e-12)


def test_domain_padding_restatement():
    """Padding puts round(p * n) zeros on both sides and unpadding returns the
    original field (padding.py:54-150); the reference's FNO test keeps the
    output size (test_fno.py:219-253)."""
    x = torch.randn(2, 3, 12, 10, dtype=torch.float64)
    y, pads = R.domain_pad(x, [0.1, 0.2])
    assert pads == [1, 2] and list(y.shape) == [2, 3, 14, 14]
    assert torch.equal(y[:, :, :1], torch.zeros_like(y[:, :, :1]))
    assert torch.equal(y[:, :, :, -2:], torch.zeros_like(y[:, :, :, -2:]))
    assert torch.equal(R.domain_unpad(y, pads), x)


def test_channel_mlp_bf16_products_rounding():
    """The bf16-product MLP rounds each layer's input and weight to the
    nearest bf16, ties to even: 1 + 2^-8 (halfway between 1 and 1 + 2^-7)
    becomes 1 and 1 + 3 * 2^-8 becomes 1 + 2^-6; GELU(1) between the layers is
    rounded before the second product; bf16-exact operands change nothing."""
    one = torch.ones(1, 1, 1, dtype=torch.float64)
    w = [one.reshape(1, 1), one.reshape(1, 1)]
    b = [torch.zeros(1, dtype=torch.float64)] * 2
    y = R.channel_mlp(one * (1 + 2.0 ** -8), w, b, bf16_products=True)
    g1 = 0.5 * (1 + math.erf(1 / math.sqrt(2)))       # GELU(1)
    assert y.item() == torch.tensor(g1).to(torch.bfloat16).item()
    y = R.channel_mlp(one * (1 + 3 * 2.0 ** -8), [one.reshape(1, 1) * 2, one.reshape(1, 1)], b,
                      bf16_products=True)
    x2 = 2 * (1 + 2.0 ** -6)
    assert y.item() == torch.tensor(0.5 * x2 * (1 + math.erf(x2 / math.sqrt(2)))).to(torch.bfloat16).item()
    g = torch.Generator().manual_seed(5)
    xs = torch.randn(2, 3, 7, generator=g).to(torch.bfloat16).double()
    ws = [torch.randn(4, 3, generator=g).to(torch.bfloat16).double(),
          torch.randn(2, 4, generator=g).to(torch.bfloat16).double()]
    bs = [torch.randn(4, generator=g, dtype=torch.float64), torch.randn(2, generator=g, dtype=torch.float64)]
    ref = R.channel_mlp(xs, ws, bs)
    h = R.gelu(torch.einsum("oi,bip->bop", ws[0], xs) + bs[0][:, None])
    exact_hidden = R.bf16_round(h)
    assert torch.allclose(R.channel_mlp(xs, ws, bs, bf16_products=True),
                          torch.einsum("oi,bip->bop", ws[1], exact_hidden) + bs[1][:, None], atol=1e-12)
    assert (R.channel_mlp(xs, ws, bs, bf16_products=True) - ref).abs().max() > 0


def test_fno_forward_bf16_storage_rounds_at_layer_boundaries():
    """bf16_storage rounds the lifting's output and each layer's output to the
    nearest bfloat16, ties to even, and nothing else: closed forms on a model
    whose stored activations are constants.  Lifting: zero weights, output bias
    1 + 2^-8, halfway between the bf16 neighbours 1 and 1 + 2^-7 (so 1.0 under
    ties-to-even).  Layer: zero spectral weight and bias, zero skips, output
    bias 1 + 3 * 2^-8, halfway between 1 + 2^-7 and 1 + 2^-6 (even: 1 + 2^-6).
    Projection: GELU of its input (unit weights, no rounding of products)."""
    z = lambda *s: torch.zeros(*s, dtype=torch.float64)
    one = torch.ones(1, 1, dtype=torch.float64)
    x = z(1, 1, 8, 8)
    lift = {"weights": [z(1, 1), z(1, 1)], "biases": [z(1), torch.tensor([1 + 2.0 ** -8], dtype=torch.float64)]}
    proj = {"weights": [one, one], "biases": [z(1), z(1)]}
    g = lambda v: 0.5 * v * (1 + math.erf(v / math.sqrt(2)))
    params = {"lifting": lift, "projection": proj, "layers": [], "positional_embedding": False}
    close = lambda y, v: torch.allclose(y, torch.full_like(y, v), rtol=0, atol=1e-12)
    y = R.fno_forward(x, params, bf16_storage=True)
    assert close(y, g(1.0))
    y = R.fno_forward(x, params)
    assert close(y, g(1 + 2.0 ** -8))
    layer = {"conv": dict(weight=torch.zeros(1, 1, 4, 3, dtype=torch.complex128), bias=z(1, 1, 1),
                          n_modes=(4, 3), max_n_modes=(4, 3)),
             "fno_skip": {"type": "linear", "w": z(1, 1)},
             "mlp": {"weights": [z(1, 1), z(1, 1)],
                     "biases": [z(1), torch.tensor([1 + 3 * 2.0 ** -8], dtype=torch.float64)]},
             "mlp_skip": {"type": "soft-gating", "w": z(1)}}
    params["layers"] = [layer]
    y = R.fno_forward(x, params, bf16_storage=True)
    assert close(y, g(1 + 2.0 ** -6))
    y = R.fno_forward(x, params)
    assert close(y, g(1 + 3 * 2.0 ** -8))


def _wave(shape, freqs):
    """cos(2 pi sum_d f_d n_d / N_d) on a grid of the given shape."""
    grids = torch.meshgrid(*[torch.arange(n, dtype=torch.float64) for n in shape], indexing="ij")
    return torch.cos(sum(2 * math.pi * f * g / n for f, g, n in zip(freqs, grids, shape)))


@pytest.mark.parametrize("old,new,freqs", [
    ((8, 10, 12), (16, 20, 24), (3, -2, 5)),     # upsampling, even grids
    ((16, 20, 24), (8, 10, 12), (3, -4, 5)),     # downsampling below both Nyquists
    ((9, 11, 13), (12, 7, 20), (2, -3, 3)),      # odd grids, mixed up / down
    ((6, 6, 6, 8), (12, 9, 6, 4), (1, 2, -2, 1)),  # 4D
])
def test_spectral_resample_band_limited(old, new, freqs):
    """A plane wave strictly inside both grids' bands is resampled exactly."""
    x = _wave(old, freqs)[None, None]
    y = R.spectral_resample(x, new)
    assert list(y.shape) == [1, 1, *new]
    assert torch.allclose(y[0, 0], _wave(new, freqs), atol=1e-12)


def test_spectral_resample_odd_grid_residues():
    """On an odd axis of size 2k+1 the kept frequencies are -k-1 .. k-1 (the
    slices [:m//2] and [-m//2:]): upsampling moves the old +k to -k-1, and
    downsampling onto 2k+1 brings the old -k-1 to +k (same residue)."""
    k = 3
    old, new = (2 * k + 1, 4, 6), (12, 4, 6)
    n = torch.arange(new[0], dtype=torch.float64)
    x = _wave(old, (k, 0, 0))[None, None]          # e^{+ik..} + e^{-ik..}, halves
    y = R.spectral_resample(x, new)[0, 0, :, 0, 0]
    want = 0.5 * (torch.cos(2 * math.pi * (-k - 1) * n / new[0]) + torch.cos(2 * math.pi * k * n / new[0]))
    assert torch.allclose(y, want, atol=1e-12)
    x = _wave((12, 4, 6), (-k - 1, 0, 0))[None, None]
    y = R.spectral_resample(x, (2 * k + 1, 4, 6))[0, 0, :, 0, 0]
    m = torch.arange(2 * k + 1, dtype=torch.float64)
    # the old +k+1 component is dropped (outside -k-1 .. k-1), -k-1 lands on +k
    want = 0.5 * torch.cos(2 * math.pi * k * m / (2 * k + 1))
    assert torch.allclose(y, want, atol=1e-12)


def test_complex_valued_wrappers():
    """apply_complex is the complex-linear map with matrix A + iB when the real
    parts apply A and B; CGELU is GELU on each part."""
    g = torch.Generator().manual_seed(31)
    A = torch.randn(4, 5, generator=g, dtype=torch.float64)
    B = torch.randn(4, 5, generator=g, dtype=torch.float64)
    x = torch.complex(torch.randn(5, 3, generator=g, dtype=torch.float64),
                      torch.randn(5, 3, generator=g, dtype=torch.float64))
    y = R.complex_apply(lambda t: A @ t, lambda t: B @ t, x)
    assert torch.allclose(y, torch.complex(A, B) @ x, atol=1e-12)
    z = R.cgelu(x)
    assert torch.equal(z.real, R.gelu(x.real)) and torch.equal(z.imag, R.gelu(x.imag))


def test_circular_shift_equivariance():
    torch.manual_seed(2)
    nms = R.stored_n_modes((6, 6))
    x = torch.randn(2, 3, 12, 10, dtype=torch.float64)
    w = torch.randn(3, 4, *nms, dtype=torch.complex128)
    y = R.spectral_conv_forward(x, w, None, nms, nms)
    ys = R.spectral_conv_forward(torch.roll(x, shifts=(3, -2), dims=(2, 3)), w, None, nms, nms)
    assert torch.allclose(torch.roll(y, shifts=(3, -2), dims=(2, 3)), ys, atol=1e-12)


def test_linearity():
    torch.manual_seed(3)
    nms = R.stored_n_modes((4, 6))
    x1 = torch.randn(2, 3, 8, 12, dtype=torch.float64)
    x2 = torch.randn(2, 3, 8, 12, dtype=torch.float64)
    w = torch.randn(3, 2, *nms, dtype=torch.complex128)
    f = lambda x: R.spectral_conv_forward(x, w, None, nms, nms)
    assert torch.allclose(f(2.5 * x1 - x2), 2.5 * f(x1) - f(x2), atol=1e-12)


@pytest.mark.parametrize("implementation", ["factorized", "reconstructed"])
@pytest.mark.parametrize("dim", [1, 2, 3])
def test_tucker_equals_dense(implementation, dim):
    torch.manual_seed(4)
    sizes = (10,) * dim
    nms = R.stored_n_modes((6,) * dim)
    shape = (3, 4, *nms)
    ranks = [2, 3] + [3] * dim
    core = torch.randn(*ranks, dtype=torch.complex128)
    factors = [torch.randn(s, r, dtype=torch.complex128) for s, r in zip(shape, ranks)]
    x = torch.randn(2, 3, *sizes, dtype=torch.float64)
    full = R.tucker_to_tensor(core, factors)
    yf = R.spectral_conv_forward(x, {"tucker": (core, factors)}, None, nms, nms,
                                 implementation=implementation)
    yd = R.spectral_conv_forward(x, full, None, nms, nms)
    assert torch.allclose(yf, yd, atol=1e-10)


def test_tucker_window_slices_mode_factors():
    torch.manual_seed(5)
    nms = R.stored_n_modes((4, 6))
    mxs = R.stored_n_modes((8, 8))
    shape = (3, 2, *mxs)
    ranks = [2, 2, 3, 3]
    core = torch.randn(*ranks, dtype=torch.complex128)
    factors = [torch.randn(s, r, dtype=torch.complex128) for s, r in zip(shape, ranks)]
    x = torch.randn(1, 3, 12, 12, dtype=torch.float64)
    yf = R.spectral_conv_forward(x, {"tucker": (core, factors)}, None, nms, mxs,
                                 implementation="factorized")
    yd = R.spectral_conv_forward(x, R.tucker_to_tensor(core, factors), None, nms, mxs)
    assert torch.allclose(yf, yd, atol=1e-10)


def test_cp_and_tt_equal_dense():
    torch.manual_seed(6)
    nms = R.stored_n_modes((4, 6))
    shape = (3, 2, *nms)
    x = torch.randn(2, 3, 9, 10, dtype=torch.float64)
    wts = torch.randn(5, dtype=torch.complex128)
    cf = [torch.randn(s, 5, dtype=torch.complex128) for s in shape]
    y1 = R.spectral_conv_forward(x, {"cp": (wts, cf)}, None, nms, nms, implementation="factorized")
    y2 = R.spectral_conv_forward(x, R.cp_to_tensor(wts, cf), None, nms, nms)
    assert torch.allclose(y1, y2, atol=1e-10)
    ranks = [1, 2, 3, 2, 1]
    tf = [torch.randn(ranks[k], s, ranks[k + 1], dtype=torch.complex128) for k, s in enumerate(shape)]
    y1 = R.spectral_conv_forward(x, {"tt": tf}, None, nms, nms, implementation="factorized")
    y2 = R.spectral_conv_forward(x, R.tt_to_tensor(tf), None, nms, nms)
    assert torch.allclose(y1, y2, atol=1e-10)


def test_separable_matches_closed_form():
    torch.manual_seed(7)
    nms = R.stored_n_modes((4, 6))
    x = torch.randn(2, 3, 9, 12, dtype=torch.float64)
    w = torch.randn(3, *nms, dtype=torch.complex128)
    y = R.spectral_conv_forward(x, w, None, nms, nms, separable=True)
    yd = dft64.spectral_conv(x.numpy(), w.numpy(), None, nms, nms, separable=True)
    assert np.abs(y.numpy() - yd).max() < 1e-12


def test_gelu_is_exact_erf():
    xs = torch.tensor([-3.0, -1.0, 0.0, 0.5, 1.0, 2.0], dtype=torch.float64)
    ref = torch.tensor([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in xs.tolist()], dtype=torch.float64)
    assert torch.allclose(R.gelu(xs), ref, atol=1e-15)
    # gelu(1) = Phi(1) = 0.8413447460685429 (standard normal CDF)
    assert abs(R.gelu(torch.tensor(1.0, dtype=torch.float64)).item() - 0.8413447460685429) < 1e-15
    # the tanh approximation differs by more than the 1e-4 tolerance somewhere
    t = torch.linspace(-5, 5, 2001, dtype=torch.float64)
    tanh_gelu = torch.nn.functional.gelu(t, approximate="tanh")
    assert (tanh_gelu - R.gelu(t)).abs().max() > 1e-4


def test_grid_embedding_coordinates():
    x = torch.zeros(2, 1, 4, 8)
    e = R.grid_embedding_nd(x)
    assert e.shape == (2, 3, 4, 8)
    assert torch.allclose(e[0, 1, :, 0], torch.tensor([0.0, 0.25, 0.5, 0.75]))
    assert torch.allclose(e[0, 2, 0, :], torch.arange(8) / 8.0)


def test_linear_skip_is_channel_matmul():
    torch.manual_seed(8)
    x = torch.randn(2, 3, 5, 6)
    ws = torch.randn(4, 3)
    assert torch.allclose(R.linear_skip(x, ws), torch.einsum("oi,bihw->bohw", ws, x), atol=1e-6)


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "*.npz"))),
                         ids=lambda p: os.path.basename(p)[:-4])
def test_oracle_reproduces_golden(path):
    d = np.load(path)
    x = torch.from_numpy(d["x"]).double()
    w = torch.from_numpy(d["w"]).to(torch.complex128)
    b = torch.from_numpy(d["bias"]).double()
    nms = d["stored_n_modes"].tolist()
    mxs = d["max_n_modes"].tolist()
    outs = tuple(d["out_sizes"].tolist())
    norm = str(d["norm"])
    y = R.spectral_conv_forward(x, w, b, nms, mxs, fft_norm=norm, output_shape=outs)
    if "skip_w" in d:
        y = R.gelu(y + R.linear_skip(x, torch.from_numpy(d["skip_w"]).double()))
    exp = d["expected"]
    assert np.abs(y.numpy() - exp).max() <= 1e-6 * np.abs(exp).max()


# ------------------------------------------------- fno_block_precision half
def test_fp16_round_ties_to_even():
    """float16 has 10 fraction bits: 1 + 2^-11 is half way between 1 and
    1 + 2^-10 (goes to the even 1), 1 + 3 2^-11 half way between 1 + 2^-10
    and 1 + 2^-9 (goes to the even 1 + 2^-9); 2049 lies between 2048 and
    2050 (spacing 2) and goes to 2048; complex parts round separately."""
    t = torch.tensor([1 + 2 ** -11, 1 + 3 * 2 ** -11, 2049.0, -2049.0, 1 + 2 ** -10],
                     dtype=torch.float64)
    want = torch.tensor([1.0, 1 + 2 ** -9, 2048.0, -2048.0, 1 + 2 ** -10], dtype=torch.float64)
    assert torch.equal(R.fp16_round(t), want)
    c = torch.complex(t, t.flip(0))
    assert torch.equal(R.fp16_round(c), torch.complex(want, want.flip(0)))


def test_complexhalf_contraction_rounds_partial_sums():
    """einsum_utils.py:10-34 rounds each real partial contraction to float16
    before Re = t00 - t11: with Xr = (2048, 1), Wr = (1, 1) the exact
    t00 = 2049 becomes 2048, and t11 = Xi . Wi = 1, so Re = 2047 where the
    exact complex product gives 2048; Im = fp16(t10 + t01) = fp16(1 + 2048) =
    2048.  Swapping the pairing (Re = t00 - t10, say) or dropping a rounding
    changes the answer."""
    f64 = lambda v: torch.tensor(v, dtype=torch.float64)
    x = torch.complex(f64([2048.0, 1.0]), f64([1.0, 0.0]))
    w = torch.complex(f64([1.0, 1.0]), f64([1.0, 0.0]))
    xs = x.reshape(1, 2, 1)          # [B, Ci, mode]
    ws = w.reshape(2, 1, 1)          # [Ci, Co, mode]
    y = R.contract_dense_complexhalf(xs, ws)
    assert y.shape == (1, 1, 1)
    assert y.real.item() == 2047.0 and y.imag.item() == 2048.0
    exact = R.contract_dense(xs, ws)
    assert exact.real.item() == 2048.0 and exact.imag.item() == 2049.0


def test_complexhalf_contraction_exact_on_small_integers():
    """With operands and every partial sum exactly representable in float16
    (small integers), the complex-half contraction equals the exact one."""
    g = torch.Generator().manual_seed(5)
    xs = torch.complex(torch.randint(-4, 5, (2, 3, 4, 3), generator=g).double(),
                       torch.randint(-4, 5, (2, 3, 4, 3), generator=g).double())
    ws = torch.complex(torch.randint(-4, 5, (3, 5, 4, 3), generator=g).double(),
                       torch.randint(-4, 5, (3, 5, 4, 3), generator=g).double())
    assert torch.equal(R.contract_dense_complexhalf(xs, ws), R.contract_dense(xs, ws))


@pytest.mark.parametrize("precision", ["half", "mixed"])
def test_half_precision_forward_output_is_float16(precision):
    """The half forward's output (before the bias) is float16-valued, and
    with x exactly representable in float16 'half' and 'mixed' agree (they
    differ only in rounding x before the transform)."""
    g = torch.Generator().manual_seed(6)
    x = (torch.randint(-64, 65, (2, 3, 16, 12), generator=g) / 32).double()
    w = torch.complex(torch.randn(3, 4, 8, 7, generator=g, dtype=torch.float64),
                      torch.randn(3, 4, 8, 7, generator=g, dtype=torch.float64))
    y = R.spectral_conv_forward(x, w, None, [8, 7], [8, 7], precision=precision)
    assert torch.equal(R.fp16_round(y), y)
    other = "mixed" if precision == "half" else "half"
    assert torch.equal(y, R.spectral_conv_forward(x, w, None, [8, 7], [8, 7], precision=other))
    full = R.spectral_conv_forward(x, w, None, [8, 7], [8, 7])
    assert 0 < (y - full).abs().max().item() <= 4e-3 * full.abs().max().item()
