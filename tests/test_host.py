"""Host-side behaviour of the drop-in modules (no GPU needed): constructor
semantics, n_modes bookkeeping, weight windows and error conventions, as the
reference's own tests exercise them (neuralop/layers/tests/
test_spectral_convolution.py, test_fno_block.py:25-34, models/tests/test_fno.py)."""
import math

import pytest
import torch

import neuraloperator_amd as na
from neuraloperator_amd.spectral_convolution import get_contract_fun
from oracle import spectral_ref as R


def test_n_modes_last_dim_halved():
    conv = na.SpectralConv(3, 4, (10, 8, 6))
    assert conv.n_modes == [10, 8, 4]
    conv.n_modes = (6, 6, 4)
    assert conv.n_modes == [6, 6, 3]
    assert list(conv.max_n_modes) == [10, 8, 4]


def test_n_modes_30_keeps_16_rfft_modes():
    # the 1D benchmark's W[64,64,16] corresponds to n_modes=30 in the API
    conv = na.SpectralConv(64, 64, 30)
    assert conv.n_modes == [16]
    assert conv.weight.shape == (64, 64, 16)
    assert na.SpectralConv(64, 64, 16).weight.shape == (64, 64, 9)


def test_fno_block_n_modes_setter():
    for dim in [1, 2, 3]:
        mx = [8, 8, 8][:dim]
        block = na.FNOBlocks(3, 4, mx, max_n_modes=mx, n_layers=1, channel_mlp_skip="linear")
        assert block.convs[0].n_modes[:-1] == mx[:-1]
        assert block.convs[0].n_modes[-1] == mx[-1] // 2 + 1
        block.n_modes = [4, 4, 4][:dim]
        assert block.convs[0].n_modes[-1] == 4 // 2 + 1


def test_weight_shapes_and_init_std():
    conv = na.SpectralConv(8, 6, (12, 12), bias=True)
    assert conv.weight.shape == (8, 6, 12, 7)
    assert conv.bias.shape == (6, 1, 1)
    w = conv.weight.to_tensor().detach()
    std = (2 / (8 + 6)) ** 0.5
    assert torch.is_complex(conv.weight)
    assert abs(w.abs().pow(2).mean().sqrt().item() - std) < 0.15 * std


def test_window_matches_reference_slices():
    conv = na.SpectralConv(3, 3, (8, 8), max_n_modes=(12, 12))
    conv.n_modes = (6, 8)
    for sizes in [(16, 16), (9, 10), (5, 6)]:
        kept, sl = conv.window(sizes)
        fft_size = [sizes[0], sizes[1] // 2 + 1]
        ref_sl = R.weight_slices(fft_size, conv.n_modes, conv.max_n_modes)
        assert sl == ref_sl
        w = conv.weight.to_tensor()
        assert list(w[sl].shape[2:]) == kept


def test_factorized_weights_reconstruct():
    for fact in ["Tucker", "CP", "TT"]:
        conv = na.SpectralConv(4, 5, (6, 6), factorization=fact, rank=0.5, implementation="factorized")
        full = conv.weight.to_tensor()
        assert full.shape == (4, 5, 6, 4)
        assert torch.is_complex(full)
        sub = conv.weight[:, :, 1:5, :3]
        assert torch.allclose(sub.to_tensor(), full[:, :, 1:5, :3], atol=1e-5)


C4_TUCKER_RANK = (20, 20, 10, 10, 6)


def test_tfno_default_ranks():
    """TFNO's default Tucker rank 0.1 on the 3D workload's (32, 32, 16, 16, 9)
    weight gives the tuple the 3D TFNO benchmark records."""
    t = na.TFNO((16, 16, 16), in_channels=1, out_channels=1, hidden_channels=32, n_layers=1)
    w = t.fno_blocks.convs[0].weight
    assert w.name == "ComplexTucker"
    assert tuple(w.rank) == C4_TUCKER_RANK


def _cardano(p, q):
    """Real root of t^3 + p t + q = 0 for p > 0 (one real root)."""
    d = math.sqrt(q * q / 4 + p ** 3 / 27)
    cb = lambda v: math.copysign(abs(v) ** (1 / 3), v)
    return cb(-q / 2 + d) + cb(-q / 2 - d)


def test_tucker_rank_closed_forms():
    """tucker_rank solves prod(s) x^N + sum(s^2) x = rank prod(s) (core plus
    factor parameters equal to the requested fraction of the dense count) and
    rounds s_i x.  Pinned by the equation's closed-form roots: linear (one
    mode), quadratic (two modes), Cardano's cubic (three equal modes), and by
    the integer / tuple / "same" special cases."""
    from neuraloperator_amd.factorized_tensors import tucker_rank
    # one mode: s x + s^2 x = r s  ->  x = r / (1 + s)
    for s, r in [(9, 2.0), (31, 4.0), (15, 1.0)]:
        x = r / (1 + s)
        assert tucker_rank((s,), r) == [max(round(s * x), 1)]
    # two equal modes at rank 1: x^2 + 2x - 1 = 0  ->  x = sqrt(2) - 1
    for s in (10, 20, 30, 64):
        assert tucker_rank((s, s), 1.0) == [round(s * (math.sqrt(2) - 1))] * 2
        assert tucker_rank((s, s), "same") == tucker_rank((s, s), 1.0)
    # two modes: a b x^2 + (a^2 + b^2) x - r a b = 0
    for a, b, r in [(32, 9, 0.5), (64, 17, 0.25), (12, 40, 0.8)]:
        x = (-(a * a + b * b) + math.sqrt((a * a + b * b) ** 2 + 4 * a * b * r * a * b)) / (2 * a * b)
        assert tucker_rank((a, b), r) == [max(round(a * x), 1), max(round(b * x), 1)]
    # three equal modes: x^3 + (3 / s) x - r = 0
    for s, r in [(16, 0.1), (32, 0.05), (24, 0.3)]:
        x = _cardano(3.0 / s, -r)
        assert abs(x ** 3 + 3 * x / s - r) < 1e-12
        assert tucker_rank((s, s, s), r) == [round(s * x)] * 3
    # the rank tuple of the 3D workload: its unrounded fraction reproduces
    # 10% of the dense count, and each rank is s_i x rounded
    shape = (32, 32, 16, 16, 9)
    ranks = tucker_rank(shape, 0.1)
    x = ranks[0] / 32
    lo, hi = (ranks[0] - 0.5) / 32, (ranks[0] + 0.5) / 32
    n = math.prod(shape)
    f = lambda v: n * v ** 5 + sum(s * s for s in shape) * v - 0.1 * n
    assert f(lo) < 0 < f(hi)          # the root lies where 32 x rounds to ranks[0]
    assert tuple(ranks) == C4_TUCKER_RANK
    # integer and tuple ranks pass through
    assert tucker_rank((4, 5, 6), 3) == [3, 3, 3]
    assert tucker_rank((4, 5, 6), (1, 2, 3)) == [1, 2, 3]


def test_errors_follow_reference_conventions():
    with pytest.raises(ValueError):
        na.SpectralConv(3, 4, (4, 4), separable=True)
    with pytest.raises(ValueError):
        na.SpectralConv(3, 3, (4, 4), implementation="bogus")
    with pytest.raises(ValueError):
        na.SpectralConv(3, 3, (4, 4), factorization="bogus")
    with pytest.raises(ValueError):
        na.skip_connection(3, 3, skip_type="bogus")
    with pytest.raises(ValueError):
        na.SoftGating(3, 4)
    assert get_contract_fun(torch.zeros(1), "factorized") == "dense"


def test_cpu_forward_fails_loudly():
    conv = na.SpectralConv(3, 4, (4, 4))
    with pytest.raises(RuntimeError, match="GPU"):
        conv(torch.randn(1, 3, 8, 8))


def test_fno_construction_and_param_count():
    m = na.FNO((64, 64), in_channels=1, out_channels=1, hidden_channels=64, n_layers=4)
    n_spec = 4 * 64 * 64 * 64 * 33
    assert sum(p.numel() for p in m.fno_blocks.convs.parameters() if p.is_complex()) == n_spec
    assert m.lifting.fcs[0].in_channels == 3   # 1 channel + 2 grid coordinates
    assert m.projection.fcs[-1].out_channels == 1


def test_profiler_sections():
    prof = na.TimingProfiler()
    with na.profiling(prof):
        assert na.get_active_profiler() is prof
        with na.maybe_profile(prof, "a/b"):
            pass
    assert na.get_active_profiler() is None
    assert "a/b" in prof.stats()


def test_validate_scaling_factor():
    assert na.validate_scaling_factor(None, 2) is None
    assert na.validate_scaling_factor(2, 2) == [2.0, 2.0]
    assert na.validate_scaling_factor(0.5, 2, 3) == [[0.5, 0.5]] * 3
    assert na.validate_scaling_factor([1, 2], 2) == [1.0, 2.0]


def test_fno_staged_construction():
    """FNOStaged (fno_staged.py:24-190): per-layer mode counts, the
    reference's argument checks and top-level attribute names."""
    m = na.FNOStaged([(8, 8), (6, 6), (4, 4)], in_channels=1, out_channels=2, hidden_channels=16)
    assert m.n_layers == 3
    assert [c.n_modes for c in m.convs] == [[8, 5], [6, 4], [4, 3]]
    # max_n_modes_per_layer defaults to the raw per-layer tuples, which
    # SpectralConv takes as given (not halved): the weights keep those shapes
    assert [tuple(c.weight.shape[2:]) for c in m.convs] == [(8, 8), (6, 6), (4, 4)]
    assert {"convs", "fno_skips", "channel_mlp", "channel_mlp_skips", "lifting", "projection"} <= \
        {k.split(".")[0] for k in m.state_dict()}
    assert m.lifting.in_channels == 3 and m.projection.out_channels == 2
    with pytest.raises(ValueError):
        na.FNOStaged([(8, 8), (6, 6)], in_channels=1, out_channels=1, hidden_channels=8, n_layers=3)
    with pytest.raises(ValueError):
        na.FNOStaged([(8, 8), (6, 6)], 1, 1, 8, max_n_modes_per_layer=[(8, 8)])
    with pytest.raises(NotImplementedError):
        na.FNOStaged([(8, 8)], 1, 1, 8, no_br=True, resolution_scaling_factor=2)


def test_fno_staged_bitrev():
    """_bitrev_spatial is an involution on power-of-two dims and leaves other
    sizes alone (reference test_fno_staged_no_br.py:32-62)."""
    x = torch.randn(2, 3, 16, 12)
    y = na.FNOStaged._bitrev_spatial(x)
    assert torch.equal(x, na.FNOStaged._bitrev_spatial(y))
    assert not torch.equal(x, y)
    assert torch.equal(y[:, :, :, :], x[:, :, [0, 8, 4, 12, 2, 10, 6, 14, 1, 9, 5, 13, 3, 11, 7, 15], :])
    z = torch.randn(1, 1, 9, 10)
    assert torch.equal(z, na.FNOStaged._bitrev_spatial(z))


def test_ada_in_norm_closed_form():
    """AdaIN (normalization_layers.py:5-56): per-channel instance statistics,
    then scale and shift from the two halves of mlp(embedding); one embedding
    for every norm layer or one per layer (fno_block.py:304-321)."""
    torch.manual_seed(3)
    block = na.FNOBlocks(3, 4, (8, 8), n_layers=1, norm="ada_in", ada_in_features=5,
                         channel_mlp_skip="linear")
    e = torch.randn(5)
    block.set_ada_in_embeddings(e)
    x = torch.randn(2, 4, 10, 6)
    norm = block.norm[0]
    scale, shift = norm.mlp(e).split(4)
    mean = x.mean(dim=(2, 3), keepdim=True)
    var = x.var(dim=(2, 3), unbiased=False, keepdim=True)
    want = (x - mean) / torch.sqrt(var + 1e-5) * scale.view(1, 4, 1, 1) + shift.view(1, 4, 1, 1)
    assert torch.allclose(norm(x), want, atol=1e-5)
    e2 = [torch.randn(5), torch.randn(5)]
    block.set_ada_in_embeddings(*e2)
    assert torch.equal(block.norm[1].embedding, e2[1])
    cblock = na.FNOBlocks(3, 4, (8, 8), n_layers=1, norm="ada_in", ada_in_features=5,
                          channel_mlp_skip="linear", complex_data=True)
    cblock.set_ada_in_embeddings(e)
    assert torch.equal(cblock.norm[0].fi.embedding, e)


# ---- backward algebra of the spectral convolution, on the CPU -------------
# _SpectralConvFn's backward (index maps of resized outputs, the zeroed
# column's symmetrisation, separable products, dual-norm scaling) with the
# library's window transforms restated in torch.fft (float64), against
# autograd through the same restated forward: checks the host-side gradient
# logic without a GPU; the GPU tests check the transforms themselves.
def _fft_size(sizes):
    f = list(sizes)
    f[-1] = f[-1] // 2 + 1
    return f


def _rfft_window(x, modes, norm="forward"):
    nd = len(modes)
    dims = list(range(-nd, 0))
    xf = torch.fft.rfftn(x.to(torch.float64), norm=norm, dim=dims)
    if nd > 1:
        xf = torch.fft.fftshift(xf, dim=dims[:-1])
    return xf[R.x_slices(_fft_size(x.shape[2:]), list(modes))]


def _irfft_window(yhat, in_sizes, out_sizes, bias=None, norm="forward", enforce=True):
    B, C, *m = yhat.shape
    nd = len(m)
    dims = list(range(-nd, 0))
    fs = _fft_size(in_sizes)
    out = torch.zeros(B, C, *fs, dtype=torch.complex128)
    out[R.x_slices(fs, m)] = yhat
    if nd > 1:
        out = torch.fft.ifftshift(out, dim=dims[:-1])
    ms = list(out_sizes)
    if enforce:
        out = torch.fft.ifftn(out, s=ms[:-1], dim=dims[:-1], norm=norm) if nd > 1 else out.clone()
        out[..., 0].imag.zero_()
        if ms[-1] % 2 == 0:
            out[..., -1].imag.zero_()
        y = torch.fft.irfft(out, n=ms[-1], dim=dims[-1], norm=norm)
    else:
        y = torch.fft.irfftn(out, s=ms, dim=dims, norm=norm)
    return y if bias is None else y + bias.view(1, -1, *([1] * nd))


def _contract(x, w, separable=False):
    return R.contract_dense_separable(x, w) if separable else R.contract_dense(x, w)


@pytest.mark.parametrize("sizes,kept,outs,sep", [
    ((16,), (9,), (32,), False), ((16,), (9,), (8,), False), ((15,), (8,), (30,), False),
    ((8, 8), (6, 5), (16, 16), False), ((8, 8), (8, 5), (4, 6), False),
    ((12, 10), (6, 6), (24, 20), True), ((9, 7), (8, 4), (18, 14), False),
    ((6, 8, 10), (6, 8, 6), (3, 16, 20), True), ((8, 8), (6, 5), (8, 8), True),
])
@pytest.mark.parametrize("norm", ["forward", "ortho"])
@pytest.mark.parametrize("enforce", [True, False])
def test_spectral_conv_backward_algebra(sizes, kept, outs, sep, norm, enforce, monkeypatch):
    from neuraloperator_amd import functional as Fh
    from neuraloperator_amd import spectral_convolution as S
    monkeypatch.setattr(Fh, "rfft_window", _rfft_window)
    monkeypatch.setattr(Fh, "irfft_window", _irfft_window)
    monkeypatch.setattr(Fh, "contract_dense", _contract)
    torch.manual_seed(0)
    C, B = 3, 2
    x = torch.randn(B, C, *sizes, dtype=torch.float64)
    wshape = (C, *kept) if sep else (C, C, *kept)
    w = torch.complex(torch.randn(*wshape, dtype=torch.float64),
                      torch.randn(*wshape, dtype=torch.float64))
    bias = torch.randn(1, C, *([1] * len(sizes)), dtype=torch.float64)
    g = torch.randn(B, C, *outs, dtype=torch.float64)
    leaves = [t.clone().requires_grad_(True) for t in (x, w, bias)]
    y = S._SpectralConvFn.apply(*leaves, list(kept), norm, list(outs), sep, enforce)
    got = torch.autograd.grad((y * g).sum(), leaves)
    ref_leaves = [t.clone().requires_grad_(True) for t in (x, w, bias)]
    xr, wr, br = ref_leaves
    yr = _irfft_window(_contract(_rfft_window(xr, kept, norm), wr, sep), sizes, outs, None, norm,
                       enforce) + br
    want = torch.autograd.grad((yr * g).sum(), ref_leaves)
    # the backward runs in float32 (as on the GPU)
    for a, b in zip(got, want):
        assert ((a - b).abs().max() / b.abs().max()).item() < 1e-5


def _fft_window(x, modes, norm="forward"):
    nd = len(modes)
    dims = list(range(-nd, 0))
    xf = torch.fft.fftn(x.to(torch.complex128), norm=norm, dim=dims)
    if nd > 1:
        xf = torch.fft.fftshift(xf, dim=dims)
    return xf[R.x_slices(list(x.shape[2:]), list(modes))]


def _ifft_window(yhat, in_sizes, out_sizes, bias=None, norm="forward"):
    B, C, *m = yhat.shape
    nd = len(m)
    dims = list(range(-nd, 0))
    out = torch.zeros(B, C, *in_sizes, dtype=torch.complex128)
    out[R.x_slices(list(in_sizes), m)] = yhat
    if nd > 1:   # the reference un-shifts the non-last axes only (:531-532)
        out = torch.fft.ifftshift(out, dim=dims[:-1])
    y = torch.fft.ifftn(out, s=list(out_sizes), dim=dims, norm=norm)
    return y if bias is None else y + bias.view(1, -1, *([1] * nd))


@pytest.mark.parametrize("sizes,kept,outs,sep", [
    ((16,), (7,), (16,), False), ((16,), (7,), (32,), False), ((15,), (9,), (8,), True),
    ((8, 8), (6, 5), (8, 8), False), ((8, 8), (6, 5), (16, 12), False),
    ((8, 10), (8, 10), (5, 20), True), ((9, 7), (5, 7), (18, 6), False),
    ((6, 8, 10), (4, 6, 6), (12, 4, 20), True),
])
@pytest.mark.parametrize("norm", ["backward", "ortho"])
def test_complex_spectral_conv_backward_algebra(sizes, kept, outs, sep, norm, monkeypatch):
    from neuraloperator_amd import functional as Fh
    from neuraloperator_amd import spectral_convolution as S
    monkeypatch.setattr(Fh, "fft_window", _fft_window)
    monkeypatch.setattr(Fh, "ifft_window", _ifft_window)
    monkeypatch.setattr(Fh, "contract_dense", _contract)
    torch.manual_seed(1)
    C, B = 3, 2
    cplx = lambda *s: torch.complex(torch.randn(*s, dtype=torch.float64),
                                    torch.randn(*s, dtype=torch.float64))
    x = cplx(B, C, *sizes)
    w = cplx(*((C, *kept) if sep else (C, C, *kept)))
    bias = torch.randn(1, C, *([1] * len(sizes)), dtype=torch.float64)
    g = cplx(B, C, *outs)
    leaves = [t.clone().requires_grad_(True) for t in (x, w, bias)]
    y = S._SpectralConvComplexFn.apply(*leaves, list(kept), norm, list(outs), sep)
    got = torch.autograd.grad((y * g).real.sum(), leaves)
    ref_leaves = [t.clone().requires_grad_(True) for t in (x, w, bias)]
    xr, wr, br = ref_leaves
    yr = _ifft_window(_contract(_fft_window(xr, kept, norm), wr, sep), sizes, outs, None, norm)
    yr = yr + br
    want = torch.autograd.grad((yr * g).real.sum(), ref_leaves)
    for a, b in zip(got, want):
        assert ((a - b).abs().max() / b.abs().max()).item() < 1e-5


def test_boundary_resolves_lazy_conjugates():
    """w.conj() is a view with torch's conjugate bit over w's storage, and
    .contiguous() keeps it when the view is already contiguous: the C-ABI
    would read w itself.  The boundary helpers resolve the bit (so the data
    handed over is conj(w)), and the pointer helper refuses an unresolved
    view."""
    from neuraloperator_amd import functional as Fh
    w = torch.randn(3, 4, dtype=torch.complex64)
    v = w.conj().contiguous()
    assert v.is_conj() and v.data_ptr() == w.data_ptr()
    r = Fh._c64(v)
    assert not r.is_conj()
    assert torch.equal(torch.view_as_real(r), torch.view_as_real(w.conj().resolve_conj()))
    assert torch.equal(torch.view_as_real(Fh._c64(-w.conj())),
                       torch.view_as_real((-w.conj()).resolve_conj().resolve_neg()))
    with pytest.raises(RuntimeError, match="conjugate"):
        Fh._ptr(v)
