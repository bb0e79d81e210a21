"""Plain-torch CPU restatement of the reference FNO spectral path.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Every function follows
the reference op sequence one step at a time, citing the file:line it
restates (paths relative to the reference repository root).
"""
from __future__ import annotations

import math
from typing import List, Optional, Sequence

import torch
import torch.nn.functional as F

EINSUM_SYMBOLS = "abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ"


# ---------------------------------------------------------------------------
# n_modes bookkeeping
# ---------------------------------------------------------------------------
def stored_n_modes(n_modes, complex_data: bool = False) -> List[int]:
    """n_modes as stored by the setter (spectral_convolution.py:404-415):
    the last entry becomes n//2+1 for real data."""
    if isinstance(n_modes, int):
        n_modes = [n_modes]
    else:
        n_modes = list(n_modes)
    if not complex_data:
        n_modes[-1] = n_modes[-1] // 2 + 1
    return n_modes


def weight_slices(fft_size, n_modes, max_n_modes, separable=False, complex_data=False):
    """Weight window (spectral_convolution.py:465-489)."""
    starts = [
        (max_modes - min(size, n_mode))
        for (size, n_mode, max_modes) in zip(fft_size, n_modes, max_n_modes)
    ]
    sl = [slice(None)] if separable else [slice(None), slice(None)]
    if complex_data:
        sl += [slice(s // 2, -s // 2) if s else slice(s, None) for s in starts]
    else:
        sl += [slice(s // 2, -s // 2) if s else slice(s, None) for s in starts[:-1]]
        sl += [slice(None, -starts[-1]) if starts[-1] else slice(None)]
    return tuple(sl)


def x_slices(fft_size, kept_modes):
    """Input-spectrum window (spectral_convolution.py:500-519)."""
    sl = [slice(None), slice(None)]
    for all_modes, kept in zip(fft_size, kept_modes):
        center = all_modes // 2
        neg = kept // 2
        pos = kept // 2 + kept % 2
        sl.append(slice(center - neg, center + pos))
    if kept_modes[-1] < fft_size[-1]:
        sl[-1] = slice(None, kept_modes[-1])
    else:
        sl[-1] = slice(None)
    return tuple(sl)


# ---------------------------------------------------------------------------
# contractions
# ---------------------------------------------------------------------------
def einsum_pairwise(eq: str, *operands):
    """Multi-operand einsum evaluated as a sequence of two-operand einsums,
    each step contracting the pair whose result is smallest (a greedy
    contraction path).  The reference's tl.einsum goes through opt_einsum's
    path search (spectral_convolution.py:16-17); torch.einsum without
    opt_einsum contracts left to right, which for the Tucker equations builds
    intermediates of hundreds of GB.  The path only changes rounding."""
    lhs, out = eq.split("->")
    terms = lhs.split(",")
    ops = list(operands)
    sizes = {}
    for t, op in zip(terms, ops):
        for s, n in zip(t, op.shape):
            sizes[s] = n
    while len(ops) > 2:
        best = None
        for a in range(len(ops)):
            for b in range(a + 1, len(ops)):
                others = set(out).union(*[set(t) for k, t in enumerate(terms) if k not in (a, b)])
                keep = "".join(s for s in dict.fromkeys(terms[a] + terms[b]) if s in others)
                cost = math.prod(sizes[s] for s in keep)
                if best is None or cost < best[0]:
                    best = (cost, a, b, keep)
        _, a, b, keep = best
        r = torch.einsum(f"{terms[a]},{terms[b]}->{keep}", ops[a], ops[b])
        terms = [t for k, t in enumerate(terms) if k not in (a, b)] + [keep]
        ops = [o for k, o in enumerate(ops) if k not in (a, b)] + [r]
    return torch.einsum(f"{','.join(terms)}->{out}", *ops)


def contract_dense(x, weight, separable=False):
    """spectral_convolution.py:21-46 (tl.einsum -> opt_einsum -> torch)."""
    order = x.ndim
    x_syms = list(EINSUM_SYMBOLS[:order])
    weight_syms = list(x_syms[1:])
    if separable:
        out_syms = [x_syms[0]] + list(weight_syms)
    else:
        weight_syms.insert(1, EINSUM_SYMBOLS[order])
        out_syms = list(weight_syms)
        out_syms[0] = x_syms[0]
    eq = f'{"".join(x_syms)},{"".join(weight_syms)}->{"".join(out_syms)}'
    return torch.einsum(eq, x, weight)


def contract_dense_separable(x, weight, separable=True):
    """spectral_convolution.py:49-52."""
    return x * weight


def fp16_round(t):
    """Round to the nearest float16 (ties to even) and widen back; complex
    tensors part by part (the values a complex32 tensor holds)."""
    if t.is_complex():
        return torch.complex(fp16_round(t.real), fp16_round(t.imag))
    return t.to(torch.float16).to(t.dtype)


def contract_dense_complexhalf(x, weight, separable=False):
    """_contract_dense on complex32 operands (spectral_convolution.py:41-43 ->
    einsum_utils.py:10-34): both operands viewed as real pairs and rounded to
    float16, one real contraction per (x part, weight part) pair, each result
    rounded to float16 (half GEMM, fp32 accumulation: float64 here), then
    Re = tmp[0, 0] - tmp[1, 1] and Im = tmp[1, 0] + tmp[0, 1] in float16."""
    xr, xi = fp16_round(x.real), fp16_round(x.imag)
    wr, wi = fp16_round(weight.real), fp16_round(weight.imag)
    c = lambda a, b: fp16_round(contract_dense(a, b, separable))
    t00, t11 = c(xr, wr), c(xi, wi)
    t10, t01 = c(xi, wr), c(xr, wi)
    return torch.complex(fp16_round(t00 - t11), fp16_round(t10 + t01))


def contract_tucker(x, core, factors, separable=False):
    """spectral_convolution.py:76-103 (einsum with core and all factors)."""
    order = x.ndim
    x_syms = str(EINSUM_SYMBOLS[:order])
    out_sym = EINSUM_SYMBOLS[order]
    out_syms = list(x_syms)
    if separable:
        core_syms = EINSUM_SYMBOLS[order + 1: 2 * order]
        factor_syms = [xs + rs for (xs, rs) in zip(x_syms[1:], core_syms)]
    else:
        core_syms = EINSUM_SYMBOLS[order + 1: 2 * order + 1]
        out_syms[1] = out_sym
        factor_syms = [EINSUM_SYMBOLS[1] + core_syms[0], out_sym + core_syms[1]]
        factor_syms += [xs + rs for (xs, rs) in zip(x_syms[2:], core_syms[2:])]
    eq = f'{x_syms},{core_syms},{",".join(factor_syms)}->{"".join(out_syms)}'
    return einsum_pairwise(eq, x, core, *factors)


def contract_cp(x, weights, factors, separable=False):
    """spectral_convolution.py:55-73."""
    order = x.ndim
    x_syms = str(EINSUM_SYMBOLS[:order])
    rank_sym = EINSUM_SYMBOLS[order]
    out_sym = EINSUM_SYMBOLS[order + 1]
    out_syms = list(x_syms)
    if separable:
        factor_syms = [EINSUM_SYMBOLS[1] + rank_sym]
    else:
        out_syms[1] = out_sym
        factor_syms = [EINSUM_SYMBOLS[1] + rank_sym, out_sym + rank_sym]
    factor_syms += [xs + rank_sym for xs in x_syms[2:]]
    eq = f'{x_syms},{rank_sym},{",".join(factor_syms)}->{"".join(out_syms)}'
    return einsum_pairwise(eq, x, weights, *factors)


def contract_tt(x, factors, separable=False):
    """spectral_convolution.py:106-132."""
    order = x.ndim
    x_syms = list(EINSUM_SYMBOLS[:order])
    weight_syms = list(x_syms[1:])
    if not separable:
        weight_syms.insert(1, EINSUM_SYMBOLS[order])
        out_syms = list(weight_syms)
        out_syms[0] = x_syms[0]
    else:
        out_syms = list(x_syms)
    rank_syms = list(EINSUM_SYMBOLS[order + 1:])
    tt_syms = [[rank_syms[i], s, rank_syms[i + 1]] for i, s in enumerate(weight_syms)]
    eq = "".join(x_syms) + "," + ",".join("".join(f) for f in tt_syms) + "->" + "".join(out_syms)
    return einsum_pairwise(eq, x, *factors)


# ---------------------------------------------------------------------------
# factorized weight reconstruction (tltorch semantics, restated)
# ---------------------------------------------------------------------------
def tucker_to_tensor(core, factors):
    """Full tensor of a Tucker decomposition: core x_0 U_0 x_1 U_1 ..."""
    t = core
    for mode, U in enumerate(factors):
        t = torch.movedim(torch.tensordot(t, U, dims=([mode], [1])), -1, mode)
    return t


def cp_to_tensor(weights, factors):
    """Full tensor of a CP decomposition sum_r w_r u_0r o u_1r o ..."""
    order = len(factors)
    syms = EINSUM_SYMBOLS[:order]
    eq = "z," + ",".join(s + "z" for s in syms) + "->" + syms
    return torch.einsum(eq, weights, *factors)


def tt_to_tensor(factors):
    """Full tensor of a tensor train (cores r_k x n_k x r_{k+1})."""
    full = factors[0]
    for f in factors[1:]:
        full = torch.tensordot(full, f, dims=([-1], [0]))
    return full.squeeze(0).squeeze(-1)


# ---------------------------------------------------------------------------
# SpectralConv.forward restated (spectral_convolution.py:417-570)
# ---------------------------------------------------------------------------
def spectral_conv_forward(
    x: torch.Tensor,
    weight,
    bias: Optional[torch.Tensor],
    n_modes,
    max_n_modes=None,
    *,
    fft_norm: str = "forward",
    separable: bool = False,
    complex_data: bool = False,
    enforce_hermitian_symmetry: bool = True,
    output_shape=None,
    resolution_scaling_factor=None,
    factorization: Optional[str] = None,
    implementation: str = "reconstructed",
    precision: str = "full",
):
    """Forward of a SpectralConv, op for op.

    ``n_modes`` / ``max_n_modes`` are the *stored* lists (last entry already
    n//2+1 for real data).  ``weight`` is either a dense complex tensor of the
    max_n_modes window, or a dict describing a factorized weight:
    {"tucker": (core, factors)}, {"cp": (weights, factors)}, {"tt": factors}.

    ``precision`` is fno_block_precision (spectral_convolution.py:436-462):
    'half' rounds x to float16 before the transform, 'half' and 'mixed' hold
    the spectrum in complex32 (``fp16_round`` after the forward transform),
    contract through the complex-half einsum and hold out_fft, the
    intermediate of the split inverse and the inverse's output in half
    precision.  The float16 transforms themselves are restated as exact
    transforms rounded once, and only dense (or reconstructed) real-data
    weights are covered.
    """
    half = precision in ("half", "mixed")
    if half and (complex_data or (isinstance(weight, dict) and implementation == "factorized")):
        raise NotImplementedError("half precision: dense / reconstructed real-data weights only")
    if precision == "half":                            # :436-437
        x = fp16_round(x)
    if max_n_modes is None:
        max_n_modes = list(n_modes)
    order = len(n_modes)
    batchsize, channels, *mode_sizes = x.shape
    fft_size = list(mode_sizes)
    if not complex_data:
        fft_size[-1] = fft_size[-1] // 2 + 1          # :431-433
    fft_dims = list(range(-order, 0))                  # :434

    if complex_data:                                   # :439-446
        xf = torch.fft.fftn(x, norm=fft_norm, dim=fft_dims)
        dims_to_fft_shift = fft_dims
    else:
        xf = torch.fft.rfftn(x, norm=fft_norm, dim=fft_dims)
        dims_to_fft_shift = fft_dims[:-1]
    if order > 1:                                      # :448-449
        xf = torch.fft.fftshift(xf, dim=dims_to_fft_shift)
    if half:                                           # :451-454 (and the half rfftn)
        xf = fp16_round(xf)

    cdtype = xf.dtype
    if isinstance(weight, dict):
        out_channels = _factorized_out_channels(weight, separable, channels)
    else:
        out_channels = weight.shape[0] if separable else weight.shape[1]
    out_fft = torch.zeros([batchsize, out_channels, *fft_size], dtype=cdtype)  # :460-462

    sl_w = weight_slices(fft_size, n_modes, max_n_modes, separable, complex_data)
    w_start = 1 if separable else 2
    if isinstance(weight, dict):
        kept = _factorized_window_shape(weight, sl_w, w_start)
    else:
        w = weight[sl_w]                               # :489
        kept = list(w.shape[w_start:])
    sl_x = x_slices(fft_size, kept)                    # :500-519
    xs = xf[sl_x]

    if half and isinstance(weight, dict):              # reconstructed, then dense
        w = _reconstruct_window(weight, sl_w).to(cdtype)
    if half and separable:
        # complex32 x times the complex64 weight promotes to complex64; the
        # store into the complex32 out_fft rounds
        y = fp16_round(contract_dense_separable(xs, w.to(cdtype)))
    elif half:
        y = contract_dense_complexhalf(xs, w.to(cdtype))
    elif isinstance(weight, dict):
        y = _contract_factorized(xs, weight, sl_w, w_start, separable, implementation, cdtype)
    elif separable:
        y = contract_dense_separable(xs, w.to(cdtype))
    else:
        y = contract_dense(xs, w.to(cdtype))
    out_fft[sl_x] = y                                  # :520-522

    if resolution_scaling_factor is not None and output_shape is None:   # :524-525
        mode_sizes = tuple(round(s * r) for (s, r) in zip(mode_sizes, resolution_scaling_factor))
    if output_shape is not None:                       # :527-528
        mode_sizes = output_shape
    mode_sizes = list(mode_sizes)

    if order > 1:                                      # :531-532
        out_fft = torch.fft.ifftshift(out_fft, dim=fft_dims[:-1])

    if complex_data:                                   # :536-538
        out = torch.fft.ifftn(out_fft, s=mode_sizes, dim=fft_dims, norm=fft_norm)
    elif enforce_hermitian_symmetry:                   # :547-559
        if order > 1:
            out_fft = torch.fft.ifftn(out_fft, s=mode_sizes[:-1], dim=fft_dims[:-1], norm=fft_norm)
            if half:
                out_fft = fp16_round(out_fft)
        else:
            # ifftn over zero dims is the identity, but torch still returns a copy
            out_fft = out_fft.clone()
        out_fft[..., 0].imag.zero_()
        if mode_sizes[-1] % 2 == 0:
            out_fft[..., -1].imag.zero_()
        out = torch.fft.irfft(out_fft, n=mode_sizes[-1], dim=fft_dims[-1], norm=fft_norm)
    else:                                              # :564
        out = torch.fft.irfftn(out_fft, s=mode_sizes, dim=fft_dims, norm=fft_norm)
    if half:
        out = fp16_round(out)

    if bias is not None:                               # :567-568
        out = out + bias
    return out


def _factorized_out_channels(weight, separable, channels):
    if separable:
        return channels
    if "tucker" in weight:
        return weight["tucker"][1][1].shape[0]
    if "cp" in weight:
        return weight["cp"][1][1].shape[0]
    return weight["tt"][1].shape[1]


def _slice_factor_list(factors, sl_w):
    return [U[s] for U, s in zip(factors, sl_w)]


def _factorized_window_shape(weight, sl_w, w_start):
    if "tucker" in weight:
        core, factors = weight["tucker"]
        return [U[s].shape[0] for U, s in zip(factors[w_start:], sl_w[w_start:])]
    if "cp" in weight:
        _, factors = weight["cp"]
        return [U[s].shape[0] for U, s in zip(factors[w_start:], sl_w[w_start:])]
    factors = weight["tt"]
    return [G[:, s, :].shape[1] for G, s in zip(factors[w_start:], sl_w[w_start:])]


def _contract_factorized(xs, weight, sl_w, w_start, separable, implementation, cdtype):
    """Slicing a factorized tensor slices the mode factors (tltorch
    FactorizedTensor.__getitem__), then either contracts the factors directly
    ('factorized', spectral_convolution.py:156-169) or reconstructs
    ('reconstructed', :151-155)."""
    if "tucker" in weight:
        core, factors = weight["tucker"]
        fs = [U[s].to(cdtype) for U, s in zip(factors, sl_w)]
        core = core.to(cdtype)
        if implementation == "factorized":
            return contract_tucker(xs, core, fs, separable)
        full = tucker_to_tensor(core, fs)
    elif "cp" in weight:
        w, factors = weight["cp"]
        fs = [U[s].to(cdtype) for U, s in zip(factors, sl_w)]
        w = w.to(cdtype)
        if implementation == "factorized":
            return contract_cp(xs, w, fs, separable)
        full = cp_to_tensor(w, fs)
    else:
        factors = weight["tt"]
        fs = [G[:, s, :].to(cdtype) for G, s in zip(factors, sl_w)]
        if implementation == "factorized":
            return contract_tt(xs, fs, separable)
        full = tt_to_tensor(fs)
    if separable:
        return contract_dense_separable(xs, full)
    return contract_dense(xs, full)


def _reconstruct_window(weight, sl_w):
    """The dense window of a sliced factorized weight (tltorch to_tensor of
    FactorizedTensor.__getitem__, as _contract_factorized's 'reconstructed')."""
    if "tucker" in weight:
        core, factors = weight["tucker"]
        return tucker_to_tensor(core, [U[s] for U, s in zip(factors, sl_w)])
    if "cp" in weight:
        w, factors = weight["cp"]
        return cp_to_tensor(w, [U[s] for U, s in zip(factors, sl_w)])
    return tt_to_tensor([G[:, s, :] for G, s in zip(weight["tt"], sl_w)])


# ---------------------------------------------------------------------------
# skip connections, channel MLP, grid embedding (torch modules restated)
# ---------------------------------------------------------------------------
def gelu(x):
    """Exact erf GELU, torch.nn.functional.gelu default (fno_block.py:118)."""
    return F.gelu(x)


def linear_skip(x, ws):
    """Flattened1dConv with kernel 1, no bias (skip_connections.py:96-130):
    s[b,o,p] = sum_i ws[o,i] x[b,i,p]."""
    size = list(x.shape)
    xf = x.reshape(size[0], size[1], -1)
    out = F.conv1d(xf, ws.reshape(ws.shape[0], ws.shape[1], 1))
    return out.reshape(size[0], ws.shape[0], *size[2:])


def soft_gating(x, w, b=None):
    """SoftGating (skip_connections.py:88-93)."""
    return w * x + b if b is not None else w * x


def bf16_round(t):
    """Round to the nearest bfloat16 (ties to even) and widen back."""
    return t.to(torch.bfloat16).to(t.dtype)


def channel_mlp(x, weights, biases, non_linearity=gelu, bf16_products=False):
    """ChannelMLP.forward (channel_mlp.py:212-249) with 1x1 Conv1d layers.

    bf16_products: each layer's input and weight rounded to bf16 before the
    product, accumulation and bias at full precision.  The reference's mixed
    precision wraps the model in torch.autocast (training/trainer.py:671);
    with dtype=torch.bfloat16, Conv1d takes operands rounded this way.  The
    layer outputs are not rounded here."""
    size = list(x.shape)
    h = x.reshape(size[0], size[1], -1)
    n = len(weights)
    rnd = bf16_round if bf16_products else (lambda t: t)
    for i, (w, b) in enumerate(zip(weights, biases)):
        h = F.conv1d(rnd(h), rnd(w.reshape(w.shape[0], w.shape[1], 1)), b)
        if i < n - 1:
            h = non_linearity(h)
    return h.reshape(size[0], h.shape[1], *size[2:])


def regular_grid_nd(resolutions, grid_boundaries):
    """embeddings.py:351-383: linspace(start, stop, res+1)[:-1] per dim."""
    inputs = [torch.linspace(a, b, r + 1)[:-1] for r, (a, b) in zip(resolutions, grid_boundaries)]
    return tuple(torch.meshgrid(*inputs, indexing="ij"))


def grid_embedding_nd(x, grid_boundaries=None):
    """GridEmbeddingND.forward (embeddings.py:147-164)."""
    dim = x.ndim - 2
    if grid_boundaries is None:
        grid_boundaries = [[0.0, 1.0]] * dim
    grids = regular_grid_nd(list(x.shape[2:]), grid_boundaries)
    grids = [g.to(x.dtype).unsqueeze(0).unsqueeze(0).repeat(x.shape[0], *[1] * (dim + 1)) for g in grids]
    return torch.cat((x, *grids), dim=1)


# ---------------------------------------------------------------------------
# FNO block and FNO forward (fno_block.py:327-381, fno.py:342-408)
# ---------------------------------------------------------------------------
def spectral_block_forward(x, conv: dict, ws, activation=True):
    """The fused block measured by the benchmark: GELU(SpectralConv(x) + Ws x).

    Composed explicitly (not via FNOBlocks(use_channel_mlp=False), which
    applies GELU twice for non-last layers, fno_block.py:359-361,377-379)."""
    y = spectral_conv_forward(x, **conv)
    y = y + linear_skip(x, ws)
    return gelu(y) if activation else y


def cgelu(x):
    """CGELU (layers/complex.py:8-27): GELU on the real and imaginary parts."""
    return torch.complex(gelu(x.real), gelu(x.imag))


def complex_apply(fr, fi, x):
    """apply_complex (layers/complex.py:54-63): the real maps fr, fi as the
    complex-linear map fr + i fi."""
    return torch.complex(fr(x.real) - fi(x.imag), fr(x.imag) + fi(x.real))


def fno_block_forward(x, index, n_layers, conv: dict, fno_skip: Optional[dict], mlp: Optional[dict],
                      mlp_skip: Optional[dict], non_linearity=gelu, output_shape=None,
                      bf16_products=False):
    """FNOBlocks.forward_with_postactivation (fno_block.py:327-381) without
    norms/stabilizer.  ``fno_skip``/``mlp_skip`` are {"type": "linear", "w": ..}
    or {"type": "soft-gating", "w": .., "b": ..} or {"type": "identity"} or None.
    bf16_products: the channel MLP's two 1x1 layers on bf16-rounded operands
    (``channel_mlp``); everything else at full precision."""
    complex_data = conv.get("complex_data", False)

    def apply_skip(s, inp):
        if complex_data and s["type"] != "identity":
            # ComplexValued skip (fno_block.py:226-227): real and imaginary copies
            real = lambda part: (lambda t: real_skip(dict(part, type=s["type"]), t))
            return complex_apply(real(s["fr"]), real(s["fi"]), inp)
        return real_skip(s, inp)

    def real_skip(s, inp):
        if s["type"] == "linear":
            return linear_skip(inp, s["w"])
        if s["type"] == "soft-gating":
            return soft_gating(inp, s["w"], s.get("b"))
        return inp

    def transform(t):
        # SpectralConv.transform (spectral_convolution.py:383-398)
        in_shape = list(t.shape[2:])
        rsf = conv.get("resolution_scaling_factor")
        if rsf is not None and output_shape is None:
            out_shape = [round(s * r) for s, r in zip(in_shape, rsf)]
        elif output_shape is not None:
            out_shape = list(output_shape)
        else:
            out_shape = in_shape
        if in_shape == out_shape:
            return t
        if len(in_shape) == 1:
            return F.interpolate(t, size=out_shape[0], mode="linear", align_corners=True)
        if len(in_shape) == 2:
            return F.interpolate(t, size=out_shape, mode="bicubic", align_corners=True)
        raise NotImplementedError("3D spectral resample is not restated")

    x_skip_fno = transform(apply_skip(fno_skip, x)) if fno_skip is not None else None
    x_skip_mlp = None
    if mlp is not None and mlp_skip is not None:
        x_skip_mlp = transform(apply_skip(mlp_skip, x))
    x_fno = spectral_conv_forward(x, output_shape=output_shape, **conv)
    x = x_fno + x_skip_fno if x_skip_fno is not None else x_fno
    if index < n_layers - 1:
        x = non_linearity(x)
    if mlp is not None:
        if complex_data:
            x = complex_apply(lambda t: channel_mlp(t, mlp["fr"]["weights"], mlp["fr"]["biases"]),
                              lambda t: channel_mlp(t, mlp["fi"]["weights"], mlp["fi"]["biases"]), x)
        else:
            x = channel_mlp(x, mlp["weights"], mlp["biases"], non_linearity,
                            bf16_products=bf16_products)
        if x_skip_mlp is not None:
            x = x + x_skip_mlp
    if index < n_layers - 1:
        x = non_linearity(x)
    return x


def spectral_resample(x, new_size):
    """Spectral resample of 3+ spatial axes (resample.py:54-69): rfftn with
    norm "forward", the first floor(m/2) and last ceil(m/2) entries of every
    non-last axis (m = min(old, new) per axis) and the first min(old, new)//2+1
    bins of the last axis copied to the same offsets from each end of a zero
    spectrum of the new size, irfftn (norm "forward") to new_size."""
    axes = list(range(2, x.ndim))
    X = torch.fft.rfftn(x, dim=axes, norm="forward")
    new_half = list(new_size[:-1]) + [new_size[-1] // 2 + 1]
    Y = X
    for d, ax in enumerate(axes):
        n_old, n_new = Y.shape[ax], new_half[d]
        if d == len(axes) - 1:
            m = min(n_old, n_new)
            src = torch.arange(m)
            dst = src
        else:
            m = min(n_old, n_new)
            lo, hi = m // 2, m - m // 2
            src = torch.cat([torch.arange(lo), torch.arange(n_old - hi, n_old)])
            dst = torch.cat([torch.arange(lo), torch.arange(n_new - hi, n_new)])
        shape = list(Y.shape)
        shape[ax] = n_new
        Z = torch.zeros(shape, dtype=Y.dtype)
        Z.index_copy_(ax, dst, Y.index_select(ax, src))
        Y = Z
    return torch.fft.irfftn(Y, s=list(new_size), dim=axes, norm="forward")


def domain_pad(x, fractions):
    """DomainPadding.pad without resolution scaling (padding.py:54-138):
    round(p * n) zeros on both sides of every spatial axis."""
    pads = [round(p * n) for p, n in zip(fractions, x.shape[2:])]
    flat = []
    for p in reversed(pads):
        flat += [p, p]
    return F.pad(x, flat, mode="constant"), pads


def domain_unpad(x, pads):
    """DomainPadding.unpad (padding.py:140-150)."""
    return x[(Ellipsis,) + tuple(slice(p, -p) if p else slice(None) for p in pads)]


def fno_forward(x, params: dict, bf16_products=False, bf16_storage=False):
    """FNO.forward (fno.py:342-408): grid embedding, lifting, domain padding,
    blocks, unpadding, projection.

    ``params`` = {"lifting": {"weights", "biases"}, "projection": {...},
    "layers": [ {conv, fno_skip, mlp, mlp_skip}, ...], "positional_embedding": bool,
    "domain_padding": per-axis fractions or None}
    bf16_products: the lifting, channel and projection MLPs take bf16-rounded
    operands (``channel_mlp``), as their Conv1d layers do under
    torch.autocast(dtype=bfloat16) (training/trainer.py:669-672); the spectral
    path and the block skips stay at full precision.
    bf16_storage: the activations between the lifting, the layers and the
    projection are held in bfloat16 (``bf16_round`` of the lifting's and each
    layer's output), the storage of the bf16 FNO forward; the lifting output
    is a Conv1d output, bf16 under the reference's autocast as well.
    """
    complex_data = params.get("complex_data", False)

    def mlp(p, t):
        if complex_data:   # ComplexValued lifting / projection (fno.py:327-340)
            return complex_apply(lambda u: channel_mlp(u, p["fr"]["weights"], p["fr"]["biases"]),
                                 lambda u: channel_mlp(u, p["fi"]["weights"], p["fi"]["biases"]), t)
        return channel_mlp(t, p["weights"], p["biases"], bf16_products=bf16_products)

    if params.get("positional_embedding", True):
        x = grid_embedding_nd(x)
    x = mlp(params["lifting"], x)
    if bf16_storage:
        x = bf16_round(x)
    pads = None
    if params.get("domain_padding") is not None:
        x, pads = domain_pad(x, params["domain_padding"])
    n_layers = len(params["layers"])
    for i, layer in enumerate(params["layers"]):
        x = fno_block_forward(x, i, n_layers, layer["conv"], layer.get("fno_skip"),
                              layer.get("mlp"), layer.get("mlp_skip"),
                              non_linearity=cgelu if complex_data else gelu,
                              bf16_products=bf16_products)
        if bf16_storage:
            x = bf16_round(x)
    if pads is not None:
        x = domain_unpad(x, pads)
    return mlp(params["projection"], x)
