"""Oracle for the FNO spectral path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the reference results are
compared against (or, for the CPU baseline, as the thing timed on the host).  The product path in
``neuraloperator_amd`` never imports it: the GPU modules fail loudly when the
HIP library is missing instead of falling back to anything in here.

Contents
--------
``spectral_ref``   plain-torch CPU restatement of the reference op sequence
                   (rfftn -> fftshift -> window -> einsum -> ifftshift ->
                   ifftn -> Hermitian fix-up -> irfft -> bias), the FNO block
                   composition and the FNO forward, each function citing the
                   reference file:line it follows.
``dft64``          independent float64 formulation of the same mathematics
                   from the DFT closed form (explicit exponentials, frequency
                   of window index stated as a formula, no fftshift/slicing
                   bookkeeping).  It pins ``spectral_ref``.

Pinning status (what checks each function; see tests/test_oracle.py):
  spectral_conv_forward (dense, 1-3D, even/odd sizes, n_modes < max_n_modes,
    output_shape / resolution scaling, all fft_norm values, separable,
    enforce_hermitian_symmetry on/off)  -> dft64 at float64, plane-wave known
    answers, circular-shift equivariance, linearity.
  tucker / cp / tt factorized contraction -> equality with the dense
    contraction on the reconstructed weight (the reference's own invariant,
    neuralop/layers/tests/test_spectral_convolution.py:53-65).
  gelu -> closed-form erf values.
  fno_block_forward / fno_forward -> composition of pinned pieces plus
    GridEmbeddingND coordinates checked against the linspace(0,1,N+1)[:-1]
    closed form.
  spectral_conv_forward(complex_data=True) -> closed-form plane waves that
    fix the last-axis window of the reference (frequency j - N/2 forward,
    put back at j by the inverse).
  domain_pad / domain_unpad -> round-trip identity and the padded sizes
    round(p * n) on both sides.
  cgelu / complex_apply -> GELU of each part; the complex matrix (A + iB) x.
  channel_mlp(bf16_products=True) / bf16_round -> ties-to-even closed forms
    (1 + 2^-8 -> 1, 1 + 3 * 2^-8 -> 1 + 2^-6, the hidden GELU rounded) and
    bf16-exact operands, where the rounding must change nothing.
  spectral_resample -> band-limited plane waves resampled exactly, and the
    odd-grid residue rule of the reference's slices (-k-1 .. k-1).

Not in the oracle: the float-rank -> Tucker-rank rule of tensorly 0.9.0.  The
tests pass explicit rank tuples (the 3D TFNO workload records (20, 20, 10, 10,
6)), and the product's own restatement of the rule is pinned in
tests/test_host.py by closed forms of its parameter-count equation.
"""
