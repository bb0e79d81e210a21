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
  tucker_rank_from_fraction -> parity unpinned (restates tensorly 0.9.0's
    rank rule; tensorly is not importable here, and no reference test pins
    the resulting tuple).
"""
