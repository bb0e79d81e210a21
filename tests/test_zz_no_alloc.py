"""The no-allocation spectral block (fno_spectral_block_f32_noalloc) through
the C ABI against the workspace entry point (fno_spectral_block_f32) on the
same inputs: two calls in a row, the second on a smaller input, so the
second call runs on scratch the first one left behind."""
import ctypes

import pytest
import torch

from neuraloperator_amd import _native as nat

pytestmark = pytest.mark.gpu

SCRATCH = 64 << 20


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _inputs(B, C, sizes, modes, seed, dev):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, C, *sizes, generator=g)
    w = torch.complex(torch.randn(C, C, *modes, generator=g), torch.randn(C, C, *modes, generator=g))
    w = w / C
    ws = torch.randn(C, C, generator=g) / C ** 0.5
    bias = torch.randn(C, generator=g) / 8
    return [t.to(dev) for t in (x, w, ws, bias)]


def _run_both(B, C, sizes, modes, seed, dev, skip=nat.SKIP_LINEAR):
    lib = nat.load()
    x, w, ws, bias = _inputs(B, C, sizes, modes, seed, dev)
    nd = len(sizes)
    sz, md = nat.i32_array(sizes), nat.i32_array(modes)
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    wsb = lib.fno_spectral_block_workspace_bytes(B, C, C, nd, sz, md)
    work = torch.empty(wsb, dtype=torch.uint8, device=dev)
    y_ref = torch.empty_like(x)
    y = torch.full_like(x, float("nan"))
    nat.check(lib.fno_spectral_block_f32(_ptr(x), _ptr(w), _ptr(bias), _ptr(ws), _ptr(y_ref), B, C,
                                         C, nd, sz, md, 1, skip, nat.ACT_GELU,
                                         _ptr(work), wsb, st), "fno_spectral_block_f32")
    nat.check(lib.fno_spectral_block_f32_noalloc(_ptr(x), _ptr(w), _ptr(bias), _ptr(ws), _ptr(y), B,
                                                 C, C, nd, sz, md, 1, skip,
                                                 nat.ACT_GELU, st),
              "fno_spectral_block_f32_noalloc")
    torch.cuda.synchronize()
    return y, y_ref, wsb


@pytest.mark.parametrize("first,second", [
    # fused 2D path: 32 samples (2.2 MB of window spectra each) need two
    # chunks of the 64 MiB array, then a smaller call on another shape
    ((32, 64, (256, 256), (64, 33)), (3, 32, (64, 128), (16, 9))),
    # generic 3D path: 4 samples of 64^3 need two chunks, then a smaller 1D call
    ((4, 32, (64, 64, 64), (16, 16, 9)), (2, 16, (256,), (20,))),
])
def test_noalloc_matches_workspace_entry_point(first, second, cuda_device):
    for i, (B, C, sizes, modes) in enumerate((first, second)):
        print(f"noalloc call {i}: B{B} C{C} {sizes} modes {modes}", flush=True)
        y, y_ref, wsb = _run_both(B, C, sizes, modes, 100 + i, cuda_device)
        if i == 0:
            assert wsb > SCRATCH, "the first call should span several chunks"
        assert torch.isfinite(y).all()
        err = ((y - y_ref).abs().max() / y_ref.abs().max()).item()
        assert err <= 1e-6, err


@pytest.mark.parametrize("skip", [nat.SKIP_IDENTITY, nat.SKIP_NONE, nat.SKIP_SOFT_GATING])
def test_noalloc_1d_line_path(skip, cuda_device):
    """The 1D block without a linear skip (one DFT wave per line, then the
    contraction and synthesis per 4 output channels, the spectra passing
    through the scratch array): 16 x 64 lines of 1024 points with 16 bins,
    then 3 x 32 lines of 256 points with 9 bins."""
    for i, (B, C, sizes, modes) in enumerate(((16, 64, (1024,), (16,)), (3, 32, (256,), (9,)))):
        print(f"noalloc 1d call {i}: B{B} C{C} {sizes} modes {modes} skip {skip}", flush=True)
        y, y_ref, _ = _run_both(B, C, sizes, modes, 200 + i, cuda_device, skip)
        assert torch.isfinite(y).all()
        err = ((y - y_ref).abs().max() / y_ref.abs().max()).item()
        assert err <= 1e-6, err
