"""Checkpoint round trip: state_dict save -> load (weights_only, nothing
executed from the file) -> identical parameters and, on the GPU, bitwise
identical outputs; plus run-to-run determinism of the forward.  The
reference's Trainer saves and restores model state_dicts
(neuralop/training/training_state.py:14-158); the SpectralConv weight is a
(possibly factorized) parameter set whose state_dict entries must survive the
trip."""
import io

import pytest
import torch

import neuraloperator_amd as na

MODELS = [
    ("fno_dense_2d", lambda: na.FNO((8, 8), in_channels=2, out_channels=1, hidden_channels=8,
                                    n_layers=2)),
    ("tfno_tucker_2d", lambda: na.TFNO((8, 8), in_channels=2, out_channels=1, hidden_channels=8,
                                       n_layers=2, factorization="tucker", rank=0.5)),
    ("tfno_cp_3d", lambda: na.FNO((4, 4, 4), in_channels=2, out_channels=1, hidden_channels=8,
                                  n_layers=2, factorization="cp", rank=0.5)),
    ("fno_separable_1d", lambda: na.FNO((12,), in_channels=2, out_channels=1, hidden_channels=8,
                                        n_layers=2, separable=True)),
]


def _round_trip(model, make):
    buf = io.BytesIO()
    torch.save(model.state_dict(), buf)
    buf.seek(0)
    sd = torch.load(buf, weights_only=True)
    torch.manual_seed(12345)             # a different initialisation
    fresh = make()
    fresh.load_state_dict(sd)
    return fresh


@pytest.mark.parametrize("name,make", MODELS, ids=[m[0] for m in MODELS])
def test_state_dict_round_trip(name, make):
    torch.manual_seed(0)
    model = make()
    fresh = _round_trip(model, make)
    a, b = model.state_dict(), fresh.state_dict()
    assert list(a) == list(b)
    for k in a:
        assert a[k].dtype == b[k].dtype and a[k].shape == b[k].shape, k
        assert torch.equal(a[k], b[k]), k
    # and the fresh initialisation did differ before loading
    torch.manual_seed(12345)
    other = make().state_dict()
    assert any(not torch.equal(a[k], other[k]) for k in a if a[k].is_floating_point() or
               a[k].is_complex())


@pytest.mark.gpu
@pytest.mark.parametrize("name,make", MODELS, ids=[m[0] for m in MODELS])
def test_round_trip_outputs_bitwise(name, make, cuda_device):
    print(f"checkpoint round trip {name}", flush=True)
    torch.manual_seed(0)
    model = make().to(cuda_device)
    dims = len(model.n_modes)
    x = torch.randn(2, 2, *([16] * dims), device=cuda_device)
    with torch.no_grad():
        y0 = model(x)
        y1 = model(x)
    assert torch.equal(y0, y1)            # the forward is deterministic
    fresh = _round_trip(model.cpu(), make).to(cuda_device)
    model.to(cuda_device)
    with torch.no_grad():
        y2 = fresh(x)
    torch.cuda.synchronize()
    assert torch.equal(y0, y2)
