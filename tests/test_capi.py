"""The C-ABI library loads here (no GPU) and exports every symbol that
include/fno_hip.h declares; host-side validation returns the documented error
codes without touching a device."""
import ctypes

import pytest

from neuraloperator_amd import _native as nat


def test_header_declares_expected_entry_points():
    syms = nat.header_symbols()
    for s in ["fno_rfft_window_f32", "fno_contract_dense_c64", "fno_contract_tucker_c64",
              "fno_irfft_window_f32", "fno_block_epilogue_f32", "fno_spectral_block_f32",
              "fno_spectral_block_workspace_bytes", "fno_last_error"]:
        assert s in syms


def test_library_exports_every_header_symbol():
    lib = ctypes.CDLL(str(nat.LIB_PATH))
    missing = [s for s in nat.header_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_validation_errors_without_device():
    lib = nat.load()
    sz, md = nat.i32_array([8, 8]), nat.i32_array([4, 5])
    rc = lib.fno_rfft_window_f32(None, None, 1, 2, sz, md, 1, None, 0, None)
    assert rc == 1 and "NULL" in nat.last_error()
    bad_modes = nat.i32_array([4, 6])          # 6 > 8//2+1
    rc = lib.fno_rfft_window_f32(ctypes.c_void_p(16), ctypes.c_void_p(16), 1, 2, sz, bad_modes, 1,
                                 None, 0, None)
    assert rc == 1 and "modes[1]" in nat.last_error()
    rc = lib.fno_spectral_block_f32(ctypes.c_void_p(16), ctypes.c_void_p(16), None, None,
                                    ctypes.c_void_p(16), 1, 3, 4, 2, sz, md, 1, 3, 0, None, 0, None)
    assert rc == 1 and "in_channels == out_channels" in nat.last_error()
    big = nat.i32_array([8192, 8])
    rc = lib.fno_rfft_window_f32(ctypes.c_void_p(16), ctypes.c_void_p(16), 1, 2, big,
                                 nat.i32_array([4, 4]), 1, None, 0, None)
    assert rc == 2


def test_workspace_and_fused_queries():
    lib = nat.load()
    sz, md = nat.i32_array([256, 256]), nat.i32_array([64, 33])
    assert lib.fno_spectral_block_is_fused(32, 64, 64, 2, sz, md, 1) == 1
    ws = lib.fno_spectral_block_workspace_bytes(32, 64, 64, 2, sz, md)
    # xhat + yhat (B*C*M each) + Z (B*Co*H*m2h), complex64
    assert ws == (32 * 64 * 64 * 33 * 2 + 32 * 64 * 256 * 33) * 8
    odd = nat.i32_array([9, 10])
    assert lib.fno_spectral_block_is_fused(2, 3, 4, 2, odd, nat.i32_array([4, 3]), 1) == 0
