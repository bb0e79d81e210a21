"""ctypes binding of libfnohip.so (the gfx950 HIP library).

The library is built in-tree (``python -m neuraloperator_amd.build``); this
module loads it on first use and raises if it is missing -- there is no
fallback implementation.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

_PKG = Path(__file__).resolve().parent
LIB_PATH = _PKG / "libfnohip.so"
HEADER_PATH = _PKG.parent / "include" / "fno_hip.h"

FNO_OK = 0
NORMS = {"backward": 0, "forward": 1, "ortho": 2}
SKIP_NONE, SKIP_LINEAR, SKIP_SOFT_GATING, SKIP_IDENTITY = 0, 1, 2, 3
ACT_NONE, ACT_GELU = 0, 1

_c_i32 = ctypes.c_int32
_c_i64 = ctypes.c_int64
_c_size = ctypes.c_size_t
_c_vp = ctypes.c_void_p
_c_i32p = ctypes.POINTER(ctypes.c_int32)

_SIGNATURES = {
    "fno_version": (ctypes.c_char_p, []),
    "fno_last_error": (ctypes.c_char_p, []),
    "fno_rfft_window_f32": (_c_i32, [_c_vp, _c_vp, _c_i64, _c_i32, _c_i32p, _c_i32p, _c_i32, _c_vp,
                                     _c_size, _c_vp]),
    "fno_rfft_window_workspace_bytes": (_c_size, [_c_i64, _c_i32, _c_i32p, _c_i32p]),
    "fno_contract_dense_c64": (_c_i32, [_c_vp, _c_vp, _c_vp, _c_i32, _c_i32, _c_i32, _c_i64, _c_i32,
                                        _c_vp]),
    "fno_contract_tucker_c64": (_c_i32, [_c_vp, _c_vp, ctypes.POINTER(_c_vp), _c_i32p, _c_vp,
                                         _c_i32, _c_i32, _c_i32, _c_i32, _c_i32p, _c_vp, _c_size,
                                         _c_vp]),
    "fno_contract_tucker_workspace_bytes": (_c_size, [_c_i32, _c_i32, _c_i32p, _c_i32p]),
    "fno_irfft_window_f32": (_c_i32, [_c_vp, _c_vp, _c_vp, _c_i64, _c_i32, _c_i32, _c_i32p, _c_i32p,
                                      _c_i32p, _c_i32, _c_i32, _c_vp, _c_size, _c_vp]),
    "fno_irfft_window_workspace_bytes": (_c_size, [_c_i64, _c_i32, _c_i32p, _c_i32p]),
    "fno_block_epilogue_f32": (_c_i32, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i32, _c_i32, _c_i32, _c_i64,
                                        _c_i32, _c_i32, _c_vp]),
    "fno_spectral_block_f32": (_c_i32, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i32, _c_i32, _c_i32,
                                        _c_i32, _c_i32p, _c_i32p, _c_i32, _c_i32, _c_i32, _c_vp,
                                        _c_size, _c_vp]),
    "fno_spectral_block_workspace_bytes": (_c_size, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32p,
                                                     _c_i32p]),
    "fno_spectral_block_is_fused": (_c_i32, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32p, _c_i32p,
                                             _c_i32]),
    "fno_spectral_block_f32_noalloc": (_c_i32, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i32, _c_i32,
                                                _c_i32, _c_i32, _c_i32p, _c_i32p, _c_i32, _c_i32,
                                                _c_i32, _c_vp]),
    "fno_channel_mlp_f32": (_c_i32, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                     _c_i64, _c_i32, _c_i32, _c_i32, _c_i64, _c_i32, _c_i32, _c_i32,
                                     _c_vp]),
    "fno_channel_mlp_is_supported": (_c_i32, [_c_i32, _c_i32, _c_i32, _c_i64]),
    "fno_channel_mlp_io": (_c_i32, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i32, _c_i32,
                                    _c_i32, _c_i64, _c_i32, _c_i32, _c_i32, _c_vp]),
    "fno_channel_mlp_io_is_supported": (_c_i32, [_c_i32, _c_i32, _c_i32, _c_i64, _c_i32, _c_i32]),
    "fno_irfft_window_epilogue_f32": (_c_i32, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i32, _c_i32,
                                               _c_i32, _c_i32, _c_i32p, _c_i32p, _c_i32, _c_i32,
                                               _c_i32, _c_vp, _c_size, _c_vp]),
    "fno_layer_is_fused": (_c_i32, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32p, _c_i32p, _c_i32,
                                    _c_i32]),
    "fno_layer_bf16_is_fused": (_c_i32, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32p, _c_i32p, _c_i32,
                                         _c_i32]),
    "fno_layer_f32": (_c_i32, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                               _c_vp, _c_vp, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32p, _c_i32p,
                               _c_i32, _c_i32, _c_i32, _c_i32, _c_vp, _c_size, _c_vp]),
    "fno_layer_bf16": (_c_i32, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                               _c_vp, _c_vp, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32p, _c_i32p,
                               _c_i32, _c_i32, _c_i32, _c_i32, _c_vp, _c_size, _c_vp]),
    "fno_fft_window_c64": (_c_i32, [_c_vp, _c_vp, _c_i64, _c_i32, _c_i32p, _c_i32p, _c_i32, _c_vp,
                                    _c_size, _c_vp]),
    "fno_fft_window_workspace_bytes": (_c_size, [_c_i64, _c_i32, _c_i32p, _c_i32p]),
    "fno_ifft_window_c64": (_c_i32, [_c_vp, _c_vp, _c_vp, _c_i64, _c_i32, _c_i32, _c_i32p, _c_i32p,
                                     _c_i32p, _c_i32, _c_vp, _c_size, _c_vp]),
    "fno_ifft_window_workspace_bytes": (_c_size, [_c_i64, _c_i32, _c_i32p, _c_i32p]),
}

_lib = None


def header_symbols():
    """Function names declared in include/fno_hip.h."""
    text = HEADER_PATH.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(fno_\w+)\s*\(", text, re.M)))


def load():
    """Load libfnohip.so (once).  Raises RuntimeError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m neuraloperator_amd.build` "
            "(the FNO spectral path has no fallback)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def i32_array(values):
    values = [int(v) for v in values]
    return (ctypes.c_int32 * max(1, len(values)))(*values)


def last_error() -> str:
    msg = load().fno_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str):
    if rc != FNO_OK:
        raise RuntimeError(f"{what} failed (code {rc}): {last_error()}")
