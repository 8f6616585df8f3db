"""ctypes binding of the measurement-aid library ``libflat_diag.so`` (``include/flat_diag.h``):
the practical MFMA and streaming-read ceilings that ``bench.py --ceilings`` prints. Not imported
by the package; the attention library carries none of it."""

from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libflat_diag.so")
DTYPE_F32, DTYPE_BF16 = 0, 2
_lib = None


class DiagError(RuntimeError):
    pass


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise DiagError(f"{LIB_PATH} is not built (make -C flat-attention_amd)")
        _lib = ctypes.CDLL(LIB_PATH)
        d = ctypes.POINTER(ctypes.c_double)
        _lib.fad_mfma_ceiling.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, d]
        _lib.fad_stream_read.argtypes = [ctypes.c_int32, ctypes.c_int32, d]
    return _lib


def _check(rc: int, what: str):
    if rc != 0:
        raise DiagError(f"{what} failed with status {rc}")


def mfma_ceiling(device: int = 0, constant_operands: bool = False, dtype: int = DTYPE_BF16) -> float:
    """TFLOP/s of a pure MFMA stream (bf16 32x32x16 or f32 32x32x2; random or constant
    operands), measured after the clock settles (~1.5 s)."""
    out = ctypes.c_double()
    _check(lib().fad_mfma_ceiling(device, dtype, int(constant_operands), ctypes.byref(out)),
           "fad_mfma_ceiling")
    return out.value


def stream_read(device: int = 0, loads_in_flight: int = 8) -> float:
    """TB/s of non-temporal 16-byte streaming reads of a 4 GiB buffer."""
    out = ctypes.c_double()
    _check(lib().fad_stream_read(device, loads_in_flight, ctypes.byref(out)), "fad_stream_read")
    return out.value
