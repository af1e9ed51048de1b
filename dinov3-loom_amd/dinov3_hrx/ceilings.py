"""Binding of the machine-ceiling probes (include/dinov3_probe.h), built into
their own library, lib/libdinov3_probe.so, apart from the forward pass's
libdinov3_hrx.so. Measurement tooling for bench.py and the tests: one wave per
SIMD running 32x32x16 f16 MFMAs alone, beside VALU or exp2 work, beside buffer
loads from L1-, L2- or HBM-sized footprints, or on a number of independent
accumulators."""
from __future__ import annotations

import ctypes
import os

from . import DINOv3Error

PROBE_LIB_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "lib",
                              "libdinov3_probe.so")

PROBE_KINDS = {"mfma_random": 0, "mfma_zeros": 1, "valu": 2, "exp2": 3, "loads_l1": 4, "loads_l2": 5,
               "loads_hbm": 6, "chains": 7}

_lib = None


def _load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(PROBE_LIB_PATH):
            raise ImportError(f"{PROBE_LIB_PATH} is not built; run `python dinov3-loom_amd/build.py` first")
        lib = ctypes.CDLL(PROBE_LIB_PATH)
        lib.dhx_probe.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.POINTER(ctypes.c_double)]
        _lib = lib
    return _lib


def probe(kind: str, param: int = 0, device: int = 0) -> dict:
    """dhx_probe: one wave per SIMD running 32x32x16 f16 MFMAs alone or beside
    `param` VALU FMAs / exp2 per MFMA or `param` buffer loads per 8 MFMAs,
    or ("chains") on `param` independent accumulators. Returns cycles per 8
    MFMAs of a wave, TFLOP/s over the GPU and the clock they imply (GHz)."""
    out = (ctypes.c_double * 3)()
    rc = _load().dhx_probe(int(device), PROBE_KINDS[kind], int(param), out)
    if rc == 2:
        raise DINOv3Error(f"unsupported probe {kind} with param {param}")
    if rc != 0:
        raise DINOv3Error(f"probe {kind} failed (HIP error)")
    return {"cycles_per_8_mfma": out[0], "tflops": out[1], "clock_ghz": out[2]}
