"""valu_probe.py -- ctypes binding of libxtqprobe.so (probe/valu_probe.hip), the
VALU issue-rate probe the benchmark uses to state the forward DP's
instruction-mix ceiling on the GPU it runs on.  A measurement helper: the
encoder library (libexl3vit.so) and its C-ABI do not include it.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.normpath(os.path.join(_HERE, "..", "lib", "libxtqprobe.so"))

PROBES = ("v_mul_f32", "v_add_f32", "v_fma_f32", "v_fma_mix_f32", "v_min_f64",
          "candidate mix, dependency order", "candidate mix, grouped by opcode",
          "fp32-code candidate mix, dependency order",
          "fp32-code candidate mix, grouped by opcode", "v_min3_f32",
          "deferred-argmin mix (3.5 instructions per candidate), grouped by opcode",
          "fp32-code candidate mix, grouped by opcode, one workgroup per CU",
          "deferred-argmin mix (3.5 instructions per candidate), grouped by opcode, "
          "one workgroup per CU")

_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libxtqprobe.so not found at {LIB_PATH}; build it with "
                               "`make -C exl3xpu-mixedk_amd`")
        L = ctypes.CDLL(LIB_PATH)
        L.xtq_valu_probe.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
        L.xtq_valu_probe.restype = ctypes.c_int
        _LIB = L
    return _LIB


def rate(which: int) -> float:
    """VALU lane-instructions/s of probe `which` (index into PROBES) on the
    current HIP device."""
    v = ctypes.c_double()
    rc = lib().xtq_valu_probe(int(which), ctypes.byref(v))
    if rc:
        raise RuntimeError(f"xtq_valu_probe({which}) rc={rc}")
    return v.value
