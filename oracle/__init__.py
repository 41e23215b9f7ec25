"""Oracle package -- TEST INFRASTRUCTURE ONLY.

CPU restatements of the reference's FP8 W8A8 Mega MoE path (megamoe_oracle.py: torch/numpy;
megamoe_oracle.c: plain C for the integer/byte parts). Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg may import this package, and only as the checker.
"""
import ctypes
import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def build_c_oracle() -> str:
    """Compile megamoe_oracle.c into oracle/liboracle.so (make)."""
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)
    return os.path.join(_HERE, "liboracle.so")


def c_oracle():
    """ctypes handle of liboracle.so (built on first use if missing)."""
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build_c_oracle()
        lib = ctypes.CDLL(path)
        lib.oracle_e4m3_from_f32.restype = ctypes.c_uint8
        lib.oracle_e4m3_from_f32.argtypes = [ctypes.c_float]
        lib.oracle_e4m3_from_f32_array.restype = None
        lib.oracle_e4m3_from_f32_array.argtypes = [ctypes.c_void_p, ctypes.c_void_p,
                                                   ctypes.c_int64]
        lib.oracle_e4m3_to_f32.restype = ctypes.c_float
        lib.oracle_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        lib.oracle_marlin_offset.restype = ctypes.c_int64
        lib.oracle_marlin_offset.argtypes = [ctypes.c_int] * 5
        lib.oracle_route.restype = ctypes.c_int64
        lib.oracle_route.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                     ctypes.c_int, ctypes.c_int] + [ctypes.c_void_p] * 7
        _LIB = lib
    return _LIB
