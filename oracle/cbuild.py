"""Build oracle/libcref.so from oracle/cref.c (gcc, OpenMP) — TEST INFRASTRUCTURE ONLY.

The C restatement is the timed CPU baseline of bench.py.  The reference's own
native code cannot be built here (native/cuda/*.cu needs nvcc; the NIF
c_src/edifice_cuda_nif.c needs erl_nif.h), so there is no oracle/_ref build.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "cref.c")
LIB = os.path.join(HERE, "libcref.so")


def build(verbose: bool = False) -> str:
    tmp = LIB + ".tmp"
    cmd = ["gcc", "-O3", "-march=x86-64-v3", "-fopenmp", "-fPIC", "-shared", "-o", tmp, SRC, "-lm"]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


_LIB = None


def lib():
    """Load the C restatement (building it first if it is missing)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB):
            build()
        _LIB = ctypes.CDLL(LIB)
    return _LIB
