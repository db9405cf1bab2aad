"""ctypes wrapper of ``oracle/libssm_oracle.so`` (built by ``oracle/Makefile``).

TEST INFRASTRUCTURE ONLY (tests/ and bench.py's cpu_baseline leg).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libssm_oracle.so")

_lib = None


def build() -> str:
    subprocess.run(["make", "-B", "-C", HERE, "libssm_oracle.so"], check=True, capture_output=True)
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        h = ctypes.CDLL(LIB)
        i = ctypes.c_int
        for sfx, dt in (("", np.float32), ("_f64", np.float64)):
            fp = np.ctypeslib.ndpointer(dtype=dt, flags="C_CONTIGUOUS")
            f = getattr(h, "oracle_scan_fwd" + sfx)
            f.restype = i
            f.argtypes = [i, i, i, i, fp, fp, fp, fp, fp, fp, i, i, i]
            g = getattr(h, "oracle_scan_bwd" + sfx)
            g.restype = i
            g.argtypes = [i, i, i, i, fp, fp, fp, fp, fp, fp, fp, fp, fp, fp, fp, i, i, i]
        _lib = h
    return _lib


_PREC = {"f32": ("", np.float32), "f64": ("_f64", np.float64)}


def scan_fwd(u, dt, A, B, C, min_recursion_length=2, recursive_split=2, nthreads=0, precision="f32"):
    """y of the reference's recursive custom-VJP forward, in float32 or float64."""
    sfx, dtype = _PREC[precision]
    u, dt, A, B, C = (np.ascontiguousarray(x, dtype=dtype) for x in (u, dt, A, B, C))
    Bt, L, D = u.shape
    N = A.shape[1]
    y = np.empty((Bt, L, D), dtype)
    rc = getattr(lib(), "oracle_scan_fwd" + sfx)(Bt, L, D, N, u, dt, A, B, C, y, min_recursion_length,
                                                 recursive_split, nthreads)
    if rc:
        raise ValueError("oracle_scan_fwd rejected the arguments")
    return y


def scan_bwd(u, dt, A, B, C, dy, min_recursion_length=2, recursive_split=2, nthreads=0, precision="f32"):
    """(du, ddt, dA, dB, dC) of the reference's custom-VJP backward, in float32 or float64."""
    sfx, dtype = _PREC[precision]
    u, dt, A, B, C, dy = (np.ascontiguousarray(x, dtype=dtype) for x in (u, dt, A, B, C, dy))
    Bt, L, D = u.shape
    N = A.shape[1]
    du = np.empty((Bt, L, D), dtype)
    ddt = np.empty((Bt, L, D), dtype)
    dA = np.empty((D, N), dtype)
    dB = np.empty((Bt, L, N), dtype)
    dC = np.empty((Bt, L, N), dtype)
    rc = getattr(lib(), "oracle_scan_bwd" + sfx)(Bt, L, D, N, u, dt, A, B, C, dy, du, ddt, dA, dB, dC,
                                                 min_recursion_length, recursive_split, nthreads)
    if rc:
        raise ValueError("oracle_scan_bwd rejected the arguments")
    return du, ddt, dA, dB, dC
