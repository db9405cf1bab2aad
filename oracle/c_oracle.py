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
        fp = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
        i = ctypes.c_int
        h.oracle_scan_fwd.restype = i
        h.oracle_scan_fwd.argtypes = [i, i, i, i, fp, fp, fp, fp, fp, fp, i, i, i]
        h.oracle_scan_bwd.restype = i
        h.oracle_scan_bwd.argtypes = [i, i, i, i, fp, fp, fp, fp, fp, fp, fp, fp, fp, fp, fp, i, i, i]
        _lib = h
    return _lib


def _f32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def scan_fwd(u, dt, A, B, C, min_recursion_length=2, recursive_split=2, nthreads=0):
    u, dt, A, B, C = map(_f32, (u, dt, A, B, C))
    Bt, L, D = u.shape
    N = A.shape[1]
    y = np.empty((Bt, L, D), np.float32)
    rc = lib().oracle_scan_fwd(Bt, L, D, N, u, dt, A, B, C, y, min_recursion_length, recursive_split, nthreads)
    if rc:
        raise ValueError("oracle_scan_fwd rejected the arguments")
    return y


def scan_bwd(u, dt, A, B, C, dy, min_recursion_length=2, recursive_split=2, nthreads=0):
    u, dt, A, B, C, dy = map(_f32, (u, dt, A, B, C, dy))
    Bt, L, D = u.shape
    N = A.shape[1]
    du = np.empty((Bt, L, D), np.float32)
    ddt = np.empty((Bt, L, D), np.float32)
    dA = np.empty((D, N), np.float32)
    dB = np.empty((Bt, L, N), np.float32)
    dC = np.empty((Bt, L, N), np.float32)
    rc = lib().oracle_scan_bwd(Bt, L, D, N, u, dt, A, B, C, dy, du, ddt, dA, dB, dC, min_recursion_length,
                               recursive_split, nthreads)
    if rc:
        raise ValueError("oracle_scan_bwd rejected the arguments")
    return du, ddt, dA, dB, dC
