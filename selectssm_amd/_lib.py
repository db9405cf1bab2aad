"""ctypes binding of the C ABI declared in ``include/selectssm.h``.

The shared library is built in-tree (``selectssm_amd/libselectssm.so``).  There
is no fallback: if the library is missing or fails to load, every op raises.
"""
from __future__ import annotations

import ctypes
import os

from .build import LIB

SSM_OK = 0
SSM_ERR_INVALID = 1
SSM_ERR_UNSUPPORTED = 2
SSM_ERR_HIP = 3

SSM_F32 = 0
SSM_BF16 = 1

SSM_REVERSE = 1
SSM_COMPLEMENT = 2
SSM_SKIP = 4
SSM_GATE = 8
SSM_DELTA_SOFTPLUS = 16
SSM_SKIP_MAP = 32
SSM_SKIP_REVERSE = 64
SSM_SKIP_COMPLEMENT = 128
SSM_ACCUMULATE = 256

SSM_ACT_NONE = 0
SSM_ACT_SILU = 1
SSM_ACT_RELU = 2

ABI_VERSION = 9

STATIC_SCRATCH_BYTES = 64 << 20  # SSM_STATIC_SCRATCH_BYTES: ssm_bwd_static's workspace

# every symbol include/selectssm.h declares
EXPORTS = (
    "ssm_abi_version",
    "ssm_last_error",
    "ssm_ckpt_bytes",
    "ssm_fwd_workspace_bytes",
    "ssm_bwd_workspace_bytes",
    "ssm_fwd",
    "ssm_bwd",
    "ssm_bwd_static",
    "ssm_fwd_pair",
    "ssm_bwd_pair",
    "ssm_conv_bwd_workspace_bytes",
    "ssm_conv_fwd",
    "ssm_conv_bwd",
)


class SsmDesc(ctypes.Structure):
    """Mirror of ``ssm_desc_t``."""

    _fields_ = [
        ("batch", ctypes.c_int64),
        ("seqlen", ctypes.c_int64),
        ("dim", ctypes.c_int64),
        ("dstate", ctypes.c_int64),
        ("dtype", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
        ("delta_broadcast", ctypes.c_int32),
        ("segments", ctypes.c_int32),
        ("ld_y", ctypes.c_int64),
        ("ld_z", ctypes.c_int64),
        ("ld_bc", ctypes.c_int64),
    ]


_vp = ctypes.c_void_p


class SsmFwdIo(ctypes.Structure):
    """Mirror of ``ssm_fwd_io_t``."""

    _fields_ = [(n, _vp) for n in ("u", "delta", "A", "B", "C", "D", "z", "y", "ckpt", "workspace")]


class SsmBwdIo(ctypes.Structure):
    """Mirror of ``ssm_bwd_io_t``."""

    _fields_ = [(n, _vp) for n in ("u", "delta", "A", "B", "C", "D", "z", "ckpt", "dy", "du", "ddelta", "dA", "dB",
                                   "dC", "dD", "dz", "workspace")]


class SsmConvDesc(ctypes.Structure):
    """Mirror of ``ssm_conv_desc_t``."""

    _fields_ = [
        ("batch", ctypes.c_int64),
        ("seqlen", ctypes.c_int64),
        ("dim", ctypes.c_int64),
        ("ksize", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
        ("activation", ctypes.c_int32),
        ("ld_x", ctypes.c_int64),
    ]


class SsmError(RuntimeError):
    """A nonzero return code from the library, with its ssm_last_error() text."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"selectssm error {code}: {msg}")
        self.code = code


_lib = None


def _declare(lib):
    vp = ctypes.c_void_p
    fp = ctypes.c_void_p
    dp = ctypes.POINTER(SsmDesc)
    lib.ssm_abi_version.restype = ctypes.c_int
    lib.ssm_abi_version.argtypes = []
    lib.ssm_last_error.restype = ctypes.c_char_p
    lib.ssm_last_error.argtypes = []
    lib.ssm_ckpt_bytes.restype = ctypes.c_size_t
    lib.ssm_ckpt_bytes.argtypes = [dp]
    lib.ssm_fwd_workspace_bytes.restype = ctypes.c_size_t
    lib.ssm_fwd_workspace_bytes.argtypes = [dp]
    lib.ssm_bwd_workspace_bytes.restype = ctypes.c_size_t
    lib.ssm_bwd_workspace_bytes.argtypes = [dp]
    lib.ssm_fwd.restype = ctypes.c_int
    lib.ssm_fwd.argtypes = [vp, dp, vp, vp, fp, vp, vp, fp, vp, vp, fp, vp]
    lib.ssm_bwd.restype = ctypes.c_int
    lib.ssm_bwd.argtypes = [vp, dp, vp, vp, fp, vp, vp, fp, vp, fp, vp, vp, vp, fp, vp, vp, fp, vp, vp]
    lib.ssm_bwd_static.restype = ctypes.c_int
    lib.ssm_bwd_static.argtypes = [vp, dp, vp, vp, fp, vp, vp, fp, vp, fp, vp, vp, vp, fp, vp, vp, fp, vp]
    lib.ssm_fwd_pair.restype = ctypes.c_int
    lib.ssm_fwd_pair.argtypes = [vp, dp, ctypes.POINTER(SsmFwdIo)]
    lib.ssm_bwd_pair.restype = ctypes.c_int
    lib.ssm_bwd_pair.argtypes = [vp, dp, ctypes.POINTER(SsmBwdIo)]
    cp = ctypes.POINTER(SsmConvDesc)
    lib.ssm_conv_bwd_workspace_bytes.restype = ctypes.c_size_t
    lib.ssm_conv_bwd_workspace_bytes.argtypes = [cp]
    lib.ssm_conv_fwd.restype = ctypes.c_int
    lib.ssm_conv_fwd.argtypes = [vp, cp, vp, fp, vp]
    lib.ssm_conv_bwd.restype = ctypes.c_int
    lib.ssm_conv_bwd.argtypes = [vp, cp, vp, fp, vp, vp, fp, vp]


def lib():
    """The loaded library (loaded on first use).  Raises if it cannot load."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise RuntimeError(
                f"{LIB} is missing: build it with `python -m selectssm_amd.build` "
                "(there is no CPU fallback for the selective scan)")
        handle = ctypes.CDLL(LIB)
        _declare(handle)
        got = handle.ssm_abi_version()
        if got != ABI_VERSION:
            raise RuntimeError(f"{LIB} has ABI version {got}, expected {ABI_VERSION}")
        _lib = handle
    return _lib


def check(code: int) -> None:
    if code != SSM_OK:
        raise SsmError(code, lib().ssm_last_error().decode())


def make_desc(batch, seqlen, dim, dstate, dtype=SSM_F32, flags=0, delta_broadcast=False, segments=0,
              ld_y=0, ld_z=0, ld_bc=0) -> SsmDesc:
    return SsmDesc(int(batch), int(seqlen), int(dim), int(dstate), int(dtype), int(flags),
                   1 if delta_broadcast else 0, int(segments), int(ld_y), int(ld_z), int(ld_bc))


def size_query(fn, desc, allow_zero=False) -> int:
    """Call a ``ssm_*_bytes`` query; a 0 with an error message set is an invalid desc."""
    n = fn(ctypes.byref(desc))
    if n == 0:
        msg = lib().ssm_last_error().decode()
        if msg or not allow_zero:
            raise SsmError(SSM_ERR_INVALID, msg or "size query returned 0")
    return n
