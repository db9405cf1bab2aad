"""The C ABI library loads, exports every function include/selectssm.h declares and
rejects invalid requests with error codes (no GPU work is launched here)."""
import ctypes
import os
import re

import pytest

from selectssm_amd import _lib as L

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "selectssm.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ssm_\w+)\s*\(", text)))


def test_header_declares_the_bound_symbols():
    assert header_functions() == sorted(L.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = L.lib()
    for name in header_functions():
        assert hasattr(lib, name), name
    assert lib.ssm_abi_version() == L.ABI_VERSION


def test_header_constants_match_binding():
    text = open(HEADER).read()
    consts = dict(re.findall(r"#define (SSM_\w+) (\d+)u?", text))
    for k in ("SSM_OK", "SSM_ERR_INVALID", "SSM_ERR_UNSUPPORTED", "SSM_ERR_HIP", "SSM_F32", "SSM_BF16",
              "SSM_REVERSE", "SSM_COMPLEMENT", "SSM_SKIP", "SSM_GATE", "SSM_DELTA_SOFTPLUS", "SSM_SKIP_MAP",
              "SSM_SKIP_REVERSE", "SSM_SKIP_COMPLEMENT", "SSM_ACCUMULATE",
              "SSM_ACT_NONE", "SSM_ACT_SILU", "SSM_ACT_RELU"):
        assert int(consts[k]) == getattr(L, k), k
    assert int(consts["SSM_ABI_VERSION"]) == L.ABI_VERSION
    m = re.search(r"#define SSM_STATIC_SCRATCH_BYTES \((\d+)u << (\d+)\)", text)
    assert m and int(m[1]) << int(m[2]) == L.STATIC_SCRATCH_BYTES
    assert ctypes.sizeof(L.SsmDesc) == 72


def test_size_queries():
    lib = L.lib()
    d = L.make_desc(8, 8192, 2048, 16)
    # checkpoints: one f32 state per (b, block of 16 steps, n, d)
    assert lib.ssm_ckpt_bytes(ctypes.byref(d)) == 8 * (8192 // 16) * 16 * 2048 * 4
    # with the gate, y before the gate follows: B*L*D elements of the I/O type
    for dt, w in ((L.SSM_F32, 4), (L.SSM_BF16, 2)):
        g = L.make_desc(8, 8192, 2048, 16, dtype=dt, flags=L.SSM_GATE)
        assert lib.ssm_ckpt_bytes(ctypes.byref(g)) == 8 * (8192 // 16) * 16 * 2048 * 4 + 8 * 8192 * 2048 * w
        s = L.make_desc(8, 8192, 2048, 16, dtype=dt, flags=L.SSM_SKIP)
        assert lib.ssm_ckpt_bytes(ctypes.byref(s)) == 8 * (8192 // 16) * 16 * 2048 * 4
    # an odd bf16 residual is rounded up to whole 16-byte granules
    odd = L.make_desc(1, 3, 5, 4, dtype=L.SSM_BF16, flags=L.SSM_GATE)
    assert lib.ssm_ckpt_bytes(ctypes.byref(odd)) == 1 * 1 * 4 * 5 * 4 + 32
    assert lib.ssm_bwd_workspace_bytes(ctypes.byref(d)) > 0
    bad = L.make_desc(8, 8192, 2048, 33)
    assert lib.ssm_ckpt_bytes(ctypes.byref(bad)) == 0
    assert b"dstate" in lib.ssm_last_error()


def fwd_ws(**kw):
    lib = L.lib()
    return L.size_query(lib.ssm_fwd_workspace_bytes, L.make_desc(**kw), allow_zero=True)


def test_time_split_workspace_follows_the_segment_rule():
    # enough rows to fill the chip: one segment, no forward workspace
    assert fwd_ws(batch=8, seqlen=8192, dim=2048, dstate=16) == 0
    assert fwd_ws(batch=16, seqlen=4096, dim=5120, dstate=16, dtype=L.SSM_BF16) == 0
    # long-sequence shapes split in time: B*ceil(D/32)*ceil(N/4) waves, 2048 slots
    # config 3 (1 x 1M x 1024): 128 waves -> 16 segments; config 2 per direction: 256 -> 8
    per_seg = lambda B, N, D: B * 2 * N * D * 4  # end state and decay product per (row, state, channel)
    # each segment's aggregate walk is split into asub pieces while the walks of
    # every segment but one leave fewer than 2048 forward waves (4 per 64
    # channels) and a piece stays >= 16384 steps; with pieces, each (row, piece,
    # 64-channel block) also holds an int flag after the aggregates.
    # config 3: 960 waves, 65536-step segments -> 4 pieces; config 2: 16384-step
    # segments -> none
    per_piece = lambda B, N, D: per_seg(B, N, D) + B * ((D + 63) // 64) * 4
    assert fwd_ws(batch=1, seqlen=1 << 20, dim=1024, dstate=16) == 16 * 4 * per_piece(1, 16, 1024)
    assert fwd_ws(batch=4, seqlen=131072, dim=512, dstate=16) == 8 * per_seg(4, 16, 512)
    assert fwd_ws(batch=1, seqlen=65536, dim=40, dstate=8, segments=2) == 2 * 2 * per_piece(1, 8, 40)
    # segments never shorter than 512 steps when chosen automatically
    assert fwd_ws(batch=1, seqlen=1024, dim=32, dstate=4) == 2 * per_seg(1, 4, 32)
    assert fwd_ws(batch=1, seqlen=511, dim=32, dstate=4) == 0
    # forced: 3 segments of L=100 round to 64-step segments (whole 32-step tiles) -> 2
    assert fwd_ws(batch=2, seqlen=100, dim=8, dstate=4, segments=3) == 2 * per_seg(2, 4, 8)
    assert fwd_ws(batch=2, seqlen=100, dim=8, dstate=4, segments=1) == 0
    lib = L.lib()
    d1 = L.make_desc(2, 100, 8, 4, segments=1)
    d3 = L.make_desc(2, 100, 8, 4, segments=3)
    # the backward also holds per-segment dA / dD partials and adjoint carries
    assert lib.ssm_bwd_workspace_bytes(ctypes.byref(d3)) > lib.ssm_bwd_workspace_bytes(ctypes.byref(d1))


def test_split_forward_needs_its_workspace():
    lib = L.lib()
    d = L.make_desc(2, 100, 8, 4, segments=3)
    p = ctypes.c_void_p(16)
    assert lib.ssm_fwd(None, ctypes.byref(d), p, p, p, p, p, None, None, p, None, None) == L.SSM_ERR_INVALID
    assert b"workspace" in lib.ssm_last_error()


@pytest.mark.parametrize("field,value,msg", [
    ("batch", 0, b"batch, seqlen and dim"), ("dstate", 0, b"dstate"), ("dtype", 7, b"dtype"),
    ("flags", 512, b"unknown flag"), ("flags", 64, b"SKIP_MAP"), ("flags", 128, b"SKIP_MAP"),
    ("flags", 256, b"needs SSM_GATE"),
    ("delta_broadcast", 3, b"delta_broadcast"),
    ("segments", -1, b"segments"), ("segments", 1025, b"segments"), ("ld_y", 63, b"ld_y"), ("ld_z", 1, b"ld_z"),
    ("ld_y", 1 << 28, b"seqlen*ld_y"), ("ld_bc", 15, b"ld_bc"), ("ld_bc", 1 << 28, b"ld_bc"),
])
def test_invalid_desc_is_rejected_before_any_launch(field, value, msg):
    lib = L.lib()
    d = L.make_desc(2, 64, 64, 16)
    setattr(d, field, value)
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    rc = lib.ssm_fwd(None, ctypes.byref(d), p, p, p, p, p, None, None, p, None, None)
    assert rc == L.SSM_ERR_INVALID
    assert msg in lib.ssm_last_error()


def test_reduction_grid_bound_is_checked_before_any_launch():
    """B*L*N above 2^33 (each extent valid on its own) is refused up front: the
    backward's partial-sum reduction grid would not fit a 1-D launch."""
    lib = L.lib()
    d = L.make_desc(65535, 1 << 20, 64, 16)
    p = ctypes.c_void_p(16)
    rc = lib.ssm_bwd(None, ctypes.byref(d), p, p, p, p, p, None, None, p, p, p, p, p, p, p, None, None, p)
    assert rc == L.SSM_ERR_INVALID
    assert b"batch*seqlen*dstate" in lib.ssm_last_error()
    d = L.make_desc(8192, 1 << 16, 64, 16)  # 2^33 sums: the bound itself is accepted
    assert lib.ssm_bwd_workspace_bytes(ctypes.byref(d)) > 0


def test_null_pointers_and_missing_epilogue_operands_are_rejected():
    lib = L.lib()
    d = L.make_desc(2, 64, 64, 16)
    p = ctypes.c_void_p(16)
    assert lib.ssm_fwd(None, ctypes.byref(d), None, p, p, p, p, None, None, p, None, None) == L.SSM_ERR_INVALID
    d.flags = L.SSM_SKIP
    assert lib.ssm_fwd(None, ctypes.byref(d), p, p, p, p, p, None, None, p, None, None) == L.SSM_ERR_INVALID
    assert b"Dskip" in lib.ssm_last_error()
    d.flags = L.SSM_GATE
    rc = lib.ssm_bwd(None, ctypes.byref(d), p, p, p, p, p, None, p, p, p, p, p, p, p, p, None, None, p)
    assert rc == L.SSM_ERR_INVALID and b"dz" in lib.ssm_last_error()
    assert lib.ssm_fwd(None, None, p, p, p, p, p, None, None, p, None, None) == L.SSM_ERR_INVALID


def test_conv_desc_validation():
    lib = L.lib()
    assert ctypes.sizeof(L.SsmConvDesc) == 48
    p = ctypes.c_void_p(16)
    good = dict(batch=2, seqlen=64, dim=64, ksize=4, dtype=L.SSM_F32, flags=0, activation=L.SSM_ACT_SILU)
    d = L.SsmConvDesc(**good)
    # dw partial sums: one (K, D) slab per (batch row, 128-step tile)
    assert lib.ssm_conv_bwd_workspace_bytes(ctypes.byref(d)) == 2 * 1 * 4 * 64 * 4
    # more than 64 slabs: plus a staging area of one slab per 64 for the two-launch reduction
    long = L.SsmConvDesc(**dict(good, seqlen=128 * 100))
    assert lib.ssm_conv_bwd_workspace_bytes(ctypes.byref(long)) == (200 + 4) * 4 * 64 * 4
    for field, value, msg in [("ksize", 0, b"ksize"), ("ksize", 9, b"ksize"), ("activation", 3, b"activation"),
                              ("flags", L.SSM_SKIP, b"conv flags"),
                              ("dtype", 5, b"dtype"), ("seqlen", 0, b"seqlen"), ("ld_x", 8, b"ld_x")]:
        bad = L.SsmConvDesc(**{**good, field: value})
        assert lib.ssm_conv_fwd(None, ctypes.byref(bad), p, p, p) == L.SSM_ERR_INVALID, field
        assert msg in lib.ssm_last_error(), (field, lib.ssm_last_error())
    assert lib.ssm_conv_fwd(None, ctypes.byref(d), None, p, p) == L.SSM_ERR_INVALID
    assert lib.ssm_conv_bwd(None, ctypes.byref(d), p, p, p, p, p, None) == L.SSM_ERR_INVALID
    assert b"workspace" in lib.ssm_last_error()


def test_pair_entry_points_validate_before_launching():
    """ssm_fwd_pair / ssm_bwd_pair reject missing arrays and invalid descs without touching a GPU."""
    lib = L.lib()
    assert lib.ssm_fwd_pair(None, None, None) == L.SSM_ERR_INVALID
    assert lib.ssm_bwd_pair(None, None, None) == L.SSM_ERR_INVALID
    good = L.make_desc(2, 64, 64, 16)
    bad = L.make_desc(2, 64, 64, 64)  # dstate beyond 32
    descs = (L.SsmDesc * 2)(good, bad)
    p = ctypes.c_void_p(16)
    fio = (L.SsmFwdIo * 2)(*[L.SsmFwdIo(p, p, p, p, p, None, None, p, None, None)] * 2)
    assert lib.ssm_fwd_pair(None, descs, fio) == L.SSM_ERR_INVALID
    assert b"dstate" in lib.ssm_last_error()
    descs = (L.SsmDesc * 2)(good, good)
    fio[1].y = None
    assert lib.ssm_fwd_pair(None, descs, fio) == L.SSM_ERR_INVALID
    assert b"NULL" in lib.ssm_last_error()
    bio = (L.SsmBwdIo * 2)()
    assert lib.ssm_bwd_pair(None, descs, bio) == L.SSM_ERR_INVALID


def test_pair_rejects_mixed_dtypes_before_launching():
    """A pair runs one element type: an f32 desc with a bf16 desc is an invalid request
    (its second call would otherwise run f32 kernels over bf16 buffers)."""
    lib = L.lib()
    p = ctypes.c_void_p(16)
    for first, second in ((L.SSM_F32, L.SSM_BF16), (L.SSM_BF16, L.SSM_F32)):
        descs = (L.SsmDesc * 2)(L.make_desc(2, 64, 64, 16, dtype=first), L.make_desc(2, 64, 64, 16, dtype=second))
        fio = (L.SsmFwdIo * 2)(*[L.SsmFwdIo(p, p, p, p, p, None, None, p, None, None)] * 2)
        assert lib.ssm_fwd_pair(None, descs, fio) == L.SSM_ERR_INVALID
        assert b"same dtype" in lib.ssm_last_error()
        bio = (L.SsmBwdIo * 2)(*[L.SsmBwdIo(p, p, p, p, p, None, None, p, p, p, p, p, p, p, None, None, p)] * 2)
        assert lib.ssm_bwd_pair(None, descs, bio) == L.SSM_ERR_INVALID
        assert b"same dtype" in lib.ssm_last_error()


def test_static_scratch_backward_rejects_oversized_workspace():
    """ssm_bwd_static uses a fixed static scratch: a desc whose workspace exceeds it
    is an invalid request, refused before any GPU work (config 1 needs 268 MB of
    dB / dC partial sums)."""
    lib = L.lib()
    desc = L.make_desc(8, 8192, 2048, 16)
    assert L.size_query(lib.ssm_bwd_workspace_bytes, desc) > L.STATIC_SCRATCH_BYTES
    p = ctypes.c_void_p(16)
    rc = lib.ssm_bwd_static(None, ctypes.byref(desc), *([p] * 5), None, None, p, p, p, p, p, p, p, None, None)
    assert rc == L.SSM_ERR_INVALID
    assert b"static scratch" in lib.ssm_last_error()
    assert lib.ssm_bwd_static(None, None, *([p] * 16)) == L.SSM_ERR_INVALID
