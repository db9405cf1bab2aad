"""Host side of the selective scan: torch tensors in, HIP kernels through the C ABI.

Public functions keep the reference's names, argument order and errors:

* ``ssm_chunked_scan``   — selectssm.py:37-109
* ``ssm_recursive_scan`` — ssmrecscan.py:36-77
* ``ssm_scan``           — ssmrecscan.py:80-88, 163-183 (custom VJP)

All three run the same fused kernel pair (``ssm_fwd`` / ``ssm_bwd``) and are
differentiable through :class:`SelectiveScanFn`, whose backward is the custom
VJP's adjoint.  The reference's chunking / recursion arguments are validated
exactly as the reference does and otherwise do not change the result (the
reference's strategies agree up to fp32 rounding; the kernel's blocking is
internal).

:func:`selective_scan` is the fused op with the scan-adjacent epilogue of
``SelectiveSSM`` / ``BidirectionalMamba``: D-skip (selectssm.py:238), silu(z)
gate (selectssm.py:335-336) and the reverse / complement index maps
(selectssm.py:167-168, 230-231).
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _lib as L


# ---------------------------------------------------------------- host logic

def largest_factor_up_to(b: int, n: int) -> int:
    """Largest divisor of ``n`` not above ``b``; ``n`` itself when n < 2 (selectssm.py:24-30)."""
    if n < 2:
        return n
    k = b
    while n % k != 0:
        k -= 1
    return k


def resolve_chunking(L_: int, D: int, chunk_size=None, n_channel_groups=1):
    """``(chunk_size, K)`` with the reference's defaults and ValueErrors (selectssm.py:43-55)."""
    K = n_channel_groups if n_channel_groups is not None else 1
    if D % K != 0:
        raise ValueError(f"n_channel_groups={n_channel_groups} must divide D={D}")
    if chunk_size is None:
        chunk_size = largest_factor_up_to(int(math.sqrt(K * L_)), L_)
    if L_ % chunk_size != 0:
        raise ValueError(f"chunk_size={chunk_size} must divide L={L_}")
    return chunk_size, K


_IO_DTYPES = {torch.float32: L.SSM_F32, torch.bfloat16: L.SSM_BF16}


def _io_dtype(*ts):
    dt = None
    for t in ts:
        if t is None:
            continue
        dt = t.dtype if dt is None else torch.promote_types(dt, t.dtype)
    if dt not in _IO_DTYPES:
        raise TypeError(f"selective scan supports float32 and bfloat16 activations, got {dt}")
    return dt


def _check_shapes(u, delta, A, B, C, Dskip, z):
    if u.dim() != 3:
        raise ValueError(f"x must be (B, L, D), got shape {tuple(u.shape)}")
    Bt, Ln, D = u.shape
    if A.dim() != 2 or A.shape[0] != D:
        raise ValueError(f"Acoeff must be (D, N) with D={D}, got {tuple(A.shape)}")
    N = A.shape[1]
    for name, t in (("Bcoeff", B), ("Ccoeff", C)):
        if tuple(t.shape) != (Bt, Ln, N):
            raise ValueError(f"{name} must be (B, L, N)=({Bt}, {Ln}, {N}), got {tuple(t.shape)}")
    if tuple(delta.shape) not in ((Bt, Ln, D), (Bt, Ln, 1)):
        raise ValueError(f"dt must be (B, L, D) or (B, L, 1), got {tuple(delta.shape)}")
    if Dskip is not None and tuple(Dskip.shape) != (D,):
        raise ValueError(f"D must be ({D},), got {tuple(Dskip.shape)}")
    if z is not None and tuple(z.shape) != (Bt, Ln, D):
        raise ValueError(f"z must be (B, L, D), got {tuple(z.shape)}")
    for t in (u, delta, A, B, C, Dskip, z):
        if t is not None and not t.is_cuda:
            raise ValueError("selective scan inputs must be GPU tensors (there is no CPU path)")
    return Bt, Ln, D, N


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _flags(skip, gate, reverse, complement, delta_softplus=False, skip_map=None):
    """desc.flags.  ``reverse`` / ``complement``: the output map (time / channel
    reversal of the scan position, independently); ``skip_map``: None (the skip's u
    is read at the output position, the reference's convention) or a (time, channel)
    pair of bits giving the map of the scan position it is read at instead."""
    f = L.SSM_DELTA_SOFTPLUS if delta_softplus else 0
    if reverse:
        f |= L.SSM_REVERSE
    if complement:
        f |= L.SSM_COMPLEMENT
    if skip:
        f |= L.SSM_SKIP
    if gate:
        f |= L.SSM_GATE
    if skip_map is not None:
        f |= L.SSM_SKIP_MAP
        if skip_map[0]:
            f |= L.SSM_SKIP_REVERSE
        if skip_map[1]:
            f |= L.SSM_SKIP_COMPLEMENT
    return f


def _desc(u, delta, A, flags, segments=0, ld_y=0, ld_z=0, ld_bc=0):
    Bt, Ln, D = u.shape
    return L.make_desc(Bt, Ln, D, A.shape[1], _IO_DTYPES[u.dtype], flags,
                       delta_broadcast=(delta.shape[-1] == 1 and D != 1), segments=segments, ld_y=ld_y, ld_z=ld_z,
                       ld_bc=ld_bc)


def row_stride(t):
    """Row stride (elements between time rows) if ``t`` (B, L, D) is a column slice of a
    contiguous (B, L, W) array -- the layout the kernels read in place -- else None."""
    if t is None or t.dim() != 3 or t.stride(-1) != 1:
        return None
    Bt, Ln, D = t.shape
    ld = t.stride(1)
    if ld < D or (Bt > 1 and t.stride(0) != Ln * ld):
        return None
    return ld


def as_rows(t, dtype):
    """``t`` in ``dtype`` as a row-strided view the kernels can read, copying only if needed."""
    if t is None:
        return None, 0
    if t.dtype == dtype and row_stride(t) is not None:
        return t, row_stride(t)
    t = t.to(dtype).contiguous()
    return t, t.shape[-1]


def needs_grad(*ts) -> bool:
    """Whether an autograd graph will be recorded for an op on ``ts``: grad mode is
    on and some input requires a gradient.  Decided before ``Function.apply``,
    since inside ``forward`` grad mode is off and ``ctx.needs_input_grad`` does
    not reflect an enclosing ``torch.no_grad()``.  Only then are the forward's
    checkpoints (the backward's residuals) written."""
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ts)


def bc_stride(B, C):
    """The common row stride of B and C (:func:`row_stride`), which the kernels take
    as desc.ld_bc: B and C may be column slices of one wider array, e.g. of the BC
    projection's output.  Raises if they are not both readable in place with one stride."""
    ld_b, ld_c = row_stride(B), row_stride(C)
    if ld_b is None or ld_c is None or ld_b != ld_c:
        raise ValueError("B and C must be contiguous or column slices with one row stride of a contiguous "
                         "(B, L, W) tensor")
    return ld_b


def bc_rows(B, C, dtype):
    """B and C in ``dtype`` as views the kernels read in place (one row stride), copying
    both to contiguous arrays only if they are not."""
    if B.dtype == dtype and C.dtype == dtype:
        ld_b, ld_c = row_stride(B), row_stride(C)
        if ld_b is not None and ld_b == ld_c:
            return B, C
    return B.to(dtype).contiguous(), C.to(dtype).contiguous()


def _bc_grads(B, C, ld_bc, dbc_out):
    """Output arrays for dB and dC with the row stride ld_bc of B and C: two column
    slices of ``dbc_out`` ((B, L, W) with W = ld_bc >= 2N: dB in columns [0, N),
    dC in [N, 2N)), of a new such array, or two new arrays."""
    N = B.shape[-1]
    if ld_bc == N:
        return torch.empty_like(B), torch.empty_like(C)
    shape = (*B.shape[:-1], ld_bc)
    if dbc_out is not None:
        if tuple(dbc_out.shape) != shape or not dbc_out.is_contiguous() or dbc_out.dtype != B.dtype:
            raise ValueError(f"dbc_out must be a contiguous {B.dtype} array of shape {shape}")
        return dbc_out[..., :N], dbc_out[..., N:2 * N]
    if ld_bc >= 2 * N:
        buf = torch.empty(shape, dtype=B.dtype, device=B.device)
        return buf[..., :N], buf[..., N:2 * N]
    return (torch.empty(shape, dtype=B.dtype, device=B.device)[..., :N],
            torch.empty(shape, dtype=C.dtype, device=C.device)[..., :N])


def _scratch(nbytes, device):
    return torch.empty(nbytes // 4, dtype=torch.float32, device=device) if nbytes else None


# ------------------------------------------------------------- raw launchers

def scan_fwd(u, delta, A, B, C, Dskip=None, z=None, reverse=False, complement=False, want_ckpt=True,
             segments=0, delta_softplus=False, y_out=None, skip_map=None):
    """Run ``ssm_fwd``.  Tensors on one GPU, I/O dtype shared; u, delta, B, C contiguous,
    ``z`` and ``y_out`` contiguous or row-strided column slices (:func:`row_stride`).

    ``segments`` splits each row's time axis (0: chosen from the shape);
    ``delta_softplus``: ``delta`` is the pre-activation and the scan uses
    softplus(delta); ``y_out``: where to write y (allocated if None).  B and C
    may be column slices of one array (:func:`bc_stride`).  ``reverse`` /
    ``complement`` map the output (independently) and ``skip_map`` the skip's
    source (:func:`_flags`).
    Returns ``(y, ckpt)``: ``ckpt`` is the residual buffer :func:`scan_bwd` needs
    (the states entering each 16-step block and, with the gate, y before the
    gate), or None when ``want_ckpt`` is False.
    """
    flags = _flags(Dskip is not None, z is not None, reverse, complement, delta_softplus, skip_map)
    y = torch.empty_like(u) if y_out is None else y_out
    ld_y, ld_z = row_stride(y), (row_stride(z) if z is not None else 0)
    if ld_y is None or ld_z is None:
        raise ValueError("y_out and z must be contiguous or column slices of a contiguous (B, L, W) tensor")
    desc = _desc(u, delta, A, flags, segments, ld_y=ld_y, ld_z=ld_z, ld_bc=bc_stride(B, C))
    lib = L.lib()
    ckpt = _scratch(L.size_query(lib.ssm_ckpt_bytes, desc), u.device) if want_ckpt else None
    ws = _scratch(L.size_query(lib.ssm_fwd_workspace_bytes, desc, allow_zero=True), u.device)
    L.check(lib.ssm_fwd(_stream(), ctypes.byref(desc), _ptr(u), _ptr(delta), _ptr(A), _ptr(B), _ptr(C),
                        _ptr(Dskip), _ptr(z), _ptr(y), _ptr(ckpt), _ptr(ws)))
    return y, ckpt


def scan_bwd(u, delta, A, B, C, Dskip, z, ckpt, dy, reverse=False, complement=False, segments=0,
             delta_softplus=False, dbc_out=None, skip_map=None, dz_out=None, dz_accumulate=False):
    """Run ``ssm_bwd``.  Returns ``(du, ddelta, dA, dB, dC, dD, dz)`` (dD / dz None when unused);
    with ``delta_softplus``, ``ddelta`` is the gradient w.r.t. the pre-activation.
    ``dy`` and ``z`` may be row-strided column slices; dz is always contiguous.  When
    B and C are column slices of one array, dB and dC are the matching slices of
    ``dbc_out`` (or of a new array of that width).  ``dz_out``: the dz array to
    write, or with ``dz_accumulate`` to add the gate's gradient to (SSM_ACCUMULATE)."""
    flags = _flags(Dskip is not None, z is not None, reverse, complement, delta_softplus, skip_map)
    flags |= _acc_flag(z, dz_out, dz_accumulate)
    ld_y, ld_z = row_stride(dy), (row_stride(z) if z is not None else 0)
    if ld_y is None or ld_z is None:
        raise ValueError("dy and z must be contiguous or column slices of a contiguous (B, L, W) tensor")
    ld_bc = bc_stride(B, C)
    desc = _desc(u, delta, A, flags, segments, ld_y=ld_y, ld_z=ld_z, ld_bc=ld_bc)
    lib = L.lib()
    du = torch.empty_like(u)
    ddelta = torch.empty_like(delta)
    dA = torch.empty_like(A)
    dB, dC = _bc_grads(B, C, ld_bc, dbc_out)
    dD = torch.empty_like(Dskip) if Dskip is not None else None
    dz = _dz(z, dz_out)
    ws = _scratch(L.size_query(lib.ssm_bwd_workspace_bytes, desc), u.device)
    L.check(lib.ssm_bwd(_stream(), ctypes.byref(desc), _ptr(u), _ptr(delta), _ptr(A), _ptr(B), _ptr(C),
                        _ptr(Dskip), _ptr(z), _ptr(ckpt), _ptr(dy), _ptr(du), _ptr(ddelta), _ptr(dA),
                        _ptr(dB), _ptr(dC), _ptr(dD), _ptr(dz), _ptr(ws)))
    return du, ddelta, dA, dB, dC, dD, dz


def _acc_flag(z, dz_out, accumulate):
    if not accumulate:
        return 0
    if z is None or dz_out is None:
        raise ValueError("dz_accumulate needs the gate (z) and the dz_out array to add to")
    return L.SSM_ACCUMULATE


def _dz(z, dz_out):
    if z is None:
        return None
    if dz_out is None:
        return torch.empty(z.shape, dtype=z.dtype, device=z.device)
    if dz_out.shape != z.shape or dz_out.dtype != z.dtype or not dz_out.is_contiguous():
        raise ValueError("dz_out must be a contiguous array of z's shape and dtype")
    return dz_out


def scan_fwd_pair(calls):
    """Run ``ssm_fwd_pair``: two :func:`scan_fwd` calls, given as dicts of its
    keyword arguments, with the time-split aggregate passes of both in one
    launch where their shapes allow (results equal the two calls bit for bit).
    Returns ``[(y, ckpt), (y, ckpt)]``."""
    if len(calls) != 2:
        raise ValueError("scan_fwd_pair takes two calls")
    lib = L.lib()
    descs, ios, outs = (L.SsmDesc * 2)(), (L.SsmFwdIo * 2)(), []
    for k, c in enumerate(calls):
        u, delta, A, B, C = c["u"], c["delta"], c["A"], c["B"], c["C"]
        Dskip, z = c.get("Dskip"), c.get("z")
        flags = _flags(Dskip is not None, z is not None, c.get("reverse", False), c.get("complement", False),
                       c.get("delta_softplus", False), c.get("skip_map"))
        y = torch.empty_like(u) if c.get("y_out") is None else c["y_out"]
        ld_y, ld_z = row_stride(y), (row_stride(z) if z is not None else 0)
        if ld_y is None or ld_z is None:
            raise ValueError("y_out and z must be contiguous or column slices of a contiguous (B, L, W) tensor")
        descs[k] = _desc(u, delta, A, flags, c.get("segments", 0), ld_y=ld_y, ld_z=ld_z, ld_bc=bc_stride(B, C))
        ckpt = (_scratch(L.size_query(lib.ssm_ckpt_bytes, descs[k]), u.device) if c.get("want_ckpt", True)
                else None)
        ws = _scratch(L.size_query(lib.ssm_fwd_workspace_bytes, descs[k], allow_zero=True), u.device)
        ios[k] = L.SsmFwdIo(_ptr(u), _ptr(delta), _ptr(A), _ptr(B), _ptr(C), _ptr(Dskip), _ptr(z), _ptr(y),
                            _ptr(ckpt), _ptr(ws))
        outs.append((y, ckpt, ws))
    L.check(lib.ssm_fwd_pair(_stream(), descs, ios))
    return [(y, ckpt) for y, ckpt, _ in outs]


def scan_bwd_pair(calls):
    """Run ``ssm_bwd_pair``: two :func:`scan_bwd` calls, given as dicts of its
    keyword arguments (``u, delta, A, B, C, Dskip, z, ckpt, dy``, the flags and
    optionally ``dbc_out``, ``dz_out``, ``dz_accumulate``).  The second call may
    accumulate into the first call's ``dz_out`` (BidirectionalMamba's tied gate).
    Returns the two ``(du, ddelta, dA, dB, dC, dD, dz)`` tuples."""
    if len(calls) != 2:
        raise ValueError("scan_bwd_pair takes two calls")
    lib = L.lib()
    descs, ios, outs = (L.SsmDesc * 2)(), (L.SsmBwdIo * 2)(), []
    for k, c in enumerate(calls):
        u, delta, A, B, C, dy = c["u"], c["delta"], c["A"], c["B"], c["C"], c["dy"]
        Dskip, z = c.get("Dskip"), c.get("z")
        flags = _flags(Dskip is not None, z is not None, c.get("reverse", False), c.get("complement", False),
                       c.get("delta_softplus", False), c.get("skip_map"))
        flags |= _acc_flag(z, c.get("dz_out"), c.get("dz_accumulate", False))
        ld_y, ld_z = row_stride(dy), (row_stride(z) if z is not None else 0)
        if ld_y is None or ld_z is None:
            raise ValueError("dy and z must be contiguous or column slices of a contiguous (B, L, W) tensor")
        ld_bc = bc_stride(B, C)
        descs[k] = _desc(u, delta, A, flags, c.get("segments", 0), ld_y=ld_y, ld_z=ld_z, ld_bc=ld_bc)
        g = (torch.empty_like(u), torch.empty_like(delta), torch.empty_like(A),
             *_bc_grads(B, C, ld_bc, c.get("dbc_out")), torch.empty_like(Dskip) if Dskip is not None else None,
             _dz(z, c.get("dz_out")))
        ws = _scratch(L.size_query(lib.ssm_bwd_workspace_bytes, descs[k]), u.device)
        ios[k] = L.SsmBwdIo(_ptr(u), _ptr(delta), _ptr(A), _ptr(B), _ptr(C), _ptr(Dskip), _ptr(z), _ptr(c["ckpt"]),
                            _ptr(dy), *(_ptr(t) for t in g), _ptr(ws))
        outs.append((g, ws))
    L.check(lib.ssm_bwd_pair(_stream(), descs, ios))
    return [g for g, _ in outs]


# ------------------------------------------------------------------- autograd

class SelectiveScanFn(torch.autograd.Function):
    """y = epilogue(scan(u, delta, A, B, C)) with the custom-VJP backward.

    The saved residuals are the inputs plus the forward's state checkpoints
    (the reference saves only the inputs, ssmrecscan.py:88, and recomputes
    recursively in the backward, ssmrecscan.py:111-161).
    """

    @staticmethod
    def forward(ctx, u, delta, A, B, C, Dskip, z, reverse, complement, segments, delta_softplus, want_ckpt):
        y, ckpt = scan_fwd(u, delta, A, B, C, Dskip, z, reverse, complement, want_ckpt=want_ckpt, segments=segments,
                           delta_softplus=delta_softplus)
        ctx.save_for_backward(u, delta, A, B, C, Dskip, z, ckpt)
        ctx.flags = (reverse, complement)
        ctx.segments = segments
        ctx.delta_softplus = delta_softplus
        return y

    @staticmethod
    def backward(ctx, dy):
        u, delta, A, B, C, Dskip, z, ckpt = ctx.saved_tensors
        dy, _ = as_rows(dy, u.dtype)
        du, ddelta, dA, dB, dC, dD, dz = scan_bwd(u, delta, A, B, C, Dskip, z, ckpt, dy, *ctx.flags,
                                                  segments=ctx.segments, delta_softplus=ctx.delta_softplus)
        return du, ddelta, dA, dB, dC, dD, dz, None, None, None, None, None


def selective_scan(u, delta, A, B, C, D=None, z=None, reverse=False, complement=False, segments=0,
                   delta_softplus=False):
    """Fused selective scan with the SelectiveSSM / BidirectionalMamba epilogue.

    u, delta, B, C are in the scan domain (flipped already when ``reverse``,
    as SelectiveSSM builds them from the flipped x, selectssm.py:167-210);
    the output is in the original domain:
        y = scan(u, delta, A, B, C)              (selectssm.py:222-228)
        y = flip(y)            if reverse        (selectssm.py:230-231)
        y = y + u * D          if D is given     (selectssm.py:238; u stays flipped)
        y = y * silu(z)        if z is given     (selectssm.py:335-336)
    ``complement`` (with ``reverse``) also mirrors the channel axis.
    ``delta_softplus``: ``delta`` is the pre-activation of selectssm.py:210;
    the scan uses softplus(delta) and the gradient flows to the pre-activation.
    ``segments`` > 0 forces that many time segments per row (0: the library
    splits rows only when there are too few to fill the GPU); the result
    agrees with one segment up to fp32 rounding.
    """
    Bt, Ln, Dm, N = _check_shapes(u, delta, A, B, C, D, z)
    if complement and not reverse:
        complement = False  # the reference only looks at complement when reverse (selectssm.py:116)
    io = _io_dtype(u, delta, B, C, z)
    cast = lambda t: None if t is None else t.to(io).contiguous()
    fcast = lambda t: None if t is None else t.to(torch.float32).contiguous()
    if not 0 <= int(segments) <= 1024:
        raise ValueError(f"segments must be in 0..1024, got {segments}")
    Bk, Ck = bc_rows(B, C, io)
    return SelectiveScanFn.apply(cast(u), cast(delta), fcast(A), Bk, Ck, fcast(D), as_rows(z, io)[0],
                                 bool(reverse), bool(complement), int(segments), bool(delta_softplus),
                                 needs_grad(u, delta, A, B, C, D, z))


class BidirectionalScanFn(torch.autograd.Function):
    """The two scans of BidirectionalMamba (forward direction, and reverse with the
    optional complement) written straight into the concatenated (B, L, 2D) output,
    each with its D skip and silu(z) gate fused (selectssm.py:325-336)."""

    @staticmethod
    def forward(ctx, uf, dtf, Af, Bf, Cf, Df, zf, ur, dtr, Ar, Br, Cr, Dr, zr, complement, delta_softplus, want):
        Bt, Ln, D = uf.shape
        y = torch.empty(Bt, Ln, 2 * D, dtype=uf.dtype, device=uf.device)
        # one pair call: the time-split aggregate passes of both directions share a launch
        (_, ckf), (_, ckr) = scan_fwd_pair([
            dict(u=uf, delta=dtf, A=Af, B=Bf, C=Cf, Dskip=Df, z=zf, want_ckpt=want, delta_softplus=delta_softplus,
                 y_out=y[..., :D]),
            dict(u=ur, delta=dtr, A=Ar, B=Br, C=Cr, Dskip=Dr, z=zr, reverse=True, complement=complement,
                 want_ckpt=want, delta_softplus=delta_softplus, y_out=y[..., D:])])
        ctx.save_for_backward(uf, dtf, Af, Bf, Cf, Df, zf, ckf, ur, dtr, Ar, Br, Cr, Dr, zr, ckr)
        ctx.cfg = (complement, delta_softplus)
        return y

    @staticmethod
    def backward(ctx, dy):
        uf, dtf, Af, Bf, Cf, Df, zf, ckf, ur, dtr, Ar, Br, Cr, Dr, zr, ckr = ctx.saved_tensors
        complement, dsp = ctx.cfg
        D = uf.shape[-1]
        dy, _ = as_rows(dy, uf.dtype)
        gf, gr = scan_bwd_pair([
            dict(u=uf, delta=dtf, A=Af, B=Bf, C=Cf, Dskip=Df, z=zf, ckpt=ckf, dy=dy[..., :D], delta_softplus=dsp),
            dict(u=ur, delta=dtr, A=Ar, B=Br, C=Cr, Dskip=Dr, z=zr, ckpt=ckr, dy=dy[..., D:], reverse=True,
                 complement=complement, delta_softplus=dsp)])
        return (*gf, *gr, None, None, None)


def bidirectional_selective_scan(fwd, rev, complement=False, delta_softplus=False):
    """concat([scan_f(...) , scan_r(...)], -1) for BidirectionalMamba in one output buffer.

    ``fwd`` / ``rev``: dicts with u, delta, A, B, C, D, z of each direction (the
    reverse direction's in its scan domain, as for :func:`selective_scan` with
    ``reverse=True``).  z may be a column slice of in_proj's output (read in place).
    """
    io = _io_dtype(fwd["u"], fwd["delta"], fwd["B"], fwd["C"], fwd["z"], rev["u"], rev["delta"], rev["B"],
                   rev["C"], rev["z"])
    cast = lambda t: None if t is None else t.to(io).contiguous()
    fcast = lambda t: None if t is None else t.to(torch.float32).contiguous()
    args = []
    for d in (fwd, rev):
        _check_shapes(d["u"], d["delta"], d["A"], d["B"], d["C"], d.get("D"), d.get("z"))
        args += [cast(d["u"]), cast(d["delta"]), fcast(d["A"]), *bc_rows(d["B"], d["C"], io), fcast(d.get("D")),
                 as_rows(d.get("z"), io)[0]]
    if fwd["u"].shape != rev["u"].shape:
        raise ValueError("the two directions must have the same (B, L, D)")
    want = needs_grad(*(d.get(k) for d in (fwd, rev) for k in ("u", "delta", "A", "B", "C", "D", "z")))
    return BidirectionalScanFn.apply(*args, bool(complement), bool(delta_softplus), want)


# ------------------------------------------------------- reference-named API

def ssm_chunked_scan(x, Acoeff, Bcoeff, Ccoeff, dt, chunk_size: int = None, n_channel_groups: int = 1):
    """Drop-in for ``ssm_chunked_scan`` (selectssm.py:37-109).

    Same arguments and ValueErrors (selectssm.py:47-48, 53-54); the result does
    not depend on ``chunk_size`` / ``n_channel_groups`` beyond fp32 rounding.
    """
    if x.dim() != 3:
        raise ValueError(f"x must be (B, L, D), got shape {tuple(x.shape)}")
    resolve_chunking(x.shape[-2], x.shape[-1], chunk_size, n_channel_groups)
    return selective_scan(x, dt, Acoeff, Bcoeff, Ccoeff)


def _check_recursion(L_, min_recursion_length, recursive_split):
    """The reference's recursion test at the top level (ssmrecscan.py:56): it splits a
    chunk only while ``len > min_recursion_length and len % recursive_split == 0``.
    A row that short never recurses and returns a result whatever the split; a
    split of 1 that does recurse never shortens the chunk (the reference recurses
    without end), and a split of 0 divides by zero in that test."""
    if L_ <= min_recursion_length:
        return
    if recursive_split == 0:
        raise ZeroDivisionError("integer division or modulo by zero (recursive_split=0)")
    if L_ % recursive_split != 0:
        return
    if recursive_split == 1:
        raise RecursionError(f"recursive_split={recursive_split} never shortens the sequence")
    if recursive_split < 0:
        raise ValueError(f"recursive_split={recursive_split} must be positive")


def ssm_recursive_scan(x, Acoeff, Bcoeff, Ccoeff, Delta, min_recursion_length: int = 2, recursive_split: int = 2):
    """Drop-in for ``ssm_recursive_scan`` (ssmrecscan.py:36-77)."""
    if x.dim() != 3:
        raise ValueError(f"x must be (B, L, D), got shape {tuple(x.shape)}")
    _check_recursion(x.shape[-2], min_recursion_length, recursive_split)
    return selective_scan(x, Delta, Acoeff, Bcoeff, Ccoeff)


def ssm_scan(x, Acoeff, Bcoeff, Ccoeff, Delta, min_recursion_length: int = 2, recursive_split: int = 2):
    """Drop-in for the custom-VJP ``ssm_scan`` (ssmrecscan.py:80-88, 163-183).

    Its gradient is the custom VJP's adjoint (du, dA, dB, dC, ddelta), computed
    by ``ssm_bwd`` from the inputs and the forward's checkpoints.
    """
    if x.dim() != 3:
        raise ValueError(f"x must be (B, L, D), got shape {tuple(x.shape)}")
    _check_recursion(x.shape[-2], min_recursion_length, recursive_split)
    return selective_scan(x, Delta, Acoeff, Bcoeff, Ccoeff)
