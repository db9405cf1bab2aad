"""``SelectiveSSM`` and ``BidirectionalMamba`` as torch modules over the HIP kernels.

Same constructor fields, defaults, parameter tree and call signature as the
reference's Flax modules (selectssm.py:112-238 and 240-364); a Flax parameter
tree loads 1:1 with :meth:`load_flax_params` (Flax ``a/b`` is torch ``a.b``;
Dense kernels keep Flax's (in, out) layout).  Like Flax modules, the parameters
take their shapes from the first input unless ``features`` is given.

The hot path is fused:
  * flip + ``shift_conv`` + activation  -> one ``ssm_conv_fwd`` launch
  * softplus(dt), the scan, the un-flip, the D skip (with the reference's
    flipped-domain ``u``), and in BidirectionalMamba the silu gate
                                        -> one ``ssm_fwd`` per direction, the two
    as one ``ssm_fwd_pair`` call (their time-split aggregate passes share a
    launch), both writing straight into the concatenated output; the conv
    inputs and the gates are read in place from in_proj's output
  * the Dense projections (BC, dt, dt_proj, in_proj, out_proj) run on hipBLASLt
    through torch.
Every strategy flag (chunked / ``recursive_scan`` / ``custom_vjp_scan``) runs the
same kernels after the reference's own argument checks (the strategies agree
up to fp32 rounding); the backward is the custom VJP's adjoint.

Activations are computed in the input's dtype (float32, or bfloat16 with fp32
scan state and accumulation); parameters are float32.
"""
from __future__ import annotations

import math
from typing import Optional, Union

import torch
import torch.nn.functional as F

from .conv import conv1d_act, conv1d_act_map, conv1d_act_pair
from .scan import (_check_recursion, as_rows, bidirectional_selective_scan, needs_grad, resolve_chunking, scan_bwd,
                   scan_bwd_pair, scan_fwd, scan_fwd_pair, selective_scan)

_FUSED_CONV_ACTS = ("silu", "relu", None)


def _activation_fn(name):
    if name == "gelu":
        return lambda t: F.gelu(t, approximate="tanh")  # flax.linen.gelu default: tanh approximation
    if name == "silu":
        return F.silu
    if name == "relu":
        return F.relu
    raise Exception(f"Unknown activation: {name}")


def lecun_normal_(t: torch.Tensor, fan_in: int, generator=None) -> torch.Tensor:
    """Truncated normal in [-2, 2] std units with variance 1/fan_in (lecun_normal)."""
    std = math.sqrt(1.0 / fan_in) / 0.87962566103423978  # std of a unit normal truncated to [-2, 2]
    with torch.no_grad():
        t.normal_(0.0, 1.0, generator=generator)
        # redraw outside [-2, 2] until none remain
        for _ in range(100):
            bad = t.abs() > 2
            if not bad.any():
                break
            t[bad] = torch.randn(int(bad.sum()), device=t.device, dtype=t.dtype, generator=generator)
        t.clamp_(-2, 2).mul_(std)
    return t


def inverse_softplus(x):
    """x + log(1 - e^-x) (selectssm.py:18-19)."""
    return x + torch.log(-torch.expm1(-x))


class Dense(torch.nn.Module):
    """flax.linen.Dense: y = x @ kernel + bias, kernel (in, out)."""

    def __init__(self, in_features, out_features, use_bias=True, device=None, generator=None, bias_init=None):
        super().__init__()
        self.kernel = torch.nn.Parameter(lecun_normal_(torch.empty(in_features, out_features, device=device),
                                                       in_features, generator))
        if use_bias:
            b = torch.zeros(out_features, device=device) if bias_init is None else bias_init
            self.bias = torch.nn.Parameter(b)
        else:
            self.register_parameter("bias", None)

    def forward(self, x, flip_in: bool = False, flip_out: bool = False):
        """x @ kernel + bias.  ``flip_in`` / ``flip_out`` reverse the kernel's input rows /
        output columns (and the bias): the layer conjugated by a channel flip of its
        input / output, as an RC-conjugated block needs (parameters are permuted, the
        activations are not)."""
        w = self.kernel.to(x.dtype)
        b = None if self.bias is None else self.bias.to(x.dtype)
        if flip_in:
            w = w.flip(0)
        if flip_out:
            w = w.flip(1)
            b = None if b is None else b.flip(0)
        x2 = x.reshape(-1, x.shape[-1])
        y = _DenseFn.apply(x2, w, b)
        return y.reshape(*x.shape[:-1], w.shape[1])

    def forward_split(self, x, widths, flip_in: bool = False):
        """The output's consecutive column blocks of the given widths (views of
        one output array), as ``jnp.split(dense(x), ...)`` gives them; the
        backward consumes the blocks' gradients without assembling the full
        width (:class:`_DenseSplitFn`)."""
        w = self.kernel.to(x.dtype)
        b = None if self.bias is None else self.bias.to(x.dtype)
        if flip_in:
            w = w.flip(0)
        x2 = x.reshape(-1, x.shape[-1])
        blocks = _DenseSplitFn.apply(x2, w, b, *widths)
        return tuple(h.view(*x.shape[:-1], h.shape[-1]) for h in blocks)


class _DenseFn(torch.autograd.Function):
    """x2 @ w + b with the weight gradient through _tn (split over the rows)."""

    @staticmethod
    def forward(ctx, x2, w, b):
        ctx.save_for_backward(x2, w)
        ctx.has_bias = b is not None
        return x2 @ w if b is None else torch.addmm(b, x2, w)

    @staticmethod
    def backward(ctx, dy):
        x2, w = ctx.saved_tensors
        dy = dy.contiguous()
        dx = dy @ w.t() if ctx.needs_input_grad[0] else None
        dw = _tn(x2, dy) if ctx.needs_input_grad[1] else None
        db = dy.sum(0) if ctx.has_bias and ctx.needs_input_grad[2] else None
        return dx, dw, db


class _ShiftConv(torch.nn.Module):
    def __init__(self, K, D, device=None, generator=None):
        super().__init__()
        # Flax Conv kernel (K, in/groups = 1, D); fan_in = K * 1
        self.kernel = torch.nn.Parameter(lecun_normal_(torch.empty(K, 1, D, device=device), K, generator))


class _FlaxModule(torch.nn.Module):
    """Lazy build on first call + Flax parameter-tree import / export."""

    def load_flax_params(self, params: dict) -> None:
        """Copy a Flax parameter tree (nested dict of arrays, no 'params' root) into this module."""
        flat = {}

        def walk(prefix, tree):
            for k, v in tree.items():
                if isinstance(v, dict):
                    walk(prefix + k + ".", v)
                else:
                    flat[prefix + k] = v

        walk("", params)
        own = dict(self.named_parameters())
        if set(flat) != set(own):
            raise ValueError(f"parameter trees differ: missing {sorted(set(own) - set(flat))}, "
                             f"unexpected {sorted(set(flat) - set(own))}")
        with torch.no_grad():
            for k, v in flat.items():
                t = torch.as_tensor(v)
                if tuple(t.shape) != tuple(own[k].shape):
                    raise ValueError(f"{k}: shape {tuple(t.shape)} != {tuple(own[k].shape)}")
                own[k].copy_(t)

    def flax_params(self) -> dict:
        """This module's parameters as a Flax-style nested dict of CPU tensors."""
        tree = {}
        for name, p in self.named_parameters():
            node = tree
            *path, leaf = name.split(".")
            for part in path:
                node = node.setdefault(part, {})
            node[leaf] = p.detach().cpu()
        return tree


_TN_SLICE = 8192  # rows of K per slice of a split weight-gradient product


def _tn(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """``a.t() @ b`` for the weight gradients, whose K = B*L is long and whose
    M, N are a few hundred at most (e.g. (2^19 x 512)^T (2^19 x 32) for a
    4 x 131072 BidirectionalMamba batch).  One GEMM call over that K re-reads
    ``a`` many times (19 GB fetched for a 1 GB operand on hipBLASLt), so for float32 the K axis
    is cut into slices of _TN_SLICE rows whose products run as one batched
    GEMM, then summed over the slices in order: deterministic, and each
    partial sum is shorter than the single call's.  bfloat16 keeps the single
    call, whose output is rounded once rather than once per slice."""
    K = a.shape[0]
    S = K // _TN_SLICE
    if a.dtype != torch.float32 or S < 2 or K % _TN_SLICE:
        return a.t() @ b
    a3 = a.reshape(S, _TN_SLICE, a.shape[1])
    b3 = b.reshape(S, _TN_SLICE, b.shape[1])
    # (S, N, M): the transposed view is the left operand, the right one is contiguous
    return torch.bmm(b3.transpose(1, 2), a3).sum(0).t()


def _core_project(u, A_log, Wbc, bbc, Wdt, bdt, Wp, bp, N, rank):
    """The scan's operands from u (selectssm.py:190-210): (A, dt_low, dt, B, C),
    dt before its softplus, which the scan applies."""
    B_, L_, D = u.shape
    u2 = u.reshape(-1, D)
    BC = torch.addmm(bbc.to(u.dtype), u2, Wbc.to(u.dtype))
    dt_low = torch.addmm(bdt.to(u.dtype), u2, Wdt.to(u.dtype))
    if Wp is not None:
        dt = torch.addmm(bp.to(u.dtype), dt_low, Wp.to(u.dtype)).reshape(B_, L_, D)
    elif rank > 1:
        dt = torch.repeat_interleave(dt_low, D // rank, dim=-1).reshape(B_, L_, D)
    else:
        dt = dt_low.reshape(B_, L_, 1)
    # B and C stay column slices of the projection's (B, L, 2N) output, which the
    # scan reads in place (desc.ld_bc = 2N)
    BC3 = BC.reshape(B_, L_, 2 * N)
    Bc, Cc = BC3[..., :N], BC3[..., N:]
    A = -torch.exp(A_log)
    return A, dt_low, dt.contiguous(), Bc, Cc


def _core_forward(u, A_log, Wbc, bbc, Wdt, bdt, Wp, bp, Dp, z, N, rank, reverse, complement, want_ckpt, y_out=None,
                  skip_map=None):
    """Projections + scan (selectssm.py:190-238); returns (y, saved tensors).  The scan
    writes its checkpoints only when ``want_ckpt`` (a backward will run).  ``reverse``,
    ``complement``: the output map; ``skip_map``: the skip's source map (scan_fwd)."""
    A, dt_low, dt, Bc, Cc = _core_project(u, A_log, Wbc, bbc, Wdt, bdt, Wp, bp, N, rank)
    y, ckpt = scan_fwd(u, dt, A, Bc, Cc, Dp, z, reverse, complement, want_ckpt=want_ckpt, delta_softplus=True,
                       y_out=y_out, skip_map=skip_map)
    return y, (u, A, Wbc, Wdt, Wp, Dp, z, dt_low, dt, Bc, Cc, ckpt)


def _dbc_buffer(u, N):
    """The BC projection's gradient (B, L, 2N): the scan's backward writes dB and dC
    straight into its two column halves."""
    return torch.empty(*u.shape[:-1], 2 * N, dtype=u.dtype, device=u.device)


def _scan_call(saved, reverse, complement, N, skip_map=None):
    """The scan's arguments for the scan_*_pair launchers, from _core_forward's saved tensors."""
    u, A, _, _, _, Dp, z, _, dt, Bc, Cc, ckpt = saved
    return dict(u=u, delta=dt, A=A, B=Bc, C=Cc, Dskip=Dp, z=z, reverse=reverse, complement=complement,
                delta_softplus=True, dbc_out=_dbc_buffer(u, N), skip_map=skip_map)


def _core_backward(saved, dy, N, rank, reverse, complement, skip_map=None):
    """Gradients of _core_forward for (u, A_log, Wbc, bbc, Wdt, bdt, Wp, bp, D, z)."""
    u, A, Wbc, Wdt, Wp, Dp, z, dt_low, dt, Bc, Cc, ckpt = saved
    dbc = _dbc_buffer(u, N)
    grads = scan_bwd(u, dt, A, Bc, Cc, Dp, z, ckpt, dy, reverse, complement, delta_softplus=True, dbc_out=dbc,
                     skip_map=skip_map)
    return _core_param_grads(saved, grads, dbc, N, rank)


def _core_param_grads(saved, grads, dbc, N, rank):
    """_core_backward after the scan's backward (which wrote dB, dC into ``dbc``): the
    projections' and u's gradients."""
    u, A, Wbc, Wdt, Wp, Dp, z, dt_low, dt, Bc, Cc, ckpt = saved
    du, ddt, dA, dB, dC, dD, dz = grads
    D = u.shape[-1]
    u2 = u.reshape(-1, D)
    du2 = du.reshape(-1, D)
    dBC = dbc.reshape(-1, 2 * N)
    dWbc = _tn(u2, dBC)
    dbbc = dBC.sum(0)
    du2.addmm_(dBC, Wbc.to(u.dtype).t())  # u's gradient through BC, accumulated in place
    if Wp is not None:
        ddt2 = ddt.reshape(-1, D)
        dWp = _tn(dt_low, ddt2).to(Wp.dtype)
        dbp = ddt2.sum(0).to(Wp.dtype)
        ddt_low = ddt2 @ Wp.to(u.dtype).t()
    else:
        dWp = dbp = None
        ddt_low = ddt.reshape(-1, rank, D // rank).sum(-1) if rank > 1 else ddt.reshape(-1, 1)
    dWdt = _tn(u2, ddt_low)
    dbdt = ddt_low.sum(0)
    du2.addmm_(ddt_low, Wdt.to(u.dtype).t())  # and through dt
    dA_log = dA * A  # A = -exp(A_log)
    f32 = lambda g: g.to(torch.float32)
    return du, dA_log, f32(dWbc), f32(dbbc), f32(dWdt), f32(dbdt), dWp, dbp, dD, dz


class _DenseSplitFn(torch.autograd.Function):
    """h2 = x2 @ w + b returned as its consecutive column blocks (in_proj followed
    by the ``jnp.split`` of selectssm.py:319), each a view of h2.  The backward
    takes the blocks' gradients as they come: dx = sum_i g_i @ w_i^T accumulates
    block by block, and dw, db are built per block, so no gradient of h2's full
    width is ever assembled (slicing h2 would give each block a zero-filled
    full-width gradient to add up; concatenating the blocks' gradients would
    copy them all once more)."""

    @staticmethod
    def forward(ctx, x2, w, b, *widths):
        if sum(widths) != w.shape[1]:
            raise ValueError(f"column blocks {widths} do not cover the {w.shape[1]} outputs")
        ctx.save_for_backward(x2, w)
        ctx.widths = widths
        ctx.has_bias = b is not None
        h2 = x2 @ w if b is None else torch.addmm(b, x2, w)
        outs, o = [], 0
        for wd in widths:
            outs.append(h2[:, o:o + wd])
            o += wd
        return tuple(outs)

    @staticmethod
    def backward(ctx, *grads):
        x2, w = ctx.saved_tensors
        dx = None
        dw_parts, db_parts, o = [], [], 0
        for g, wd in zip(grads, ctx.widths):
            wb = w[:, o:o + wd]
            o += wd
            if g is None:  # an unused block: zero gradient
                dw_parts.append(torch.zeros_like(wb))
                db_parts.append(torch.zeros(wd, dtype=w.dtype, device=w.device))
                continue
            g = g.contiguous()
            if ctx.needs_input_grad[0]:
                if dx is None:
                    dx = g @ wb.t()
                else:
                    dx.addmm_(g, wb.t())
            if ctx.needs_input_grad[1]:
                dw_parts.append(_tn(x2, g))
            if ctx.has_bias and ctx.needs_input_grad[2]:
                db_parts.append(g.sum(0))
        if dx is None and ctx.needs_input_grad[0]:
            dx = torch.zeros_like(x2)
        dw = torch.cat(dw_parts, dim=1) if ctx.needs_input_grad[1] else None
        db = torch.cat(db_parts) if ctx.has_bias and ctx.needs_input_grad[2] else None
        return (dx, dw, db, *([None] * len(ctx.widths)))


class _SSMCoreFn(torch.autograd.Function):
    """u -> BC, dt (-> dt_proj) projections -> scan with softplus(dt), D skip and
    optional silu(z) gate (selectssm.py:190-238), with a hand-written backward
    that accumulates u's three gradient contributions in place (addmm with
    beta = 1) instead of separate addition kernels."""

    @staticmethod
    def forward(ctx, u, A_log, Wbc, bbc, Wdt, bdt, Wp, bp, Dp, z, N, rank, reverse, complement, skip_map, want_ckpt):
        y, saved = _core_forward(u, A_log, Wbc, bbc, Wdt, bdt, Wp, bp, Dp, z, N, rank, reverse, complement, want_ckpt,
                                 skip_map=skip_map)
        ctx.save_for_backward(*saved)
        ctx.cfg = (N, rank, reverse, complement, skip_map)
        return y

    @staticmethod
    def backward(ctx, dy):
        dy, _ = as_rows(dy, ctx.saved_tensors[0].dtype)
        return (*_core_backward(ctx.saved_tensors, dy, *ctx.cfg), None, None, None, None, None, None)


class _PairCoreFn(torch.autograd.Function):
    """Both BidirectionalMamba directions' cores (_SSMCoreFn), each writing its y
    straight into its half of the concatenated output (selectssm.py:325-336).
    ``maps``: per direction, the scan's output map (time, channel) and skip map
    (SelectiveSSM._maps)."""

    @staticmethod
    def forward(ctx, uf, A_logf, Wbcf, bbcf, Wdtf, bdtf, Wpf, bpf, Df, zf,
                ur, A_logr, Wbcr, bbcr, Wdtr, bdtr, Wpr, bpr, Dr, zr, N, rank, maps, want_ckpt, tied_z=False):
        B_, L_, E = uf.shape
        y = torch.empty(B_, L_, 2 * E, dtype=uf.dtype, device=uf.device)
        pf = _core_project(uf, A_logf, Wbcf, bbcf, Wdtf, bdtf, Wpf, bpf, N, rank)
        pr = _core_project(ur, A_logr, Wbcr, bbcr, Wdtr, bdtr, Wpr, bpr, N, rank)
        # both directions' scans in one pair call (one launch per kernel for the two)
        calls = [dict(u=u, delta=p[2], A=p[0], B=p[3], C=p[4], Dskip=Dp, z=z, reverse=om[0], complement=om[1],
                      skip_map=sm, delta_softplus=True, y_out=yo, want_ckpt=want_ckpt)
                 for u, p, Dp, z, (om, sm), yo in ((uf, pf, Df, zf, maps[0], y[..., :E]),
                                                   (ur, pr, Dr, zr, maps[1], y[..., E:]))]
        (_, ckf), (_, ckr) = scan_fwd_pair(calls)
        sf = (uf, pf[0], Wbcf, Wdtf, Wpf, Df, zf, pf[1], pf[2], pf[3], pf[4], ckf)
        sr = (ur, pr[0], Wbcr, Wdtr, Wpr, Dr, zr, pr[1], pr[2], pr[3], pr[4], ckr)
        ctx.save_for_backward(*sf, *sr)
        ctx.cfg = (N, rank, maps, len(sf))
        ctx.tied_z = bool(tied_z) and zf is not None
        return y

    @staticmethod
    def backward(ctx, dy):
        N, rank, maps, k = ctx.cfg
        saved = ctx.saved_tensors
        E = saved[0].shape[-1]
        dy, _ = as_rows(dy, saved[0].dtype)
        sf, sr = saved[:k], saved[k:]
        (omf, smf), (omr, smr) = maps
        cf, cr = _scan_call(sf, omf[0], omf[1], N, smf), _scan_call(sr, omr[0], omr[1], N, smr)
        cf, cr = dict(cf, ckpt=sf[-1], dy=dy[..., :E]), dict(cr, ckpt=sr[-1], dy=dy[..., E:])
        if ctx.tied_z:
            # one z for both directions: the second scan adds its dz to the first's
            z = sf[6]
            cf["dz_out"] = torch.empty(z.shape, dtype=z.dtype, device=z.device)
            cr["dz_out"], cr["dz_accumulate"] = cf["dz_out"], True
        scan_gf, scan_gr = scan_bwd_pair([cf, cr])
        gf = _core_param_grads(sf, scan_gf, cf["dbc_out"], N, rank)
        gr = _core_param_grads(sr, scan_gr, cr["dbc_out"], N, rank)
        if ctx.tied_z:
            gr = (*gr[:-1], None)  # zr is zf: its gradient is all in gf's dz
        return (*gf, *gr, None, None, None, None, None)


def _xor(a, b):
    """Composition of two flips given as (time, channel) reversal bits (they commute)."""
    return (bool(a[0]) != bool(b[0]), bool(a[1]) != bool(b[1]))


RC_MAP = (True, True)  # RC(x)[b,l,d] = x[b,L-1-l,D-1-d] (rcps.py:10-13, 37-39)
TIME_MAP = (True, False)


def rc_flip(x: torch.Tensor) -> torch.Tensor:
    """The RC action on an activation, as a materialised flip (modules without index maps)."""
    return torch.flip(x, dims=(-2, -1))


class SelectiveSSM(_FlaxModule):
    """A variation on MAMBA (selectssm.py:112-238), on MI355X kernels."""

    def __init__(self, reverse: bool = False, complement: bool = False, hidden_features: int = 16,
                 chunk_size: Optional[int] = None, n_channel_groups: Optional[int] = None,
                 dt_rank: Union[int, str] = "auto", dt_proj: bool = True, dt_min: float = 0.001,
                 dt_max: float = 0.1, regularize: bool = True, shift_l2_scale: float = 1e-7,
                 ssm_l2_scale: float = 1e-6, shift_conv_size: int = 3, activation: str = "silu",
                 diagnostics: Optional[dict] = None, recursive_scan: bool = False, min_recursion_length: int = 2,
                 recursive_split: int = 2, custom_vjp_scan: bool = False, features: Optional[int] = None,
                 device=None, generator: Optional[torch.Generator] = None):
        super().__init__()
        self.reverse = reverse
        self.complement = complement
        self.hidden_features = hidden_features
        self.chunk_size = chunk_size
        self.n_channel_groups = n_channel_groups
        self.dt_rank = dt_rank
        self.dt_proj_enabled = dt_proj
        self.dt_min = dt_min
        self.dt_max = dt_max
        self.regularize = regularize
        self.shift_l2_scale = shift_l2_scale
        self.ssm_l2_scale = ssm_l2_scale
        self.shift_conv_size = shift_conv_size
        self.activation = activation
        self.diagnostics = dict(diagnostics or {})
        self.recursive_scan = recursive_scan
        self.min_recursion_length = min_recursion_length
        self.recursive_split = recursive_split
        self.custom_vjp_scan = custom_vjp_scan
        self.generator = generator
        self.sown = {}
        self.features = None
        if features is not None:
            self._build(features, device)

    def _build(self, D, device):
        N = self.hidden_features
        R = math.ceil(D / 16) if self.dt_rank == "auto" else int(self.dt_rank)
        g = self.generator
        self.features, self.rank = D, R
        self.shift_conv = _ShiftConv(self.shift_conv_size, D, device, g)
        # A = -exp(A_log), A_log initialised to log(1..N) per channel (selectssm.py:190)
        self.A_log = torch.nn.Parameter(torch.log(torch.arange(1, N + 1, dtype=torch.float32, device=device))
                                        .repeat(D, 1))
        self.BC = Dense(D, 2 * N, device=device, generator=g)
        self.D = torch.nn.Parameter(torch.ones(D, device=device))
        lo, hi = self.dt_min, self.dt_max

        def dt_bias(n):
            r = torch.rand(n, device=device, generator=g) * (hi - lo) + lo
            return inverse_softplus(r)

        self.dt = Dense(D, R, device=device, generator=g, bias_init=None if self.dt_proj_enabled else dt_bias(R))
        if self.dt_proj_enabled:
            self.dt_proj = Dense(R, D, device=device, generator=g, bias_init=dt_bias(D))

    def _sow(self, col, name, value):
        self.sown.setdefault(col, {})[name] = value

    def _needs_intermediates(self) -> bool:
        d = self.diagnostics
        return bool(d) and any(k in d for k in ("ssm_coeffs", "ssm_residual", "ssm_output_norm"))

    def _flip(self):
        """The module's own flip of x (selectssm.py:167-168) as (time, channel) bits."""
        return (bool(self.reverse), bool(self.reverse and self.complement))

    def _maps(self, conj=None):
        """(conv map, scan output map, skip map) of the fused path.  Without ``conj``
        the conv reads x through the module's flip F, the scan writes y through F and
        the skip adds u at the output position (skip map None, the reference's
        convention).  Conjugated by a flip G, x -> G(M(G(x))), the conv reads through
        G o F, y is written through G o F and the skip's u is read at F of the scan
        position: the scan itself and every projection are unchanged, only the
        index maps move."""
        F = self._flip()
        if conj is None:
            return F, F, None
        GF = _xor(conj, F)
        return GF, GF, F

    def _prepare(self, x: torch.Tensor, projections: bool = True, conv_map=None, conv_out=None) -> dict:
        """Everything of __call__ before the scan (selectssm.py:156-228): the scan's
        operands in the scan domain, with delta before its softplus (only the conv
        output u when ``projections`` is False).  ``conv_map``: the conv's (time,
        channel) index map when not the module's own flip (a conjugation).
        ``conv_out``: the fused conv's output, already computed (for
        :meth:`_conv_fused` modules only)."""
        if self.features is None:
            self._build(x.shape[-1], x.device)
        B, L, D = x.shape
        if D != self.features:
            raise ValueError(f"x has {D} features, the module was built for {self.features}")
        N = self.hidden_features
        self.sown = {}
        diag = self.diagnostics
        if diag and "ssm_input_norm" in diag:
            self._sow("diagnostics", "ssm_input_mean", x.mean())
            self._sow("diagnostics", "ssm_input_sd", x.std(unbiased=False))

        # flip + shift_conv + activation (selectssm.py:167-185), one kernel; the
        # activation runs separately for gelu and when the raw conv output is sown
        if self.activation not in _FUSED_CONV_ACTS and self.activation != "gelu":
            raise Exception(f"Unknown activation: {self.activation}")
        coeffs = bool(diag) and "ssm_coeffs" in diag
        fused = self._conv_fused()
        cmap = self._flip() if conv_map is None else conv_map
        if conv_out is not None:
            if not fused:
                raise ValueError("conv_out is the fused conv's output; this module runs its activation apart")
            u = conv_out
        else:
            u = conv1d_act_map(x, self.shift_conv.kernel, cmap[0], cmap[1], self.activation if fused else None)
        if coeffs:
            self._sow("diagnostics", "conv_mean", u.mean())
            self._sow("diagnostics", "conv_sd", u.std(unbiased=False))
        if not fused and self.activation is not None:
            u = _activation_fn(self.activation)(u)
        if not projections:
            if self.custom_vjp_scan or self.recursive_scan:
                _check_recursion(L, self.min_recursion_length, self.recursive_split)
            else:
                resolve_chunking(L, D, self.chunk_size, self.n_channel_groups)
            if not self.dt_proj_enabled and self.rank > 1 and D % self.rank != 0:
                raise ValueError(f"dt_rank={self.rank} must divide D={D}")
            return dict(u=u)

        A = -torch.exp(self.A_log)
        BC = self.BC(u)
        Bc, Cc = BC[..., :N], BC[..., N:]
        dt = self.dt(u)
        if coeffs:
            self._sow("diagnostics", "dt_lowrank_mean", dt.mean())
            self._sow("diagnostics", "dt_lowrank_sd", dt.std(unbiased=False))
        if self.dt_proj_enabled:
            dt = self.dt_proj(dt)
        elif self.rank > 1:
            if D % self.rank != 0:
                raise ValueError(f"dt_rank={self.rank} must divide D={D}")
            dt = torch.repeat_interleave(dt, D // self.rank, dim=-1)
        if coeffs:
            dsp = F.softplus(dt)
            for k, v in (("activated_conv_mean", u.mean()), ("activated_conv_sd", u.std(unbiased=False)),
                         ("dt_mean", dsp.mean()), ("dt_sd", dsp.std(unbiased=False)), ("A_mean", A.mean()),
                         ("A_sd", A.std(unbiased=False)), ("B_sd", Bc.std(unbiased=False)),
                         ("C_sd", Cc.std(unbiased=False))):
                self._sow("diagnostics", k, v)

        # the reference's strategy dispatch (selectssm.py:223-228) and its argument checks
        if self.custom_vjp_scan or self.recursive_scan:
            _check_recursion(L, self.min_recursion_length, self.recursive_split)
        else:
            resolve_chunking(L, D, self.chunk_size, self.n_channel_groups)
        return dict(u=u, delta=dt, A=A, B=Bc, C=Cc, D=self.D)

    def _conv_fused(self) -> bool:
        """Whether the conv kernel applies the activation (no raw conv output sown)."""
        d = self.diagnostics
        return self.activation in _FUSED_CONV_ACTS and not (bool(d) and "ssm_coeffs" in d)

    def _unfused_outputs(self) -> bool:
        """Diagnostics that sow values the fused epilogue never materialises."""
        d = self.diagnostics
        return bool(d) and ("ssm_residual" in d or "ssm_output_norm" in d)

    def _finish(self, y_pre_gate: Optional[torch.Tensor]) -> None:
        if self.regularize:
            kernels = [self.BC.kernel, self.dt.kernel] + ([self.dt_proj.kernel] if self.dt_proj_enabled else [])
            reg = (self.shift_l2_scale * torch.sum(self.shift_conv.kernel ** 2)
                   + self.ssm_l2_scale * sum(torch.sum(k ** 2) for k in kernels))
            self._sow("losses", "ssm_regularizer", reg)
        if y_pre_gate is not None and self.diagnostics and "ssm_output_norm" in self.diagnostics:
            self._sow("diagnostics", "ssm_output_mean", y_pre_gate.mean())
            self._sow("diagnostics", "ssm_output_sd", y_pre_gate.std(unbiased=False))

    def forward(self, x: torch.Tensor, train: bool = False, gate: Optional[torch.Tensor] = None,
                gate_activation: str = "silu") -> torch.Tensor:
        """y (B, L, D) for x (B, L, D).  ``gate`` (BidirectionalMamba's z) multiplies the
        output by gate_activation(z) (selectssm.py:335-336), fused into the scan for silu."""
        fuse_gate = gate is not None and gate_activation == "silu"
        if not self._needs_intermediates():
            u = self._prepare(x, projections=False)["u"]
            y = self._core(u, gate if fuse_gate else None)
            if gate is not None and not fuse_gate:
                y = y * _activation_fn(gate_activation)(gate)
            self._finish(None)
            return y
        p = self._prepare(x)
        u = p["u"]
        if self._unfused_outputs():
            # the scan without its epilogue, so the residual and pre-gate values exist
            y = selective_scan(u, p["delta"], p["A"], p["B"], p["C"], reverse=self.reverse,
                               complement=self.complement, delta_softplus=True)
            if "ssm_residual" in self.diagnostics:
                self._sow("diagnostics", "ssm_residual_mean", y.mean())
                self._sow("diagnostics", "ssm_residual_sd", y.std(unbiased=False))
            y = y + u * self.D  # u stays in the scan domain (selectssm.py:238)
            self._finish(y)
            return y if gate is None else y * _activation_fn(gate_activation)(gate)
        y = selective_scan(u, p["delta"], p["A"], p["B"], p["C"], D=p["D"], z=gate if fuse_gate else None,
                           reverse=self.reverse, complement=self.complement, delta_softplus=True)
        if gate is not None and not fuse_gate:
            y = y * _activation_fn(gate_activation)(gate)
        self._finish(None)
        return y

    def _core_args(self, u, z):
        return (u, self.A_log, self.BC.kernel, self.BC.bias, self.dt.kernel, self.dt.bias,
                self.dt_proj.kernel if self.dt_proj_enabled else None,
                self.dt_proj.bias if self.dt_proj_enabled else None, self.D, z)

    def _core(self, u: torch.Tensor, z: Optional[torch.Tensor] = None, conj=None) -> torch.Tensor:
        """Projections + scan from the conv output u in one autograd node (see _SSMCoreFn),
        with the output and skip maps of :meth:`_maps`."""
        zz = None if z is None else as_rows(z, u.dtype)[0]
        args = self._core_args(u, zz)
        _, om, sm = self._maps(conj)
        return _SSMCoreFn.apply(*args, self.hidden_features, self.rank, om[0], om[1], sm, needs_grad(*args))

    def _conj_fusable(self, gate_activation="silu") -> bool:
        """Whether a conjugated call runs on index maps alone (the fused path: no
        diagnostics that need intermediates, a fused conv activation and gate)."""
        return (not self._needs_intermediates() and self.activation in _FUSED_CONV_ACTS
                and gate_activation == "silu")

    def forward_conj(self, x: torch.Tensor, conj, train: bool = False, gate: Optional[torch.Tensor] = None,
                     gate_activation: str = "silu") -> torch.Tensor:
        """G(self(G(x))) for a flip G = ``conj`` ((time, channel) reversal bits), with
        ``gate`` applied at the output positions: G(self(G(x)) * act(G(gate)))
        = G(self(G(x))) * act(gate).  No activation is flipped: the conv reads x
        through G o F, the scan writes through G o F and takes the skip's u at F of
        the scan position (:meth:`_maps`).  Falls back to materialised flips where
        the fused path does not apply."""
        if not self._conj_fusable(gate_activation if gate is not None else "silu"):
            flip = lambda t: torch.flip(t, dims=[d for d, on in ((-2, conj[0]), (-1, conj[1])) if on])
            g = None if gate is None else flip(gate)
            return flip(self.forward(flip(x), train, gate=g, gate_activation=gate_activation))
        if self.features is None:
            self._build(x.shape[-1], x.device)
        cmap, _, _ = self._maps(conj)
        u = self._prepare(x, projections=False, conv_map=cmap)["u"]
        y = self._core(u, gate, conj)
        self._finish(None)
        return y

    def forward_rc(self, x: torch.Tensor, train: bool = False) -> torch.Tensor:
        """RC(self(RC(x))): this module as the inner module of an RCPSWrapper's
        antisense half (rcps.py:61-72), on index maps (:meth:`forward_conj`)."""
        return self.forward_conj(x, RC_MAP, train)


class RMSNorm(torch.nn.Module):
    """flax.linen.RMSNorm (epsilon 1e-6, learned scale), computed in float32."""

    def __init__(self, D, eps=1e-6, device=None):
        super().__init__()
        self.eps = eps
        self.scale = torch.nn.Parameter(torch.ones(D, device=device))

    def forward(self, x, flip: bool = False):
        """``flip``: the per-channel scale reversed (the norm conjugated by a channel flip)."""
        # x * rsqrt(mean(x^2) + eps) * scale over the last axis, as one op
        y = F.rms_norm(x.float(), (x.shape[-1],), self.scale.flip(0) if flip else self.scale, self.eps)
        return y.to(x.dtype)


def _norm_forward_rc(self, x):
    """RC(norm(RC(x))) = the norm with its per-channel parameters reversed."""
    return self.forward(x, flip=True)


class LayerNorm(torch.nn.Module):
    """flax.linen.LayerNorm (epsilon 1e-6, learned scale and bias), computed in float32."""

    def __init__(self, D, eps=1e-6, device=None):
        super().__init__()
        self.eps = eps
        self.scale = torch.nn.Parameter(torch.ones(D, device=device))
        self.bias = torch.nn.Parameter(torch.zeros(D, device=device))

    def forward(self, x, flip: bool = False):
        s, b = (self.scale.flip(0), self.bias.flip(0)) if flip else (self.scale, self.bias)
        return F.layer_norm(x.float(), (x.shape[-1],), s, b, self.eps).to(x.dtype)


class GroupNorm(torch.nn.Module):
    """flax.linen.GroupNorm (32 groups over the feature axis, epsilon 1e-6)."""

    def __init__(self, D, groups=32, eps=1e-6, device=None):
        super().__init__()
        if D % groups != 0:
            raise ValueError(f"GroupNorm: {groups} groups must divide {D} features")
        self.groups, self.eps = groups, eps
        self.scale = torch.nn.Parameter(torch.ones(D, device=device))
        self.bias = torch.nn.Parameter(torch.zeros(D, device=device))

    def forward(self, x, flip: bool = False):
        """``flip``: scale and bias reversed.  A channel flip maps group g onto group
        groups-1-g with the same statistics, so that is the whole conjugation."""
        B, L, D = x.shape
        xf = x.float().reshape(B, L, self.groups, D // self.groups)
        # statistics over every non-batch axis within a group (time and the group's features)
        mean = xf.mean(dim=(1, 3), keepdim=True)
        var = xf.var(dim=(1, 3), keepdim=True, unbiased=False)
        s, b = (self.scale.flip(0), self.bias.flip(0)) if flip else (self.scale, self.bias)
        y = ((xf - mean) * torch.rsqrt(var + self.eps)).reshape(B, L, D) * s + b
        return y.to(x.dtype)


RMSNorm.forward_rc = _norm_forward_rc
LayerNorm.forward_rc = _norm_forward_rc
GroupNorm.forward_rc = _norm_forward_rc


class BatchNorm(torch.nn.Module):
    """flax.linen.BatchNorm over (batch, time), momentum as Flax (running = m*running + (1-m)*batch)."""

    def __init__(self, D, momentum=0.9, eps=1e-5, device=None):
        super().__init__()
        self.momentum, self.eps = momentum, eps
        self.scale = torch.nn.Parameter(torch.ones(D, device=device))
        self.bias = torch.nn.Parameter(torch.zeros(D, device=device))
        self.register_buffer("mean", torch.zeros(D, device=device))
        self.register_buffer("var", torch.ones(D, device=device))

    def forward(self, x, train=False):
        xf = x.float()
        if train:
            mean = xf.mean(dim=(0, 1))
            var = xf.var(dim=(0, 1), unbiased=False)
            with torch.no_grad():
                self.mean.mul_(self.momentum).add_((1 - self.momentum) * mean)
                self.var.mul_(self.momentum).add_((1 - self.momentum) * var)
        else:
            mean, var = self.mean, self.var
        return ((xf - mean) * torch.rsqrt(var + self.eps) * self.scale + self.bias).to(x.dtype)


class BidirectionalMamba(_FlaxModule):
    """Bidirectional Mamba block (selectssm.py:240-364), on MI355X kernels."""

    def __init__(self, hidden_features: int, expansion_factor: float, dt_rank: Union[int, str] = "auto",
                 complement: bool = False, tie_in_proj: bool = False, tie_gate: bool = False,
                 concatenate_fwd_rev: bool = True, activation: str = "silu", norm_type: str = "rms",
                 bn_momentum: float = 0.9, mlp_layer: bool = False, dense_expansion: int = 2,
                 mlp_dropout_rate: float = 0.1, ssm_args: Optional[dict] = None, diagnostics: Optional[dict] = None,
                 features: Optional[int] = None, device=None, generator: Optional[torch.Generator] = None):
        super().__init__()
        self.hidden_features = hidden_features
        self.expansion_factor = expansion_factor
        self.dt_rank = dt_rank
        self.complement = complement
        self.tie_in_proj = tie_in_proj
        self.tie_gate = tie_gate
        self.concatenate_fwd_rev = concatenate_fwd_rev
        self.activation = activation
        self.norm_type = norm_type
        self.bn_momentum = bn_momentum
        self.mlp_layer = mlp_layer
        self.dense_expansion = dense_expansion
        self.mlp_dropout_rate = mlp_dropout_rate
        self.ssm_args = dict(ssm_args or {})
        self.diagnostics = dict(diagnostics or {})
        self.generator = generator
        self.sown = {}
        self.features = None
        _activation_fn(activation)  # unknown names raise at construction, as at the reference's first call
        if features is not None:
            self._build(features, device)

    def _build(self, D, device):
        g = self.generator
        self.features = D
        R = math.ceil(D / 16) if self.dt_rank == "auto" else self.dt_rank
        if self.norm_type == "batch":
            self.BatchNorm_0 = BatchNorm(D, self.bn_momentum, device=device)
        elif self.norm_type == "layer":
            self.LayerNorm_0 = LayerNorm(D, device=device)
        elif self.norm_type == "group":
            self.GroupNorm_0 = GroupNorm(D, device=device)
        elif self.norm_type == "rms":
            self.RMSNorm_0 = RMSNorm(D, device=device)
        ED = math.ceil(self.expansion_factor * D)
        self.ED = ED
        n_in = 1 if self.tie_in_proj else 2
        n_gate = 1 if self.tie_gate else 2
        self.in_proj = Dense(D, (n_in + n_gate) * ED, device=device, generator=g)
        self.ssm_fwd = SelectiveSSM(hidden_features=self.hidden_features, reverse=False, dt_rank=R,
                                    diagnostics=self.diagnostics, **self.ssm_args, features=ED, device=device,
                                    generator=g)
        self.ssm_rev = SelectiveSSM(hidden_features=self.hidden_features, reverse=True, complement=self.complement,
                                    dt_rank=R, diagnostics=self.diagnostics, **self.ssm_args, features=ED,
                                    device=device, generator=g)
        self.out_proj = Dense(2 * ED if self.concatenate_fwd_rev else ED, D, device=device, generator=g)
        if self.mlp_layer:
            self.mlp = Dense(D, self.dense_expansion * D, device=device, generator=g)
            self.mlp_proj = Dense(self.dense_expansion * D, D, device=device, generator=g)

    def forward(self, x: torch.Tensor, train: bool = False) -> torch.Tensor:
        return self._run(x, train, rc=False)

    def forward_rc(self, x: torch.Tensor, train: bool = False) -> torch.Tensor:
        """RC(self(RC(x))): this block as the inner module of an RCPSWrapper's antisense
        half (rcps.py:61-72), without flipping any activation.  With x' = RC(x):
          * norm(x') = RC(norm~(x)), norm~ with its per-channel parameters reversed;
          * in_proj(RC(n)) = T(n @ W~ + b), W~ = in_proj's kernel with its input rows
            reversed, T the time reversal: every in_proj column block arrives
            time-reversed and in its own channel order;
          * each SSM therefore runs conjugated by T (SelectiveSSM._maps), its gate at
            its output positions;
          * RC(concat(..) @ W_out + b_out) = T(concat(..)) @ W^ + b^ with W^, b^ the
            output columns (and bias) reversed; the residual RC(x') = x; the MLP
            conjugates the same way (input rows, then output columns).
        Only parameters are permuted.  BatchNorm (running statistics) and the unfused
        diagnostics paths fall back to materialised flips."""
        if self.norm_type == "batch" or self.diagnostics:
            return rc_flip(self._run(rc_flip(x), train, rc=False))
        return self._run(x, train, rc=True)

    def _run(self, x: torch.Tensor, train: bool, rc: bool) -> torch.Tensor:
        if self.features is None:
            self._build(x.shape[-1], x.device)
        activate = _activation_fn(self.activation)
        skip = x
        if self.norm_type == "batch":
            x = self.BatchNorm_0(x, train)
        elif self.norm_type == "layer":
            x = self.LayerNorm_0(x, flip=rc)
        elif self.norm_type == "group":
            x = self.GroupNorm_0(x, flip=rc)
        elif self.norm_type == "rms":
            x = self.RMSNorm_0(x, flip=rc)
        ED = self.ED
        n_in = 1 if self.tie_in_proj else 2
        conj = TIME_MAP if rc else None
        # in_proj, then jnp.split at [ED, n_in*ED, (n_in+1)*ED] (selectssm.py:319-321)
        n_gate = 1 if self.tie_gate else 2
        blocks = self.in_proj.forward_split(x, [ED] * (n_in + n_gate), flip_in=rc)
        xf, zf = blocks[0], blocks[n_in]
        xr = xf if self.tie_in_proj else blocks[1]
        zr = zf if self.tie_gate else blocks[n_in + 1]
        # the gate of selectssm.py:335-336 is applied inside each SSM's scan
        # epilogue; xf, xr, zf, zr are read in place from in_proj's output
        if (self.concatenate_fwd_rev and self.activation == "silu" and not self.ssm_fwd._unfused_outputs()
                and not self.ssm_rev._unfused_outputs()):
            f, r = self.ssm_fwd, self.ssm_rev
            if f._needs_intermediates() or r._needs_intermediates():
                assert not rc  # forward_rc takes the materialised flips for diagnostics
                pf = f._prepare(xf)
                pr = r._prepare(xr)
                pf["z"], pr["z"] = zf, zr
                # both directions straight into the concatenated output (selectssm.py:335)
                x = bidirectional_selective_scan(pf, pr, complement=self.complement, delta_softplus=True)
            else:
                mf, mr = f._maps(conj), r._maps(conj)
                cf = cr = None
                if xr is xf and f._conv_fused() and r._conv_fused():
                    # tied in_proj block: both convs in one node, whose backward sums
                    # their x-gradients inside the second conv kernel
                    cf, cr = conv1d_act_pair(xf, f.shift_conv.kernel, r.shift_conv.kernel, mf[0], mr[0],
                                             f.activation, r.activation)
                uf = f._prepare(xf, projections=False, conv_map=mf[0], conv_out=cf)["u"]
                ur = r._prepare(xr, projections=False, conv_map=mr[0], conv_out=cr)["u"]
                io = uf.dtype
                args = (*f._core_args(uf, as_rows(zf, io)[0]), *r._core_args(ur, as_rows(zr, io)[0]))
                # tied gate: one z for both directions, whose dz the second scan backward adds to
                x = _PairCoreFn.apply(*args, f.hidden_features, f.rank, (mf[1:], mr[1:]), needs_grad(*args),
                                      zr is zf)
            f._finish(None)
            r._finish(None)
        elif rc:
            yf = self.ssm_fwd.forward_conj(xf, TIME_MAP, train, gate=zf, gate_activation=self.activation)
            yr = self.ssm_rev.forward_conj(xr, TIME_MAP, train, gate=zr, gate_activation=self.activation)
            x = torch.cat([yf, yr], dim=-1) if self.concatenate_fwd_rev else yf + yr
        else:
            yf = self.ssm_fwd(xf, train, gate=zf, gate_activation=self.activation)
            yr = self.ssm_rev(xr, train, gate=zr, gate_activation=self.activation)
            x = torch.cat([yf, yr], dim=-1) if self.concatenate_fwd_rev else yf + yr
        x = self.out_proj(x, flip_out=rc)
        x = skip + x
        if self.mlp_layer:
            skip = x
            x = self.mlp(x, flip_in=rc)
            x = F.dropout(x, self.mlp_dropout_rate, training=train)
            x = activate(x)
            x = self.mlp_proj(x, flip_out=rc)
            x = F.dropout(x, self.mlp_dropout_rate, training=train)
            x = skip + x
        return x
