"""Causal depthwise conv1d + activation: the step before the scan.

``conv1d_act`` is SelectiveSSM's flip -> ``shift_conv`` -> activation
(selectssm.py:167-185) as one HIP kernel pair (``ssm_conv_fwd`` /
``ssm_conv_bwd``).  The flip is an index map inside the kernels: x is given in
its original domain, u comes back in the scan domain (the domain the scan and
the Dense projections of SelectiveSSM see), and dx in x's domain.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib as L
from .scan import _IO_DTYPES, _ptr, _scratch, _stream, as_rows, row_stride

_ACTS = {None: L.SSM_ACT_NONE, "none": L.SSM_ACT_NONE, "silu": L.SSM_ACT_SILU, "relu": L.SSM_ACT_RELU}


def _act_code(activation):
    if activation not in _ACTS:
        # the reference raises for an unknown activation name (selectssm.py:184-185)
        raise Exception(f"Unknown activation: {activation}")
    return _ACTS[activation]


def _conv_desc(x, K, reverse, complement, activation, accumulate=False):
    """``reverse`` / ``complement``: time and channel reversal of x's index map, independently;
    ``accumulate``: the backward adds to dx (SSM_ACCUMULATE)."""
    Bt, Ln, D = x.shape
    flags = L.SSM_ACCUMULATE if accumulate else 0
    if reverse:
        flags |= L.SSM_REVERSE
    if complement:
        flags |= L.SSM_COMPLEMENT
    ld = row_stride(x)
    if ld is None:
        raise ValueError("x must be contiguous or a column slice of a contiguous (B, L, W) tensor")
    return L.SsmConvDesc(Bt, Ln, D, int(K), _IO_DTYPES[x.dtype], flags, _act_code(activation), ld)


def _weight(w, D):
    w = w.reshape(w.shape[0], -1) if w.dim() == 3 else w  # Flax (K, 1, D) kernel
    if w.dim() != 2 or w.shape[1] != D:
        raise ValueError(f"conv kernel must be (K, D) or (K, 1, D) with D={D}, got {tuple(w.shape)}")
    return w


def conv_fwd(x, w, reverse=False, complement=False, activation="silu"):
    """u = act(conv(x_s, w)) in the scan domain (``ssm_conv_fwd``); x may be a row-strided slice."""
    desc = _conv_desc(x, w.shape[0], reverse, complement, activation)
    u = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    L.check(L.lib().ssm_conv_fwd(_stream(), ctypes.byref(desc), _ptr(x), _ptr(w), _ptr(u)))
    return u


def conv_bwd(x, w, du, reverse=False, complement=False, activation="silu", need_dx=True, need_dw=True,
             dx_out=None, accumulate=False):
    """(dx, dw) of :func:`conv_fwd` (``ssm_conv_bwd``); either may be skipped (None).
    ``dx_out``: the (B, L, D) array to write dx into, or with ``accumulate`` to add it to."""
    if accumulate and (dx_out is None or not need_dx):
        raise ValueError("accumulate needs dx_out")
    desc = _conv_desc(x, w.shape[0], reverse, complement, activation, accumulate)
    lib = L.lib()
    if dx_out is not None and (dx_out.shape != x.shape or dx_out.dtype != x.dtype or not dx_out.is_contiguous()):
        raise ValueError("dx_out must be a contiguous array of x's shape and dtype")
    dx = (dx_out if dx_out is not None else torch.empty(x.shape, dtype=x.dtype, device=x.device)) if need_dx else None
    dw = torch.empty_like(w) if need_dw else None
    ws = _scratch(L.size_query(lib.ssm_conv_bwd_workspace_bytes, desc), x.device) if need_dw else None
    L.check(lib.ssm_conv_bwd(_stream(), ctypes.byref(desc), _ptr(x), _ptr(w), _ptr(du), _ptr(dx), _ptr(dw),
                             _ptr(ws)))
    return dx, dw


class ConvActFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, reverse, complement, activation):
        ctx.save_for_backward(x, w)
        ctx.cfg = (reverse, complement, activation)
        return conv_fwd(x, w, reverse, complement, activation)

    @staticmethod
    def backward(ctx, du):
        x, w = ctx.saved_tensors
        dx, dw = conv_bwd(x, w, du.to(x.dtype).contiguous(), *ctx.cfg, need_dx=ctx.needs_input_grad[0],
                          need_dw=ctx.needs_input_grad[1])
        return dx, dw, None, None, None


class ConvActPairFn(torch.autograd.Function):
    """Two convs of one input x (BidirectionalMamba with tie_in_proj feeds xf to
    both directions, selectssm.py:320): the backward writes the first conv's dx
    and adds the second's to it in its kernel (SSM_ACCUMULATE), instead of two dx
    arrays summed afterwards.  The sum is the same: one fp32 addition per element."""

    @staticmethod
    def forward(ctx, x, w1, w2, cfg1, cfg2):
        ctx.save_for_backward(x, w1, w2)
        ctx.cfg = (cfg1, cfg2)
        return conv_fwd(x, w1, *cfg1), conv_fwd(x, w2, *cfg2)

    @staticmethod
    def backward(ctx, du1, du2):
        x, w1, w2 = ctx.saved_tensors
        cfg1, cfg2 = ctx.cfg
        need_dx = ctx.needs_input_grad[0]
        dx = None
        dw = []
        for du, w, cfg, need_dw in ((du1, w1, cfg1, ctx.needs_input_grad[1]), (du2, w2, cfg2, ctx.needs_input_grad[2])):
            if du is None or not (need_dx or need_dw):
                dw.append(None)
                continue
            d, g = conv_bwd(x, w, du.to(x.dtype).contiguous(), *cfg, need_dx=need_dx, need_dw=need_dw, dx_out=dx,
                            accumulate=dx is not None)
            dx = d if need_dx else None
            dw.append(g)
        return dx, dw[0], dw[1], None, None


def conv1d_act_pair(x, w1, w2, map1, map2, activation1="silu", activation2="silu"):
    """The two convs of one input, :func:`conv1d_act_map` with (time, channel) maps
    ``map1`` and ``map2``, whose x-gradients are summed inside the second backward kernel."""
    if x.dim() != 3:
        raise ValueError(f"x must be (B, L, D), got shape {tuple(x.shape)}")
    if not (x.is_cuda and w1.is_cuda and w2.is_cuda):
        raise ValueError("conv1d_act inputs must be GPU tensors (there is no CPU path)")
    if x.dtype not in _IO_DTYPES:
        raise TypeError(f"conv1d_act supports float32 and bfloat16 activations, got {x.dtype}")
    _act_code(activation1)
    _act_code(activation2)
    D = x.shape[-1]
    w1 = _weight(w1, D).to(torch.float32).contiguous()
    w2 = _weight(w2, D).to(torch.float32).contiguous()
    cfg1 = (bool(map1[0]), bool(map1[1]), activation1)
    cfg2 = (bool(map2[0]), bool(map2[1]), activation2)
    return ConvActPairFn.apply(as_rows(x, x.dtype)[0], w1, w2, cfg1, cfg2)


def conv1d_act(x, w, reverse=False, complement=False, activation="silu"):
    """SelectiveSSM's flip + causal depthwise conv + activation (selectssm.py:167-185).

    x: (B, L, D) float32 / bfloat16 GPU tensor in its original domain.
    w: the ``shift_conv`` kernel, (K, 1, D) as Flax stores it, or (K, D); float32.
    Returns u (B, L, D) in the scan domain: u[b,t,d] = act(sum_k w[k,d] x_s[b,t-(K-1)+k,d])
    with x_s = x, or x flipped in time (and in channels with ``complement``) when
    ``reverse``.  ``activation``: "silu" (the reference's default), "relu" or None.
    """
    if complement and not reverse:
        complement = False  # the reference only looks at complement when reverse (selectssm.py:116, 167-168)
    return conv1d_act_map(x, w, reverse, complement, activation)


def conv1d_act_map(x, w, time_rev=False, chan_rev=False, activation="silu"):
    """:func:`conv1d_act` with x read through any of the four flips of its (time,
    channel) index map, independently: x_s[b,t,d] = x[b, L-1-t if time_rev else t,
    D-1-d if chan_rev else d].  The module conjugations (an RCPS wrapper's RC map
    composed with SelectiveSSM's own flip) need the channel-only map as well."""
    if x.dim() != 3:
        raise ValueError(f"x must be (B, L, D), got shape {tuple(x.shape)}")
    if not (x.is_cuda and w.is_cuda):
        raise ValueError("conv1d_act inputs must be GPU tensors (there is no CPU path)")
    if x.dtype not in _IO_DTYPES:
        raise TypeError(f"conv1d_act supports float32 and bfloat16 activations, got {x.dtype}")
    _act_code(activation)
    w = _weight(w, x.shape[-1]).to(torch.float32).contiguous()
    return ConvActFn.apply(as_rows(x, x.dtype)[0], w, bool(time_rev), bool(chan_rev), activation)
