"""numpy oracle for the selective scan — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may use this module; the product (``selectssm_amd``) never imports it.

Two kinds of functions live here:

* fp64 closed forms (``scan_forward``, ``scan_backward``, the module epilogue and
  the causal conv).  These are the parity reference for the HIP kernels.
* fp32 restatements of the reference's own algorithms (``chunked_scan``,
  ``recursive_scan``, ``recursive_scan_backward``, ``associative_scan``).  They
  exist to pin the closed forms against the reference's algorithm structure
  (chunking, recursion, custom-VJP adjoint), since the reference (JAX/Flax)
  cannot be imported in this environment.

Every function cites the reference lines it restates.  Paths are relative to the
reference checkout (``src/selectssm/...``).

Pinning (what checks each function, in ``tests/test_oracle.py``):
  scan_forward            scipy.signal.lfilter on LTI inputs, brute-force double
                          sum, special cases (dt=0, B=0, A->-inf, C=e_n), linearity
  scan_backward           torch.autograd in fp64 on an independent torch
                          restatement, central finite differences, dot-product test
  associative_scan        sequential fold on random pairs (fp64, exact operator)
  chunked_scan            == scan_forward for many (chunk_size, K)
  recursive_scan          == scan_forward for many (min_len, split), odd leaves
  recursive_scan_backward == scan_backward for many (min_len, split)
  largest_factor_up_to    brute-force definition for all L <= 600, K <= 8
  causal_conv1d(_bwd)     numpy.convolve per channel; finite differences
  conv_act_forward/_bwd   explicit np.flip composition, relu/silu closed forms;
                          finite differences
  selective_ssm_forward   the pinned pieces above composed as selectssm.py:146-238;
                          the reverse map and skip quirk checked as an identity
                          between the reverse module and the forward module on
                          the flipped input; reduces to scan_forward + skip for
                          a unit 1-tap conv, no activation and identity dt;
                          the dt_proj branch equals one Dense with the composed
                          kernel (non-square and square non-symmetric dt_proj)
  bidirectional_mamba_forward  composition of selectssm.py:282-364, checked
                          against an expected output assembled from separately
                          drawn in_proj column blocks (every tie_in_proj /
                          tie_gate combination, concat and sum, rms and layer
                          norm, the MLP); dt_rank from the block's input width
  rms_norm, layer_norm    closed forms on constant and sign-alternating rows;
                          torch's fp64 rms_norm / layer_norm
  gelu_tanh               gelu(x) - gelu(-x) = x, asymptotes, torch's fp64
                          tanh-approximate gelu
  ssm_block_forward/_bwd  explicit np.flip composition; finite differences;
                          the general index maps (out_map, skip_map) reduce to the
                          reference's defaults and are checked element by element
                          on a brute-force loop; finite differences for all of them
  flip_maps               the four flips against explicit index loops
"""
from __future__ import annotations

import math

import numpy as np


# --------------------------------------------------------------------------
# A1: chunk-size rule (selectssm.py:24-30, 43-55)
# --------------------------------------------------------------------------

def largest_factor_up_to(b: int, n: int) -> int:
    """Largest divisor of ``n`` that is <= ``b`` (selectssm.py:24-30).

    Mirrors the reference's loop exactly, including ``n < 2 -> n``.
    """
    if n < 2:
        return n
    k = b
    while n % k != 0:
        k -= 1
    return k


def resolve_chunking(L: int, D: int, chunk_size=None, n_channel_groups=1):
    """(chunk_size, K) as ``ssm_chunked_scan`` resolves them (selectssm.py:43-55).

    Raises the same ValueErrors with the same messages.
    """
    K = n_channel_groups if n_channel_groups is not None else 1
    if D % K != 0:
        raise ValueError(f"n_channel_groups={n_channel_groups} must divide D={D}")
    if chunk_size is None:
        chunk_size = largest_factor_up_to(int(math.sqrt(K * L)), L)
    if L % chunk_size != 0:
        raise ValueError(f"chunk_size={chunk_size} must divide L={L}")
    return chunk_size, K


# --------------------------------------------------------------------------
# fp64 closed forms (Appendix A of the hot-path math)
# --------------------------------------------------------------------------

def _f64(*xs):
    return [np.asarray(x, dtype=np.float64) for x in xs]


def scan_forward(u, delta, A, B, C, h0=None, return_state=False):
    """Sequential fp64 recurrence, the reference's forward y.

    a_t = exp(A*dt_t)           (ssmrecscan.py:19-22; selectssm.py:74-75)
    b_t = B_t * dt_t * u_t      (ssmrecscan.py:24-29; selectssm.py:78)
    h_t = a_t*h_{t-1} + b_t     (ssmrecscan.py:90-94)
    y_t = sum_n C_t,n h_t,n     (selectssm.py:90; ssmrecscan.py:72)

    u: (B,L,D); delta: (B,L,D) or (B,L,1); A: (D,N); B, C: (B,L,N).
    """
    u, delta, A, B, C = _f64(u, delta, A, B, C)
    Bt, L, D = u.shape
    N = A.shape[-1]
    h = np.zeros((Bt, D, N)) if h0 is None else np.array(h0, dtype=np.float64)
    y = np.empty((Bt, L, D))
    for t in range(L):
        dt = np.broadcast_to(delta[:, t, :], (Bt, D))
        a = np.exp(A[None, :, :] * dt[:, :, None])
        h = a * h + B[:, t, None, :] * (dt * u[:, t, :])[:, :, None]
        y[:, t, :] = np.einsum("bdn,bn->bd", h, C[:, t, :])
    if return_state:
        return y, h
    return y


def scan_backward(u, delta, A, B, C, dy):
    """Closed-form adjoint of ``scan_forward`` in fp64 (ssmrecscan.py:150-160,174-175).

    With h_{-1}=0 and f_L=0:
      f_t   = C_t dy_t + a_{t+1} f_{t+1}
      du    = sum_n f dt B                        (ssmrecscan.py:156)
      dA    = sum_{b,t} f dt a_t h_{t-1}          (ssmrecscan.py:157)
      dB    = sum_d f dt u                        (ssmrecscan.py:158)
      dC    = sum_d dy h_t                        (ssmrecscan.py:159)
      ddt   = sum_n f (A a_t h_{t-1} + B u)       (ssmrecscan.py:160)
    For a broadcast dt of shape (B,L,1) the returned ddt is summed over D (the
    true gradient; the reference's custom VJP returns an un-reduced (B,L,D)).
    Returns (du, ddelta, dA, dB, dC).
    """
    u, delta, A, B, C, dy = _f64(u, delta, A, B, C, dy)
    Bt, L, D = u.shape
    N = A.shape[-1]
    dtf = np.broadcast_to(delta, (Bt, L, D))
    hprev = np.empty((L, Bt, D, N))
    alpha = np.empty((L, Bt, D, N))
    h = np.zeros((Bt, D, N))
    for t in range(L):
        a = np.exp(A[None] * dtf[:, t, :, None])
        hprev[t] = h
        alpha[t] = a
        h = a * h + B[:, t, None, :] * (dtf[:, t, :] * u[:, t, :])[:, :, None]
    du = np.empty((Bt, L, D))
    ddt = np.empty((Bt, L, D))
    dB = np.empty((Bt, L, N))
    dC = np.empty((Bt, L, N))
    dA = np.zeros((D, N))
    f_next = np.zeros((Bt, D, N))  # a_{t+1} f_{t+1}
    for t in range(L - 1, -1, -1):
        f = C[:, t, None, :] * dy[:, t, :, None] + f_next
        a = alpha[t]
        hp = hprev[t]
        ht = a * hp + B[:, t, None, :] * (dtf[:, t, :] * u[:, t, :])[:, :, None]
        dtt = dtf[:, t, :]
        du[:, t] = dtt * np.einsum("bdn,bn->bd", f, B[:, t])
        dA += np.einsum("bd,bdn->dn", dtt, f * a * hp)
        dB[:, t] = np.einsum("bdn,bd->bn", f, dtt * u[:, t])
        dC[:, t] = np.einsum("bd,bdn->bn", dy[:, t], ht)
        ddt[:, t] = np.einsum("bdn->bd", f * (A[None] * a * hp + B[:, t, None, :] * u[:, t, :, None]))
        f_next = a * f
    if delta.shape[-1] == 1 and D != 1:
        ddt = ddt.sum(axis=-1, keepdims=True)
    return du, ddt, dA, dB, dC


# --------------------------------------------------------------------------
# Module epilogue: flips, D-skip, silu(z) gate (selectssm.py:167-168, 230-238,
# 335-336; rcps.py:10-19, 37-39)
# --------------------------------------------------------------------------

def silu(x):
    x = np.asarray(x, dtype=np.float64)
    return x / (1.0 + np.exp(-x))


def silu_grad(x):
    x = np.asarray(x, dtype=np.float64)
    s = 1.0 / (1.0 + np.exp(-x))
    return s * (1.0 + x * (1.0 - s))


def softplus(x):
    """log(1 + e^x) in fp64 (selectssm.py:210, jax.nn.softplus = logaddexp(x, 0))."""
    return np.logaddexp(np.asarray(x, np.float64), 0.0)


def sigmoid(x):
    """softplus'(x)."""
    return 1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))


def flip_domain(x, complement: bool):
    """Reverse map of ``SelectiveSSM(reverse=True)`` (selectssm.py:168, 231).

    complement=True is the RC action RC(x)[b,l,d] = x[b,L-1-l,D-1-d]
    (rcps.py:10-13, 37-39).  The map is an involution.
    """
    return np.flip(x, axis=(-2, -1) if complement else -2)


def flip_maps(x, time_rev: bool, chan_rev: bool):
    """x read through an index map reversing time and/or channels:
    out[..., t, d] = x[..., L-1-t if time_rev else t, D-1-d if chan_rev else d].
    ``flip_domain`` (selectssm.py:168) and the RC action (rcps.py:10-13) are two of
    its four cases.  An involution."""
    axes = tuple(ax for ax, on in ((-2, time_rev), (-1, chan_rev)) if on)
    x = np.asarray(x, np.float64)
    return np.flip(x, axis=axes) if axes else x


def _block_maps(reverse, complement, out_map, skip_map):
    """(output map, skip source map) as (time, channel) bits: by default the module's
    flip (selectssm.py:167-168) and, for the skip, the output position itself
    (selectssm.py:238 adds u at the output position: the reverse-mode quirk)."""
    om = tuple(out_map) if out_map is not None else (bool(reverse), bool(reverse and complement))
    return om, (om if skip_map is None else tuple(skip_map))


def ssm_block_forward(u, delta, A, B, C, Dskip=None, z=None, reverse=False, complement=False,
                      delta_softplus=False, out_map=None, skip_map=None):
    """Scan + the scan-adjacent epilogue of ``SelectiveSSM``/``BidirectionalMamba``.

    u, delta, B, C are in the scan domain (already flipped when reverse=True,
    as the reference builds them from the flipped x: selectssm.py:167-210).
      y = scan(u, delta, A, B, C)                     (selectssm.py:222-228)
      y = flip(y) if reverse                          (selectssm.py:230-231)
      y = y + u * D      u NOT un-flipped (quirk)     (selectssm.py:238)
      y = y * silu(z)    BidirectionalMamba gate      (selectssm.py:335-336)
    delta_softplus: ``delta`` is the pre-activation, the scan uses softplus(delta)
    (selectssm.py:210).

    General index maps (the conjugated modules of an RCPS stack): ``out_map``
    (time, channel) places scan position (t, d) at O(t, d) of the output, and
    ``skip_map`` S reads the skip's u at S(t, d) (D of its channel):
      y_out[O(t,d)] = y_scan[t,d] + u[S(t,d)] * D[col S(t,d)],  then the gate.
    The defaults reproduce the reference: O the module's flip, S = O.
    """
    om, sm = _block_maps(reverse, complement, out_map, skip_map)
    if delta_softplus:
        delta = softplus(delta)
    y = scan_forward(u, delta, A, B, C)
    if Dskip is not None:
        y = y + flip_maps(np.asarray(u, np.float64) * np.asarray(Dskip, np.float64), *sm)
    y = flip_maps(y, *om)
    if z is not None:
        y = y * silu(z)
    return y


def ssm_block_backward(u, delta, A, B, C, dout, Dskip=None, z=None, reverse=False, complement=False,
                       delta_softplus=False, out_map=None, skip_map=None):
    """Chain rule through ``ssm_block_forward`` in fp64.

    Returns (du, ddelta, dA, dB, dC, dD, dz); dD / dz are None when unused.
    With delta_softplus, ddelta is w.r.t. the pre-activation (times sigmoid).
    """
    om, sm = _block_maps(reverse, complement, out_map, skip_map)
    dsig = None
    if delta_softplus:
        dsig = sigmoid(delta)
        delta = softplus(delta)
    u64 = np.asarray(u, np.float64)
    dout = np.asarray(dout, np.float64)
    dz = None
    if z is not None:
        pre = scan_forward(u, delta, A, B, C)
        if Dskip is not None:
            pre = pre + flip_maps(u64 * np.asarray(Dskip, np.float64), *sm)
        pre = flip_maps(pre, *om)
        dz = dout * pre * silu_grad(z)
        dy = dout * silu(z)
    else:
        dy = dout
    dys = flip_maps(dy, *om)  # the gradient at the scan positions
    du, ddt, dA, dB, dC = scan_backward(u, delta, A, B, C, dys)
    dD = None
    if Dskip is not None:
        ws = flip_maps(dys, *sm)  # the gradient reaching u[s] through the skip term read at s
        dD = np.einsum("bld,bld->d", ws, u64)
        du = du + ws * np.asarray(Dskip, np.float64)
    if dsig is not None:
        ddt = ddt * dsig
    return du, ddt, dA, dB, dC, dD, dz


# --------------------------------------------------------------------------
# Causal depthwise conv + activation (selectssm.py:170-187)
# --------------------------------------------------------------------------

def causal_conv1d(x, w):
    """u[b,l,d] = sum_k w[k,d] * x[b, l-(K-1)+k, d], zero left padding.

    Flax ``nn.Conv(features=D, feature_group_count=D, kernel_size=(K,),
    padding=[(K-1, 0)], use_bias=False)`` (selectssm.py:170-174), kernel of
    shape (K,1,D) passed here as w=(K,D).  Cross-correlation, as XLA's conv.
    """
    x, w = _f64(x, w)
    K = w.shape[0]
    Bt, L, D = x.shape
    xp = np.concatenate([np.zeros((Bt, K - 1, D)), x], axis=1)
    out = np.zeros((Bt, L, D))
    for k in range(K):
        out += w[k][None, None, :] * xp[:, k:k + L, :]
    return out


def causal_conv1d_backward(x, w, dv):
    """(dx, dw) of ``causal_conv1d`` for upstream gradient dv."""
    x, w, dv = _f64(x, w, dv)
    K = w.shape[0]
    Bt, L, D = x.shape
    xp = np.concatenate([np.zeros((Bt, K - 1, D)), x], axis=1)
    dxp = np.zeros_like(xp)
    dw = np.zeros((K, D))
    for k in range(K):
        dxp[:, k:k + L, :] += w[k][None, None, :] * dv
        dw[k] = np.einsum("bld,bld->d", dv, xp[:, k:k + L, :])
    return dxp[:, K - 1:, :], dw


def conv1d_silu(x, w):
    """silu(causal_conv1d(x, w)) (selectssm.py:170-185)."""
    return silu(causal_conv1d(x, w))


def conv1d_silu_backward(x, w, du):
    v = causal_conv1d(x, w)
    dv = np.asarray(du, np.float64) * silu_grad(v)
    return causal_conv1d_backward(x, w, dv)


def gelu_tanh(x):
    """0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))): flax.linen.gelu's default
    (approximate=True).  The closed form is pinned (identities, torch); that
    Flax's default is the tanh form lives in Flax, not in the reference (unpinned)."""
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def activate(x, activation):
    """SelectiveSSM's activation after the conv (selectssm.py:176-185) and
    BidirectionalMamba's gate activation (298-305): silu, relu, gelu or none."""
    x = np.asarray(x, np.float64)
    if activation == "silu":
        return silu(x)
    if activation == "relu":
        return np.maximum(x, 0.0)
    if activation == "gelu":
        return gelu_tanh(x)
    if activation is None or activation == "none":
        return x
    raise ValueError(activation)


def activate_grad(x, activation):
    """d activate / dx; relu'(0) = 0 as jax.nn.relu's gradient."""
    x = np.asarray(x, np.float64)
    if activation == "silu":
        return silu_grad(x)
    if activation == "relu":
        return (x > 0).astype(np.float64)
    return np.ones_like(x)


def conv_act_forward(x, w, activation="silu", reverse=False, complement=False):
    """SelectiveSSM's flip -> shift_conv -> activation (selectssm.py:167-185).

    x in its original domain; the result u is in the scan domain.
    """
    xs = flip_domain(x, complement) if reverse else np.asarray(x, np.float64)
    return activate(causal_conv1d(xs, w), activation)


def conv_act_backward(x, w, du, activation="silu", reverse=False, complement=False):
    """(dx, dw) of ``conv_act_forward``; dx in x's domain."""
    xs = flip_domain(x, complement) if reverse else np.asarray(x, np.float64)
    dv = np.asarray(du, np.float64) * activate_grad(causal_conv1d(xs, w), activation)
    dxs, dw = causal_conv1d_backward(xs, w, dv)
    return (flip_domain(dxs, complement) if reverse else dxs), dw


# --------------------------------------------------------------------------
# Modules (selectssm.py:112-364) with explicit Flax-named parameter dicts
# --------------------------------------------------------------------------

def dense(x, p):
    """flax.linen.Dense: x @ kernel + bias, kernel (in, out)."""
    y = np.asarray(x, np.float64) @ np.asarray(p["kernel"], np.float64)
    return y + np.asarray(p["bias"], np.float64) if "bias" in p else y


def selective_ssm_forward(p, x, reverse=False, complement=False, hidden_features=16, dt_rank="auto",
                          dt_proj=True, activation="silu", gate=None, gate_activation="silu", **_unused):
    """SelectiveSSM.__call__ (selectssm.py:146-238) in fp64; ``gate`` applies
    BidirectionalMamba's ``y * activate(z)`` (selectssm.py:335-336).  The chunk /
    recursion arguments do not change y and are not taken."""
    x = np.asarray(x, np.float64)
    D = x.shape[-1]
    N = hidden_features
    R = math.ceil(D / 16) if dt_rank == "auto" else dt_rank                       # 158-161
    xs = flip_domain(x, complement) if reverse else x                             # 167-168
    w = np.asarray(p["shift_conv"]["kernel"], np.float64)
    u = activate(causal_conv1d(xs, w.reshape(w.shape[0], D)), activation)          # 170-187
    A = -np.exp(np.asarray(p["A_log"], np.float64))                               # 190
    BC = dense(u, p["BC"])                                                         # 191
    Bc, Cc = BC[..., :N], BC[..., N:]
    dt = dense(u, p["dt"])                                                         # 195-197
    if dt_proj:
        dt = dense(dt, p["dt_proj"])                                               # 203-204
    elif R > 1:
        dt = np.repeat(dt, D // R, axis=-1)                                        # 206-209
    dt = softplus(dt)                                                              # 210
    y = scan_forward(u, dt, A, Bc, Cc)                                             # 222-228
    if reverse:
        y = flip_domain(y, complement)                                             # 230-231
    y = y + u * np.asarray(p["D"], np.float64)                                     # 238
    if gate is not None:
        y = y * activate(gate, gate_activation)
    return y


def rms_norm(x, scale, eps=1e-6):
    """flax.linen.RMSNorm.  The formula is pinned (closed forms, torch); the epsilon
    1e-6 is Flax's default, which the reference leaves implicit (unpinned)."""
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * np.asarray(scale, np.float64)


def layer_norm(x, scale, bias, eps=1e-6):
    """flax.linen.LayerNorm.  The formula is pinned (closed forms, torch); the epsilon
    1e-6 is Flax's default, which the reference leaves implicit (unpinned)."""
    x = np.asarray(x, np.float64)
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    return (x - m) / np.sqrt(v + eps) * np.asarray(scale, np.float64) + np.asarray(bias, np.float64)


def bidirectional_mamba_forward(p, x, hidden_features, expansion_factor, dt_rank="auto", complement=False,
                                tie_in_proj=False, tie_gate=False, concatenate_fwd_rev=True, activation="silu",
                                norm_type="rms", mlp_layer=False, ssm_args=None):
    """BidirectionalMamba.__call__ (selectssm.py:282-364) in fp64, inference mode
    (no dropout, batch statistics not updated)."""
    ssm_args = dict(ssm_args or {})
    x = np.asarray(x, np.float64)
    D = x.shape[-1]
    R = math.ceil(D / 16) if dt_rank == "auto" else dt_rank                       # 286-289
    skip = x
    if norm_type == "rms":
        x = rms_norm(x, p["RMSNorm_0"]["scale"])
    elif norm_type == "layer":
        x = layer_norm(x, p["LayerNorm_0"]["scale"], p["LayerNorm_0"]["bias"])
    elif norm_type is not None:
        raise ValueError(norm_type)
    ED = math.ceil(expansion_factor * D)                                           # 315
    n_in = 1 if tie_in_proj else 2
    n_gate = 1 if tie_gate else 2
    h = dense(x, p["in_proj"])
    xf, _xr, zf, _zr = np.split(h, [ED, n_in * ED, (n_in + 1) * ED], axis=-1)      # 319
    xr = xf if tie_in_proj else _xr                                                # 320
    zr = zf if tie_gate else _zr                                                   # 321
    yf = selective_ssm_forward(p["ssm_fwd"], xf, reverse=False, hidden_features=hidden_features, dt_rank=R,
                               gate=zf, gate_activation=activation, **ssm_args)    # 325
    yr = selective_ssm_forward(p["ssm_rev"], xr, reverse=True, complement=complement,
                               hidden_features=hidden_features, dt_rank=R, gate=zr, gate_activation=activation,
                               **ssm_args)                                         # 326
    x = np.concatenate([yf, yr], axis=-1) if concatenate_fwd_rev else yf + yr      # 335-338
    x = skip + dense(x, p["out_proj"])                                             # 345-352
    if mlp_layer:
        skip = x
        x = skip + dense(activate(dense(x, p["mlp"]), activation), p["mlp_proj"])  # 354-362
    return x


# --------------------------------------------------------------------------
# fp32 restatements of the reference's algorithms
# --------------------------------------------------------------------------

def associative_scan(fn, elems):
    """Inclusive scan along axis 0 with the odd/even recursion of
    ``jax.lax.associative_scan`` (third-party: jax>=0.4.20, pyproject.toml:12-15,
    called at selectssm.py:86 and ssmrecscan.py:68).

    Pair adjacent elements, scan the pairs recursively, then fill in the even
    positions by combining each odd prefix with the next original element.
    ``fn(left, right)`` combines an earlier prefix with a later element.
    """
    n = elems[0].shape[0]
    if n < 2:
        return list(elems)
    reduced = fn([e[0:-1:2] for e in elems], [e[1::2] for e in elems])
    odd = associative_scan(fn, reduced)
    if n % 2 == 0:
        even = fn([e[:-1] for e in odd], [e[2::2] for e in elems])
    else:
        even = fn(list(odd), [e[2::2] for e in elems])
    even = [np.concatenate([e[0:1], r], axis=0) for e, r in zip(elems, even)]
    out = []
    for ev, od in zip(even, odd):
        res = np.empty((ev.shape[0] + od.shape[0],) + ev.shape[1:], dtype=ev.dtype)
        res[0::2] = ev
        res[1::2] = od
        out.append(res)
    return out


def _combine(l, r):
    """(g_l,h_l) o (g_r,h_r) = (g_l g_r, g_r h_l + h_r) (selectssm.py:81-85; ssmrecscan.py:13-17)."""
    g_l, h_l = l
    g_r, h_r = r
    return [g_l * g_r, g_r * h_l + h_r]


def chunked_scan(u, delta, A, B, C, chunk_size=None, n_channel_groups=1, dtype=np.float32):
    """Restatement of ``ssm_chunked_scan`` (selectssm.py:37-109) in ``dtype``.

    Layout 'b (c l) (k d) -> c k l b d' (59-63); per chunk and channel group:
    alpha = exp(A dt), beta = B u dt (74-78), associative scan (86),
    hs = gs*h_init + hs (87), y = C.hs (90); carry (g_last*g_init, h_last) (91);
    sequential over chunks with init (ones, zeros) (107).
    """
    u = np.asarray(u, dtype)
    delta = np.asarray(delta, dtype)
    A = np.asarray(A, dtype)
    B = np.asarray(B, dtype)
    C = np.asarray(C, dtype)
    Bt, L, D = u.shape
    N = A.shape[-1]
    T, K = resolve_chunking(L, D, chunk_size, n_channel_groups)
    nc = L // T
    Dk = D // K
    dtf = np.broadcast_to(delta, (Bt, L, D))
    y = np.empty((Bt, L, D), dtype)
    for k in range(K):
        sl = slice(k * Dk, (k + 1) * Dk)
        Ak = A[sl]
        g = np.ones((Bt, Dk, N), dtype)
        h = np.zeros((Bt, Dk, N), dtype)
        for c in range(nc):
            ts = slice(c * T, (c + 1) * T)
            x_c = np.transpose(u[:, ts, sl], (1, 0, 2))        # l b d
            dt_c = np.transpose(dtf[:, ts, sl], (1, 0, 2))
            B_c = np.transpose(B[:, ts, :], (1, 0, 2))          # l b n
            C_c = np.transpose(C[:, ts, :], (1, 0, 2))
            dA = np.exp(np.einsum("dn,lbd->lbdn", Ak, dt_c)).astype(dtype)
            dB = np.einsum("lbn,lbd,lbd->lbdn", B_c, x_c, dt_c).astype(dtype)
            gs, hs = associative_scan(_combine, [dA, dB])
            hs = gs * h[None] + hs
            y[:, ts, sl] = np.transpose(np.einsum("lbn,lbdn->lbd", C_c, hs), (1, 0, 2))
            g = gs[-1] * g
            h = hs[-1]
    return y


def recursive_scan(u, delta, A, B, C, min_recursion_length=2, recursive_split=2, dtype=np.float32):
    """Restatement of ``ssm_recursive_scan`` (ssmrecscan.py:36-77) in ``dtype``.

    Split while len > min_recursion_length and len % recursive_split == 0 (56);
    scan the pieces in order threading (g, h) (59-65); leaves run the
    associative scan (67-73).
    """
    u = np.asarray(u, dtype)
    A = np.asarray(A, dtype)
    Bc = np.asarray(B, dtype)
    Cc = np.asarray(C, dtype)
    Bt, L, D = u.shape
    N = A.shape[-1]
    dtf = np.broadcast_to(np.asarray(delta, dtype), (Bt, L, D))
    x = np.transpose(u, (1, 0, 2))
    Bl = np.transpose(Bc, (1, 0, 2))
    Cl = np.transpose(Cc, (1, 0, 2))
    Dl = np.transpose(dtf, (1, 0, 2))

    def scan_chunk(g, h, xs, bs, cs, ds):
        n = xs.shape[0]
        if n > min_recursion_length and n % recursive_split == 0:
            m = n // recursive_split
            ys = []
            for i in range(recursive_split):
                s = slice(i * m, (i + 1) * m)
                g, h, yc = scan_chunk(g, h, xs[s], bs[s], cs[s], ds[s])
                ys.append(yc)
            return g, h, np.concatenate(ys, axis=0)
        alpha = np.exp(np.einsum("dn,lbd->lbdn", A, ds)).astype(dtype)
        beta = np.einsum("lbn,lbd,lbd->lbdn", bs, xs, ds).astype(dtype)
        gs, hs = associative_scan(_combine, [alpha, beta])
        hs = gs * h[None] + hs
        yc = np.einsum("lbn,lbdn->lbd", cs, hs)
        return gs[-1] * g, hs[-1], yc

    _, _, y = scan_chunk(np.ones((Bt, D, N), dtype), np.zeros((Bt, D, N), dtype), x, Bl, Cl, Dl)
    return np.transpose(y, (1, 0, 2))


def recursive_scan_backward(u, delta, A, B, C, dy, min_recursion_length=2, recursive_split=2,
                            dtype=np.float32):
    """Restatement of the custom-VJP backward (ssmrecscan.py:111-181) in ``dtype``.

    Recursive case (114-148): a reverse scan over the pieces computes the
    adjoint entering each piece from the right (f_alpha, 121-133, recomputing
    alpha per step), then a forward scan recurses into each piece threading
    h and accumulating dA (134-143).  Leaf (149-161): forward scan stores
    h_{t-1}, reverse scan stores f_t, then the einsums of 154-160.
    Returns (du, ddelta, dA, dB, dC) in the (B,L,*) layout (177-181).
    """
    u = np.asarray(u, dtype)
    A = np.asarray(A, dtype)
    Bc = np.asarray(B, dtype)
    Cc = np.asarray(C, dtype)
    dy = np.asarray(dy, dtype)
    Bt, L, D = u.shape
    N = A.shape[-1]
    dtf = np.broadcast_to(np.asarray(delta, dtype), (Bt, L, D))
    tr = lambda a: np.transpose(a, (1, 0, 2))

    def rec(x, bs, cs, ds, dys, h_left, fa_right):
        n = x.shape[0]
        if n > min_recursion_length and n % recursive_split == 0:
            m = n // recursive_split
            pieces = [slice(i * m, (i + 1) * m) for i in range(recursive_split)]
            # reverse scan over pieces: f_alpha entering each piece from its right
            fas = [None] * recursive_split
            fa = fa_right
            for i in range(recursive_split - 1, -1, -1):
                fas[i] = fa
                s = pieces[i]
                for t in range(m - 1, -1, -1):
                    alpha_t = np.exp(np.einsum("dn,bd->bdn", A, ds[s][t])).astype(dtype)
                    f_t = fa + np.einsum("bn,bd->bdn", cs[s][t], dys[s][t])
                    fa = f_t * alpha_t
            dA = np.zeros_like(A)
            h = h_left
            outs = []
            for i in range(recursive_split):
                s = pieces[i]
                dx_c, dA_c, dB_c, dC_c, dD_c, h = rec(x[s], bs[s], cs[s], ds[s], dys[s], h, fas[i])
                dA = dA + dA_c
                outs.append((dx_c, dB_c, dC_c, dD_c))
            cat = lambda j: np.concatenate([o[j] for o in outs], axis=0)
            return cat(0), dA, cat(1), cat(2), cat(3), h
        alpha = np.exp(np.einsum("dn,lbd->lbdn", A, ds)).astype(dtype)
        beta = np.einsum("lbn,lbd,lbd->lbdn", bs, x, ds).astype(dtype)
        C_dy = np.einsum("lbn,lbd->lbdn", cs, dys)
        hs = np.empty_like(alpha)
        h = h_left
        for t in range(n):
            hs[t] = h
            h = h * alpha[t] + beta[t]
        h_right = h
        fs = np.empty_like(alpha)
        fa = fa_right
        for t in range(n - 1, -1, -1):
            f_t = fa + C_dy[t]
            fs[t] = f_t
            fa = f_t * alpha[t]
        Delta_fs = ds[..., None] * fs
        alpha_hs = alpha * hs
        dx = np.einsum("lbdn,lbn->lbd", Delta_fs, bs)
        dA = np.einsum("lbdn,lbdn->dn", Delta_fs, alpha_hs)
        dB = np.einsum("lbdn,lbd->lbn", Delta_fs, x)
        hs_next = np.concatenate([hs[1:], h_right[None]], axis=0)
        dC = np.einsum("lbd,lbdn->lbn", dys, hs_next)
        dDelta = np.einsum("lbdn,lbdn->lbd", fs, A[None, None] * alpha_hs
                           + np.einsum("lbn,lbd->lbdn", bs, x))
        return dx, dA, dB, dC, dDelta, h_right

    z = np.zeros((Bt, D, N), dtype)
    dx, dA, dB, dC, dD, _ = rec(tr(u), tr(Bc), tr(Cc), tr(dtf), tr(dy), z, z)
    return tr(dx), tr(dD), dA, tr(dB), tr(dC)
