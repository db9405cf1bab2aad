"""Pins the CPU oracle (oracle/ssm_oracle.py, oracle/ssm_oracle.c) without the reference.

The reference (JAX/Flax) cannot be imported here and holds no golden vectors,
so each oracle function is checked against something independent of its own
formula: a library routine (scipy.signal.lfilter, numpy.convolve), a
different closed form (explicit double sums), special cases, torch.autograd on
an independent restatement, finite differences, and the restatements of the
reference's own algorithms (chunked / recursive / custom VJP) against each
other.  Each check is chosen so a plausible slip (a dropped term, an
off-by-one in the decay product, a wrong sign, transposed operands) fails it.
"""
import math
import zlib

import numpy as np
import pytest
import scipy.signal

from oracle import ssm_oracle as O
from selectssm_amd.synthetic import make_inputs


def _rand(shape, seed, N=None):
    Bt, L, D, N = shape
    return make_inputs(Bt, L, D, N, seed=seed, dtype=np.float64)


# ------------------------------------------------------------------ forward

@pytest.mark.parametrize("seed", [0, 1, 2])
def test_forward_lti_equals_lfilter(seed):
    """Constant dt, B, C over time: each state is a first-order IIR filter of u."""
    rng = np.random.default_rng(seed)
    Bt, L, D, N = 2, 300, 5, 4
    u = rng.standard_normal((Bt, L, D))
    A = -np.exp(rng.uniform(0, np.log(16), (D, N)))
    dt_d = rng.uniform(0.01, 0.3, (Bt, D))
    Bn = rng.standard_normal((Bt, N))
    Cn = rng.standard_normal((Bt, N))
    delta = np.broadcast_to(dt_d[:, None, :], (Bt, L, D)).copy()
    Bc = np.broadcast_to(Bn[:, None, :], (Bt, L, N)).copy()
    Cc = np.broadcast_to(Cn[:, None, :], (Bt, L, N)).copy()
    y = O.scan_forward(u, delta, A, Bc, Cc)
    ref = np.zeros_like(y)
    for b in range(Bt):
        for d in range(D):
            for n in range(N):
                a = math.exp(A[d, n] * dt_d[b, d])
                h = scipy.signal.lfilter([Bn[b, n] * dt_d[b, d]], [1.0, -a], u[b, :, d])
                ref[b, :, d] += Cn[b, n] * h
    np.testing.assert_allclose(y, ref, rtol=1e-12, atol=1e-12)


def _brute_forward(u, delta, A, B, C):
    """y_t = sum_n C_t,n sum_{s<=t} (prod_{s<r<=t} a_r,n) B_s,n dt_s u_s, expanded."""
    Bt, L, D = u.shape
    N = A.shape[1]
    y = np.zeros((Bt, L, D))
    for b in range(Bt):
        for d in range(D):
            for n in range(N):
                a = np.exp(A[d, n] * delta[b, :, d])
                for t in range(L):
                    acc = 0.0
                    for s in range(t + 1):
                        acc += np.prod(a[s + 1:t + 1]) * B[b, s, n] * delta[b, s, d] * u[b, s, d]
                    y[b, t, d] += C[b, t, n] * acc
    return y


@pytest.mark.parametrize("shape", [(1, 8, 3, 2), (2, 13, 2, 3)])
def test_forward_equals_brute_force_sum(shape):
    x = _rand(shape, 3)
    y = O.scan_forward(x["u"], x["dt"], x["A"], x["B"], x["C"])
    np.testing.assert_allclose(y, _brute_forward(x["u"], x["dt"], x["A"], x["B"], x["C"]), rtol=1e-12, atol=1e-14)


def test_forward_special_cases():
    x = _rand((2, 40, 6, 4), 4)
    u, dt, A, B, C = x["u"], x["dt"], x["A"], x["B"], x["C"]
    assert np.all(O.scan_forward(u, 0 * dt, A, B, C) == 0)          # dt = 0: no input, no decay
    assert np.all(O.scan_forward(u, dt, A, 0 * B, C) == 0)           # B = 0
    # A -> -inf: a = 0, memoryless: y_t = sum_n C B dt u
    y = O.scan_forward(u, dt, np.full_like(A, -1e300), B, C)
    ref = np.einsum("bln,bln->bl", C, B)[..., None] * dt * u
    np.testing.assert_allclose(y, ref, rtol=1e-13, atol=1e-15)
    # C = e_n isolates state n: h_t = a h + B dt u, recursion unrolled by hand
    n = 2
    e = np.zeros_like(C)
    e[..., n] = 1.0
    y = O.scan_forward(u, dt, A, B, e)
    h = np.zeros((2, 6))
    for t in range(40):
        h = np.exp(A[:, n][None] * dt[:, t]) * h + B[:, t, n][:, None] * dt[:, t] * u[:, t]
        np.testing.assert_allclose(y[:, t], h, rtol=1e-13, atol=1e-15)


def test_forward_linear_and_causal():
    x = _rand((2, 50, 4, 3), 5)
    u2 = np.random.default_rng(9).standard_normal(x["u"].shape)
    f = lambda uu: O.scan_forward(uu, x["dt"], x["A"], x["B"], x["C"])
    np.testing.assert_allclose(f(2.0 * x["u"] - 3.0 * u2), 2.0 * f(x["u"]) - 3.0 * f(u2), rtol=1e-11, atol=1e-13)
    up = x["u"].copy()
    up[:, 30] += 1.0
    assert np.array_equal(f(up)[:, :30], f(x["u"])[:, :30])
    assert not np.allclose(f(up)[:, 30:], f(x["u"])[:, 30:])


def test_forward_broadcast_delta():
    x = _rand((2, 30, 5, 3), 6)
    dt1 = x["dt"][..., :1]
    y1 = O.scan_forward(x["u"], dt1, x["A"], x["B"], x["C"])
    yf = O.scan_forward(x["u"], np.repeat(dt1, 5, axis=-1), x["A"], x["B"], x["C"])
    np.testing.assert_array_equal(y1, yf)


# ----------------------------------------------------------------- backward

def _torch_forward(u, dt, A, B, C):
    """Independent restatement: cumulative-log-decay form, materialised over (t, s)."""
    import torch

    L = u.shape[1]
    la = A[None, None] * dt[..., None]                       # (B,L,D,N) log a_t
    cum = torch.cumsum(la, dim=1)                            # sum_{r<=t} log a_r
    beta = B[:, :, None, :] * (dt * u)[..., None]            # (B,L,D,N)
    # h_t = sum_{s<=t} exp(cum_t - cum_s) beta_s
    w = torch.exp(cum[:, :, None] - cum[:, None, :])         # (B,t,s,D,N)
    mask = torch.tril(torch.ones(L, L, dtype=torch.bool))[None, :, :, None, None]
    h = (torch.where(mask, w, torch.zeros_like(w)) * beta[:, None]).sum(2)
    return torch.einsum("bldn,bln->bld", h, C)


@pytest.mark.parametrize("shape,bcast", [((2, 12, 3, 4), False), ((1, 20, 5, 2), False), ((2, 9, 4, 3), True)])
def test_backward_equals_torch_autograd(shape, bcast):
    torch = pytest.importorskip("torch")
    x = make_inputs(*shape, seed=7, dtype=np.float64, delta_broadcast=bcast)
    t = {k: torch.tensor(x[k], requires_grad=True) for k in ("u", "dt", "A", "B", "C")}
    y = _torch_forward(t["u"], t["dt"].expand(*shape[:3]) if bcast else t["dt"], t["A"], t["B"], t["C"])
    np.testing.assert_allclose(y.detach().numpy(), O.scan_forward(x["u"], x["dt"], x["A"], x["B"], x["C"]),
                               rtol=1e-10, atol=1e-13)
    (y * torch.tensor(x["g"])).sum().backward()
    got = O.scan_backward(x["u"], x["dt"], x["A"], x["B"], x["C"], x["g"])
    for name, gg in zip(("u", "dt", "A", "B", "C"), got):
        np.testing.assert_allclose(gg, t[name].grad.numpy(), rtol=1e-9, atol=1e-12, err_msg=name)


def test_backward_finite_differences():
    x = _rand((1, 10, 3, 3), 8)
    keys = ("u", "dt", "A", "B", "C")
    grads = dict(zip(keys, O.scan_backward(x["u"], x["dt"], x["A"], x["B"], x["C"], x["g"])))
    loss = lambda xx: float(np.sum(O.scan_forward(*(xx[k] for k in keys)) * x["g"]))
    rng = np.random.default_rng(0)
    for k in keys:
        v = rng.standard_normal(x[k].shape)
        eps = 1e-6
        xp = dict(x)
        xm = dict(x)
        xp[k] = x[k] + eps * v
        xm[k] = x[k] - eps * v
        fd = (loss(xp) - loss(xm)) / (2 * eps)
        assert abs(fd - np.sum(grads[k] * v)) <= 1e-6 * max(1.0, abs(fd)), k


# ------------------------------------------------ reference-algorithm restatements

def test_associative_scan_equals_sequential_fold():
    rng = np.random.default_rng(1)
    for n in list(range(1, 40)) + [64, 97]:
        g = rng.uniform(0.1, 1.0, (n, 3))
        h = rng.standard_normal((n, 3))
        gs, hs = O.associative_scan(O._combine, [g, h])
        G, H = np.ones(3), np.zeros(3)
        for i in range(n):
            G, H = G * g[i], g[i] * H + h[i]
            np.testing.assert_allclose(gs[i], G, rtol=1e-13)
            np.testing.assert_allclose(hs[i], H, rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("L,cs,K", [(96, None, 1), (96, 8, 2), (96, 1, 1), (96, 96, 4), (100, None, 2), (64, 16, 8)])
def test_chunked_scan_restatement(L, cs, K):
    x = _rand((2, L, 8, 4), 10)
    ref = O.scan_forward(x["u"], x["dt"], x["A"], x["B"], x["C"])
    y64 = O.chunked_scan(x["u"], x["dt"], x["A"], x["B"], x["C"], cs, K, dtype=np.float64)
    np.testing.assert_allclose(y64, ref, rtol=1e-12, atol=1e-15)
    y32 = O.chunked_scan(x["u"], x["dt"], x["A"], x["B"], x["C"], cs, K, dtype=np.float32)
    np.testing.assert_allclose(y32, ref, rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("L,ml,sp", [(96, 2, 2), (1000, 2, 2), (64, 3, 4), (81, 2, 3), (7, 2, 2), (1, 2, 2)])
def test_recursive_scan_and_custom_vjp_restatements(L, ml, sp):
    x = _rand((2, L, 5, 3), 11)
    args = (x["u"], x["dt"], x["A"], x["B"], x["C"])
    np.testing.assert_allclose(O.recursive_scan(*args, ml, sp, dtype=np.float64), O.scan_forward(*args),
                               rtol=1e-12, atol=1e-15)
    got = O.recursive_scan_backward(*args, x["g"], ml, sp, dtype=np.float64)
    ref = O.scan_backward(*args, x["g"])
    for a, r, name in zip(got, ref, ("du", "ddt", "dA", "dB", "dC")):
        np.testing.assert_allclose(a, r, rtol=1e-11, atol=1e-14, err_msg=name)


# ------------------------------------------------------------- chunk rule (A1)

def _brute_chunk(L, K):
    b = int(math.sqrt(K * L))
    return max(c for c in range(1, L + 1) if L % c == 0 and c <= b) if L >= 2 else L


def test_chunk_rule_brute_force_and_known_values():
    from selectssm_amd.scan import resolve_chunking

    for L in range(1, 601):
        for K in range(1, 9):
            want = _brute_chunk(L, K)
            assert O.resolve_chunking(L, 8 * K, None, K)[0] == want
            assert resolve_chunking(L, 8 * K, None, K)[0] == want
    known = {1024: 32, 8192: 64, 131072: 256, 1048576: 1024, 4096: 64, 1000: 25, 96: 8}
    for L, c in known.items():
        assert O.resolve_chunking(L, 64)[0] == c
        assert resolve_chunking(L, 64)[0] == c
    assert O.resolve_chunking(96, 64, None, None) == (8, 1)


def test_chunk_rule_errors_match_reference_messages():
    from selectssm_amd.scan import resolve_chunking

    for f in (O.resolve_chunking, resolve_chunking):
        with pytest.raises(ValueError, match=r"n_channel_groups=3 must divide D=64"):
            f(96, 64, None, 3)
        with pytest.raises(ValueError, match=r"chunk_size=7 must divide L=96"):
            f(96, 64, 7, 1)


# ------------------------------------------------------ epilogue, flips, conv

def test_block_forward_reverse_skip_quirk_and_gate():
    x = _rand((2, 20, 6, 3), 12)
    u, dt, A, B, C, D, z = (x[k] for k in ("u", "dt", "A", "B", "C", "D", "z"))
    D = D * np.linspace(0.5, 1.5, 6)
    ys = O.scan_forward(u, dt, A, B, C)
    silu = z / (1 + np.exp(-z))
    # reverse: y_out[p] = y_scan[L-1-p] + u[p] * D   (u stays in the scan domain)
    got = O.ssm_block_forward(u, dt, A, B, C, Dskip=D, reverse=True)
    np.testing.assert_allclose(got, ys[:, ::-1, :] + u * D, rtol=1e-13)
    # complement: y_out[p, q] = y_scan[L-1-p, D-1-q] + u[p, q] * D[q]
    got = O.ssm_block_forward(u, dt, A, B, C, Dskip=D, z=z, reverse=True, complement=True)
    np.testing.assert_allclose(got, (ys[:, ::-1, ::-1] + u * D) * silu, rtol=1e-13)
    # the flip is an involution and equals the RC action of rcps.py:10-13
    assert np.array_equal(O.flip_domain(O.flip_domain(u, True), True), u)
    assert O.flip_domain(u, True)[1, 0, 0] == u[1, -1, -1]


def test_softplus_closed_forms():
    x = np.linspace(-30, 30, 601)
    # log(1 + e^x) where it is representable directly, x and e^x at the tails
    mid = np.abs(x) < 15
    np.testing.assert_allclose(O.softplus(x[mid]), np.log1p(np.exp(x[mid])), rtol=1e-14)
    np.testing.assert_allclose(O.softplus(x[x > 25]), x[x > 25], rtol=1e-10)
    np.testing.assert_allclose(O.softplus(x[x < -25]), np.exp(x[x < -25]), rtol=1e-10)
    # softplus' = sigmoid, by central differences
    h = 1e-6
    np.testing.assert_allclose((O.softplus(x + h) - O.softplus(x - h)) / (2 * h), O.sigmoid(x), atol=1e-8)
    # the synthetic delta is softplus(0.5 N(0,1) - 4): softplus(-4) = log(1 + e^-4)
    assert abs(O.softplus(-4.0) - 0.01814992791780973) < 1e-15


@pytest.mark.parametrize("flags", [dict(), dict(skip=1), dict(gate=1), dict(skip=1, gate=1, reverse=1),
                                   dict(skip=1, gate=1, reverse=1, complement=1), dict(softplus=1),
                                   dict(softplus=1, skip=1, gate=1, reverse=1)])
def test_block_backward_finite_differences(flags):
    x = _rand((1, 9, 4, 2), 13)
    x["D"] = x["D"] * np.linspace(0.5, 1.5, 4)
    if flags.get("softplus"):
        x["dt"] = np.log(np.expm1(x["dt"]))  # the pre-activation of the same delta
    kw = dict(Dskip=x["D"] if flags.get("skip") else None, z=x["z"] if flags.get("gate") else None,
              reverse=bool(flags.get("reverse")), complement=bool(flags.get("complement")),
              delta_softplus=bool(flags.get("softplus")))
    keys = ["u", "dt", "A", "B", "C"]
    grads = O.ssm_block_backward(x["u"], x["dt"], x["A"], x["B"], x["C"], x["g"], **kw)
    named = dict(zip(keys + ["D", "z"], grads))
    if kw["Dskip"] is not None:
        keys.append("D")
    if kw["z"] is not None:
        keys.append("z")

    def loss(xx):
        kk = dict(kw)
        if kk["Dskip"] is not None:
            kk["Dskip"] = xx["D"]
        if kk["z"] is not None:
            kk["z"] = xx["z"]
        return float(np.sum(O.ssm_block_forward(xx["u"], xx["dt"], xx["A"], xx["B"], xx["C"], **kk) * x["g"]))

    rng = np.random.default_rng(1)
    for k in keys:
        v = rng.standard_normal(x[k].shape)
        eps = 1e-6
        xp, xm = dict(x), dict(x)
        xp[k] = x[k] + eps * v
        xm[k] = x[k] - eps * v
        fd = (loss(xp) - loss(xm)) / (2 * eps)
        assert abs(fd - np.sum(named[k] * v)) <= 1e-6 * max(1.0, abs(fd)), k


def test_causal_conv1d_equals_numpy_convolve_and_fd():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((2, 30, 5))
    w = rng.standard_normal((4, 5))
    u = O.causal_conv1d(x, w)
    for b in range(2):
        for d in range(5):
            np.testing.assert_allclose(u[b, :, d], np.convolve(x[b, :, d], w[::-1, d])[:30], rtol=1e-13, atol=1e-14)
    g = rng.standard_normal(u.shape)
    dx, dw = O.conv1d_silu_backward(x, w, g)
    loss = lambda xx, ww: float(np.sum(O.conv1d_silu(xx, ww) * g))
    vx, vw = rng.standard_normal(x.shape), rng.standard_normal(w.shape)
    eps = 1e-6
    fd = (loss(x + eps * vx, w + eps * vw) - loss(x - eps * vx, w - eps * vw)) / (2 * eps)
    np.testing.assert_allclose(fd, np.sum(dx * vx) + np.sum(dw * vw), rtol=1e-6)


# --------------------------------------------------------------- C restatement

@pytest.mark.parametrize("shape,ml,sp", [((2, 96, 8, 4), 2, 2), ((2, 1000, 16, 16), 2, 2), ((1, 64, 5, 3), 3, 4),
                                         ((3, 37, 9, 16), 2, 2), ((1, 1, 4, 2), 2, 2)])
def test_c_port_matches_numpy_oracle(shape, ml, sp):
    from oracle import c_oracle

    x = make_inputs(*shape, seed=0)
    args = (x["u"], x["dt"], x["A"], x["B"], x["C"])
    y = c_oracle.scan_fwd(*args, ml, sp, nthreads=2)
    yr = O.scan_forward(*args)
    np.testing.assert_allclose(y, yr, rtol=1e-4, atol=1e-6)
    got = c_oracle.scan_bwd(*args, x["g"], ml, sp, nthreads=2)
    ref = O.scan_backward(*args, x["g"])
    for a, r, name in zip(got, ref, ("du", "ddt", "dA", "dB", "dC")):
        np.testing.assert_allclose(a, r, rtol=1e-4, atol=1e-5, err_msg=name)


@pytest.mark.parametrize("shape,ml,sp", [((2, 96, 8, 4), 2, 2), ((2, 1000, 16, 16), 1000, 2), ((1, 64, 5, 3), 3, 4),
                                         ((3, 37, 9, 16), 2, 2)])
def test_c_port_f64_matches_numpy_oracle(shape, ml, sp):
    """The float64 build of the C port agrees with the fp64 numpy restatement
    to fp64 rounding (used as the oracle at sizes numpy cannot reach)."""
    from oracle import c_oracle

    x = make_inputs(*shape, seed=1)
    args = (x["u"], x["dt"], x["A"], x["B"], x["C"])
    y = c_oracle.scan_fwd(*args, ml, sp, nthreads=2, precision="f64")
    assert y.dtype == np.float64
    np.testing.assert_allclose(y, O.scan_forward(*args), rtol=1e-11, atol=1e-13)
    got = c_oracle.scan_bwd(*args, x["g"], ml, sp, nthreads=2, precision="f64")
    ref = O.scan_backward(*args, x["g"])
    for a, r, name in zip(got, ref, ("du", "ddt", "dA", "dB", "dC")):
        np.testing.assert_allclose(a, r, rtol=1e-10, atol=1e-12, err_msg=name)


@pytest.mark.parametrize("activation", ["silu", "relu", None])
@pytest.mark.parametrize("rev,comp", [(False, False), (True, False), (True, True)])
def test_conv_act_flip_composition_and_fd(activation, rev, comp):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 17, 6))
    w = rng.standard_normal((3, 6))
    u = O.conv_act_forward(x, w, activation, rev, comp)
    # the flip is applied to x before the conv, by index: x_s[b,t,d] = x[b,L-1-t,(D-1-d)]
    xs = x[:, ::-1, ::-1] if comp else (x[:, ::-1, :] if rev else x)
    v = np.zeros_like(x)
    for t in range(17):
        for k in range(3):
            if t - 2 + k >= 0:
                v[:, t, :] += w[k] * xs[:, t - 2 + k, :]
    ref = {"silu": v / (1 + np.exp(-v)), "relu": np.maximum(v, 0), None: v}[activation]
    np.testing.assert_allclose(u, ref, rtol=1e-13, atol=1e-13)
    g = rng.standard_normal(u.shape)
    dx, dw = O.conv_act_backward(x, w, g, activation, rev, comp)
    loss = lambda xx, ww: float(np.sum(O.conv_act_forward(xx, ww, activation, rev, comp) * g))
    vx, vw = rng.standard_normal(x.shape), rng.standard_normal(w.shape)
    eps = 1e-6
    fd = (loss(x + eps * vx, w + eps * vw) - loss(x - eps * vx, w - eps * vw)) / (2 * eps)
    np.testing.assert_allclose(fd, np.sum(dx * vx) + np.sum(dw * vw), rtol=1e-6)


def _ssm_params(rng, D, N=4, K=3, R=None, dt_proj=True):
    R = R or -(-D // 16)
    p = {"shift_conv": {"kernel": rng.standard_normal((K, 1, D)) / np.sqrt(K)},
         "A_log": np.log(rng.uniform(1, 16, (D, N))),
         "BC": {"kernel": rng.standard_normal((D, 2 * N)) / np.sqrt(D), "bias": rng.standard_normal(2 * N) * 0.1},
         "D": rng.uniform(0.5, 1.5, D),
         "dt": {"kernel": rng.standard_normal((D, R)) / np.sqrt(D), "bias": rng.standard_normal(R) * 0.1 - 4}}
    if dt_proj:
        p["dt_proj"] = {"kernel": rng.standard_normal((R, D)) / np.sqrt(R), "bias": rng.standard_normal(D) * 0.1 - 4}
    return p


@pytest.mark.parametrize("complement", [False, True])
def test_selective_ssm_reverse_is_forward_on_flipped_input_plus_skip_quirk(complement):
    """SelectiveSSM(reverse) flips x, runs the forward module's body, un-flips the scan
    output and adds u*D with u left in the flipped domain (selectssm.py:167-168, 230-238):
    rev(x) = flip(fwd(flip x) - u D) + u D, u = act(conv(flip x))."""
    rng = np.random.default_rng(8)
    x = rng.standard_normal((2, 12, 5))
    p = _ssm_params(rng, 5)
    xs = O.flip_domain(x, complement)
    u = O.silu(O.causal_conv1d(xs, p["shift_conv"]["kernel"].reshape(3, 5)))
    rev = O.selective_ssm_forward(p, x, reverse=True, complement=complement, hidden_features=4)
    fwd = O.selective_ssm_forward(p, xs, hidden_features=4)
    np.testing.assert_allclose(rev, O.flip_domain(fwd - u * p["D"], complement) + u * p["D"], rtol=1e-12,
                               atol=1e-12)
    # the quirk is visible: un-flipping the skip term too would give another answer
    assert not np.allclose(rev, O.flip_domain(fwd, complement))


def test_selective_ssm_reduces_to_scan_plus_skip():
    """1-tap unit conv, no activation, dt_rank=1 without dt_proj (delta broadcast):
    y = scan(x, softplus(dt), A, B, C) + x D with dt = x @ dt.kernel + dt.bias."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((2, 10, 6))
    p = _ssm_params(rng, 6, K=1, R=1, dt_proj=False)
    p["shift_conv"]["kernel"] = np.ones((1, 1, 6))
    y = O.selective_ssm_forward(p, x, hidden_features=4, dt_rank=1, dt_proj=False, activation=None)
    BC = x @ p["BC"]["kernel"] + p["BC"]["bias"]
    dt = O.softplus(x @ p["dt"]["kernel"] + p["dt"]["bias"])
    ref = O.scan_forward(x, dt, -np.exp(p["A_log"]), BC[..., :4], BC[..., 4:]) + x * p["D"]
    np.testing.assert_allclose(y, ref, rtol=1e-12)


# ----------------------------------------------------- module-level functions

def test_norms_closed_forms_and_torch():
    """rms_norm / layer_norm (Flax RMSNorm / LayerNorm, epsilon 1e-6) on rows whose
    result is known in closed form, and against torch's fp64 library routines."""
    import torch
    import torch.nn.functional as F

    eps = 1e-6
    scale = np.array([0.5, 1.0, 2.0, -1.5, 3.0, 0.25])
    bias = np.array([0.1, -0.2, 0.3, 0.0, 1.0, -1.0])
    c = 3.0
    const = np.full((1, 1, 6), c)
    alt = np.array([[[c, -c, c, -c, c, -c]]])
    # constant row: rms = |c|; mean = c, variance 0
    np.testing.assert_allclose(O.rms_norm(const, scale), (c / math.sqrt(c * c + eps)) * scale[None, None], rtol=1e-14)
    np.testing.assert_allclose(O.layer_norm(const, scale, bias), np.broadcast_to(bias, (1, 1, 6)), atol=1e-14)
    # sign-alternating row: rms = |c|; mean 0, variance c^2
    sgn = np.array([1, -1, 1, -1, 1, -1], dtype=np.float64)
    np.testing.assert_allclose(O.rms_norm(alt, scale)[0, 0], (c / math.sqrt(c * c + eps)) * sgn * scale, rtol=1e-14)
    np.testing.assert_allclose(O.layer_norm(alt, scale, bias)[0, 0], (c / math.sqrt(c * c + eps)) * sgn * scale + bias,
                               rtol=1e-14)
    # a row with mean != 0: layer_norm centres, rms_norm does not
    rng = np.random.default_rng(21)
    x = rng.standard_normal((2, 5, 6)) + 2.0
    xt = torch.from_numpy(x)
    ref_rms = F.rms_norm(xt, (6,), torch.from_numpy(scale), eps).numpy()
    ref_ln = F.layer_norm(xt, (6,), torch.from_numpy(scale), torch.from_numpy(bias), eps).numpy()
    np.testing.assert_allclose(O.rms_norm(x, scale), ref_rms, rtol=1e-12)
    np.testing.assert_allclose(O.layer_norm(x, scale, bias), ref_ln, rtol=1e-12, atol=1e-14)
    assert not np.allclose(O.rms_norm(x, scale), ref_ln)


def test_gelu_tanh_identities_and_torch():
    """gelu_tanh: gelu(0) = 0, gelu(x) - gelu(-x) = x (the tanh term is odd),
    gelu(x) -> x for large x and -> 0 for large -x, and torch's tanh-approximate gelu in fp64."""
    import torch
    import torch.nn.functional as F

    x = np.linspace(-6.0, 6.0, 241)
    g = O.gelu_tanh(x)
    assert O.gelu_tanh(np.array([0.0]))[0] == 0.0
    np.testing.assert_allclose(g - O.gelu_tanh(-x), x, rtol=1e-13, atol=1e-14)
    np.testing.assert_allclose(O.gelu_tanh(np.array([30.0, -30.0])), [30.0, 0.0], atol=1e-12)
    np.testing.assert_allclose(g, F.gelu(torch.from_numpy(x), approximate="tanh").numpy(), rtol=1e-13, atol=1e-15)
    # and it is not the erf form (flax.linen.gelu's default is approximate=True)
    assert not np.allclose(g, F.gelu(torch.from_numpy(x)).numpy(), rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(O.activate(x, "gelu"), g, rtol=0, atol=0)


@pytest.mark.parametrize("R", [2, 6])
def test_selective_ssm_dt_proj_branch_is_composed_dense(R):
    """dt = softplus(dt_proj(dt(u))) (selectssm.py:195-210) with a non-square
    (R < D) and a square non-symmetric dt_proj: equal to one Dense whose kernel
    is dt.kernel @ dt_proj.kernel (and bias dt.bias @ dt_proj.kernel + dt_proj.bias),
    run through the dt_proj=False path with dt_rank = D (no repeat)."""
    rng = np.random.default_rng(31 + R)
    D = 6
    x = rng.standard_normal((2, 14, D))
    p = _ssm_params(rng, D, R=R)
    Wd, bd = p["dt"]["kernel"], p["dt"]["bias"]
    Wp, bp = p["dt_proj"]["kernel"], p["dt_proj"]["bias"]
    merged = {k: v for k, v in p.items() if k not in ("dt", "dt_proj")}
    merged["dt"] = {"kernel": Wd @ Wp, "bias": bd @ Wp + bp}
    y = O.selective_ssm_forward(p, x, hidden_features=4, dt_rank=R, dt_proj=True)
    ref = O.selective_ssm_forward(merged, x, hidden_features=4, dt_rank=D, dt_proj=False)
    np.testing.assert_allclose(y, ref, rtol=1e-11, atol=1e-12)
    if R == D:
        # a transposed dt_proj kernel would give another answer
        swapped = dict(p, dt_proj={"kernel": Wp.T.copy(), "bias": bp})
        assert not np.allclose(O.selective_ssm_forward(swapped, x, hidden_features=4, dt_rank=R), y)


def _bm_case(rng, Dm, E, N, tie_in, tie_gate, concat, norm, mlp, dt_proj):
    """Parameters of a BidirectionalMamba built from separately drawn sub-kernels
    (in_proj's column blocks xf, xr, zf, zr in the reference's order,
    selectssm.py:319), plus the expected output assembled from those blocks
    directly: norm -> each block's own Dense -> SelectiveSSM pair -> gate ->
    concat or sum -> out_proj -> residual (selectssm.py:306-362)."""
    ED = math.ceil(E * Dm)
    R = -(-Dm // 16)  # dt_rank 'auto' from the block's input width (selectssm.py:286-289)
    blk = {k: {"kernel": rng.standard_normal((Dm, ED)) / np.sqrt(Dm), "bias": rng.standard_normal(ED) * 0.1}
           for k in ("xf", "xr", "zf", "zr")}
    order = ["xf"] + ([] if tie_in else ["xr"]) + ["zf"] + ([] if tie_gate else ["zr"])
    p = {"in_proj": {"kernel": np.concatenate([blk[k]["kernel"] for k in order], axis=1),
                     "bias": np.concatenate([blk[k]["bias"] for k in order])},
         "ssm_fwd": _ssm_params(rng, ED, N=N, K=4, R=R, dt_proj=dt_proj),
         "ssm_rev": _ssm_params(rng, ED, N=N, K=4, R=R, dt_proj=dt_proj),
         "out_proj": {"kernel": rng.standard_normal((2 * ED if concat else ED, Dm)) / np.sqrt(ED),
                      "bias": rng.standard_normal(Dm) * 0.1}}
    if norm == "rms":
        p["RMSNorm_0"] = {"scale": rng.uniform(0.5, 1.5, Dm)}
    else:
        p["LayerNorm_0"] = {"scale": rng.uniform(0.5, 1.5, Dm), "bias": rng.standard_normal(Dm) * 0.1}
    if mlp:
        p["mlp"] = {"kernel": rng.standard_normal((Dm, 2 * Dm)) / np.sqrt(Dm), "bias": rng.standard_normal(2 * Dm) * .1}
        p["mlp_proj"] = {"kernel": rng.standard_normal((2 * Dm, Dm)) / np.sqrt(2 * Dm),
                         "bias": rng.standard_normal(Dm) * 0.1}
    return p, blk, ED, R


@pytest.mark.parametrize("tie_in,tie_gate", [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize("concat,complement,norm,mlp,dt_proj", [
    (True, True, "rms", False, True), (False, False, "layer", True, True), (True, False, "rms", False, False)])
def test_bidirectional_mamba_is_composition_of_blocks(tie_in, tie_gate, concat, complement, norm, mlp, dt_proj):
    rng = np.random.default_rng(zlib.crc32(repr((tie_in, tie_gate, concat, complement, norm, mlp, dt_proj)).encode()))
    Dm, E, N = 32, 1.5, 4
    p, blk, ED, R = _bm_case(rng, Dm, E, N, tie_in, tie_gate, concat, norm, mlp, dt_proj)
    x = rng.standard_normal((2, 12, Dm))
    got = O.bidirectional_mamba_forward(p, x, N, E, complement=complement, tie_in_proj=tie_in, tie_gate=tie_gate,
                                        concatenate_fwd_rev=concat, norm_type=norm, mlp_layer=mlp,
                                        ssm_args={"dt_proj": dt_proj})
    # expected, assembled from the named blocks (no split offsets)
    if norm == "rms":
        xn = x / np.sqrt(np.mean(x * x, -1, keepdims=True) + 1e-6) * p["RMSNorm_0"]["scale"]
    else:
        m = x.mean(-1, keepdims=True)
        xn = (x - m) / np.sqrt(((x - m) ** 2).mean(-1, keepdims=True) + 1e-6) * p["LayerNorm_0"]["scale"] \
            + p["LayerNorm_0"]["bias"]
    proj = {k: xn @ v["kernel"] + v["bias"] for k, v in blk.items()}
    xf, zf = proj["xf"], proj["zf"]
    xr = xf if tie_in else proj["xr"]
    zr = zf if tie_gate else proj["zr"]
    yf = O.selective_ssm_forward(p["ssm_fwd"], xf, hidden_features=N, dt_rank=R, dt_proj=dt_proj) * O.silu(zf)
    yr = O.selective_ssm_forward(p["ssm_rev"], xr, reverse=True, complement=complement, hidden_features=N,
                                 dt_rank=R, dt_proj=dt_proj) * O.silu(zr)
    mix = np.concatenate([yf, yr], -1) if concat else yf + yr
    ref = x + mix @ p["out_proj"]["kernel"] + p["out_proj"]["bias"]
    if mlp:
        h1 = ref @ p["mlp"]["kernel"] + p["mlp"]["bias"]
        ref = ref + O.silu(h1) @ p["mlp_proj"]["kernel"] + p["mlp_proj"]["bias"]
    np.testing.assert_allclose(got, ref, rtol=1e-11, atol=1e-12)
    # the check sees the wiring: the directions' inputs or gates exchanged give another answer
    if not tie_in or not tie_gate:
        yf2 = O.selective_ssm_forward(p["ssm_fwd"], xr, hidden_features=N, dt_rank=R, dt_proj=dt_proj) * O.silu(zr)
        yr2 = O.selective_ssm_forward(p["ssm_rev"], xf, reverse=True, complement=complement, hidden_features=N,
                                      dt_rank=R, dt_proj=dt_proj) * O.silu(zf)
        mix2 = np.concatenate([yf2, yr2], -1) if concat else yf2 + yr2
        assert not np.allclose(x + mix2 @ p["out_proj"]["kernel"] + p["out_proj"]["bias"], ref)


def test_bidirectional_mamba_dt_rank_comes_from_block_width():
    """dt_rank='auto' is ceil(d_model / 16) of the block's input, not of the SSM width
    E*d_model (selectssm.py:286-289, 325-326): with dt_proj=False the low-rank dt is
    repeated D_inner / dt_rank times, so the other choice cannot even be evaluated."""
    rng = np.random.default_rng(40)
    Dm, E, N = 32, 2.0, 4
    p, _, ED, R = _bm_case(rng, Dm, E, N, True, True, True, "rms", False, False)
    assert (R, ED) == (2, 64)
    x = rng.standard_normal((1, 8, Dm))
    y = O.bidirectional_mamba_forward(p, x, N, E, tie_in_proj=True, tie_gate=True, ssm_args={"dt_proj": False})
    assert np.isfinite(y).all()
    with pytest.raises(ValueError):
        O.bidirectional_mamba_forward(p, x, N, E, dt_rank=math.ceil(ED / 16), tie_in_proj=True, tie_gate=True,
                                      ssm_args={"dt_proj": False})


# ------------------------------------------- general index maps (RCPS conjugation)

MAPS = [(False, False), (True, False), (False, True), (True, True)]


@pytest.mark.parametrize("tr,cr", MAPS)
def test_flip_maps_against_index_loops(tr, cr):
    x = np.random.default_rng(30).standard_normal((2, 5, 4))
    got = O.flip_maps(x, tr, cr)
    for b in range(2):
        for t in range(5):
            for d in range(4):
                assert got[b, t, d] == x[b, 4 - t if tr else t, 3 - d if cr else d]
    assert np.array_equal(O.flip_maps(got, tr, cr), x)


@pytest.mark.parametrize("om", MAPS)
@pytest.mark.parametrize("sm", MAPS + [None])
def test_block_forward_general_maps_brute_force(om, sm):
    """y_out[O(t,d)] = (y_scan[t,d] + u[S(t,d)] D[col S(t,d)]) silu(z[O(t,d)]), element by
    element; S = O when no skip map is given (the reference's skip at the output position)."""
    x = _rand((2, 11, 5, 3), 14)
    u, dt, A, B, C, z = (x[k] for k in ("u", "dt", "A", "B", "C", "z"))
    Dp = np.linspace(0.5, 1.5, 5)
    got = O.ssm_block_forward(u, dt, A, B, C, Dskip=Dp, z=z, out_map=om, skip_map=sm)
    ys = O.scan_forward(u, dt, A, B, C)
    s = om if sm is None else sm
    ref = np.empty_like(ys)
    L_, Dn = 11, 5
    for b in range(2):
        for t in range(L_):
            for d in range(Dn):
                p, q = (L_ - 1 - t if om[0] else t), (Dn - 1 - d if om[1] else d)
                ts, ds = (L_ - 1 - t if s[0] else t), (Dn - 1 - d if s[1] else d)
                zz = z[b, p, q]
                ref[b, p, q] = (ys[b, t, d] + u[b, ts, ds] * Dp[ds]) * zz / (1 + np.exp(-zz))
    np.testing.assert_allclose(got, ref, rtol=1e-13, atol=1e-15)


@pytest.mark.parametrize("rev,comp", [(False, False), (True, False), (True, True)])
@pytest.mark.parametrize("G", [(True, True), (True, False)])
def test_conjugated_op_is_the_flipped_module_op(rev, comp, G):
    """Conjugating SelectiveSSM's epilogue by a flip G (the RC map of an RCPS wrapper, or
    the time reversal BidirectionalMamba's in_proj leaves behind) keeps the scan and
    moves the maps: with F the module's flip, output map G o F and skip source F give
    G(op_F(...)) with the gate read through G as well."""
    x = _rand((2, 9, 6, 3), 15)
    u, dt, A, B, C, z = (x[k] for k in ("u", "dt", "A", "B", "C", "z"))
    Dp = np.linspace(0.5, 1.5, 6)
    F = (rev, rev and comp)
    GF = (G[0] != F[0], G[1] != F[1])
    conj = O.ssm_block_forward(u, dt, A, B, C, Dskip=Dp, z=O.flip_maps(z, *G), out_map=GF, skip_map=F)
    ref = O.flip_maps(O.ssm_block_forward(u, dt, A, B, C, Dskip=Dp, z=z, reverse=rev, complement=comp), *G)
    np.testing.assert_allclose(conj, ref, rtol=1e-13, atol=1e-15)


@pytest.mark.parametrize("om,sm", [((True, False), (False, False)), ((False, True), (True, False)),
                                   ((False, False), (True, True)), ((True, True), (False, True))])
def test_block_backward_general_maps_finite_differences(om, sm):
    x = _rand((1, 8, 4, 2), 16)
    Dp = np.linspace(0.5, 1.5, 4)
    kw = dict(out_map=om, skip_map=sm)
    grads = O.ssm_block_backward(x["u"], x["dt"], x["A"], x["B"], x["C"], x["g"], Dskip=Dp, z=x["z"], **kw)
    named = dict(zip(["u", "dt", "A", "B", "C", "D", "z"], grads))
    x = dict(x, D=Dp)

    def loss(xx):
        y = O.ssm_block_forward(xx["u"], xx["dt"], xx["A"], xx["B"], xx["C"], Dskip=xx["D"], z=xx["z"], **kw)
        return float(np.sum(y * x["g"]))

    rng = np.random.default_rng(2)
    for k in ("u", "dt", "A", "B", "C", "D", "z"):
        v = rng.standard_normal(np.shape(x[k]))
        eps = 1e-6
        fd = (loss(dict(x, **{k: x[k] + eps * v})) - loss(dict(x, **{k: x[k] - eps * v}))) / (2 * eps)
        assert abs(fd - np.sum(named[k] * v)) <= 1e-6 * max(1.0, abs(fd)), k
