"""Time-split scans (a row's time axis in segments joined by carries) on the GPU.

* forced segment counts against the fp64 oracle, every epilogue flag, fp32 and
  bf16, delta broadcast, ragged last segments (rtol 1e-4 / atol 1e-5);
* the automatic split of a long row against the fp64 oracle;
* split and unsplit runs of the same inputs agree (rtol 1e-4 / atol 1e-5);
* the config-3 shape (B=1, L=2^20, D=1024, N=16), split automatically into 16
  segments: exact linearity, agreement with the unsplit run, and channels 0-15
  and 1008-1023 against the float64 build of the C port of the reference's
  algorithm, run as one sequential pass (min_recursion_length = L).  dA there
  is a sum over 2^20 steps; float64 keeps the oracle's own rounding out of
  the comparison.
"""
import numpy as np
import pytest

from oracle import ssm_oracle as O
from selectssm_amd.synthetic import make_inputs

from test_gpu_scan import RTOL, ATOL, _close, _cuda, _oracle

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def _run(inp, flags=(), dtype=torch.float32, segments=0):
    from selectssm_amd import selective_scan

    t = {k: _cuda(v) for k, v in inp.items()}
    for k in ("u", "dt", "B", "C", "z"):
        t[k] = t[k].to(dtype).requires_grad_(True)
    t["A"].requires_grad_(True)
    t["D"].requires_grad_(True)
    y = selective_scan(t["u"], t["dt"], t["A"], t["B"], t["C"], D=t["D"] if "skip" in flags else None,
                       z=t["z"] if "gate" in flags else None, reverse="reverse" in flags,
                       complement="complement" in flags, segments=segments, delta_softplus="softplus" in flags)
    y.backward(t["g"].to(dtype))
    torch.cuda.synchronize()
    return y, {k: t[k].grad for k in ("u", "dt", "A", "B", "C", "D", "z")}


FLAGS = [(), ("skip",), ("gate",), ("reverse",), ("reverse", "complement", "skip", "gate"), ("reverse", "skip")]


@pytest.mark.parametrize("shape,segments", [
    ((2, 300, 40, 5), 4),      # 96-step segments, last one 12 steps
    ((1, 1000, 70, 16), 7),    # ragged channel block, 160-step segments
    ((2, 96, 8, 4), 3),        # 32-step segments (one tile each)
    ((3, 257, 33, 2), 9),      # N=2, last segment a single step
])
@pytest.mark.parametrize("flags", FLAGS, ids=lambda f: "+".join(f) or "plain")
def test_forced_segments_match_oracle(shape, segments, flags):
    print(f"segments={segments} shape={shape} flags={flags}", flush=True)
    inp = make_inputs(*shape, seed=11)
    y, g = _run(inp, flags, segments=segments)
    yr, gr = _oracle(inp, flags)
    _close("y", y, yr)
    for k in ("u", "dt", "A", "B", "C"):
        _close(f"d{k}", g[k], gr[k])
    if "skip" in flags:
        _close("dD", g["D"], gr["D"])
    if "gate" in flags:
        _close("dz", g["z"], gr["z"])


def test_forced_segments_delta_broadcast():
    inp = make_inputs(2, 200, 24, 4, seed=5, delta_broadcast=True)
    y, g = _run(inp, segments=5)
    yr, gr = _oracle(inp)
    _close("y", y, yr)
    for k in ("u", "dt", "A", "B", "C"):
        _close(f"d{k}", g[k], gr[k])


def test_forced_segments_bf16():
    inp = make_inputs(2, 512, 64, 16, seed=8)
    bf = {k: (torch.from_numpy(v).to(torch.bfloat16).float().numpy().astype(np.float64)
              if k in ("u", "dt", "B", "C", "z", "g") else v) for k, v in inp.items()}
    y, g = _run(bf, ("skip", "gate"), dtype=torch.bfloat16, segments=6)
    yr, gr = _oracle(bf, ("skip", "gate"))
    at = lambda r: 2e-2 * max(1.0, float(np.abs(r).max()))
    _close("y", y, yr, 2e-2, at(yr))
    for k in ("u", "dt", "A", "B", "C", "D", "z"):
        _close(f"d{k}", g[k], gr[k], 2e-2, at(gr[k]))


def test_automatic_split_of_a_long_row():
    from selectssm_amd import _lib as L

    shape = (1, 16384, 64, 16)
    d = L.make_desc(*shape)
    # 1 x 2 channel blocks x 4 waves: split into 512-step segments
    assert L.size_query(L.lib().ssm_fwd_workspace_bytes, d) == 32 * 32 * 64 * 4
    inp = make_inputs(*shape, seed=2)
    y, g = _run(inp)
    yr, gr = _oracle(inp)
    _close("y", y, yr)
    for k in ("u", "dt", "A", "B", "C"):
        _close(f"d{k}", g[k], gr[k])


@pytest.mark.parametrize("decay,flags", [
    ("fast", ()),                                   # products flush within a piece: the pieces' flags
    ("fast", ("reverse", "complement", "skip", "gate")),  # the gated aggregate variant (dy times the gate)
    ("slow", ("reverse", "complement", "skip")),    # no flush: every piece walked whole and folded
])
def test_aggregate_pieces_match_oracle(decay, flags):
    from selectssm_amd import _lib as L

    # 2 segments of 32768 steps, each aggregate walked in 2 pieces of 16384 (with one int
    # flag per piece and 64-channel block), 40 channels: a ragged channel block
    shape = (1, 65536, 40, 8)
    per_piece = 2 * 8 * 40 * 4 + 4
    assert L.size_query(L.lib().ssm_fwd_workspace_bytes, L.make_desc(*shape, segments=2)) == 2 * 2 * per_piece
    print(f"pieces decay={decay} flags={flags} shape={shape}", flush=True)
    inp = make_inputs(*shape, seed=6)
    if decay == "slow":
        # delta about 2e-4: the sum of a*delta over any piece stays above -53 (seed 6), so no
        # product reaches 2^-126 = e^-87.3 (with the synthetic delta the slowest state
        # flushes after some 4300 steps)
        inp["dt"] = (inp["dt"] * 0.01).astype(np.float32)
    y, g = _run(inp, flags, segments=2)
    yr, gr = _oracle(inp, flags)
    got = dict(y=y, **{f"d{k}": g[k] for k in ("u", "dt", "A", "B", "C", "D", "z")})
    ref = dict(y=yr, **{f"d{k}": gr[k] for k in ("u", "dt", "A", "B", "C", "D", "z")})
    names = (["y", "du", "ddt", "dA", "dB", "dC"] + (["dD"] if "skip" in flags else [])
             + (["dz"] if "gate" in flags else []))
    if decay == "fast":
        at = lambda r: ATOL * max(1.0, float(np.abs(r).max()))
        for k in names:
            _close(k, got[k], ref[k], RTOL, at(ref[k]))
        return
    # With some 5000 steps of memory the fp32 adjoint sums round at about 1e-5 of the
    # largest gradient: each result within 1e-4 of its largest reference value, and no
    # farther from the oracle than the unsplit run of the same inputs (the fold of the
    # pieces' carries adds no error of its own)
    y1, g1 = _run(inp, flags, segments=1)
    one = dict(y=y1, **{f"d{k}": g1[k] for k in ("u", "dt", "A", "B", "C", "D", "z")})
    for k in names:
        scale = max(1.0, float(np.abs(ref[k]).max()))
        _close(k, got[k], ref[k], 0.0, 1e-4 * scale)
        err = lambda t: float(np.abs(t.detach().double().cpu().numpy() - np.asarray(ref[k], np.float64)).max())
        e2, e1 = err(got[k]), err(one[k])
        print(f"  {k}: max err split {e2:.3e}, unsplit {e1:.3e}, max |ref| {scale:.3e}", flush=True)
        assert e2 <= 2.0 * e1 + 1e-6 * scale, (k, e2, e1)


def test_aggregate_pieces_ragged_last_segment():
    from selectssm_amd import _lib as L

    # L = 70000 in 2 forced segments: 35008 steps (whole 32-step tiles), then 34992; each
    # aggregate walked in 2 pieces of 17504, so the backward's last piece ends at L, 16 steps
    # short of its length
    shape = (1, 70000, 40, 8)
    assert L.size_query(L.lib().ssm_fwd_workspace_bytes, L.make_desc(*shape, segments=2)) == 4 * (2 * 8 * 40 + 1) * 4
    print(f"pieces ragged shape={shape}", flush=True)
    inp = make_inputs(*shape, seed=10)
    flags = ("reverse", "skip")
    y, g = _run(inp, flags, segments=2)
    yr, gr = _oracle(inp, flags)
    at = lambda r: ATOL * max(1.0, float(np.abs(r).max()))
    _close("y", y, yr, RTOL, at(yr))
    for k in ("u", "dt", "A", "B", "C", "D"):
        _close(f"d{k}", g[k], gr[k], RTOL, at(gr[k]))


def test_aggregate_pieces_bf16():
    # bf16 I/O through the pieces (2 segments of 2 pieces), skip and gate fused; the oracle
    # runs on the bf16-rounded inputs, tolerances as for the other bf16 time splits
    shape = (1, 65536, 40, 8)
    print(f"pieces bf16 shape={shape}", flush=True)
    inp = make_inputs(*shape, seed=9)
    bf = {k: (torch.from_numpy(v).to(torch.bfloat16).float().numpy().astype(np.float64)
              if k in ("u", "dt", "B", "C", "z", "g") else v) for k, v in inp.items()}
    y, g = _run(bf, ("skip", "gate"), dtype=torch.bfloat16, segments=2)
    yr, gr = _oracle(bf, ("skip", "gate"))
    at = lambda r: 2e-2 * max(1.0, float(np.abs(r).max()))
    _close("y", y, yr, 2e-2, at(yr))
    for k in ("u", "dt", "A", "B", "C", "D", "z"):
        _close(f"d{k}", g[k], gr[k], 2e-2, at(gr[k]))


def test_split_and_unsplit_agree():
    inp = make_inputs(2, 4096, 96, 16, seed=4)
    y1, g1 = _run(inp, ("skip", "gate"), segments=1)
    y2, g2 = _run(inp, ("skip", "gate"), segments=16)
    _close("y", y2, y1.detach().double().cpu().numpy())
    for k in ("u", "dt", "A", "B", "C", "D", "z"):
        _close(f"d{k}", g2[k], g1[k].double().cpu().numpy())


def _tail_log_decay(inp, lo, hi):
    """log of each (batch, channel, state) decay product over steps [lo, hi): A * sum(delta)."""
    dsum = inp["dt"][:, lo:hi, :].astype(np.float64).sum(axis=1)  # (B, D)
    return dsum[:, :, None] * inp["A"].astype(np.float64)[None]


@pytest.mark.parametrize("flags", [(), ("reverse", "complement", "skip", "gate")], ids=lambda f: "+".join(f) or "plain")
def test_aggregate_walks_stop_at_underflow(flags):
    """Strong decay in long segments: every decay product of segment 0's last
    1024 steps and of segment 1's first 1024 steps is below exp(-150), so both
    aggregate walks reach exact zeros part-way through their segment and stop."""
    inp = make_inputs(1, 4096, 64, 16, seed=21)
    inp["dt"] = (inp["dt"] * 8.0).astype(np.float32)
    assert _tail_log_decay(inp, 1024, 2048).max() < -150
    assert _tail_log_decay(inp, 2048, 3072).max() < -150
    y, g = _run(inp, flags, segments=2)
    yr, gr = _oracle(inp, flags)
    _close("y", y, yr)
    for k in ("u", "dt", "A", "B", "C"):
        _close(f"d{k}", g[k], gr[k])
    if "skip" in flags:
        _close("dD", g["D"], gr["D"])
    if "gate" in flags:
        _close("dz", g["z"], gr["z"])


def test_aggregates_without_decay():
    """States with A = 0 (decay 1 throughout) and A = -1e-6 in some channels keep
    their workgroup walking the whole segment; the other channel block stops early."""
    inp = make_inputs(2, 3072, 64, 16, seed=22)
    inp["dt"] = (inp["dt"] * 8.0).astype(np.float32)
    inp["A"][3, :] = 0.0
    inp["A"][5, 7] = 0.0
    inp["A"][17, 2] = -1e-6
    assert _tail_log_decay(inp, 0, 1024)[:, 32:].max() < -150  # channels 32..63 decay to 0
    y, g = _run(inp, ("skip",), segments=3)
    yr, gr = _oracle(inp, ("skip",))
    # undecayed states sum thousands of steps (|h| ~ 10), so y and the gradients
    # carry fp32 rounding at the scale of their largest values
    at = lambda r: ATOL * max(1.0, float(np.abs(r).max()))
    _close("y", y, yr, RTOL, at(yr))
    for k in ("u", "dt", "A", "B", "C", "D"):
        _close(f"d{k}", g[k], gr[k], RTOL, at(gr[k]))


# ------------------------------------------------------------ config 3 shape

SHAPE3 = (1, 1 << 20, 1024, 16)


@pytest.fixture(scope="module")
def inputs3():
    from selectssm_amd.synthetic import make_inputs_gpu

    return make_inputs_gpu(*SHAPE3, seed=9)


@pytest.fixture(scope="module")
def split3(inputs3):
    from selectssm_amd.scan import scan_bwd, scan_fwd

    x = inputs3
    y, ck = scan_fwd(x["u"], x["dt"], x["A"], x["B"], x["C"])
    g = scan_bwd(x["u"], x["dt"], x["A"], x["B"], x["C"], None, None, ck, x["g"])
    torch.cuda.synchronize()
    return y, g


def test_config3_split_is_automatic():
    from selectssm_amd import _lib as L

    d = L.make_desc(*SHAPE3)
    # 16 segments x 4 aggregate pieces, P and H per piece and an int flag per 64 channels
    assert L.size_query(L.lib().ssm_fwd_workspace_bytes, d) == 16 * 4 * (32 * 1024 + 16) * 4


def test_config3_exact_linearity(inputs3, split3):
    from selectssm_amd.scan import scan_bwd, scan_fwd

    x = inputs3
    y1, g1 = split3
    assert torch.isfinite(y1).all()
    y2, ck2 = scan_fwd(2 * x["u"], x["dt"], x["A"], x["B"], x["C"])
    assert torch.equal(y2, 2 * y1)
    del y2, ck2
    _, ck = scan_fwd(x["u"], x["dt"], x["A"], x["B"], x["C"])
    g2 = scan_bwd(x["u"], x["dt"], x["A"], x["B"], x["C"], None, None, ck, 2 * x["g"])
    for a, b in zip(g1[:5], g2[:5]):
        assert torch.isfinite(a).all()
        assert torch.equal(b, 2 * a)


def test_config3_split_matches_unsplit(inputs3, split3):
    from selectssm_amd.scan import scan_bwd, scan_fwd

    x = inputs3
    y, g = split3
    y1, ck1 = scan_fwd(x["u"], x["dt"], x["A"], x["B"], x["C"], segments=1)
    _close("y", y, y1.double().cpu().numpy())
    del y1
    g1 = scan_bwd(x["u"], x["dt"], x["A"], x["B"], x["C"], None, None, ck1, x["g"], segments=1)
    for name, a, b in zip(("du", "ddt", "dA", "dB", "dC"), g[:5], g1[:5]):
        print(name, float((a - b).abs().max()), float(b.abs().max()), flush=True)
        _close(name, a, b.double().cpu().numpy())


def test_config3_channels_match_c_port(inputs3, split3):
    from oracle import c_oracle

    x = inputs3
    y, g = split3
    L_ = SHAPE3[1]
    for lo in (0, SHAPE3[2] - 16):
        sl = slice(lo, lo + 16)
        h = {k: x[k][..., sl].contiguous().cpu().numpy() for k in ("u", "dt", "g")}
        A = x["A"][sl].contiguous().cpu().numpy()
        Bc = x["B"].cpu().numpy()
        Cc = x["C"].cpu().numpy()
        # channels are independent for y, du, ddelta and dA
        yr = c_oracle.scan_fwd(h["u"], h["dt"], A, Bc, Cc, min_recursion_length=L_, nthreads=16, precision="f64")
        gr = c_oracle.scan_bwd(h["u"], h["dt"], A, Bc, Cc, h["g"], min_recursion_length=L_, nthreads=16,
                               precision="f64")
        _close(f"y[{lo}]", y[..., sl], yr)
        _close(f"du[{lo}]", g[0][..., sl], gr[0])
        _close(f"ddt[{lo}]", g[1][..., sl], gr[1])
        _close(f"dA[{lo}]", g[2][sl], gr[2])


@pytest.mark.parametrize("N", [3, 7, 16, 29], ids=lambda n: f"N{n}")
@pytest.mark.parametrize("flags", [(), ("reverse", "complement", "skip", "gate", "softplus")], ids=lambda f: "+".join(f) or "plain")
@pytest.mark.parametrize("segments", [1, 3])
def test_every_state_count_variant(N, flags, segments):
    """1, 2, 4 and 8 waves per workgroup (N up to 4, 8, 16, 32), with and without the
    fused epilogue, unsplit and split, against the fp64 oracle."""
    print(f"N={N} flags={flags} segments={segments}", flush=True)
    inp = make_inputs(2, 150, 40, N, seed=20 + N)
    if "softplus" in flags:
        inp["dt"] = np.log(np.expm1(inp["dt"].astype(np.float64))).astype(np.float32)
    y, g = _run(inp, flags, segments=segments)
    yr, gr = _oracle(inp, flags)
    _close("y", y, yr)
    for k in ("u", "dt", "A", "B", "C"):
        _close(f"d{k}", g[k], gr[k])
    if "skip" in flags:
        _close("dD", g["D"], gr["D"])
    if "gate" in flags:
        _close("dz", g["z"], gr["z"])
