"""BASELINE.json configs 2 and 4 at their full sizes on the GPU.

Config 2 (B=4, L=131072, D=512, N=16, fp32): both directions of a
BidirectionalMamba pass (forward, and reverse + complement with its own A)
through ssm_fwd_pair / ssm_bwd_pair, with the automatic time split of 8
segments per row.  Config 4 (B=16, L=4096, D=5120, N=16): bf16 I/O, fp32 state.

The fp64 oracle cannot run these sizes inside a test, so the checks are:
  * exact linearity: y(2u) == 2 y(u), grads(2 dy) == 2 grads(dy), bitwise
    (scaling by 2 commutes with every rounding of the recurrence, the segment
    carries and the bf16 stores);
  * the pair equals the two single calls bit for bit (config 2);
  * finiteness of every output;
  * whole batch rows (every channel, so the sums over channels dB and dC are
    complete) against the float64 C port of the reference's custom-VJP
    algorithm (oracle/ssm_oracle.c): fp32 at rtol 1e-4 / atol 1e-5, bf16 I/O at
    rtol 2e-2 (atol 2e-2 x max|ref|) on the bf16-rounded inputs; dA (a sum over
    batch rows) through a GPU run on the same rows.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

SHAPE2 = (4, 131072, 512, 16)
SHAPE4 = (16, 4096, 5120, 16)
NTHREADS = 16


def _close(name, got, ref, rtol=1e-4, atol=1e-5):
    got = got.double().cpu().numpy() if isinstance(got, torch.Tensor) else np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    print(f"  {name}: max err {err.max():.3e}, max |ref| {np.abs(ref).max():.3e}", flush=True)
    assert not bad.any(), f"{name}: {bad.sum()}/{bad.size} outside, max err {err.max():.3e}"


def _nseg(desc_shape, nbytes_fwd_ws):
    """Time segments per row the forward workspace holds aggregates for (shapes whose segments
    are walked whole: one end state and decay product per segment, state and channel)."""
    B, L, D, N = desc_shape
    return nbytes_fwd_ws // (2 * B * N * D * 4) if nbytes_fwd_ws else 1


# ------------------------------------------------------------------ config 2

@pytest.fixture(scope="module")
def c2():
    from selectssm_amd.synthetic import make_inputs_gpu

    x = make_inputs_gpu(*SHAPE2, seed=5)
    x["A2"] = (x["A"] * 0.5).contiguous()  # the reverse direction's own A, as bench.py --config 2
    return x


def _c2_calls(x, u=None):
    u = x["u"] if u is None else u
    base = dict(u=u, delta=x["dt"], B=x["B"], C=x["C"])
    return [dict(base, A=x["A"]), dict(base, A=x["A2"], reverse=True, complement=True)]


def test_c2_pair_auto_segments_linearity_and_single_calls(c2):
    from selectssm_amd import _lib as L
    from selectssm_amd.scan import _desc, scan_bwd, scan_bwd_pair, scan_fwd, scan_fwd_pair

    x = c2
    print(f"config 2 pair {SHAPE2}", flush=True)
    desc = _desc(x["u"], x["dt"], x["A"], 0)
    assert _nseg(SHAPE2, L.lib().ssm_fwd_workspace_bytes(desc)) == 8
    calls = _c2_calls(x)
    pair = scan_fwd_pair(calls)
    pair2 = scan_fwd_pair(_c2_calls(x, 2 * x["u"]))
    for (y, _), (y2, _) in zip(pair, pair2):
        assert torch.isfinite(y).all()
        assert torch.equal(y2, 2 * y)
    del pair2
    g = x["g"]
    pg = scan_bwd_pair([dict(c, ckpt=ck, dy=g) for c, (_, ck) in zip(calls, pair)])
    pg2 = scan_bwd_pair([dict(c, ckpt=ck, dy=2 * g) for c, (_, ck) in zip(calls, pair)])
    for gr, gr2 in zip(pg, pg2):
        for a, b in zip(gr[:5], gr2[:5]):
            assert torch.isfinite(a).all()
            assert torch.equal(b, 2 * a)
    del pg2
    torch.cuda.synchronize()
    print("  linearity and finiteness ok", flush=True)
    for c, (yp, cp), gp in zip(calls, pair, pg):
        ys, cs = scan_fwd(**c)
        assert torch.equal(ys, yp) and torch.equal(cs, cp)
        gs = scan_bwd(**dict(c, Dskip=None, z=None), ckpt=cs, dy=g)
        for a, b in zip(gs[:5], gp[:5]):
            assert torch.equal(a, b)
    print("  pair == two single calls", flush=True)


def test_c2_row0_both_directions_match_f64_port(c2):
    from oracle import c_oracle
    from selectssm_amd.scan import scan_bwd_pair, scan_fwd_pair

    x = c2
    calls = _c2_calls(x)
    pair = scan_fwd_pair(calls)
    pg = scan_bwd_pair([dict(c, ckpt=ck, dy=x["g"]) for c, (_, ck) in zip(calls, pair)])
    torch.cuda.synchronize()
    h = {k: x[k][:1].cpu().numpy() for k in ("u", "dt", "B", "C", "g")}
    for k, (c, (y, _), grads) in enumerate(zip(calls, pair, pg)):
        rev = c.get("reverse", False)
        A = c["A"].cpu().numpy()
        # the reverse + complement call reads its inputs in the scan domain and
        # writes y at (L-1-t, D-1-d); its dy is read through the same map
        dy = np.ascontiguousarray(h["g"][:, ::-1, ::-1]) if rev else h["g"]
        print(f"config 2 direction {k} row 0: fp64 C port", flush=True)
        yr = c_oracle.scan_fwd(h["u"], h["dt"], A, h["B"], h["C"], nthreads=NTHREADS, precision="f64")
        gr = c_oracle.scan_bwd(h["u"], h["dt"], A, h["B"], h["C"], dy, nthreads=NTHREADS, precision="f64")
        y0 = y[:1].cpu().numpy()
        _close("y", np.ascontiguousarray(y0[:, ::-1, ::-1]) if rev else y0, yr)
        for name, got, ref in (("du", grads[0], gr[0]), ("ddelta", grads[1], gr[1]), ("dB", grads[3], gr[3]),
                               ("dC", grads[4], gr[4])):
            _close(name, got[:1], ref)
        # dA sums over the batch rows: the GPU's row-0 contribution from a one-row pair call
        one = [dict(c2_, u=c2_["u"][:1], delta=c2_["delta"][:1], B=c2_["B"][:1], C=c2_["C"][:1]) for c2_ in calls]
        p1 = scan_fwd_pair(one)
        g1 = scan_bwd_pair([dict(c1, ckpt=ck, dy=x["g"][:1]) for c1, (_, ck) in zip(one, p1)])
        _close("dA(row0)", g1[k][2], gr[2])
        del p1, g1


# ------------------------------------------------------------------ config 4

@pytest.fixture(scope="module")
def c4():
    from selectssm_amd.synthetic import make_inputs_gpu

    x = make_inputs_gpu(*SHAPE4, seed=6)
    for k in ("u", "dt", "B", "C", "z", "g"):
        x[k] = x[k].to(torch.bfloat16).contiguous()
    return x


def test_c4_bf16_linearity_gate_and_finiteness(c4):
    from selectssm_amd.scan import scan_bwd, scan_fwd

    x = c4
    print(f"config 4 bf16 {SHAPE4}, skip + gate", flush=True)
    Dp = torch.linspace(0.5, 1.5, SHAPE4[2], device="cuda")
    for z in (None, x["z"]):
        y, ck = scan_fwd(x["u"], x["dt"], x["A"], x["B"], x["C"], Dp, z)
        y2, _ = scan_fwd((2 * x["u"].float()).to(torch.bfloat16), x["dt"], x["A"], x["B"], x["C"], Dp, z)
        assert y.dtype == torch.bfloat16 and torch.isfinite(y.float()).all()
        assert torch.equal(y2, (2 * y.float()).to(torch.bfloat16))
        g1 = scan_bwd(x["u"], x["dt"], x["A"], x["B"], x["C"], Dp, z, ck, x["g"])
        g2 = scan_bwd(x["u"], x["dt"], x["A"], x["B"], x["C"], Dp, z, ck, (2 * x["g"].float()).to(torch.bfloat16))
        for a, b in zip(g1, g2):
            if a is None:
                continue
            assert torch.isfinite(a.float()).all()
            assert torch.equal(b.float(), 2 * a.float())
        del y, y2, ck, g1, g2
    torch.cuda.synchronize()


def test_c4_bf16_rows_match_f64_port(c4):
    from oracle import c_oracle
    from selectssm_amd.scan import scan_bwd, scan_fwd

    x = c4
    y, ck = scan_fwd(x["u"], x["dt"], x["A"], x["B"], x["C"])
    du, ddt, _, dB, dC, _, _ = scan_bwd(x["u"], x["dt"], x["A"], x["B"], x["C"], None, None, ck, x["g"])
    torch.cuda.synchronize()
    rows = slice(0, 2)
    # the port sees exactly the bf16 values the kernels read
    h = {k: x[k][rows].float().cpu().numpy() for k in ("u", "dt", "B", "C", "g")}
    A = x["A"].cpu().numpy()
    print("config 4 rows 0-1: fp64 C port on the bf16-rounded inputs", flush=True)
    yr = c_oracle.scan_fwd(h["u"], h["dt"], A, h["B"], h["C"], nthreads=NTHREADS, precision="f64")
    gr = c_oracle.scan_bwd(h["u"], h["dt"], A, h["B"], h["C"], h["g"], nthreads=NTHREADS, precision="f64")
    bar = lambda ref: dict(rtol=2e-2, atol=2e-2 * float(np.abs(ref).max()))
    _close("y", y[rows], yr, **bar(yr))
    for name, got, ref in (("du", du, gr[0]), ("ddelta", ddt, gr[1]), ("dB", dB, gr[3]), ("dC", dC, gr[4])):
        _close(name, got[rows], ref, **bar(ref))
    sub = {k: x[k][rows].contiguous() for k in ("u", "dt", "B", "C", "g")}
    y1, ck1 = scan_fwd(sub["u"], sub["dt"], x["A"], sub["B"], sub["C"])
    g1 = scan_bwd(sub["u"], sub["dt"], x["A"], sub["B"], sub["C"], None, None, ck1, sub["g"])
    _close("dA(rows 0-1)", g1[2], gr[2], **bar(gr[2]))
