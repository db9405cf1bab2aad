"""Row-strided operands (ld_y, ld_z, ld_x) and the bidirectional pair launch.

Strides change addressing only, so every check here is bitwise against the
same kernels on contiguous copies: y / dy / z as column slices of wider
arrays, the conv reading x in place from a wider array, and the two
BidirectionalMamba scans written straight into the concatenated output.
"""
import pytest

from selectssm_amd.synthetic import make_inputs_gpu

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def _wide(t, left, right, seed):
    """t as the column slice [left, left + D) of a wider contiguous (B, L, left + D + right) array."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    B, L, D = t.shape
    w = torch.randn(B, L, left + D + right, device="cuda", dtype=t.dtype, generator=g)
    w[..., left:left + D] = t
    return w[..., left:left + D]


@pytest.mark.parametrize("flags", [("gate",), ("gate", "skip", "reverse", "complement")], ids="+".join)
def test_scan_reads_z_and_writes_y_in_place(flags):
    from selectssm_amd.scan import row_stride, scan_bwd, scan_fwd

    x = make_inputs_gpu(2, 200, 96, 16, seed=1)
    rev, comp = "reverse" in flags, "complement" in flags
    D = x["D"] if "skip" in flags else None
    y0, ck0 = scan_fwd(x["u"], x["dt"], x["A"], x["B"], x["C"], D, x["z"], rev, comp)
    zs = _wide(x["z"], 3, 29, 2)
    assert row_stride(zs) == 128
    out = torch.full((2, 200, 2 * 96), 7.0, device="cuda")
    y1, ck1 = scan_fwd(x["u"], x["dt"], x["A"], x["B"], x["C"], D, zs, rev, comp, y_out=out[..., 96:])
    assert torch.equal(y1, y0) and torch.equal(ck1, ck0)
    assert torch.equal(out[..., :96], torch.full_like(y0, 7.0))  # the other half is untouched
    dyw = _wide(x["g"], 96, 0, 3)
    g0 = scan_bwd(x["u"], x["dt"], x["A"], x["B"], x["C"], D, x["z"], ck0, x["g"], rev, comp)
    g1 = scan_bwd(x["u"], x["dt"], x["A"], x["B"], x["C"], D, zs, ck0, dyw, rev, comp)
    for a, b in zip(g0, g1):
        assert (a is None and b is None) or torch.equal(a, b)


@pytest.mark.parametrize("rev,comp", [(False, False), (True, True)])
def test_conv_reads_x_in_place(rev, comp):
    from selectssm_amd.conv import conv_bwd, conv_fwd

    g = torch.Generator(device="cuda").manual_seed(4)
    x = torch.randn(2, 300, 80, device="cuda", generator=g)
    w = torch.randn(4, 80, device="cuda", generator=g)
    du = torch.randn(2, 300, 80, device="cuda", generator=g)
    xs = _wide(x, 80, 160, 5)
    assert torch.equal(conv_fwd(xs, w, rev, comp), conv_fwd(x, w, rev, comp))
    a = conv_bwd(x, w, du, rev, comp)
    b = conv_bwd(xs, w, du, rev, comp)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("complement", [False, True])
def test_bidirectional_pair_equals_two_scans_and_concat(complement):
    from selectssm_amd import selective_scan
    from selectssm_amd.scan import bidirectional_selective_scan

    f = make_inputs_gpu(2, 160, 64, 16, seed=6)
    r = make_inputs_gpu(2, 160, 64, 16, seed=7)
    for d in (f, r):
        d["dt"] = torch.log(torch.expm1(d["dt"]))  # pre-softplus
    h = torch.randn(2, 160, 4 * 64, device="cuda")  # an in_proj output: [xf | xr | zf | zr]
    zf, zr = h[..., 128:192], h[..., 192:]

    def leaves(d):
        return {k: d[k].clone().requires_grad_(True) for k in ("u", "dt", "A", "B", "C", "D")}

    a_f, a_r, b_f, b_r = leaves(f), leaves(r), leaves(f), leaves(r)
    ha = h.clone().requires_grad_(True)
    hb = h.clone().requires_grad_(True)
    ya = torch.cat([
        selective_scan(a_f["u"], a_f["dt"], a_f["A"], a_f["B"], a_f["C"], D=a_f["D"], z=ha[..., 128:192],
                       delta_softplus=True),
        selective_scan(a_r["u"], a_r["dt"], a_r["A"], a_r["B"], a_r["C"], D=a_r["D"], z=ha[..., 192:],
                       reverse=True, complement=complement, delta_softplus=True)], dim=-1)
    pack = lambda d, z: dict(u=d["u"], delta=d["dt"], A=d["A"], B=d["B"], C=d["C"], D=d["D"], z=z)
    yb = bidirectional_selective_scan(pack(b_f, hb[..., 128:192]), pack(b_r, hb[..., 192:]), complement=complement,
                                      delta_softplus=True)
    assert torch.equal(ya, yb)
    g = torch.randn_like(ya)
    ya.backward(g)
    yb.backward(g)
    assert torch.equal(ha.grad, hb.grad)
    for k in ("u", "dt", "A", "B", "C", "D"):
        assert torch.equal(a_f[k].grad, b_f[k].grad), k
        assert torch.equal(a_r[k].grad, b_r[k].grad), k


def test_bidirectional_mamba_pair_path_equals_per_direction_path():
    """The module's fused pair path and its per-direction path (forced here through
    the diagnostics that need unfused values) agree to fp32 rounding."""
    from selectssm_amd import BidirectionalMamba

    g = torch.Generator(device="cuda")
    a = BidirectionalMamba(hidden_features=16, expansion_factor=2.0, complement=True, features=32, device="cuda",
                           generator=g.manual_seed(8))
    b = BidirectionalMamba(hidden_features=16, expansion_factor=2.0, complement=True, features=32, device="cuda",
                           generator=g.manual_seed(9), diagnostics={"ssm_output_norm": True, "ssm_residual": True})
    b.load_flax_params(a.flax_params())
    x = torch.randn(2, 48, 32, device="cuda", generator=g.manual_seed(10))
    ya, yb = a(x), b(x)
    assert torch.allclose(ya, yb, rtol=1e-5, atol=1e-6)
    assert {"ssm_output_mean", "ssm_residual_sd"} <= set(b.ssm_rev.sown["diagnostics"])
    ya.square().sum().backward()
    yb.square().sum().backward()
    pa, pb = dict(a.named_parameters()), dict(b.named_parameters())
    for k in pa:
        # the two paths add u's gradient contributions in different orders; the
        # weight gradients are sums over B*L terms, so compare at their scale
        ref = pb[k].grad
        assert torch.allclose(pa[k].grad, ref, rtol=1e-4, atol=1e-5 * float(ref.abs().max())), k


@pytest.mark.parametrize("dtype,width,segments,flags", [
    (torch.float32, 2, 0, ()),
    (torch.float32, 3, 3, ("gate", "skip", "reverse", "complement", "softplus")),
    (torch.bfloat16, 2, 2, ("gate", "skip")),
], ids=lambda v: str(v))
def test_scan_reads_bc_in_place_and_writes_dbc(dtype, width, segments, flags):
    """B and C read as column slices of one (B, L, width*N) array (the BC projection's
    output, desc.ld_bc), and dB, dC written into the matching slices of one gradient
    array: bitwise the results on contiguous B, C, dB, dC."""
    from selectssm_amd.scan import bc_stride, scan_bwd, scan_fwd

    x = make_inputs_gpu(2, 333, 72, 16, seed=7)
    io = {k: x[k].to(dtype).contiguous() for k in ("u", "dt", "B", "C", "z", "g")}
    N = 16
    bc = torch.randn(2, 333, width * N, device="cuda").to(dtype)
    bc[..., :N] = io["B"]
    bc[..., N:2 * N] = io["C"]
    Bs, Cs = bc[..., :N], bc[..., N:2 * N]
    assert bc_stride(Bs, Cs) == width * N
    rev, comp = "reverse" in flags, "complement" in flags
    D = x["D"] if "skip" in flags else None
    z = io["z"] if "gate" in flags else None
    kw = dict(segments=segments, delta_softplus="softplus" in flags)
    y0, ck0 = scan_fwd(io["u"], io["dt"], x["A"], io["B"], io["C"], D, z, rev, comp, **kw)
    y1, ck1 = scan_fwd(io["u"], io["dt"], x["A"], Bs, Cs, D, z, rev, comp, **kw)
    assert torch.equal(y0, y1) and torch.equal(ck0, ck1)
    g0 = scan_bwd(io["u"], io["dt"], x["A"], io["B"], io["C"], D, z, ck0, io["g"], rev, comp, **kw)
    dbc = torch.full((2, 333, width * N), 5.0, device="cuda", dtype=dtype)
    g1 = scan_bwd(io["u"], io["dt"], x["A"], Bs, Cs, D, z, ck0, io["g"], rev, comp, dbc_out=dbc, **kw)
    for a, b in zip(g0, g1):
        assert (a is None and b is None) or torch.equal(a, b)
    assert torch.equal(dbc[..., :N], g0[3]) and torch.equal(dbc[..., N:2 * N], g0[4])
    assert torch.equal(dbc[..., 2 * N:], torch.full_like(dbc[..., 2 * N:], 5.0))  # columns beyond 2N untouched
    # the pair entry points with both calls reading B, C in place (one joint launch per kernel)
    from selectssm_amd.scan import scan_bwd_pair, scan_fwd_pair

    calls = [dict(u=io["u"], delta=io["dt"], A=x["A"], B=Bs, C=Cs, Dskip=D, z=z, **kw),
             dict(u=io["u"], delta=io["dt"], A=(x["A"] * 0.5).contiguous(), B=Bs, C=Cs, Dskip=D, z=z,
                  reverse=True, complement=True, **kw)]
    pair = scan_fwd_pair(calls)
    single = [scan_fwd(**dict(c, B=io["B"], C=io["C"])) for c in calls]
    for (yp, cp), (ys, cs) in zip(pair, single):
        assert torch.equal(yp, ys) and torch.equal(cp, cs)
    pg = scan_bwd_pair([dict(c, ckpt=ck, dy=io["g"]) for c, (_, ck) in zip(calls, pair)])
    for c, (_, ck), gp in zip(calls, single, pg):
        gs = scan_bwd(**dict(dict(Dskip=None, z=None), **dict(c, B=io["B"], C=io["C"])), ckpt=ck, dy=io["g"])
        for a, b in zip(gs, gp):
            assert (a is None and b is None) or torch.equal(a, b)


def test_module_bc_projection_read_in_place_matches_copies(monkeypatch):
    """SelectiveSSM passes B, C as slices of the BC projection output and receives dB, dC
    in one (B, L, 2N) gradient: the same module with B, C copied to contiguous arrays
    (and dB, dC concatenated) gives the same output and parameter gradients bit for bit."""
    from selectssm_amd import SelectiveSSM, modules

    g = torch.Generator(device="cuda").manual_seed(9)
    m = SelectiveSSM(hidden_features=16, shift_conv_size=4, features=96, device="cuda", generator=g)
    x = torch.randn(2, 700, 96, device="cuda", generator=g)
    dy = torch.randn(2, 700, 96, device="cuda", generator=g)

    def run():
        for p in m.parameters():
            p.grad = None
        xx = x.clone().requires_grad_(True)
        y = m(xx)
        y.backward(dy)
        return y.detach(), xx.grad, {k: p.grad.clone() for k, p in m.named_parameters()}

    ref = run()
    orig = modules._core_project

    def copying(*a, **k):
        A, dt_low, dt, Bc, Cc = orig(*a, **k)
        return A, dt_low, dt, Bc.contiguous(), Cc.contiguous()

    monkeypatch.setattr(modules, "_core_project", copying)
    orig_grads = modules._core_param_grads

    def cat_grads(saved, grads, dbc, N, rank):
        du, ddt, dA, dB, dC, dD, dz = grads
        return orig_grads(saved, grads, torch.cat([dB, dC], dim=-1), N, rank)

    monkeypatch.setattr(modules, "_core_param_grads", cat_grads)
    got = run()
    assert torch.equal(ref[0], got[0]) and torch.equal(ref[1], got[1])
    for k in ref[2]:
        assert torch.equal(ref[2][k], got[2][k]), k
