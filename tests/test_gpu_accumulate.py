"""SSM_ACCUMULATE: ssm_bwd adding the gate's gradient to dz, ssm_conv_bwd adding to
dx (BidirectionalMamba's tied gate and in_proj blocks, selectssm.py:320-321).

The accumulated result is the sum of the two separately computed gradients: bit
for bit in fp32 (one addition per element either way), within bf16 rounding for
bf16 I/O.  Covered: single calls, a pair call whose second call adds into the
first call's dz, forced time segments, and the conv with both flip maps."""
import numpy as np
import pytest

from selectssm_amd.synthetic import make_inputs

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def _gpu(inp, dtype):
    t = {k: torch.from_numpy(np.ascontiguousarray(v)).cuda() for k, v in inp.items()}
    for k in ("u", "dt", "B", "C", "z", "g"):
        t[k] = t[k].to(dtype)
    return t


def _scan_pair_inputs(shape, dtype, seed):
    B, L, D, N = shape
    t = _gpu(make_inputs(B, L, D, N, seed=seed), dtype)
    Dp = torch.linspace(0.5, 1.5, D, device="cuda")
    f = dict(u=t["u"], delta=t["dt"], A=t["A"], B=t["B"], C=t["C"], Dskip=Dp, z=t["z"], delta_softplus=True)
    r = dict(f, A=(t["A"] * 0.5).contiguous(), reverse=True, complement=True)
    return f, r, t["g"]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("segments", [0, 3])
def test_scan_dz_accumulates(dtype, segments):
    from selectssm_amd.scan import scan_bwd, scan_bwd_pair, scan_fwd

    print(f"dz accumulate dtype={dtype} segments={segments}", flush=True)
    f, r, g = _scan_pair_inputs((2, 1100, 96, 16), dtype, seed=41)
    outs = []
    for c in (f, r):
        y, ck = scan_fwd(c["u"], c["delta"], c["A"], c["B"], c["C"], c["Dskip"], c["z"], c.get("reverse", False),
                         c.get("complement", False), segments=segments, delta_softplus=True)
        outs.append(ck)
    args = lambda c, ck: (c["u"], c["delta"], c["A"], c["B"], c["C"], c["Dskip"], c["z"], ck, g,
                          c.get("reverse", False), c.get("complement", False))
    gf = scan_bwd(*args(f, outs[0]), segments=segments, delta_softplus=True)
    gr = scan_bwd(*args(r, outs[1]), segments=segments, delta_softplus=True)
    ref = gf[-1].float() + gr[-1].float()
    # single calls: the second adds into the first's dz
    acc = gf[-1].clone()
    g2 = scan_bwd(*args(r, outs[1]), segments=segments, delta_softplus=True, dz_out=acc, dz_accumulate=True)
    assert g2[-1] is acc
    for a, b in zip(g2[:-1], gr[:-1]):  # every other gradient is the call's own
        assert torch.equal(a, b)
    # a pair call with one dz buffer
    dz = torch.empty_like(gf[-1])
    pf, pr = scan_bwd_pair([dict(f, ckpt=outs[0], dy=g, segments=segments, dz_out=dz),
                            dict(r, ckpt=outs[1], dy=g, segments=segments, dz_out=dz, dz_accumulate=True)])
    assert pf[-1] is dz and pr[-1] is dz
    torch.cuda.synchronize()
    if dtype == torch.float32:
        assert torch.equal(acc, ref) and torch.equal(dz, ref)
    else:  # the kernel rounds the sum once, the reference each part and the sum
        tol = 2e-2 * float(ref.abs().max())
        assert torch.allclose(acc.float(), ref, rtol=2e-2, atol=tol)
        assert torch.equal(dz, acc)


def test_scan_accumulate_needs_the_gate_and_a_buffer():
    from selectssm_amd.scan import scan_bwd, scan_fwd

    f, _, g = _scan_pair_inputs((1, 64, 64, 8), torch.float32, seed=42)
    y, ck = scan_fwd(f["u"], f["delta"], f["A"], f["B"], f["C"], f["Dskip"], None)
    with pytest.raises(ValueError):
        scan_bwd(f["u"], f["delta"], f["A"], f["B"], f["C"], f["Dskip"], None, ck, g, dz_accumulate=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("maps", [((False, False), (True, True)), ((True, False), (False, True))],
                         ids=["id+rc", "time+chan"])
def test_conv_dx_accumulates_and_pair_node(dtype, maps):
    from selectssm_amd.conv import conv1d_act_map, conv1d_act_pair, conv_bwd

    print(f"conv accumulate dtype={dtype} maps={maps}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(43)
    x = torch.randn(2, 300, 96, device="cuda", generator=gen).to(dtype)
    w1 = torch.randn(4, 96, device="cuda", generator=gen)
    w2 = torch.randn(4, 96, device="cuda", generator=gen)
    du1 = torch.randn(x.shape, device="cuda", generator=gen).to(dtype)
    du2 = torch.randn(x.shape, device="cuda", generator=gen).to(dtype)
    dx1, _ = conv_bwd(x, w1, du1, *maps[0], "silu")
    dx2, _ = conv_bwd(x, w2, du2, *maps[1], "silu")
    acc = dx1.clone()
    conv_bwd(x, w2, du2, *maps[1], "silu", need_dw=False, dx_out=acc, accumulate=True)
    ref = dx1.float() + dx2.float()
    # the autograd node of the two convs of one input
    xx = x.clone().requires_grad_(True)
    p1, p2 = (w.clone().requires_grad_(True) for w in (w1, w2))
    u1, u2 = conv1d_act_pair(xx, p1, p2, maps[0], maps[1])
    torch.autograd.backward([u1, u2], [du1, du2])
    assert torch.equal(u1, conv1d_act_map(x, w1, *maps[0])) and torch.equal(u2, conv1d_act_map(x, w2, *maps[1]))
    q1, q2 = (w.clone().requires_grad_(True) for w in (w1, w2))
    torch.autograd.backward([conv1d_act_map(x, q1, *maps[0]), conv1d_act_map(x, q2, *maps[1])], [du1, du2])
    assert torch.equal(p1.grad, q1.grad) and torch.equal(p2.grad, q2.grad)
    torch.cuda.synchronize()
    if dtype == torch.float32:
        assert torch.equal(acc, ref) and torch.equal(xx.grad, ref)
    else:
        tol = 2e-2 * float(ref.abs().max())
        assert torch.allclose(acc.float(), ref, rtol=2e-2, atol=tol)
        assert torch.equal(xx.grad, acc)


def test_conv_pair_node_partial_gradients():
    """The pair node when only some inputs need a gradient: x alone, or one kernel alone."""
    from selectssm_amd.conv import conv1d_act_map, conv1d_act_pair

    gen = torch.Generator(device="cuda").manual_seed(44)
    x = torch.randn(1, 200, 64, device="cuda", generator=gen)
    w1 = torch.randn(3, 64, device="cuda", generator=gen)
    w2 = torch.randn(3, 64, device="cuda", generator=gen)
    du = torch.randn(x.shape, device="cuda", generator=gen)
    maps = ((False, False), (True, True))
    # only w2 needs a gradient: the first conv's backward is skipped
    p2 = w2.clone().requires_grad_(True)
    u1, u2 = conv1d_act_pair(x, w1, p2, *maps)
    (u1 * du).sum().add((u2 * du).sum()).backward()
    q2 = w2.clone().requires_grad_(True)
    (conv1d_act_map(x, q2, *maps[1]) * du).sum().backward()
    assert torch.equal(p2.grad, q2.grad)
    # only x needs a gradient, and only the second output is used
    xx = x.clone().requires_grad_(True)
    _, u2 = conv1d_act_pair(xx, w1, w2, *maps)
    (u2 * du).sum().backward()
    xr = x.clone().requires_grad_(True)
    (conv1d_act_map(xr, w2, *maps[1]) * du).sum().backward()
    assert torch.equal(xx.grad, xr.grad)
