"""General index maps of the scan (output map and skip source map, SSM_SKIP_MAP) and
the conjugated modules built on them (SelectiveSSM / BidirectionalMamba forward_rc,
RCPSWrapper without flipped activations).

* the kernels against the fp64 oracle's ``ssm_block_forward/backward`` with the same
  maps, every output map x every skip map, with and without the gate, time-split
  rows and bf16 I/O (rtol 1e-4 / atol 1e-5; bf16 2e-2);
* SelectiveSSM.forward_rc(x) against RC(module(RC(x))) with materialised flips: the
  conjugation only moves index maps, so the output is bitwise the same;
* BidirectionalMamba.forward_rc against RC(block(RC(x))) (the permuted in_proj /
  out_proj sum in another order: fp32 tolerance), values and every gradient;
* RCPSWrapper(BidirectionalMamba) flips no tensor larger than a parameter.
"""
import numpy as np
import pytest

from oracle import ssm_oracle as O
from selectssm_amd.synthetic import make_inputs

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

MAPS = [(False, False), (True, False), (False, True), (True, True)]


def _close(name, got, ref, rtol=1e-4, atol=1e-5):
    got = got.detach().double().cpu().numpy()
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    assert not bad.any(), f"{name}: {bad.sum()}/{bad.size} outside, max err {err.max():.3e}"


def _run_maps(inp, om, sm, gate, segments=0, dtype=torch.float32):
    from selectssm_amd.scan import scan_bwd, scan_fwd

    t = {k: torch.from_numpy(np.ascontiguousarray(v)).cuda() for k, v in inp.items()}
    io = {k: t[k].to(dtype) for k in ("u", "dt", "B", "C", "z", "g")}
    z = io["z"] if gate else None
    y, ck = scan_fwd(io["u"], io["dt"], t["A"], io["B"], io["C"], t["D"], z, om[0], om[1], segments=segments,
                     skip_map=sm)
    g = scan_bwd(io["u"], io["dt"], t["A"], io["B"], io["C"], t["D"], z, ck, io["g"], om[0], om[1],
                 segments=segments, skip_map=sm)
    torch.cuda.synchronize()
    return y, g


@pytest.mark.parametrize("om", MAPS, ids=lambda m: f"out{int(m[0])}{int(m[1])}")
@pytest.mark.parametrize("sm", MAPS + [None], ids=lambda m: "skipdefault" if m is None else f"skip{int(m[0])}{int(m[1])}")
@pytest.mark.parametrize("gate", [False, True], ids=["nogate", "gate"])
def test_kernel_maps_match_oracle(om, sm, gate):
    print(f"maps out={om} skip={sm} gate={gate}", flush=True)
    inp = make_inputs(2, 77, 96, 16, seed=31)
    inp["D"] = np.linspace(0.5, 1.5, 96).astype(np.float32)
    y, g = _run_maps(inp, om, sm, gate)
    kw = dict(Dskip=inp["D"], z=inp["z"] if gate else None, out_map=om, skip_map=sm)
    _close("y", y, O.ssm_block_forward(inp["u"], inp["dt"], inp["A"], inp["B"], inp["C"], **kw))
    ref = O.ssm_block_backward(inp["u"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["g"], **kw)
    for name, a, r in zip(("du", "ddt", "dA", "dB", "dC", "dD", "dz"), g, ref):
        if r is not None:
            _close(name, a, r)


@pytest.mark.parametrize("om,sm", [((True, False), (False, False)), ((False, True), (True, False)),
                                   ((False, False), (True, True))])
def test_kernel_maps_time_split_and_bf16(om, sm):
    print(f"maps split/bf16 out={om} skip={sm}", flush=True)
    inp = make_inputs(2, 1100, 70, 16, seed=32)
    inp["D"] = np.linspace(0.5, 1.5, 70).astype(np.float32)
    kw = dict(Dskip=inp["D"], z=inp["z"], out_map=om, skip_map=sm)
    y, g = _run_maps(inp, om, sm, True, segments=3)
    _close("y split", y, O.ssm_block_forward(inp["u"], inp["dt"], inp["A"], inp["B"], inp["C"], **kw))
    ref = O.ssm_block_backward(inp["u"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["g"], **kw)
    for name, a, r in zip(("du", "ddt", "dA", "dB", "dC", "dD", "dz"), g, ref):
        _close(name + " split", a, r)
    # bf16 I/O on the bf16-rounded inputs
    for k in ("u", "dt", "B", "C", "z", "g"):
        inp[k] = torch.from_numpy(inp[k]).to(torch.bfloat16).float().numpy()
    y, g = _run_maps(inp, om, sm, True, dtype=torch.bfloat16)
    yr = O.ssm_block_forward(inp["u"], inp["dt"], inp["A"], inp["B"], inp["C"], **kw)
    _close("y bf16", y, yr, rtol=2e-2, atol=2e-2 * np.abs(yr).max())
    ref = O.ssm_block_backward(inp["u"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["g"], **kw)
    for name, a, r in zip(("du", "ddt", "dA", "dB", "dC", "dD", "dz"), g, ref):
        _close(name + " bf16", a, r, rtol=2e-2, atol=2e-2 * np.abs(r).max())


def _rc(t):
    return torch.flip(t, dims=(-2, -1))


def _grads(m, x, fn, dy):
    for p in m.parameters():
        p.grad = None
    xx = x.clone().requires_grad_(True)
    y = fn(xx)
    y.backward(dy)
    return y.detach(), xx.grad, {k: p.grad.clone() for k, p in m.named_parameters()}


@pytest.mark.parametrize("rev,comp", [(False, False), (True, False), (True, True)])
def test_selective_ssm_forward_rc_is_bitwise_the_flipped_module(rev, comp):
    from selectssm_amd import SelectiveSSM

    g = torch.Generator(device="cuda").manual_seed(11)
    m = SelectiveSSM(hidden_features=16, shift_conv_size=4, reverse=rev, complement=comp, features=72,
                     device="cuda", generator=g)
    x = torch.randn(2, 300, 72, device="cuda", generator=g)
    dy = torch.randn(2, 300, 72, device="cuda", generator=g)
    a = _grads(m, x, m.forward_rc, dy)
    b = _grads(m, x, lambda xx: _rc(m(_rc(xx))), dy)
    assert torch.equal(a[0], b[0])
    assert torch.allclose(a[1], b[1], rtol=1e-6, atol=1e-7)
    for k in a[2]:
        assert torch.allclose(a[2][k], b[2][k], rtol=1e-5, atol=1e-7 * float(b[2][k].abs().max())), k


@pytest.mark.parametrize("case", [
    dict(complement=True, tie_in_proj=True, tie_gate=True),
    dict(complement=False),
    dict(complement=True, norm_type="layer", mlp_layer=True),
    dict(complement=True, concatenate_fwd_rev=False, norm_type="group", tie_gate=True),
], ids=lambda c: ",".join(f"{k}={v}" for k, v in c.items()))
def test_bidirectional_mamba_forward_rc_matches_flipped_block(case):
    from selectssm_amd import BidirectionalMamba

    print(f"forward_rc case {case}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(12)
    m = BidirectionalMamba(hidden_features=16, expansion_factor=2.0, features=64, device="cuda", generator=g,
                           ssm_args=dict(shift_conv_size=4), **case)
    x = torch.randn(2, 200, 64, device="cuda", generator=g)
    dy = torch.randn(2, 200, 64, device="cuda", generator=g)
    a = _grads(m, x, m.forward_rc, dy)
    b = _grads(m, x, lambda xx: _rc(m(_rc(xx))), dy)
    close = lambda u, v: torch.allclose(u, v, rtol=1e-4, atol=1e-5 * max(1.0, float(v.abs().max())))
    assert close(a[0], b[0])
    assert close(a[1], b[1])
    for k in a[2]:
        assert close(a[2][k], b[2][k]), k


def test_rcps_wrapper_flips_no_activation(monkeypatch):
    """RCPSWrapper(BidirectionalMamba): forward and backward flip only parameters
    (no tensor larger than the largest parameter goes through a flip), and the
    result is RC-equivariant."""
    from selectssm_amd import BidirectionalMamba
    from selectssm_amd.rcps import RCPSWrapper

    model = RCPSWrapper(module_cls=BidirectionalMamba,
                        module_kwargs=dict(hidden_features=16, expansion_factor=2.0, complement=True,
                                           tie_in_proj=True, tie_gate=True,
                                           generator=torch.Generator(device="cuda").manual_seed(13)))
    x = torch.randn(2, 256, 64, device="cuda", generator=torch.Generator(device="cuda").manual_seed(14))
    model(x)  # builds the parameters
    biggest = max(p.numel() for p in model.parameters())
    flipped = []
    orig_t, orig_m = torch.flip, torch.Tensor.flip

    def rec_t(t, *a, **k):
        flipped.append(t.numel())
        return orig_t(t, *a, **k)

    def rec_m(t, *a, **k):
        flipped.append(t.numel())
        return orig_m(t, *a, **k)

    monkeypatch.setattr(torch, "flip", rec_t)
    monkeypatch.setattr(torch.Tensor, "flip", rec_m)
    y = model(x)
    y.square().sum().backward()
    monkeypatch.undo()
    assert flipped and max(flipped) <= biggest, (max(flipped), biggest)
    # RC equivariance of the whole wrapper
    with torch.no_grad():
        y1 = _rc(model(x))
        y2 = model(_rc(x))
    assert torch.allclose(y1, y2, rtol=1e-4, atol=1e-4 * max(1.0, float(y1.abs().max())))
