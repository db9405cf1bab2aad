"""GPU parity of the HIP selective scan against the fp64 oracle.

Tolerances (stated by the task, applied elementwise as |x-ref| <= atol + rtol |ref|):
  fp32 I/O:  rtol 1e-4, atol 1e-5 for y and every gradient
  bf16 I/O:  rtol 2e-2 (atol 2e-2 x max|ref|), the oracle run on the bf16-rounded inputs
Reverse / complement index maps are checked bit-exactly against explicit flips.
"""
import numpy as np
import pytest

from oracle import ssm_oracle as O
from selectssm_amd.synthetic import make_inputs

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 1e-5

SHAPES = [
    (1, 8, 3, 2),
    (2, 64, 8, 4),
    (2, 96, 8, 4),
    (2, 1024, 128, 16),   # config 0
    (1, 100, 70, 16),     # ragged channel block and time block
    (2, 33, 130, 5),      # N not a multiple of the per-wave state count
    (1, 37, 64, 32),      # N = 32
    (3, 1, 65, 16),       # L = 1
    (2, 50, 1, 1),        # D = 1, N = 1: one live channel and one live state per workgroup
    (1, 45, 3, 32),       # N = 32 over 3 channels
    # config-1 width with more rows than fill the chip once (9 x 32 channel blocks)
    (9, 40, 2048, 16),
    (9, 37, 2046, 13),
]


def _cuda(x, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    return t.to(dtype) if dtype is not None else t


def _close(name, got, ref, rtol=RTOL, atol=ATOL):
    got = got.detach().float().cpu().numpy().astype(np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    assert not bad.any(), (f"{name}: {bad.sum()} of {bad.size} outside tolerance; max err "
                           f"{err.max():.3e}, max |ref| {np.abs(ref).max():.3e}")


def _run(inp, flags=(), dtype=torch.float32):
    from selectssm_amd import selective_scan

    reverse = "reverse" in flags
    complement = "complement" in flags
    t = {k: _cuda(v) for k, v in inp.items()}
    act = ["u", "dt", "B", "C", "z"]
    for k in act:
        t[k] = t[k].to(dtype).requires_grad_(True)
    t["A"].requires_grad_(True)
    t["D"].requires_grad_(True)
    D = t["D"] if "skip" in flags else None
    z = t["z"] if "gate" in flags else None
    y = selective_scan(t["u"], t["dt"], t["A"], t["B"], t["C"], D=D, z=z, reverse=reverse, complement=complement,
                       delta_softplus="softplus" in flags)
    y.backward(t["g"].to(dtype))
    torch.cuda.synchronize()
    grads = {k: (t[k].grad if t[k].grad is not None else None) for k in ("u", "dt", "A", "B", "C", "D", "z")}
    return y, grads


def _oracle(inp, flags=()):
    kw = dict(Dskip=inp["D"] if "skip" in flags else None, z=inp["z"] if "gate" in flags else None,
              reverse="reverse" in flags, complement="complement" in flags, delta_softplus="softplus" in flags)
    y = O.ssm_block_forward(inp["u"], inp["dt"], inp["A"], inp["B"], inp["C"], **kw)
    du, ddt, dA, dB, dC, dD, dz = O.ssm_block_backward(inp["u"], inp["dt"], inp["A"], inp["B"], inp["C"],
                                                        inp["g"], **kw)
    return y, dict(u=du, dt=ddt, A=dA, B=dB, C=dC, D=dD, z=dz)


def _compare(inp, flags=(), dtype=torch.float32, rtol=RTOL, atol=ATOL, scale_atol=False):
    y, g = _run(inp, flags, dtype)
    yr, gr = _oracle(inp, flags)
    at = lambda ref: atol * max(1.0, float(np.abs(ref).max())) if scale_atol else atol
    _close("y", y, yr, rtol, at(yr))
    for k in ("u", "dt", "A", "B", "C"):
        _close("d" + k, g[k], gr[k], rtol, at(gr[k]))
    if "skip" in flags:
        _close("dD", g["D"], gr["D"], rtol, at(gr["D"]))
    if "gate" in flags:
        _close("dz", g["z"], gr["z"], rtol, at(gr["z"]))


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_scan_fp32_matches_oracle(shape):
    inp = make_inputs(*shape, seed=1)
    _compare(inp)


@pytest.mark.parametrize("flags", [("skip",), ("gate",), ("skip", "gate"), ("reverse",), ("reverse", "skip"),
                                   ("reverse", "complement", "skip"), ("reverse", "complement", "skip", "gate")],
                         ids=lambda f: "+".join(f))
def test_epilogue_flags_match_oracle(flags):
    inp = make_inputs(2, 77, 96, 16, seed=2)
    _compare(inp, flags)


def _pre_softplus(inp):
    """Replace dt by the pre-activation of the same delta (softplus is fused in the scan)."""
    inp = dict(inp)
    inp["dt"] = np.log(np.expm1(inp["dt"].astype(np.float64))).astype(np.float32)
    return inp


@pytest.mark.parametrize("flags", [("softplus",), ("softplus", "reverse", "complement", "skip", "gate")],
                         ids=lambda f: "+".join(f))
def test_fused_delta_softplus_matches_oracle(flags):
    inp = _pre_softplus(make_inputs(2, 77, 96, 16, seed=12))
    _compare(inp, flags)


def test_fused_delta_softplus_broadcast_and_split():
    from test_gpu_segments import _run as run_seg

    inp = _pre_softplus(make_inputs(2, 300, 40, 8, seed=13, delta_broadcast=True))
    _compare(inp, ("softplus",))
    inp = _pre_softplus(make_inputs(2, 300, 40, 8, seed=14))
    y, g = run_seg(inp, ("softplus", "skip"), segments=4)
    yr, gr = _oracle(inp, ("softplus", "skip"))
    _close("y", y, yr)
    for k in ("u", "dt", "A", "B", "C", "D"):
        _close("d" + k, g[k], gr[k])


def test_delta_broadcast_matches_oracle():
    inp = make_inputs(2, 50, 72, 8, seed=3, delta_broadcast=True)
    _compare(inp)


def test_bf16_io_matches_oracle():
    inp = make_inputs(2, 256, 128, 16, seed=4)
    # the oracle sees exactly the bf16 values the kernel reads
    for k in ("u", "dt", "B", "C", "z", "g"):
        inp[k] = torch.from_numpy(inp[k]).to(torch.bfloat16).float().numpy()
    _compare(inp, ("skip", "gate"), dtype=torch.bfloat16, rtol=2e-2, atol=2e-2, scale_atol=True)


@pytest.mark.parametrize("case", [
    ((2, 77, 96, 16), ("reverse", "complement", "skip", "gate")),  # partial tile and channel block
    ((2, 77, 98, 16), ("skip",)),                                   # D % 4 != 0: element-wise staging
    ((1, 100, 72, 32), ("gate",)),                                  # N = 32: 8 / 4 states per lane
    ((2, 77, 96, 16), ("softplus", "skip")),
], ids=lambda c: "x".join(map(str, c[0])) + "-" + "+".join(c[1]))
def test_bf16_io_variants_match_oracle(case):
    """bf16 staging (raw 16-bit registers widened at the commit) on every staging path."""
    shape, flags = case
    inp = make_inputs(*shape, seed=21)
    if "softplus" in flags:
        inp = _pre_softplus(inp)
    for k in ("u", "dt", "B", "C", "z", "g"):
        inp[k] = torch.from_numpy(inp[k]).to(torch.bfloat16).float().numpy()
    _compare(inp, flags, dtype=torch.bfloat16, rtol=2e-2, atol=2e-2, scale_atol=True)


def test_reverse_complement_index_map_is_exact():
    """reverse(+complement) output == explicit flip of the forward scan output, bitwise."""
    from selectssm_amd import selective_scan

    inp = make_inputs(2, 64, 96, 16, seed=5)
    t = {k: _cuda(v) for k, v in inp.items()}
    y_fwd = selective_scan(t["u"], t["dt"], t["A"], t["B"], t["C"])
    y_rev = selective_scan(t["u"], t["dt"], t["A"], t["B"], t["C"], reverse=True)
    y_rc = selective_scan(t["u"], t["dt"], t["A"], t["B"], t["C"], reverse=True, complement=True)
    assert torch.equal(y_rev, torch.flip(y_fwd, dims=(1,)))
    assert torch.equal(y_rc, torch.flip(y_fwd, dims=(1, 2)))


def test_reference_named_api_and_errors():
    from selectssm_amd import ssm_chunked_scan, ssm_recursive_scan, ssm_scan

    inp = make_inputs(2, 96, 64, 16, seed=6)
    t = {k: _cuda(v) for k, v in inp.items()}
    args = (t["u"], t["A"], t["B"], t["C"], t["dt"])
    y0 = ssm_chunked_scan(*args)
    y1 = ssm_chunked_scan(*args, chunk_size=8, n_channel_groups=4)
    y2 = ssm_recursive_scan(*args)
    y3 = ssm_scan(*args, min_recursion_length=3, recursive_split=4)
    yr = O.scan_forward(inp["u"], inp["dt"], inp["A"], inp["B"], inp["C"])
    for y in (y0, y1, y2, y3):
        _close("y", y, yr)
    with pytest.raises(ValueError, match="must divide D"):
        ssm_chunked_scan(*args, n_channel_groups=5)
    with pytest.raises(ValueError, match="must divide L"):
        ssm_chunked_scan(*args, chunk_size=7)


def test_deterministic():
    inp = make_inputs(2, 200, 130, 16, seed=7)
    y1, g1 = _run(inp, ("skip",))
    y2, g2 = _run(inp, ("skip",))
    assert torch.equal(y1, y2)
    for k in ("u", "dt", "A", "B", "C", "D"):
        assert torch.equal(g1[k], g2[k]), k


def test_fused_delta_softplus_extreme_preactivations():
    """softplus on the device over pre-activations from -30 to 30, where log1p(e^-|x|)
    rounds 1 + y to 1 and both asymptotes hold."""
    inp = make_inputs(1, 256, 64, 8, seed=15)
    pre = np.linspace(-30.0, 30.0, 256 * 64).reshape(1, 256, 64)
    inp["dt"] = np.random.default_rng(3).permutation(pre.ravel()).reshape(pre.shape).astype(np.float32)
    inp["A"] = -np.exp(np.random.default_rng(4).uniform(-6, -2, inp["A"].shape))  # keep a = exp(A softplus(x)) away from 0
    y, g = _run(inp, ("softplus", "skip"))
    yr, gr = _oracle(inp, ("softplus", "skip"))
    _close("y", y, yr)
    for k in ("u", "dt", "D"):
        _close("d" + k, g[k], gr[k])
    # with delta up to 30 the terms of the sums dA (over time), dB and dC (over
    # channels) reach 1e2..1e4 and cancel: fp32 sums carry an absolute error that
    # scales with the largest term, not with the result
    for k in ("A", "B", "C"):
        _close("d" + k, g[k], gr[k], atol=1e-6 * float(np.abs(gr[k]).max()))
