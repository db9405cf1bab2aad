"""Full BASELINE.json config-1 size (B=8, L=8192, D=2048, N=16) on the GPU.

The fp64 oracle cannot run this size in a test, so the checks are
size-independent properties plus a per-row comparison:
  * exact linearity: y(2u) == 2 y(u) and grads(2 dy) == 2 grads(dy), bitwise
    (scaling by 2 commutes with every fp32 rounding in the recurrence);
  * reverse / complement outputs are bitwise flips of the forward output;
  * batch row 0 against the C port of the reference's custom-VJP algorithm run
    in float64 (oracle/ssm_oracle.c) at rtol 1e-4 / atol 1e-5, every output;
  * finiteness of every output.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

SHAPE = (8, 8192, 2048, 16)


@pytest.fixture(scope="module")
def inputs():
    from selectssm_amd.synthetic import make_inputs_gpu

    return make_inputs_gpu(*SHAPE, seed=3)


def test_fullsize_exact_linearity(inputs):
    from selectssm_amd.scan import scan_bwd, scan_fwd

    x = inputs
    y1, ck1 = scan_fwd(x["u"], x["dt"], x["A"], x["B"], x["C"])
    y2, ck2 = scan_fwd(2 * x["u"], x["dt"], x["A"], x["B"], x["C"])
    assert torch.equal(y2, 2 * y1)
    assert torch.isfinite(y1).all()
    g1 = scan_bwd(x["u"], x["dt"], x["A"], x["B"], x["C"], None, None, ck1, x["g"])
    g2 = scan_bwd(x["u"], x["dt"], x["A"], x["B"], x["C"], None, None, ck1, 2 * x["g"])
    for a, b in zip(g1[:5], g2[:5]):
        assert torch.isfinite(a).all()
        assert torch.equal(b, 2 * a)


def test_fullsize_reverse_maps_are_exact(inputs):
    from selectssm_amd import selective_scan

    x = inputs
    y = selective_scan(x["u"], x["dt"], x["A"], x["B"], x["C"])
    assert torch.equal(selective_scan(x["u"], x["dt"], x["A"], x["B"], x["C"], reverse=True),
                       torch.flip(y, dims=(1,)))
    assert torch.equal(selective_scan(x["u"], x["dt"], x["A"], x["B"], x["C"], reverse=True, complement=True),
                       torch.flip(y, dims=(1, 2)))


def test_fullsize_row0_matches_c_port(inputs):
    from oracle import c_oracle
    from selectssm_amd.scan import scan_bwd, scan_fwd

    x = inputs
    y, ck = scan_fwd(x["u"], x["dt"], x["A"], x["B"], x["C"])
    du, ddt, dA, dB, dC, _, _ = scan_bwd(x["u"], x["dt"], x["A"], x["B"], x["C"], None, None, ck, x["g"])
    torch.cuda.synchronize()
    h = {k: x[k][:1].cpu().numpy() for k in ("u", "dt", "B", "C", "g")}
    A = x["A"].cpu().numpy()
    yr = c_oracle.scan_fwd(h["u"], h["dt"], A, h["B"], h["C"], nthreads=16, precision="f64")
    gr = c_oracle.scan_bwd(h["u"], h["dt"], A, h["B"], h["C"], h["g"], nthreads=16, precision="f64")

    def close(name, got, ref, rtol=1e-4, atol=1e-5):
        got = got.double().cpu().numpy()
        err = np.abs(got - ref)
        bad = err > atol + rtol * np.abs(ref)
        assert not bad.any(), f"{name}: {bad.sum()}/{bad.size} outside, max err {err.max():.3e}"

    close("y", y[:1], yr)
    close("du", du[:1], gr[0])
    close("ddt", ddt[:1], gr[1])
    close("dB", dB[:1], gr[3])
    close("dC", dC[:1], gr[4])
    # dA sums over every batch row; the port saw one row: compare the GPU's
    # row-0 contribution through a one-row GPU run instead
    y1, ck1 = scan_fwd(x["u"][:1].contiguous(), x["dt"][:1].contiguous(), x["A"], x["B"][:1].contiguous(),
                       x["C"][:1].contiguous())
    g1 = scan_bwd(x["u"][:1].contiguous(), x["dt"][:1].contiguous(), x["A"], x["B"][:1].contiguous(),
                  x["C"][:1].contiguous(), None, None, ck1, x["g"][:1].contiguous())
    close("dA(row0)", g1[2], gr[2])
