"""HIP kernels against the committed golden fixtures (fp32, rtol 1e-4 / atol 1e-5)."""
import os

import numpy as np
import pytest

from test_golden import HERE, SMALL, load_small

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 1e-5


def _close(name, got, ref):
    got = got.detach().double().cpu().numpy()
    err = np.abs(got - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), f"{name}: {bad.sum()}/{bad.size} outside tolerance, max err {err.max():.3e}"


@pytest.mark.parametrize("path", SMALL, ids=os.path.basename)
def test_kernels_match_small_fixture(path):
    from selectssm_amd import selective_scan

    x, flags, out = load_small(path)
    t = {k: torch.from_numpy(np.ascontiguousarray(v)).cuda().requires_grad_(True) for k, v in x.items()}
    y = selective_scan(t["u"], t["dt"], t["A"], t["B"], t["C"], D=t["D"] if "skip" in flags else None,
                       z=t["z"] if "gate" in flags else None, reverse="reverse" in flags,
                       complement="complement" in flags)
    y.backward(t["g"].detach())
    _close("y", y, out["y"])
    for name, key in (("du", "u"), ("ddt", "dt"), ("dA", "A"), ("dB", "B"), ("dC", "C"), ("dD", "D"), ("dz", "z")):
        if name in out:
            _close(name, t[key].grad, out[name])


def test_kernels_match_config0_fixture():
    from selectssm_amd import ssm_scan
    from selectssm_amd.synthetic import make_inputs

    f = np.load(os.path.join(HERE, "config0_2x1024x128x16.npz"), allow_pickle=False)
    x = make_inputs(*f["shape"], seed=int(f["seed"]))
    t = {k: torch.from_numpy(v).cuda().requires_grad_(True) for k, v in x.items()}
    y = ssm_scan(t["u"], t["A"], t["B"], t["C"], t["dt"])
    y.backward(t["g"].detach())
    ch, ts = f["channels"], f["times"]
    _close("y", y[:, :, ch], f["y"])
    _close("du", t["u"].grad[:, :, ch], f["du"])
    _close("ddt", t["dt"].grad[:, :, ch], f["ddt"])
    _close("dA", t["A"].grad, f["dA"])
    _close("dB", t["B"].grad[:, ts], f["dB"])
    _close("dC", t["C"].grad[:, ts], f["dC"])
