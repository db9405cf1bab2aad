"""The committed fixtures (tests/golden/*.npz) against the CPU oracle and the C port.

The fixtures were written by tests/golden/gen_golden.py from the fp64 oracle; these
tests fail if the oracle, the synthetic-input generator or the C port drift.
The GPU kernels are checked against the same fixtures in test_gpu_golden.py.
"""
import glob
import os

import numpy as np
import pytest

from oracle import ssm_oracle as O

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SMALL = sorted(p for p in glob.glob(os.path.join(HERE, "*.npz")) if "config0" not in p)


def load_small(path):
    f = np.load(path, allow_pickle=False)
    x = {k[3:]: f[k] for k in f.files if k.startswith("in_")}
    flags = tuple(s for s in str(f["flags"]).split(",") if s)
    out = {k: f[k] for k in f.files if not k.startswith("in_") and k != "flags"}
    return x, flags, out


def test_fixture_files_present():
    names = {os.path.basename(p) for p in glob.glob(os.path.join(HERE, "*.npz"))}
    assert len(SMALL) >= 5 and "config0_2x1024x128x16.npz" in names


@pytest.mark.parametrize("path", SMALL, ids=os.path.basename)
def test_oracle_reproduces_small_fixture(path):
    x, flags, out = load_small(path)
    kw = dict(Dskip=x["D"] if "skip" in flags else None, z=x["z"] if "gate" in flags else None,
              reverse="reverse" in flags, complement="complement" in flags)
    y = O.ssm_block_forward(x["u"], x["dt"], x["A"], x["B"], x["C"], **kw)
    np.testing.assert_allclose(y, out["y"], rtol=1e-12, atol=1e-15)
    got = O.ssm_block_backward(x["u"], x["dt"], x["A"], x["B"], x["C"], x["g"], **kw)
    for name, g in zip(("du", "ddt", "dA", "dB", "dC", "dD", "dz"), got):
        if g is not None:
            np.testing.assert_allclose(g, out[name], rtol=1e-12, atol=1e-15, err_msg=name)


def test_config0_fixture_inputs_and_outputs():
    from selectssm_amd.synthetic import make_inputs

    import importlib.util

    spec = importlib.util.spec_from_file_location("gen_golden", os.path.join(HERE, "gen_golden.py"))
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)
    f = np.load(os.path.join(HERE, "config0_2x1024x128x16.npz"), allow_pickle=False)
    x = make_inputs(*f["shape"], seed=int(f["seed"]))
    np.testing.assert_allclose(gen.input_checksum(x), f["checksum"], rtol=1e-12)
    ch, ts = f["channels"], f["times"]
    y = O.scan_forward(x["u"], x["dt"], x["A"], x["B"], x["C"])
    np.testing.assert_allclose(y[:, :, ch], f["y"], rtol=1e-6, atol=1e-9)
    du, ddt, dA, dB, dC = O.scan_backward(x["u"], x["dt"], x["A"], x["B"], x["C"], x["g"])
    np.testing.assert_allclose(du[:, :, ch], f["du"], rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(dA, f["dA"], rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(dB[:, ts], f["dB"], rtol=1e-6, atol=1e-9)


@pytest.mark.parametrize("path", [p for p in SMALL if "revcomp" not in p], ids=os.path.basename)
def test_c_port_reproduces_small_fixture(path):
    from oracle import c_oracle

    x, flags, out = load_small(path)
    dt = np.broadcast_to(x["dt"], x["u"].shape)
    args = (x["u"], dt, x["A"], x["B"], x["C"])
    np.testing.assert_allclose(c_oracle.scan_fwd(*args, nthreads=2), out["y"], rtol=2e-4, atol=1e-6)
    got = c_oracle.scan_bwd(*args, x["g"], nthreads=2)
    for name, g in zip(("du", "ddt", "dA", "dB", "dC"), got):
        ref = out[name]
        if name == "ddt" and ref.shape[-1] == 1 and g.shape[-1] != 1:
            g = g.sum(-1, keepdims=True)  # the C port returns the per-channel (un-reduced) ddt
        np.testing.assert_allclose(g, ref, rtol=2e-4, atol=1e-5, err_msg=name)
