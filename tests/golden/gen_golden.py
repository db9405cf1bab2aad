"""Writes the golden fixtures in tests/golden/*.npz from the fp64 oracle.

The reference publishes no golden vectors and cannot run here (JAX/Flax are not
installed), so these fixtures freeze the fp64 oracle's outputs on seeded inputs
(selectssm_amd.synthetic.make_inputs, numpy PCG64).  Small cases store inputs
and every output; the config-0-shaped case stores the seed, a checksum of the
regenerated inputs and subsampled outputs.

    python tests/golden/gen_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import ssm_oracle as O  # noqa: E402
from selectssm_amd.synthetic import make_inputs  # noqa: E402

# name: (shape, seed, flags, delta_broadcast)
SMALL = {
    "tiny_1x8x3x2": ((1, 8, 3, 2), 100, (), False),
    "small_2x64x8x4": ((2, 64, 8, 4), 101, (), False),
    "oddL_2x96x8x4": ((2, 96, 8, 4), 102, (), False),
    "bcast_2x40x10x4": ((2, 40, 10, 4), 103, (), True),
    "revcomp_skip_gate_2x48x20x16": ((2, 48, 20, 16), 104, ("skip", "gate", "reverse", "complement"), False),
}
CONFIG0 = ((2, 1024, 128, 16), 0)


def _block(x, flags):
    kw = dict(Dskip=x["D"] if "skip" in flags else None, z=x["z"] if "gate" in flags else None,
              reverse="reverse" in flags, complement="complement" in flags)
    y = O.ssm_block_forward(x["u"], x["dt"], x["A"], x["B"], x["C"], **kw)
    g = O.ssm_block_backward(x["u"], x["dt"], x["A"], x["B"], x["C"], x["g"], **kw)
    return y, g


def input_checksum(x):
    return np.array([float(np.sum(x[k].astype(np.float64) * (1 + np.arange(x[k].size).reshape(x[k].shape) % 7)))
                     for k in ("u", "dt", "A", "B", "C", "g")])


def main():
    for name, (shape, seed, flags, bcast) in SMALL.items():
        x = make_inputs(*shape, seed=seed, delta_broadcast=bcast)
        x["D"] = (x["D"] * np.linspace(0.5, 1.5, shape[2])).astype(np.float32)
        y, (du, ddt, dA, dB, dC, dD, dz) = _block(x, flags)
        out = dict(flags=np.array(",".join(flags)), y=y, du=du, ddt=ddt, dA=dA, dB=dB, dC=dC,
                   **{f"in_{k}": v for k, v in x.items()})
        if dD is not None:
            out["dD"] = dD
        if dz is not None:
            out["dz"] = dz
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **out)
    shape, seed = CONFIG0
    x = make_inputs(*shape, seed=seed)
    y = O.scan_forward(x["u"], x["dt"], x["A"], x["B"], x["C"])
    du, ddt, dA, dB, dC = O.scan_backward(x["u"], x["dt"], x["A"], x["B"], x["C"], x["g"])
    ch = np.arange(0, shape[2], 16)
    ts = np.arange(0, shape[1], 4)
    np.savez_compressed(os.path.join(HERE, "config0_2x1024x128x16.npz"), shape=np.array(shape), seed=np.array(seed),
                        checksum=input_checksum(x), channels=ch, times=ts,
                        y=y[:, :, ch].astype(np.float32), du=du[:, :, ch].astype(np.float32),
                        ddt=ddt[:, :, ch].astype(np.float32), dA=dA.astype(np.float32),
                        dB=dB[:, ts].astype(np.float32), dC=dC[:, ts].astype(np.float32))


if __name__ == "__main__":
    main()
