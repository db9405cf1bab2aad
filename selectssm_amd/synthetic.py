"""Synthetic inputs for the selective scan, with the benchmark configs' distributions.

  u  ~ N(0, 1)
  dt = softplus(0.5 N(0,1) - 4)            (about 0.005 .. 0.05)
  A  = -exp(U[0, ln 16]) per (d, n)         (A in [-16, -1])
  B, C ~ N(0, sigma^2), sigma = N^-1/2      ("N(0, 1/sqrt N)" read as the std)
  D  = 1;  z ~ N(0, 1);  g (= dy) ~ N(0, 1)

``make_inputs`` draws with numpy PCG64 from one SeedSequence, one child per
tensor in the fixed order u, dt, A, B, C, z, g, so the same seed gives the same
arrays on every machine.  ``make_inputs_gpu`` draws the same distributions with
torch's generator directly on the GPU (for sizes where host generation and
upload would dominate a benchmark run).
"""
from __future__ import annotations

import math

import numpy as np

ORDER = ("u", "dt", "A", "B", "C", "z", "g")


def _softplus(x):
    return np.logaddexp(0.0, x)


def make_inputs(batch, seqlen, dim, dstate, seed=0, dtype=np.float32, delta_broadcast=False):
    """dict of numpy arrays u, dt, A, B, C, D, z, g (float32 unless ``dtype``)."""
    ss = np.random.SeedSequence(seed)
    kids = ss.spawn(len(ORDER))
    rng = {k: np.random.Generator(np.random.PCG64(s)) for k, s in zip(ORDER, kids)}
    sig = 1.0 / math.sqrt(dstate)
    dshape = (batch, seqlen, 1 if delta_broadcast else dim)
    out = {
        "u": rng["u"].standard_normal((batch, seqlen, dim)),
        "dt": _softplus(0.5 * rng["dt"].standard_normal(dshape) - 4.0),
        "A": -np.exp(rng["A"].uniform(0.0, math.log(16.0), (dim, dstate))),
        "B": sig * rng["B"].standard_normal((batch, seqlen, dstate)),
        "C": sig * rng["C"].standard_normal((batch, seqlen, dstate)),
        "D": np.ones((dim,)),
        "z": rng["z"].standard_normal((batch, seqlen, dim)),
        "g": rng["g"].standard_normal((batch, seqlen, dim)),
    }
    return {k: v.astype(dtype) for k, v in out.items()}


def make_inputs_gpu(batch, seqlen, dim, dstate, seed=0, dtype=None, device="cuda", delta_broadcast=False):
    """Same distributions as :func:`make_inputs`, drawn by torch on ``device``."""
    import torch

    dtype = dtype or torch.float32
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    sig = 1.0 / math.sqrt(dstate)
    f32 = dict(dtype=torch.float32, device=device, generator=gen)
    dshape = (batch, seqlen, 1 if delta_broadcast else dim)
    u = torch.randn((batch, seqlen, dim), **f32)
    dt = torch.nn.functional.softplus(0.5 * torch.randn(dshape, **f32) - 4.0)
    A = -torch.exp(torch.rand((dim, dstate), **f32) * math.log(16.0))
    B = sig * torch.randn((batch, seqlen, dstate), **f32)
    C = sig * torch.randn((batch, seqlen, dstate), **f32)
    z = torch.randn((batch, seqlen, dim), **f32)
    g = torch.randn((batch, seqlen, dim), **f32)
    D = torch.ones((dim,), dtype=torch.float32, device=device)
    act = lambda t: t.to(dtype)
    return {"u": act(u), "dt": act(dt), "A": A, "B": act(B), "C": act(C), "D": D, "z": act(z), "g": act(g)}
