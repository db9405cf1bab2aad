"""ssm_bwd_static: ssm_bwd with the library's static device scratch in place of a
caller-supplied workspace (for callers that cannot allocate).  Called through the
C ABI, it must give ssm_bwd's results bit for bit, on two calls in a row with
the second on a smaller input (the scratch keeps the first call's contents),
and on two calls of one pieces-split shape whose first leaves aggregate flags
in the scratch that the second must not see (the refusal of a desc whose
workspace exceeds the scratch is a CPU test in test_abi.py)."""
import ctypes

import pytest

torch = pytest.importorskip("torch")

from selectssm_amd import _lib as L  # noqa: E402
from selectssm_amd.scan import _desc, _flags, _ptr, _stream, scan_bwd, scan_fwd  # noqa: E402
from selectssm_amd.synthetic import make_inputs_gpu  # noqa: E402

pytestmark = pytest.mark.gpu

SCRATCH = L.STATIC_SCRATCH_BYTES


def _static_bwd(x, Dskip, z, ckpt, dy, reverse, complement, segments):
    lib = L.lib()
    flags = _flags(Dskip is not None, z is not None, reverse, complement)
    desc = _desc(x["u"], x["dt"], x["A"], flags, segments)
    out = dict(du=torch.empty_like(x["u"]), ddelta=torch.empty_like(x["dt"]), dA=torch.empty_like(x["A"]),
               dB=torch.empty_like(x["B"]), dC=torch.empty_like(x["C"]),
               dD=torch.empty_like(Dskip) if Dskip is not None else None,
               dz=torch.empty_like(z) if z is not None else None)
    rc = lib.ssm_bwd_static(_stream(), ctypes.byref(desc), _ptr(x["u"]), _ptr(x["dt"]), _ptr(x["A"]), _ptr(x["B"]),
                            _ptr(x["C"]), _ptr(Dskip), _ptr(z), _ptr(ckpt), _ptr(dy), _ptr(out["du"]),
                            _ptr(out["ddelta"]), _ptr(out["dA"]), _ptr(out["dB"]), _ptr(out["dC"]), _ptr(out["dD"]),
                            _ptr(out["dz"]))
    L.check(rc)
    return (out["du"], out["ddelta"], out["dA"], out["dB"], out["dC"], out["dD"], out["dz"])


@pytest.mark.parametrize("flags", ["plain", "epi"])
def test_static_scratch_backward_equals_ssm_bwd(flags):
    lib = L.lib()
    # first a larger call (time-split rows: aggregate carries in the scratch too), then a smaller one
    for shape, segments in (((2, 2048, 200, 16), 4), ((1, 300, 70, 8), 0)):
        print(f"ssm_bwd_static {flags} shape={shape} segments={segments}", flush=True)
        x = make_inputs_gpu(*shape, seed=sum(shape))
        Dp = torch.linspace(0.5, 1.5, shape[2], device="cuda") if flags == "epi" else None
        z = x["z"] if flags == "epi" else None
        rev = flags == "epi"
        desc = _desc(x["u"], x["dt"], x["A"], _flags(Dp is not None, z is not None, rev, rev), segments)
        assert 0 < L.size_query(lib.ssm_bwd_workspace_bytes, desc) <= SCRATCH
        _, ck = scan_fwd(x["u"], x["dt"], x["A"], x["B"], x["C"], Dp, z, rev, rev, segments=segments)
        ref = scan_bwd(x["u"], x["dt"], x["A"], x["B"], x["C"], Dp, z, ck, x["g"], rev, rev, segments=segments)
        got = _static_bwd(x, Dp, z, ck, x["g"], rev, rev, segments)
        torch.cuda.synchronize()
        for name, a, b in zip(("du", "ddelta", "dA", "dB", "dC", "dD", "dz"), ref, got):
            assert (a is None) == (b is None), name
            if a is not None:
                assert torch.equal(a, b), name



def test_static_scratch_clears_the_pieces_flags():
    # A time split whose aggregates are walked in pieces (2 segments of 32768 steps, 2
    # pieces each).  The first call's fast decays flush inside a piece and raise its end
    # flag in the scratch; the second call, same shape and so same flag slots, decays too
    # slowly for any flag, so a flag left over from the first would stop its pieces and
    # change its gradients: both calls must equal ssm_bwd bit for bit.
    lib = L.lib()
    shape, segments = (1, 65536, 40, 8), 2
    for decay in ("fast", "slow"):
        print(f"ssm_bwd_static pieces decay={decay} shape={shape} segments={segments}", flush=True)
        x = make_inputs_gpu(*shape, seed=7)
        if decay == "slow":
            x["dt"] = (x["dt"] * 0.01).contiguous()  # no product reaches 2^-126 within a piece
        desc = _desc(x["u"], x["dt"], x["A"], _flags(False, False, False, False), segments)
        assert 0 < L.size_query(lib.ssm_bwd_workspace_bytes, desc) <= SCRATCH
        _, ck = scan_fwd(x["u"], x["dt"], x["A"], x["B"], x["C"], None, None, False, False, segments=segments)
        ref = scan_bwd(x["u"], x["dt"], x["A"], x["B"], x["C"], None, None, ck, x["g"], False, False,
                       segments=segments)
        got = _static_bwd(x, None, None, ck, x["g"], False, False, segments)
        torch.cuda.synchronize()
        for name, a, b in zip(("du", "ddelta", "dA", "dB", "dC", "dD", "dz"), ref, got):
            assert (a is None) == (b is None), name
            if a is not None:
                assert torch.equal(a, b), name
