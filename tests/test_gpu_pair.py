"""ssm_fwd_pair / ssm_bwd_pair: both directions of a BidirectionalMamba pass in
one call, the time-split aggregate passes of both in one launch.  Each result
must equal the single ssm_fwd / ssm_bwd call bit for bit (the pair keeps each
call's own time segments), with and without a time split, for every epilogue
flag, when the two calls need different kernel variants (no joint launch),
for bf16 I/O, for N = 32 and for segments long enough to be aggregated in
pieces."""
import pytest

torch = pytest.importorskip("torch")

from selectssm_amd.scan import scan_bwd, scan_bwd_pair, scan_fwd, scan_fwd_pair  # noqa: E402
from selectssm_amd.synthetic import make_inputs_gpu  # noqa: E402

pytestmark = pytest.mark.gpu

CASES = [
    # (B, L, D, N), segments, dtype, flags of the two calls
    ((2, 1024, 96, 16), 4, torch.float32, "plain"),
    ((2, 1024, 96, 16), 1, torch.float32, "plain"),
    ((1, 2048, 64, 16), 0, torch.float32, "epi"),
    ((2, 1100, 70, 16), 3, torch.float32, "epi"),
    ((2, 1024, 64, 16), 4, torch.float32, "mixed"),
    ((2, 1024, 128, 16), 4, torch.bfloat16, "epi"),
    ((1, 1024, 64, 32), 4, torch.float32, "epi"),
    # 2 segments of 32768 steps whose aggregates are walked in 2 pieces each: the joint
    # aggregate launch clears both calls' piece flags (each in its own workspace)
    ((1, 65536, 40, 8), 2, torch.float32, "plain"),
]


def _calls(shape, segments, dtype, kind, seed):
    B, L, D, N = shape
    x = make_inputs_gpu(B, L, D, N, seed=seed)
    io = {k: x[k].to(dtype).contiguous() for k in ("u", "dt", "B", "C", "g", "z")}
    A2 = (x["A"] * 0.5).contiguous()
    Dp = torch.linspace(0.5, 1.5, D, device="cuda")
    base = dict(u=io["u"], delta=io["dt"], B=io["B"], C=io["C"], segments=segments)
    if kind == "plain":
        f = dict(base, A=x["A"])
        r = dict(base, A=A2, reverse=True, complement=True)
    elif kind == "epi":
        f = dict(base, A=x["A"], Dskip=Dp, z=io["z"], delta_softplus=True)
        r = dict(base, A=A2, Dskip=Dp.flip(0).contiguous(), z=io["z"], reverse=True, complement=True,
                 delta_softplus=True)
    else:  # the forward call has no epilogue staging, the reverse one stages the mirrored skip
        f = dict(base, A=x["A"], Dskip=Dp)
        r = dict(base, A=A2, Dskip=Dp, reverse=True)
    return f, r, io["g"]


@pytest.mark.parametrize("shape,segments,dtype,kind", CASES,
                         ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else str(v))
def test_pair_equals_two_calls(shape, segments, dtype, kind):
    print(f"pair shape={shape} segments={segments} dtype={dtype} kind={kind}", flush=True)
    f, r, g = _calls(shape, segments, dtype, kind, seed=sum(shape) + segments)
    single = [scan_fwd(**c) for c in (f, r)]
    pair = scan_fwd_pair([f, r])
    torch.cuda.synchronize()
    for (ys, cs), (yp, cp) in zip(single, pair):
        assert torch.equal(ys, yp)
        assert torch.equal(cs, cp)
    sg = [scan_bwd(**dict(dict(Dskip=None, z=None), **c), ckpt=ck, dy=g) for c, (_, ck) in zip((f, r), single)]
    pg = scan_bwd_pair([dict(c, ckpt=ck, dy=g) for c, (_, ck) in zip((f, r), single)])
    torch.cuda.synchronize()
    names = ("du", "ddelta", "dA", "dB", "dC", "dD", "dz")
    for gs, gp in zip(sg, pg):
        for n, a, b in zip(names, gs, gp):
            assert (a is None) == (b is None), n
            if a is not None:
                assert torch.equal(a, b), n
