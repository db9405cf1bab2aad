"""Inference writes no checkpoints.

The forward's state checkpoints are the backward's residuals (the reference
keeps residuals only under differentiation, ssmrecscan.py:85-88).  Under
``torch.no_grad()`` (or with no input requiring a gradient) the scan op, the
SelectiveSSM module and the BidirectionalMamba module must not allocate them:
the allocator's high-water mark of a forward drops by at least the checkpoint
size, and y is bitwise the same.
"""
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def _peak(fn):
    """(result, high-water allocation above what was live before fn).  fn runs once
    before the measured call, so one-time allocations (e.g. a GEMM library's
    workspace on its first use) are not counted."""
    with torch.no_grad():
        fn()
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    out = fn()
    torch.cuda.synchronize()
    return out, torch.cuda.max_memory_allocated() - base


def _ckpt_bytes(u, A):
    from selectssm_amd import _lib as L
    from selectssm_amd.scan import _desc

    return L.size_query(L.lib().ssm_ckpt_bytes, _desc(u, u, A, 0))


def test_scan_op_no_grad_has_no_checkpoints():
    from selectssm_amd import selective_scan
    from selectssm_amd.synthetic import make_inputs_gpu

    x = make_inputs_gpu(2, 4096, 256, 16, seed=1)
    args = [x[k].requires_grad_(True) for k in ("u", "dt", "A", "B", "C")]
    ck = _ckpt_bytes(x["u"], x["A"])
    assert ck == 2 * (4096 // 16) * 16 * 256 * 4
    with torch.no_grad():
        y0, p0 = _peak(lambda: selective_scan(*args, D=x["D"], z=x["z"]))
    y1, p1 = _peak(lambda: selective_scan(*args, D=x["D"], z=x["z"]))
    print(f"scan op: peak {p0} B under no_grad, {p1} B with grad; checkpoints {ck} B", flush=True)
    assert torch.equal(y0, y1)
    assert p1 - p0 >= 0.9 * ck
    # inputs that need no gradient: no graph, no checkpoints either
    plain = [a.detach() for a in args]
    y2, p2 = _peak(lambda: selective_scan(*plain, D=x["D"], z=x["z"]))
    assert torch.equal(y2, y1) and p1 - p2 >= 0.9 * ck


def test_selective_ssm_module_no_grad_has_no_checkpoints():
    from selectssm_amd import SelectiveSSM

    g = torch.Generator(device="cuda").manual_seed(0)
    m = SelectiveSSM(hidden_features=16, shift_conv_size=4, features=256, device="cuda", generator=g)
    x = torch.randn(2, 4096, 256, device="cuda", generator=g)
    ck = _ckpt_bytes(x, m.A_log)
    with torch.no_grad():
        y0, p0 = _peak(lambda: m(x))
    y1, p1 = _peak(lambda: m(x))
    print(f"SelectiveSSM: peak {p0} B under no_grad, {p1} B with grad; checkpoints {ck} B", flush=True)
    assert torch.equal(y0, y1)
    assert p1 - p0 >= 0.9 * ck


def test_bidirectional_mamba_no_grad_has_no_checkpoints():
    from selectssm_amd import BidirectionalMamba

    g = torch.Generator(device="cuda").manual_seed(1)
    m = BidirectionalMamba(hidden_features=16, expansion_factor=2.0, complement=True, tie_in_proj=True,
                           tie_gate=True, features=128, device="cuda", generator=g)
    x = torch.randn(2, 4096, 128, device="cuda", generator=g)
    ck = _ckpt_bytes(torch.empty(2, 4096, 256, device="cuda"), m.ssm_fwd.A_log)
    with torch.no_grad():
        y0, p0 = _peak(lambda: m(x))
    y1, p1 = _peak(lambda: m(x))
    print(f"BidirectionalMamba: peak {p0} B under no_grad, {p1} B with grad; checkpoints 2 x {ck} B", flush=True)
    assert torch.equal(y0, y1)
    assert p1 - p0 >= 2 * 0.9 * ck
