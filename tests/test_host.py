"""Host-side logic of the torch API (runs without a GPU): validation, errors, no CPU fallback."""
import os
import subprocess
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import selectssm_amd  # noqa: E402
from selectssm_amd import scan as S  # noqa: E402

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _cpu_inputs(Bt=2, L=32, D=8, N=4, dtype=torch.float32):
    g = torch.Generator().manual_seed(0)
    return (torch.randn(Bt, L, D, generator=g, dtype=dtype), torch.rand(Bt, L, D, generator=g, dtype=dtype),
            -torch.rand(D, N, generator=g), torch.randn(Bt, L, N, generator=g, dtype=dtype),
            torch.randn(Bt, L, N, generator=g, dtype=dtype))


def test_public_names_mirror_the_reference_exports():
    # the scan entry points of selectssm/__init__.py:1-2
    for name in ("ssm_chunked_scan", "ssm_recursive_scan", "ssm_scan"):
        assert callable(getattr(selectssm_amd, name))


def test_cpu_tensors_are_rejected_not_computed():
    u, dt, A, B, C = _cpu_inputs()
    with pytest.raises(ValueError, match="GPU tensors"):
        selectssm_amd.ssm_scan(u, A, B, C, dt)


@pytest.mark.parametrize("bad,msg", [
    (lambda a: (a[0][0], *a[1:]), "x must be"),
    (lambda a: (a[0], a[1], a[2][:, :3], a[3], a[4]), "Bcoeff must be"),
    (lambda a: (a[0], a[1][..., :3], *a[2:]), "dt must be"),
])
def test_shape_errors(bad, msg):
    u, dt, A, B, C = _cpu_inputs()
    args = bad((u, dt, A, B, C))
    with pytest.raises(ValueError, match=msg):
        S.selective_scan(*args)


def test_unsupported_dtype():
    with pytest.raises(TypeError, match="float32 and bfloat16"):
        S._io_dtype(torch.zeros(1, dtype=torch.float64))
    assert S._io_dtype(torch.zeros(1, dtype=torch.bfloat16), torch.zeros(1)) == torch.float32
    assert S._io_dtype(torch.zeros(1, dtype=torch.bfloat16), None) == torch.bfloat16


def test_reference_errors_raised_before_any_gpu_work():
    u, dt, A, B, C = _cpu_inputs(L=96, D=64)
    with pytest.raises(ValueError, match="n_channel_groups=5 must divide D=64"):
        selectssm_amd.ssm_chunked_scan(u, A, B, C, dt, n_channel_groups=5)
    with pytest.raises(ValueError, match="chunk_size=7 must divide L=96"):
        selectssm_amd.ssm_chunked_scan(u, A, B, C, dt, chunk_size=7)
    with pytest.raises(RecursionError):
        selectssm_amd.ssm_recursive_scan(u, A, B, C, dt, recursive_split=1)


def test_recursion_check_follows_the_reference_condition():
    """ssmrecscan.py:56 recurses only while len > min_recursion_length and
    len % recursive_split == 0: a short row never recurses (any split returns a
    result), split 1 recursing never ends, split 0 divides by zero in the test."""
    from selectssm_amd.scan import _check_recursion

    for L_, ml, sp in ((2, 2, 1), (1, 2, 0), (5, 8, 1), (97, 2, 2), (96, 2, 2), (81, 2, 3), (7, 2, 2)):
        _check_recursion(L_, ml, sp)  # no error
    with pytest.raises(RecursionError):
        _check_recursion(3, 2, 1)
    with pytest.raises(ZeroDivisionError):
        _check_recursion(3, 2, 0)
    with pytest.raises(ValueError):
        _check_recursion(8, 2, -2)


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    from selectssm_amd import _lib

    monkeypatch.setattr(_lib, "LIB", str(tmp_path / "absent.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _lib.lib()


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_synthetic_inputs_follow_the_config_distributions():
    from selectssm_amd.synthetic import make_inputs

    x = make_inputs(2, 512, 64, 16, seed=0)
    assert x["u"].dtype == np.float32 and x["u"].shape == (2, 512, 64)
    assert 0.005 < float(np.median(x["dt"])) < 0.05
    assert x["A"].min() >= -16.0 and x["A"].max() <= -1.0
    assert abs(float(x["B"].std()) - 0.25) < 0.01
    y = make_inputs(2, 512, 64, 16, seed=0)
    assert all(np.array_equal(x[k], y[k]) for k in x)


@pytest.mark.parametrize("K,M,N,dtype", [(3 * 8192, 40, 24, torch.float32), (8192 + 8, 16, 8, torch.float32),
                                         (2 * 8192, 16, 8, torch.bfloat16), (100, 7, 5, torch.float32)])
def test_split_weight_gradient_product(K, M, N, dtype):
    """The modules' weight-gradient product a^T b: split over K into slices (float32,
    K a multiple of the slice) or one call (otherwise) -- the same matrix."""
    from selectssm_amd.modules import _tn

    g = torch.Generator().manual_seed(0)
    a = torch.randn(K, M, generator=g).to(dtype)
    b = torch.randn(K, N, generator=g).to(dtype)
    ref = a.double().t() @ b.double()
    got = _tn(a, b)
    assert got.shape == (M, N) and got.dtype == dtype
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    assert torch.allclose(got.double(), ref, rtol=tol, atol=tol * float(ref.abs().max()))


def test_dense_split_views_and_gradient():
    """in_proj followed by its column split (selectssm.py:319): the blocks are views
    of one output, and the gradients (x, kernel, bias) equal those of the unsplit
    product sliced by the same blocks, with an unused block contributing zero."""
    from selectssm_amd.modules import _DenseSplitFn

    g = torch.Generator().manual_seed(5)
    x2 = torch.randn(10, 6, dtype=torch.float64, generator=g, requires_grad=True)
    w = torch.randn(6, 12, dtype=torch.float64, generator=g, requires_grad=True)
    b = torch.randn(12, dtype=torch.float64, generator=g, requires_grad=True)
    a, m, c = _DenseSplitFn.apply(x2, w, b, 4, 3, 5)
    assert a.data_ptr() + 4 * 8 == m.data_ptr() and m.data_ptr() + 3 * 8 == c.data_ptr()
    assert a.stride() == (12, 1)
    (2 * a.sum() + (c * c).sum()).backward()  # the middle block unused
    got = (x2.grad.clone(), w.grad.clone(), b.grad.clone())
    for t in (x2, w, b):
        t.grad = None
    h = x2 @ w + b
    (2 * h[:, :4].sum() + (h[:, 7:] ** 2).sum()).backward()
    for u, v in zip(got, (x2.grad, w.grad, b.grad)):
        assert torch.allclose(u, v, rtol=1e-12, atol=1e-12)
    assert torch.autograd.gradcheck(lambda xx, ww, bb: _DenseSplitFn.apply(xx, ww, bb, 3, 9),
                                    (torch.randn(4, 3, dtype=torch.float64, requires_grad=True),
                                     torch.randn(3, 12, dtype=torch.float64, requires_grad=True),
                                     torch.randn(12, dtype=torch.float64, requires_grad=True)))
    with pytest.raises(ValueError):
        _DenseSplitFn.apply(x2, w, b, 4, 4)
