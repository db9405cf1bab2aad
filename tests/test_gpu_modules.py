"""SelectiveSSM / BidirectionalMamba modules on the GPU kernels.

* the reference's own module tests (tests/test_selectssm.py:17-95 of the
  reference): output shapes, the recursive_scan / custom_vjp_scan flags,
  complement mode, concatenation, finite non-zero gradients;
* forward parity with the fp64 oracle modules under the same parameters
  (rtol 1e-4 / atol 1e-5; gelu at the same bar, its tanh form a Flax default);
* every parameter's gradient (and the input's) against a central finite
  difference of the fp64 oracle along a random direction (rtol 1e-4 of the
  directional derivative);
* bf16 activations against the oracle at rtol 2e-2 (x max|ref| absolute).
"""
import math

import numpy as np
import pytest

from oracle import ssm_oracle as O

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def _x(shape, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(shape, device="cuda", generator=g)


def _gen(seed):
    return torch.Generator(device="cuda").manual_seed(seed)


def _np_tree(tree):
    return {k: (_np_tree(v) if isinstance(v, dict) else v.double().numpy()) for k, v in tree.items()}


# ------------------------------------------- the reference's module tests

class TestSelectiveSSM:
    def test_forward_shape(self):
        from selectssm_amd import SelectiveSSM

        model = SelectiveSSM(hidden_features=16, generator=_gen(0))
        x = _x((2, 32, 64), 0)
        assert model(x).shape == x.shape

    def test_recursive_scan(self):
        from selectssm_amd import SelectiveSSM

        model = SelectiveSSM(hidden_features=16, recursive_scan=True, generator=_gen(0))
        x = _x((2, 32, 64), 0)
        assert model(x).shape == x.shape

    def test_custom_vjp_scan(self):
        from selectssm_amd import SelectiveSSM

        model = SelectiveSSM(hidden_features=16, custom_vjp_scan=True, generator=_gen(0))
        x = _x((2, 32, 64), 0)
        assert model(x).shape == x.shape


class TestBidirectionalMamba:
    def test_forward_shape(self):
        from selectssm_amd import BidirectionalMamba

        model = BidirectionalMamba(hidden_features=16, expansion_factor=2.0, generator=_gen(0))
        x = _x((2, 32, 64), 0)
        assert model(x).shape == x.shape

    def test_complement_mode(self):
        from selectssm_amd import BidirectionalMamba

        model = BidirectionalMamba(hidden_features=16, expansion_factor=2.0, complement=True, tie_in_proj=True,
                                   tie_gate=True, generator=_gen(0))
        x = _x((2, 32, 64), 0)
        assert model(x).shape == x.shape

    def test_concatenate_fwd_rev(self):
        from selectssm_amd import BidirectionalMamba

        model = BidirectionalMamba(hidden_features=16, expansion_factor=2.0, concatenate_fwd_rev=True,
                                   generator=_gen(0))
        x = _x((2, 32, 64), 0)
        assert model(x).shape == x.shape

    def test_gradient_flow(self):
        from selectssm_amd import BidirectionalMamba

        model = BidirectionalMamba(hidden_features=16, expansion_factor=2.0, generator=_gen(0))
        x = _x((2, 16, 32), 0)
        loss = torch.sum(model(x) ** 2)
        loss.backward()
        grads = [p.grad for p in model.parameters()]
        assert all(g is not None and torch.isfinite(g).all() for g in grads)
        assert any(g.abs().max() > 0 for g in grads)


# ----------------------------------------------------- parity with the oracle

SSM_CASES = [
    dict(),
    dict(reverse=True),
    dict(reverse=True, complement=True),
    dict(activation="relu", shift_conv_size=4),
    dict(activation="gelu"),
    dict(dt_rank=1, dt_proj=False),                 # (B, L, 1) delta, broadcast in the scan
    dict(dt_rank=4, dt_proj=False),                 # jnp.repeat to D
    dict(custom_vjp_scan=True, reverse=True, complement=True, shift_conv_size=4),
]


def _close(name, got, ref, rtol=1e-4, atol=1e-5):
    got = got.detach().double().cpu().numpy()
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    assert not bad.any(), f"{name}: {bad.sum()}/{bad.size} outside, max err {err.max():.3e}"


def _oracle_kwargs(case):
    kw = {k: v for k, v in case.items() if k in ("reverse", "complement", "dt_rank", "activation")}
    if "dt_proj" in case:
        kw["dt_proj"] = case["dt_proj"]
    return kw


def _fd_check(model, x, g, oracle_fn, seed=0, rtol=1e-4, slack=2e-6):
    """Each parameter's (and x's) gradient of sum(y * g) along a random direction
    against a central difference of the fp64 oracle: within ``rtol`` of the
    directional derivative plus ``slack`` times the sum of its terms' magnitudes
    (the rounding of the I/O type when the terms cancel)."""
    x = x.clone().requires_grad_(True)
    y = model(x)
    (y * g).sum().backward()
    params = dict(model.named_parameters())
    base = _np_tree(model.flax_params())
    xn = x.detach().double().cpu().numpy()
    gn = g.double().cpu().numpy()
    rng = np.random.default_rng(seed)

    def loss(tree, xx):
        return float(np.sum(oracle_fn(tree, xx) * gn))

    def perturbed(name, delta):
        tree = _np_tree(model.flax_params())
        node = tree
        *path, leaf = name.split(".")
        for part in path:
            node = node[part]
        node[leaf] = node[leaf] + delta
        return tree

    eps = 1e-5
    for name, p in list(params.items()) + [("<input>", x)]:
        v = rng.standard_normal(tuple(p.shape))
        if name == "<input>":
            fd = (loss(base, xn + eps * v) - loss(base, xn - eps * v)) / (2 * eps)
        else:
            fd = (loss(perturbed(name, eps * v), xn) - loss(perturbed(name, -eps * v), xn)) / (2 * eps)
        terms = p.grad.double().cpu().numpy() * v
        got = float(terms.sum())
        # fp32 gradients: relative error of the directional derivative, plus the
        # fp32 rounding of its terms when they cancel
        tol = rtol * abs(fd) + slack * float(np.abs(terms).sum())
        assert abs(got - fd) <= tol, f"{name}: autograd {got:.8e} vs fd {fd:.8e} (tol {tol:.2e})"


@pytest.mark.parametrize("case", SSM_CASES, ids=lambda c: ",".join(f"{k}={v}" for k, v in c.items()) or "default")
def test_selective_ssm_matches_oracle(case):
    from selectssm_amd import SelectiveSSM

    print(f"SelectiveSSM case {case}", flush=True)
    model = SelectiveSSM(hidden_features=8, generator=_gen(1), **case)
    x = _x((2, 40, 48), 1)
    y = model(x)
    kw = _oracle_kwargs(case)
    fn = lambda tree, xx: O.selective_ssm_forward(tree, xx, hidden_features=8, **kw)
    _close("y", y, fn(_np_tree(model.flax_params()), x.double().cpu().numpy()))
    _fd_check(model, x, _x(y.shape, 2), fn)


MAMBA_CASES = [
    dict(),
    dict(complement=True, tie_in_proj=True, tie_gate=True),
    dict(concatenate_fwd_rev=False, norm_type="layer"),
    dict(activation="gelu", mlp_layer=True),
    dict(activation="relu", tie_gate=True, ssm_args=dict(shift_conv_size=4, custom_vjp_scan=True)),
    # one tie at a time on the fused pair path: the x-gradient summed in the second
    # conv kernel, or the dz summed in the second scan kernel
    dict(tie_in_proj=True),
    dict(complement=True, tie_gate=True),
]


@pytest.mark.parametrize("case", MAMBA_CASES, ids=lambda c: ",".join(f"{k}={v}" for k, v in c.items()) or "default")
def test_bidirectional_mamba_matches_oracle(case):
    from selectssm_amd import BidirectionalMamba

    print(f"BidirectionalMamba case {case}", flush=True)
    model = BidirectionalMamba(hidden_features=8, expansion_factor=1.5, generator=_gen(3), **case)
    x = _x((2, 24, 32), 3)
    y = model(x)
    # the oracle takes the conv width from the kernel's shape; the scan strategy does not change y
    okw = {k: v for k, v in case.items() if k != "ssm_args"}
    fn = lambda tree, xx: O.bidirectional_mamba_forward(tree, xx, 8, 1.5, **okw)
    _close("y", y, fn(_np_tree(model.flax_params()), x.double().cpu().numpy()))
    _fd_check(model, x, _x(y.shape, 4), fn)


def test_config4_block_bf16_matches_oracle():
    """Config 4's mixed precision (bf16 activations, fp32 state), small shape."""
    from selectssm_amd import SelectiveSSM

    model = SelectiveSSM(hidden_features=16, shift_conv_size=4, generator=_gen(5))
    x = _x((2, 64, 80), 5).to(torch.bfloat16)
    y = model(x)
    assert y.dtype == torch.bfloat16
    ref = O.selective_ssm_forward(_np_tree(model.flax_params()), x.float().double().cpu().numpy())
    _close("y", y, ref, rtol=2e-2, atol=2e-2 * float(np.abs(ref).max()))
    # the backward against the fp64 oracle: every parameter's and the input's
    # gradient along a random direction, at the bf16 bar (2e-2 of the directional
    # derivative, plus bf16 rounding, 2^-8, of its terms where they cancel)
    g = _x(y.shape, 6).to(torch.bfloat16)
    fn = lambda tree, xx: O.selective_ssm_forward(tree, xx)
    _fd_check(model, x, g, fn, seed=5, rtol=2e-2, slack=2.0 ** -8)
    # and elementwise: the same module in fp32 on the same bf16-valued input and
    # upstream gradient (the fp32 module's gradients are pinned by the fp32 tests)
    from selectssm_amd import SelectiveSSM as S

    twin = S(hidden_features=16, shift_conv_size=4, features=80, device="cuda", generator=_gen(7))
    twin.load_flax_params(model.flax_params())
    grads = {}
    for m, xx, gg in ((model, x, g), (twin, x.float(), g.float())):
        for p in m.parameters():
            p.grad = None
        xx = xx.clone().requires_grad_(True)
        (m(xx).float() * gg.float()).sum().backward()
        grads[m] = {**{k: p.grad.double().cpu().numpy() for k, p in m.named_parameters()},
                    "<input>": xx.grad.double().cpu().numpy()}
    for k, ref in grads[twin].items():
        _close(k, torch.from_numpy(grads[model][k]), ref, rtol=2e-2, atol=2e-2 * float(np.abs(ref).max()))


def test_flax_param_tree_roundtrip():
    from selectssm_amd import BidirectionalMamba

    a = BidirectionalMamba(hidden_features=4, expansion_factor=2.0, generator=_gen(6), features=16, device="cuda")
    b = BidirectionalMamba(hidden_features=4, expansion_factor=2.0, generator=_gen(7), features=16, device="cuda")
    tree = a.flax_params()
    assert set(tree) == {"RMSNorm_0", "in_proj", "ssm_fwd", "ssm_rev", "out_proj"}
    assert set(tree["ssm_fwd"]) == {"shift_conv", "A_log", "BC", "D", "dt", "dt_proj"}
    assert tuple(tree["ssm_fwd"]["shift_conv"]["kernel"].shape) == (3, 1, 32)
    assert tuple(tree["in_proj"]["kernel"].shape) == (16, 4 * 32)
    b.load_flax_params({k: v for k, v in tree.items()})
    x = _x((1, 8, 16), 8)
    assert torch.equal(a(x), b(x))
    with pytest.raises(ValueError, match="parameter trees differ"):
        b.load_flax_params({"in_proj": tree["in_proj"]})


def test_regularizer_and_init_distributions():
    from selectssm_amd import SelectiveSSM

    model = SelectiveSSM(hidden_features=16, generator=_gen(9))
    x = _x((1, 16, 256), 9)
    model(x)
    reg = model.sown["losses"]["ssm_regularizer"]
    ref = 1e-7 * (model.shift_conv.kernel ** 2).sum() + 1e-6 * sum(
        (k ** 2).sum() for k in (model.BC.kernel, model.dt.kernel, model.dt_proj.kernel))
    assert torch.allclose(reg, ref)
    # A_log = log(1..N) per channel (selectssm.py:190); D = 1
    assert torch.allclose(model.A_log[3], torch.log(torch.arange(1, 17, device="cuda", dtype=torch.float32)))
    assert torch.equal(model.D, torch.ones(256, device="cuda"))
    # dt_proj bias = inverse_softplus(U[dt_min, dt_max]) -> softplus(bias) in [0.001, 0.1]
    sp = torch.nn.functional.softplus(model.dt_proj.bias.detach())
    assert float(sp.min()) >= 0.001 - 1e-6 and float(sp.max()) <= 0.1 + 1e-6
    # lecun_normal: std 1/sqrt(fan_in), truncated at 2 std
    k = model.BC.kernel
    assert abs(float(k.std()) * math.sqrt(256) - 1.0) < 0.1
    assert float(k.abs().max()) <= 2.0 / 0.87962566103423978 / math.sqrt(256) + 1e-6


def test_split_weight_gradients_match_single_product(monkeypatch):
    """B*L = 2 * 8192 rows: the BC / dt / dt_proj weight gradients through the split
    product equal those of one a^T b call (same module, same input)."""
    from selectssm_amd import SelectiveSSM, modules

    m = SelectiveSSM(hidden_features=16, shift_conv_size=4, dt_rank=4, features=32, device="cuda", generator=_gen(3))
    x = _x((2, 8192, 32), 4)

    def grads():
        for p in m.parameters():
            p.grad = None
        m(x).square().sum().backward()
        return {k: p.grad.clone() for k, p in m.named_parameters()}

    split = grads()
    monkeypatch.setattr(modules, "_TN_SLICE", 1 << 40)
    single = grads()
    for k in split:
        ref = single[k].double()
        assert torch.allclose(split[k].double(), ref, rtol=1e-4, atol=1e-5 * float(ref.abs().max())), k
