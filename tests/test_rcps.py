"""RCPS wrappers (the reference's rcps.py): the reference's own tests
(tests/test_selectssm.py:98-150 of the reference: shapes and RC equivariance of
RCPSWrapper) plus equivariance of RCPSNorm, RCPSEmbedding and RCPSLMHead.
The wrappers are plain torch around the wrapped module and run on the CPU here;
the GPU test wraps BidirectionalMamba on the HIP kernels.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from selectssm_amd.rcps import Dense, RCPSEmbedding, RCPSLMHead, RCPSNorm, RCPSWrapper, RMSNorm, rc_conjugate

CMAP = [3, 2, 1, 0]  # A C G T -> T G C A


def _x(shape, seed, device="cpu"):
    g = torch.Generator(device=device).manual_seed(seed)
    return torch.randn(shape, generator=g, device=device)


def rc(z):
    return torch.flip(z, dims=(-2, -1))


class TestRCPS:
    def test_wrapper_shape(self):
        model = RCPSWrapper(module_cls=Dense, module_kwargs={"features": 32})
        x = _x((2, 16, 64), 0)  # 2D = 64 -> D = 32
        assert model(x).shape == x.shape

    def test_equivariance(self):
        """RC(f(x)) == f(RC(x)) for RCPSWrapper."""
        model = RCPSWrapper(module_cls=Dense, module_kwargs={"features": 32})
        x = _x((1, 16, 64), 1)
        y1 = rc(model(x))
        y2 = model(rc(x))
        assert torch.allclose(y1, y2, atol=1e-5)

    def test_norm_shape(self):
        model = RCPSNorm()
        x = _x((2, 16, 64), 2)
        assert model(x).shape == x.shape

    def test_embedding(self):
        model = RCPSEmbedding(vocab_size=4, d_model=16, complement_map=CMAP)
        tokens = torch.tensor([[0, 1, 2, 3]])
        assert model(tokens).shape == (1, 4, 32)  # 2 * d_model

    def test_lm_head(self):
        model = RCPSLMHead(vocab_size=4, complement_map=CMAP)
        x = _x((1, 8, 32), 3)
        assert model(x).shape == (1, 8, 4)


def test_rc_conjugate_is_the_group_action():
    x = _x((2, 5, 6), 4)
    y = rc_conjugate(x)
    assert torch.equal(y[1, 0, 0], x[1, -1, -1]) and torch.equal(y[0, 2, 1], x[0, 2, 4])
    assert torch.equal(rc_conjugate(y), x)


def test_norm_equivariance_with_a_non_symmetric_scale():
    model = RCPSNorm()
    x = _x((2, 9, 12), 5)
    model(x)
    with torch.no_grad():
        model.norm.scale.copy_(torch.linspace(0.5, 2.0, 6))
    assert torch.allclose(rc(model(x)), model(rc(x)), atol=1e-6)


def test_embedding_and_head_equivariance():
    """embed(RC(ids)) == RC(embed(ids)), and the head maps an RC'd input to the
    reversed sequence of complemented logits: head(RC(h))[l, v] = head(h)[L-1-l, cmap[v]]."""
    emb = RCPSEmbedding(vocab_size=4, d_model=8, complement_map=CMAP, generator=torch.Generator().manual_seed(6))
    ids = torch.tensor([[0, 1, 1, 3, 2, 0, 2]])
    rc_ids = torch.flip(torch.tensor(CMAP)[ids], dims=(-1,))
    assert torch.allclose(emb(rc_ids), rc(emb(ids)), atol=1e-7)
    head = RCPSLMHead(vocab_size=4, complement_map=CMAP, generator=torch.Generator().manual_seed(7))
    h = _x((2, 7, 16), 8)
    a = head(rc(h))
    b = head(h)[:, torch.arange(6, -1, -1)][..., torch.tensor(CMAP)]
    assert torch.allclose(a, b, atol=1e-5)
    # a sense-only input with a zero antisense half gives sense @ kernel + 2 bias... check the formula directly
    x = torch.cat([h[..., :8], torch.zeros_like(h[..., 8:])], dim=-1)
    assert torch.allclose(head(x), h[..., :8] @ head.kernel + 2 * head.bias, atol=1e-6)


def test_parameter_names_match_the_reference_tree():
    w = RCPSWrapper(module_cls=Dense, module_kwargs={"features": 4})
    w(_x((1, 3, 8), 9))
    assert set(dict(w.named_parameters())) == {"inner.kernel", "inner.bias"}
    n = RCPSNorm(norm_cls=RMSNorm)
    n(_x((1, 3, 8), 9))
    assert set(dict(n.named_parameters())) == {"norm.scale"}
    e = RCPSEmbedding(4, 8, CMAP)
    assert set(dict(e.named_parameters())) == {"embed.embedding"}
    h = RCPSLMHead(4, CMAP)
    h(_x((1, 3, 8), 9))
    assert set(dict(h.named_parameters())) == {"kernel", "bias"}
    with pytest.raises(ValueError, match="complement_map"):
        RCPSEmbedding(5, 8, CMAP)


@pytest.mark.gpu
def test_rcps_bidirectional_mamba_is_rc_equivariant_on_gpu():
    """The Caduceus-style stack: RCPSWrapper(BidirectionalMamba(complement, tied)) on the
    HIP kernels commutes with RC to fp32 rounding."""
    from selectssm_amd import BidirectionalMamba

    model = RCPSWrapper(module_cls=BidirectionalMamba,
                        module_kwargs=dict(hidden_features=16, expansion_factor=2.0, complement=True,
                                           tie_in_proj=True, tie_gate=True,
                                           generator=torch.Generator(device="cuda").manual_seed(0)))
    x = _x((2, 64, 64), 10, device="cuda")
    y1 = rc(model(x))
    y2 = model(rc(x))
    torch.cuda.synchronize()
    err = (y1 - y2).abs().max().item()
    assert err <= 1e-4 * max(1.0, y1.abs().max().item()), err
    (y1.square().sum()).backward()
    assert all(torch.isfinite(p.grad).all() for p in model.parameters())
