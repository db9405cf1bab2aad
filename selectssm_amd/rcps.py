"""Reverse-complement parameter sharing (RCPS) wrappers, as torch modules.

Same classes, fields and parameter names as the reference's Flax wrappers
(rcps.py:42-174).  The group action is RC(x)[b, l, d] = x[b, L-1-l, D-1-d]
(rcps.py:10-19, 37-39).  The wrappers hold no scan of their own: the wrapped
module (e.g. :class:`~selectssm_amd.BidirectionalMamba`) runs on the HIP
kernels.  When the wrapped module (or norm) has a ``forward_rc`` method, as this
package's SelectiveSSM, BidirectionalMamba and norms do, the antisense half runs
through it: RC(M(RC(x))) computed by index maps in the kernels and permuted
parameters, with no flipped copy of an activation.  Any other module gets the
conjugation as materialised flips.

``module_cls`` / ``norm_cls`` are torch module classes whose instances build
their parameters from the first input, as Flax modules do (the modules of this
package, :class:`Dense` and :class:`RMSNorm` below).
"""
from __future__ import annotations

import math
from typing import Optional, Sequence

import torch
import torch.nn.functional as F

from .modules import _FlaxModule, lecun_normal_


def rc_conjugate(x: torch.Tensor) -> torch.Tensor:
    """Flip along the sequence (-2) and channel (-1) axes (rcps.py:37-39)."""
    return torch.flip(x, dims=(-2, -1))


def conjugated(module, x, **kwargs):
    """RC(module(RC(x))) (rcps.py:71): through ``module.forward_rc`` (index maps, no
    flipped activations) when the module has one, else with materialised flips."""
    if hasattr(module, "forward_rc"):
        return module.forward_rc(x, **kwargs)
    return rc_conjugate(module(rc_conjugate(x), **kwargs))


class Dense(_FlaxModule):
    """flax.linen.Dense(features): kernel (in, out) built from the first input, lecun_normal init."""

    def __init__(self, features: int, use_bias: bool = True, generator: Optional[torch.Generator] = None):
        super().__init__()
        self.out_features = features
        self.use_bias = use_bias
        self.generator = generator
        self.built = False

    def forward(self, x):
        if not self.built:
            fan_in = x.shape[-1]
            self.kernel = torch.nn.Parameter(lecun_normal_(
                torch.empty(fan_in, self.out_features, device=x.device), fan_in, self.generator))
            if self.use_bias:
                self.bias = torch.nn.Parameter(torch.zeros(self.out_features, device=x.device))
            self.built = True
        y = x @ self.kernel.to(x.dtype)
        return y + self.bias.to(x.dtype) if self.use_bias else y


class RMSNorm(_FlaxModule):
    """flax.linen.RMSNorm (epsilon 1e-6, learned scale), scale built from the first input."""

    def __init__(self, epsilon: float = 1e-6):
        super().__init__()
        self.epsilon = epsilon
        self.built = False

    def forward(self, x, flip: bool = False):
        if not self.built:
            self.scale = torch.nn.Parameter(torch.ones(x.shape[-1], device=x.device))
            self.built = True
        xf = x.float()
        scale = self.scale.flip(0) if flip else self.scale
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.epsilon) * scale
        return y.to(x.dtype)

    def forward_rc(self, x):
        """RC(self(RC(x))): the statistics of a row do not depend on its channel order,
        so this is the norm with its scale reversed."""
        return self.forward(x, flip=True)


class RCPSWrapper(_FlaxModule):
    """(B, L, 2D) -> (B, L, 2D): the inner (B, L, D) module on the sense half and,
    with shared weights, on the RC-conjugated antisense half (rcps.py:42-78)."""

    def __init__(self, module_cls: type, module_kwargs: Optional[dict] = None):
        super().__init__()
        self.module_cls = module_cls
        self.module_kwargs = dict(module_kwargs or {})
        self.inner = module_cls(**self.module_kwargs)

    def forward(self, x, **kwargs):
        D = x.shape[-1] // 2
        sense, antisense = x[..., :D], x[..., D:]
        sense_out = self.inner(sense, **kwargs)
        antisense_out = conjugated(self.inner, antisense, **kwargs)
        return torch.cat([sense_out, antisense_out], dim=-1)


class RCPSNorm(_FlaxModule):
    """RC-equivariant normalisation: one norm for both halves, the antisense half
    conjugated around it (rcps.py:81-105).  ``norm_cls`` defaults to RMSNorm."""

    def __init__(self, norm_cls: Optional[type] = None, norm_kwargs: Optional[dict] = None):
        super().__init__()
        self.norm_cls = norm_cls
        self.norm_kwargs = dict(norm_kwargs or {})
        self.norm = (norm_cls or RMSNorm)(**self.norm_kwargs)

    def forward(self, x, **kwargs):
        D = x.shape[-1] // 2
        sense = self.norm(x[..., :D], **kwargs)
        antisense = conjugated(self.norm, x[..., D:], **kwargs)
        return torch.cat([sense, antisense], dim=-1)


def _complement_map(cmap, n):
    cm = torch.as_tensor(list(cmap), dtype=torch.long)
    if cm.shape != (n,):
        raise ValueError(f"complement_map must have vocab_size={n} entries, got {tuple(cm.shape)}")
    return cm


class RCPSEmbedding(_FlaxModule):
    """(B, L) token ids -> (B, L, 2 d_model): embed(ids) and RC_conjugate(embed(RC(ids)))
    with RC(ids) the reversed, complemented ids (rcps.py:108-143)."""

    def __init__(self, vocab_size: int, d_model: int, complement_map: Sequence[int], device=None,
                 generator: Optional[torch.Generator] = None):
        super().__init__()
        self.vocab_size, self.d_model = vocab_size, d_model
        self.register_buffer("cmap", _complement_map(complement_map, vocab_size).to(device), persistent=False)
        self.embed = torch.nn.Module()
        # flax.linen.Embed default init: normal with variance 1/d_model
        w = torch.empty(vocab_size, d_model, device=device)
        with torch.no_grad():
            w.normal_(0.0, 1.0 / math.sqrt(d_model), generator=generator)
        self.embed.embedding = torch.nn.Parameter(w)

    def forward(self, input_ids):
        table = self.embed.embedding
        sense = F.embedding(input_ids, table)
        # RC(embed(RC(ids)))[l, d] = table[cmap[ids[l]], D-1-d]: the sequence reversals
        # cancel and the channel reversal moves onto the (vocab, D) table
        antisense = F.embedding(self.cmap.to(input_ids.device)[input_ids], table.flip(-1))
        return torch.cat([sense, antisense], dim=-1)


class RCPSLMHead(_FlaxModule):
    """(B, L, 2D) -> (B, L, vocab): sense logits plus channel-flipped antisense logits
    through the complement-reindexed kernel (rcps.py:146-174)."""

    def __init__(self, vocab_size: int, complement_map: Sequence[int], generator: Optional[torch.Generator] = None):
        super().__init__()
        self.vocab_size = vocab_size
        self.register_buffer("cmap", _complement_map(complement_map, vocab_size), persistent=False)
        self.generator = generator
        self.built = False

    def forward(self, x):
        D = x.shape[-1] // 2
        if not self.built:
            self.kernel = torch.nn.Parameter(lecun_normal_(torch.empty(D, self.vocab_size, device=x.device), D,
                                                           self.generator))
            self.bias = torch.nn.Parameter(torch.zeros(self.vocab_size, device=x.device))
            self.built = True
        sense, antisense = x[..., :D], x[..., D:]
        k = self.kernel.to(x.dtype)
        b = self.bias.to(x.dtype)
        fwd_logits = sense @ k + b
        # flip(antisense, channels) @ k[:, cmap] = antisense @ (k with its rows reversed)[:, cmap]
        rc_logits = antisense @ k.flip(0)[:, self.cmap.to(x.device)] + b
        return fwd_logits + rc_logits
