"""selectssm_amd — MI355X (gfx950) selective scan behind the selectssm API.

The hot path of ``selectssm`` (the selective scan y = scan(u, dt, A, B, C) with
its custom-VJP backward, plus the scan-adjacent epilogue of ``SelectiveSSM`` /
``BidirectionalMamba`` and the causal conv + activation before the scan) runs as
hand-written HIP kernels exported through the C ABI in ``include/selectssm.h``.
There is no CPU fallback.
"""
from .conv import conv1d_act
from .modules import BidirectionalMamba, SelectiveSSM
from .rcps import RCPSEmbedding, RCPSLMHead, RCPSNorm, RCPSWrapper
from .scan import (
    SelectiveScanFn,
    largest_factor_up_to,
    resolve_chunking,
    selective_scan,
    ssm_chunked_scan,
    ssm_recursive_scan,
    ssm_scan,
)

__all__ = [
    "BidirectionalMamba",
    "RCPSEmbedding",
    "RCPSLMHead",
    "RCPSNorm",
    "RCPSWrapper",
    "SelectiveSSM",
    "SelectiveScanFn",
    "conv1d_act",
    "largest_factor_up_to",
    "resolve_chunking",
    "selective_scan",
    "ssm_chunked_scan",
    "ssm_recursive_scan",
    "ssm_scan",
]
