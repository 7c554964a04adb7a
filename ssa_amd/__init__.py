"""ssa_amd — SSA's routed block-sparse attention hot path, native to MI355X (gfx950).

Python host code over PyTorch-ROCm (device memory and streams) calling hand-written HIP kernels
in libssa_hip.so through its C ABI (include/ssa_hip.h). Modules mirror the reference's operator
API so callers switch by import path:

    ssa.ssa_kernel  -> ssa_amd.ssa_kernel   (block_route, block_route_budget, ssa_flex, dense)
    ssa.gemma_ssa   -> ssa_amd.gemma_ssa    (SSAConfig, ssa_attention_forward, install_ssa)
    ssa.ivf_decode  -> ssa_amd.ivf_decode   (decode_attend, dense_decode, RoutedDecoder)
"""
from . import _lib  # noqa: F401
from . import torch_ops  # noqa: F401  (registers the ssa_amd:: custom ops for torch.compile)

__all__ = ["ssa_kernel", "gemma_ssa", "ivf_decode", "workloads"]
