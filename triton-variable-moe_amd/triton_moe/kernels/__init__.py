"""gfx950 HIP kernel implementations of the MoE operations (same export
surface as triton_moe/kernels/__init__.py:18-40 of the reference)."""

from .gather import padded_gather, padded_gather_autograd
from .scatter import padded_scatter, padded_scatter_autograd
from .grouped_gemm import (
    grouped_gemm_up,
    grouped_gemm_down,
    grouped_gemm_up_backward,
    grouped_gemm_down_backward,
    grouped_gemm_up_autograd,
    grouped_gemm_down_autograd,
    precompute_gather_map,
    GroupedGemmUp,
    GroupedGemmDown,
)
from .fused_cumsum import fused_route

__all__ = [
    # Gather/Scatter
    "padded_gather",
    "padded_gather_autograd",
    "padded_scatter",
    "padded_scatter_autograd",
    # Forward kernels
    "grouped_gemm_up",
    "grouped_gemm_down",
    # Backward kernels
    "grouped_gemm_up_backward",
    "grouped_gemm_down_backward",
    # Autograd wrappers
    "grouped_gemm_up_autograd",
    "grouped_gemm_down_autograd",
    # Gather map for fused gather
    "precompute_gather_map",
    # Autograd Function classes
    "GroupedGemmUp",
    "GroupedGemmDown",
    # Routing
    "fused_route",
]
