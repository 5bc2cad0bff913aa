"""MI355X-native variable-width MoE MLP (drop-in for triton_moe of
hbfreed/triton-variable-moe), running on hand-written gfx950 HIP kernels."""

from .moe import TritonMoEConfig, TritonMoEMLP

__all__ = ["TritonMoEConfig", "TritonMoEMLP"]
