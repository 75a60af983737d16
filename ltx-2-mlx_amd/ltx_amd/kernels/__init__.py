"""HIP kernels of the denoise path (drop-in for LTX_2_MLX.kernels)."""

from .fused_ops import adaln_norm_fused, gated_add_fused

__all__ = ["adaln_norm_fused", "gated_add_fused"]
