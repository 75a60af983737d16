"""Weights into HBM: random initialisation, stock checkpoints (bf16 / FP8)
and the reference's transformer cache."""

from .transformer_cache import (  # noqa: F401
    TransformerCacheResult,
    build_transformer_cache,
    load_transformer_cache,
    open_transformer_cache,
)
from .weight_converter import convert_pytorch_key_to_mlx, load_transformer_weights  # noqa: F401
