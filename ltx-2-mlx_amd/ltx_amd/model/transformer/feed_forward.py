"""Feed-forward network: Linear -> GELU(tanh) -> Linear (feed_forward.py:37-112).

The GELU is fused into the first GEMM's epilogue; the second GEMM's epilogue
can fuse the block's gated residual add (see transformer.py).
"""

from __future__ import annotations

import torch

from ...kernels import gemm


class FeedForward:
    def __init__(self, project_in: gemm.LinearWeight, project_out: gemm.LinearWeight):
        self.project_in = project_in
        self.project_out = project_out
        self.dim = project_in.in_features
        self.inner_dim = project_in.out_features
        self.dim_out = project_out.out_features

    def weights(self) -> list[gemm.LinearWeight]:
        return [self.project_in, self.project_out]

    def hidden(self, x: torch.Tensor) -> torch.Tensor | gemm.MxRows:
        """bf16(gelu_tanh(bf16(x W1^T + b1))).  On the opt-in MX path
        (``gemm.MX_ACTIVATIONS``, MXFP8 weights, both products large enough)
        the hidden rows leave the up-projection already quantised
        (``gemm.MxRows``) for the down-projection."""
        m = x.numel() // self.dim
        if (gemm._mx_eligible(m, self.inner_dim, self.dim, self.project_in, gemm.TILE_AUTO)
                and gemm._mx_eligible(m, self.dim_out, self.inner_dim, self.project_out, gemm.TILE_AUTO)
                and x.dim() == 2):
            return gemm.linear_mx_gelu(gemm.MxRows(*gemm.quantize_rows_mxfp8(x)), self.project_in)
        return gemm.linear(x, self.project_in, epilogue=gemm.EPI_GELU)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        squeeze = x.dim() == 3
        x2 = x[0] if squeeze else x
        out = gemm.linear(self.hidden(x2), self.project_out)  # accepts MxRows
        return out[None] if squeeze else out
