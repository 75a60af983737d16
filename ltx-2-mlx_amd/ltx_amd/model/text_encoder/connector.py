"""Text-embeddings connector (model/text_encoder/connector.py:12-281).

``Embeddings1DConnector`` turns the projected Gemma features of one modality
into the transformer's text context: the sequence is extended with learnable
register tokens to a multiple of the register count of at least 1024 tokens
(the mask is cleared, every position attends to every other), RoPE over the
1-D token index, ``num_layers`` ``BasicTransformerBlock1D``s, and a final
RMSNorm.  A block is ``x + attn1(rms_norm(x))`` then ``x + ff(rms_norm(x))``
with the same gated self-attention and feed-forward as the DiT blocks.

Kernels: ``rms_norm`` is the AdaLN kernel with zero scale/shift (one
rounding, ``mx.fast.rms_norm`` without weight); each residual add rides on
the to_out / FF-down GEMM epilogue with a unit gate (``bf16(x + y)``, the
bf16 add of the reference); attention is the fused QKV+gate GEMM, QK-norm +
RoPE and flash attention of the DiT.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from ...kernels import gemm
from ...loader.weights import build_attention, build_ff
from ..transformer.rope import rope_tables
from ..transformer.transformer import adaln


class BasicTransformerBlock1D:
    """Self-attention + feed-forward block without modulation (connector.py:12-97)."""

    def __init__(self, dim: int, heads: int, dim_head: int, norm_eps: float = 1e-6, *, device="cuda",
                 weight_format: str = "bf16", init: str = "random", generator=None):
        self.dim = dim
        self.norm_eps = norm_eps
        self.attn1 = build_attention(dim, None, heads, dim_head, gen=generator, device=device,
                                     weight_format=weight_format, norm_eps=norm_eps, init=init)
        self.ff = build_ff(dim, gen=generator, device=device, weight_format=weight_format, init=init)
        self._zeros = torch.zeros(dim, dtype=torch.float32, device=device)
        self._ones = torch.ones(dim, dtype=torch.float32, device=device)

    def rms_norm(self, x: torch.Tensor) -> torch.Tensor:
        return adaln(x, self._zeros, self._zeros, self.norm_eps, 0)

    def __call__(self, x: torch.Tensor, pe=None) -> torch.Tensor:
        """x: (T, D) bf16 -> new (T, D) bf16."""
        o = self.attn1.core(self.rms_norm(x), pe=pe)
        x = gemm.linear(o, self.attn1.to_out, epilogue=gemm.EPI_RESIDUAL, residual=x, gate=self._ones)
        f = self.ff.hidden(self.rms_norm(x))
        return gemm.linear(f, self.ff.project_out, epilogue=gemm.EPI_RESIDUAL, residual=x, gate=self._ones)


class Embeddings1DConnector:
    """Register extension, 1-D RoPE, transformer blocks, final RMSNorm
    (connector.py:100-281)."""

    def __init__(self, attention_head_dim: int = 128, num_attention_heads: int = 32, num_layers: int = 8,
                 positional_embedding_theta: float = 10000.0, positional_embedding_max_pos: list | None = None,
                 num_learnable_registers: int | None = 128, norm_eps: float = 1e-6, *, device="cuda",
                 weight_format: str = "bf16", init: str = "random", seed: int = 0):
        self.device = torch.device(device)
        self.num_attention_heads = num_attention_heads
        self.inner_dim = num_attention_heads * attention_head_dim
        self.positional_embedding_theta = positional_embedding_theta
        self.positional_embedding_max_pos = list(positional_embedding_max_pos or [1])
        self.norm_eps = norm_eps
        gen = None
        if init == "random":
            gen = torch.Generator(device=self.device)
            gen.manual_seed(seed)
        self.transformer_1d_blocks = [
            BasicTransformerBlock1D(self.inner_dim, num_attention_heads, attention_head_dim, norm_eps,
                                    device=self.device, weight_format=weight_format, init=init, generator=gen)
            for _ in range(num_layers)]
        self.num_learnable_registers = num_learnable_registers
        self.learnable_registers = None
        if num_learnable_registers:
            if init == "random":  # uniform in [-1, 1], as the reference initialises them
                r = torch.rand((num_learnable_registers, self.inner_dim), generator=gen, device=self.device)
                self.learnable_registers = (r * 2 - 1).to(torch.bfloat16)
            else:
                self.learnable_registers = torch.zeros((num_learnable_registers, self.inner_dim),
                                                       dtype=torch.bfloat16, device=self.device)
        self._zeros = torch.zeros(self.inner_dim, dtype=torch.float32, device=self.device)
        self._pe_cache: dict = {}

    def extended_length(self, seq_len: int) -> int:
        """Sequence length after the register extension."""
        if not self.num_learnable_registers:
            return seq_len
        n = self.num_learnable_registers
        return math.ceil(max(1024, seq_len) / n) * n

    def append_learnable_registers(self, x: torch.Tensor) -> torch.Tensor:
        """(T, D) -> (L, D): rows T.. of the tiled registers appended (row i is
        register i mod R) (connector.py:174-222)."""
        t = x.shape[0]
        total = self.extended_length(t)
        if total == t:
            return x
        reps = total // self.num_learnable_registers
        tiled = self.learnable_registers.repeat(reps, 1)
        return torch.cat([x, tiled[t:]], 0)

    def rope(self, seq_len: int):
        """cos/sin tables over token indices 0..L-1 (connector.py:248-262): the
        fractional position is index / max_pos, float64 frequency grid."""
        if seq_len not in self._pe_cache:
            idx = np.arange(seq_len, dtype=np.float32)
            positions = np.stack([idx, idx], -1)[None, None]  # start == end: the index itself
            self._pe_cache[seq_len] = rope_tables(positions, self.inner_dim, self.positional_embedding_max_pos,
                                                  self.device, theta=self.positional_embedding_theta)
        return self._pe_cache[seq_len]

    def __call__(self, hidden_states: torch.Tensor, attention_mask=None):
        """(1, T, D) or (T, D) bf16 -> ((1, L, D) bf16, additive mask zeros (1, 1, 1, L))."""
        x = hidden_states[0] if hidden_states.dim() == 3 else hidden_states
        if x.dtype != torch.bfloat16:
            raise TypeError("the connector runs on bf16 features")
        if self.num_learnable_registers:
            x = self.append_learnable_registers(x)
        x = x.contiguous()
        pe = self.rope(x.shape[0])
        for block in self.transformer_1d_blocks:
            x = block(x, pe=pe)
        x = adaln(x, self._zeros, self._zeros, self.norm_eps, 0)
        mask = torch.zeros((1, 1, 1, x.shape[0]), dtype=torch.float32, device=x.device)
        return x[None], mask
