"""AdaLN timestep MLPs on the per-step scalar timestep (timestep_embedding.py).

``AdaLayerNormSingle(t) -> (emb (N*D), embedded_timestep (D))`` with
sinusoid(256, flip_sin_to_cos, shift 0) -> linear_1 -> SiLU -> linear_2
(= embedded_timestep) -> SiLU -> linear(D -> N*D) (:126-201).  The three
layers run as fp32-activation / bf16-weight GEMV kernels; the final layer
writes straight into a slice of the caller's modulation-row buffer.
"""

from __future__ import annotations

import torch

from ... import _lib

SINUSOID_DIM = 256


class AdaLayerNormSingle:
    def __init__(self, dim: int, num_embeddings: int, *, device="cuda", generator: torch.Generator | None = None,
                 std: float = 0.02, init: str = "random"):
        g = generator

        def rnd(shape):
            if init == "empty":  # storage for a checkpoint loader
                return torch.empty(shape, dtype=torch.bfloat16, device=device)
            return (torch.randn(shape, generator=g, device=device, dtype=torch.float32) * std).to(torch.bfloat16)

        self.dim = dim
        self.num_embeddings = num_embeddings
        self.w1, self.b1 = rnd((dim, SINUSOID_DIM)), torch.zeros(dim, device=device)
        self.w2, self.b2 = rnd((dim, dim)), torch.zeros(dim, device=device)
        self.w, self.b = rnd((num_embeddings * dim, dim)), torch.zeros(num_embeddings * dim, device=device)

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.w1, self.b1, self.w2, self.b2, self.w, self.b))

    def __call__(self, t_value: torch.Tensor, multiplier: float, out: torch.Tensor,
                 embedded: torch.Tensor | None = None, scratch: tuple | None = None) -> None:
        """t_value: fp32 device scalar (1,); writes emb (N*D) into ``out`` and,
        if given, embedded_timestep (D) into ``embedded``."""
        dev = out.device
        stream = _lib.stream_of(out)
        if scratch is None:
            sin = torch.empty(SINUSOID_DIM, device=dev)
            h1 = torch.empty(self.dim, device=dev)
            h2 = torch.empty(self.dim, device=dev) if embedded is None else embedded
        else:
            sin, h1, h2 = scratch
            if embedded is not None:
                h2 = embedded
        _lib.call("ltx_timestep_embedding_f32", t_value.data_ptr(), 1, float(multiplier), sin.data_ptr(),
                  SINUSOID_DIM, stream)
        _lib.call("ltx_gemv_f32_bf16w", sin.data_ptr(), 1, SINUSOID_DIM, self.w1.data_ptr(), self.b1.data_ptr(),
                  h1.data_ptr(), self.dim, _lib.GEMV_SILU_OUTPUT, stream)
        _lib.call("ltx_gemv_f32_bf16w", h1.data_ptr(), 1, self.dim, self.w2.data_ptr(), self.b2.data_ptr(),
                  h2.data_ptr(), self.dim, 0, stream)
        _lib.call("ltx_gemv_f32_bf16w", h2.data_ptr(), 1, self.dim, self.w.data_ptr(), self.b.data_ptr(),
                  out.data_ptr(), self.num_embeddings * self.dim, _lib.GEMV_SILU_INPUT, stream)
