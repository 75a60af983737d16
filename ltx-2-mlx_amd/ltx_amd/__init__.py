"""ltx_amd: MI355X-native (gfx950) LTX-2.3 audio+video DiT denoise path.

Host code is PyTorch-ROCm; every hot-path computation runs in the HIP kernels
of libltx_hip.so (C ABI declared in include/ltx_hip.h, bound in ``_lib``).
Module layout mirrors the reference package LTX_2_MLX:

    kernels/            fused_ops (adaln_norm_fused, gated_add_fused),
                        gemm (bf16 / int8 W8A16 / MXFP8 projections),
                        attention (flash attention, maybe_steel_attention)
    model/transformer/  rope, attention, feed_forward, transformer
                        (BasicAVTransformerBlock), timestep_embedding, model
    loader/             quantized weight formats (MXFP8, int8 per-channel)
    components/         distilled sigmas, Euler step, noiser, positions
"""

__version__ = "0.1.0"
