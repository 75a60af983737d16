"""Audio+video text conditioning after Gemma (model/text_encoder/encoder.py:
52-122, :283-338): the V2 feature extractor and one connector per modality.

``encode_from_hidden_states(hidden_states, attention_mask)`` returns the
video and audio contexts of the denoise loop; the Gemma language model that
produces the hidden states is not part of this build (its hidden states are
an input).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .connector import Embeddings1DConnector
from .feature_extractor import GemmaFeaturesExtractorV2


@dataclass
class AudioVideoGemmaEncoderOutput:
    video_encoding: torch.Tensor
    audio_encoding: torch.Tensor
    attention_mask: torch.Tensor


class AudioVideoTextConnector:
    """``AudioVideoGemmaTextEncoderModel`` without the Gemma model."""

    def __init__(self, feature_extractor: GemmaFeaturesExtractorV2, embeddings_connector: Embeddings1DConnector,
                 audio_embeddings_connector: Embeddings1DConnector):
        self.feature_extractor = feature_extractor
        self.embeddings_connector = embeddings_connector
        self.audio_embeddings_connector = audio_embeddings_connector

    def encode_from_hidden_states(self, hidden_states, attention_mask: torch.Tensor,
                                  padding_side: str = "left") -> AudioVideoGemmaEncoderOutput:
        video_in, audio_in = self.feature_extractor.extract_from_hidden_states(hidden_states, attention_mask,
                                                                               padding_side)
        # with learnable registers the connector clears the mask: every
        # output position is valid, so the binary mask is all ones
        video, out_mask = self.embeddings_connector(video_in)
        audio, _ = self.audio_embeddings_connector(audio_in)
        binary = (out_mask.reshape(1, -1) >= -0.5).to(torch.int32)
        return AudioVideoGemmaEncoderOutput(video_encoding=video, audio_encoding=audio, attention_mask=binary)

    __call__ = encode_from_hidden_states


def create_av_text_connector_v2(hidden_dim: int = 3840, num_gemma_layers: int = 49, video_inner_dim: int = 4096,
                                audio_inner_dim: int = 2048, video_connector_heads: int = 32,
                                video_connector_head_dim: int = 128, audio_connector_heads: int = 32,
                                audio_connector_head_dim: int = 64, connector_layers: int = 8,
                                num_registers: int = 128, positional_embedding_max_pos: list | None = None,
                                *, device="cuda", init: str = "random", seed: int = 0) -> AudioVideoTextConnector:
    """The V2 (LTX-2.3) configuration (encoder.py:283-338)."""
    fe = GemmaFeaturesExtractorV2(hidden_dim, num_gemma_layers, video_inner_dim, audio_inner_dim, device=device,
                                  init=init, seed=seed)
    kw = dict(num_layers=connector_layers, num_learnable_registers=num_registers,
              positional_embedding_max_pos=positional_embedding_max_pos, device=device, init=init)
    video = Embeddings1DConnector(video_connector_head_dim, video_connector_heads, seed=seed + 1, **kw)
    audio = Embeddings1DConnector(audio_connector_head_dim, audio_connector_heads, seed=seed + 2, **kw)
    return AudioVideoTextConnector(fe, video, audio)
