"""Text-connector weights from a stock LTX-2.3 checkpoint
(model/text_encoder/encoder.py:147-222, :409-434).

Keys read:
  text_embedding_projection.{video,audio}_aggregate_embed.{weight,bias}
  model.diffusion_model.{video,audio}_embeddings_connector.learnable_registers
  model.diffusion_model.{video,audio}_embeddings_connector.transformer_1d_blocks.<i>.
      attn1.{to_q,to_k,to_v,to_out.0,to_gate_logits}.{weight,bias},
      attn1.{q_norm,k_norm}.weight, ff.net.0.proj.{weight,bias}, ff.net.2.{weight,bias}
The block projections go into the fused self-attention layout
[to_q; to_k; to_v; to_gate_logits] like the DiT's; the aggregate-embedding
weights get their input columns permuted to the feature extractor's
layer-major order.  Missing, unexpected and mis-shaped tensors are reported
before anything is written (``strict``).
"""

from __future__ import annotations

import re
from pathlib import Path

from .resident import _FileSource, _Planner, run_plan
from .safetensors_file import SafetensorsFile

_PREFIXES = {
    "text_embedding_projection.": "feature_extractor.",
    "model.diffusion_model.video_embeddings_connector.": "embeddings_connector.",
    "model.diffusion_model.audio_embeddings_connector.": "audio_embeddings_connector.",
}
_RENAMES = (
    (re.compile(r"\.to_out\.0\."), ".to_out."),
    (re.compile(r"\.ff\.net\.0\.proj\."), ".ff.project_in.proj."),
    (re.compile(r"\.ff\.net\.2\."), ".ff.project_out."),
)


class TextConnectorSource(_FileSource):
    """The connector / text-projection tensors of a checkpoint by module path."""

    def __init__(self, path: str | Path):
        super().__init__()
        f = SafetensorsFile(path)
        self.names: dict[str, str] = {}
        for k in f.keys():
            self._where[k] = f
            for pre, repl in _PREFIXES.items():
                if k.startswith(pre):
                    name = repl + k[len(pre):]
                    for pat, sub in _RENAMES:
                        name = pat.sub(sub, name)
                    self.names[name] = k
                    break

    def source_keys(self) -> set[str]:
        return set(self.names.values())

    def tensor_key(self, name: str) -> str | None:
        return self.names.get(name)

    def linear(self, base: str):
        from .resident import LinearRecord

        k = self.names.get(base + ".weight")
        if k is None:
            return None
        n, kk = self.shape(k)
        return LinearRecord(base, "bf16", (n, kk), (k,))


def load_av_text_connector_weights(encoder, weights_path: str | Path, *, strict: bool = True) -> int:
    """Load the feature-extractor projections and both connectors; returns the
    number of tensors loaded."""
    from ..model.text_encoder.feature_extractor import permute_aggregate_weight

    src = TextConnectorSource(weights_path)
    p = _Planner(src)
    fe = encoder.feature_extractor
    for name in ("video_aggregate_embed", "audio_aggregate_embed"):
        lw = getattr(fe, name)
        p.matrix(lw, "w", f"feature_extractor.{name}",
                 transform=lambda w: permute_aggregate_weight(w, fe.hidden_dim, fe.num_layers))
        p.vector(lw.bias, f"feature_extractor.{name}.bias")
    for cname in ("embeddings_connector", "audio_embeddings_connector"):
        c = getattr(encoder, cname)
        if c.learnable_registers is not None:
            p.vector(c.learnable_registers, f"{cname}.learnable_registers")
        for i, blk in enumerate(c.transformer_1d_blocks):
            p.attention(blk.attn1, f"{cname}.transformer_1d_blocks.{i}.attn1")
            p.ff(blk.ff, f"{cname}.transformer_1d_blocks.{i}.ff")
    plan = p.plan
    extra = sorted(src.source_keys() - plan.consumed)
    if plan.errors:
        raise ValueError("weights do not fit the connector: " + "; ".join(plan.errors[:8]))
    if strict and plan.missing:
        raise ValueError(f"{len(plan.missing)} tensors missing, e.g. " + ", ".join(plan.missing[:8]))
    if strict and extra:
        raise ValueError(f"{len(extra)} tensors have no place in the connector, e.g. " + ", ".join(extra[:8]))
    run_plan(plan, src, None, encoder.embeddings_connector.device)
    return len(plan.consumed)
