"""STG attention perturbations (components/perturbations.py:1-200).

A perturbation names an attention sub-layer to skip (the whole residual
update vanishes, transformer.py:430-470, :576-625) in a set of blocks (None:
all blocks).  The block asks ``all_in_batch(type, block_idx)``; with batch
size 1 that is the one sample's configuration.  Host-side configuration only.
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import Enum


class PerturbationType(Enum):
    SKIP_A2V_CROSS_ATTN = "skip_a2v_cross_attn"
    SKIP_V2A_CROSS_ATTN = "skip_v2a_cross_attn"
    SKIP_VIDEO_SELF_ATTN = "skip_video_self_attn"
    SKIP_AUDIO_SELF_ATTN = "skip_audio_self_attn"


def _as_type(t) -> PerturbationType:
    return t if isinstance(t, PerturbationType) else PerturbationType(t)


@dataclass(frozen=True)
class Perturbation:
    """Skip ``type`` in ``blocks`` (None: every block)."""

    type: PerturbationType
    blocks: list[int] | None = None

    def is_perturbed(self, perturbation_type, block: int) -> bool:
        if self.type != _as_type(perturbation_type):
            return False
        return self.blocks is None or block in self.blocks


@dataclass(frozen=True)
class PerturbationConfig:
    """The perturbations of one sample."""

    perturbations: list[Perturbation] | None = None

    def is_perturbed(self, perturbation_type, block: int) -> bool:
        if not self.perturbations:
            return False
        return any(p.is_perturbed(perturbation_type, block) for p in self.perturbations)

    @staticmethod
    def empty() -> "PerturbationConfig":
        return PerturbationConfig(perturbations=[])


@dataclass(frozen=True)
class BatchedPerturbationConfig:
    """One ``PerturbationConfig`` per batch sample."""

    perturbations: list[PerturbationConfig]

    def mask(self, perturbation_type, block: int) -> list[float]:
        """1.0 keeps, 0.0 skips the attention, per sample."""
        return [0.0 if p.is_perturbed(perturbation_type, block) else 1.0 for p in self.perturbations]

    def all_in_batch(self, perturbation_type, block: int) -> bool:
        return all(p.is_perturbed(perturbation_type, block) for p in self.perturbations)

    @staticmethod
    def empty(batch_size: int) -> "BatchedPerturbationConfig":
        return BatchedPerturbationConfig(perturbations=[PerturbationConfig.empty() for _ in range(batch_size)])


def create_stg_perturbation(skip_video_self_attn: bool = True, blocks: list[int] | None = None) -> PerturbationConfig:
    """The usual STG configuration: video self-attention skipped."""
    perturbations = []
    if skip_video_self_attn:
        perturbations.append(Perturbation(type=PerturbationType.SKIP_VIDEO_SELF_ATTN, blocks=blocks))
    return PerturbationConfig(perturbations=perturbations)


def create_batched_stg_config(batch_size: int, skip_video_self_attn: bool = True,
                              blocks: list[int] | None = None) -> BatchedPerturbationConfig:
    """The same STG perturbation for every sample of a batch."""
    return BatchedPerturbationConfig(
        perturbations=[create_stg_perturbation(skip_video_self_attn, blocks) for _ in range(batch_size)])


def modality_isolation_config() -> BatchedPerturbationConfig:
    """Both cross-modal attentions skipped in every block: the modality-isolated
    pass of the multi-modal guider (pipelines/two_stage.py:349-354)."""
    return BatchedPerturbationConfig([PerturbationConfig([
        Perturbation(type=PerturbationType.SKIP_A2V_CROSS_ATTN, blocks=None),
        Perturbation(type=PerturbationType.SKIP_V2A_CROSS_ATTN, blocks=None),
    ])])
