"""Job-config fields of the converter (src/sfu_repro/torchtitan/config.py:1-29)."""

from dataclasses import dataclass, field
from typing import Literal


@dataclass
class SFUConfig:
    """One intervention (case B1..B5) and its variant."""

    case: Literal["b1", "b2", "b3", "b4", "b5"] = "b1"
    variant: Literal["native", "polynomial", "pwl2_safe_f16", "d2_safe"] = "native"
    strict: bool = True
    """Require the expected model family and number of patched modules."""


@dataclass
class JobConfig:
    """Fields merged into TorchTitan's ``JobConfig`` at parse time."""

    sfu: SFUConfig = field(default_factory=SFUConfig)


__all__ = ["JobConfig", "SFUConfig"]
