"""TorchTitan adapter for the B1--B5 interventions (the reference's
``src/sfu_repro/torchtitan``): ``SFUConfig`` job fields and the
``SFUReproConverter`` model converter in :mod:`sfu_repro.torchtitan.plugin`.
The package imports without TorchTitan; the plugin registers itself with
TorchTitan only where TorchTitan is installed."""

from .config import JobConfig, SFUConfig

__all__ = ["JobConfig", "SFUConfig"]
