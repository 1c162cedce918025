"""The part of moe-engine's ``pkg.models`` that sits in front of the routed path: ``RMSNorm`` and
``ToyMoEBlock`` (moe-engine/pkg/models/moe.py L:63-126).  The language-model wrappers of that package
(``ToyMoEModel``, the registry) are outside this build's scope."""

from .moe import RMSNorm, ToyMoEBlock

__all__ = ["RMSNorm", "ToyMoEBlock"]
