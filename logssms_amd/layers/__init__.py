"""Layer-level mirrors of ``logssms.layers`` for the GDN path."""

from .gated_delta import GatedDeltaConfig, GatedDeltaNet
from .norm import RMSNormGated

__all__ = ["GatedDeltaConfig", "GatedDeltaNet", "RMSNormGated"]
