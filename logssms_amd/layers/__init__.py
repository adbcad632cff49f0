"""Layer-level mirrors of ``logssms.layers`` for the GDN path."""

from .gated_delta import GatedDeltaConfig
from .norm import RMSNormGated

__all__ = ["GatedDeltaConfig", "RMSNormGated"]
