"""Layer-level mirrors of ``logssms.layers`` for the GDN path."""

from .gated_delta import GatedDeltaConfig

__all__ = ["GatedDeltaConfig"]
