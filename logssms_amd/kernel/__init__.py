"""Kernel entry points mirroring ``logssms.kernel`` for the GDN path."""

from .fused import prepare_gdn
from .norm import rms_norm_gated
from .store import store_state

__all__ = ["prepare_gdn", "rms_norm_gated", "store_state"]
