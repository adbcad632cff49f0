"""Kernel entry points mirroring ``logssms.kernel`` for the GDN path."""

from .fused import prepare_gdn
from .store import store_state

__all__ = ["prepare_gdn", "store_state"]
