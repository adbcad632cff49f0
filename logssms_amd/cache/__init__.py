"""State pools and prefix-cache state I/O for the GDN path.

* ``LinearStatePool`` -- conv-window pool + recurrent-state pool
  (reference ``python/logssms/cache/radix/state_pool.py:12-41``), with the
  recurrent state in fp32 by default.
* ``HybridBlockLayout`` / ``HybridBlockPool`` -- the Marconi shared KV/state
  block storage and its state copy / zero / metadata mapping
  (``python/logssms/cache/marconi/{layout,block_pool}.py``);
  ``MarconiCheckpointer`` / ``MarconiRequestState`` -- its checkpoint
  placement and post-forward checkpoint copies
  (``cache/marconi/manager.py:248-278``).
* ``commit_speculative`` (host slot remap) and ``commit_accepted`` (device
  copy) -- spec-decode verify commit (``python/logssms/cache/radix/manager.py:248-268``).
"""

from .marconi import HybridBlockLayout, HybridBlockPool, MarconiCheckpointer, MarconiRequestState
from .speculative import commit_accepted, commit_speculative
from .state_pool import LinearStatePool

__all__ = ["HybridBlockLayout", "HybridBlockPool", "LinearStatePool", "MarconiCheckpointer", "MarconiRequestState",
           "commit_accepted", "commit_speculative"]
