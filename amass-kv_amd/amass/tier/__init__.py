"""mem-v tier: pinned device-mapped host V pool, exact-LRU HBM hot buffer, miss fetch
(kernel or copy engine) and the tiered decode (reference surface tier/__init__.py:28-41)."""
from __future__ import annotations

from .decode_mem import mem_decode, mem_dynamic_decode
from .dma import CopyEngine
from .pool import MappedHostVPool
from .residency import Residency
from .staging import Staging
from .tier import Tier, TierVSource

__all__ = ["Tier", "TierVSource", "MappedHostVPool", "Residency", "Staging", "CopyEngine",
           "mem_decode", "mem_dynamic_decode"]
