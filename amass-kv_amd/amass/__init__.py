"""AMASS decode-time sparse attention, MI355X-native (gfx950 HIP kernels).

Drop-in for the hot path of Js-Hwang1/amass-kv (``src/amass/__init__.py:19-31``):

  from amass import AmassConfig, register        # register() = vLLM general plugin

  config.py     AmassConfig (same fields / AMASS_CONFIG rules as the reference)
  selection/    Stage A: quad / r8 page scores, derive, top-b and coverage selection
  attention/    Stage B: split-K / fused sparse paged decode (+ dense paged baseline)
  tier/         mem-v: pinned host V pool, exact-LRU hot buffer, fetch, tiered decode
  backend/      vLLM plugin boundary (attention impl, metadata builder, register())
  _hip.py       ctypes binding of libamass_hip.so (include/amass_hip.h)
"""
from __future__ import annotations

from .config import AmassConfig  # noqa: F401

__all__ = ["AmassConfig", "register"]

__version__ = "0.1.1"


def register() -> None:
    """vLLM general-plugin entry point (re-export of amass.backend.register.register)."""
    from .backend.register import register as _register
    _register()
