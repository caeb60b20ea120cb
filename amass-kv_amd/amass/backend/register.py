"""register() -- the vLLM general-plugin entry point, for vLLM on ROCm.

Reference: ``backend/register.py:26-86``.  There, register() builds the one AmassConfig
and patches ``CudaPlatform.get_attn_backend_cls`` so that where vLLM would choose the
FlashAttention backend it gets a FlashAttentionBackend subclass carrying the AMASS impl
and metadata builder.  On ROCm, vLLM chooses among several attention backends (Triton,
ROCm, AITER flash attention ...), so this register() patches ``RocmPlatform.
get_attn_backend_cls`` and, for whichever non-MLA decoder backend it returns, hands
back a subclass of THAT backend whose impl and builder are the AMASS mixins over the
backend's own impl and builder (attn.py, builder.py).  ``get_name()`` is inherited, so
vLLM's backend-name lookups still resolve; every non-decode path stays the stock one.

``AMASS_DISABLE=1`` makes register() inert (reference register.py:53); the config is
read from ``AMASS_CONFIG`` plus explicit overrides (``AmassConfig.load``).
"""
from __future__ import annotations

import importlib
import os
import sys

from ..config import AmassConfig
from . import _runtime
from .attn import make_impl
from .builder import make_builder

_APPLIED = False
_WRAPPED: dict = {}          # base backend qualname -> generated class name


def _resolve(qualname: str):
    mod, _, attr = qualname.rpartition(".")
    return getattr(importlib.import_module(mod), attr)


def wrap_backend(base_path: str) -> str:
    """Qualified name of the AMASS subclass of the backend at ``base_path`` (created
    once and published in this module so vLLM can import it by name)."""
    name = _WRAPPED.get(base_path)
    if name is None:
        base = _resolve(base_path)
        impl = make_impl(base.get_impl_cls())
        builder = make_builder(base.get_builder_cls())
        name = f"Amass_{base.__name__}"
        cls = type(name, (base,), {
            "get_impl_cls": staticmethod(lambda: impl),
            "get_builder_cls": staticmethod(lambda: builder),
            "__doc__": f"{base.__name__} with the AMASS decode impl and metadata builder.",
        })
        setattr(sys.modules[__name__], name, cls)
        _WRAPPED[base_path] = name
    return f"{__name__}.{name}"


def _is_mla(args, kwargs) -> bool:
    if kwargs.get("use_mla"):
        return True
    attn_sel = kwargs.get("attn_selector_config")
    return bool(getattr(attn_sel, "use_mla", False))


def register(overrides: dict | None = None) -> None:
    """vLLM general-plugin entry point (runs in every engine process)."""
    global _APPLIED
    if _APPLIED or os.environ.get("AMASS_DISABLE"):
        return
    cfg = AmassConfig.load(overrides)
    _runtime.set_config(cfg)

    from vllm.platforms import rocm
    target = next(k for k in rocm.RocmPlatform.__mro__
                  if "get_attn_backend_cls" in k.__dict__)
    orig = target.__dict__["get_attn_backend_cls"].__func__

    def get_attn_backend_cls(cls, *args, **kwargs):
        path = orig(cls, *args, **kwargs)
        if not isinstance(path, str) or _is_mla(args, kwargs) or path.startswith(__name__):
            return path
        ours = wrap_backend(path)
        print(f"[amass] variant={cfg.variant} score={cfg.score} budget={cfg.budget} "
              f"coverage={cfg.coverage} sink={cfg.sink_pages} window={cfg.window_pages} "
              f"-> {ours}", flush=True)
        return ours

    target.get_attn_backend_cls = classmethod(get_attn_backend_cls)
    _APPLIED = True
    print("[amass] registered (patched RocmPlatform.get_attn_backend_cls)", flush=True)


_ATTENTION_LAYERS = ("vllm.attention.layer.Attention",
                     "vllm.model_executor.layers.attention.Attention")


def patch_kv_cache_spec_k_only() -> None:
    """Opt-in for mem variants whose every attention reads V from the tier: the engine's
    block pool holds K only, so ``num_gpu_blocks`` doubles at the same memory budget
    (reference backend/register.py:90-101, a documented follow-up there).  Wraps the
    attention layer's ``get_kv_cache_spec`` to return the plain full-attention spec with
    ``head_size_v = 0``; any other spec (sliding window, MLA, asymmetric heads) raises.
    register() does not call it: this build's mem-v backend attends with the stock
    attention, which still reads V from the engine cache."""
    import dataclasses
    cls = None
    for qualname in _ATTENTION_LAYERS:
        try:
            cls = _resolve(qualname)
            break
        except (ImportError, AttributeError):
            continue
    if cls is None:
        raise RuntimeError("vLLM's attention layer class was not found")
    orig = cls.get_kv_cache_spec
    if getattr(orig, "_amass_k_only", False):
        return

    def get_kv_cache_spec(self, *args, **kwargs):
        spec = orig(self, *args, **kwargs)
        if spec is None:
            return spec
        if type(spec).__name__ != "FullAttentionSpec" or not dataclasses.is_dataclass(spec):
            raise ValueError(f"K-only KV cache: {type(spec).__name__} layers are not "
                             "supported (plain full attention only)")
        hv = getattr(spec, "head_size_v", spec.head_size)
        if hv != spec.head_size:
            raise ValueError(f"K-only KV cache: asymmetric heads (head_size "
                             f"{spec.head_size}, head_size_v {hv})")
        return dataclasses.replace(spec, head_size_v=0)

    get_kv_cache_spec._amass_k_only = True
    cls.get_kv_cache_spec = get_kv_cache_spec
