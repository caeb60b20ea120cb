"""AMASS attention impl: stock vLLM-ROCm attention + AMASS decode-time page selection.

Reference: ``backend/attn.py:31-82`` (a FlashAttentionImpl subclass).  Here the impl is
a mixin placed in front of whichever attention impl vLLM's ROCm platform picked (see
register.py), so every path that is not a plain single-token decode -- prefill, mixed
batches, cascade, encoder layers, sliding window, ALiBi, sinks, quantised caches --
runs the stock implementation unchanged.  A pure decode step runs

    select(...)           Stage A: score + selection -> st.page_table / st.page_cnt
    decode_dispatch(...)  Stage B: sparse paged decode -> output (in place)

(``_runtime.select_and_decode``; a quad state takes ``select_then_attend``, which runs
small batches through the per-unit pipeline -- both stages in one launch where top-b
bounds the kept pages -- with the same outputs)

with K and V read from the resident paged cache.  ``forward`` has the reference's
signature and returns ``output``.

mem-v (reference attn.py:84-118, shadow): every step writes the layer's V into the
tier's staging pool (the write path, ``tier.write_kv``; the builder ran the step's
lifecycle) and attends with the stock attention, the engine cache still holding V.
"""
from __future__ import annotations

from ..attention.decode import ResidentVSource
from . import _runtime

_ANNOUNCED = False


def _quantized(kv_cache_dtype) -> bool:
    return str(kv_cache_dtype or "auto") not in ("auto", "bfloat16", "float16", "bf16",
                                                  "fp16")


def _decoder_type(impl) -> bool:
    t = getattr(impl, "attn_type", None)
    return t is None or str(getattr(t, "value", t)).lower() == "decoder"


class AmassAttentionImplMixin:
    """Mixed in front of the platform's attention impl class."""

    def _amass_pure_decode(self, m, kv_cache, output) -> bool:
        cfg = _runtime.get_config()
        st = getattr(m, "amass", None) if m is not None else None
        sw = getattr(self, "sliding_window", None)
        return not (cfg is None or cfg.variant != "fast" or st is None or output is None
                    or getattr(m, "max_query_len", None) != 1
                    or kv_cache is None or kv_cache.numel() == 0
                    or getattr(m, "use_cascade", False)
                    or getattr(m, "causal", True) is not True
                    or not _decoder_type(self)
                    or sw not in (None, (-1, -1), -1)
                    or getattr(self, "alibi_slopes", None) is not None
                    or getattr(self, "sinks", None) is not None
                    or getattr(self, "dcp_world_size", 1) > 1
                    or _quantized(getattr(self, "kv_cache_dtype", "auto")))

    def _amass_write_v(self, m, value, kv_cache) -> None:
        """mem-v write path of this layer: the step's V -> the tier's staging pool."""
        tier = getattr(m, "amass_tier", None) if m is not None else None
        if tier is None or value is None or kv_cache is None:
            return
        lidx = _runtime.layer_index(tier, kv_cache)
        v3 = value if value.dim() == 3 else value.view(value.shape[0], self.num_kv_heads, -1)
        tier.write_kv(lidx, v3, v3.shape[0])

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None,
                output_scale=None, output_block_scale=None):
        m = attn_metadata
        cfg = _runtime.get_config()
        if cfg is not None and cfg.is_mem:
            self._amass_write_v(m, value, kv_cache)
            return super().forward(layer, query, key, value, kv_cache, m, output,
                                   output_scale=output_scale,
                                   output_block_scale=output_block_scale)
        if not self._amass_pure_decode(m, kv_cache, output):
            return super().forward(layer, query, key, value, kv_cache, m, output,
                                   output_scale=output_scale,
                                   output_block_scale=output_block_scale)
        cfg = _runtime.get_config()
        st = m.amass
        n_req = m.seq_lens.shape[0]
        out3 = output if output.dim() == 3 else output.view(output.shape[0],
                                                            self.num_heads, -1)
        _runtime.select_and_decode(query, kv_cache, m.block_table, m.seq_lens, st, out3,
                                   ResidentVSource(kv_cache), n_req, self.scale, cfg)
        global _ANNOUNCED
        if not _ANNOUNCED:
            _ANNOUNCED = True
            print(f"[amass] decode path active (n_req={n_req} score={cfg.score} "
                  f"budget={cfg.budget} coverage={cfg.coverage})", flush=True)
        return output


def make_impl(base: type) -> type:
    """The AMASS impl class over the platform's impl class ``base``."""
    return type(f"Amass{base.__name__}", (AmassAttentionImplMixin, base), {})
