"""mem-v tiered decode for one layer (reference ``tier/decode_mem.py:225-274``).

``mem_dynamic_decode``: residency gather of this layer's selection (plan + fetch, or the
copy-engine variant, or none), then the sparse decode with V_SRC = 1, whose per-page
address select reads the hot slot, the staging pool or the pinned pool -- the same bytes
as the resident path, so the output equals the resident decode bit for bit.
"""
from __future__ import annotations

from ..attention.decode import sparse_paged_decode_batched

_FETCH_MODES = ("kernel", "dma", "off")


def mem_decode(q, kv_cache, block_table, seq_lens, st, out, tier, lidx: int, *,
               scale=None, path: str = "auto") -> None:
    sparse_paged_decode_batched(q, kv_cache, block_table, seq_lens, st, out,
                                tier.vsource(lidx), scale=scale, path=path)


def mem_dynamic_decode(q, kv_cache, block_table, seq_lens, st, out, tier, lidx: int, *,
                       scale=None, fetch: str = "kernel", path: str = "auto") -> None:
    if fetch not in _FETCH_MODES:
        raise ValueError(f"fetch must be one of {_FETCH_MODES}, got {fetch!r}")
    n_req = seq_lens.shape[0]
    if fetch == "kernel":
        tier.step(lidx, st.page_table, st.page_cnt, block_table, seq_lens, n_req)
    elif fetch == "dma":
        tier.step_dma(lidx, st.page_table, st.page_cnt, block_table, seq_lens, n_req)
    mem_decode(q, kv_cache, block_table, seq_lens, st, out, tier, lidx, scale=scale, path=path)
