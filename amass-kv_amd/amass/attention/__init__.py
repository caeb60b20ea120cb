"""Stage B -- sparse paged decode attention over the Stage-A-selected pages.

  sparse_paged_decode_batched(q, kv_cache, block_table, seq_lens, st, out, vsource)
  dense_paged_decode(q, kv_cache, block_table, seq_lens, st, out, scale=...)
  ResidentVSource / VSource      the fast / mem-v V-source seam
  ensure_stage_b_buffers         split-K partial buffers (allocated once)
"""
from __future__ import annotations

from .decode import (SPLIT, ResidentVSource, VSource, _split_kv, dense_paged_decode,
                     ensure_stage_b_buffers, sparse_paged_decode_batched)

__all__ = ["sparse_paged_decode_batched", "dense_paged_decode", "ResidentVSource", "VSource",
           "ensure_stage_b_buffers", "SPLIT"]
