"""Staging -- the bounded HBM V staging pool the tiered decode addresses (mem-v tier).

Only the part of the reference ``tier/staging.py`` that the decode hot path reads is
built here: ``v_pool`` (L, NV, page, n_kv, d) holding V of pages that are not yet flushed
to the pinned pool (the partial tail and fresh prefill pages) and ``vbo`` (NB,) int32,
the staging block of a physical block or -1 (tier/staging.py:264-268, 312-364).  The
write path (scatter of new tokens) and the flush lifecycle are outside this build's hot
path; callers fill v_pool / vbo directly (``stage``).
"""
from __future__ import annotations

import torch


class Staging:
    def __init__(self, *, num_layers: int, num_blocks: int, n_kv: int, page: int, d: int,
                 v_blocks: int, dtype: torch.dtype, device):
        self.L, self.NB, self.n_kv, self.page, self.d = num_layers, num_blocks, n_kv, page, d
        self.NV = int(v_blocks)
        self.v_pool = torch.zeros((num_layers, self.NV, page, n_kv, d), dtype=dtype,
                                  device=device)
        self.vbo = torch.full((num_blocks,), -1, dtype=torch.int32, device=device)

    def stage(self, layer: int, blocks, staging_blocks, v_pages) -> None:
        """Place V pages (n, page, n_kv, d) of physical ``blocks`` at ``staging_blocks``."""
        self.v_pool[layer, staging_blocks] = v_pages.to(self.v_pool.dtype)
        self.vbo[blocks] = staging_blocks.to(torch.int32)

    def bytes_report(self) -> str:
        n = self.v_pool.numel() * self.v_pool.element_size()
        return f"staging={n / 2**30:.3f}GiB (NV={self.NV})"
