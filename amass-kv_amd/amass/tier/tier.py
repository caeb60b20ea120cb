"""Tier -- the mem-v facade (pinned pool + residency + staging) and its V source.

Mirror of the reference ``tier/tier.py:37-265``.  ``step`` is the per-layer residency
gather run before the layer's Stage-B decode (plan + fetch, both graph capturable);
``step_dma`` is the copy-engine variant (host-planned, not capturable); ``begin_step`` /
``write_kv`` are the write path (invalidate + staging lifecycle once per step, the V
scatter per layer); ``vsource``
returns the ``TierVSource`` the decode consumes (V_SRC = 1: per page hot slot if the page
is complete and resident, else the staging pool, else the pinned pool over the host link).
"""
from __future__ import annotations

import torch

from .dma import CopyEngine
from .pool import MappedHostVPool
from .residency import Residency
from .staging import Staging


class Tier:
    def __init__(self, *, num_layers: int, num_blocks: int, n_kv: int, page: int, d: int,
                 hot_slots: int, max_reqs: int, max_pages: int, dtype=torch.bfloat16,
                 device="cuda", v_blocks=None, max_pool_gb: float = 256.0,
                 offload_k: bool = False, max_tokens: int = 0):
        if offload_k:
            raise NotImplementedError("mem-kv is outside this build's hot path")
        self.L, self.NB, self.n_kv, self.page, self.d = num_layers, num_blocks, n_kv, page, d
        self.device = torch.device(device)
        self.dtype = dtype
        self.offload_k = False
        self.pool = MappedHostVPool(num_layers=num_layers, num_blocks=num_blocks, n_kv=n_kv,
                                    page=page, d=d, dtype=dtype, device=device,
                                    max_pool_gb=max_pool_gb)
        self.residency = Residency(num_layers=num_layers, num_blocks=num_blocks, n_kv=n_kv,
                                   hot_slots=hot_slots, page=page, d=d, max_reqs=max_reqs,
                                   max_pages=max_pages, dtype=dtype, device=device)
        self.staging = Staging(num_layers=num_layers, num_blocks=num_blocks, n_kv=n_kv,
                               page=page, d=d, dtype=dtype, device=device, max_reqs=max_reqs,
                               max_pages=max_pages, max_tokens=max(max_tokens, max_reqs),
                               v_blocks=v_blocks)
        self._copy_engine = None

    @classmethod
    def from_config(cls, cfg, *, num_layers, num_blocks, n_kv, page, d, max_reqs, max_pages,
                    max_tokens=0, dtype=torch.bfloat16, device="cuda") -> "Tier":
        if not cfg.is_mem:
            raise ValueError(f"Tier requires a mem variant, got {cfg.variant!r}")
        return cls(num_layers=num_layers, num_blocks=num_blocks, n_kv=n_kv, page=page, d=d,
                   hot_slots=cfg.hot_slots, max_reqs=max_reqs, max_pages=max_pages,
                   dtype=dtype, device=device, v_blocks=cfg.v_blocks,
                   max_pool_gb=cfg.max_pool_gb, offload_k=cfg.offload_k,
                   max_tokens=max_tokens)

    def begin_step(self, block_table, seq_lens, query_start_loc, n_tokens: int) -> None:
        """The one per-step entry (tier/tier.py:86-104), before the layers: pages written
        this step leave the hot buffer and the pool's validity, then the staging
        lifecycle (flush complete pages, allocate staging blocks, token slots)."""
        self.residency.invalidate_written(block_table, seq_lens, query_start_loc)
        self.staging.begin_step(block_table, seq_lens, query_start_loc, n_tokens, self.pool,
                                self.residency.pool_valid)

    def write_kv(self, lidx: int, value: torch.Tensor, n_tokens: int, key=None) -> None:
        """Write path of layer ``lidx`` (after begin_step): this step's V into the
        staging pool (tier/tier.py:125-130)."""
        self.staging.scatter_kv(lidx, key, value, n_tokens)

    def assert_invariants(self, block_table, seq_lens, query_start_loc) -> None:
        """I1 / I3 checks (host-synchronising; debug), tier/tier.py:106-120."""
        if int(self.staging.overflow.item()) != 0:
            raise AssertionError("I1 capacity: the staging free stack underflowed (a written "
                                 "page got no staging block); raise v_blocks")
        self.staging.assert_free_partition()
        self.residency.assert_maps_inverse()
        self.staging.assert_no_lost_v(block_table, seq_lens, query_start_loc,
                                      self.residency.pool_valid)

    def flush_layer(self, layer: int, v_blocks: torch.Tensor, valid: bool = True) -> None:
        """Write a layer's full V (NB, page, n_kv, d) to the pinned pool and mark every
        block flushed (bulk load; the per-token write path is not part of the hot path)."""
        self.pool.write_layer(layer, v_blocks)
        self.residency.pool_valid[layer].fill_(1 if valid else 0)

    def step(self, lidx, page_table, page_cnt, block_table, seq_lens, n_req) -> None:
        self.residency.gather(lidx, page_table, page_cnt, block_table, seq_lens, n_req,
                              self.staging, self.pool)

    @property
    def copy_engine(self) -> CopyEngine:
        if self._copy_engine is None:
            self._copy_engine = CopyEngine(self.device)
        return self._copy_engine

    def step_dma(self, lidx, page_table, page_cnt, block_table, seq_lens, n_req,
                 wait: bool = True):
        """Plan on device, then copy the pinned misses with the copy engine on a side
        stream; staged misses (if any) go through the fetch kernel."""
        r5 = self.residency
        r5.gather_plan(lidx, page_table, page_cnt, block_table, seq_lens, n_req)
        runs, has_staged = r5.build_dma_plan(lidx, self.pool, n_req)
        ev = self.copy_engine.issue(runs)
        if has_staged:
            r5.gather_fetch(lidx, self.staging, self.pool, n_req)
        if wait:
            torch.cuda.current_stream(self.device).wait_event(ev)
        return ev

    def vsource(self, lidx: int) -> "TierVSource":
        return TierVSource(self, lidx)

    def bytes_report(self) -> str:
        return (f"[amass tier mem-v] {self.pool.vram_note()} | {self.residency.bytes_report()}"
                f" | {self.staging.bytes_report()}")


class TierVSource:
    """Stage-B V source for layer ``lidx`` of a :class:`Tier` (source id 1)."""

    SRC_ID = 1

    def __init__(self, tier: Tier, lidx: int):
        self.tier, self.lidx = tier, lidx

    def args(self):
        vp = self.tier.staging.v_pool[self.lidx]          # (NV, page, n_kv, d)
        return vp, vp.stride(0), vp.stride(1), vp.stride(2)

    def tier_fields(self) -> dict:
        r5 = self.tier.residency
        return dict(hot=r5.hot[self.lidx].data_ptr(),
                    page2slot=r5.page2slot[self.lidx].data_ptr(),
                    vbo=self.tier.staging.vbo.data_ptr(), pool=self.tier.pool.dev_ptr,
                    layer=self.lidx, nb=r5.NB, slots=r5.S)
