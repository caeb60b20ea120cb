"""Residency -- exact-LRU HBM hot buffer for the selected V pages (mem-v tier).

Buffers and invariants follow the reference ``tier/residency.py:281-577``:

  hot        (L, n_kv, S, page, d)  the V bytes of resident pages
  page2slot  (L, n_kv, NB) int32    slot of a physical block or -1
  slot2page  (L, n_kv, S)  int32    block in a slot or -1   (I3: mutual inverses)
  lru_clock  (L, n_kv, S)  int32    last step a slot was touched / claimed
  pool_valid (L, n_kv, NB) int8     block's V is in the pinned pool
  clock (1,), overflow (1,)         step clock (a view of a 2-element buffer whose second
                                    word the plan launch uses), hot-buffer exhaustion latch
  miss_pages / victim_slots (R, n_kv, MP), miss_cnt (R, n_kv), fetch_list (FCAP, 3),
  fetch_cnt (1,), first_pos (n_kv, NB) (dedup scratch, INT32_MAX at rest)

``gather_plan`` (two launches: hits/misses, then the victims, whose last workgroup
advances the clock) and ``gather_fetch``
(flat fetch kernel) are the HIP entry points ``amass_tier_gather_plan`` and
``amass_tier_fetch``; both are fixed-shape, host-sync free and graph capturable.
``build_dma_plan`` / ``issue_dma_plan`` are the host-planned copy-engine alternative
(tier/residency.py:438-525) over ``amass_tier_dma``.
"""
from __future__ import annotations

import numpy as np
import torch

from .._hip import (CopyRun, InvalidateArgs, TierFetchArgs, TierPlanArgs, call,
                     current_stream, ptr)

I32_MAX = 2 ** 31 - 1


class Residency:
    def __init__(self, *, num_layers: int, num_blocks: int, n_kv: int, hot_slots: int,
                 page: int, d: int, max_reqs: int, max_pages: int, dtype: torch.dtype,
                 device, offload_k: bool = False):
        if offload_k:
            raise NotImplementedError("mem-kv (K offload) is outside this build's hot path")
        self.L, self.NB, self.n_kv = num_layers, num_blocks, n_kv
        self.S, self.page, self.d = hot_slots, page, d
        self.R, self.MP = max_reqs, max_pages
        self.dtype = dtype
        dev = torch.device(device)
        self.device = dev
        i32, i8 = torch.int32, torch.int8
        self.hot = torch.zeros((num_layers, n_kv, hot_slots, page, d), dtype=dtype, device=dev)
        self.page2slot = torch.full((num_layers, n_kv, num_blocks), -1, dtype=i32, device=dev)
        self.slot2page = torch.full((num_layers, n_kv, hot_slots), -1, dtype=i32, device=dev)
        self.lru_clock = torch.zeros((num_layers, n_kv, hot_slots), dtype=i32, device=dev)
        self.pool_valid = torch.zeros((num_layers, n_kv, num_blocks), dtype=i8, device=dev)
        # [step clock, the plan launch's arrival count (zero between calls)]
        self._clock2 = torch.tensor([1, 0], dtype=i32, device=dev)
        self.clock = self._clock2[:1]
        self.overflow = torch.zeros((1,), dtype=i32, device=dev)
        self.miss_pages = torch.zeros((max_reqs, n_kv, max_pages), dtype=i32, device=dev)
        self.miss_cnt = torch.zeros((max_reqs, n_kv), dtype=i32, device=dev)
        self.victim_slots = torch.zeros((max_reqs, n_kv, max_pages), dtype=i32, device=dev)
        self.FCAP = max_reqs * n_kv * max_pages
        self.fetch_list = torch.zeros((self.FCAP, 3), dtype=i32, device=dev)
        self.fetch_cnt = torch.zeros((1,), dtype=i32, device=dev)
        self.first_pos = torch.full((n_kv, num_blocks), I32_MAX, dtype=i32, device=dev)
        self.fetch_grid = 1024
        self.plan_width = max_pages
        elem = torch.empty(0, dtype=dtype).element_size()
        self.hot_gib = self.hot.numel() * elem / 2**30

    # ---- per step (once, before staging) ---------------------------------------------
    def invalidate_written(self, block_table, seq_lens, query_start_loc) -> None:
        """Every page (re)written this step leaves the pinned pool's validity and the hot
        buffer in every layer and kv head (tier/residency.py:251-278,352-367): block reuse
        and chunked prefill make both copies stale."""
        n_req = seq_lens.shape[0]
        a = InvalidateArgs(
            block_table=ptr(block_table), bt_st=block_table.stride(0),
            seq_lens=ptr(seq_lens), query_start_loc=ptr(query_start_loc),
            page2slot=ptr(self.page2slot), slot2page=ptr(self.slot2page),
            pool_valid=ptr(self.pool_valid), n_req=n_req, n_layers=self.L, nb=self.NB,
            n_kv=self.n_kv, slots=self.S, page=self.page, max_pages=block_table.shape[1])
        call("amass_tier_invalidate", a, current_stream(self.device))

    # ---- per step, per layer -------------------------------------------------------
    def gather_plan(self, layer, page_table, page_cnt, block_table, seq_lens, n_req) -> None:
        """Classify the selected complete pages as hits (touch LRU) or misses and assign
        exact-LRU victim slots to the distinct new misses (advances the clock)."""
        a = TierPlanArgs(
            page_table=ptr(page_table), pt_sr=page_table.stride(0), pt_sh=page_table.stride(1),
            page_cnt=ptr(page_cnt), pc_sr=page_cnt.stride(0),
            block_table=ptr(block_table), bt_st=block_table.stride(0),
            seq_lens=ptr(seq_lens), page2slot=ptr(self.page2slot[layer]),
            slot2page=ptr(self.slot2page[layer]), lru_clock=ptr(self.lru_clock[layer]),
            clock=ptr(self._clock2), miss_pages=ptr(self.miss_pages),
            miss_cnt=ptr(self.miss_cnt), victim_slots=ptr(self.victim_slots),
            overflow=ptr(self.overflow), fetch_list=ptr(self.fetch_list),
            fetch_cnt=ptr(self.fetch_cnt), first_pos=ptr(self.first_pos),
            n_req=n_req, n_kv=self.n_kv, nb=self.NB, slots=self.S,
            max_pages=page_table.shape[2], page=self.page, fcap=self.FCAP)
        if page_table.shape[2] > self.MP or n_req > self.R:
            raise ValueError("selection wider than the residency scratch")
        call("amass_tier_gather_plan", a, current_stream(self.device))
        # the kernel writes miss_pages / victim_slots rows at this stride
        self.plan_width = page_table.shape[2]

    def gather_fetch(self, layer, staging, pool, n_req=None, stream=None) -> None:
        """Copy every planned miss page into its hot slot (pinned pool, or the staged
        pool with write-through)."""
        vp = staging.v_pool[layer] if staging is not None else None
        a = TierFetchArgs(
            fetch_list=ptr(self.fetch_list), fetch_cnt=ptr(self.fetch_cnt),
            hot=ptr(self.hot[layer]), pool=pool.dev_ptr,
            vpool=ptr(vp), v_sb=vp.stride(0) if vp is not None else 0,
            v_st=vp.stride(1) if vp is not None else 0,
            v_sh=vp.stride(2) if vp is not None else 0,
            vbo=ptr(staging.vbo) if staging is not None else None,
            pool_valid=ptr(self.pool_valid[layer]), t_layer=layer, nb=self.NB,
            n_kv=self.n_kv, slots=self.S, page=self.page, d=self.d, fcap=self.FCAP,
            grid=self.fetch_grid)
        s = stream.cuda_stream if stream is not None else current_stream(self.device)
        call("amass_tier_fetch", a, s)

    def gather(self, layer, page_table, page_cnt, block_table, seq_lens, n_req, staging,
               pool) -> None:
        self.gather_plan(layer, page_table, page_cnt, block_table, seq_lens, n_req)
        self.gather_fetch(layer, staging, pool, n_req)

    # ---- copy-engine alternative (host planned) ---------------------------------------
    def build_dma_plan(self, layer, pool, n_req):
        """Copy-engine plan for this step's misses (the host-planned alternative to the
        fetch kernel; reference tier/residency.py:438-493).  A miss whose V is valid in the
        pinned pool joins a 2-D copy run; a run is a maximal chain of misses that follow
        each other in one (request, kv head) miss list with victim slot AND block both one
        higher than the previous one's, i.e. consecutive hot slots filled from consecutive
        pool blocks (row pitch: one page in the hot buffer, n_kv pages in the pool).

        The chains are found on the device with whole-tensor ops (a miss "extends" its
        predecessor; heads are fetchable misses that do not; a head's run ends at the next
        entry that does not extend), and the host receives one compact table of (kv, slot,
        block, height) rows.  Returns (runs, has_staged): runs is an (n, 6) int64 array of
        amass_copy_run rows (dst, src, dpitch, spitch, width, height); has_staged tells
        that some miss's V is only in the staging pool, which the fetch kernel copies."""
        n_kv, S, NB, page, d = self.n_kv, self.S, self.NB, self.page, self.d
        pbytes = page * d * torch.empty(0, dtype=self.dtype).element_size()
        if n_req <= 0:
            return np.zeros((0, 6), np.int64), False
        dev = self.miss_pages.device
        rows = n_req * n_kv * self.plan_width   # the last plan's rows, at its row stride
        blk = self.miss_pages.view(-1)[:rows].view(n_req, n_kv, self.plan_width).long()
        slot = self.victim_slots.view(-1)[:rows].view(n_req, n_kv, self.plan_width).long()
        live = (torch.arange(blk.shape[-1], device=dev) < self.miss_cnt[:n_req, :, None]) \
            & (slot >= 0)
        kvi = torch.arange(n_kv, device=dev).view(1, n_kv, 1).expand_as(blk)
        in_pool = self.pool_valid[layer][kvi, blk.clamp(0, NB - 1)] != 0
        fetch = live & in_pool
        ext = torch.zeros_like(fetch)
        ext[..., 1:] = (fetch[..., 1:] & fetch[..., :-1]
                        & (slot[..., 1:] == slot[..., :-1] + 1)
                        & (blk[..., 1:] == blk[..., :-1] + 1))
        heads = torch.nonzero((fetch & ~ext).flatten()).flatten()
        ends = torch.nonzero((~ext).flatten()).flatten()
        ends = torch.cat([ends, ends.new_tensor([ext.numel()])])
        height = ends[torch.searchsorted(ends[:-1], heads, right=True)] - heads
        table = torch.stack([(heads // blk.shape[-1]) % n_kv, slot.flatten()[heads],
                             blk.flatten()[heads], height], dim=1)
        flag = (live & ~in_pool).any().long().view(1, 1).expand(1, 4)
        host = torch.cat([flag, table]).cpu().numpy()          # the one device -> host copy
        has_staged, (kv, sl, bk, h) = bool(host[0, 0]), host[1:].T
        hot_base = self.hot[layer].data_ptr()
        pool_base = pool._host_ptr + layer * NB * n_kv * pbytes
        runs = np.empty((host.shape[0] - 1, 6), np.int64)
        runs[:, 0] = hot_base + (kv * S + sl) * pbytes
        runs[:, 1] = pool_base + (bk * n_kv + kv) * pbytes
        runs[:, 2] = pbytes
        runs[:, 3] = n_kv * pbytes
        runs[:, 4] = pbytes
        runs[:, 5] = h
        return runs, has_staged

    @staticmethod
    def issue_dma_plan(runs, stream) -> None:
        """Issue an (n, 6) int64 run table (amass_copy_run rows) on `stream`."""
        if len(runs) == 0:
            return
        import ctypes
        from .._hip import check, load_library
        runs = np.ascontiguousarray(runs, dtype=np.int64)
        assert runs.shape[1] * 8 == ctypes.sizeof(CopyRun)
        check(load_library().amass_tier_dma(runs.ctypes.data_as(ctypes.POINTER(CopyRun)),
                                            len(runs), ctypes.c_void_p(stream.cuda_stream)),
              "amass_tier_dma")

    # ---- invariants ------------------------------------------------------------------
    def assert_maps_inverse(self, layer=None) -> None:
        """I2/I3: page2slot and slot2page are mutual inverses (one slot per page, one page
        per slot).  Host sync; debug only."""
        layers = range(self.L) if layer is None else [layer]
        for l in layers:
            for kv in range(self.n_kv):
                s2p = self.slot2page[l, kv]
                occ = s2p >= 0
                pages = s2p[occ]
                if pages.numel() != torch.unique(pages).numel():
                    raise AssertionError(f"I3: layer {l} kv {kv} has a page in two slots")
                slots = torch.nonzero(occ, as_tuple=False).flatten()
                back = self.page2slot[l, kv][pages.long()]
                if not torch.equal(back, slots.to(back.dtype)):
                    raise AssertionError(f"I2: layer {l} kv {kv} maps are not inverses")
                if int((self.page2slot[l, kv] >= 0).sum()) != int(occ.sum()):
                    raise AssertionError(f"I2: layer {l} kv {kv} stale page2slot entries")

    def bytes_report(self) -> str:
        return f"hot={self.hot_gib:.3f}GiB (S={self.S} slots/kv)"
