"""Staging -- the bounded HBM V staging pool and its per-step lifecycle (mem-v tier).

Mirror of the reference ``tier/staging.py:235-507``.  Under mem-v the V of every token
written in a step lands first in ``v_pool`` (L, NV, page, n_kv, d), a VRAM pool bounded
to the concurrent working set (the partial tail of each request and the pages of a
prefill chunk), and once a page is complete its V is flushed to the pinned host pool and
the staging block is recycled.  Buffers:

  v_pool (L, NV, page, n_kv, d)   staged V        vbo (NB,) int32   staging block or -1
  v_flushed (NB,) int32           flush latch     v_free_stack (NV,), v_free_top (1,)
  v_slot_mapping (max_tokens,) int64  per-token write slot (-1 = none)
  flush_list (MAXF, 2), flush_cnt (1,), overflow (1,) (free-stack underflow latch)
  mark (R, ceil(MP/256)), first (NB,)  device scratch of begin_step

``begin_step`` (``amass_stage_begin_step``) runs the ordered lifecycle -- flushed-bit
clear, flush collect, flush copy, staging-block alloc, token slots -- and ``scatter_kv``
(``amass_stage_scatter``) is the per-layer write path; both are fixed-shape, host-sync
free and graph capturable.  The invariants are the reference's: I1 (no lost V: a
complete written page is staged or flushed), I3 (assigned and free staging blocks
partition [0, NV)), I4 (the flush copy reads a staging block before the alloc reuses it:
the launch order inside ``begin_step``).
"""
from __future__ import annotations

import torch

from .._hip import ScatterArgs, StageArgs, call, current_stream, ptr, require_cuda

I32_MAX = 2 ** 31 - 1
MARK_CHUNK = 256


class Staging:
    def __init__(self, *, num_layers: int, num_blocks: int, n_kv: int, page: int, d: int,
                 dtype: torch.dtype, device, max_reqs: int = 1, max_pages: int = 1,
                 max_tokens: int = 0, v_blocks: int | None = None,
                 max_flush: int | None = None, offload_k: bool = False):
        if offload_k:
            raise NotImplementedError("mem-kv (K offload) is outside this build's hot path")
        self.L, self.NB, self.n_kv, self.page, self.d = num_layers, num_blocks, n_kv, page, d
        self.R, self.MP = max(int(max_reqs), 1), max(int(max_pages), 1)
        self.max_tokens = max(int(max_tokens), 1)
        dev = torch.device(device)
        self.device = dev
        i32, i64 = torch.int32, torch.int64
        # working-set bound (tier/staging.py:264-268): a step writes at most
        # ceil(max_tokens / page) new pages, flushed on the next step, so about two chunks
        # plus a partial tail per request are staged at once -- O(chunk), not O(context)
        chunk_pages = (self.max_tokens + page - 1) // page
        if v_blocks is None or v_blocks <= 0:
            v_blocks = 2 * chunk_pages + 4 * self.R
        if max_flush is None or max_flush <= 0:
            max_flush = chunk_pages + 2 * self.R + 64
        self.NV, self.MAXF, self.chunk_pages = int(v_blocks), int(max_flush), chunk_pages
        self.v_pool = torch.zeros((num_layers, self.NV, page, n_kv, d), dtype=dtype, device=dev)
        self.vbo = torch.full((num_blocks,), -1, dtype=i32, device=dev)
        self.v_flushed = torch.zeros((num_blocks,), dtype=i32, device=dev)
        self.v_free_stack = torch.arange(self.NV, dtype=i32, device=dev)
        self.v_free_top = torch.full((1,), self.NV, dtype=i32, device=dev)
        self.v_slot_mapping = torch.full((self.max_tokens,), -1, dtype=i64, device=dev)
        self.flush_list = torch.zeros((self.MAXF, 2), dtype=i32, device=dev)
        self.flush_cnt = torch.zeros((1,), dtype=i32, device=dev)
        self.overflow = torch.zeros((1,), dtype=i32, device=dev)
        self.mark = torch.zeros((self.R, (self.MP + MARK_CHUNK - 1) // MARK_CHUNK), dtype=i32,
                                device=dev)
        self.first = torch.full((num_blocks,), I32_MAX, dtype=i32, device=dev)
        elem = torch.empty(0, dtype=dtype).element_size()
        self.vpool_gib = self.v_pool.numel() * elem / 2**30

    # ---- per step (once, before the layers) ---------------------------------------------
    def begin_step(self, block_table, seq_lens, query_start_loc, n_tokens: int, pool,
                   pool_valid) -> None:
        """The ordered stage / flush / alloc lifecycle for this step's tokens
        (tier/staging.py:312-343).  ``pool`` is the MappedHostVPool, ``pool_valid`` the
        residency's (L, n_kv, NB) map."""
        require_cuda(block_table, seq_lens, query_start_loc, pool_valid)
        n_req = seq_lens.shape[0]
        if n_tokens > self.max_tokens:
            raise ValueError(f"{n_tokens} tokens > v_slot_mapping capacity {self.max_tokens}")
        if n_req > self.R or block_table.shape[1] > self.MP:
            raise ValueError("batch wider than the staging scratch (max_reqs, max_pages)")
        if query_start_loc.shape[0] < n_req + 1:
            raise ValueError("query_start_loc needs n_req + 1 entries")
        vp = self.v_pool
        a = StageArgs(
            block_table=ptr(block_table), bt_st=block_table.stride(0),
            seq_lens=ptr(seq_lens), query_start_loc=ptr(query_start_loc),
            vbo=ptr(self.vbo), v_flushed=ptr(self.v_flushed),
            free_stack=ptr(self.v_free_stack), free_top=ptr(self.v_free_top),
            v_slot=ptr(self.v_slot_mapping), flush_list=ptr(self.flush_list),
            flush_cnt=ptr(self.flush_cnt), overflow=ptr(self.overflow), mark=ptr(self.mark),
            first=ptr(self.first), v_pool=ptr(vp), vp_sl=vp.stride(0), vp_sb=vp.stride(1),
            vp_st=vp.stride(2), vp_sh=vp.stride(3), pool=pool.dev_ptr,
            pool_valid=ptr(pool_valid), n_req=n_req, n_tokens=n_tokens,
            max_pages=block_table.shape[1], n_layers=self.L, nb=self.NB, nv=self.NV,
            n_kv=self.n_kv, page=self.page, d=self.d, maxf=self.MAXF)
        call("amass_stage_begin_step", a, current_stream(self.device))

    # ---- write path (per layer, after begin_step) -----------------------------------------
    def scatter_kv(self, lidx: int, key, value: torch.Tensor, n_tokens: int) -> None:
        """Scatter ``value`` (n_tokens, n_kv, d) into layer ``lidx``'s staging pool at this
        step's ``v_slot_mapping`` (tier/staging.py:348-364; ``key`` is unused under
        mem-v, K stays in the engine cache)."""
        require_cuda(value)
        if value.dtype != self.v_pool.dtype or value.stride(2) != 1:
            raise ValueError("value must match the pool dtype with unit stride on d")
        vp = self.v_pool[lidx]
        a = ScatterArgs(value=ptr(value), v_st=value.stride(0), v_sh=value.stride(1),
                        v_slot=ptr(self.v_slot_mapping), v_pool=ptr(vp), vp_sb=vp.stride(0),
                        vp_st=vp.stride(1), vp_sh=vp.stride(2), n_tokens=n_tokens,
                        n_kv=self.n_kv, d=self.d, page=self.page, nv=self.NV)
        call("amass_stage_scatter", a, current_stream(self.device))

    def stage(self, layer: int, blocks, staging_blocks, v_pages) -> None:
        """Place V pages (n, page, n_kv, d) of physical ``blocks`` at ``staging_blocks``
        directly (benchmarks and tests that stage pages without running steps); the free
        stack is rebuilt so the assigned and free staging blocks stay a partition."""
        self.v_pool[layer, staging_blocks] = v_pages.to(self.v_pool.dtype)
        self.vbo[blocks] = staging_blocks.to(torch.int32)
        used = torch.zeros(self.NV, dtype=torch.bool, device=self.vbo.device)
        assigned = self.vbo[self.vbo >= 0].long()
        used[assigned] = True
        free = torch.nonzero(~used).flatten().to(torch.int32)
        self.v_free_stack[:free.numel()] = free
        self.v_free_top.fill_(free.numel())

    # ---- invariant checks (host-synchronising; debug) --------------------------------------
    def assert_free_partition(self) -> None:
        """I3: assigned (vbo >= 0) and free (v_free_stack[:top]) staging blocks partition
        [0, NV)."""
        top = int(self.v_free_top.item())
        if not 0 <= top <= self.NV:
            raise AssertionError(f"I3 staging: free_top={top} outside [0, {self.NV}]")
        assigned = self.vbo[self.vbo >= 0]
        both = torch.cat([assigned, self.v_free_stack[:top]]).sort().values
        if both.numel() != self.NV or not torch.equal(
                both.cpu(), torch.arange(self.NV, dtype=both.dtype)):
            raise AssertionError("I3 staging: assigned + free staging blocks are not a "
                                 f"partition of [0, {self.NV})")

    def assert_no_lost_v(self, block_table, seq_lens, query_start_loc, pool_valid) -> None:
        """I1: every complete page of the settled context is staged or flushed for every
        layer and kv head."""
        sl = seq_lens.tolist()
        qsl = query_start_loc.tolist()
        vbo = self.vbo.cpu()
        pv = pool_valid.cpu()
        for r in range(len(sl)):
            ql = qsl[r + 1] - qsl[r]
            if sl[r] <= 0 or ql <= 0:
                continue
            for p in range((sl[r] - ql) // self.page):
                blk = int(block_table[r, p])
                if int(vbo[blk]) < 0 and not bool((pv[:, :, blk] == 1).all()):
                    raise AssertionError(f"I1: request {r} page {p} (block {blk}) is neither "
                                         "staged nor flushed")

    def assert_capacity(self) -> None:
        """The working-set bound: NV covers one chunk plus a tail per request."""
        floor = self.chunk_pages + self.R
        if self.NV < floor:
            raise AssertionError(f"I1 capacity: NV={self.NV} < {floor} (chunk_pages="
                                 f"{self.chunk_pages} + max_reqs={self.R})")

    def bytes_report(self) -> str:
        return f"staging={self.vpool_gib:.3f}GiB (NV={self.NV}, MAXF={self.MAXF})"
