"""mem-v write path: staging lifecycle and residency invalidation (test oracle).

TEST INFRASTRUCTURE: only tests/, smoke() and bench.py's cpu_baseline may use it.

Request r of a step has seq_lens[r] tokens after the step and writes the last
ql = qsl[r+1] - qsl[r] of them; its written pages are p0 = (sl - ql) // page ..
p1 = (sl - 1) // page, its complete settled pages [0, (sl - ql) // page).  Everything
is processed sequentially in (request, page) order -- the order the reference's
serialized kernels walk (their grid-(1,) loops over requests and page blocks), with the
lanes of a block taken in page order -- so the flush list, the free stack and the
staging-block assignment are deterministic.

invalidate   tier/residency.py:251-278,352-367 (_invalidate_kernel): for requests with
             sl > 0, every written page: pool_valid[l, kv, blk] = 0 and, if resident,
             page2slot / slot2page cleared, for all layers and kv heads.
begin_step   tier/staging.py:312-343 with the sub-steps
  vflush_clear  :87-102   v_flushed[blk] = 0 for written pages (sl > 0 and ql > 0)
  flush_collect :105-146  every complete page of an active request whose block is staged
                          (vbo >= 0): if not flushed it is claimed (flush list entry
                          (blk, vb), v_flushed = 1) while the list has room, else it is
                          "over" (kept staged, retried next step); every staged page that
                          is not over is freed (vbo = -1, vb pushed on the free stack)
  flush_copy    :196-232  v_pool[l, vb, t, kv] -> pool[l, blk, kv, t] for every list
                          entry, all layers and heads; pool_valid = 1
  valloc        :149-178  every written page without a staging block pops the free
                          stack (top - 1 first); an empty stack sets overflow
  vslot         :181-193  v_slot[t] = vbo[blk] * page + pos % page for this step's
                          tokens (-1 when the block has no staging block)
scatter      tier/staging.py:51-80,348-364 (_scatter_kv_kernel): v_pool[l, vs // page,
             vs % page] = value[t] for v_slot[t] = vs >= 0.
"""
from __future__ import annotations

import numpy as np


def _written(sl, ql, page):
    return (sl - ql) // page, (sl - 1) // page


def invalidate(block_table, seq_lens, qsl, page2slot, slot2page, pool_valid, *, page):
    """In place on numpy arrays: page2slot (L, n_kv, NB), slot2page (L, n_kv, S),
    pool_valid (L, n_kv, NB)."""
    for r in range(len(seq_lens)):
        sl = int(seq_lens[r])
        if sl <= 0:
            continue
        ql = int(qsl[r + 1]) - int(qsl[r])
        p0, p1 = _written(sl, ql, page)
        for p in range(p0, p1 + 1):
            blk = int(block_table[r, p])
            pool_valid[:, :, blk] = 0
            for l in range(page2slot.shape[0]):
                for kv in range(page2slot.shape[1]):
                    s = int(page2slot[l, kv, blk])
                    if s >= 0:
                        page2slot[l, kv, blk] = -1
                        slot2page[l, kv, s] = -1


def begin_step(block_table, seq_lens, qsl, n_tokens, st, pool, pool_valid, *, page, maxf):
    """In place on the dict ``st`` (numpy: vbo, v_flushed, free_stack, top (int),
    v_slot, flush_list (maxf, 2), flush_cnt (int), overflow (int), v_pool
    (L, NV, page, n_kv, d)) and on pool (L, NB, n_kv, page, d), pool_valid
    (L, n_kv, NB)."""
    vbo, vfl, stack = st["vbo"], st["v_flushed"], st["free_stack"]
    n_req = len(seq_lens)
    st["v_slot"][:n_tokens] = -1
    active = []
    for r in range(n_req):
        sl = int(seq_lens[r])
        ql = int(qsl[r + 1]) - int(qsl[r])
        if sl > 0 and ql > 0:
            active.append((r, sl, ql))
    # vflush_clear
    for r, sl, ql in active:
        p0, p1 = _written(sl, ql, page)
        for p in range(p0, p1 + 1):
            vfl[int(block_table[r, p])] = 0
    # flush_collect
    fcnt, top = 0, int(st["top"])
    for r, sl, ql in active:
        for p in range((sl - ql) // page):
            blk = int(block_table[r, p])
            vb = int(vbo[blk])
            if vb < 0:
                continue
            over = False
            if vfl[blk] == 0:
                if fcnt < maxf:
                    st["flush_list"][fcnt] = (blk, vb)
                    fcnt += 1
                    vfl[blk] = 1
                else:
                    over = True
            if not over:
                vbo[blk] = -1
                stack[top] = vb
                top += 1
    st["flush_cnt"] = fcnt
    # flush_copy
    v_pool = st["v_pool"]
    for i in range(fcnt):
        blk, vb = (int(x) for x in st["flush_list"][i])
        pool[:, blk] = np.swapaxes(v_pool[:, vb], 1, 2)      # (L, page, n_kv, d) -> kv-major
        pool_valid[:, :, blk] = 1
    # valloc
    for r, sl, ql in active:
        p0, p1 = _written(sl, ql, page)
        for p in range(p0, p1 + 1):
            blk = int(block_table[r, p])
            if vbo[blk] >= 0:
                continue
            if top == 0:
                st["overflow"] = 1
            else:
                top -= 1
                vbo[blk] = stack[top]
    st["top"] = top
    # vslot
    for r, sl, ql in active:
        q0 = int(qsl[r])
        for i in range(ql):
            pos = sl - ql + i
            vb = int(vbo[int(block_table[r, pos // page])])
            st["v_slot"][q0 + i] = vb * page + pos % page if vb >= 0 else -1


def scatter(v_pool_layer, value, v_slot, n_tokens, *, page):
    """In place: v_pool_layer (NV, page, n_kv, d); value (T, n_kv, d)."""
    for t in range(n_tokens):
        vs = int(v_slot[t])
        if vs >= 0:
            v_pool_layer[vs // page, vs % page] = value[t]


def read_v(blk, t, layer, kv, *, vbo, v_pool, pool, pool_valid, hot=None, page2slot=None,
           complete=True):
    """V row (d,) of token t of physical block blk as the tiered decode addresses it
    (tier/decode_mem.py:78-166): the hot slot of a complete resident page, else the
    staging pool, else the pinned pool.  None when none of them holds it."""
    if hot is not None and complete and page2slot[layer, kv, blk] >= 0:
        return hot[layer, kv, page2slot[layer, kv, blk], t]
    if vbo[blk] >= 0:
        return v_pool[layer, vbo[blk], t, kv]
    if pool_valid[layer, kv, blk]:
        return pool[layer, blk, kv, t]
    return None
