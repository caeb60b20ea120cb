"""mem-v tier residency plan (test oracle).

plan restates tier/residency.py:45-139 sequentially:
  clock += 1 (residency.py:394); for every (request, kv-head) unit and selected page j
  (in page_table order): blk = block_table[r, pt]; complete = (pt+1)*page <= seq_len;
  resident (page2slot >= 0) complete pages touch lru = clock; complete non-resident pages
  are misses, compacted in order (_miss_diff_kernel).  Then per kv-head, for r in order,
  for each miss i in order: if page2slot[blk] >= 0 (installed earlier this step) the
  victim is -1; else the victim is argmin over slots with lru < clock of lru (ties ->
  lowest slot index); none -> overflow, -1; else evict slot2page[victim], install, set
  lru = clock and append (kv, blk, slot) to the fetch list (_select_victims_kernel).
"""
from __future__ import annotations

import numpy as np


def plan(page_table, page_cnt, block_table, seq_lens, page2slot, slot2page, lru, clock, *,
         page: int):
    """Mutates copies; returns dict of the new state and per-step outputs."""
    p2s = np.array(page2slot, np.int64, copy=True)       # (n_kv, NB)
    s2p = np.array(slot2page, np.int64, copy=True)       # (n_kv, S)
    lru = np.array(lru, np.int64, copy=True)             # (n_kv, S)
    clk = int(clock) + 1
    R, n_kv, MP = page_table.shape
    S = s2p.shape[1]
    miss = [[[] for _ in range(n_kv)] for _ in range(R)]
    for r in range(R):
        sl = int(seq_lens[r])
        for kv in range(n_kv):
            for j in range(int(page_cnt[r, kv])):
                pt = int(page_table[r, kv, j])
                blk = int(block_table[r, pt])
                if (pt + 1) * page > sl:
                    continue
                s = p2s[kv, blk]
                if s >= 0:
                    lru[kv, s] = clk
                else:
                    miss[r][kv].append(blk)
    victims = [[[] for _ in range(n_kv)] for _ in range(R)]
    fetch = set()
    overflow = False
    for kv in range(n_kv):
        for r in range(R):
            for blk in miss[r][kv]:
                if p2s[kv, blk] >= 0:
                    victims[r][kv].append(-1)
                    continue
                cand = np.nonzero(lru[kv] < clk)[0]
                if cand.size == 0:
                    overflow = True
                    victims[r][kv].append(-1)
                    continue
                best = int(cand[np.argmin(lru[kv, cand])])   # argmin -> lowest index
                old = s2p[kv, best]
                if old >= 0:
                    p2s[kv, old] = -1
                p2s[kv, blk] = best
                s2p[kv, best] = blk
                lru[kv, best] = clk
                victims[r][kv].append(best)
                fetch.add((kv, blk, best))
    return dict(page2slot=p2s, slot2page=s2p, lru=lru, clock=clk, miss=miss,
                victims=victims, fetch=fetch, overflow=overflow)

