"""The tier's host-side copy-engine planner (Residency.build_dma_plan, reference
tier/residency.py:438-493) on the CPU: a hand-worked miss list and the runs it must give.

A run is a chain of misses that follow each other in one (request, kv head) miss list
with victim slot and block both one higher than the previous one's and V valid in the
pinned pool; a miss with no slot (-1) or whose V is only staged breaks a chain (and the
latter sets has_staged)."""
import types

import numpy as np
import torch

from amass.tier.residency import Residency

PB = 16 * 128 * 2           # bytes of one V page (page 16, d 128, bf16)


def _res():
    r = Residency(num_layers=2, num_blocks=40, n_kv=2, hot_slots=12, page=16, d=128,
                  max_reqs=2, max_pages=8, dtype=torch.bfloat16, device="cpu")
    r.pool_valid.fill_(1)
    return r


def _miss(r, req, kv, blocks, slots):
    r.miss_cnt[req, kv] = len(blocks)
    r.miss_pages[req, kv, :len(blocks)] = torch.tensor(blocks, dtype=torch.int32)
    r.victim_slots[req, kv, :len(slots)] = torch.tensor(slots, dtype=torch.int32)
    # entries past the count hold leftovers that must be ignored
    r.miss_pages[req, kv, len(blocks):] = 7
    r.victim_slots[req, kv, len(slots):] = 3


def test_dma_runs_hand_worked():
    r = _res()
    pool = types.SimpleNamespace(_host_ptr=1 << 40)
    layer = 1
    _miss(r, 0, 0, [5, 6, 7, 9, 10], [2, 3, 4, 5, 6])      # -> (slot 2, blk 5, 3), (5, 9, 2)
    _miss(r, 0, 1, [3, 4, 20], [-1, 0, 1])                 # -> (0, 4, 1), (1, 20, 1)
    _miss(r, 1, 0, [11, 12, 13, 14], [7, 8, 9, 10])        # blk 13 only staged in layer 1
    r.pool_valid[layer, 0, 13] = 0                         # -> (7, 11, 2), (10, 14, 1)
    _miss(r, 1, 1, [], [])
    runs, staged = r.build_dma_plan(layer, pool, 2)
    assert staged
    hot = r.hot[layer].data_ptr()
    base = pool._host_ptr + layer * 40 * 2 * PB
    want = [(0, 2, 5, 3), (0, 5, 9, 2), (1, 0, 4, 1), (1, 1, 20, 1), (0, 7, 11, 2),
            (0, 10, 14, 1)]
    exp = np.array([[hot + (kv * 12 + s) * PB, base + (b * 2 + kv) * PB, PB, 2 * PB, PB, h]
                    for kv, s, b, h in want], np.int64)
    assert runs.dtype == np.int64 and np.array_equal(runs, exp)
    # the same lists with every page valid: nothing staged, blk 13 joins its chain
    r.pool_valid[layer, 0, 13] = 1
    runs, staged = r.build_dma_plan(layer, pool, 2)
    assert not staged
    assert list(runs[:, 5]) == [3, 2, 1, 1, 4]
    # only request 0 planned: request 1's lists are not read
    runs, staged = r.build_dma_plan(layer, pool, 1)
    assert not staged and list(runs[:, 5]) == [3, 2, 1, 1]
    runs, staged = r.build_dma_plan(layer, pool, 0)
    assert runs.shape == (0, 6) and not staged


def test_dma_runs_never_cross_lists():
    """Consecutive slots and blocks at the end of one list and the start of the next
    (another kv head / request) are separate runs."""
    r = _res()
    pool = types.SimpleNamespace(_host_ptr=1 << 40)
    _miss(r, 0, 0, [1, 2], [0, 1])
    _miss(r, 0, 1, [3, 4], [2, 3])
    r.miss_cnt[0, 0] = 8                                  # a full list: 8 entries
    r.miss_pages[0, 0] = torch.arange(1, 9, dtype=torch.int32)
    r.victim_slots[0, 0] = torch.arange(0, 8, dtype=torch.int32)
    _miss(r, 1, 0, [9], [8])
    runs, _ = r.build_dma_plan(0, pool, 2)
    assert list(runs[:, 5]) == [8, 2, 1]
