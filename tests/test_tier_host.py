"""The tier's host-side copy-engine planner (Residency.build_dma_plan, reference
tier/residency.py:438-493) on the CPU: a hand-worked miss list and the runs it must give,
and generated miss lists against a plain sequential walk.

A run is a chain of misses that follow each other in one (request, kv head) miss list
with victim slot and block both one higher than the previous one's and V valid in the
pinned pool; a miss with no slot (-1) or whose V is only staged breaks a chain (and the
latter sets has_staged)."""
import types

import numpy as np
import torch
from hypothesis import given, settings
from hypothesis import strategies as hs

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


def _sequential_runs(r, layer, n_req):
    """The plan by a plain walk over each (request, kv head) miss list: a run starts at a
    fetchable miss (slot >= 0, V valid in the pool) that does not continue the previous
    entry, and grows while the next entry is fetchable with slot and block one higher."""
    out, staged = [], False
    n_kv = r.n_kv
    for req in range(n_req):
        for kv in range(n_kv):
            m = int(r.miss_cnt[req, kv])
            blk = [int(x) for x in r.miss_pages[req, kv, :m]]
            slot = [int(x) for x in r.victim_slots[req, kv, :m]]
            ok = [slot[i] >= 0 and int(r.pool_valid[layer, kv, blk[i]]) == 1 for i in range(m)]
            staged |= any(slot[i] >= 0 and not ok[i] for i in range(m))
            i = 0
            while i < m:
                if not ok[i]:
                    i += 1
                    continue
                j = i + 1
                while j < m and ok[j] and slot[j] == slot[j - 1] + 1 and blk[j] == blk[j - 1] + 1:
                    j += 1
                out.append((kv, slot[i], blk[i], j - i))
                i = j
    return out, staged


@settings(max_examples=200, deadline=None, derandomize=True, database=None)
@given(data=hs.data())
def test_dma_runs_match_a_sequential_walk(data):
    """Generated miss lists (chains of consecutive slots and blocks broken at random, slots
    -1, pages valid only in staging, leftover entries past each count): the planner's run
    table equals the sequential walk's, run for run, and has_staged agrees."""
    n_req, n_kv, NB, MP, S = 3, 2, 64, 12, 24
    r = Residency(num_layers=1, num_blocks=NB, n_kv=n_kv, hot_slots=S, page=16, d=128,
                  max_reqs=n_req, max_pages=MP, dtype=torch.bfloat16, device="cpu")
    valid = data.draw(hs.lists(hs.booleans(), min_size=n_kv * NB, max_size=n_kv * NB))
    r.pool_valid[0] = torch.tensor(valid, dtype=torch.int8).view(n_kv, NB).to(r.pool_valid.dtype)
    for req in range(n_req):
        for kv in range(n_kv):
            m = data.draw(hs.integers(0, MP))
            b0, s0 = data.draw(hs.integers(0, NB - 1)), data.draw(hs.integers(0, S - 1))
            blocks, slots = [], []
            for _ in range(m):
                if data.draw(hs.booleans()):      # continue the chain
                    b0, s0 = (b0 + 1) % NB, (s0 + 1) % S
                else:
                    b0, s0 = data.draw(hs.integers(0, NB - 1)), data.draw(hs.integers(0, S - 1))
                blocks.append(b0)
                slots.append(-1 if data.draw(hs.integers(0, 9)) == 0 else s0)
            _miss(r, req, kv, blocks, slots)
    n = data.draw(hs.integers(0, n_req))
    pool = types.SimpleNamespace(_host_ptr=1 << 40)
    runs, staged = r.build_dma_plan(0, pool, n)
    want, want_staged = _sequential_runs(r, 0, n)
    hot = r.hot[0].data_ptr()
    exp = np.array([[hot + (kv * S + s) * PB, (1 << 40) + (b * n_kv + kv) * PB, PB,
                     n_kv * PB, PB, h] for kv, s, b, h in want], np.int64).reshape(-1, 6)
    assert staged == want_staged
    assert np.array_equal(runs, exp)


def test_dma_runs_at_a_narrower_plan_width():
    """A selection narrower than the residency's max_pages: the plan kernel writes the
    miss rows at the page table's width, and the planner reads them at that stride."""
    W = 5
    wide, narrow = _res(), Residency(num_layers=2, num_blocks=40, n_kv=2, hot_slots=12,
                                     page=16, d=128, max_reqs=2, max_pages=W,
                                     dtype=torch.bfloat16, device="cpu")
    narrow.pool_valid.fill_(1)
    pool = types.SimpleNamespace(_host_ptr=1 << 40)
    lists = {(0, 0): ([5, 6, 7, 9, 10], [2, 3, 4, 5, 6]), (0, 1): ([3, 4], [0, 1]),
             (1, 0): ([11, 12, 13], [7, 8, 9]), (1, 1): ([20], [11])}
    for (req, kv), (b, s) in lists.items():
        _miss(narrow, req, kv, b, s)
    # the wide residency's buffers hold the same rows at stride W, as the kernel writes them
    wide.miss_pages.view(-1)[:2 * 2 * W] = narrow.miss_pages.view(-1)
    wide.victim_slots.view(-1)[:2 * 2 * W] = narrow.victim_slots.view(-1)
    wide.miss_cnt.copy_(narrow.miss_cnt)
    wide.plan_width = W
    runs, staged = wide.build_dma_plan(0, pool, 2)
    want, _ = narrow.build_dma_plan(0, pool, 2)
    want[:, 0] += wide.hot[0].data_ptr() - narrow.hot[0].data_ptr()
    assert not staged and np.array_equal(runs, want)
    assert list(runs[:, 5]) == [3, 2, 2, 3, 1]
