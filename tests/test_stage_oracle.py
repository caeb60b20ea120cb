"""CPU pins of the mem-v write-path oracle (oracle/stage.py).

Pinned by: a hand-worked two-step example (exact staging blocks, free stack, flush list
and token slots derived by hand from the reference's rules), a hand-worked invalidation,
and multi-request simulations in which every written token's V must read back through the
tier's address rule (staged, else flushed) after every step (I1) while assigned and free
staging blocks partition [0, NV) (I3) -- with a block shared by two requests, a flush
list too small for one step, and staging exhaustion.
"""
import numpy as np

import oracle.stage as ost


def _state(NB, NV, L, page, n_kv, d, maxf, max_tokens):
    return dict(vbo=np.full(NB, -1, np.int64), v_flushed=np.zeros(NB, np.int64),
                free_stack=np.arange(NV, dtype=np.int64), top=NV,
                v_slot=np.full(max_tokens, -1, np.int64),
                flush_list=np.zeros((maxf, 2), np.int64), flush_cnt=0, overflow=0,
                v_pool=np.zeros((L, NV, page, n_kv, d), np.float32))


def test_hand_worked_two_steps():
    page, NB, NV, L, n_kv, d = 2, 8, 4, 1, 1, 2
    st = _state(NB, NV, L, page, n_kv, d, maxf=4, max_tokens=4)
    pool = np.zeros((L, NB, n_kv, page, d), np.float32)
    pv = np.zeros((L, n_kv, NB), np.int8)
    bt = np.array([[5, 3, 7]])
    # step A: prefill 3 tokens -> pages 0 (blk 5) and 1 (blk 3) popped from the top
    ost.begin_step(bt, np.array([3]), np.array([0, 3]), 3, st, pool, pv, page=page, maxf=4)
    assert list(st["vbo"]) == [-1, -1, -1, 2, -1, 3, -1, -1]
    assert st["top"] == 2 and list(st["free_stack"][:2]) == [0, 1]
    assert list(st["v_slot"][:3]) == [6, 7, 4]            # vb*page + pos%page
    assert st["flush_cnt"] == 0
    vals = np.arange(3 * d, dtype=np.float32).reshape(3, 1, d) + 1
    ost.scatter(st["v_pool"][0], vals, st["v_slot"], 3, page=page)
    # step B: decode 1 token -> page 0 is complete: flushed, its block freed and pushed
    ost.begin_step(bt, np.array([4]), np.array([0, 1]), 1, st, pool, pv, page=page, maxf=4)
    assert st["flush_cnt"] == 1 and list(st["flush_list"][0]) == [5, 3]
    assert list(st["vbo"]) == [-1, -1, -1, 2, -1, -1, -1, -1]
    assert st["top"] == 3 and list(st["free_stack"][:3]) == [0, 1, 3]
    assert st["v_flushed"][5] == 1 and pv[0, 0, 5] == 1
    assert np.array_equal(pool[0, 5, 0], vals[:2, 0])     # the two tokens of page 0
    assert st["v_slot"][0] == 2 * 2 + 1                   # token 3 -> page 1, offset 1


def test_hand_worked_invalidate():
    page = 4
    p2s = np.full((2, 2, 10), -1, np.int64)
    s2p = np.full((2, 2, 3), -1, np.int64)
    pv = np.ones((2, 2, 10), np.int8)
    p2s[:, :, 6] = 1
    s2p[:, :, 1] = 6
    p2s[:, :, 2] = 0
    s2p[:, :, 0] = 2
    bt = np.array([[2, 6, 9]])
    # 9 tokens, 2 written this step -> pages 1 (blk 6) and 2 (blk 9)
    ost.invalidate(bt, np.array([9]), np.array([0, 2]), p2s, s2p, pv, page=page)
    assert (p2s[:, :, 6] == -1).all() and (s2p[:, :, 1] == -1).all()
    assert (p2s[:, :, 2] == 0).all() and (s2p[:, :, 0] == 2).all()   # page 0 untouched
    assert (pv[:, :, [6, 9]] == 0).all() and (pv[:, :, 2] == 1).all()


def _simulate(seed, *, maxf, NV, shared, steps=24, check=True):
    rng = np.random.default_rng(seed)
    page, L, n_kv, d, NB = 4, 2, 2, 4, 96
    R = 3
    perm = rng.permutation(NB)
    tables = [list(perm[0:20]), list(perm[20:40]), list(perm[40:60])]
    if shared:
        tables[2][0] = tables[0][0]          # request 2 reuses request 0's first block
    # per-step query lengths: request 0 prefill 9 then decode; request 1 joins at step 3
    # with a chunked prefill (6, 5); request 2 starts with its shared page present
    sched = np.zeros((steps, R), np.int64)
    sched[0, 0] = 9
    sched[1:, 0] = 1
    sched[3, 1], sched[4, 1] = 6, 5
    sched[5:, 1] = 1
    r2 = 1 if shared else 6                  # shared: both see the staged block in step 1
    sched[r2, 2] = 3
    sched[r2 + 1:, 2] = 1
    sl = np.zeros(R, np.int64)
    if shared:
        sl[2] = page                         # its first page is the shared, complete one
    truth = {}
    max_tokens = 16
    st = _state(NB, NV, L, page, n_kv, d, maxf, max_tokens)
    pool = np.zeros((L, NB, n_kv, page, d), np.float32)
    pv = np.zeros((L, n_kv, NB), np.int8)
    p2s = np.full((L, n_kv, NB), -1, np.int64)
    s2p = np.full((L, n_kv, 4), -1, np.int64)
    bt = np.array(tables)
    for s in range(steps):
        ql = sched[s]
        sl_new = sl + ql
        sl_step = np.where(ql > 0, sl_new, sl)
        qsl = np.concatenate([[0], np.cumsum(ql)])
        n_tok = int(qsl[-1])
        ost.invalidate(bt, sl_step, qsl, p2s, s2p, pv, page=page)
        ost.begin_step(bt, sl_step, qsl, n_tok, st, pool, pv, page=page, maxf=maxf)
        vals = rng.standard_normal((L, max(n_tok, 1), n_kv, d)).astype(np.float32)
        for l in range(L):
            ost.scatter(st["v_pool"][l], vals[l], st["v_slot"], n_tok, page=page)
        for r in range(R):
            for i in range(int(ql[r])):
                pos = int(sl[r]) + i
                blk = int(bt[r, pos // page])
                for l in range(L):
                    truth[(l, blk, pos % page)] = vals[l, int(qsl[r]) + i]
        sl = sl_step
        if not check:
            continue
        # I3: assigned + free staging blocks partition [0, NV)
        assigned = st["vbo"][st["vbo"] >= 0]
        both = np.sort(np.concatenate([assigned, st["free_stack"][:st["top"]]]))
        assert np.array_equal(both, np.arange(NV)), s
        # I1: every written token reads back (staged, else flushed)
        for (l, blk, t), v in truth.items():
            for kv in range(n_kv):
                got = ost.read_v(blk, t, l, kv, vbo=st["vbo"], v_pool=st["v_pool"], pool=pool,
                                 pool_valid=pv)
                assert got is not None, (s, l, blk, t)
                assert np.array_equal(got, v[kv]), (s, l, blk, t, kv)
    return st, pool, pv


def test_simulation_lifecycle_keeps_every_v():
    st, pool, pv = _simulate(1, maxf=64, NV=16, shared=False)
    assert st["overflow"] == 0
    # after the last step only the partial tails and the pages completed by the last
    # step are staged
    assert (st["vbo"] >= 0).sum() <= 6


def test_shared_block_is_flushed_and_freed_once():
    _simulate(2, maxf=64, NV=16, shared=True)


def test_small_flush_list_defers_but_loses_nothing():
    st, _, _ = _simulate(3, maxf=1, NV=24, shared=False)
    assert st["overflow"] == 0


def test_staging_exhaustion_sets_overflow():
    page, NB, NV = 4, 16, 2
    st = _state(NB, NV, 1, page, 1, 2, maxf=4, max_tokens=16)
    pool = np.zeros((1, NB, 1, page, 2), np.float32)
    pv = np.zeros((1, 1, NB), np.int8)
    bt = np.array([[3, 4, 5, 6]])
    ost.begin_step(bt, np.array([12]), np.array([0, 12]), 12, st, pool, pv, page=page, maxf=4)
    assert st["overflow"] == 1 and st["top"] == 0
    assert list(st["vbo"][[3, 4, 5]]) == [1, 0, -1]        # the third page got none
    assert (st["v_slot"][8:12] == -1).all()
