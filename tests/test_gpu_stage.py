"""GPU parity of the mem-v write path against the oracle (oracle/stage.py).

A multi-request scenario (prefill, chunked prefill, decode, a block shared by two
requests) is stepped through ``Residency.invalidate_written``, ``Staging.begin_step`` and
``Staging.scatter_kv`` on the GPU and through the oracle on the CPU; after every step the
staging-block map, flushed latches, free stack and its top, flush list, token slots,
overflow latch, staged pool, pinned pool, pool validity and residency maps are compared
bit for bit.  Also: a flush list too small for one step, staging exhaustion, and the
tiered decode reading written-path V (staged and flushed) equal to the resident decode.
"""
import numpy as np
import pytest
import torch

import oracle.stage as ost
from amass.tier.pool import MappedHostVPool
from amass.tier.residency import Residency
from amass.tier.staging import Staging
from helpers import announce

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _np(t):
    if t.dtype == torch.bfloat16:
        return t.detach().float().cpu().numpy()
    return t.detach().cpu().numpy().astype(np.int64)


class _Scenario:
    def __init__(self, *, seed, NV, maxf, shared, L=2, n_kv=2, d=16, page=4, NB=96, R=3,
                 MP=20, max_tokens=16, slots=4):
        self.L, self.n_kv, self.d, self.page, self.NB, self.R, self.MP = L, n_kv, d, page, NB, R, MP
        self.maxf, self.NV, self.max_tokens = maxf, NV, max_tokens
        rng = np.random.default_rng(seed)
        self.gen = torch.Generator().manual_seed(seed)
        perm = rng.permutation(NB)
        tables = [list(perm[0:MP]), list(perm[MP:2 * MP]), list(perm[2 * MP:3 * MP])]
        if shared:
            tables[2][0] = tables[0][0]
        self.bt = np.array(tables, np.int64)
        self.bt_d = torch.tensor(self.bt, dtype=torch.int32, device=DEV)
        self.sl = np.zeros(R, np.int64)
        if shared:
            self.sl[2] = page
        self.shared = shared
        # GPU side
        self.pool = MappedHostVPool(num_layers=L, num_blocks=NB, n_kv=n_kv, page=page, d=d,
                                    dtype=torch.bfloat16, device=DEV)
        self.res = Residency(num_layers=L, num_blocks=NB, n_kv=n_kv, hot_slots=slots,
                             page=page, d=d, max_reqs=R, max_pages=MP, dtype=torch.bfloat16,
                             device=DEV)
        self.stg = Staging(num_layers=L, num_blocks=NB, n_kv=n_kv, page=page, d=d,
                           dtype=torch.bfloat16, device=DEV, max_reqs=R, max_pages=MP,
                           max_tokens=max_tokens, v_blocks=NV, max_flush=maxf)
        # resident pages that later steps rewrite (request 1's first pages)
        p2s = np.full((L, n_kv, NB), -1, np.int64)
        s2p = np.full((L, n_kv, slots), -1, np.int64)
        for s, blk in enumerate(self.bt[1, :2]):
            p2s[:, :, blk] = s
            s2p[:, :, s] = blk
        self.res.page2slot.copy_(torch.tensor(p2s, dtype=torch.int32))
        self.res.slot2page.copy_(torch.tensor(s2p, dtype=torch.int32))
        # oracle side
        self.p2s, self.s2p = p2s, s2p
        self.pv = np.zeros((L, n_kv, NB), np.int8)
        self.opool = np.zeros((L, NB, n_kv, page, d), np.float32)
        self.ost = dict(vbo=np.full(NB, -1, np.int64), v_flushed=np.zeros(NB, np.int64),
                        free_stack=np.arange(NV, dtype=np.int64), top=NV,
                        v_slot=np.full(max_tokens, -1, np.int64),
                        flush_list=np.zeros((maxf, 2), np.int64), flush_cnt=0, overflow=0,
                        v_pool=np.zeros((L, NV, page, n_kv, d), np.float32))

    def step(self, ql):
        ql = np.asarray(ql, np.int64)
        sl_step = np.where(ql > 0, self.sl + ql, self.sl)
        qsl = np.concatenate([[0], np.cumsum(ql)])
        n_tok = int(qsl[-1])
        vals = torch.randn(self.L, max(n_tok, 1), self.n_kv, self.d,
                           generator=self.gen).to(torch.bfloat16)
        sl_d = torch.tensor(sl_step, dtype=torch.int32, device=DEV)
        qsl_d = torch.tensor(qsl, dtype=torch.int32, device=DEV)
        self.res.invalidate_written(self.bt_d, sl_d, qsl_d)
        self.stg.begin_step(self.bt_d, sl_d, qsl_d, n_tok, self.pool, self.res.pool_valid)
        vd = vals.to(DEV)
        for l in range(self.L):
            self.stg.scatter_kv(l, None, vd[l], n_tok)
        torch.cuda.synchronize()
        ost.invalidate(self.bt, sl_step, qsl, self.p2s, self.s2p, self.pv, page=self.page)
        ost.begin_step(self.bt, sl_step, qsl, n_tok, self.ost, self.opool, self.pv,
                       page=self.page, maxf=self.maxf)
        vf = vals.float().numpy()
        for l in range(self.L):
            ost.scatter(self.ost["v_pool"][l], vf[l], self.ost["v_slot"], n_tok, page=self.page)
        self.sl = sl_step
        self.check(n_tok)

    def check(self, n_tok):
        o, g = self.ost, self.stg
        assert np.array_equal(_np(g.vbo), o["vbo"])
        assert np.array_equal(_np(g.v_flushed), o["v_flushed"])
        top = int(g.v_free_top.item())
        assert top == o["top"]
        assert np.array_equal(_np(g.v_free_stack)[:top], o["free_stack"][:top])
        cnt = int(g.flush_cnt.item())
        assert cnt == o["flush_cnt"]
        assert np.array_equal(_np(g.flush_list)[:cnt], o["flush_list"][:cnt])
        assert np.array_equal(_np(g.v_slot_mapping)[:n_tok], o["v_slot"][:n_tok])
        assert int(g.overflow.item()) == o["overflow"]
        assert np.array_equal(_np(g.v_pool), o["v_pool"])
        assert np.array_equal(self.pool.host.float().numpy(), self.opool)
        assert np.array_equal(_np(self.res.pool_valid), self.pv.astype(np.int64))
        assert np.array_equal(_np(self.res.page2slot), self.p2s)
        assert np.array_equal(_np(self.res.slot2page), self.s2p)
        assert int(self.stg.first.min().item()) == 2 ** 31 - 1      # scratch back at rest


def _schedule(steps, shared):
    R = 3
    sched = np.zeros((steps, R), np.int64)
    sched[0, 0] = 9
    sched[1:, 0] = 1
    sched[3, 1], sched[4, 1] = 6, 5
    sched[5:, 1] = 1
    r2 = 1 if shared else 6
    sched[r2, 2] = 3
    sched[r2 + 1:, 2] = 1
    return sched


@pytest.mark.parametrize("shared", [False, True])
@pytest.mark.parametrize("maxf", [64, 1])
def test_write_path_matches_oracle(shared, maxf):
    announce(f"write path shared={shared} maxf={maxf}")
    sc = _Scenario(seed=5 + maxf + 2 * shared, NV=24, maxf=maxf, shared=shared)
    for ql in _schedule(20, shared):
        sc.step(ql)
    sc.stg.assert_free_partition()


def test_staging_exhaustion_matches_oracle():
    announce("write path staging exhaustion")
    sc = _Scenario(seed=9, NV=2, maxf=8, shared=False)
    sc.step([9, 0, 0])                     # three written pages, two staging blocks
    assert int(sc.stg.overflow.item()) == 1


def test_tiered_decode_reads_written_path_v():
    """Prefill through the write path (scatter, flush), then the tiered decode of the
    selected pages equals the resident decode bit for bit: pages the lifecycle has
    flushed come from the pinned pool, the partial tails from the staging pool."""
    announce("tiered decode over written-path V")
    from amass.attention import ensure_stage_b_buffers
    from amass.attention.decode import ResidentVSource, sparse_paged_decode_batched
    from amass.tier.tier import Tier, TierVSource

    B, n_kv, G, d, page, NB, MP, L = 3, 8, 4, 128, 16, 64, 8, 1
    gen = torch.Generator().manual_seed(3)
    tier = Tier(num_layers=L, num_blocks=NB, n_kv=n_kv, page=page, d=d, hot_slots=8,
                max_reqs=B, max_pages=MP, device=DEV, max_tokens=128, v_blocks=32)
    bt = torch.randperm(NB, generator=gen)[:B * MP].view(B, MP).to(torch.int32)
    kv = torch.randn(NB, 2, page, n_kv, d, generator=gen).to(torch.bfloat16)
    lens = [70, 35, 50]                     # tokens per request, written in two steps
    sl = torch.zeros(B, dtype=torch.int32)
    bt_d = bt.to(DEV)
    for part in (0.5, 1.0):
        tgt = torch.tensor([int(x * part) for x in lens], dtype=torch.int32)
        ql = tgt - sl
        qsl = torch.cat([torch.zeros(1, dtype=torch.int32), torch.cumsum(ql, 0).to(torch.int32)])
        n_tok = int(qsl[-1])
        vals = torch.empty(n_tok, n_kv, d, dtype=torch.bfloat16)
        for r in range(B):
            for i in range(int(ql[r])):
                pos = int(sl[r]) + i
                vals[int(qsl[r]) + i] = kv[int(bt[r, pos // page]), 1, pos % page]
        tier.begin_step(bt_d, tgt.to(DEV), qsl.to(DEV), n_tok)
        tier.write_kv(0, vals.to(DEV), n_tok)
        sl = tgt
    # complete pages of the first part were flushed by the second step; the rest are staged
    torch.cuda.synchronize()
    tier.assert_invariants(bt_d, sl.to(DEV), qsl.to(DEV))
    assert int((tier.staging.vbo >= 0).sum().item()) > 0
    assert int(tier.residency.pool_valid.sum().item()) > 0
    # select every written page of every head and decode both ways
    class _St:
        pass

    st = _St()
    st.max_reqs, st.n_kv, st.G, st.D = B, n_kv, G, d
    npg = (sl + page - 1) // page
    tab = torch.full((B, n_kv, MP), -1, dtype=torch.int32)
    cnt = torch.zeros(B, n_kv, dtype=torch.int32)
    for r in range(B):
        tab[r, :, :int(npg[r])] = torch.arange(int(npg[r]), dtype=torch.int32)
        cnt[r] = int(npg[r])
    st.page_table, st.page_cnt = tab.to(DEV), cnt.to(DEV)
    ensure_stage_b_buffers(st, DEV)
    q = torch.randn(B, n_kv * G, d, generator=gen).to(torch.bfloat16).to(DEV)
    kvd = kv.to(DEV)
    outs = []
    for vs in (ResidentVSource(kvd), TierVSource(tier, 0)):
        out = torch.zeros(B, n_kv * G, d, dtype=torch.bfloat16, device=DEV)
        sparse_paged_decode_batched(q, kvd, bt_d, sl.to(DEV), st, out, vs,
                                    scale=d ** -0.5, path="fused")
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


def test_write_path_graph_replay_matches_eager():
    """Decode steps (every request appends one token) through begin_step + write_kv:
    one tier runs them eagerly, a second replays one captured step from static input
    buffers refreshed between replays; after every step the staging map, flush state,
    token slots, staged pool, pinned pool and pool validity agree bit for bit (the
    lifecycle crosses a page boundary, so flushes replay too)."""
    announce("write path graph replay vs eager")
    from amass.tier.tier import Tier
    R, n_kv, d, page, NB, MP = 3, 2, 128, 16, 48, 8
    gen = torch.Generator().manual_seed(17)
    bt = torch.randperm(NB, generator=gen)[:R * MP].view(R, MP).to(torch.int32).to(DEV)
    mk = lambda: Tier(num_layers=1, num_blocks=NB, n_kv=n_kv, page=page, d=d,  # noqa: E731
                      hot_slots=4, max_reqs=R, max_pages=MP, device=DEV, max_tokens=R,
                      v_blocks=2 * R + 4)
    ta, tb = mk(), mk()
    sl0 = torch.tensor([20, 9, 31], dtype=torch.int32)
    qsl = torch.arange(R + 1, dtype=torch.int32, device=DEV)
    sl_buf = torch.zeros(R, dtype=torch.int32, device=DEV)
    v_buf = torch.zeros(R, n_kv, d, dtype=torch.bfloat16, device=DEV)

    def step(t):
        t.begin_step(bt, sl_buf, qsl, R)
        t.write_kv(0, v_buf, R)

    sl_buf.copy_(sl0 + 1)
    step(tb)                                    # warm-up outside capture, mirrored on ta
    step(ta)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step(tb)
    torch.cuda.synchronize()
    for k in range(2, 20):
        sl_buf.copy_(sl0 + k)
        v_buf.copy_(torch.randn(R, n_kv, d, generator=gen).to(torch.bfloat16))
        step(ta)
        g.replay()
        torch.cuda.synchronize()
        sa, sb = ta.staging, tb.staging
        for name in ("vbo", "v_flushed", "v_free_top", "flush_cnt", "overflow", "v_pool"):
            assert torch.equal(getattr(sa, name), getattr(sb, name)), (k, name)
        top = int(sa.v_free_top.item())
        assert torch.equal(sa.v_free_stack[:top], sb.v_free_stack[:top]), k
        assert torch.equal(sa.v_slot_mapping[:R], sb.v_slot_mapping[:R]), k
        assert torch.equal(ta.pool.host, tb.pool.host), k
        assert torch.equal(ta.residency.pool_valid, tb.residency.pool_valid), k
    assert int(ta.residency.pool_valid.sum().item()) > 0     # some page was flushed
