"""GPU parity of the mem-v tier: gather plan vs the sequential oracle (bit-exact maps,
victims, miss lists; fetch list as a set), fetch from the pinned host pool, and the
tiered decode equal bit for bit to the resident decode (same bytes, same kernels)."""
import numpy as np
import pytest
import torch

import oracle.select as osel
import oracle.tier as otier
from amass.attention import ensure_stage_b_buffers
from amass.attention.decode import ResidentVSource, sparse_paged_decode_batched
from amass.bench.synth import make_case
from amass.tier import Tier, mem_dynamic_decode
from helpers import announce, npi

pytestmark = pytest.mark.gpu
DEV = "cuda"


class _St:
    pass


def _selection(case, frac, seed):
    B, n_kv, MP = case.q.shape[0], case.n_kv, case.max_pages
    gen = torch.Generator().manual_seed(seed)
    sc = torch.randn(B, n_kv, MP, generator=gen).numpy()
    npg, nsh, bfix = osel.derive(case.seq_lens.numpy(), frac, 16, 1, 1)
    tab, cnt, _ = osel.select(sc, npg, nsh, bfix, sink=1, max_pages=MP, mode=0)
    return tab, cnt


def _tier(case, slots):
    NB = case.kv_cache.shape[0]
    t = Tier(num_layers=1, num_blocks=NB, n_kv=case.n_kv, page=16, d=128, hot_slots=slots,
             max_reqs=case.q.shape[0], max_pages=case.max_pages, device=DEV, v_blocks=4)
    t.flush_layer(0, case.kv_cache[:, 1])
    return t


@pytest.mark.parametrize("slots", [64, 600])
def test_plan_matches_oracle_over_steps(slots):
    announce(f"tier plan slots={slots}")
    case = make_case(B=4, ctx=(500, 2500), n_kv=8, G=4, heavy=0.0, seed=5)
    tier = _tier(case, slots)
    r5 = tier.residency
    bt, sl = case.block_table.to(DEV), case.seq_lens.to(DEV)
    p2s = npi(r5.page2slot[0]).astype(np.int64)
    s2p = npi(r5.slot2page[0]).astype(np.int64)
    lru = npi(r5.lru_clock[0]).astype(np.int64)
    clock = int(r5.clock[0])
    for step in range(6):
        # overlapping selections across steps so hits, misses and evictions all occur
        tab, cnt = _selection(case, 0.15, seed=step % 3)
        ref = otier.plan(tab, cnt, npi(case.block_table), npi(case.seq_lens), p2s, s2p, lru,
                         clock, page=16)
        r5.overflow.zero_()
        r5.gather_plan(0, torch.from_numpy(tab).to(DEV), torch.from_numpy(cnt).to(DEV), bt, sl,
                       4)
        torch.cuda.synchronize()
        assert int(r5.clock[0]) == ref["clock"]
        assert np.array_equal(npi(r5.page2slot[0]), ref["page2slot"])
        assert np.array_equal(npi(r5.slot2page[0]), ref["slot2page"])
        assert np.array_equal(npi(r5.lru_clock[0]), ref["lru"])
        assert bool(r5.overflow[0]) == ref["overflow"]
        mc, mp, vs = npi(r5.miss_cnt), npi(r5.miss_pages), npi(r5.victim_slots)
        for r in range(4):
            for kv in range(8):
                m = ref["miss"][r][kv]
                assert mc[r, kv] == len(m)
                assert list(mp[r, kv, :len(m)]) == m
                assert list(vs[r, kv, :len(m)]) == ref["victims"][r][kv]
        n = int(r5.fetch_cnt[0])
        fl = npi(r5.fetch_list[:n])
        assert set(map(tuple, fl.tolist())) == ref["fetch"]
        r5.assert_maps_inverse(0)
        p2s, s2p, lru, clock = ref["page2slot"], ref["slot2page"], ref["lru"], ref["clock"]


@pytest.mark.parametrize("slots,span,fill", [(3000, 40, 0.75), (700, 200, 1.0),
                                            (700, 5000, 1.0), (6553, 40, 1.0),
                                            (8192, 200, 0.9), (8192, 5000, 1.0)])
def test_plan_matches_oracle_with_aged_clocks(slots, span, fill):
    """Victim order over an aged hot buffer: slots already hold pages with LRU clocks
    spread over `span` steps (clocks within 255 of the oldest take the histogram path,
    wider spans the full radix sort), more slots than threads per kv head (3000; 6553,
    config 4's buffer, seven slots per thread; 8192, the most a kv head may hold), and
    repeated clocks (ties broken by slot index), empty slots (clock 0) or a full buffer.
    Bit-exact against the sequential oracle over four steps."""
    announce(f"tier plan aged clocks slots={slots} span={span} fill={fill}")
    big = slots > 3000
    case = make_case(B=4, ctx=(40000, 60000) if big else (2000, 6000), n_kv=8, G=4,
                     heavy=0.0, seed=15, device=DEV if big else "cpu")
    case.block_table, case.seq_lens = case.block_table.cpu(), case.seq_lens.cpu()
    tier = _tier(case, slots)
    r5 = tier.residency
    NB = case.kv_cache.shape[0]
    gen = np.random.default_rng(slots + span)
    assert NB >= (slots if big else 700)
    p2s = np.full((8, NB), -1, np.int64)
    s2p = np.full((8, slots), -1, np.int64)
    lru = np.zeros((8, slots), np.int64)
    clock = span + 10
    for kv in range(8):
        nres = int(min(slots, NB) * fill)
        blks = gen.choice(NB, nres, replace=False)
        sl_ = gen.choice(slots, nres, replace=False)
        p2s[kv, blks] = sl_
        s2p[kv, sl_] = blks
        lru[kv, sl_] = gen.integers(clock - span, clock, nres)   # repeats at small spans
    r5.page2slot[0].copy_(torch.from_numpy(p2s.astype(np.int32)))
    r5.slot2page[0].copy_(torch.from_numpy(s2p.astype(np.int32)))
    r5.lru_clock[0].copy_(torch.from_numpy(lru.astype(np.int32)))
    r5.clock.fill_(clock)
    bt, sl = case.block_table.to(DEV), case.seq_lens.to(DEV)
    for step in range(4):
        tab, cnt = _selection(case, 0.3, seed=10 + step)
        ref = otier.plan(tab, cnt, npi(case.block_table), npi(case.seq_lens), p2s, s2p, lru,
                         clock, page=16)
        r5.overflow.zero_()
        r5.gather_plan(0, torch.from_numpy(tab).to(DEV), torch.from_numpy(cnt).to(DEV), bt, sl,
                       4)
        torch.cuda.synchronize()
        assert int(r5.clock[0]) == ref["clock"]
        assert np.array_equal(npi(r5.page2slot[0]), ref["page2slot"])
        assert np.array_equal(npi(r5.slot2page[0]), ref["slot2page"])
        assert np.array_equal(npi(r5.lru_clock[0]), ref["lru"])
        assert bool(r5.overflow[0]) == ref["overflow"]
        vs = npi(r5.victim_slots)
        for r in range(4):
            for kv in range(8):
                assert list(vs[r, kv, :len(ref["miss"][r][kv])]) == ref["victims"][r][kv]
        p2s, s2p, lru, clock = ref["page2slot"], ref["slot2page"], ref["lru"], ref["clock"]


def test_plan_without_requests_advances_the_clock():
    """A plan over zero requests changes no map, installs nothing, and still advances the
    step clock (the victims launch runs alone and its last workgroup stores it)."""
    announce("tier plan with no requests")
    case = make_case(B=2, ctx=(500, 900), n_kv=8, G=4, heavy=0.0, seed=3)
    tier = _tier(case, 64)
    r5 = tier.residency
    bt, sl = case.block_table.to(DEV), case.seq_lens.to(DEV)
    tab, cnt = _selection(case, 0.5, seed=1)
    r5.gather_plan(0, torch.from_numpy(tab).to(DEV), torch.from_numpy(cnt).to(DEV), bt, sl, 2)
    torch.cuda.synchronize()
    before = [npi(x).copy() for x in (r5.page2slot, r5.slot2page, r5.lru_clock)]
    clk = int(r5.clock[0])
    r5.fetch_cnt.fill_(5)
    for i in range(3):
        r5.gather_plan(0, torch.from_numpy(tab).to(DEV), torch.from_numpy(cnt).to(DEV), bt,
                       sl, 0)
        torch.cuda.synchronize()
        assert int(r5.clock[0]) == clk + 1 + i
        assert int(r5._clock2[1]) == 0 and int(r5.fetch_cnt[0]) == 0
    for x, y in zip(before, (r5.page2slot, r5.slot2page, r5.lru_clock)):
        assert np.array_equal(x, npi(y))


@pytest.mark.parametrize("fetch", ["kernel", "dma", "off"])
def test_tiered_decode_bitexact_vs_resident(fetch):
    announce(f"tiered decode fetch={fetch}")
    case = make_case(B=3, ctx=(400, 2000), n_kv=8, G=4, heavy=0.0, seed=9)
    tier = _tier(case, 128)
    kv = case.kv_cache.to(DEV)
    bt, sl, q = case.block_table.to(DEV), case.seq_lens.to(DEV), case.q.to(DEV)
    st = _St()
    st.max_reqs, st.n_kv, st.G, st.D = 3, 8, 4, 128
    ensure_stage_b_buffers(st, DEV)
    for step in range(3):
        tab, cnt = _selection(case, 0.1, seed=step)
        st.page_table = torch.from_numpy(tab).to(DEV)
        st.page_cnt = torch.from_numpy(cnt).to(DEV)
        ref = torch.zeros(3, 32, 128, dtype=torch.bfloat16, device=DEV)
        sparse_paged_decode_batched(q, kv, bt, sl, st, ref, ResidentVSource(kv),
                                    scale=case.scale, path="split")
        out = torch.zeros_like(ref)
        mem_dynamic_decode(q, kv, bt, sl, st, out, tier, 0, scale=case.scale, fetch=fetch,
                           path="split")
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"step {step}"
    if fetch != "off":
        # every resident slot holds exactly its page's bytes (I2)
        r5 = tier.residency
        s2p = npi(r5.slot2page[0])
        hot = r5.hot[0].cpu()
        V = case.kv_cache[:, 1]
        for kvh in range(8):
            for s in np.nonzero(s2p[kvh] >= 0)[0][:50]:
                assert torch.equal(hot[kvh, s], V[int(s2p[kvh, s]), :, kvh, :])
