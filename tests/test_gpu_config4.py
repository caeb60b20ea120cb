"""Config 4 (mem-v) at its benched shape, and the tier step captured in a HIP graph.

Shape: B = 32, 32768-token contexts (2048 pages), Llama-3.1-8B GQA (8 kv heads, G = 4),
quad r'=8 int8 nrm, coverage 0.95, literal +2 sigma boost; V in the pinned, device-mapped
host pool; hot buffer 10 % of the pages, 6553 slots per kv head (seven slots per thread in
the victims launch).  Two query streams, as the bench runs them: "fresh" (config 4's
literal N(0, 1) query each step; the nucleus keeps ~93 % of the pages, so most misses
find no slot and the decode reads them over the host link) and "correlated" (the case's
query + 0.3 N(0, 1)).

Every step: the tiered decode equals the resident decode of the same selection bit for
bit; page2slot and slot2page are mutual inverses; every occupied slot holds its page's V
bytes.  On the first two steps, for kv heads 0 and 5 (the plan is per kv head; the
sequential oracle, reference tier/residency.py:45-139, takes ~1 s per head here), the
maps, LRU clocks, miss and victim lists and the fetch list equal the oracle's.

Graph: select + residency plan + fetch + tiered decode captured in one HIP graph (the
reference's tier step is graph-safe, tier/decode_mem.py:32-33,240-246) and replayed from
the same cold state as an eager run, the query copied into the graph's input between
replays: every replay equals the eager step bit for bit -- output, page table, maps,
LRU clocks, hot buffer, miss counts, fetch count, overflow latch, the step clock, and the
victims launch's arrival word back at zero.
"""
import numpy as np
import pytest
import torch

import oracle.tier as otier
from amass.attention.decode import ResidentVSource, sparse_paged_decode_batched
from amass.bench.synth import build_quad_state, config_case
from amass.selection import derive_page_params, select_pages_quad
from amass.tier import Tier, mem_dynamic_decode
from helpers import announce, npi

pytestmark = pytest.mark.gpu
DEV = "cuda"
ORACLE_HEADS = (0, 5)


def _setup(boost, seed=0):
    case = config_case(4, seed=seed, device=DEV, boost=boost)
    st = build_quad_state(case, rank=8, v_bits=8, combine="nrm", coverage=0.95)
    B, MP = case.q.shape[0], case.max_pages
    NB = case.kv_cache.shape[0]
    slots = (B * MP) // 10
    assert (B, MP, slots) == (32, 2048, 6553)
    tier = Tier(num_layers=1, num_blocks=NB, n_kv=case.n_kv, page=16, d=128,
                hot_slots=slots, max_reqs=B, max_pages=MP, device=DEV, v_blocks=2 * B + 8)
    tier.flush_layer(0, case.kv_cache[:, 1])
    derive_page_params(st, case.seq_lens, B)
    return case, st, tier


def _queries(case, stream, n, seed):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    B, H = case.q.shape[0], case.n_kv * case.G
    qs = []
    for _ in range(n):
        z = torch.randn(B, H, 128, generator=gen, device=DEV)
        qs.append((z if stream == "fresh" else case.q.float() + 0.3 * z).to(torch.bfloat16))
    return qs


def _slots_hold_their_pages(tier, case):
    """I2 on the bytes: every occupied slot of the hot buffer holds its page's V."""
    r5 = tier.residency
    V = case.kv_cache[:, 1]                           # (NB, page, n_kv, d)
    for kv in range(case.n_kv):
        s2p = r5.slot2page[0, kv]
        occ = torch.nonzero(s2p >= 0).flatten()
        want = V[s2p[occ].long(), :, kv, :]
        assert torch.equal(r5.hot[0, kv, occ].view(torch.int16), want.view(torch.int16)), kv


def _oracle_heads(pre, st, case, r5):
    """The sequential plan on kv heads ORACLE_HEADS from the pre-step state."""
    p2s, s2p, lru, clock = pre
    tab, cnt = npi(st.page_table), npi(st.page_cnt)
    bt, sl = npi(case.block_table), npi(case.seq_lens)
    mc, mp, vs = npi(r5.miss_cnt), npi(r5.miss_pages), npi(r5.victim_slots)
    n_f = int(r5.fetch_cnt[0])
    fl = {tuple(x) for x in npi(r5.fetch_list[:n_f]).tolist()}
    for kv in ORACLE_HEADS:
        ref = otier.plan(tab[:, kv:kv + 1], cnt[:, kv:kv + 1], bt, sl, p2s[kv:kv + 1],
                         s2p[kv:kv + 1], lru[kv:kv + 1], clock, page=16)
        assert int(r5.clock[0]) == ref["clock"]
        assert np.array_equal(npi(r5.page2slot[0, kv]), ref["page2slot"][0]), kv
        assert np.array_equal(npi(r5.slot2page[0, kv]), ref["slot2page"][0]), kv
        assert np.array_equal(npi(r5.lru_clock[0, kv]), ref["lru"][0]), kv
        if ref["overflow"]:
            assert int(r5.overflow[0]) != 0
        for r in range(tab.shape[0]):
            m = ref["miss"][r][0]
            assert mc[r, kv] == len(m), (r, kv)
            assert list(mp[r, kv, :len(m)]) == m, (r, kv)
            assert list(vs[r, kv, :len(m)]) == ref["victims"][r][0], (r, kv)
        assert {x for x in fl if x[0] == kv} == {(kv, b, s) for _, b, s in ref["fetch"]}, kv


@pytest.mark.parametrize("stream", ["fresh", "correlated"])
def test_config4_full_shape(stream):
    announce(f"config 4 full shape: B=32 ctx 32768, 6553 slots per kv head, stream={stream}")
    case, st, tier = _setup("sigma")
    r5 = tier.residency
    B = case.q.shape[0]
    bt, sl = case.block_table, case.seq_lens
    hits = sel = 0
    for step, q in enumerate(_queries(case, stream, 8, seed=404)):
        select_pages_quad(st, 0, q, bt, sl, B, case.scale, derive=False)
        if step < 2:
            pre = tuple(npi(x[0]).astype(np.int64)
                        for x in (r5.page2slot, r5.slot2page, r5.lru_clock)) + (int(r5.clock[0]),)
        ref = torch.zeros(B, case.n_kv * case.G, 128, dtype=torch.bfloat16, device=DEV)
        sparse_paged_decode_batched(q, case.kv_cache, bt, sl, st, ref,
                                    ResidentVSource(case.kv_cache), scale=case.scale)
        out = torch.zeros_like(ref)
        mem_dynamic_decode(q, case.kv_cache, bt, sl, st, out, tier, 0, scale=case.scale,
                           fetch="kernel")
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"step {step}"
        assert int(r5._clock2[1]) == 0
        r5.assert_maps_inverse(0)
        _slots_hold_their_pages(tier, case)
        if step < 2:
            _oracle_heads(pre, st, case, r5)
        cnt = int(st.page_cnt.sum())
        sel += cnt
        hits += cnt - int(r5.miss_cnt.sum())
        announce(f"  step {step}: {cnt} pages selected, hit rate so far {hits / sel:.3f}, "
                 f"overflow {int(r5.overflow[0])}")


STATE = ("page2slot", "slot2page", "lru_clock", "_clock2", "overflow", "hot", "miss_cnt",
         "fetch_cnt")


@pytest.mark.parametrize("boost,stream", [("sigma", "fresh"), ("keynorm", "correlated")])
def test_config4_tier_step_in_graph(boost, stream):
    announce(f"config 4 tier step in a HIP graph: boost={boost} stream={stream}")
    case, st, tier = _setup(boost)
    r5 = tier.residency
    B = case.q.shape[0]
    bt, sl = case.block_table, case.seq_lens
    qs = _queries(case, stream, 4, seed=77)
    q_in = torch.empty_like(qs[0])
    out = torch.zeros(B, case.n_kv * case.G, 128, dtype=torch.bfloat16, device=DEV)

    def step():
        select_pages_quad(st, 0, q_in, bt, sl, B, case.scale, derive=False)
        mem_dynamic_decode(q_in, case.kv_cache, bt, sl, st, out, tier, 0, scale=case.scale,
                           fetch="kernel")

    cold = {k: getattr(r5, k).clone() for k in STATE}

    def restore():
        for k in STATE:
            getattr(r5, k).copy_(cold[k])

    # capture first (its warm-up runs the step), then the eager reference from cold
    q_in.copy_(qs[0])
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()

    restore()
    eager = []
    for q in qs:
        q_in.copy_(q)
        step()
        torch.cuda.synchronize()
        snap = {k: getattr(r5, k).clone() for k in STATE}
        snap.update(out=out.clone(), page_table=st.page_table.clone(),
                    page_cnt=st.page_cnt.clone())
        eager.append(snap)
    assert int(eager[-1]["_clock2"][0]) == int(cold["_clock2"][0]) + len(qs)

    restore()
    for i, q in enumerate(qs):
        out.view(torch.int16).fill_(0x5A5A)
        q_in.copy_(q)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = {k: getattr(r5, k) for k in STATE}
        got.update(out=out, page_table=st.page_table, page_cnt=st.page_cnt)
        for k, want in eager[i].items():
            assert torch.equal(got[k].view(torch.uint8), want.view(torch.uint8)), \
                f"replay {i}: {k}"
        assert int(r5._clock2[1]) == 0
        # eager work between replays (the graph must not depend on leftover state)
        torch.zeros(1 << 20, device=DEV).add_(1.0)
    del g
