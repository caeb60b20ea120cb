"""Parity at the BASELINE configurations' real shapes (full context lengths and head
geometry; batch reduced so the CPU oracle finishes in seconds).

config 2: r8 score, 6 ragged sequences spanning 2048..65536 tokens, fixed 5 % budget,
          random pool block tables -> r8 int32 sums exact, scores 1e-3, page sets exact,
          decode 2e-2 / 1e-2;
config 3: 70B GQA shape (G = 8), 131072-token contexts (8192 pages), 2 % heavy pages,
          quad r'=8 nrm, coverage 0.95 -> scores 1e-3, page sets exact, decode;
config 4: mem-v, 32768-token contexts, hot buffer = 10 % of the pages per kv head,
          64 decode steps with a fresh query each step: every step's tiered decode is
          bit-identical to the resident decode of the same selection, the residency plan
          matches the sequential oracle on the first steps, and the hot-buffer hit rate
          is reported.
"""
import numpy as np
import pytest
import torch

import oracle.decode as odec
import oracle.score as osc
import oracle.select as osel
import oracle.tier as otier
from amass.attention.decode import ResidentVSource, sparse_paged_decode_batched
from amass.bench.synth import build_quad_state, build_r8_state, make_case
from amass.selection import derive_page_params, select_pages_quad
from amass.tier import Tier, mem_dynamic_decode
from helpers import announce, npf, npi, rel_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _decode_check(case, st, rows, atol=2e-2, rtol=1e-2):
    B = case.q.shape[0]
    H = case.n_kv * case.G
    out = torch.zeros(B, H, 128, dtype=torch.bfloat16, device=DEV)
    sparse_paged_decode_batched(case.q, case.kv_cache, case.block_table, case.seq_lens, st,
                                out, ResidentVSource(case.kv_cache), scale=case.scale)
    torch.cuda.synchronize()
    tab, cnt = npi(st.page_table), npi(st.page_cnt)
    K, V = case.kv_cache[:, 0], case.kv_cache[:, 1]
    got = npf(out)
    for r in rows:
        # the oracle attends one request at a time over its own blocks only
        blk = np.unique(npi(case.block_table[r, :int(np.ceil(int(case.seq_lens[r]) / 16))]))
        remap = np.full(K.shape[0], -1, np.int64)
        remap[blk] = np.arange(blk.size)
        Kr = npf(K[torch.from_numpy(blk).to(DEV)])
        Vr = npf(V[torch.from_numpy(blk).to(DEV)])
        bt = remap[npi(case.block_table[r:r + 1]).clip(0)]
        want = odec.attend(npf(case.q[r:r + 1]), Kr, Vr, bt, npi(case.seq_lens[r:r + 1]),
                           tab[r:r + 1], cnt[r:r + 1], scale=case.scale, G=case.G)
        assert np.allclose(got[r:r + 1], want, atol=atol, rtol=rtol), \
            f"req {r}: {float(np.abs(got[r:r + 1] - want).max())}"


def test_config2_r8_ragged():
    announce("config 2: r8 ragged 2K..64K, budget 5%")
    case = make_case(B=6, ctx=(2048, 65536), n_kv=8, G=4, heavy=0.05, table="pool", seed=2,
                     device=DEV)
    case.seq_lens[0] = 2048                  # the shortest length of the range
    B, MP = 6, case.max_pages
    st = build_r8_state(case, vk_bits=8, c_bits=8, budget=0.05)
    comb = torch.zeros(B, 8, MP, 4, 9, dtype=torch.int32, device=DEV)
    from amass.selection.score import r8_score
    from amass.selection.select import select_pages
    derive_page_params(st, case.seq_lens, B)
    r8_score(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale, comb_out=comb)
    select_pages(st, B)
    torch.cuda.synchronize()
    mu, mus, _, Vks, c, cs, _ = st.layer_state(0)
    Vk = st.reference_Vk(0)
    nsh = npi(st.n_sel_hi)
    rows = [0, 1, 4]
    sub = lambda t: npi(t)  # noqa: E731
    for r in rows:
        n = int(nsh[r])
        blk = npi(case.block_table[r, :n]).astype(np.int64)
        idx = torch.from_numpy(blk).to(DEV)
        bt = np.arange(n, dtype=np.int32)[None]
        ref_comb = osc.r8_comb(npf(case.q[r:r + 1]), sub(mu[idx]), sub(Vk[idx]), bt,
                               np.array([n]), G=4, vk_bits=8, max_pages=n)
        assert np.array_equal(npi(comb[r:r + 1, :, :n]).astype(np.int64), ref_comb)
        ref = osc.r8_score(npf(case.q[r:r + 1]), sub(mu[idx]), npf(mus[idx]), sub(Vk[idx]),
                           npf(Vks[idx]), sub(c[idx]), npf(cs[idx]), bt,
                           npi(case.seq_lens[r:r + 1]), np.array([n]), scale=case.scale,
                           page=16, G=4, vk_bits=8, c_bits=8, max_pages=n)
        assert rel_close(npf(st.score[r, :, :n]), ref[0], 1) <= 1e-3
    tab, cnt, _ = osel.select(npf(st.score), npi(st.n_pages), nsh, npi(st.b_fix), sink=1,
                              max_pages=MP, mode=0)
    assert np.array_equal(npi(st.page_table), tab) and np.array_equal(npi(st.page_cnt), cnt)
    _decode_check(case, st, rows)


def test_config3_g8_131k_coverage():
    announce("config 3: G=8, 131072 tokens, quad r'=8 nrm, coverage 0.95")
    case = make_case(B=2, ctx=131072, n_kv=8, G=8, heavy=0.02, table="perm", seed=3,
                     device=DEV)
    B, MP = 2, case.max_pages
    assert MP == 8192
    st = build_quad_state(case, rank=8, v_bits=8, combine="nrm", coverage=0.95)
    derive_page_params(st, case.seq_lens, B)
    select_pages_quad(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale,
                      derive=False)
    torch.cuda.synchronize()
    mu, mus, _, Vs, sg, _ = st.layer_state(0)
    nsh = npi(st.n_sel_hi)
    V = st.reference_V(0)
    for r in range(B):
        n = int(nsh[r])
        idx = case.block_table[r, :n].long()
        bt = np.arange(n, dtype=np.int32)[None]
        ref_h = osc.quad_score(npf(case.q[r:r + 1]), npi(mu[idx]), npf(mus[idx]), npi(V[idx]),
                               npf(Vs[idx]), npf(sg[idx]), bt, np.array([n]),
                               scale=case.scale, page=16, G=8, v_bits=8, max_pages=n,
                               combine="nrm")
        assert rel_close(npf(st.score_h[r, :, :, :n]), ref_h[0], 1) <= 1e-3
        ref = osc.nrm_combine(npf(st.score_h[r:r + 1, :, :, :n]).astype(np.float64),
                              np.array([n]))
        assert rel_close(npf(st.score[r, :, :n]), ref[0], 1) <= 1e-5
    tab, cnt, _ = osel.select(npf(st.score), npi(st.n_pages), nsh, npi(st.b_fix), sink=1,
                              max_pages=MP, mode=1, coverage=0.95, score_kind=1)
    assert np.array_equal(npi(st.page_table), tab) and np.array_equal(npi(st.page_cnt), cnt)
    _decode_check(case, st, range(B))


@pytest.mark.parametrize("boost", ["sigma", "keynorm"])
def test_config4_memv_64_steps(boost):
    """boost "sigma" is the literal +2 sigma generator (the 0.95 nucleus keeps ~93 % of the
    pages, far more than the hot buffer); "keynorm" boosts in key-norm units (~5 %)."""
    announce(f"config 4: mem-v 32768 tokens, hot 10%, 64 steps, boost={boost}")
    B, n_kv, G = 4, 8, 4
    case = make_case(B=B, ctx=32768, n_kv=n_kv, G=G, heavy=0.05, table="perm", seed=4,
                     device=DEV, boost=boost)
    MP = case.max_pages
    st = build_quad_state(case, rank=8, v_bits=8, combine="nrm", coverage=0.95)
    NB = case.kv_cache.shape[0]
    slots = (B * MP) // 10
    tier = Tier(num_layers=1, num_blocks=NB, n_kv=n_kv, page=16, d=128, hot_slots=slots,
                max_reqs=B, max_pages=MP, device=DEV, v_blocks=4)
    tier.flush_layer(0, case.kv_cache[:, 1])
    r5 = tier.residency
    derive_page_params(st, case.seq_lens, B)
    gen = torch.Generator(device=DEV).manual_seed(44)
    hits = sel = 0
    for step in range(64):
        # fresh queries around the case's own (the boosted direction stays meaningful)
        q = (case.q.float() + 0.3 * torch.randn(B, n_kv * G, 128, generator=gen,
                                                device=DEV)).to(torch.bfloat16)
        select_pages_quad(st, 0, q, case.block_table, case.seq_lens, B, case.scale,
                          derive=False)
        if step < 3:
            pre = (npi(r5.page2slot[0]).astype(np.int64), npi(r5.slot2page[0]).astype(np.int64),
                   npi(r5.lru_clock[0]).astype(np.int64), int(r5.clock[0]))
        ref = torch.zeros(B, n_kv * G, 128, dtype=torch.bfloat16, device=DEV)
        sparse_paged_decode_batched(q, case.kv_cache, case.block_table, case.seq_lens, st, ref,
                                    ResidentVSource(case.kv_cache), scale=case.scale)
        out = torch.zeros_like(ref)
        mem_dynamic_decode(q, case.kv_cache, case.block_table, case.seq_lens, st, out, tier, 0,
                           scale=case.scale, fetch="kernel")
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"step {step}"
        cnt = npi(st.page_cnt)
        miss = int(npi(r5.miss_cnt).sum())
        sel += int(cnt.sum())
        hits += int(cnt.sum()) - miss
        if step < 3:
            plan = otier.plan(npi(st.page_table), cnt, npi(case.block_table),
                              npi(case.seq_lens), *pre, page=16)
            assert np.array_equal(npi(r5.page2slot[0]), plan["page2slot"])
            assert np.array_equal(npi(r5.slot2page[0]), plan["slot2page"])
    r5.assert_maps_inverse(0)
    announce(f"config 4 ({boost}): hot-buffer hit rate over 64 steps = {hits / sel:.3f} "
             f"({slots} slots per kv head, {sel / 64 / (B * n_kv):.0f} pages per unit)")
