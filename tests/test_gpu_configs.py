"""Parity at the BASELINE configurations' real shapes (full context lengths and head
geometry; batch reduced so the CPU oracle finishes in seconds, except config 1).

config 1: the headline shape at its full batch -- B = 32, 16384-token contexts (1024
          pages), G = 4, quad r'=8 int8, nrm, coverage 0.95, permuted pool; the GPU runs
          all 32 requests (so every score workgroup walks several tiles), the oracle
          checks the int32 sums and the scores of four requests over their own blocks,
          the page tables of all 32 on the GPU's scores, and the decode of four requests;
          properties at the full batch: graph replay == eager, every unit's kept mass
          reaches its need, page_cnt >= b + sink + window.  Also the CLSE score with the
          reference's defaults (r'=2, int4 V and coordinates) at the same shape;
config 2: r8 score, 6 ragged sequences spanning 2048..65536 tokens, fixed 5 % budget,
          random pool block tables -> r8 int32 sums exact, scores 1e-3, page sets exact,
          decode 2e-2 / 1e-2; and the benched full batch (64 sequences): scores of three
          requests, all page tables, top-b properties, decode, graph replay == eager;
config 3: 70B GQA shape (G = 8), 131072-token contexts (8192 pages), 2 % heavy pages,
          quad r'=8 nrm, coverage 0.95 -> scores 1e-3, page sets exact, decode; and the
          benched full batch (B = 8) with the same checks plus the coverage properties
          and graph replay == eager;
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
from amass.bench.synth import build_quad_state, build_r8_state, config_case, make_case
from amass.selection import derive_page_params, select_pages_clse, select_pages_quad
from amass.selection.quad_score import clse_score, quad_score_launch
from amass.tier import Tier, mem_dynamic_decode
from helpers import announce, npf, npi, rel_err

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


def _row_blocks(case, r, n):
    """Oracle inputs restricted to request r's own first n blocks (the oracle then works on
    a (n, ...) slab and an identity block table)."""
    blk = npi(case.block_table[r, :n]).astype(np.int64)
    return torch.from_numpy(blk).to(DEV), np.arange(n, dtype=np.int32)[None]


def _graph_replay_equals_eager(step, outs, replays=3):
    """Capture `step` in one HIP graph; every replay (outputs poisoned before it, eager
    work and a synchronisation in between) must equal the eager result bit for bit."""
    step()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for i in range(replays):
        for o in outs:
            o.view(torch.uint8).fill_(0xA5)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o.view(torch.uint8), e.view(torch.uint8)), f"replay {i}"


def _coverage_properties(st, sink=1, window=1, coverage=0.95):
    """Every unit keeps its sinks and window, at least one selectable page, and selectable
    pages whose 2^-32 fixed-point masses (score_kind 1: the nrm scores are masses) reach
    ceil(coverage * total) - sink mass; dropping the lightest kept page falls short."""
    sc, tab, cnt = npf(st.score), npi(st.page_table), npi(st.page_cnt)
    nsh = npi(st.n_sel_hi)
    for r in range(sc.shape[0]):
        n = int(nsh[r])
        for kh in range(sc.shape[1]):
            c = int(cnt[r, kh])
            assert c >= 1 + sink + window, (r, kh, c)
            pages = tab[r, kh, :c]
            assert np.all(np.diff(pages) > 0) and np.all(tab[r, kh, c:] == -1)
            w = osel.mass_q(sc[r, kh, :n], 0.0, 1).astype(np.int64)
            need = int(np.ceil(coverage * float(int(w.sum())))) - int(w[:sink].sum())
            chosen = pages[(pages >= sink) & (pages < n)]
            kept = int(w[chosen].sum())
            assert kept >= need, (r, kh, kept, need)
            if chosen.size > 1 and need > 0:
                assert kept - int(w[chosen].min()) < need, (r, kh)


@pytest.mark.parametrize("boost", ["sigma", "keynorm"])
def test_config1_b32_16k_coverage(boost):
    """The headline configuration at its full batch (quad_score.py:35-107, nrm
    :276-315, the per-(request, kv-head) nucleus of _selection_bridge.py:117-133,
    decode.py:128-241)."""
    announce(f"config 1: B=32, 16384 tokens, quad r'=8 int8 nrm, coverage 0.95, boost={boost}")
    case = config_case(1, seed=1, device=DEV, boost=boost)
    B, MP, G = 32, case.max_pages, 4
    assert case.q.shape[0] == B and MP == 1024
    st = build_quad_state(case, rank=8, v_bits=8, combine="nrm", coverage=0.95)
    derive_page_params(st, case.seq_lens, B)
    nsh = npi(st.n_sel_hi)
    assert np.all(nsh == 1023)
    # the exact int32 contractions over the multi-tile walk (the comb_out instance walks
    # the same tiles), then the production step overwrites score_h
    comb = torch.zeros(B, 8, MP, G, 9, dtype=torch.int32, device=DEV)
    quad_score_launch(st, 0, case.q, case.block_table, B, case.scale, comb_out=comb)
    out = torch.zeros(B, 32, 128, dtype=torch.bfloat16, device=DEV)
    vsrc = ResidentVSource(case.kv_cache)

    def step():
        select_pages_quad(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale,
                          derive=False)
        sparse_paged_decode_batched(case.q, case.kv_cache, case.block_table, case.seq_lens,
                                    st, out, vsrc, scale=case.scale)

    step()
    torch.cuda.synchronize()
    mu, mus, _, Vs, sg, _ = st.layer_state(0)
    V = st.reference_V(0)
    sh = npf(st.score_h)
    rows = [0, 9, 22, 31]
    for r in rows:
        idx, bt = _row_blocks(case, r, 1023)
        o = dict(q=npf(case.q[r:r + 1]), mu=npi(mu[idx]), mu_scale=npf(mus[idx]),
                 V=npi(V[idx]), V_scale=npf(Vs[idx]), sig2=npf(sg[idx]), block_table=bt,
                 n_sel_hi=np.array([1023]))
        ref_comb = osc.quad_comb(o["q"], o["mu"], o["V"], bt, o["n_sel_hi"], G=G, v_bits=8,
                                 max_pages=1023)
        assert np.array_equal(npi(comb[r:r + 1, :, :1023]).astype(np.int64), ref_comb), r
        kw = dict(scale=case.scale, page=16, G=G, v_bits=8, max_pages=1023, combine="nrm")
        ref_f = osc.quad_score(**o, **kw, q_mode="float")
        ref_l = osc.quad_score(**o, **kw, q_mode="limbs")
        assert rel_err(sh[r, :, :, :1023], ref_f[0]) <= 1e-3, r
        assert rel_err(sh[r, :, :, :1023], ref_l[0]) <= 2e-5, r
    ref_n = osc.nrm_combine(sh.astype(np.float64), nsh)
    assert rel_err(npf(st.score)[:, :, :1023], ref_n[:, :, :1023]) <= 1e-5
    # page tables of all 32 requests from the GPU's own scores
    tab, cnt, _ = osel.select(npf(st.score), npi(st.n_pages), nsh, npi(st.b_fix), sink=1,
                              max_pages=MP, mode=1, coverage=0.95, score_kind=1)
    assert np.array_equal(npi(st.page_table), tab) and np.array_equal(npi(st.page_cnt), cnt)
    _coverage_properties(st)
    frac = float(cnt.sum()) / (B * 8 * MP)
    announce(f"config 1 ({boost}): selected fraction {frac:.4f}")
    if boost == "keynorm":
        assert frac < 0.2
    _decode_check(case, st, rows)
    score_eager = st.score[:, :, :1023].clone()
    _graph_replay_equals_eager(step, [out, st.page_table, st.page_cnt])
    assert torch.equal(st.score[:, :, :1023], score_eager)


@pytest.mark.parametrize("boost", ["sigma", "keynorm"])
def test_config1_clse_reference_defaults(boost):
    """The CLSE score with the reference's defaults (cfg:69-82: r'=2, int4 V, int4
    per-token coordinates, nrm) at the config-1 shape: the CLSE tile walk
    (quad_score.py:156-393) over 32 x 1023 pages."""
    announce(f"config 1 shape, CLSE r'=2 int4/int4 nrm coverage 0.95, boost={boost}")
    case = config_case(1, seed=1, device=DEV, boost=boost)
    B, MP, G = 32, case.max_pages, 4
    st = build_quad_state(case, rank=2, v_bits=4, combine="nrm", coverage=0.95,
                          coords="lse", c_bits=4, c_grain="token")
    derive_page_params(st, case.seq_lens, B)
    comb = torch.zeros(B, 8, MP, G, 3, dtype=torch.int32, device=DEV)
    clse_score(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale, comb_out=comb)
    select_pages_clse(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale,
                      derive=False)
    torch.cuda.synchronize()
    nsh = npi(st.n_sel_hi)
    mu, mus, _, Vs, _sg, _ = st.layer_state(0)
    V, c, cs, res = st.reference_V(0), st.quad_c[0], st.c_scale[0], st.quad_resid[0]
    sh = npf(st.score_h)
    rows = [0, 13, 31]
    for r in rows:
        idx, bt = _row_blocks(case, r, 1023)
        q = npf(case.q[r:r + 1])
        ref_comb = osc.quad_comb(q, npi(mu[idx]), npi(V[idx]), bt, np.array([1023]), G=G,
                                 v_bits=4, max_pages=1023)
        assert np.array_equal(npi(comb[r:r + 1, :, :1023]).astype(np.int64), ref_comb), r
        ref = osc.clse_score(q, npi(mu[idx]), npf(mus[idx]), npi(V[idx]), npf(Vs[idx]),
                             npi(c[idx]), npf(cs[idx]), npf(res[idx]), bt,
                             npi(case.seq_lens[r:r + 1]), np.array([1023]), scale=case.scale,
                             page=16, G=G, v_bits=4, c_bits=4, max_pages=1023,
                             combine="nrm")
        assert rel_err(sh[r, :, :, :1023], ref[0]) <= 1e-3, r
    tab, cnt, _ = osel.select(npf(st.score), npi(st.n_pages), nsh, npi(st.b_fix), sink=1,
                              max_pages=MP, mode=1, coverage=0.95, score_kind=1)
    assert np.array_equal(npi(st.page_table), tab) and np.array_equal(npi(st.page_cnt), cnt)
    _coverage_properties(st)
    _decode_check(case, st, [0, 31])


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
        assert rel_err(npf(st.score[r, :, :n]), ref[0]) <= 1e-3
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
        assert rel_err(npf(st.score_h[r, :, :, :n]), ref_h[0]) <= 1e-3
        ref = osc.nrm_combine(npf(st.score_h[r:r + 1, :, :, :n]).astype(np.float64),
                              np.array([n]))
        assert rel_err(npf(st.score[r, :, :n]), ref[0]) <= 1e-5
    tab, cnt, _ = osel.select(npf(st.score), npi(st.n_pages), nsh, npi(st.b_fix), sink=1,
                              max_pages=MP, mode=1, coverage=0.95, score_kind=1)
    assert np.array_equal(npi(st.page_table), tab) and np.array_equal(npi(st.page_cnt), cnt)
    _decode_check(case, st, range(B))


def _topb_properties(st, sink=1, window=1):
    """Top-b with the index tie rule: every unit keeps its sinks and window and exactly b
    selectable pages, ascending with -1 padding, and no dropped selectable page scores
    above a kept one (ties at the cut go to the lower page index)."""
    sc, tab, cnt = npf(st.score), npi(st.page_table), npi(st.page_cnt)
    nsh, npg, bfix = npi(st.n_sel_hi), npi(st.n_pages), npi(st.b_fix)
    for r in range(sc.shape[0]):
        n, S = int(nsh[r]), int(nsh[r]) - sink
        if S <= 1:
            continue
        b = min(max(int(bfix[r]), 1), S)
        for kh in range(sc.shape[1]):
            c = int(cnt[r, kh])
            assert c == b + sink + (int(npg[r]) - n), (r, kh, c, b)
            pages = tab[r, kh, :c]
            assert np.all(np.diff(pages) > 0) and np.all(tab[r, kh, c:] == -1)
            sel = pages[(pages >= sink) & (pages < n)]
            rest = np.setdiff1d(np.arange(sink, n), sel)
            if rest.size:
                lo_kept = sc[r, kh, sel].min()
                assert sc[r, kh, rest].max() <= lo_kept, (r, kh)
                tied = rest[sc[r, kh, rest] == lo_kept]
                assert tied.size == 0 or tied.min() > sel[sc[r, kh, sel] == lo_kept].max()


def test_config2_full_batch():
    """Config 2 at its full batch, the benched workload: 64 ragged sequences (2928..65104
    tokens), r8 r=8 int8, top-b 5 %.  Scores of three requests against the oracle over
    their own blocks, the page tables of all 64 on the GPU's scores, the top-b properties,
    the decode of two requests, and four graph replays of the step equal to eager."""
    announce("config 2 full batch: B=64 ragged, r8, top-b 5%")
    case = config_case(2, seed=2, device=DEV)
    B, MP = case.q.shape[0], case.max_pages
    assert B == 64
    st = build_r8_state(case, rank=8, vk_bits=8, c_bits=8, budget=0.05)
    from amass.selection import select_pages_r8
    out = torch.zeros(B, 32, 128, dtype=torch.bfloat16, device=DEV)
    vsrc = ResidentVSource(case.kv_cache)
    derive_page_params(st, case.seq_lens, B)

    def step():
        select_pages_r8(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale,
                        derive=False)
        sparse_paged_decode_batched(case.q, case.kv_cache, case.block_table, case.seq_lens,
                                    st, out, vsrc, scale=case.scale)

    step()
    torch.cuda.synchronize()
    mu, mus, _, Vks, c, cs, _ = st.layer_state(0)
    Vk = st.reference_Vk(0)
    nsh = npi(st.n_sel_hi)
    lens = npi(case.seq_lens)
    rows = [int(np.argmin(lens)), int(np.argmax(lens)), 17]
    for r in rows:
        n = int(nsh[r])
        idx, bt = _row_blocks(case, r, n)
        ref = osc.r8_score(npf(case.q[r:r + 1]), npi(mu[idx]), npf(mus[idx]), npi(Vk[idx]),
                           npf(Vks[idx]), npi(c[idx]), npf(cs[idx]), bt, lens[r:r + 1],
                           np.array([n]), scale=case.scale, page=16, G=4, vk_bits=8,
                           c_bits=8, max_pages=n)
        assert rel_err(npf(st.score[r, :, :n]), ref[0]) <= 1e-3, r
    tab, cnt, _ = osel.select(npf(st.score), npi(st.n_pages), nsh, npi(st.b_fix), sink=1,
                              max_pages=MP, mode=0)
    assert np.array_equal(npi(st.page_table), tab) and np.array_equal(npi(st.page_cnt), cnt)
    _topb_properties(st)
    _decode_check(case, st, rows[:2])
    _graph_replay_equals_eager(step, [out, st.page_table, st.page_cnt])


def test_config3_full_batch():
    """Config 3 at its full batch, the benched workload: B = 8, 131072-token contexts
    (8192 pages), G = 8, quad r'=8 int8 nrm, coverage 0.95 -- the nrm pre-pass and the
    1024-thread selection.  Per-head scores of one request against the oracle, the page
    tables of all 8 on the GPU's scores, the coverage properties, the decode of two
    requests, and four graph replays of the step equal to eager."""
    announce("config 3 full batch: B=8, 131072 tokens, G=8, coverage 0.95")
    case = config_case(3, seed=3, device=DEV)
    B, MP = case.q.shape[0], case.max_pages
    assert B == 8 and MP == 8192
    st = build_quad_state(case, rank=8, v_bits=8, combine="nrm", coverage=0.95)
    out = torch.zeros(B, 64, 128, dtype=torch.bfloat16, device=DEV)
    vsrc = ResidentVSource(case.kv_cache)
    derive_page_params(st, case.seq_lens, B)

    def step():
        select_pages_quad(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale,
                          derive=False)
        sparse_paged_decode_batched(case.q, case.kv_cache, case.block_table, case.seq_lens,
                                    st, out, vsrc, scale=case.scale)

    step()
    torch.cuda.synchronize()
    mu, mus, _, Vs, sg, _ = st.layer_state(0)
    V = st.reference_V(0)
    nsh = npi(st.n_sel_hi)
    r, n = 5, int(nsh[5])
    idx, bt = _row_blocks(case, r, n)
    ref_h = osc.quad_score(npf(case.q[r:r + 1]), npi(mu[idx]), npf(mus[idx]), npi(V[idx]),
                           npf(Vs[idx]), npf(sg[idx]), bt, np.array([n]), scale=case.scale,
                           page=16, G=8, v_bits=8, max_pages=n, combine="nrm")
    assert rel_err(npf(st.score_h[r, :, :, :n]), ref_h[0]) <= 1e-3
    ref_n = osc.nrm_combine(npf(st.score_h).astype(np.float64), nsh)
    assert rel_err(npf(st.score)[:, :, :n], ref_n[:, :, :n]) <= 1e-5
    tab, cnt, _ = osel.select(npf(st.score), npi(st.n_pages), nsh, npi(st.b_fix), sink=1,
                              max_pages=MP, mode=1, coverage=0.95, score_kind=1)
    assert np.array_equal(npi(st.page_table), tab) and np.array_equal(npi(st.page_cnt), cnt)
    _coverage_properties(st)
    _decode_check(case, st, [0, 7])
    _graph_replay_equals_eager(step, [out, st.page_table, st.page_cnt])


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
