"""GPU parity of derive / top-b / coverage selection against the CPU oracle.

Bar: given the same scores, page_table, page_cnt and the chosen count are bit-exact for
both tie rules (lower page index; the reference's keep-all-ties threshold), both nucleus
mass kinds, forced ties (+0.0 / -0.0 included), padded rows, short sequences, b >= S, and
up to 16384 pages (the largest page count the selection accepts).
"""
import numpy as np
import pytest
import torch

import oracle.select as osel
from amass.selection import QuadState, coverage_select, derive_page_params, topb_select
from amass.selection.select import select_pages
from helpers import announce, mass_cut_case, npf, npi

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _state(R, MP, G=4, n_kv=8, budget=0.05, combine="max"):
    st = QuadState(DEV, num_layers=1, num_blocks=4, n_kv=n_kv, G=G, head_dim=128, page=16,
                   max_reqs=R, max_pages=MP, rank=2, budget=budget, combine=combine)
    return st


def _seq_lens(R, MP, gen, special=True):
    sl = torch.randint(16, MP * 16 + 1, (R,), generator=gen).to(torch.int32)
    if special and R >= 4:
        sl[0] = 0            # padded row
        sl[1] = 20           # 2 pages: S <= 1 -> keep all
        sl[2] = MP * 16      # full
        sl[3] = 3 * 16 + 5   # partial tail page
    return sl


def _scores(R, n_kv, MP, gen, ties: bool, kind: int):
    if kind == 1:
        sc = torch.rand(R, n_kv, MP, generator=gen) * 4.0
    else:
        sc = torch.randn(R, n_kv, MP, generator=gen) * 3.0
    if ties:
        sc = torch.round(sc * 4) / 4            # many exact ties
        sc[..., 5::11] = -0.0                   # -0.0 and +0.0 compare equal: one tie class
        sc[..., 9::13] = 0.0
    return sc


def _run(st, R, mode, tie, kind, cov, gen, ties, MP, sc=None):
    sl = _seq_lens(R, MP, gen)
    sl_d = sl.to(DEV)
    derive_page_params(st, sl_d, R)
    if sc is None:
        sc = _scores(R, st.n_kv, MP, gen, ties, kind)
    st.score.copy_(sc.to(DEV))
    st.page_table.fill_(-7)
    st.combine = "nrm" if kind == 1 else "max"
    if mode == 0:
        topb_select(st, R, tie_mode=["index", "all"][tie])
    else:
        coverage_select(st, R, cov, tie_mode=["index", "all"][tie])
    torch.cuda.synchronize()
    npg, nsh, bfix = npi(st.n_pages), npi(st.n_sel_hi), npi(st.b_fix)
    ref_tab, ref_cnt, ref_nsel = osel.select(sc.numpy(), npg, nsh, bfix, sink=1, max_pages=MP,
                                             mode=mode, coverage=cov, tie_mode=tie,
                                             score_kind=kind)
    got_tab, got_cnt, got_nsel = npi(st.page_table), npi(st.page_cnt), npi(st.n_sel)
    assert np.array_equal(got_cnt, ref_cnt)
    assert np.array_equal(got_tab, ref_tab)
    if tie == 0:
        assert np.array_equal(got_nsel, ref_nsel)
    return got_cnt


@pytest.mark.parametrize("tie", [0, 1])
@pytest.mark.parametrize("ties", [False, True])
@pytest.mark.parametrize("MP", [37, 1024])
def test_topb(tie, ties, MP):
    announce(f"topb tie={tie} ties={ties} MP={MP}")
    gen = torch.Generator().manual_seed(100 + MP + tie)
    R = 6
    st = _state(R, MP, budget=0.07)
    _run(st, R, 0, tie, 0, 1.0, gen, ties, MP)


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("tie", [0, 1])
@pytest.mark.parametrize("cov", [0.5, 0.95, 1.0])
@pytest.mark.parametrize("ties", [False, True])
def test_coverage(kind, tie, cov, ties):
    announce(f"coverage kind={kind} tie={tie} cov={cov} ties={ties}")
    gen = torch.Generator().manual_seed(int(cov * 100) + 7 * kind + tie)
    R, MP = 6, 700
    st = _state(R, MP)
    _run(st, R, 1, tie, kind, cov, gen, ties, MP)


def test_coverage_cut_on_exact_exp_mass():
    """Coverage by exp mass (the group-max combine) with the cut exactly on the mass of
    the top 11 selectable pages: the GPU keeps what the oracle keeps, so every page mass
    is exp_det's separately rounded value (an FMA anywhere in it moves masses by an ulp
    and the cut by a page)."""
    announce("coverage cut on exact exp mass")
    sc, cov = mass_cut_case(osel.exp_det)
    R, MP = 1, sc.size
    st = _state(R, MP)
    derive_page_params(st, torch.tensor([MP * 16], dtype=torch.int32, device=DEV), R)
    full = np.broadcast_to(sc, (R, st.n_kv, MP)).copy()
    st.score.copy_(torch.from_numpy(full).to(DEV))
    st.combine = "max"
    coverage_select(st, R, cov, tie_mode="index")
    torch.cuda.synchronize()
    ref_tab, ref_cnt, ref_nsel = osel.select(full, npi(st.n_pages), npi(st.n_sel_hi),
                                             npi(st.b_fix), sink=1, max_pages=MP, mode=1,
                                             coverage=cov, tie_mode=0, score_kind=0)
    assert (ref_nsel == 11).all()
    assert np.array_equal(npi(st.n_sel), ref_nsel)
    assert np.array_equal(npi(st.page_cnt), ref_cnt)
    assert np.array_equal(npi(st.page_table), ref_tab)


def test_budget_one_keeps_all():
    announce("budget 1.0")
    gen = torch.Generator().manual_seed(3)
    R, MP = 4, 300
    st = _state(R, MP, budget=1.0)
    cnt = _run(st, R, 0, 0, 0, 1.0, gen, False, MP)
    npg = npi(st.n_pages)
    for r in range(R):
        assert (cnt[r] == max(npg[r], 0)).all()


def test_long_context_8192_pages():
    announce("topb + coverage at MP=8192")
    gen = torch.Generator().manual_seed(9)
    R, MP = 2, 8192
    st = _state(R, MP, G=8, budget=0.02)
    _run(st, R, 0, 0, 0, 1.0, gen, False, MP)
    _run(st, R, 1, 0, 1, 0.95, gen, False, MP)


def test_max_pages_16384():
    """The largest page count the selection accepts (scores staged in LDS)."""
    announce("topb + coverage at MP=16384")
    gen = torch.Generator().manual_seed(10)
    R, MP = 2, 16384
    st = _state(R, MP, G=4, budget=0.02)
    _run(st, R, 0, 0, 0, 1.0, gen, False, MP)
    _run(st, R, 1, 0, 1, 0.95, gen, True, MP)


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("tie", [0, 1])
def test_clustered_scores(mode, tie):
    """Most scores a few ulps apart plus far outliers: the first radix digits put thousands
    of pages in one bin, so the search takes several passes before the chosen bin is small
    enough to be ranked all-pairs; a second cluster of exact ties sits at the cut."""
    announce(f"clustered scores mode={mode} tie={tie}")
    gen = torch.Generator().manual_seed(31 + mode + 2 * tie)
    R, MP = 4, 4096
    st = _state(R, MP, budget=0.3)
    base = torch.full((R, st.n_kv, MP), 0.5)
    ulps = torch.randint(0, 3000, (R, st.n_kv, MP), generator=gen).to(torch.int32)
    sc = (base.view(torch.int32) + ulps).view(torch.float32)
    sc[..., 7::97] = 3.5                              # far outliers above
    sc[..., 11::89] = 1e-30                           # and below
    sc[..., 5::3] = 0.5                               # one large exact tie class
    _run(st, R, mode, tie, 1, 0.9, gen, False, MP, sc=sc)


def test_nrm_fused_into_select():
    """select_pages with score_h: st.score equals the standalone nrm combine and the
    selection equals the oracle's on that score."""
    announce("nrm fused select")
    gen = torch.Generator().manual_seed(21)
    R, MP, G = 5, 513, 4
    st = _state(R, MP, G=G, combine="nrm")
    st.coverage = 0.9
    sl = _seq_lens(R, MP, gen).to(DEV)
    derive_page_params(st, sl, R)
    st.score_h.copy_((torch.randn(R, 8, G, MP, generator=gen) * 2).to(DEV))
    select_pages(st, R, score_h=st.score_h)
    torch.cuda.synchronize()
    got_score = npf(st.score)
    got_tab = npi(st.page_table)
    from amass.selection import nrm_combine
    st.score.fill_(0)
    nrm_combine(st, R)
    torch.cuda.synchronize()
    nsh = npi(st.n_sel_hi)
    ref_score = npf(st.score)
    for r in range(R):
        n = max(int(nsh[r]), 0)
        assert np.array_equal(got_score[r, :, :n], ref_score[r, :, :n])
    ref_tab, _, _ = osel.select(got_score, npi(st.n_pages), nsh, npi(st.b_fix), sink=1,
                                max_pages=MP, mode=1, coverage=0.9, tie_mode=0, score_kind=1)
    assert np.array_equal(got_tab, ref_tab)


def test_config0_known_answer():
    """Config 0: B=1, ctx 4096, fixed 5% budget -> S = 254, b = 13."""
    st = _state(1, 256, budget=0.05)
    derive_page_params(st, torch.tensor([4096], dtype=torch.int32, device=DEV), 1)
    torch.cuda.synchronize()
    assert int(st.n_pages[0]) == 256 and int(st.n_sel_hi[0]) == 255 and int(st.b_fix[0]) == 13


@pytest.mark.parametrize("G,coords", [(4, "none"), (8, "none"), (4, "lse")])
def test_tile_maxima_equal_the_max_pass(G, coords):
    """The score launch's per-16-page-tile per-head maxima (st.score_tmax) are the exact
    maxima of score_h over each tile's scored pages (ragged lengths: partial last tiles),
    and the selection that takes its per-head maxima from them writes the same scores
    and page tables, bit for bit, as the one that takes them with a pass over score_h."""
    announce(f"tile maxima G={G} coords={coords}")
    from amass.bench.synth import build_quad_state, make_case
    from amass.selection.quad_score import clse_score, quad_score_launch
    R = 5
    case = make_case(B=R, ctx=(900, 9000), n_kv=8, G=G, heavy=0.05, table="perm",
                     seed=90 + G, device=DEV)
    st = build_quad_state(case, rank=2, v_bits=8, combine="nrm", coverage=0.95,
                          coords=coords, c_bits=4)
    derive_page_params(st, case.seq_lens, R)
    st.score_tmax.fill_(float("nan"))
    if coords == "lse":
        clse_score(st, 0, case.q, case.block_table, case.seq_lens, R, case.scale)
    else:
        quad_score_launch(st, 0, case.q, case.block_table, R, case.scale)
    torch.cuda.synchronize()
    nsh = npi(st.n_sel_hi)
    sh, tm = npf(st.score_h), npf(st.score_tmax)
    for r in range(R):
        n = int(nsh[r])
        nt = (n + 15) // 16
        pad = np.full((8, G, nt * 16), -np.inf, np.float32)
        pad[..., :n] = sh[r, :, :, :n]
        want = pad.reshape(8, G, nt, 16).max(axis=-1)
        assert np.array_equal(tm[r, :, :, :nt], want), r
    outs = []
    for tmax in (st.score_tmax, None):
        st.score.fill_(0)
        st.page_table.fill_(-7)
        select_pages(st, R, score_h=st.score_h, tile_max=tmax)
        torch.cuda.synchronize()
        outs.append((npf(st.score), npi(st.page_table), npi(st.page_cnt)))
    for r in range(R):
        n = int(nsh[r])
        assert np.array_equal(outs[0][0][r, :, :n].view(np.uint32),
                              outs[1][0][r, :, :n].view(np.uint32))
    assert np.array_equal(outs[0][1], outs[1][1]) and np.array_equal(outs[0][2], outs[1][2])
    tab, cnt, _ = osel.select(outs[0][0], npi(st.n_pages), nsh, npi(st.b_fix), sink=1,
                              max_pages=st.max_pages, mode=1, coverage=0.95, score_kind=1)
    assert np.array_equal(outs[0][1], tab) and np.array_equal(outs[0][2], cnt)


def _tile_max(sh, nsh):
    """Per-16-page-tile per-head maxima of score_h over each row's scored pages (what the
    score launch writes into st.score_tmax)."""
    R, n_kv, G, MP = sh.shape
    nt = (MP + 15) // 16
    pad = np.full((R, n_kv, G, nt * 16), -np.inf, np.float32)
    for r in range(R):
        n = max(int(nsh[r]), 0)
        pad[r, ..., :n] = sh[r, ..., :n]
    return pad.reshape(R, n_kv, G, nt, 16).max(axis=-1)


@pytest.mark.parametrize("case", ["plain", "sink_covers", "full_coverage_tiny", "wide"])
def test_fused_coverage_edges(case):
    """The fused nrm selection (per-head maxima from the tile maxima) at its edge cases:
    rows whose sinks alone cover the need (one selectable page kept), coverage 1.0 over
    masses down to e^-60 (the cut falls on the smallest nonzero 2^-32 mass quantum), and
    wide score spreads.  The page tables equal the oracle's on the GPU's combined
    scores, and the combined scores equal the standalone nrm combine's."""
    announce(f"fused coverage {case}")
    gen = torch.Generator().manual_seed({"plain": 1, "sink_covers": 2,
                                         "full_coverage_tiny": 3, "wide": 4}[case])
    R, MP, G = 6, 1000, 4
    st = _state(R, MP, G=G, combine="nrm")
    cov = {"plain": 0.95, "sink_covers": 0.95, "full_coverage_tiny": 1.0, "wide": 0.99}[case]
    st.coverage = cov
    sl = _seq_lens(R, MP, gen)
    sl[4] = MP * 16
    sl[5] = 700 * 16 + 3
    sl_d = sl.to(DEV)
    derive_page_params(st, sl_d, R)
    sh = torch.randn(R, 8, G, MP, generator=gen) * 2
    if case == "sink_covers":
        sh[:, :, :, 0] = 40.0                      # page 0 (the sink) holds every head's max
    elif case == "full_coverage_tiny":
        sh = -torch.rand(R, 8, G, MP, generator=gen) * 60.0   # exp down to e^-60
        sh[:, :, :, 1] = 0.5                        # one dominant selectable page
    elif case == "wide":
        sh = sh * 12.0
    st.score_h.copy_(sh.to(DEV))
    nsh = npi(st.n_sel_hi)
    st.score_tmax.copy_(torch.from_numpy(_tile_max(sh.numpy(), nsh)).to(DEV))
    st.page_table.fill_(-7)
    select_pages(st, R, score_h=st.score_h, tile_max=st.score_tmax)
    torch.cuda.synchronize()
    got_score, got_tab, got_cnt = npf(st.score), npi(st.page_table), npi(st.page_cnt)
    from amass.selection import nrm_combine
    st.score.fill_(0)
    nrm_combine(st, R)
    torch.cuda.synchronize()
    ref_score = npf(st.score)
    for r in range(R):
        n = max(int(nsh[r]), 0)
        assert np.array_equal(got_score[r, :, :n], ref_score[r, :, :n])
    ref_tab, ref_cnt, _ = osel.select(got_score, npi(st.n_pages), nsh, npi(st.b_fix), sink=1,
                                      max_pages=MP, mode=1, coverage=cov, tie_mode=0,
                                      score_kind=1)
    assert np.array_equal(got_cnt, ref_cnt)
    assert np.array_equal(got_tab, ref_tab)
