"""Property-based GPU parity: scores, selection, sparse decode, the tier plan and the mem-v
write path over generated cases.

hypothesis draws the batch shape, the sequence lengths, the score pattern and the
selection parameters (derandomized, so every run checks the same examples); each example
runs the HIP path and compares with the oracle under the same bars as the fixed-case
tests: page_table / page_cnt / chosen count bit-exact for the selection, outputs within
2e-2 absolute / 1e-2 relative of the fp64 attention for the decode.

The score kernels (quad, r8, CLSE) run over generated record layouts (rank, V / Vk bits, c
bits and c-scale grain), GQA groups, kv-head counts (workgroups of 1, 2, 4 and 8 heads
and two head groups), combines, batch sizes and lengths from one token up; their int32
contractions are bit-exact against int64 brute force and their scores within
1e-3 * max(|ref|, 1) of the fp64 oracle (quad: also 2e-5 of the limb oracle).

Score patterns target the selection's radix search: i.i.d. normal, a small value pool
(many exact ties), a run of keys a few ulps apart (every digit of the 32-bit key decides,
bins of more than 64 candidates), +0.0 / -0.0 mixtures (one tie class), and magnitudes
over 60 decades.  Page counts span every thread layout of the selection (1..8 pages per
thread of 512, 8 of 1024, 32 of 512) and the decode's whole / split / fused layouts with
ragged and empty units and NaN-poisoned slots past each sequence's end.  The nrm selection
from per-head scores and per-tile maxima (the fused staging and the pre-pass) runs over
generated GQA groups, lengths and head-score patterns (normal, a value pool with ties,
masses over ~100 nats, a sink page holding every head's maximum): its combined scores are
bit-identical to the standalone combine and its page tables equal the oracle's.  The
per-unit pipeline (score, selection and attend in one launch) runs over generated
batches (kv-head counts, GQA groups, sink and window widths, lengths from padded rows to
2048 pages, both selection modes and tie rules, with and without the attend) and equals
the separate launches bit for bit.
"""
import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as hs

import oracle.decode as odec
import oracle.score as osc
import oracle.select as osel
import oracle.tier as otier
from amass.attention import ensure_stage_b_buffers
from amass.attention.decode import ResidentVSource, sparse_paged_decode_batched
from amass.bench.synth import build_quad_state, build_r8_state, make_case
from amass.selection import (QuadState, coverage_select, derive_page_params, r8_score,
                             topb_select)
from amass.selection.quad_score import clse_score, quad_score_launch
from amass.tier import Tier
from helpers import announce, case_to, npf, npi, rel_err, to_device

pytestmark = pytest.mark.gpu
DEV = "cuda"
PROPS = settings(max_examples=25, deadline=None, derandomize=True, database=None,
                 suppress_health_check=list(HealthCheck))

PATTERNS = ("normal", "ties", "ulps", "zeros", "wide")
# row widths of every thread layout of the selection: 1, 2, 4 and 8 pages per thread of
# 512, 8 per thread of 1024, 32 per thread of 512
MPS = (2, 63, 513, 1024, 2047, 4096, 8192, 8193, 16384)


def _scores(rng, shape, pattern):
    if pattern == "normal":
        return (rng.standard_normal(shape) * 3).astype(np.float32)
    if pattern == "ties":
        pool = np.array([-2.0, 0.5, 0.5, 3.0], np.float32)
        return pool[rng.integers(0, pool.size, shape)]
    if pattern == "ulps":
        base = np.float32(rng.uniform(0.1, 4.0))
        bits = base.view(np.int32) + rng.integers(0, 300, shape).astype(np.int32)
        return bits.view(np.float32)
    if pattern == "zeros":
        pool = np.array([0.0, -0.0, 0.0, 1.5, -1.0], np.float32)
        return pool[rng.integers(0, pool.size, shape)]
    mag = 10.0 ** rng.uniform(-30, 30, shape)
    return (np.sign(rng.standard_normal(shape)) * mag).astype(np.float32)


@hs.composite
def selection_cases(draw, MP):
    R = draw(hs.integers(1, 4))
    n_kv = draw(hs.sampled_from([1, 2, 8]))
    lens = draw(hs.lists(hs.integers(0, MP * 16), min_size=R, max_size=R))
    return dict(R=R, n_kv=n_kv, MP=MP, lens=lens,
                pattern=draw(hs.sampled_from(PATTERNS)),
                seed=draw(hs.integers(0, 2 ** 31 - 1)),
                mode=draw(hs.integers(0, 1)), tie=draw(hs.integers(0, 1)),
                kind=draw(hs.integers(0, 1)),
                cov=draw(hs.floats(0.01, 1.0)), budget=draw(hs.floats(0.001, 1.0)))


@pytest.mark.parametrize("MP", MPS)
def test_selection_matches_oracle(MP):
    @PROPS
    @given(c=selection_cases(MP))
    def prop(c):
        _selection_example(c)
    prop()


def _selection_example(c):
    announce(f"selection property case {c}")
    R, n_kv, MP = c["R"], c["n_kv"], c["MP"]
    rng = np.random.default_rng(c["seed"])
    sc = _scores(rng, (R, n_kv, MP), c["pattern"])
    st = QuadState(DEV, num_layers=1, num_blocks=4, n_kv=n_kv, G=4, head_dim=128, page=16,
                   max_reqs=R, max_pages=MP, rank=2, budget=c["budget"],
                   combine="nrm" if c["kind"] == 1 else "max")
    derive_page_params(st, torch.tensor(c["lens"], dtype=torch.int32, device=DEV), R)
    st.score.copy_(torch.from_numpy(sc).to(DEV))
    st.page_table.fill_(-7)
    tie = ["index", "all"][c["tie"]]
    if c["mode"] == 0:
        topb_select(st, R, tie_mode=tie)
    else:
        coverage_select(st, R, c["cov"], tie_mode=tie)
    torch.cuda.synchronize()
    npg, nsh, bfix = npi(st.n_pages), npi(st.n_sel_hi), npi(st.b_fix)
    ref_npg, ref_nsh, ref_b = osel.derive(c["lens"], c["budget"], 16, 1, 1)
    assert np.array_equal(npg, ref_npg) and np.array_equal(nsh, ref_nsh)
    assert np.array_equal(bfix, ref_b)
    tab, cnt, nsel = osel.select(sc, npg, nsh, bfix, sink=1, max_pages=MP, mode=c["mode"],
                                 coverage=c["cov"], tie_mode=c["tie"], score_kind=c["kind"])
    assert np.array_equal(npi(st.page_cnt), cnt)
    assert np.array_equal(npi(st.page_table), tab)
    if c["tie"] == 0:
        assert np.array_equal(npi(st.n_sel), nsel)


# the nrm selection from per-head scores and per-tile maxima: the fused staging (PPT G <=
# 64) and the multi-workgroup pre-pass (8192 pages at G = 8, or any G beyond 4096 pages)
NRM_MPS = (2, 63, 513, 1024, 2047, 4096, 8192)
NRM_PATTERNS = ("normal", "ties", "spread", "sink")


def _head_scores(rng, shape, pattern):
    if pattern == "normal":
        return (rng.standard_normal(shape) * 3).astype(np.float32)
    if pattern == "ties":
        pool = np.array([-6.0, -1.0, 0.0, 0.0, 2.5], np.float32)
        return pool[rng.integers(0, pool.size, shape)]
    if pattern == "spread":                    # exp() masses over ~100 nats
        return (rng.standard_normal(shape) * 25).astype(np.float32)
    x = (rng.standard_normal(shape) * 2).astype(np.float32)
    x[..., 0] = 30.0                            # the sink page holds every head's maximum
    return x


@hs.composite
def nrm_selection_cases(draw, MP):
    R = draw(hs.integers(1, 3))
    return dict(R=R, n_kv=draw(hs.sampled_from([1, 2, 8])), G=draw(hs.sampled_from([1, 2, 4, 8])),
                MP=MP, lens=draw(hs.lists(hs.integers(0, MP * 16), min_size=R, max_size=R)),
                pattern=draw(hs.sampled_from(NRM_PATTERNS)),
                seed=draw(hs.integers(0, 2 ** 31 - 1)), mode=draw(hs.integers(0, 1)),
                tie=draw(hs.integers(0, 1)), cov=draw(hs.floats(0.01, 1.0)),
                budget=draw(hs.floats(0.001, 1.0)))


@pytest.mark.parametrize("MP", NRM_MPS)
def test_nrm_selection_from_tile_maxima_matches_oracle(MP):
    """select_pages with score_h and the per-tile maxima (the path the quad and CLSE
    steps take): the combined scores equal the standalone two-pass nrm combine bit for
    bit, and the page tables and counts equal the oracle's on those scores."""
    @PROPS
    @given(c=nrm_selection_cases(MP))
    def prop(c):
        _nrm_selection_example(c)
    prop()


def _nrm_selection_example(c):
    announce(f"nrm selection property case {c}")
    from amass.selection import nrm_combine
    from amass.selection.select import _select
    R, n_kv, G, MP = c["R"], c["n_kv"], c["G"], c["MP"]
    rng = np.random.default_rng(c["seed"])
    sh = _head_scores(rng, (R, n_kv, G, MP), c["pattern"])
    st = QuadState(DEV, num_layers=1, num_blocks=4, n_kv=n_kv, G=G, head_dim=128, page=16,
                   max_reqs=R, max_pages=MP, rank=2, budget=c["budget"], combine="nrm")
    derive_page_params(st, torch.tensor(c["lens"], dtype=torch.int32, device=DEV), R)
    nsh = npi(st.n_sel_hi)
    nt = (MP + 15) // 16
    pad = np.full((R, n_kv, G, nt * 16), -np.inf, np.float32)
    for r in range(R):
        n = max(int(nsh[r]), 0)
        pad[r, ..., :n] = sh[r, ..., :n]
    st.score_h.copy_(torch.from_numpy(sh).to(DEV))
    st.score_tmax.copy_(torch.from_numpy(pad.reshape(R, n_kv, G, nt, 16).max(-1)).to(DEV))
    st.page_table.fill_(-7)
    tie = ["index", "all"][c["tie"]]
    _select(st, R, mode="coverage" if c["mode"] else "topb", coverage=c["cov"],
            score_h=st.score_h, tile_max=st.score_tmax, tie_mode=tie)
    torch.cuda.synchronize()
    got_sc, got_tab, got_cnt = npf(st.score), npi(st.page_table), npi(st.page_cnt)
    st.score.fill_(0)
    nrm_combine(st, R)
    torch.cuda.synchronize()
    ref_sc = npf(st.score)
    for r in range(R):
        n = max(int(nsh[r]), 0)
        assert np.array_equal(got_sc[r, :, :n].view(np.uint32), ref_sc[r, :, :n].view(np.uint32))
    tab, cnt, _ = osel.select(got_sc, npi(st.n_pages), nsh, npi(st.b_fix), sink=1,
                              max_pages=MP, mode=c["mode"], coverage=c["cov"],
                              tie_mode=c["tie"], score_kind=1)
    assert np.array_equal(got_cnt, cnt)
    assert np.array_equal(got_tab, tab)


@hs.composite
def decode_cases(draw, path):
    n_kv, G = draw(hs.sampled_from([(1, 8), (2, 4), (8, 1), (8, 4), (8, 8)]))
    return dict(B=draw(hs.integers(1, 5)), n_kv=n_kv, G=G,
                hi=draw(hs.sampled_from([40, 600, 3000])),
                shape=draw(hs.sampled_from(["sparse", "ragged", "full"])),
                path=path, seed=draw(hs.integers(0, 2 ** 31 - 1)))


@pytest.mark.parametrize("path", ["auto", "split", "fused"])
def test_sparse_decode_matches_oracle(path):
    @PROPS
    @given(c=decode_cases(path))
    def prop(c):
        _decode_example(c)
    prop()


def _decode_example(c):
    announce(f"decode property case {c}")
    B, n_kv, G = c["B"], c["n_kv"], c["G"]
    rng = np.random.default_rng(c["seed"])
    case = make_case(B=B, ctx=(1, c["hi"]), n_kv=n_kv, G=G, heavy=0.0, table="perm",
                     seed=c["seed"] % 100003)
    sl = case.seq_lens - torch.from_numpy(rng.integers(0, 16, B)).to(case.seq_lens.dtype)
    sl = torch.clamp(sl, min=1).to(torch.int32)
    for r in range(B):                          # poison the slots past each sequence's end
        n = int(sl[r])
        last = (n - 1) // 16
        if n - last * 16 < 16:
            case.kv_cache[int(case.block_table[r, last]), :, n - last * 16:] = float("nan")
    case.seq_lens = sl
    MP = case.max_pages
    npg = (npi(sl) + 15) // 16
    tab = np.full((B, n_kv, MP), -1, np.int32)
    cnt = np.zeros((B, n_kv), np.int32)
    for r in range(B):
        for kh in range(n_kv):
            P = int(npg[r])
            if c["shape"] == "full":
                k = P
            elif c["shape"] == "sparse":
                k = int(rng.integers(0, min(P, 4) + 1))
            else:
                k = int(rng.integers(0, P + 1))
            pages = np.sort(rng.choice(P, size=k, replace=False)).astype(np.int32)
            tab[r, kh, :k] = pages
            cnt[r, kh] = k
    q, K, V = npf(case.q), npf(case.kv_cache[:, 0]), npf(case.kv_cache[:, 1])
    ref = odec.attend(q, K, V, npi(case.block_table), npi(sl), tab, cnt, scale=case.scale, G=G)

    class _St:
        pass
    st = _St()
    st.max_reqs, st.n_kv, st.G, st.D = B, n_kv, G, case.d
    st.page_table = torch.from_numpy(tab).to(DEV)
    st.page_cnt = torch.from_numpy(cnt).to(DEV)
    ensure_stage_b_buffers(st, DEV)
    kv = case.kv_cache.to(DEV)
    out = torch.full((B, n_kv * G, case.d), float("nan"), dtype=torch.bfloat16, device=DEV)
    sparse_paged_decode_batched(case.q.to(DEV), kv, case.block_table.to(DEV), sl.to(DEV), st,
                                out, ResidentVSource(kv), scale=case.scale, path=c["path"])
    torch.cuda.synchronize()
    got = npf(out)
    assert np.isfinite(got).all()
    assert np.allclose(got, ref, atol=2e-2, rtol=1e-2), float(np.abs(got - ref).max())


# ---------------------------------------------------------------------------- scores
# Score kernels over generated record layouts, GQA groups, kv-head counts (workgroups of
# 1, 2, 4 and 8 heads, and two head groups), batch sizes and lengths from one token up:
# int32 contractions bit-exact against int64 brute force, scores within 1e-3 * max(|ref|,
# 1) of the fp64 oracle (quad: also 2e-5 of the limb oracle).
SCORE_PROPS = settings(max_examples=30, deadline=None, derandomize=True, database=None,
                       suppress_health_check=list(HealthCheck))


@hs.composite
def score_cases(draw, kind):
    G = draw(hs.integers(1, 8) if kind == "quad" else hs.sampled_from([1, 2, 4, 8]))
    rank = draw(hs.sampled_from({"quad": [2, 4, 8], "r8": [4, 8], "clse": [2, 4, 8]}[kind]))
    c = dict(kind=kind, B=draw(hs.integers(1, 6)), n_kv=draw(hs.sampled_from([1, 2, 4, 8, 16])),
             G=G, rank=rank, v_bits=draw(hs.sampled_from([8, 4])),
             c_bits=draw(hs.sampled_from([8, 4])),
             hi=draw(hs.sampled_from([16, 300, 1500, 4000])),
             combine=draw(hs.sampled_from(["max", "nrm"])),
             seed=draw(hs.integers(0, 100000)))
    c["c_grain"] = draw(hs.sampled_from({"quad": ["token"], "r8": ["page", "page_f32"],
                                         "clse": ["token", "page"]}[kind]))
    return c


def _score_example(c):
    announce(f"score property case {c}")
    kind, B, n_kv, G, rank = c["kind"], c["B"], c["n_kv"], c["G"], c["rank"]
    case = make_case(B=B, ctx=(1, c["hi"]), n_kv=n_kv, G=G, heavy=0.05, table="perm",
                     seed=c["seed"])
    rng = np.random.default_rng(c["seed"])
    case.seq_lens = torch.clamp(case.seq_lens - torch.from_numpy(rng.integers(0, 16, B)).to(
        case.seq_lens.dtype), min=1).to(torch.int32)
    if kind == "r8":
        st = build_r8_state(case, rank=rank, vk_bits=c["v_bits"], c_bits=c["c_bits"],
                            c_grain=c["c_grain"])
    else:
        st = build_quad_state(case, rank=rank, v_bits=c["v_bits"], combine=c["combine"],
                              coords="lse" if kind == "clse" else "none", c_bits=c["c_bits"],
                              c_grain=c["c_grain"], budget=0.05)
    to_device(st, DEV)
    case_to(case, DEV)
    derive_page_params(st, case.seq_lens, B)
    MP = st.max_pages
    comb = torch.zeros(B, n_kv, MP, G, rank + 1, dtype=torch.int32, device=DEV)
    if kind == "quad":
        quad_score_launch(st, 0, case.q, case.block_table, B, case.scale, comb_out=comb)
    elif kind == "r8":
        r8_score(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale, comb_out=comb)
    else:
        clse_score(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale,
                   comb_out=comb)
    torch.cuda.synchronize()
    q, bt, sl, nsh = npf(case.q), npi(case.block_table), npi(case.seq_lens), npi(st.n_sel_hi)
    kw = dict(scale=case.scale, page=16, G=G, max_pages=MP)
    if kind == "r8":
        mu, mus, _, Vks, cc, cs, _ = st.layer_state(0)
        Vk = npi(st.reference_Vk(0))
        ref_comb = osc.r8_comb(q, npi(mu), Vk, bt, nsh, G=G, vk_bits=c["v_bits"], max_pages=MP)
        refs = [(osc.r8_score(q, npi(mu), npf(mus), Vk, npf(Vks), npi(cc), npf(cs), bt, sl,
                              nsh, vk_bits=c["v_bits"], c_bits=c["c_bits"], **kw), 1e-3)]
        got = npf(st.score)
    else:
        mu, mus, _, Vs, sg, _ = st.layer_state(0)
        V = npi(st.reference_V(0))
        ref_comb = osc.quad_comb(q, npi(mu), V, bt, nsh, G=G, v_bits=c["v_bits"], max_pages=MP)
        if kind == "quad":
            o = dict(q=q, mu=npi(mu), mu_scale=npf(mus), V=V, V_scale=npf(Vs), sig2=npf(sg),
                     block_table=bt, n_sel_hi=nsh)
            refs = [(osc.quad_score(**o, **kw, v_bits=c["v_bits"], combine=c["combine"],
                                    q_mode=m), tol) for m, tol in (("float", 1e-3),
                                                                   ("limbs", 2e-5))]
        else:
            refs = [(osc.clse_score(q, npi(mu), npf(mus), V, npf(Vs), npi(st.quad_c[0]),
                                    npf(st.c_scale[0]), npf(st.quad_resid[0]), bt, sl, nsh,
                                    v_bits=c["v_bits"], c_bits=c["c_bits"],
                                    combine=c["combine"], **kw), 1e-3)]
        got = npf(st.score_h if c["combine"] == "nrm" else st.score)
    gc = npi(comb).astype(np.int64)
    for r in range(B):
        n = int(nsh[r])
        assert np.array_equal(gc[r, :, :n], ref_comb[r, :, :n]), f"contractions, request {r}"
        for ref, tol in refs:
            assert rel_err(got[r, ..., :n], ref[r, ..., :n]) <= tol, f"scores, request {r}"


@pytest.mark.parametrize("kind", ["quad", "r8", "clse"])
def test_scores_match_oracle(kind):
    @SCORE_PROPS
    @given(c=score_cases(kind))
    def prop(c):
        _score_example(c)
    prop()


# ---------------------------------------------------------------------------- tier plan
# The mem-v gather plan over generated hot-buffer states and request streams: slot counts
# from 1 to 3000 (more slots than threads per kv head), buffers empty, half full or full
# with LRU clocks spread over 1 .. 5000 steps (the histogram cut up to 255 steps of age,
# the radix sort beyond), several steps of top-b selections of 2 .. 100 % of the pages
# (hits, misses, evictions, overflow), bit-exact against the sequential oracle: maps,
# clocks, miss and victim lists, overflow flag, fetch list as a set.
TIER_PROPS = settings(max_examples=12, deadline=None, derandomize=True, database=None,
                      suppress_health_check=list(HealthCheck))


@hs.composite
def tier_cases(draw, slots):
    return dict(B=draw(hs.integers(1, 5)), n_kv=draw(hs.sampled_from([1, 2, 8])),
                hi=draw(hs.sampled_from([300, 2000, 6000])), slots=slots,
                fill=draw(hs.sampled_from([0.0, 0.5, 1.0])),
                span=draw(hs.sampled_from([1, 40, 255, 256, 5000])),
                fracs=draw(hs.lists(hs.sampled_from([0.02, 0.15, 0.5, 1.0]), min_size=1,
                                    max_size=4)),
                seed=draw(hs.integers(0, 100000)))


def _tier_example(c):
    announce(f"tier property case {c}")
    B, n_kv, slots = c["B"], c["n_kv"], c["slots"]
    case = make_case(B=B, ctx=(16, c["hi"]), n_kv=n_kv, G=4, heavy=0.0, seed=c["seed"])
    NB = case.kv_cache.shape[0]
    tier = Tier(num_layers=1, num_blocks=NB, n_kv=n_kv, page=16, d=128, hot_slots=slots,
                max_reqs=B, max_pages=case.max_pages, device=DEV, v_blocks=4)
    tier.flush_layer(0, case.kv_cache[:, 1])
    r5 = tier.residency
    rng = np.random.default_rng(c["seed"])
    p2s = np.full((n_kv, NB), -1, np.int64)
    s2p = np.full((n_kv, slots), -1, np.int64)
    lru = np.zeros((n_kv, slots), np.int64)
    clock = c["span"] + 10
    for kv in range(n_kv):
        nres = int(min(slots, NB) * c["fill"])
        blks = rng.choice(NB, nres, replace=False)
        sl_ = rng.choice(slots, nres, replace=False)
        p2s[kv, blks] = sl_
        s2p[kv, sl_] = blks
        lru[kv, sl_] = rng.integers(clock - c["span"], clock, nres)
    r5.page2slot[0].copy_(torch.from_numpy(p2s.astype(np.int32)))
    r5.slot2page[0].copy_(torch.from_numpy(s2p.astype(np.int32)))
    r5.lru_clock[0].copy_(torch.from_numpy(lru.astype(np.int32)))
    r5.clock.fill_(clock)
    bt, sl = case.block_table.to(DEV), case.seq_lens.to(DEV)
    MP = case.max_pages
    for frac in c["fracs"]:
        sc = rng.standard_normal((B, n_kv, MP)).astype(np.float32)
        npg, nsh, bfix = osel.derive(npi(case.seq_lens), frac, 16, 1, 1)
        tab, cnt, _ = osel.select(sc, npg, nsh, bfix, sink=1, max_pages=MP, mode=0)
        ref = otier.plan(tab, cnt, npi(case.block_table), npi(case.seq_lens), p2s, s2p, lru,
                         clock, page=16)
        r5.overflow.zero_()
        r5.gather_plan(0, torch.from_numpy(tab).to(DEV), torch.from_numpy(cnt).to(DEV), bt,
                       sl, B)
        torch.cuda.synchronize()
        assert int(r5.clock[0]) == ref["clock"]
        assert np.array_equal(npi(r5.page2slot[0]), ref["page2slot"])
        assert np.array_equal(npi(r5.slot2page[0]), ref["slot2page"])
        assert np.array_equal(npi(r5.lru_clock[0]), ref["lru"])
        assert bool(r5.overflow[0]) == ref["overflow"]
        mc, mp, vs = npi(r5.miss_cnt), npi(r5.miss_pages), npi(r5.victim_slots)
        for r in range(B):
            for kv in range(n_kv):
                m = ref["miss"][r][kv]
                assert mc[r, kv] == len(m)
                assert list(mp[r, kv, :len(m)]) == m
                assert list(vs[r, kv, :len(m)]) == ref["victims"][r][kv]
        n = int(r5.fetch_cnt[0])
        assert set(map(tuple, npi(r5.fetch_list[:n]).tolist())) == ref["fetch"]
        p2s, s2p, lru, clock = ref["page2slot"], ref["slot2page"], ref["lru"], ref["clock"]


@pytest.mark.parametrize("slots", [1, 7, 64, 600, 3000, 6553, 8192])
def test_tier_plan_matches_oracle(slots):
    @TIER_PROPS
    @given(c=tier_cases(slots))
    def prop(c):
        _tier_example(c)
    prop()


# ---------------------------------------------------------------------------- write path
# The mem-v write path over generated schedules: per step, each of three requests appends
# 0 .. 5 tokens (prefill chunks, decode steps and idle steps in any order, pages of 4
# tokens), with or without a block shared by two requests, flush lists of 1, 3 or 64
# entries per step; staging holds every page a schedule can write, so no step exhausts
# it.  After every step the staging map, flush state, token slots, staged and pinned
# pools, pool validity and residency maps equal the oracle's bit for bit.
STAGE_PROPS = settings(max_examples=40, deadline=None, derandomize=True, database=None,
                       suppress_health_check=list(HealthCheck))


@hs.composite
def write_schedules(draw):
    steps = draw(hs.integers(1, 14))
    return dict(shared=draw(hs.booleans()), maxf=draw(hs.sampled_from([1, 3, 64])),
                seed=draw(hs.integers(0, 100000)),
                sched=draw(hs.lists(hs.lists(hs.integers(0, 5), min_size=3, max_size=3),
                                    min_size=steps, max_size=steps)))


@STAGE_PROPS
@given(c=write_schedules())
def test_write_path_matches_oracle_on_generated_schedules(c):
    from test_gpu_stage import _Scenario
    announce(f"write path property case {c}")
    sc = _Scenario(seed=c["seed"], NV=64, maxf=c["maxf"], shared=c["shared"])
    for ql in c["sched"]:
        sc.step(ql)
    sc.stg.assert_free_partition()


# ------------------------------------------------------------------ per-unit pipeline
# amass_quad_select_attend against the separate launches (quad score, selection with the
# fused nrm staging, the decode's one-workgroup-per-unit layout) over generated batches:
# kv-head counts, GQA groups (odd ones included), sink and window widths, lengths from 0
# (padded rows) to 2048 pages, top-b and coverage, both tie rules, both boosts, with and
# without the attend in the launch, 1 to 16 workgroups per unit or the balanced plan.
# Every output bit-identical, the tickets back at zero.
@hs.composite
def unit_cases(draw):
    R = draw(hs.integers(1, 6))
    hi = draw(hs.sampled_from([16, 700, 4096, 16384, 32768]))
    return dict(R=R, n_kv=draw(hs.sampled_from([1, 2, 4, 8])),
                G=draw(hs.sampled_from([1, 2, 3, 4, 8])), hi=hi,
                zero=draw(hs.booleans()), sink=draw(hs.sampled_from([0, 1, 3])),
                window=draw(hs.sampled_from([1, 2])),
                mode=draw(hs.sampled_from(["topb", "coverage"])),
                tie=draw(hs.sampled_from(["index", "all"])),
                budget=draw(hs.floats(0.01, 0.6)), cov=draw(hs.floats(0.3, 1.0)),
                boost=draw(hs.sampled_from(["sigma", "keynorm"])),
                attend=draw(hs.booleans()), wgs=draw(hs.sampled_from([0, 1, 2, 5, 16])),
                seed=draw(hs.integers(0, 100000)))


@PROPS
@given(c=unit_cases())
def test_unit_pipeline_matches_separate_launches(c):
    from test_gpu_unit import _compare
    announce(f"unit pipeline property case {c}")
    case = make_case(B=c["R"], ctx=(1, c["hi"]), n_kv=c["n_kv"], G=c["G"], heavy=0.05,
                     table="perm", boost=c["boost"], seed=c["seed"], device=DEV)
    if c["zero"]:
        case.seq_lens[0] = 0
    kw = dict(coverage=c["cov"]) if c["mode"] == "coverage" else dict(budget=c["budget"])
    st = build_quad_state(case, rank=8, v_bits=8, combine="nrm", sink=c["sink"],
                          window=c["window"], **kw)
    st.tie_mode = c["tie"]
    _compare(case, st, attend=c["attend"], wgs=c["wgs"])
