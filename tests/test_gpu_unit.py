"""The per-unit pipeline (amass_quad_select_attend) against the separate launches.

One workgroup per (request, kv head) runs the quad score, the nrm combine + selection and
(optionally) the attend of the unit; every output must equal what amass_quad_score,
amass_topb_select / amass_coverage_select and amass_sparse_decode write for the same
inputs, bit for bit: score_h and the per-tile maxima over the scored pages, score,
page_table, page_cnt and the attention output (the decode's one-workgroup-per-unit
layout, path "fused", which "auto" also picks for these batches).  Cases: config 0
(B = 1, 4096 tokens, top-b 5 %, the shape the pipeline is for) checked against the CPU
oracle as well; ragged batches over the three row widths (1, 2 and 4 pages per selection
thread: rows of 256, 1024 and 2048 pages), G = 4 and 8, top-b with both tie rules and
coverage; the attend phase under coverage (called explicitly); several workgroups per
unit (the last to finish selects, behind a per-unit ticket that every launch leaves at
zero); graph replay equal to eager; shapes outside its scope refused before anything
runs.
"""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle.decode as odec
import oracle.score as osc
import oracle.select as osel
from amass import _hip
from amass.attention.decode import ResidentVSource, sparse_paged_decode_batched
from amass.bench.synth import build_quad_state, config_case, make_case
from amass.selection import derive_page_params, select_pages_quad
from amass.selection.quad_score import (_quad_args, _tile_max, kept_pages_bound,
                                        select_attend_quad, select_then_attend, unit_route,
                                        unit_step_supported)
from amass.selection.select import select_args
from helpers import announce, npf, npi

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _outputs(st, n_req):
    """The unit outputs that both routes write, restricted to what is defined: score_h
    and score over each request's scored pages, tile maxima over its tiles, the page
    table rows and counts."""
    nsh = npi(st.n_sel_hi)
    sh, sc, tm = npf(st.score_h), npf(st.score), npf(st.score_tmax)
    out = []
    for r in range(n_req):
        n = int(nsh[r])
        out += [sh[r, :, :, :n], sc[r, :, :n], tm[r, :, :, :(n + 15) // 16]]
    return out + [npi(st.page_table[:n_req]), npi(st.page_cnt[:n_req])]


def _poison(st):
    for t in (st.score_h, st.score, st.score_tmax):
        t.fill_(float("nan"))
    st.page_table.fill_(-7)
    st.page_cnt.fill_(-7)


def _equal(a, b):
    for x, y in zip(a, b):
        assert x.shape == y.shape
        assert np.array_equal(x.view(np.uint8), y.view(np.uint8))


def _compare(case, st, *, attend, wgs=1):
    """Separate launches, then the unit pipeline (wgs workgroups per unit), from poisoned
    outputs: bit-identical, and the per-unit tickets back at zero."""
    B = case.q.shape[0]
    H = case.n_kv * case.G
    derive_page_params(st, case.seq_lens, B)
    vs = ResidentVSource(case.kv_cache)
    _poison(st)
    select_pages_quad(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale,
                      derive=False)
    ref_out = torch.full((B, H, 128), float("nan"), dtype=torch.bfloat16, device=DEV)
    sparse_paged_decode_batched(case.q, case.kv_cache, case.block_table, case.seq_lens, st,
                                ref_out, vs, scale=case.scale, path="fused")
    auto_out = torch.full_like(ref_out, float("nan"))
    sparse_paged_decode_batched(case.q, case.kv_cache, case.block_table, case.seq_lens, st,
                                auto_out, vs, scale=case.scale)
    torch.cuda.synchronize()
    ref = _outputs(st, B)
    _poison(st)
    out = torch.full_like(ref_out, float("nan"))
    if attend:
        select_attend_quad(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale,
                           kv_cache=case.kv_cache, out=out, vsource=vs, wgs_per_unit=wgs)
    else:
        select_attend_quad(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale,
                           wgs_per_unit=wgs)
        sparse_paged_decode_batched(case.q, case.kv_cache, case.block_table, case.seq_lens,
                                    st, out, vs, scale=case.scale, path="fused")
    torch.cuda.synchronize()
    assert not st.unit_tickets.any()
    _equal(_outputs(st, B), ref)
    assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16))
    return out, auto_out


def test_config0_one_launch_matches_separate_and_oracle():
    announce("unit pipeline: config 0 (B=1, 4096 tokens, top-b 5 %), attend in-launch")
    case = config_case(0, seed=0, device=DEV)
    st = build_quad_state(case, rank=8, v_bits=8, combine="nrm", budget=0.05)
    assert unit_step_supported(st) and kept_pages_bound(st) <= 32
    assert unit_route(st, 1, DEV) == (2, True)
    out, auto_out = _compare(case, st, attend=True)
    # "auto" picks the same one-workgroup-per-unit layout for this batch
    assert torch.equal(out.view(torch.int16), auto_out.view(torch.int16))
    # and the oracle: scores, page set, output
    nsh = npi(st.n_sel_hi)
    mu, mus, _, Vs, sg, _ = st.layer_state(0)
    ref_h = osc.quad_score(npf(case.q), npi(mu), npf(mus), npi(st.reference_V(0)), npf(Vs),
                           npf(sg), npi(case.block_table), nsh, scale=case.scale, page=16,
                           G=4, v_bits=8, max_pages=st.max_pages, combine="nrm")
    ref_s = osc.nrm_combine(ref_h, nsh)
    n = int(nsh[0])
    sc = npf(st.score)
    assert np.max(np.abs(sc[0, :, :n] - ref_s[0, :, :n]) /
                  np.maximum(np.abs(ref_s[0, :, :n]), 1.0)) <= 1e-3
    tab, cnt, _ = osel.select(sc, npi(st.n_pages), nsh, npi(st.b_fix), sink=1,
                              max_pages=st.max_pages, mode=0)
    assert np.array_equal(npi(st.page_table), tab) and np.array_equal(npi(st.page_cnt), cnt)
    want = odec.attend(npf(case.q), npf(case.kv_cache[:, 0]), npf(case.kv_cache[:, 1]),
                       npi(case.block_table), npi(case.seq_lens), tab, cnt,
                       scale=case.scale, G=4)
    assert np.allclose(npf(out), want, atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("B,hi,G,mode,tie", [
    (3, 4096, 4, "topb", "index"),         # rows of 256 pages: 1 page per thread
    (2, 16384, 8, "topb", "index"),        # 1024 pages: 2 per thread, G = 8
    (4, 32768, 4, "topb", "all"),          # 2048 pages: 4 per thread, threshold ties
    (5, 16384, 4, "coverage", "index"),
    (2, 32768, 8, "coverage", "index"),
])
def test_ragged_batches_match_separate(B, hi, G, mode, tie):
    announce(f"unit pipeline: B={B} ctx<={hi} G={G} {mode} tie={tie}")
    case = make_case(B=B, ctx=(64, hi), n_kv=8, G=G, heavy=0.05, table="perm", seed=B + G,
                     device=DEV)
    kw = dict(coverage=0.95) if mode == "coverage" else dict(budget=0.05)
    st = build_quad_state(case, rank=8, v_bits=8, combine="nrm", **kw)
    st.tie_mode = tie
    assert unit_step_supported(st)
    _compare(case, st, attend=False)
    _compare(case, st, attend=True)


@pytest.mark.parametrize("mode", ["topb", "coverage"])
def test_short_and_padded_rows_match_separate(mode):
    """Rows with no scored page (1-2 pages: n_sel_hi <= 1), keep-all rows (a selectable
    region of one page), a padded row (seq_len 0) and a partial last page, beside rows of
    a few tiles: every output equals the separate launches'."""
    announce(f"unit pipeline: short and padded rows, {mode}")
    case = make_case(B=8, ctx=(1, 600), n_kv=8, G=4, heavy=0.05, table="perm", seed=31,
                     device=DEV)
    sl = case.seq_lens.clone()
    sl[0], sl[1], sl[2], sl[3] = 0, 16, 32, 45
    case.seq_lens.copy_(sl)
    kw = dict(coverage=0.95) if mode == "coverage" else dict(budget=0.3)
    st = build_quad_state(case, rank=8, v_bits=8, combine="nrm", **kw)
    _compare(case, st, attend=False)
    _compare(case, st, attend=True)
    assert int(st.page_cnt[0].max()) == 0          # the padded row keeps nothing


@pytest.mark.parametrize("B,hi,G,mode,tie,wgs", [
    (1, 4096, 4, "topb", "index", 2),      # config 0's shape, two workgroups per unit
    (2, 16384, 4, "coverage", "index", 8),
    (3, 32768, 8, "topb", "all", 16),
    (4, 32768, 4, "coverage", "index", 5),  # tiles not a multiple of the waves
    (1, 4096, 4, "topb", "index", 0),       # the balanced plan: 2 workgroups per unit
    (3, 32768, 8, "coverage", "all", 0),
    (8, 16384, 4, "topb", "index", 0),
    (40, 2048, 4, "coverage", "index", 0),  # 320 units > 256 CUs: one workgroup each
])
def test_multi_workgroup_units_match_separate(B, hi, G, mode, tie, wgs):
    """Several workgroups per unit (the last to finish selects and attends; wgs 0: the
    device's balanced plan): the same bits as the separate launches, the tickets back at
    zero, twice in a row."""
    announce(f"unit pipeline: {wgs} workgroups per unit, B={B} ctx<={hi} G={G} {mode}")
    case = make_case(B=B, ctx=(64, hi), n_kv=8, G=G, heavy=0.05, table="perm", seed=40 + B,
                     device=DEV)
    kw = dict(coverage=0.95) if mode == "coverage" else dict(budget=0.05)
    st = build_quad_state(case, rank=8, v_bits=8, combine="nrm", **kw)
    st.tie_mode = tie
    for attend in (False, True, True):
        _compare(case, st, attend=attend, wgs=wgs)


@pytest.mark.parametrize("B,long_rows,hi,lo,mode", [
    (8, 1, 16384, 1024, "topb"),      # one long row: its units take most workgroups
    (32, 1, 16384, 1024, "coverage"),
    (32, 16, 16384, 1024, "topb"),
    (5, 2, 32768, 0, "coverage"),     # padded rows (length 0) among long ones
])
def test_balanced_plan_ragged_batches(B, long_rows, hi, lo, mode):
    """The balanced plan on ragged batches (long rows among short or empty ones): the same
    bits as the separate launches, with and without the attend, the tickets at zero."""
    announce(f"unit pipeline balanced plan: B={B} {long_rows} x {hi} + {lo} {mode}")
    case = make_case(B=B, ctx=hi, n_kv=8, G=4, heavy=0.05, table="perm", seed=60 + B,
                     device=DEV)
    sl = case.seq_lens.clone()
    sl[long_rows:] = lo
    case.seq_lens = sl
    kw = dict(coverage=0.95) if mode == "coverage" else dict(budget=0.05)
    st = build_quad_state(case, rank=8, v_bits=8, combine="nrm", **kw)
    for attend in (False, True, True):
        _compare(case, st, attend=attend, wgs=0)


@pytest.mark.parametrize("mode", ["topb", "coverage"])
def test_balanced_plan_more_than_64_requests(mode):
    """The balanced plan's walk over more than one wave of requests (100 requests of two
    kv heads: 200 units, below a round, so the device plans): the same bits as the
    separate launches, the tickets at zero."""
    announce(f"unit pipeline balanced plan: 100 requests x 2 kv heads, {mode}")
    case = make_case(B=100, ctx=(64, 8192), n_kv=2, G=4, heavy=0.05, table="perm", seed=77,
                     device=DEV)
    kw = dict(coverage=0.95) if mode == "coverage" else dict(budget=0.05)
    st = build_quad_state(case, rank=8, v_bits=8, combine="nrm", **kw)
    for attend in (False, True):
        _compare(case, st, attend=attend, wgs=0)


def test_runtime_route_and_graph_replay():
    """select_then_attend (the route the backend and the bench take) picks the one-launch
    pipeline for config 0 (two workgroups per unit); its graph replays
    equal the eager result and leave the tickets at zero."""
    announce("unit pipeline: select_then_attend in a HIP graph")
    case = config_case(0, seed=3, device=DEV)
    st = build_quad_state(case, rank=8, v_bits=8, combine="nrm", budget=0.05)
    derive_page_params(st, case.seq_lens, 1)
    vs = ResidentVSource(case.kv_cache)
    out = torch.zeros(1, 32, 128, dtype=torch.bfloat16, device=DEV)

    def step():
        select_then_attend(st, 0, case.q, case.kv_cache, case.block_table, case.seq_lens, 1,
                           case.scale, out, vs)

    step()
    torch.cuda.synchronize()
    n = int(st.n_sel_hi[0])                 # score is written over the scored pages only
    outs = (out, st.page_table, st.page_cnt, st.score[:, :, :n])
    eager = [x.clone() for x in outs]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for i in range(3):
        for x in (out, st.page_table, st.page_cnt, st.score):
            x.view(torch.uint8).fill_(0xA5)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for x, e in zip(outs, eager):
            assert torch.equal(x, e), f"replay {i}"
        assert not st.unit_tickets.any()


def test_out_of_scope_shapes_are_refused():
    announce("unit pipeline: refusals")
    case = make_case(B=1, ctx=2048, n_kv=8, G=4, heavy=0.0, seed=9, device=DEV)
    st = build_quad_state(case, rank=4, v_bits=8, combine="nrm", budget=0.05)
    assert not unit_step_supported(st)
    with pytest.raises(ValueError):
        select_attend_quad(st, 0, case.q, case.block_table, case.seq_lens, 1, case.scale)
    # the library refuses it too, before launching (status -3, unsupported)
    derive_page_params(st, case.seq_lens, 1)
    qa = _quad_args(st, 0, case.q, case.block_table, 1, case.scale)
    sa = select_args(st, 1, score_h=st.score_h, tile_max=_tile_max(st))
    st.page_cnt.fill_(-7)
    lib = _hip.load_library()
    rc = lib.amass_quad_select_attend(C.byref(qa), C.byref(sa), None, 0, None, 1,
                                      C.c_void_p(_hip.current_stream()))
    torch.cuda.synchronize()
    assert rc == -3 and int(st.page_cnt.min()) == -7
