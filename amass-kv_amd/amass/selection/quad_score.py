"""Quad page score (Stage A.1, quad mode) -- host side of ``amass_quad_score``.

Same contract as the reference ``quad_score`` (selection/quad_score.py:110-139) and
``select_pages_quad`` (:142-153): writes ``st.score`` (R, n_kv, MP) fp32 over the scored
region [0, n_sel_hi); combine="nrm" first writes the per-head scores ``st.score_h`` and
then the per-head-normalised mass sum_g exp(S_g - max_p S_g) into ``st.score``.
``select_pages_quad`` folds that nrm combine into the selection launch instead of a
separate kernel (one less launch and one less pass over score_h); the score launch also
writes per-16-page-tile per-head maxima (``st.score_tmax``), so the selection reads
score_h once.
"""
from __future__ import annotations

import math

import torch

from .._hip import (ClseScoreArgs, NrmArgs, QuadScoreArgs, call, call_select_attend,
                    current_stream, ptr, require_cuda)
from .score import check_rec_span
from .select import derive_page_params, select_args, select_pages

# The per-unit pipeline (amass_quad_select_attend): the rows it serves and the most
# workgroups per unit.  select_then_attend's route, measured on MI355X against the
# separate score / select / decode launches (graphs of 10 steps, 8 kv heads, contexts of
# 4K-32K tokens, uniform and ragged batches, the device's balanced plan): with the attend
# in the launch it is faster at batches of 1-64 requests while each unit keeps <= ~55
# pages (at a single request only up to ~32), and slower from ~100 kept pages on (one
# workgroup attends what the decode's split layout spreads over many); without the
# attend it gains only at <= 16 units (B <= 2) with rows of <= 1024 pages, and is within
# +-4 us either way elsewhere.
UNIT_MAX_PAGES = 2048
UNIT_MAX_WGS = 16
UNIT_ATTEND_MAX_PAGES = 64      # kept-page bound up to which the launch attends ...
UNIT_ATTEND_FEW_UNITS = 16      # ... at this many units or more,
UNIT_ATTEND_MAX_PAGES_FEW = 32  # ... and up to which below it
UNIT_ROUTE_MAX_UNITS = 16       # without the attend: units ...
UNIT_ROUTE_MAX_PAGES = 1024     # ... and row width up to which it is taken
UNIT_MAX_UNITS_PER_CU = 2       # the largest batch measured: 512 units on 256 CUs

_CUS = {}


def _num_cus(device) -> int:
    idx = torch.device(device).index or 0
    if idx not in _CUS:
        _CUS[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _CUS[idx]


def _tile_max(st):
    """The state's per-tile per-head maxima buffer (nrm states), or None."""
    return getattr(st, "score_tmax", None) if st.combine == "nrm" else None


def _tile_max_fields(tm) -> dict:
    return dict(tile_max=ptr(tm), tm_sr=tm.stride(0) if tm is not None else 0,
                tm_sh=tm.stride(1) if tm is not None else 0,
                tm_sg=tm.stride(2) if tm is not None else 0)


def _quad_args(st, layer, q, block_table, n_req, scale, comb_out=None) -> QuadScoreArgs:
    rec = st.quad_rec[layer]
    require_cuda(q, block_table, rec)
    if q.dtype != torch.bfloat16 or q.stride(2) != 1:
        raise ValueError("q must be bf16 (T, H, d) with unit stride on d")
    if block_table.dtype != torch.int32 or block_table.stride(1) != 1:
        raise ValueError("block_table must be int32 with unit column stride")
    if block_table.shape[1] < st.max_pages - st.window_pages:
        raise ValueError("block_table narrower than the scored page range")
    if rec.stride(1) != 1 or rec.shape[1] != st.n_kv * st.rec_bytes:
        raise ValueError("quad_rec must hold each block's records contiguously")
    check_rec_span(rec)
    if getattr(st, "coords", "none") != "none":
        raise ValueError("a CLSE state (coords='lse') is scored by clse_score")
    nrm = st.combine == "nrm"
    sh, tm = st.score_h, _tile_max(st)
    return QuadScoreArgs(
        q=ptr(q), q_st=q.stride(0), q_hs=q.stride(1),
        rec=ptr(rec), rec_sb=rec.stride(0),
        block_table=ptr(block_table), bt_st=block_table.stride(0),
        n_sel_hi=ptr(st.n_sel_hi),
        score=ptr(st.score), sc_sr=st.score.stride(0), sc_sh=st.score.stride(1),
        score_h=ptr(sh) if nrm else None,
        sh_sr=sh.stride(0) if nrm else 0, sh_sh=sh.stride(1) if nrm else 0,
        sh_sg=sh.stride(2) if nrm else 0,
        **_tile_max_fields(tm),
        comb_out=ptr(comb_out), scale=float(scale),
        n_req=n_req, n_kv=st.n_kv, G=st.G, d=st.d, page=st.page, rank=st.r,
        v_bits=st.v_bits, max_pages=st.max_pages, combine=1 if nrm else 0)


def quad_score_launch(st, layer: int, q, block_table, n_req: int, scale: float,
                      comb_out=None) -> None:
    """The score kernel alone (combine="nrm": st.score_h only)."""
    if n_req > st.max_reqs:
        raise ValueError(f"n_req {n_req} exceeds max_reqs {st.max_reqs}")
    a = _quad_args(st, layer, q, block_table, n_req, scale, comb_out)
    call("amass_quad_score", a, current_stream(q.device))


def nrm_combine(st, n_req: int) -> None:
    """score[p] = sum_g exp(score_h[g, p] - max_p score_h[g, p]) over [0, n_sel_hi)."""
    sh, sc = st.score_h, st.score
    a = NrmArgs(score_h=ptr(sh), sh_sr=sh.stride(0), sh_sh=sh.stride(1), sh_sg=sh.stride(2),
                score=ptr(sc), sc_sr=sc.stride(0), sc_sh=sc.stride(1),
                n_sel_hi=ptr(st.n_sel_hi), n_req=n_req, n_kv=st.n_kv, G=st.G,
                max_pages=st.max_pages)
    call("amass_nrm_combine", a, current_stream(sc.device))


def quad_score(st, layer: int, q, block_table, seq_lens, n_req: int, scale: float) -> None:
    """Stage A.1: write st.score for the scored region (st.n_sel_hi must be current)."""
    quad_score_launch(st, layer, q, block_table, n_req, scale)
    if st.combine == "nrm":
        nrm_combine(st, n_req)


def select_pages_quad(st, layer: int, q, block_table, seq_lens, n_req: int, scale: float,
                      *, derive: bool = True) -> None:
    """One-call Stage A (quad mode): (derive) + score + selection -> st.page_table /
    st.page_cnt.  Two launches (three with derive)."""
    if derive:
        derive_page_params(st, seq_lens, n_req)
    quad_score_launch(st, layer, q, block_table, n_req, scale)
    nrm = st.combine == "nrm"
    select_pages(st, n_req, score_h=st.score_h if nrm else None,
                 tile_max=_tile_max(st) if nrm else None)


def clse_score(st, layer: int, q, block_table, seq_lens, n_req: int, scale: float,
               comb_out=None) -> None:
    """Stage-A.1 (CLSE mode, reference selection/quad_score.py:373-393): combine="max"
    writes st.score (R, n_kv, MP); combine="nrm" writes the per-head st.score_h, which the
    selection launch then combines (select_pages_clse)."""
    if n_req > st.max_reqs:
        raise ValueError(f"n_req {n_req} exceeds max_reqs {st.max_reqs}")
    if getattr(st, "coords", "none") != "lse":
        raise ValueError("clse_score needs a QuadState built with coords='lse'")
    rec = st.quad_rec[layer]
    require_cuda(q, block_table, seq_lens, rec)
    if q.dtype != torch.bfloat16 or q.stride(2) != 1:
        raise ValueError("q must be bf16 (T, H, d) with unit stride on d")
    if block_table.dtype != torch.int32 or block_table.stride(1) != 1:
        raise ValueError("block_table must be int32 with unit column stride")
    if seq_lens.dtype != torch.int32:
        raise ValueError("seq_lens must be int32")
    if rec.stride(1) != 1 or rec.shape[1] != st.n_kv * st.rec_bytes:
        raise ValueError("quad_rec must hold each block's records contiguously")
    check_rec_span(rec)
    nrm = st.combine == "nrm"
    sh = st.score_h
    a = ClseScoreArgs(
        q=ptr(q), q_st=q.stride(0), q_hs=q.stride(1), rec=ptr(rec), rec_sb=rec.stride(0),
        block_table=ptr(block_table), bt_st=block_table.stride(0), seq_lens=ptr(seq_lens),
        n_sel_hi=ptr(st.n_sel_hi),
        score=ptr(st.score), sc_sr=st.score.stride(0), sc_sh=st.score.stride(1),
        score_h=ptr(sh) if nrm else None,
        sh_sr=sh.stride(0) if nrm else 0, sh_sh=sh.stride(1) if nrm else 0,
        sh_sg=sh.stride(2) if nrm else 0,
        **_tile_max_fields(_tile_max(st)),
        comb_out=ptr(comb_out), scale=float(scale), n_req=n_req, n_kv=st.n_kv, G=st.G,
        d=st.d, page=st.page, rank=st.r, v_bits=st.v_bits, c_bits=st.c_bits,
        max_pages=st.max_pages, combine=1 if nrm else 0)
    call("amass_clse_score", a, current_stream(q.device))


def select_pages_clse(st, layer: int, q, block_table, seq_lens, n_req: int, scale: float,
                      *, derive: bool = True) -> None:
    """One-call Stage A (CLSE mode, reference selection/quad_score.py:396-404): (derive)
    + clse_score + selection (the nrm combine fused into it for combine="nrm")."""
    if derive:
        derive_page_params(st, seq_lens, n_req)
    clse_score(st, layer, q, block_table, seq_lens, n_req, scale)
    nrm = st.combine == "nrm"
    select_pages(st, n_req, score_h=st.score_h if nrm else None,
                 tile_max=_tile_max(st) if nrm else None)


def unit_step_supported(st) -> bool:
    """Whether amass_quad_select_attend serves this state: a quad nrm state (score_h and
    per-tile maxima), r'=8 int8 summaries, G <= 8, rows of <= 2048 pages."""
    return (getattr(st, "coords", "none") == "none" and st.combine == "nrm"
            and st.r == 8 and st.v_bits == 8 and st.G <= 8
            and st.max_pages <= UNIT_MAX_PAGES and _tile_max(st) is not None)


def kept_pages_bound(st):
    """An upper bound of any unit's page count that holds without reading the device, or
    None: top-b with the index tie rule keeps b_fix = ceil(budget * selectable) <=
    ceil(budget * max_pages) selectable pages plus the sinks, the recent window and the
    partial tail page."""
    if getattr(st, "coverage", None) is not None or getattr(st, "tie_mode", "index") != "index":
        return None       # coverage: data-dependent; the threshold rule keeps every tie
    return math.ceil(st.budget * st.max_pages) + st.sink_pages + st.window_pages + 1


def unit_route(st, n_req: int, device, resident: bool = True):
    """(workgroups per unit, attend in the launch) of the per-unit pipeline for this
    batch, or None when the separate launches are the faster route.  The workgroups per
    unit are the device's balanced plan (0: each workgroup about one CU's share of the
    batch's tiles, so the long rows of a ragged batch take more), or for one request a
    count from the row width.  The launch attends when
    top-b bounds every unit's kept pages by UNIT_ATTEND_MAX_PAGES (UNIT_ATTEND_MAX_PAGES_FEW
    below UNIT_ATTEND_FEW_UNITS units) and V is resident (``resident``); without the
    attend the route is taken for at most UNIT_ROUTE_MAX_UNITS units with rows of at most
    UNIT_ROUTE_MAX_PAGES pages."""
    if not unit_step_supported(st) or n_req < 1:
        return None
    units = n_req * st.n_kv
    cus = _num_cus(device)
    if units > UNIT_MAX_UNITS_PER_CU * cus:
        return None
    # one request cannot be ragged: its count from the row width (a tile per wave at
    # least), without the plan's prologue
    ns = 0 if n_req > 1 else max(1, min(UNIT_MAX_WGS, cus // units,
                                        ((st.max_pages + 15) // 16 + 7) // 8))
    bound = kept_pages_bound(st)
    limit = (UNIT_ATTEND_MAX_PAGES if units >= UNIT_ATTEND_FEW_UNITS
             else UNIT_ATTEND_MAX_PAGES_FEW)
    if resident and bound is not None and bound <= limit:
        return ns, True
    if units <= UNIT_ROUTE_MAX_UNITS and st.max_pages <= UNIT_ROUTE_MAX_PAGES:
        return ns, False
    return None


def select_attend_quad(st, layer: int, q, block_table, seq_lens, n_req: int, scale: float,
                       *, kv_cache=None, out=None, vsource=None, derive: bool = False,
                       wgs_per_unit: int = 1) -> None:
    """Stage A of one layer in one launch (amass_quad_select_attend): the quad score into
    st.score_h / st.score_tmax, the nrm combine into st.score and the top-b or coverage
    selection into st.page_table / st.page_cnt -- the outputs of select_pages_quad, bit
    for bit -- with one workgroup per (request, kv head).  With ``out`` (and ``kv_cache``,
    ``vsource``: resident V) the same workgroup then attends the kept pages into out, as
    sparse_paged_decode_batched(path="fused") would.  ``wgs_per_unit`` workgroups score
    each unit, or with 0 as many as the device's balanced plan gives each request (the
    last of a unit's workgroups to finish selects, counted in st.unit_tickets)."""
    if not unit_step_supported(st):
        raise ValueError("amass_quad_select_attend serves quad nrm states with r'=8 int8 "
                         f"summaries, G <= 8 and <= {UNIT_MAX_PAGES} pages per row")
    if not 0 <= wgs_per_unit <= UNIT_MAX_WGS:
        raise ValueError(f"wgs_per_unit must be 0 (balanced) or 1..{UNIT_MAX_WGS}")
    if n_req > st.max_reqs:
        raise ValueError(f"n_req {n_req} exceeds max_reqs {st.max_reqs}")
    if derive:
        derive_page_params(st, seq_lens, n_req)
    qa = _quad_args(st, layer, q, block_table, n_req, scale)
    sa = select_args(st, n_req, score_h=st.score_h, tile_max=_tile_max(st))
    da = None
    if out is not None:
        from ..attention.decode import _decode_args, _split_kv
        if vsource is None or vsource.SRC_ID != 0:
            raise ValueError("the in-launch attend reads resident V (a ResidentVSource)")
        k, _ = _split_kv(kv_cache)
        da = _decode_args(q, k, vsource, block_table, seq_lens, st, out, scale, n_req,
                          dense=False, path="fused")
    tickets = ptr(st.unit_tickets) if wgs_per_unit != 1 else None
    call_select_attend(qa, sa, da, sa.mode, tickets, wgs_per_unit, current_stream(q.device))


def select_then_attend(st, layer: int, q, kv_cache, block_table, seq_lens, n_req: int,
                       scale: float, out, vsource) -> None:
    """One layer's score + select + attend (quad states): through the per-unit pipeline
    where unit_route finds it the faster route -- in one launch when it also attends,
    else with the decode after it -- otherwise select_pages_quad then
    sparse_paged_decode_batched.  The outputs are the same either way, bit for bit."""
    from ..attention.decode import sparse_paged_decode_batched
    route = unit_route(st, n_req, q.device, resident=vsource.SRC_ID == 0)
    if route is not None:
        ns, attend = route
        if attend:
            select_attend_quad(st, layer, q, block_table, seq_lens, n_req, scale,
                               kv_cache=kv_cache, out=out, vsource=vsource, wgs_per_unit=ns)
            return
        select_attend_quad(st, layer, q, block_table, seq_lens, n_req, scale, wgs_per_unit=ns)
    else:
        select_pages_quad(st, layer, q, block_table, seq_lens, n_req, scale, derive=False)
    sparse_paged_decode_batched(q, kv_cache, block_table, seq_lens, st, out, vsource,
                                scale=scale)
