"""Stage-A selection: derive params, top-b and coverage-nucleus page selection.

Host side of ``amass_derive_params`` / ``amass_topb_select`` / ``amass_coverage_select``
(include/amass_hip.h).  Mirrors the reference entry points
``derive_page_params`` (selection/select.py:48-54), ``topb_select`` (:104-116) and
``select_pages_r8`` (:119-130).

Selection rule per (request, kv-head): the selectable region is [sink, n_sel_hi); sinks,
the recent window and the partial tail are always kept; a region of <= 1 page keeps every
page.  Top-b keeps b = b_fix[r] pages.  When the state carries ``coverage`` (set by the
builder when ``AmassConfig.budget`` is None) the unit keeps the fewest top pages whose
score-derived mass reaches ``coverage`` of the scored mass (sinks count toward it).
``tie_mode`` "index" (default) keeps exactly b pages with ties at the b-th score broken to
the lower page index; "all" is the reference threshold rule (every page >= tau).
"""
from __future__ import annotations

from .._hip import DeriveArgs, SelectArgs, call, current_stream, ptr, require_cuda

TIE_MODES = {"index": 0, "all": 1}


def derive_page_params(st, seq_lens, n_req: int) -> None:
    """Refresh st.{n_pages, n_sel_hi, b_fix} for this decode step (one launch)."""
    if n_req > st.max_reqs:
        raise ValueError(f"n_req {n_req} exceeds max_reqs {st.max_reqs}")
    require_cuda(seq_lens)
    _check_i32(seq_lens, "seq_lens")
    a = DeriveArgs(seq_lens=ptr(seq_lens), n_pages=ptr(st.n_pages), n_sel_hi=ptr(st.n_sel_hi),
                   b_fix=ptr(st.b_fix), budget=float(st.budget), n_req=n_req, page=st.page,
                   window_pages=st.window_pages, sink_pages=st.sink_pages)
    call("amass_derive_params", a, current_stream(seq_lens.device))


def _check_i32(t, name):
    import torch
    if t.dtype != torch.int32 or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous int32 tensor")


def score_kind(st) -> int:
    """Mass semantics of st.score for the nucleus: 1 = already a mass (quad nrm combine
    sum_g exp(S_g - max S_g)), 0 = a log-mass (group max / r8 logsumexp)."""
    return 1 if getattr(st, "combine", "max") == "nrm" and hasattr(st, "quad_V") else 0


def _select(st, n_req: int, *, mode: str = "auto", score_h=None, tile_max=None,
            coverage=None, tie_mode=None) -> None:
    a = select_args(st, n_req, mode=mode, score_h=score_h, tile_max=tile_max,
                    coverage=coverage, tie_mode=tie_mode)
    name = "amass_coverage_select" if a.mode == 1 else "amass_topb_select"
    call(name, a, current_stream(st.score.device))


def select_args(st, n_req: int, *, mode: str = "auto", score_h=None, tile_max=None,
                coverage=None, tie_mode=None) -> SelectArgs:
    """The amass_select_args of this selection (mode 1 = coverage, 0 = top-b)."""
    if n_req > st.max_reqs:
        raise ValueError(f"n_req {n_req} exceeds max_reqs {st.max_reqs}")
    if tile_max is not None and score_h is None:
        raise ValueError("tile_max comes with score_h (the fused nrm combine)")
    if mode == "auto":
        coverage = getattr(st, "coverage", None)
    elif mode == "topb":
        coverage = None
    elif coverage is None:
        raise ValueError("coverage mode needs a coverage value")
    tm = TIE_MODES[tie_mode or getattr(st, "tie_mode", "index")]
    sc, tab = st.score, st.page_table
    require_cuda(sc, tab)
    a = SelectArgs(
        score=ptr(sc), sc_sr=sc.stride(0), sc_sh=sc.stride(1),
        score_h=ptr(score_h),
        sh_sr=score_h.stride(0) if score_h is not None else 0,
        sh_sh=score_h.stride(1) if score_h is not None else 0,
        sh_sg=score_h.stride(2) if score_h is not None else 0,
        tile_max=ptr(tile_max), tm_sr=tile_max.stride(0) if tile_max is not None else 0,
        tm_sh=tile_max.stride(1) if tile_max is not None else 0,
        tm_sg=tile_max.stride(2) if tile_max is not None else 0,
        n_pages=ptr(st.n_pages), n_sel_hi=ptr(st.n_sel_hi), b_fix=ptr(st.b_fix),
        page_table=ptr(tab), pt_sr=tab.stride(0), pt_sh=tab.stride(1),
        page_cnt=ptr(st.page_cnt), pc_sr=st.page_cnt.stride(0),
        n_sel_out=ptr(getattr(st, "n_sel", None)),
        coverage=float(coverage) if coverage is not None else 1.0,
        n_req=n_req, n_kv=st.n_kv, G=st.G, max_pages=st.max_pages,
        sink_pages=st.sink_pages, mode=1 if coverage is not None else 0, tie_mode=tm,
        score_kind=score_kind(st))
    return a


def topb_select(st, n_req: int, *, tie_mode=None) -> None:
    """Write st.page_table / st.page_cnt from st.score with the static per-request
    budget st.b_fix (derive_page_params must have run this step)."""
    _select(st, n_req, mode="topb", tie_mode=tie_mode)


def coverage_select(st, n_req: int, coverage: float, *, tie_mode=None) -> None:
    """Per-(request, kv-head) coverage nucleus over st.score (see module doc)."""
    _select(st, n_req, mode="coverage", coverage=coverage, tie_mode=tie_mode)


def select_pages(st, n_req: int, *, score_h=None, tile_max=None) -> None:
    """Top-b or coverage selection per the state's configuration (``st.coverage``);
    with ``score_h`` the nrm GQA combine runs fused in the same launch (and writes
    st.score).  ``tile_max``: the per-tile per-head maxima the score launch that wrote
    ``score_h`` produced (st.score_tmax); without it the combine takes the maxima with
    its own pass over score_h."""
    _select(st, n_req, mode="auto", score_h=score_h, tile_max=tile_max)


def select_pages_r8(st, layer: int, q, block_table, seq_lens, n_req: int, scale: float,
                    *, derive: bool = True) -> None:
    """One-call Stage A (r8 score mode): (derive) + r8_score + selection."""
    from .score import r8_score
    if derive:
        derive_page_params(st, seq_lens, n_req)
    r8_score(st, layer, q, block_table, seq_lens, n_req, scale)
    select_pages(st, n_req)
