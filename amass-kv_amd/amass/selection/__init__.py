"""Stage A -- decode-time page selection (MI355X HIP kernels behind the reference API).

Per decode step, per layer (reference surface: selection/__init__.py:26-59):

  quad_build_refresh(st, layer, K, block_table, seq_lens, n_req)   # page finalise (off path)
  derive_page_params(st, seq_lens, n_req)                          # once per step
  select_pages_quad(st, layer, q, block_table, seq_lens, n_req, scale)
      = quad score -> st.score_h / st.score, then top-b or coverage -> st.page_table
  select_pages_r8(...) likewise with the r8 score.
"""
from __future__ import annotations

from .build import r8_build_bulk, r8_build_delta, r8_build_refresh, r8_build_tail
from .quad_build import (quad_build_bulk, quad_build_delta, quad_build_refresh,
                         quad_build_tail)
from .quad_score import (clse_score, nrm_combine, quad_score, select_attend_quad,
                         select_pages_clse, select_pages_quad, select_then_attend)
from .quad_state import QuadState
from .score import r8_score
from .select import (coverage_select, derive_page_params, select_pages, select_pages_r8,
                     topb_select)
from .state import TAGW, R8State

__all__ = [
    "R8State", "TAGW", "r8_build_refresh", "r8_build_tail", "r8_build_bulk",
    "r8_build_delta", "derive_page_params", "r8_score", "topb_select", "coverage_select",
    "select_pages", "select_pages_r8", "QuadState", "quad_build_refresh",
    "quad_build_tail", "quad_build_bulk", "quad_build_delta", "quad_score",
    "nrm_combine", "select_pages_quad", "clse_score", "select_pages_clse",
    "select_attend_quad", "select_then_attend",
]
