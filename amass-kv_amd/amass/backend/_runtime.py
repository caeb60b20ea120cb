"""Backend runtime: the one AmassConfig, the Stage-A / Stage-B dispatch, layer lookup.

The reference keeps these singletons and adapters in ``backend/_runtime.py:1-303``:
register() stores the config, the metadata builder owns the per-layer state, and the
attention impl calls the select / decode functions with the layer-index-free signature
``(q, kv_cache, block_table, seq_lens, st, n_req, scale, cfg)``.  On this build there is
one implementation of every kernel (libamass_hip.so); nothing here falls back to
another kernel family -- an unsupported configuration is refused up front and the
impl then leaves the step to the stock vLLM attention, as the reference does for every
path it does not handle (``backend/attn.py:45-59``).  mem-v runs the tier in shadow, as
the reference's backend does: the builder runs the tier's per-step lifecycle, the impl
writes each layer's V into the staging pool and attends with the stock attention while
the engine cache still holds V.
"""
from __future__ import annotations

from typing import Optional

from ..config import AmassConfig

_config: Optional[AmassConfig] = None

PAGE = 16          # page size the kernels are built for (reference: cfg page = 16)
HEAD_DIM = 128     # head dim the kernels are built for


def set_config(cfg: Optional[AmassConfig]) -> None:
    global _config
    _config = cfg


def get_config() -> Optional[AmassConfig]:
    return _config


# What the kernels of libamass_hip.so accept (their entry points return a geometry or
# unsupported status for anything else, so a layer outside these limits must keep the
# stock attention instead of failing inside forward).
SCORE_RANKS = {"quad": (2, 4, 8), "clse": (2, 4, 8), "r8": (4, 8)}
SCORE_GROUPS = {"quad": tuple(range(1, 9)), "clse": (1, 2, 4, 8), "r8": (1, 2, 4, 8)}
MAX_HEADS_PER_GROUP = 8   # kv heads of one score workgroup: n_kv <= 8 or a multiple of 8
MAX_SELECT_PAGES = 16384  # pages per request the selection kernel holds in LDS


def unsupported_reason(cfg: Optional[AmassConfig], *, head_size: int, block_size: int,
                       G: int, n_kv: Optional[int] = None,
                       max_pages: Optional[int] = None) -> Optional[str]:
    """Why this build's decode path does not serve a layer (None = it does): the limits
    the score, selection and decode kernels check (head size, page size, the GQA group
    and rank sets per score, the kv-head grouping, the pages one selection holds)."""
    if cfg is None:
        return "no AmassConfig registered"
    if cfg.offload_k:
        return "variant 'mem-kv': K offload is not part of this build"
    if head_size != HEAD_DIM or block_size != PAGE:
        return f"head_size {head_size} / block_size {block_size} (built for 128 / 16)"
    score = cfg.score
    groups = SCORE_GROUPS.get(score)
    if groups is None:
        return f"score {score!r} is not built"
    if G not in groups:
        return f"GQA group {G} with score {score!r} (built for {groups})"
    rank = cfg.r8_rank if score == "r8" else cfg.quad_rank
    if rank not in SCORE_RANKS[score]:
        return f"rank {rank} with score {score!r} (built for {SCORE_RANKS[score]})"
    if n_kv is not None and (n_kv < 1 or (n_kv > MAX_HEADS_PER_GROUP
                                          and n_kv % MAX_HEADS_PER_GROUP)):
        return f"{n_kv} kv heads (built for <= 8 or a multiple of 8)"
    if max_pages is not None and max_pages > MAX_SELECT_PAGES:
        return (f"{max_pages} pages per sequence (the selection holds at most "
                f"{MAX_SELECT_PAGES}, i.e. {MAX_SELECT_PAGES * PAGE} tokens)")
    return None


def make_state(cfg: AmassConfig, device, *, num_layers: int, num_blocks: int, n_kv: int,
               G: int, max_reqs: int, max_pages: int):
    """The persistent Stage-A state for ``cfg.score`` (reference builder.py:161-205)."""
    from ..attention.decode import ensure_stage_b_buffers
    from ..selection import QuadState, R8State
    budget = cfg.budget if cfg.budget is not None else 0.1
    common = dict(num_layers=num_layers, num_blocks=num_blocks, n_kv=n_kv, G=G,
                  head_dim=HEAD_DIM, page=PAGE, max_reqs=max_reqs, max_pages=max_pages,
                  budget=budget, sink_pages=cfg.sink_pages, window_pages=cfg.window_pages)
    if cfg.score in ("quad", "clse"):
        clse = cfg.score == "clse"
        st = QuadState(device, rank=cfg.quad_rank, v_bits=cfg.quad_v_bits,
                       combine=cfg.quad_combine, coords="lse" if clse else "none",
                       c_bits=cfg.quad_c_bits, c_grain=cfg.quad_c_grain, **common)
    else:
        st = R8State(device, rank=cfg.r8_rank, **common)
    # budget None -> the per-(request, kv-head) coverage nucleus; else fixed top-b
    st.coverage = cfg.coverage if cfg.budget is None else None
    st.scale = None
    ensure_stage_b_buffers(st, device)
    return st


def make_tier(cfg: AmassConfig, device, *, num_layers: int, num_blocks: int, n_kv: int,
              max_reqs: int, max_pages: int, max_tokens: int, dtype):
    """The mem-v tier (pinned V pool, hot buffer, staging) of reference builder.py:245-288."""
    from ..tier import Tier
    return Tier.from_config(cfg, num_layers=num_layers, num_blocks=num_blocks, n_kv=n_kv,
                            page=PAGE, d=HEAD_DIM, max_reqs=max_reqs, max_pages=max_pages,
                            max_tokens=max_tokens, dtype=dtype, device=device)


def layer_index(st, kv_cache) -> int:
    """Physical layer of ``kv_cache`` (the builder keys its data_ptr at allocation)."""
    layer_of = getattr(st, "_layer_of", None)
    if layer_of is None:
        raise RuntimeError("amass: state has no layer map (the builder did not bind it)")
    lidx = layer_of.get(kv_cache.data_ptr())
    if lidx is None:
        raise RuntimeError(f"amass: kv_cache {kv_cache.data_ptr():#x} is not a layer the "
                           "builder bound")
    return lidx


def select(q, kv_cache, block_table, seq_lens, st, n_req: int, scale: float,
           cfg: AmassConfig) -> None:
    """Stage A for one layer: score + (nrm) + top-b / coverage -> st.page_table,
    st.page_cnt.  ``derive=False``: the builder derived this step's page params."""
    from ..selection import QuadState, select_pages_clse, select_pages_quad, select_pages_r8
    lidx = layer_index(st, kv_cache)
    if isinstance(st, QuadState) and st.coords == "lse":
        select_pages_clse(st, lidx, q, block_table, seq_lens, n_req, scale, derive=False)
    elif isinstance(st, QuadState):
        select_pages_quad(st, lidx, q, block_table, seq_lens, n_req, scale, derive=False)
    else:
        select_pages_r8(st, lidx, q, block_table, seq_lens, n_req, scale, derive=False)


def select_and_decode(q, kv_cache, block_table, seq_lens, st, out, vsource, n_req: int,
                      scale: float, cfg: AmassConfig) -> None:
    """Stage A + Stage B of one layer (backend/attn.py:66-74): quad states take
    select_then_attend (one launch for short rows, else score + select then the decode),
    the r8 and CLSE states select() then decode_dispatch()."""
    from ..selection import QuadState, select_then_attend
    if isinstance(st, QuadState) and st.coords != "lse":
        select_then_attend(st, layer_index(st, kv_cache), q, kv_cache, block_table, seq_lens,
                           n_req, scale, out, vsource)
        return
    select(q, kv_cache, block_table, seq_lens, st, n_req, scale, cfg)
    decode_dispatch(q, kv_cache, block_table, seq_lens, st, out, vsource, scale, cfg)


def decode_dispatch(q, kv_cache, block_table, seq_lens, st, out, vsource, scale: float,
                    cfg: AmassConfig) -> None:
    """Stage B: sparse paged decode over st.page_table (split-K or fused, chosen by the
    library from the batch shape)."""
    from ..attention.decode import sparse_paged_decode_batched
    sparse_paged_decode_batched(q, kv_cache, block_table, seq_lens, st, out, vsource,
                                scale=scale)
