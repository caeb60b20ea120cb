"""Stage B -- sparse paged decode attention (host side of ``amass_sparse_decode``).

Same contract as the reference ``sparse_paged_decode_batched`` (attention/decode.py:
247-304): consumes st.page_table / st.page_cnt and writes rows [0, n_req) of ``out``
(T, H, d) in place, reading K from the resident paged cache and V through an injected
V source (the fast / mem-v seam, attention/decode.py:44-95).  No allocation, no host
sync.  A latency-bound batch (few selected pages) gets one workgroup per (request, kv
head) whose waves split the head's pages and merge in LDS; otherwise each request gets S
workgroups with one wave per kv head (split s attends pages s, s + S, ...) that write
split-K partials for a second launch, the LSE merge.  ``path``: "auto" (layout and S chosen on the device so the
workgroups fill the GPU), "split" (every request split, at least pps_min pages per
split, S below the partial capacity), "fused" (every request one workgroup per head).
``dense_paged_decode`` attends every page of every request (the dense baseline).
"""
from __future__ import annotations

from typing import Protocol, Tuple

import torch

from .._hip import DecodeArgs, call, current_stream, ptr, require_cuda

SPLIT = 128          # split-K width (partial buffers are (R, n_kv, SPLIT, G[, d]))
PATHS = {"auto": 0, "split": 1, "fused": 2}


class VSource(Protocol):
    SRC_ID: int

    def args(self) -> Tuple[torch.Tensor, int, int, int]:
        ...


def _split_kv(kv_cache: torch.Tensor):
    """(K, V) views (num_blocks, page, n_kv, d) of a (2, NB, ...) or (NB, 2, ...) cache;
    V is None for a K-only (NB, 1, ...) cache."""
    if kv_cache.shape[0] == 2:
        return kv_cache[0], kv_cache[1]
    if kv_cache.shape[1] == 1:
        return kv_cache.select(1, 0), None
    return kv_cache.select(1, 0), kv_cache.select(1, 1)


class ResidentVSource:
    """V from the resident engine V half (source id 0)."""

    SRC_ID = 0

    def __init__(self, kv_cache: torch.Tensor):
        _, v = _split_kv(kv_cache)
        if v is None:
            raise ValueError("ResidentVSource needs a resident V half; this cache is "
                             "K-only -- use a tier V source")
        self._v = v

    def args(self):
        v = self._v
        return v, v.stride(0), v.stride(1), v.stride(2)

    def tier_fields(self) -> dict:
        return {}


def ensure_stage_b_buffers(st, device, split: int = SPLIT) -> None:
    """Allocate the split-K partials on the state once (outside any graph capture):
    m_part / l_part (R, n_kv, split, G), acc_part (R, n_kv, split, G, D) fp32."""
    if getattr(st, "m_part", None) is not None:
        st.split = getattr(st, "split", split)
        return
    R, n_kv, G, D = st.max_reqs, st.n_kv, st.G, getattr(st, "D", getattr(st, "d", 128))
    st.split = split
    st.m_part = torch.empty(R, n_kv, split, G, device=device, dtype=torch.float32)
    st.l_part = torch.empty(R, n_kv, split, G, device=device, dtype=torch.float32)
    st.acc_part = torch.empty(R, n_kv, split, G, D, device=device, dtype=torch.float32)


def _pps_min(n_req: int) -> int:
    """Minimum pages per split (one wave per head): fewer, fatter splits once the batch
    fills the GPU."""
    return 4 if n_req == 1 else 8


def _decode_args(q, k, vsource, block_table, seq_lens, st, out, scale, n_req, *, dense,
                 path, table=None, cnt=None) -> DecodeArgs:
    require_cuda(q, k, block_table, seq_lens, out)
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or out.dtype != torch.bfloat16:
        raise ValueError("q, K and out must be bf16")
    if q.stride(2) != 1 or k.stride(3) != 1 or out.stride(2) != 1:
        raise ValueError("q / K / out need unit stride on the head dim")
    _, page, n_kv, d = k.shape
    v, svb, svt, svh = vsource.args()
    H = q.shape[1]
    if H % n_kv:
        raise ValueError(f"{H} query heads are not a multiple of {n_kv} kv heads")
    G = H // n_kv
    # the kernels index the state's partials, page tables and counts with these values
    if n_kv != st.n_kv or G != st.G:
        raise ValueError(f"cache / query geometry (n_kv {n_kv}, G {G}) differs from the "
                         f"state's (n_kv {st.n_kv}, G {st.G})")
    if n_req > st.max_reqs:
        raise ValueError(f"n_req {n_req} exceeds max_reqs {st.max_reqs}")
    if q.shape[0] < n_req or out.shape[0] < n_req or tuple(out.shape[1:]) != (H, d) \
            or block_table.shape[0] < n_req:
        raise ValueError("q, out and block_table need a row per request (out (T, H, d))")
    if not dense:
        table = st.page_table if table is None else table
        cnt = st.page_cnt if cnt is None else cnt
        if table.dtype != torch.int32 or cnt.dtype != torch.int32 or \
                table.shape[0] < n_req or table.shape[1] != n_kv or table.stride(2) != 1 or \
                cnt.shape[0] < n_req or cnt.shape[1] != n_kv or cnt.stride(1) != 1:
            raise ValueError("page_table (R, n_kv, MP) / page_cnt (R, n_kv) int32 expected")
    if path != "fused":
        m = getattr(st, "m_part", None)
        if m is None:
            raise ValueError("split-K partials missing: call ensure_stage_b_buffers(st, "
                             "device) once before decoding (outside any graph capture)")
        split = getattr(st, "split", SPLIT)
        want = (st.max_reqs, n_kv, split, G)
        if tuple(m.shape) != want or tuple(st.l_part.shape) != want or \
                tuple(st.acc_part.shape) != want + (d,) or not (
                    m.is_contiguous() and st.l_part.is_contiguous()
                    and st.acc_part.is_contiguous()):
            raise ValueError(f"split-K partials must be contiguous {want}[+(d,)] fp32")
    tf = vsource.tier_fields()
    return DecodeArgs(
        q=ptr(q), q_st=q.stride(0), q_hs=q.stride(1),
        k=ptr(k), k_sb=k.stride(0), k_st=k.stride(1), k_sh=k.stride(2),
        v=ptr(v), v_sb=svb, v_st=svt, v_sh=svh,
        block_table=ptr(block_table), bt_st=block_table.stride(0),
        seq_lens=ptr(seq_lens),
        page_table=ptr(table), pt_sr=table.stride(0) if table is not None else 0,
        pt_sh=table.stride(1) if table is not None else 0,
        page_cnt=ptr(cnt), pc_sr=cnt.stride(0) if cnt is not None else 0,
        m_part=ptr(getattr(st, "m_part", None)), l_part=ptr(getattr(st, "l_part", None)),
        acc_part=ptr(getattr(st, "acc_part", None)),
        out=ptr(out), o_st=out.stride(0), o_hs=out.stride(1),
        hot=tf.get("hot"), page2slot=tf.get("page2slot"), vbo=tf.get("vbo"),
        pool=tf.get("pool"), t_layer=tf.get("layer", 0), t_nb=tf.get("nb", 0),
        t_slots=tf.get("slots", 0), scale=float(scale), n_req=n_req, n_kv=n_kv, G=G, d=d,
        page=page, split=getattr(st, "split", SPLIT), pps_min=_pps_min(n_req),
        path=PATHS[path], dense=1 if dense else 0, v_src=vsource.SRC_ID)


def sparse_paged_decode_batched(q, kv_cache, block_table, seq_lens, st, out, vsource, *,
                                scale: float = None, path: str = "auto") -> None:
    """Attend st.page_table[r, kh, :st.page_cnt[r, kh]] of every (request, kv-head)."""
    if scale is None:
        scale = st.scale
    k, _ = _split_kv(kv_cache)
    n_req = seq_lens.shape[0]
    a = _decode_args(q, k, vsource, block_table, seq_lens, st, out, scale, n_req,
                     dense=False, path=path)
    call("amass_tier_decode" if vsource.SRC_ID == 1 else "amass_sparse_decode", a,
         current_stream(q.device))


def dense_paged_decode(q, kv_cache, block_table, seq_lens, st, out, *, scale: float,
                       path: str = "auto") -> None:
    """Dense paged decode over every page 0..ceil(seq_len/page) (the baseline the sparse
    path is measured against; same kernels with the page table bypassed)."""
    k, _ = _split_kv(kv_cache)
    n_req = seq_lens.shape[0]
    a = _decode_args(q, k, ResidentVSource(kv_cache), block_table, seq_lens, st, out,
                     scale, n_req, dense=True, path=path)
    call("amass_dense_paged_decode", a, current_stream(q.device))
