"""r8 page score (Stage A.1, r8 mode) -- host side of ``amass_r8_score``.

Same contract as the reference ``r8_score`` (selection/score.py:123-148): writes
``st.score`` (R, n_kv, MP) fp32, the group max of s*mu.q + logsumexp_t(s * c_t . q~)
over the scored region.  ``comb_out`` (optional int32 (R, n_kv, MP, G, r+1)) receives the
exact integer d-contractions sum_d qi*code (the r columns of Vk, then mu).
"""
from __future__ import annotations

import torch

from .._hip import R8ScoreArgs, call, current_stream, ptr, require_cuda


def check_rec_span(rec) -> None:
    """The score kernels address a layer's records with 32-bit byte offsets from its base
    (block * rec_sb + head and lane offsets), so the layer's record buffer must span less
    than 4 GiB."""
    if rec.shape[0] * rec.stride(0) > (1 << 32):
        raise ValueError(f"a layer's summary records span {rec.shape[0] * rec.stride(0)} "
                         "bytes; the score kernels address at most 4 GiB per layer")


def r8_score(st, layer: int, q, block_table, seq_lens, n_req: int, scale: float,
             comb_out=None) -> None:
    if n_req > st.max_reqs:
        raise ValueError(f"n_req {n_req} exceeds max_reqs {st.max_reqs}")
    rec = st.r8_rec[layer]
    require_cuda(q, block_table, seq_lens, rec)
    if q.dtype != torch.bfloat16 or q.stride(2) != 1:
        raise ValueError("q must be bf16 (T, H, d) with unit stride on d")
    if block_table.dtype != torch.int32 or seq_lens.dtype != torch.int32:
        raise ValueError("block_table / seq_lens must be int32")
    if block_table.stride(1) != 1:
        raise ValueError("block_table must have unit column stride")
    if rec.stride(1) != 1 or rec.shape[1] != st.n_kv * st.rec_bytes:
        raise ValueError("r8_rec must hold each block's records contiguously")
    check_rec_span(rec)
    if comb_out is not None and (comb_out.dtype != torch.int32 or not comb_out.is_contiguous()
                                 or tuple(comb_out.shape[1:]) != (st.n_kv, st.max_pages, st.G,
                                                                  st.r + 1)):
        raise ValueError("comb_out must be a contiguous int32 (R, n_kv, MP, G, r+1) tensor")
    a = R8ScoreArgs(
        q=ptr(q), q_st=q.stride(0), q_hs=q.stride(1),
        rec=ptr(rec), rec_sb=rec.stride(0),
        block_table=ptr(block_table), bt_st=block_table.stride(0),
        seq_lens=ptr(seq_lens), n_sel_hi=ptr(st.n_sel_hi),
        score=ptr(st.score), sc_sr=st.score.stride(0), sc_sh=st.score.stride(1),
        comb_out=ptr(comb_out), scale=float(scale),
        n_req=n_req, n_kv=st.n_kv, G=st.G, d=st.d, page=st.page, rank=st.r,
        vk_bits=st.vk_bits, c_bits=st.c_bits, max_pages=st.max_pages,
        c_fp32=1 if getattr(st, "c_grain", "page") == "page_f32" else 0)
    call("amass_r8_score", a, current_stream(q.device))
