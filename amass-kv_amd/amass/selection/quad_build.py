"""Quad page-summary builder (off the hot path).

Restates selection/quad_build.py:56-198 of the reference: the same page-gram eigh as the
r8 builder (:mod:`amass.selection.build`), storing the top-r' eigenvalues ``sig2`` instead
of the per-key coordinates.  Per (block, kv-head): quad_mu/mu_scale = int8 page mean,
quad_V/V_scale = Vk = dc^T U8 / S8 quantised per column (int8 or packed int4, stored
in the tiled kernel layout),
quad_sig2 = fp16(S2r), quad_tag = leading TAGW channels of the page's last key.  A device
K is summarised by the HIP builder (``amass_summary_build``), a host K by the torch
restatement below.
"""
from __future__ import annotations

import torch

from .build import (CHUNK, _page_eigh, _quant_c, _quant_mu, _quant_vk, _refresh, _tail_blocks,
                    _write_layers, finalized_blocks)
from .quad_state import v_to_device


def quad_write(st, Kp_flat: torch.Tensor, layer: int, blocks: torch.Tensor) -> None:
    mu, U8, S8, S2r, Vk = _page_eigh(Kp_flat, st.r)
    mu_code, mu_s = _quant_mu(mu)
    v_code, v_s = _quant_vk(Vk, st.v_grain, st.v_bits)
    st.quad_mu[layer, blocks] = mu_code
    st.mu_scale[layer, blocks] = mu_s
    st.quad_V[layer, blocks] = v_to_device(v_code, st.v_bits, tiled=st.v_tiled)
    st.V_scale[layer, blocks] = v_s
    if getattr(st, "coords", "none") == "lse":
        # CLSE extras (reference selection/quad_build.py:38-54): c = U8 * S8 quantised per
        # token ("token") or per (block, head) ("page"); resid = trace - sum(top-r' eig)
        c = U8 * S8[..., None, :]
        c_code, c_s = _quant_c(c, "page" if st.c_grain == "token" else "tensor", st.c_bits)
        Kp = Kp_flat.permute(0, 2, 1, 3).float()
        trace = Kp.pow(2).sum(dim=(2, 3)) - st.page * mu.pow(2).sum(-1)
        st.quad_c[layer, blocks] = c_code
        st._c_scale16[layer, blocks] = c_s.to(st._c_scale16.dtype)
        st.quad_resid[layer, blocks] = (trace - S2r.sum(-1)).clamp_min(0).to(
            st.quad_resid.dtype)
    else:
        st.quad_sig2[layer, blocks] = S2r.to(st.quad_sig2.dtype)
    st.quad_tag[layer, blocks] = Kp_flat[:, st.page - 1, :, :st.tagw].to(st.quad_tag.dtype)


def quad_build_refresh(st, layer: int, K, block_table, seq_lens, n_req: int, *,
                       force: bool = False) -> int:
    """(Re)build the quad summary of every stale finalised page (tag-gated)."""
    return _refresh(st, layer, K, block_table, seq_lens, n_req, force, st.quad_tag,
                    quad_write)


def quad_build_tail(st, K_layers, block_table, seq_lens, n_req: int, rows=None) -> int:
    if n_req == 0:
        return 0
    blocks = _tail_blocks(block_table, seq_lens, n_req, st.page, rows)
    _write_layers(st, K_layers, blocks, quad_write)
    return len(K_layers) * int(blocks.numel())


def quad_build_bulk(st, K_layers, block_table, seq_lens, n_req: int, max_fin: int = 0,
                    chunk_pairs: int = CHUNK) -> int:
    return sum(quad_build_refresh(st, l, K, block_table, seq_lens, n_req, force=True)
               for l, K in enumerate(K_layers))


def quad_build_delta(st, K_layers, block_table, seq_lens, n_req: int, max_fin: int = 0,
                     chunk_pairs: int = CHUNK) -> int:
    return sum(quad_build_refresh(st, l, K, block_table, seq_lens, n_req, force=False)
               for l, K in enumerate(K_layers))


__all__ = ["quad_write", "quad_build_refresh", "quad_build_tail", "quad_build_bulk",
           "quad_build_delta", "finalized_blocks"]
