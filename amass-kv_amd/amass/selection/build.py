"""Page-summary builder (off the hot path): eigh of the centred page gram + int8/int4
fake-quant, scattered into the R8State / QuadState slabs.

Restates the reference builder (selection/build.py:297-348 quant helpers, :396-412
``_page_eigh``, :415-632 r8 lifecycle) in torch; it runs on the device of the K cache
(the 16x16 eigh goes through ``torch.linalg.eigh``).  Per (block, kv-head) of a finalised
page:  mu = mean_t K ; dc = K - mu ; Gm = dc dc^T (page x page) ; S2, U = eigh(Gm)
ascending ; top-r: S2r = clamp(S2[-r:], 1e-10), U8 = U[:, -r:], S8 = sqrt(S2r) ;
Vk = dc^T U8 / S8 (d x r) ; c = U8 * S8 (page x r).
Quant: lvl = 2^(bits-1) - 1, s = max(amax/lvl, 1e-8) (fp32), code = clamp(rint(x/s)),
stored scale fp16(s).  int4 packs two nibbles per byte along the last axis, lo = even.
"""
from __future__ import annotations

import torch

from .quad_state import v_to_device

CHUNK = 16384   # (block, kv-head) records per eigh batch


def _quant(x: torch.Tensor, dim, bits: int = 8):
    lvl = float((1 << (bits - 1)) - 1)
    s = (x.abs().amax(dim=dim, keepdim=True) / lvl).clamp_min(1e-8)
    code = torch.round(x / s).clamp_(-lvl, lvl).to(torch.int8)
    return code, s


def _pack_i4(code: torch.Tensor) -> torch.Tensor:
    """(..., r) int8 in [-7, 7] -> (..., r/2) int8: lo nibble = even column."""
    if code.shape[-1] % 2:
        raise ValueError("int4 packing needs an even last dim")
    nib = code.to(torch.int32) & 0xF
    return (nib[..., 0::2] | (nib[..., 1::2] << 4)).to(torch.uint8).view(torch.int8).contiguous()


def _unpack_i4(packed: torch.Tensor) -> torch.Tensor:
    """Inverse of _pack_i4 -> (..., 2 * r/2) int8 codes."""
    b = packed.view(torch.uint8).to(torch.int32)
    lo, hi = b & 0xF, (b >> 4) & 0xF
    lo = torch.where(lo >= 8, lo - 16, lo)
    hi = torch.where(hi >= 8, hi - 16, hi)
    return torch.stack([lo, hi], dim=-1).flatten(-2).to(torch.int8)


def _quant_mu(mu):
    code, s = _quant(mu, dim=-1, bits=8)
    return code, s.squeeze(-1).to(torch.float16)


def _quant_vk(Vk, grain: str = "col", bits: int = 8):
    if grain == "col":
        code, s = _quant(Vk, dim=-2, bits=bits)
        sc = s.squeeze(-2).to(torch.float16)
    else:
        code, s = _quant(Vk, dim=(-2, -1), bits=bits)
        sc = s.squeeze(-2).expand(*Vk.shape[:-2], Vk.shape[-1]).contiguous().to(torch.float16)
    if bits == 4:
        code = _pack_i4(code)
    return code, sc


def _quant_c(c, grain: str = "page", bits: int = 8):
    if grain == "page":
        code, s = _quant(c, dim=-1, bits=bits)
        sc = s.squeeze(-1).to(torch.float16)
    else:
        code, s = _quant(c, dim=(-2, -1), bits=bits)
        sc = s.squeeze(-1).expand(*c.shape[:-2], c.shape[-2]).contiguous().to(torch.float16)
    if bits == 4:
        code = _pack_i4(code)
    return code, sc


def _eigh(Gm: torch.Tensor):
    """Batched symmetric eigh, ascending (LAPACK via torch.linalg.eigh on the host, in
    chunks; the 16x16 grams are tiny next to the K pages they summarise)."""
    flat = Gm.reshape(-1, Gm.shape[-2], Gm.shape[-1])
    S2 = torch.empty(flat.shape[:-1], device=Gm.device, dtype=Gm.dtype)
    U = torch.empty_like(flat)
    for i in range(0, flat.shape[0], CHUNK):
        s2, u = torch.linalg.eigh(flat[i:i + CHUNK].cpu())
        S2[i:i + CHUNK] = s2.to(Gm.device)
        U[i:i + CHUNK] = u.to(Gm.device)
    return S2.reshape(Gm.shape[:-1]), U.reshape(Gm.shape)


def _page_eigh(Kp_flat: torch.Tensor, r: int):
    """(N, page, n_kv, d) bf16 key pages -> (mu, U8, S8, S2r, Vk) fp32, each
    (N, n_kv, ...)."""
    Kp = Kp_flat.permute(0, 2, 1, 3).float()
    mu = Kp.mean(dim=2)
    dc = Kp - mu[:, :, None, :]
    Gm = torch.matmul(dc, dc.transpose(-1, -2))
    S2, U = _eigh(Gm)
    S2r = S2[..., -r:].clamp_min(1e-10)
    S8 = S2r.sqrt()
    U8 = U[..., -r:]
    Vk = torch.matmul(dc.transpose(-1, -2), U8) / S8[..., None, :]
    return mu, U8, S8, S2r, Vk


def finalized_blocks(block_table, seq_lens, n_req: int, page: int):
    """Physical blocks of every finalised page of the first n_req rows (host sync)."""
    sl = seq_lens[:n_req].to(torch.int64)
    nfin = sl // page
    mf = int(nfin.max().item()) if n_req else 0
    if mf == 0:
        return block_table.new_zeros(0, dtype=torch.int64)
    idx = torch.arange(mf, device=block_table.device)
    mask = idx[None, :] < nfin[:, None]
    return block_table[:n_req, :mf].to(torch.int64)[mask]


# ------------------------------------------------------------------ r8 summaries
def r8_write(st, Kp_flat: torch.Tensor, layer: int, blocks: torch.Tensor) -> None:
    """Summarise K pages (N, page, n_kv, d) of physical ``blocks`` into layer slabs."""
    mu, U8, S8, _S2r, Vk = _page_eigh(Kp_flat, st.r)
    c = U8 * S8[..., None, :]
    mu_code, mu_s = _quant_mu(mu)
    vk_code, vk_s = _quant_vk(Vk, st.vk_grain, st.vk_bits)
    c_code, c_s = _quant_c(c, st.c_grain, st.c_bits)
    st.r8_mu[layer, blocks] = mu_code
    st.mu_scale[layer, blocks] = mu_s
    st.r8_Vk[layer, blocks] = v_to_device(vk_code, st.vk_bits)
    st.Vk_scale[layer, blocks] = vk_s
    st.r8_c[layer, blocks] = c_code
    st.c_scale[layer, blocks] = c_s
    st.r8_tag[layer, blocks] = Kp_flat[:, st.page - 1, :, :st.tagw].to(st.r8_tag.dtype)


def _stale(tag_slab, K, blocks, page, tagw):
    cur = K[blocks, page - 1, :, :tagw].float()
    return (cur != tag_slab[blocks].float()).any(dim=(1, 2))   # NaN tag -> stale


def _refresh(st, layer, K, block_table, seq_lens, n_req, force, tag_slab, writer) -> int:
    blocks = finalized_blocks(block_table, seq_lens, n_req, st.page)
    if blocks.numel() == 0:
        return 0
    if not force:
        blocks = blocks[_stale(tag_slab[layer], K, blocks, st.page, st.tagw)]
    blocks = torch.unique(blocks)
    for i in range(0, blocks.numel(), CHUNK):
        b = blocks[i:i + CHUNK]
        writer(st, K[b], layer, b)
    return int(blocks.numel())


def r8_build_refresh(st, layer: int, K, block_table, seq_lens, n_req: int, *,
                     force: bool = False) -> int:
    """(Re)build the r8 summary of every stale finalised page of the batch (tag-gated,
    selection/build.py:560-632).  Returns the number of blocks rebuilt."""
    return _refresh(st, layer, K, block_table, seq_lens, n_req, force, st.r8_tag, r8_write)


def _tail_blocks(block_table, seq_lens, n_req: int, page: int, rows=None):
    sl = (seq_lens[:n_req] if rows is None else seq_lens[rows]).to(torch.int64)
    bt = block_table[:n_req] if rows is None else block_table[rows]
    last = (sl // page - 1).clamp_(min=0)
    return bt.to(torch.int64).gather(1, last[:, None]).squeeze(1)


def r8_build_tail(st, K_layers, block_table, seq_lens, n_req: int, rows=None) -> int:
    """Rebuild each request's last finalised page in every layer (idempotent)."""
    if n_req == 0:
        return 0
    blocks = _tail_blocks(block_table, seq_lens, n_req, st.page, rows)
    for l, K in enumerate(K_layers):
        r8_write(st, K[blocks], l, blocks)
    return len(K_layers) * int(blocks.numel())


def r8_build_bulk(st, K_layers, block_table, seq_lens, n_req: int, max_fin: int = 0,
                  chunk_pairs: int = CHUNK) -> int:
    """Rebuild every finalised page of the batch in every layer."""
    n = 0
    for l, K in enumerate(K_layers):
        n += r8_build_refresh(st, l, K, block_table, seq_lens, n_req, force=True)
    return n


def r8_build_delta(st, K_layers, block_table, seq_lens, n_req: int, max_fin: int = 0,
                   chunk_pairs: int = CHUNK) -> int:
    """Rebuild only blocks whose content tag went stale, in every layer."""
    n = 0
    for l, K in enumerate(K_layers):
        n += r8_build_refresh(st, l, K, block_table, seq_lens, n_req, force=False)
    return n
