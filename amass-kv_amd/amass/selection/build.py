"""Page-summary builder: eigh of the centred page gram + int8/int4 fake-quant, written
into the R8State / QuadState records.

Device-resident K (the serving case) goes through the HIP kernel ``amass_summary_build``
(one launch per layer over a block list: mean, centred Gram on the matrix cores,
parallel-Jacobi eigh, top-r factors, quantisation and the content tag, straight into the
packed records).  A K cache in host memory (CPU-only tests of the lifecycle) takes the
torch restatement below of the reference builder (selection/build.py:297-348 quant
helpers, :396-412 ``_page_eigh``, :415-632 r8 lifecycle), whose 16x16 eigh goes through
``torch.linalg.eigh``.  Per (block, kv-head) of a finalised
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
    elif grain == "page_f32":                # one fp32 scale per page (not rounded)
        code, s = _quant(c, dim=(-2, -1), bits=bits)
        sc = s[..., 0, 0].float()
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
    st.r8_Vk[layer, blocks] = v_to_device(vk_code, st.vk_bits, tiled=True)
    st.Vk_scale[layer, blocks] = vk_s
    st.r8_c[layer, blocks] = c_code
    if st.c_grain == "page_f32":
        st.c_scale_f32[layer, blocks] = c_s
    else:
        st.c_scale[layer, blocks] = c_s
    st.r8_tag[layer, blocks] = Kp_flat[:, st.page - 1, :, :st.tagw].to(st.r8_tag.dtype)


def summary_build_hip(st, layer, K, blocks: torch.Tensor) -> None:
    """Build the summaries of physical ``blocks`` (int64 device tensor) from device K
    views (NB, page, n_kv, d) with one ``amass_summary_build`` launch: ``layer`` an int
    with ``K`` one view, or ``layer`` a range of consecutive layers with ``K`` their
    list of views (same strides; the launch reads their base addresses from a device
    array cached on the state, so a graph replay sees the same array)."""
    from .._hip import BuildArgs, call, current_stream, ptr, require_cuda
    r8 = hasattr(st, "r8_rec")
    rec_all = st.r8_rec if r8 else st.quad_rec
    tag_all = st.r8_tag if r8 else st.quad_tag
    if isinstance(layer, range):
        Ks, l0, nl = list(K), layer.start, len(layer)
        if layer.step != 1 or len(Ks) != nl or nl < 1:
            raise ValueError("layers must be a unit-step range matching the K views")
    else:
        Ks, l0, nl = [K], int(layer), 1
    K0 = Ks[0]
    require_cuda(*Ks, blocks, rec_all)
    for Kl in Ks:
        if Kl.dtype != torch.bfloat16 or Kl.stride() != K0.stride() or Kl.stride(3) != 1:
            raise ValueError("K views must be bf16 (NB, page, n_kv, d) with equal strides and "
                             "unit stride on d")
    blocks = blocks.to(torch.int64).contiguous()
    kl = None
    if nl > 1:
        key = tuple(Kl.data_ptr() for Kl in Ks)
        cache = st.__dict__.setdefault("_k_layer_ptrs", {})
        kl = cache.get(key)
        if kl is None:
            kl = torch.tensor(key, dtype=torch.int64, device=K0.device)
            cache[key] = kl
    rec, tag = rec_all[l0], tag_all[l0]
    clse = not r8 and getattr(st, "coords", "none") == "lse"
    v_bits = st.vk_bits if r8 else st.v_bits
    v_grain = (st.vk_grain if r8 else st.v_grain) == "tensor"
    # c scales: per token (0), one fp16 per (block, head) (1: r8 "tensor", CLSE "page"),
    # one fp32 per (block, head) (2: r8 "page_f32")
    c_head = (r8 and st.c_grain == "tensor") or (clse and st.c_grain == "page")
    c_grain = 2 if (r8 and st.c_grain == "page_f32") else int(c_head)
    a = BuildArgs(
        k=ptr(K0), k_sb=K0.stride(0), k_st=K0.stride(1), k_sh=K0.stride(2), k_layers=ptr(kl),
        blocks=ptr(blocks), rec=ptr(rec), rec_sb=rec.stride(0), rec_lsb=rec_all.stride(0),
        tag=ptr(tag), tag_sb=tag.stride(0), tag_sh=tag.stride(1), tag_lsb=tag_all.stride(0),
        n=int(blocks.numel()), n_layers=nl, n_kv=st.n_kv, d=st.d, page=st.page,
        kind=1 if r8 else (2 if clse else 0), rank=st.r, v_bits=v_bits,
        c_bits=st.c_bits if (r8 or clse) else 8, v_grain=int(v_grain), c_grain=c_grain,
        tagw=st.tagw)
    call("amass_summary_build", a, current_stream(K0.device))


def _write_blocks(st, layer: int, K: torch.Tensor, blocks: torch.Tensor, writer) -> None:
    """Summaries of ``blocks`` into ``layer``: the HIP builder for a device K, the torch
    restatement (in chunks) for a host K."""
    if K.is_cuda:
        summary_build_hip(st, layer, K, blocks)
        return
    for i in range(0, blocks.numel(), CHUNK):
        b = blocks[i:i + CHUNK]
        writer(st, K[b], layer, b)


def _write_layers(st, K_layers, blocks: torch.Tensor, writer) -> None:
    """Summaries of ``blocks`` in every layer: one HIP launch when all layers' K views
    are on the device with equal strides, else per layer."""
    K_layers = list(K_layers)
    if (K_layers and all(K.is_cuda for K in K_layers)
            and all(K.stride() == K_layers[0].stride() for K in K_layers)):
        summary_build_hip(st, range(len(K_layers)), K_layers, blocks)
        return
    for l, K in enumerate(K_layers):
        _write_blocks(st, l, K, blocks, writer)


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
    _write_blocks(st, layer, K, blocks, writer)
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
    _write_layers(st, K_layers, blocks, r8_write)
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
