"""The reference's score -> select -> attend path restated in fp32 PyTorch for the CPU
(TEST INFRASTRUCTURE: bench.py's cpu_baseline leg times it on the host cores; the product
never imports it).

Each stage is whole-tensor torch work over one layer's batch, the way a PyTorch port of
the reference's Triton kernels runs on a CPU:

quad_score   selection/quad_score.py:35-107 (_quad_score_kernel) and :110-139: the codes
             dequantised in fp32 (int4 nibbles unpacked, even column = low nibble),
             q~ = V^T q_g, quad = s^2/(2P) sum_k sig2_k q~_k^2, qmu = s (mu . q_g),
             S_g = qmu + quad for the scored pages p < n_sel_hi; per-head scores (nrm).
nrm_combine  selection/quad_score.py:276-315: score[p] = sum_g exp(S_g[p] - max_p S_g).
derive       selection/select.py:30-54: n_pages, n_sel_hi, b = ceil(budget S) in [1, S].
select       selection/select.py:60-116 (top-b over [sink, n_sel_hi), sinks / window /
             tail kept, ascending page table with -1 padding) with the per-(request,
             kv-head) coverage nucleus of backend/_selection_bridge.py:117-133 as this
             build specifies it: 2^-32 fixed-point masses (nrm scores clipped to
             [0, 1024]), need = ceil(coverage * total) - sink mass, b = the fewest
             top pages reaching it; ties in (score desc, page asc) order.
attend       attention/decode.py:128-304 + attention/merge.py:21-50: per (request, kv
             head) softmax attention of the group's queries over the selected pages'
             tokens (bf16 K/V upcast to fp32, scale after the dot, tokens >= seq_len
             masked).  The split-K partials and their LSE merge are one pass here (the
             merge is exact up to rounding: split invariance).

Pinned against the numpy oracle (itself pinned by closed forms and brute force) in
tests/test_torch_path.py: scores, page tables and outputs on seeded cases.
"""
from __future__ import annotations

import math

import torch

from .select import _C, _LN2_HI, _LN2_LO, _LOG2E

F32 = torch.float32


def exp_det(x: torch.Tensor) -> torch.Tensor:
    """The selection's deterministic fp32 exp (oracle/select.py exp_det: Cody-Waite
    reduction, degree-7 Taylor polynomial) in torch ops; 0 below -80."""
    x = x.to(F32)
    n = torch.round(x * float(_LOG2E))
    r = (x - n * float(_LN2_HI)) - n * float(_LN2_LO)
    p = torch.full_like(r, float(_C[0]))
    for c in _C[1:]:
        p = p * r + float(c)
    p = p * r + 1.0
    p = p * r + 1.0
    out = torch.ldexp(p, n.to(torch.int32))
    return torch.where(x > -80.0, out, torch.zeros_like(out))


def unpack_codes(v: torch.Tensor, bits: int) -> torch.Tensor:
    """int8 codes, or int4 pairs along the last dim (low nibble = even column)."""
    if bits == 8:
        return v.to(F32)
    b = v.to(torch.int32) & 0xFF
    lo = ((b & 0xF) ^ 8) - 8
    hi = ((b >> 4) ^ 8) - 8
    return torch.stack([lo, hi], dim=-1).flatten(-2).to(F32)


def quad_score(q, mu, mu_scale, V, V_scale, sig2, block_table, n_sel_hi, *, scale: float,
               page: int, G: int, v_bits: int, max_pages: int) -> torch.Tensor:
    """-> score_h (R, n_kv, G, MP) fp32, NaN beyond n_sel_hi.  q (R, H, d) fp32;
    mu (NB, n_kv, d) int8, mu_scale (NB, n_kv), V (NB, n_kv, d, r' or r'/2) int8,
    V_scale / sig2 (NB, n_kv, r')."""
    R, H, d = q.shape
    n_kv = mu.shape[1]
    out = torch.full((R, n_kv, G, max_pages), float("nan"), dtype=F32)
    qcoef = scale * scale / (2.0 * page)
    for r in range(R):
        n = int(n_sel_hi[r])
        if n <= 0:
            continue
        blk = block_table[r, :n].long()
        Vd = unpack_codes(V[blk], v_bits) * V_scale[blk].to(F32)[:, :, None, :]  # (n,kv,d,r)
        mud = mu[blk].to(F32) * mu_scale[blk].to(F32)[..., None]                 # (n,kv,d)
        qr = q[r].view(n_kv, G, d)
        # (kv, G, d) x (kv, d, n r') -> (kv, G, n, r')
        qt = torch.bmm(qr, Vd.permute(1, 2, 0, 3).reshape(n_kv, d, -1)).view(n_kv, G, n, -1)
        quad = (qt * qt * sig2[blk].to(F32).permute(1, 0, 2)[:, None]).sum(-1) * qcoef
        qmu = torch.bmm(qr, mud.permute(1, 2, 0)) * scale                         # (kv,G,n)
        out[r, :, :, :n] = qmu + quad
    return out


def nrm_combine(score_h: torch.Tensor, n_sel_hi) -> torch.Tensor:
    R, n_kv, G, MP = score_h.shape
    out = torch.full((R, n_kv, MP), float("nan"), dtype=F32)
    for r in range(R):
        n = int(n_sel_hi[r])
        if n <= 0:
            continue
        s = score_h[r, :, :, :n]
        out[r, :, :n] = torch.exp(s - s.max(dim=-1, keepdim=True).values).sum(dim=1)
    return out


def derive(seq_lens, budget: float, page: int, window: int, sink: int):
    sl = torch.as_tensor(seq_lens).long()
    npg = (sl + page - 1) // page
    nsh = npg - window
    S = nsh - sink
    b = torch.tensor([min(max(math.ceil(float(s) * budget), 1), max(int(s), 1))
                      for s in S.tolist()], dtype=torch.long)
    return npg, nsh, b


def select(score, n_pages, n_sel_hi, b_fix, *, sink: int, max_pages: int, mode: int,
           coverage: float = 1.0, score_kind: int = 1):
    """-> (page_table (R, n_kv, MP) int32, page_cnt (R, n_kv) int32).  mode 0: b = b_fix;
    mode 1: the coverage nucleus (score_kind 1: the scores are masses; 0: log-masses)."""
    R, n_kv, MP = score.shape
    keep = torch.zeros((R, n_kv, MP), dtype=torch.bool)
    pos = torch.arange(MP)
    for r in range(R):
        npg, nh = int(n_pages[r]), int(n_sel_hi[r])
        if npg <= 0:
            continue
        S = nh - sink
        if S <= 1:
            keep[r, :, :npg] = True
            continue
        sc = score[r, :, :nh]
        vals, idx = torch.sort(sc[:, sink:], dim=-1, descending=True, stable=True)
        if mode == 1:
            w = (sc.clamp(0.0, 1024.0) if score_kind == 1 else
                 exp_det(sc - sc.max(dim=-1, keepdim=True).values))
            wq = (torch.nan_to_num(w, nan=0.0) * 4294967296.0).to(torch.int64)
            need = torch.ceil(coverage * wq.sum(-1).double()).long() - wq[:, :sink].sum(-1)
            cum = torch.cumsum(torch.gather(wq[:, sink:], 1, idx), dim=-1)
            b = ((cum < need[:, None]).sum(-1) + 1).clamp(1, S)
            b = torch.where(need <= 0, torch.ones_like(b), b)
        else:
            b = torch.full((n_kv,), min(max(int(b_fix[r]), 1), S), dtype=torch.long)
        chosen = torch.arange(S)[None, :] < b[:, None]
        keep[r, :, sink:nh] = torch.zeros_like(chosen).scatter(1, idx, chosen)
        keep[r, :, :sink] = True
        keep[r, :, nh:npg] = True
    cnt = keep.sum(-1)
    key = torch.where(keep, pos, pos + MP)
    order = torch.sort(key, dim=-1).values
    table = torch.where(order < MP, order, torch.full_like(order, -1))
    return table.to(torch.int32), cnt.to(torch.int32)


def attend(q, K, V, block_table, seq_lens, page_table, page_cnt, *, scale: float, G: int):
    """q (R, H, d) fp32; K, V (NB, page, n_kv, d) (bf16) -> out (R, H, d) fp32."""
    R, H, d = q.shape
    page, n_kv = K.shape[1], K.shape[2]
    out = torch.zeros((R, H, d), dtype=F32)
    kv = torch.arange(n_kv)
    for r in range(R):
        sl = int(seq_lens[r])
        cnt = page_cnt[r].long()
        c = int(cnt.max())
        if c <= 0:
            continue
        pages = page_table[r, :, :c].long()                          # (kv, c), -1 padded
        valid_pg = torch.arange(c)[None, :] < cnt[:, None]
        pages = torch.where(valid_pg, pages, torch.zeros_like(pages))
        blk = block_table[r].long()[pages]                           # (kv, c)
        k = K[blk, :, kv[:, None], :].to(F32).reshape(n_kv, c * page, d)
        v = V[blk, :, kv[:, None], :].to(F32).reshape(n_kv, c * page, d)
        tok = (pages[..., None] * page + torch.arange(page)).reshape(n_kv, -1)
        ok = (tok < sl) & valid_pg.repeat_interleave(page, dim=1)
        k = torch.where(ok[..., None], k, torch.zeros_like(k))
        v = torch.where(ok[..., None], v, torch.zeros_like(v))
        s = torch.bmm(q[r].view(n_kv, G, d), k.transpose(1, 2)) * scale   # (kv, G, T)
        s = s.masked_fill(~ok[:, None, :], float("-inf"))
        p = torch.softmax(s, dim=-1)
        p = torch.nan_to_num(p, nan=0.0)                             # empty units -> 0
        out[r] = torch.bmm(p, v).view(H, d)
    return out
