"""Page selection (test oracle): derive, top-b, coverage nucleus, deterministic exp.

derive   restates selection/select.py:30-45: n_pages = ceil(sl/P), n_sel_hi = n_pages - W,
         S = n_sel_hi - sink, b = min(max(ceil_fp64(budget * S), 1), max(S, 1)).
select   restates selection/select.py:60-101 (keep = selectable & chosen | p < sink |
         p >= n_sel_hi | S <= 1; ascending compaction, -1 pad, page_cnt) with the chosen
         set defined as:
           tie_mode 0: the first b pages in (score desc, page index asc) order;
           tie_mode 1: every selectable page with score >= the b-th largest score (the
                       reference threshold rule, select.py:84-89).
         Fixed mode: b = clamp(b_fix, 1, S).  Coverage mode (the build's per-(request,
         kv-head) nucleus; the reference's only coverage code is the eager per-request
         bridge, backend/_selection_bridge.py:117-133): page masses w in 2^-32 fixed point
         over the scored pages [0, n_sel_hi) (score_kind 0: w = exp_det(score - max),
         1: w = clip(score, 0, 1024)); need = ceil(coverage * total) - sink mass; b = the
         smallest count whose cumulative mass in (score desc, index asc) order reaches
         need (b = 1 when the sinks already cover).
exp_det  the fp32 exp the gfx950 selection kernel uses (Cody-Waite + degree-7 Taylor,
         only correctly rounded fp32 ops), restated op for op so masses match bit for bit.
"""
from __future__ import annotations

import math

import numpy as np

F32 = np.float32
_LOG2E = F32(float.fromhex("0x1.715476p+0"))
_LN2_HI = F32(float.fromhex("0x1.62e400p-1"))
_LN2_LO = F32(float.fromhex("0x1.7f7d1cp-20"))
_C = [F32(float.fromhex(h)) for h in ("0x1.a01a02p-13", "0x1.6c16c2p-10", "0x1.111112p-7",
                                       "0x1.555556p-5", "0x1.555556p-3", "0x1.000000p-1")]


def derive(seq_lens, budget: float, page: int, window: int, sink: int):
    sl = np.asarray(seq_lens, np.int64)
    npg = (sl + page - 1) // page
    nsh = npg - window
    S = nsh - sink
    b = np.array([min(max(int(math.ceil(float(s) * budget)), 1), max(int(s), 1)) for s in S],
                 np.int64)
    return npg.astype(np.int32), nsh.astype(np.int32), b.astype(np.int32)


def f2u(x):
    """fp32 -> order-preserving uint32 keys (-0.0 shares +0.0's key: they compare equal)."""
    u = np.asarray(x, np.float32).view(np.uint32)
    u = np.where(u == np.uint32(0x80000000), np.uint32(0), u)
    mask = np.where(u >> 31, np.uint32(0xFFFFFFFF), np.uint32(0x80000000))
    return u ^ mask


def exp_det(x):
    x = np.asarray(x, np.float32)
    out = np.zeros(x.shape, np.float32)
    m = x > F32(-80.0)
    xv = x[m]
    n = np.rint(xv * _LOG2E).astype(np.float32)
    r = ((xv - n * _LN2_HI) - n * _LN2_LO).astype(np.float32)
    p = _C[0]
    for c in _C[1:]:
        p = (p * r + c).astype(np.float32)
    p = (p * r + F32(1.0)).astype(np.float32)
    p = (p * r + F32(1.0)).astype(np.float32)
    out[m] = np.ldexp(p, n.astype(np.int32)).astype(np.float32)
    return out


def mass_q(score, smax, kind: int):
    score = np.asarray(score, np.float32)
    if kind == 0:
        w = exp_det((score - F32(smax)).astype(np.float32))
    else:
        w = np.clip(score, F32(0), F32(1024)).astype(np.float32)
        w = np.where(np.isnan(w), F32(0), w)
    return (w * F32(4294967296.0)).astype(np.float32).astype(np.uint64)


def select(score, n_pages, n_sel_hi, b_fix, *, sink: int, max_pages: int, mode: int = 0,
           coverage: float = 1.0, tie_mode: int = 0, score_kind: int = 0):
    """-> (page_table (R, n_kv, MP) int32, page_cnt (R, n_kv) int32, n_sel (R, n_kv))."""
    score = np.asarray(score, np.float32)
    R, n_kv = score.shape[0], score.shape[1]
    tab = np.full((R, n_kv, max_pages), -1, np.int32)
    cnt = np.zeros((R, n_kv), np.int32)
    nsel = np.zeros((R, n_kv), np.int32)
    for r in range(R):
        npg, nh = int(n_pages[r]), int(n_sel_hi[r])
        S = nh - sink
        for kh in range(n_kv):
            if npg <= 0:
                continue
            keep_all = S <= 1
            keep = np.zeros(npg, bool)
            if keep_all:
                keep[:] = True
                nsel[r, kh] = max(S, 0)
            else:
                nsc = max(min(nh, npg), 0)
                sc = score[r, kh, :nsc]
                sel = sc[sink:nh]
                idx = np.arange(sink, nh)
                key = f2u(sel).astype(np.int64)
                order = np.lexsort((idx, -key))           # score desc, index asc
                if mode == 1:
                    smax = F32(sc.max()) if score_kind == 0 else F32(0)
                    wq = mass_q(sc, smax, score_kind)
                    tot = int(wq.sum(dtype=np.uint64))
                    snk = int(wq[:sink].sum(dtype=np.uint64))
                    need = int(math.ceil(coverage * float(tot))) - snk
                    if need <= 0:
                        b = 1
                    else:
                        cum = np.cumsum(wq[sink:nh][order].astype(object))
                        hit = np.nonzero(cum >= need)[0]
                        b = int(hit[0]) + 1 if hit.size else S
                else:
                    b = min(max(int(b_fix[r]), 1), S)
                keep[:sink] = True
                keep[nh:npg] = True
                if tie_mode == 0:
                    keep[idx[order[:b]]] = True
                    nsel[r, kh] = b
                else:
                    tau = sel[order[b - 1]]
                    chosen = sel >= tau
                    keep[idx[chosen]] = True
                    nsel[r, kh] = int(chosen.sum())
            pages = np.nonzero(keep)[0]
            tab[r, kh, :pages.size] = pages
            cnt[r, kh] = pages.size
    return tab, cnt, nsel
