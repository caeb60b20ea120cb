"""Page scores (test oracle): quad, nrm combine, r8 and their exact integer cores.

quad_score  restates selection/quad_score.py:35-107 (Triton golden) in float64 on the
            dequantised summary: qh_k = (V_code[:,k] V_scale[k]) . q_g,
            quad = s^2/(2P) sum_k sig2_k qh_k^2, qmu = s (mu_code mu_scale) . q_g,
            S_g = qmu + quad; combine "max" -> max_g S_g, "nrm" -> per-head S_g.
            q_mode "float" uses q itself (the Triton reference); "limbs" uses the 2-limb
            int8 code qi*qs the int kernels contract with.
nrm_combine restates selection/quad_score.py:276-315: sum_g exp(S_g[p] - max_p S_g[p]).
r8_score    restates selection/score.py:30-120: q~ = Vk^T q, tok_t = s * c_t . q~ (c
            dequantised per token), masked 16p+t >= seq_len, S_g = s mu.q + lse_t tok.
quad_comb / r8_comb: exact sum_d qi * code (int64) for the V columns then mu, the integer
            accumulations the gfx950 kernels expose through comb_out.
"""
from __future__ import annotations

import numpy as np

from .quant import codes, q_limbs


def _q(q, mode):
    q = np.asarray(q, np.float32)
    if mode == "float":
        return q.astype(np.float64)
    qi, _hi, _lo, qs = q_limbs(q)
    return qi.astype(np.float64) * qs[..., None].astype(np.float64)


def quad_score(q, mu, mu_scale, V, V_scale, sig2, block_table, n_sel_hi, *, scale, page,
               G, v_bits, max_pages, combine="max", q_mode="float"):
    """-> score (R, n_kv, MP) [combine max] or score_h (R, n_kv, G, MP) [nrm]; NaN where
    no score is defined (p >= n_sel_hi)."""
    R = len(n_sel_hi)
    n_kv = mu.shape[1]
    out = np.full((R, n_kv, G, max_pages), np.nan)
    qcoef = scale * scale / (2.0 * page)
    for r in range(R):
        n = int(n_sel_hi[r])
        if n <= 0:
            continue
        blk = np.asarray(block_table[r, :n], np.int64)
        Vd = codes(V[blk], v_bits).astype(np.float64) * \
            np.asarray(V_scale[blk], np.float64)[:, :, None, :]          # (n, kv, d, r')
        mud = mu[blk].astype(np.float64) * np.asarray(mu_scale[blk], np.float64)[..., None]
        sg = np.asarray(sig2[blk], np.float64)                            # (n, kv, r')
        qr = _q(q[r], q_mode).reshape(n_kv, G, -1)                        # (kv, G, d)
        qh = np.einsum("kgd,nkdr->nkgr", qr, Vd)
        quad = qcoef * np.einsum("nkr,nkgr->nkg", sg, qh * qh)
        qmu = scale * np.einsum("kgd,nkd->nkg", qr, mud)
        out[r, :, :, :n] = (qmu + quad).transpose(1, 2, 0)
    if combine == "max":
        return out.max(axis=2)
    return out


def nrm_combine(score_h, n_sel_hi):
    """score_h (R, n_kv, G, MP) -> (R, n_kv, MP), NaN beyond n_sel_hi."""
    R, n_kv, G, MP = score_h.shape
    out = np.full((R, n_kv, MP), np.nan)
    for r in range(R):
        n = int(n_sel_hi[r])
        if n <= 0:
            continue
        S = np.asarray(score_h[r, :, :, :n], np.float64)
        hm = S.max(axis=-1, keepdims=True)
        out[r, :, :n] = np.exp(S - hm).sum(axis=1)
    return out


def _comb(q, mu, V, block_table, n_sel_hi, G, v_bits, max_pages):
    R = len(n_sel_hi)
    n_kv = mu.shape[1]
    rr = codes(V[:1], v_bits).shape[-1]
    out = np.zeros((R, n_kv, max_pages, G, rr + 1), np.int64)
    for r in range(R):
        n = int(n_sel_hi[r])
        if n <= 0:
            continue
        blk = np.asarray(block_table[r, :n], np.int64)
        qi = q_limbs(np.asarray(q[r], np.float32))[0].reshape(n_kv, G, -1)   # int64
        Vc = codes(V[blk], v_bits).astype(np.int64)                          # (n,kv,d,r)
        Mc = mu[blk].astype(np.int64)                                        # (n,kv,d)
        out[r, :, :n, :, :rr] = np.einsum("kgd,nkdr->kngr", qi, Vc)
        out[r, :, :n, :, rr] = np.einsum("kgd,nkd->kng", qi, Mc)
    return out


def quad_comb(q, mu, V, block_table, n_sel_hi, *, G, v_bits, max_pages):
    """Exact int64 sum_d qi*code: (R, n_kv, MP, G, r'+1) (V columns, then mu)."""
    return _comb(q, mu, V, block_table, n_sel_hi, G, v_bits, max_pages)


def r8_comb(q, mu, Vk, block_table, n_sel_hi, *, G, vk_bits, max_pages):
    return _comb(q, mu, Vk, block_table, n_sel_hi, G, vk_bits, max_pages)


def r8_score(q, mu, mu_scale, Vk, Vk_scale, c, c_scale, block_table, seq_lens, n_sel_hi,
             *, scale, page, G, vk_bits, c_bits, max_pages, q_mode="float"):
    """-> score (R, n_kv, MP) float64, NaN beyond n_sel_hi."""
    R = len(n_sel_hi)
    n_kv = mu.shape[1]
    out = np.full((R, n_kv, max_pages), np.nan)
    for r in range(R):
        n = int(n_sel_hi[r])
        if n <= 0:
            continue
        blk = np.asarray(block_table[r, :n], np.int64)
        Vd = codes(Vk[blk], vk_bits).astype(np.float64) * \
            np.asarray(Vk_scale[blk], np.float64)[:, :, None, :]
        cd = codes(c[blk], c_bits).astype(np.float64) * \
            np.asarray(c_scale[blk], np.float64)[..., None]                # (n,kv,P,r)
        mud = mu[blk].astype(np.float64) * np.asarray(mu_scale[blk], np.float64)[..., None]
        qr = _q(q[r], q_mode).reshape(n_kv, G, -1)
        qt = np.einsum("kgd,nkdr->nkgr", qr, Vd)
        tok = scale * np.einsum("nktr,nkgr->nkgt", cd, qt)                  # (n,kv,G,P)
        pos = np.arange(n)[:, None] * page + np.arange(page)[None, :]
        valid = pos < int(seq_lens[r])
        tok = np.where(valid[:, None, None, :], tok, -np.inf)
        m = tok.max(axis=-1, keepdims=True)
        lse = (m + np.log(np.exp(tok - m).sum(axis=-1, keepdims=True)))[..., 0]
        S = scale * np.einsum("kgd,nkd->nkg", qr, mud) + lse
        out[r, :, :n] = S.max(axis=-1).T
    return out


def clse_score(q, mu, mu_scale, V, V_scale, c, c_scale, resid, block_table, seq_lens,
               n_sel_hi, *, scale, page, G, v_bits, c_bits, max_pages, combine="max",
               q_mode="float"):
    """CLSE score (reference selection/quad_score.py:156-276, _clse_score_kernel) in
    float64: q~ = V^T q_g (dequantised V), tok = s (c q~) with c dequantised per token
    (c_scale (NB, n_kv, page)) or per page (c_scale (NB, n_kv)), masked logsumexp over the
    tokens, iso = max(|q_g|^2 - |q~|^2, 0) resid s^2 / (2 page max(d - r', 1)),
    S_g = s mu.q_g + lse + iso.  -> (R, n_kv, MP) group max ("max") or (R, n_kv, G, MP)
    per head ("nrm"); NaN beyond n_sel_hi."""
    R = len(n_sel_hi)
    n_kv, d = mu.shape[1], mu.shape[-1]
    r = np.asarray(V_scale).shape[-1]
    iso_coef = scale * scale / (2.0 * page * max(d - r, 1))
    shape = (R, n_kv, max_pages) if combine == "max" else (R, n_kv, G, max_pages)
    out = np.full(shape, np.nan)
    token_grain = np.asarray(c_scale).ndim == 3
    for rq in range(R):
        n = int(n_sel_hi[rq])
        if n <= 0:
            continue
        blk = np.asarray(block_table[rq, :n], np.int64)
        Vd = codes(V[blk], v_bits).astype(np.float64) * \
            np.asarray(V_scale[blk], np.float64)[:, :, None, :]
        cs = np.asarray(c_scale[blk], np.float64)
        cd = codes(c[blk], c_bits).astype(np.float64) * \
            (cs[..., None] if token_grain else cs[..., None, None])          # (n,kv,P,r)
        mud = mu[blk].astype(np.float64) * np.asarray(mu_scale[blk], np.float64)[..., None]
        qr = _q(q[rq], q_mode).reshape(n_kv, G, -1)
        qt = np.einsum("kgd,nkdr->nkgr", qr, Vd)
        tok = scale * np.einsum("nktr,nkgr->nkgt", cd, qt)
        pos = np.arange(n)[:, None] * page + np.arange(page)[None, :]
        tok = np.where((pos < int(seq_lens[rq]))[:, None, None, :], tok, -np.inf)
        m = tok.max(axis=-1, keepdims=True)
        lse = (m + np.log(np.exp(tok - m).sum(axis=-1, keepdims=True)))[..., 0]
        qsq = (qr * qr).sum(-1)                                             # (kv, G)
        qhsq = (qt * qt).sum(-1)                                            # (n, kv, G)
        iso = np.maximum(qsq[None] - qhsq, 0.0) * \
            np.asarray(resid[blk], np.float64)[..., None] * iso_coef
        S = scale * np.einsum("kgd,nkd->nkg", qr, mud) + lse + iso           # (n, kv, G)
        if combine == "max":
            out[rq, :, :n] = S.max(axis=-1).T
        else:
            out[rq, :, :, :n] = S.transpose(1, 2, 0)
    return out
