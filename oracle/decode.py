"""Sparse / dense paged decode attention (test oracle).

attend       the textbook float64 softmax attention of each (request, q-head) over the
             tokens of its selected pages (positions >= seq_len masked) -- the math of
             attention/decode.py:128-241 without the split structure.
split_merge  restates the reference split-K schedule and merge: pps = max(cdiv(cnt, SPLIT),
             PPS_MIN), split s covers selected pages [s pps, min((s+1) pps, cnt)),
             per-split online softmax partials (m, l, acc) (decode.py:146-241), then
             m* = max m_s, w_s = exp(m_s - m*) [l_s > 0], out = sum w acc / sum w l, 0 for
             empty units (merge.py:21-50).  Equal to `attend` by split invariance.
"""
from __future__ import annotations

import numpy as np


def _unit_pages(r, kh, seq_len, page, page_table, page_cnt, dense):
    if dense:
        return np.arange((seq_len + page - 1) // page if seq_len > 0 else 0)
    return np.asarray(page_table[r, kh, :int(page_cnt[r, kh])], np.int64)


def _gather(K, V, bt_row, pages, kh, page, seq_len):
    blk = np.asarray(bt_row[pages], np.int64)
    k = np.asarray(K[blk, :, kh, :], np.float64).reshape(-1, K.shape[-1])
    v = np.asarray(V[blk, :, kh, :], np.float64).reshape(-1, V.shape[-1])
    pos = (pages[:, None] * page + np.arange(page)[None, :]).reshape(-1)
    valid = pos < seq_len
    k[~valid] = 0.0          # masked loads read zeros (decode.py:193-213, other=0.0)
    v[~valid] = 0.0
    return k, v, valid


def attend(q, K, V, block_table, seq_lens, page_table=None, page_cnt=None, *, scale, G,
           dense=False):
    """q (R, H, d); K, V (NB, page, n_kv, d) -> out (R, H, d) float64."""
    q = np.asarray(q, np.float64)
    R, H, d = q.shape
    page, n_kv = K.shape[1], K.shape[2]
    out = np.zeros((R, H, d))
    for r in range(R):
        sl = int(seq_lens[r])
        for kh in range(n_kv):
            pages = _unit_pages(r, kh, sl, page, page_table, page_cnt, dense)
            if pages.size == 0:
                continue
            k, v, valid = _gather(K, V, block_table[r], pages, kh, page, sl)
            for g in range(G):
                h = kh * G + g
                s = (k @ q[r, h]) * scale
                s = np.where(valid, s, -np.inf)
                m = s.max()
                p = np.exp(s - m)
                out[r, h] = (p @ v) / p.sum()
    return out


def split_merge(q, K, V, block_table, seq_lens, page_table, page_cnt, *, scale, G, split,
                pps_min):
    q = np.asarray(q, np.float64)
    R, H, d = q.shape
    page, n_kv = K.shape[1], K.shape[2]
    out = np.zeros((R, H, d))
    for r in range(R):
        sl = int(seq_lens[r])
        for kh in range(n_kv):
            cnt = int(page_cnt[r, kh])
            pps = max(-(-cnt // split), pps_min)
            parts = []
            for sp in range(split):
                j0 = sp * pps
                if j0 >= cnt:
                    break
                j1 = min(j0 + pps, cnt)
                m = np.full(G, -np.inf)
                l = np.zeros(G)
                acc = np.zeros((G, d))
                for j in range(j0, j1):
                    pt = int(page_table[r, kh, j])
                    k, v, valid = _gather(K, V, block_table[r], np.array([pt]), kh, page, sl)
                    s = (q[r, kh * G:(kh + 1) * G] @ k.T) * scale
                    s = np.where(valid[None, :], s, -np.inf)
                    mn = np.maximum(m, s.max(axis=1))
                    alpha = np.exp(m - mn)
                    p = np.exp(s - mn[:, None])
                    l = l * alpha + p.sum(axis=1)
                    acc = acc * alpha[:, None] + p @ v
                    m = mn
                parts.append((m, l, acc))
            if not parts:
                continue
            ms = np.stack([p[0] for p in parts])
            ls = np.stack([p[1] for p in parts])
            accs = np.stack([p[2] for p in parts])
            mstar = ms.max(axis=0)
            w = np.where(ls > 0, np.exp(ms - mstar), 0.0)
            lt = (ls * w).sum(axis=0)
            o = (accs * w[:, :, None]).sum(axis=0)
            out[r, kh * G:(kh + 1) * G] = np.where(lt[:, None] > 0, o / lt[:, None], 0.0)
    return out
