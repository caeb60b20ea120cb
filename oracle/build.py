"""Page-summary builder (test oracle): the quad and r8 summaries of finalised K pages.

Restates the reference builder's math (selection/quad_build.py:1-25,124-198;
selection/build.py:297-348 quantisation, :396-412 ``_page_eigh``, :415-450 ``_r8_write``)
in float64 numpy with LAPACK's symmetric eigensolver:

  mu = mean_t K ; dc = K - mu ; Gm = dc dc^T ; S2, U = eigh(Gm) ascending
  S2r = max(S2[-r:], 1e-10) ; U8 = U[:, -r:] ; S8 = sqrt(S2r)
  Vk = dc^T U8 / S8 (d, r) ; c = U8 S8 (page, r) ; sig2 = S2r
  codes: oracle.quant.quant (mu per head over d; Vk per column over d or per head;
  c per token over r or per head), int4 packed along r (oracle.quant.pack_i4).

Eigenvectors are defined up to sign (and up to rotation inside a repeated eigenvalue);
every score built from these factors is invariant to the sign (quad uses (Vk.q)^2,
r8 uses (Vk.q)(U8 S8)), so comparisons align column signs first.  Pinned in
tests/test_oracle_pins.py: exact reconstruction of pages of rank <= r (U8 S8 Vk^T == dc),
sig2 == squared singular values of dc, Vk orthonormal, and a hand-built rank-1 page.
"""
from __future__ import annotations

import numpy as np

from .quant import pack_i4, quant


def page_factors(K, rank: int):
    """K (N, page, n_kv, d) -> (mu, dc, S2r, U8, Vk), float64, each per (N, n_kv)."""
    Kp = np.asarray(K, np.float64).transpose(0, 2, 1, 3)          # (N, n_kv, page, d)
    mu = Kp.mean(axis=2)
    dc = Kp - mu[:, :, None, :]
    Gm = dc @ dc.swapaxes(-1, -2)
    S2, U = np.linalg.eigh(Gm)
    S2r = np.maximum(S2[..., -rank:], 1e-10)
    U8 = U[..., -rank:]
    Vk = dc.swapaxes(-1, -2) @ U8 / np.sqrt(S2r)[..., None, :]
    return mu, dc, S2r, U8, Vk


def _vk_codes(Vk, bits, grain):
    axis = -2 if grain == "col" else (-2, -1)
    code, s = quant(Vk.astype(np.float32), axis=axis, bits=bits)
    s = np.broadcast_to(s, Vk.shape[:-2] + (1, Vk.shape[-1]))[..., 0, :]
    return (pack_i4(code) if bits == 4 else code), s


def quad_summary(K, rank: int, v_bits: int = 8, v_grain: str = "col"):
    """-> dict(mu, mu_scale, V (reference layout (N, n_kv, d, r[/2])), V_scale, sig2),
    scales float32 before their fp16 storage."""
    mu, _dc, S2r, _U8, Vk = page_factors(K, rank)
    mu_code, mu_s = quant(mu.astype(np.float32), axis=-1, bits=8)
    V, Vs = _vk_codes(Vk, v_bits, v_grain)
    return dict(mu=mu_code, mu_scale=mu_s[..., 0], V=V, V_scale=Vs, sig2=S2r)


def r8_summary(K, rank: int, vk_bits: int = 8, c_bits: int = 8, vk_grain: str = "col",
               c_grain: str = "page"):
    """-> dict(mu, mu_scale, Vk, Vk_scale, c (N, n_kv, page, r[/2]), c_scale (N, n_kv, page)).
    c_grain "page": a scale per token; "tensor" and "page_f32": one scale per (block,
    head) over the page's coordinates (repeated per token here; stored fp16 by the
    reference's "tensor" layout, fp32 by the per-page fp32 layout)."""
    mu, _dc, S2r, U8, Vk = page_factors(K, rank)
    mu_code, mu_s = quant(mu.astype(np.float32), axis=-1, bits=8)
    V, Vs = _vk_codes(Vk, vk_bits, vk_grain)
    c = (U8 * np.sqrt(S2r)[..., None, :]).astype(np.float32)
    axis = -1 if c_grain == "page" else (-2, -1)
    c_code, cs = quant(c, axis=axis, bits=c_bits)
    cs = np.broadcast_to(cs, c.shape[:-1] + (1,))[..., 0]
    return dict(mu=mu_code, mu_scale=mu_s[..., 0], Vk=V, Vk_scale=Vs,
                c=pack_i4(c_code) if c_bits == 4 else c_code, c_scale=cs)


def clse_summary(K, rank: int, v_bits: int = 8, c_bits: int = 4, c_grain: str = "token",
                 v_grain: str = "col"):
    """CLSE summary (reference selection/quad_build.py:38-54 _clse_extras + the quad
    summary): quad's mu / V / V_scale, c = U8 S8 quantised per token ("token") or per
    (block, head) ("page"), resid = max(trace - sum S2r, 0) (the scatter energy outside
    the top-r' subspace; trace = the sum of all eigenvalues).  c_scale is (N, n_kv, page)
    for "token" and (N, n_kv) for "page"."""
    mu, dc, S2r, U8, Vk = page_factors(K, rank)
    out = quad_summary(K, rank, v_bits, v_grain)
    del out["sig2"]
    c = (U8 * np.sqrt(S2r)[..., None, :]).astype(np.float32)
    axis = -1 if c_grain == "token" else (-2, -1)
    c_code, cs = quant(c, axis=axis, bits=c_bits)
    out["c"] = pack_i4(c_code) if c_bits == 4 else c_code
    out["c_scale"] = cs[..., 0] if c_grain == "token" else cs[..., 0, 0]
    trace = (dc * dc).sum(axis=(-2, -1))
    out["resid"] = np.maximum(trace - S2r.sum(-1), 0.0)
    return out
