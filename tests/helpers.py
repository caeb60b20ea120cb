"""Shared helpers for the GPU parity tests."""
from __future__ import annotations

import numpy as np
import torch


def to_device(obj, device):
    """Move every tensor attribute of a state object to `device` (in place)."""
    for k, v in list(vars(obj).items()):
        if isinstance(v, torch.Tensor):
            setattr(obj, k, v.to(device))
    obj.device = torch.device(device)
    return obj


def case_to(case, device):
    for k in ("q", "kv_cache", "block_table", "seq_lens"):
        setattr(case, k, getattr(case, k).to(device))
    return case


def npf(t):
    return t.detach().float().cpu().numpy()


def npi(t):
    return t.detach().cpu().numpy()


def rel_err(got, ref):
    """max |got - ref| / max(|ref|, 1) (the quad-score rule: relative error is
    ill-conditioned near 0); callers compare it with their tolerance."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref) / np.maximum(np.abs(ref), 1.0)
    return float(err.max()) if err.size else 0.0


def announce(msg: str) -> None:
    print(f"[gpu-test] {msg}", flush=True)


def exp_det_fused(x):
    """exp_det with every multiply-add fused into one rounding (an FMA), the form a
    compiler produces from `a * b + c` when contraction is on: a planted mistake for
    checking that a test tells the two apart (float64 holds the exact fp32 product)."""
    f32, f64 = np.float32, np.float64

    def fma(a, b, c):
        return (np.asarray(a, f64) * np.asarray(b, f64) + np.asarray(c, f64)).astype(f32)

    x = np.asarray(x, f32)
    out = np.zeros(x.shape, f32)
    m = x > f32(-80.0)
    xv = x[m]
    n = np.rint(xv * f32(float.fromhex("0x1.715476p+0"))).astype(f32)
    r = fma(n, -f32(float.fromhex("0x1.62e400p-1")), xv)
    r = fma(n, -f32(float.fromhex("0x1.7f7d1cp-20")), r)
    p = f32(float.fromhex("0x1.a01a02p-13"))
    for c in ("0x1.6c16c2p-10", "0x1.111112p-7", "0x1.555556p-5", "0x1.555556p-3",
              "0x1.000000p-1"):
        p = fma(p, r, f32(float.fromhex(c)))
    p = fma(p, r, f32(1.0))
    p = fma(p, r, f32(1.0))
    out[m] = np.ldexp(p, n.astype(np.int32)).astype(f32)
    return out


def mass_cut_case(exp_det, n_pages=64, k=10, sink=1, window=1):
    """Scores of one (request, kv head) whose coverage cut lies exactly on the exp mass of
    its top k + 1 pages: page 1 is the maximum (x = 0, mass exactly 1), pages 2..k+1 take
    values in (-0.7, -0.05) where `exp_det` and the fused form round differently (fused
    lower), every other scored page a value in (-5, -2) where they agree.  Returns
    (scores (n_pages,) float32, coverage): under `exp_det` the nucleus keeps exactly
    k + 1 selectable pages; with masses moved by an ulp it keeps another."""
    f32 = np.float32
    hi = np.linspace(-0.7, -0.05, 4001, dtype=f32)
    lo = np.linspace(-5.0, -2.0, 4001, dtype=f32)
    dif = hi[exp_det_fused(hi) < exp_det(hi)][:k]
    same = lo[exp_det_fused(lo) == exp_det(lo)]
    assert dif.size == k and same.size >= n_pages
    sc = same[np.linspace(0, same.size - 1, n_pages).astype(int)].copy()
    sc[sink] = f32(0.0)
    sc[sink + 1:sink + 1 + k] = dif
    nsh = n_pages - window
    w = (exp_det(sc[:nsh]).astype(np.float64) * 4294967296.0).astype(np.uint64)
    tot, snk = int(w.sum()), int(w[:sink].sum())
    cum = int(w[sink:sink + 1 + k].sum())
    cov = (cum + snk - 0.5) / tot
    return sc, cov
