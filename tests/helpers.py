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


def rel_close(got, ref, tol):
    """|got - ref| <= tol * max(|ref|, 1) (the quad-score rule: relative error is
    ill-conditioned near 0)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref) / np.maximum(np.abs(ref), 1.0)
    return float(err.max()) if err.size else 0.0


def announce(msg: str) -> None:
    print(f"[gpu-test] {msg}", flush=True)
