"""Seeded synthetic decode-step inputs for the BASELINE.json configurations.

Generator (written down, not tuned): K, V, q ~ N(0, 1) in bf16 from ``seed``.  For each
(sequence, kv-head) a fraction ``heavy`` of its pages (chosen uniformly without
replacement) is "boosted": every key of the page gets ``beta * u`` added, where u is the
unit vector of the mean of that kv-head's G group queries.  ``boost="sigma"`` reads the
config's "+2 sigma" literally (beta = 2, sigma_K = 1: about +1 logit per head);
``boost="keynorm"`` reads it in key-norm units (beta = 2 sqrt(d)).  Block tables:
"contiguous" (arange), "perm" (a random permutation of one shared pool), "pool" (random
distinct blocks of a pool larger than needed).  The paged cache uses vLLM's
(NB, 2, page, n_kv, d) layout.  Everything is generated with torch on ``device``.
"""
from __future__ import annotations

import dataclasses
import math
from typing import Optional

import torch

CONFIGS = {
    # config 0: B=1, ctx 4096, 8B GQA, fixed 5% budget (b = 13), quad r'=8
    0: dict(B=1, ctx=4096, n_kv=8, G=4, heavy=0.05, table="contiguous", score="quad",
            rank=8, budget=0.05, coverage=None),
    # config 1 (headline): B=32, ctx 16384, permuted pool, quad, coverage 0.95
    1: dict(B=32, ctx=16384, n_kv=8, G=4, heavy=0.05, table="perm", score="quad", rank=8,
            budget=None, coverage=0.95),
    # config 2: 64 ragged sequences in [2048, 65536], r8, fixed 5%
    2: dict(B=64, ctx=(2048, 65536), n_kv=8, G=4, heavy=0.05, table="pool", score="r8",
            rank=8, budget=0.05, coverage=None),
    # config 3: 70B shape (G=8), B=8, ctx 131072, 2% heavy, quad, coverage 0.95
    3: dict(B=8, ctx=131072, n_kv=8, G=8, heavy=0.02, table="perm", score="quad", rank=8,
            budget=None, coverage=0.95),
    # config 4: mem-v, B=32, ctx 32768, quad, coverage 0.95
    4: dict(B=32, ctx=32768, n_kv=8, G=4, heavy=0.05, table="perm", score="quad", rank=8,
            budget=None, coverage=0.95),
}


@dataclasses.dataclass
class Case:
    q: torch.Tensor            # (B, H, d) bf16
    kv_cache: torch.Tensor     # (NB, 2, page, n_kv, d) bf16
    block_table: torch.Tensor  # (B, max_blocks) int32
    seq_lens: torch.Tensor     # (B,) int32
    heavy_pages: torch.Tensor  # (B, n_kv, n_heavy_max) int64 logical pages (-1 pad)
    n_kv: int
    G: int
    d: int
    page: int
    max_pages: int
    scale: float
    meta: dict

    @property
    def K(self):
        return self.kv_cache[:, 0]

    @property
    def V(self):
        return self.kv_cache[:, 1]


def make_case(*, B: int, ctx, n_kv: int = 8, G: int = 4, d: int = 128, page: int = 16,
              heavy: float = 0.05, table: str = "perm", boost: str = "sigma",
              beta: Optional[float] = None, seed: int = 0, device="cpu",
              slack_blocks: int = 16, **_unused) -> Case:
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    cpu_gen = torch.Generator()
    cpu_gen.manual_seed(seed + 7919)
    if isinstance(ctx, tuple):
        lo, hi = ctx
        lens = torch.randint(lo, hi + 1, (B,), generator=cpu_gen)
        lens = ((lens + page - 1) // page) * page
    else:
        lens = torch.full((B,), int(ctx), dtype=torch.int64)
    npg = (lens + page - 1) // page
    max_pages = int(npg.max())
    total = int(npg.sum())
    NB = total + slack_blocks
    H = n_kv * G
    kv = torch.randn(NB, 2, page, n_kv, d, generator=gen, device=device, dtype=torch.float32)
    kv = kv.to(torch.bfloat16)
    q = torch.randn(B, H, d, generator=gen, device=device, dtype=torch.float32).to(torch.bfloat16)
    bt = torch.zeros(B, max_pages, dtype=torch.int32)
    if table == "contiguous":
        order = torch.arange(NB)
    elif table == "perm":
        order = torch.randperm(NB, generator=cpu_gen)
    elif table == "pool":
        order = torch.randperm(NB, generator=cpu_gen)
    else:
        raise ValueError(table)
    off = 0
    for r in range(B):
        n = int(npg[r])
        bt[r, :n] = order[off:off + n].to(torch.int32)
        off += n
    # heavy pages: per (seq, kv-head) a uniform subset of its pages
    nh_max = max(1, int(math.ceil(heavy * max_pages))) if heavy > 0 else 0
    heavy_pages = torch.full((B, n_kv, max(nh_max, 1)), -1, dtype=torch.int64)
    if heavy > 0:
        if beta is None:
            beta = 2.0 if boost == "sigma" else 2.0 * math.sqrt(d)
        qf = q.float().reshape(B, n_kv, G, d).mean(dim=2)
        u = qf / qf.norm(dim=-1, keepdim=True).clamp_min(1e-12)           # (B, n_kv, d)
        K32 = kv[:, 0].float()
        for r in range(B):
            n = int(npg[r])
            nh = max(1, int(math.ceil(heavy * n)))
            pick = torch.rand(n_kv, n, generator=cpu_gen).argsort(dim=1)[:, :nh]
            heavy_pages[r, :, :nh] = pick
            blk = bt[r, :n].to(torch.int64)[pick].to(device)              # (n_kv, nh)
            for kh in range(n_kv):
                K32[blk[kh], :, kh, :] += beta * u[r, kh]
        kv[:, 0] = K32.to(torch.bfloat16)
    return Case(q=q, kv_cache=kv, block_table=bt.to(device),
                seq_lens=lens.to(torch.int32).to(device), heavy_pages=heavy_pages,
                n_kv=n_kv, G=G, d=d, page=page, max_pages=max_pages, scale=d ** -0.5,
                meta=dict(B=B, ctx=ctx, heavy=heavy, table=table, boost=boost, beta=beta,
                          seed=seed, NB=NB))


def config_case(idx: int, *, seed: int = 0, device="cpu", boost: str = "sigma", **over) -> Case:
    cfg = dict(CONFIGS[idx])
    cfg.update(over)
    return make_case(seed=seed, device=device, boost=boost, **cfg)


def build_quad_state(case: Case, *, rank: int = 8, v_bits: int = 8, combine: str = "nrm",
                     budget: float = 0.1, coverage: Optional[float] = None, sink: int = 1,
                     window: int = 1, max_reqs: Optional[int] = None, coords: str = "none",
                     c_bits: int = 4, c_grain: str = "token"):
    """QuadState with layer 0 summarised from the case's K (the HIP builder for a device
    case, the torch builder for a host one); coords="lse" makes the CLSE state."""
    from ..selection import QuadState, quad_build_refresh
    from ..attention import ensure_stage_b_buffers
    dev = case.kv_cache.device
    st = QuadState(dev, num_layers=1, num_blocks=case.kv_cache.shape[0], n_kv=case.n_kv,
                   G=case.G, head_dim=case.d, page=case.page,
                   max_reqs=max_reqs or case.q.shape[0], max_pages=case.max_pages,
                   rank=rank, budget=budget, sink_pages=sink, window_pages=window,
                   v_bits=v_bits, combine=combine, coords=coords, c_bits=c_bits,
                   c_grain=c_grain)
    st.coverage = coverage
    st.scale = case.scale
    quad_build_refresh(st, 0, case.K, case.block_table, case.seq_lens, case.q.shape[0],
                       force=True)
    ensure_stage_b_buffers(st, dev)
    return st


def build_r8_state(case: Case, *, rank: int = 8, vk_bits: int = 8, c_bits: int = 8,
                   budget: float = 0.05, coverage: Optional[float] = None, sink: int = 1,
                   window: int = 1, c_grain: str = "page"):
    from ..selection import R8State, r8_build_refresh
    from ..attention import ensure_stage_b_buffers
    dev = case.kv_cache.device
    st = R8State(dev, num_layers=1, num_blocks=case.kv_cache.shape[0], n_kv=case.n_kv,
                 G=case.G, head_dim=case.d, page=case.page, max_reqs=case.q.shape[0],
                 max_pages=case.max_pages, rank=rank, budget=budget, sink_pages=sink,
                 window_pages=window, vk_bits=vk_bits, c_bits=c_bits, c_grain=c_grain)
    st.coverage = coverage
    st.scale = case.scale
    r8_build_refresh(st, 0, case.K, case.block_table, case.seq_lens, case.q.shape[0],
                     force=True)
    ensure_stage_b_buffers(st, dev)
    return st
