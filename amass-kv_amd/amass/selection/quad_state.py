"""QuadState -- persistent buffers of the quad (Gaussian-MGF quadratic) selector.

Same tensors, dtypes and layout as the reference (``selection/quad_state.py:36-151``):

  quad_mu    (L, NB, n_kv, d)       int8   + mu_scale  (L, NB, n_kv)      fp16
  quad_V     (L, NB, n_kv, d, r')   int8   + V_scale   (L, NB, n_kv, r')  fp16 (per column)
             int4: (L, NB, n_kv, d, r'/2), byte = lo nibble (even column) | hi << 4
  quad_sig2  (L, NB, n_kv, r')      fp16   eigenvalues of the page's centred key scatter
  quad_tag   (L, NB, n_kv, TAGW)    bf16   NaN-init content tag

Per-step outputs are those of :class:`R8State`; combine="nrm" adds score_h
(R, n_kv, G, MP) and hmax (R, n_kv, G).  The physical-block-keyed slabs put all n_kv
heads of a page next to each other (8 KB for r'=8 int8 V), which is what lets one
gfx950 wave read a whole page's summaries with coalesced 16-byte loads.
"""
from __future__ import annotations

import torch

from .state import TAGW


class QuadState:
    def __init__(self, device, *, num_layers: int, num_blocks: int, n_kv: int, G: int,
                 head_dim: int, page: int, max_reqs: int, max_pages: int, rank: int = 2,
                 budget: float = 0.1, sink_pages: int = 1, window_pages: int = 1,
                 tagw: int = TAGW, v_grain: str = "col", v_bits: int = 8, mu_bits: int = 8,
                 coords: str = "none", c_bits: int = 4, c_grain: str = "token",
                 combine: str = "max"):
        if window_pages < 1:
            raise ValueError("window_pages must be >= 1 (the partial tail lives in the "
                             "always-attended window)")
        if v_grain not in ("col", "tensor"):
            raise ValueError(f"v_grain must be 'col' or 'tensor', got {v_grain!r}")
        if v_bits not in (4, 8) or mu_bits != 8:
            raise ValueError("quad V codes are int4 or int8; mu stays int8")
        if rank < 1 or (v_bits == 4 and rank % 2):
            raise ValueError(f"rank {rank} invalid for v_bits={v_bits}")
        if coords != "none":
            raise NotImplementedError(
                "score='clse' (per-key coords) is not part of this build's hot path")
        if combine not in ("max", "nrm"):
            raise ValueError(f"combine must be 'max' or 'nrm', got {combine!r}")
        L, NB, D, r, MP, R = num_layers, num_blocks, head_dim, rank, max_pages, max_reqs
        self.L, self.NB, self.n_kv, self.G, self.d = L, NB, n_kv, G, D
        self.D = D
        self.page, self.r, self.tagw = page, r, tagw
        self.max_reqs, self.max_pages = R, MP
        self.budget = float(budget)
        self.sink_pages, self.window_pages = int(sink_pages), int(window_pages)
        self.v_grain = v_grain
        self.v_bits, self.mu_bits = int(v_bits), 8
        self.coords, self.c_bits, self.c_grain = coords, int(c_bits), c_grain
        self.combine = combine
        self.device = device
        i8, f16, bf16 = torch.int8, torch.float16, torch.bfloat16
        i32, f32, f64 = torch.int32, torch.float32, torch.float64
        rv = r // 2 if v_bits == 4 else r
        self.quad_mu = torch.zeros(L, NB, n_kv, D, device=device, dtype=i8)
        self.mu_scale = torch.zeros(L, NB, n_kv, device=device, dtype=f16)
        self.quad_V = torch.zeros(L, NB, n_kv, D, rv, device=device, dtype=i8)
        self.V_scale = torch.zeros(L, NB, n_kv, r, device=device, dtype=f16)
        self.quad_sig2 = torch.zeros(L, NB, n_kv, r, device=device, dtype=f16)
        self.quad_tag = torch.full((L, NB, n_kv, tagw), float("nan"), device=device, dtype=bf16)
        self.quad_c = self.c_scale = self.quad_resid = None
        self.score = torch.empty(R, n_kv, MP, device=device, dtype=f32)
        self.page_table = torch.empty(R, n_kv, MP, device=device, dtype=i32)
        self.page_cnt = torch.zeros(R, n_kv, device=device, dtype=i32)
        self.n_sel = torch.zeros(R, n_kv, device=device, dtype=i32)
        if combine == "nrm":
            self.score_h = torch.empty(R, n_kv, G, MP, device=device, dtype=f32)
            self.hmax = torch.zeros(R, n_kv, G, device=device, dtype=f32)
        else:
            self.score_h = self.hmax = None
        self.n_pages = torch.zeros(R, device=device, dtype=i32)
        self.n_sel_hi = torch.zeros(R, device=device, dtype=i32)
        self.b_fix = torch.ones(R, device=device, dtype=i32)
        self.budget64 = torch.tensor([self.budget], device=device, dtype=f64)

    def bytes_per_layer(self) -> int:
        return (self.quad_mu[0].numel() + self.quad_V[0].numel()
                + 2 * (self.quad_sig2[0].numel() + self.mu_scale[0].numel()
                       + self.V_scale[0].numel() + self.quad_tag[0].numel()))

    def layer_state(self, layer: int):
        """(mu, mu_scale, V, V_scale, sig2, tag) views of ``layer``."""
        return (self.quad_mu[layer], self.mu_scale[layer], self.quad_V[layer],
                self.V_scale[layer], self.quad_sig2[layer], self.quad_tag[layer])

    def load_reference(self, layer: int, mu, mu_scale, V, V_scale, sig2) -> None:
        """Write one layer's summaries given in the reference layout
        (``selection/quad_state.py:36-151``: quad_V (NB, n_kv, d, r'[/2]))."""
        dev = self.quad_mu.device
        self.quad_mu[layer].copy_(torch.as_tensor(mu).to(dev))
        self.mu_scale[layer].copy_(torch.as_tensor(mu_scale).to(dev))
        self.quad_V[layer].copy_(torch.as_tensor(V).to(dev))
        self.V_scale[layer].copy_(torch.as_tensor(V_scale).to(dev))
        self.quad_sig2[layer].copy_(torch.as_tensor(sig2).to(dev))

    def reference_V(self, layer: int) -> torch.Tensor:
        """quad_V of ``layer`` in the reference layout (NB, n_kv, d, r'[/2])."""
        return self.quad_V[layer]
