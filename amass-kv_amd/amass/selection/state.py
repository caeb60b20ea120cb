"""R8State -- persistent buffers of the r8 (low-rank per-key LSE) selector.

Same tensors, dtypes and layout as the reference (``selection/state.py:35-112``): every
buffer is allocated once from engine maxima so its address is stable across HIP-graph
replays.  Physical-block keyed, L-major summary slabs:

  r8_mu    (L, NB, n_kv, d)       int8   + mu_scale  (L, NB, n_kv)      fp16
  r8_Vk    (L, NB, n_kv, d, r)    int8   + Vk_scale  (L, NB, n_kv, r)   fp16   (int4: d, r/2)
  r8_c     (L, NB, n_kv, page, r) int8   + c_scale   (L, NB, n_kv, page) fp16  (int4: page, r/2)
  r8_tag   (L, NB, n_kv, TAGW)    bf16   NaN-init content tag

Per-step outputs (request-row keyed): score (R, n_kv, MP) fp32, page_table (R, n_kv, MP)
int32, page_cnt (R, n_kv) int32, n_pages / n_sel_hi / b_fix (R,) int32, budget64.
``n_sel`` (R, n_kv) int32 additionally receives the number of selectable pages chosen
per unit (diagnostic; the selected fraction of the coverage nucleus).
"""
from __future__ import annotations

import torch

TAGW = 8   # leading bf16 key channels of a page's last token = its content tag


class R8State:
    def __init__(self, device, *, num_layers: int, num_blocks: int, n_kv: int, G: int,
                 head_dim: int, page: int, max_reqs: int, max_pages: int, rank: int = 8,
                 budget: float = 0.1, sink_pages: int = 1, window_pages: int = 1,
                 tagw: int = TAGW, vk_grain: str = "col", c_grain: str = "page",
                 vk_bits: int = 8, c_bits: int = 8, mu_bits: int = 8):
        if window_pages < 1:
            raise ValueError("window_pages must be >= 1 (the partial tail lives in the "
                             "always-attended window)")
        if vk_grain not in ("col", "tensor") or c_grain not in ("page", "tensor"):
            raise ValueError(f"bad grain vk={vk_grain!r} c={c_grain!r}")
        if vk_bits not in (4, 8) or c_bits not in (4, 8) or mu_bits != 8:
            raise ValueError("Vk/c codes are int4 or int8; mu stays int8")
        L, NB, D, r, MP, R = num_layers, num_blocks, head_dim, rank, max_pages, max_reqs
        self.L, self.NB, self.n_kv, self.G, self.d = L, NB, n_kv, G, D
        self.D = D
        self.page, self.r, self.tagw = page, r, tagw
        self.max_reqs, self.max_pages = R, MP
        self.budget = float(budget)
        self.sink_pages, self.window_pages = int(sink_pages), int(window_pages)
        self.vk_grain, self.c_grain = vk_grain, c_grain
        self.vk_bits, self.c_bits, self.mu_bits = int(vk_bits), int(c_bits), 8
        self.device = device
        i8, f16, bf16 = torch.int8, torch.float16, torch.bfloat16
        i32, f32, f64 = torch.int32, torch.float32, torch.float64
        rvk = r // 2 if vk_bits == 4 else r
        rc = r // 2 if c_bits == 4 else r
        self.r8_mu = torch.zeros(L, NB, n_kv, D, device=device, dtype=i8)
        self.mu_scale = torch.zeros(L, NB, n_kv, device=device, dtype=f16)
        self.r8_Vk = torch.zeros(L, NB, n_kv, D, rvk, device=device, dtype=i8)
        self.Vk_scale = torch.zeros(L, NB, n_kv, r, device=device, dtype=f16)
        self.r8_c = torch.zeros(L, NB, n_kv, page, rc, device=device, dtype=i8)
        self.c_scale = torch.zeros(L, NB, n_kv, page, device=device, dtype=f16)
        self.r8_tag = torch.full((L, NB, n_kv, tagw), float("nan"), device=device, dtype=bf16)
        self.score = torch.empty(R, n_kv, MP, device=device, dtype=f32)
        self.page_table = torch.empty(R, n_kv, MP, device=device, dtype=i32)
        self.page_cnt = torch.zeros(R, n_kv, device=device, dtype=i32)
        self.n_sel = torch.zeros(R, n_kv, device=device, dtype=i32)
        self.n_pages = torch.zeros(R, device=device, dtype=i32)
        self.n_sel_hi = torch.zeros(R, device=device, dtype=i32)
        self.b_fix = torch.ones(R, device=device, dtype=i32)
        self.budget64 = torch.tensor([self.budget], device=device, dtype=f64)

    def bytes_per_layer(self) -> int:
        return (self.r8_mu[0].numel() + self.r8_Vk[0].numel() + self.r8_c[0].numel()
                + 2 * (self.mu_scale[0].numel() + self.Vk_scale[0].numel()
                       + self.c_scale[0].numel() + self.r8_tag[0].numel()))

    def layer_state(self, layer: int):
        """(mu, mu_scale, Vk, Vk_scale, c, c_scale, tag) views of ``layer``."""
        return (self.r8_mu[layer], self.mu_scale[layer], self.r8_Vk[layer],
                self.Vk_scale[layer], self.r8_c[layer], self.c_scale[layer],
                self.r8_tag[layer])
