"""R8State -- persistent buffers of the r8 (low-rank per-key LSE) selector.

Every buffer is allocated once from engine maxima so its address is stable across
HIP-graph replays.  The reference (``selection/state.py:35-112``) keeps six summary slabs
per layer; this build packs them into one block-keyed buffer and exposes the reference's
names as views into it.  Per (layer, block), REC = r*CB + 128 + 16*r*c_bits/8 + 64 bytes
per kv head:

  r8_rec   (L, NB, n_kv * REC)  int8, per block:
    n_kv records of VM = r*CB + 128 + 16*r*c_bits/8 bytes, head h at h * VM:
      r8_Vk    (L, NB, n_kv, r, CB)   int8  (r * CB bytes) tiled like quad_V: 16 bytes per
               (K-step t, d group kg, column k) at ((t * 4 + kg) * r + k) * 16, byte i =
               code[64 t + 16 kg + i]; int8 CB = d, int4 CB = d/2 with byte i of (kg, k) =
               code[16 kg + i] | code[16 kg + i + 64] << 4
               (the reference keeps (.., d, r) with two columns per int4 byte)
      r8_mu    (L, NB, n_kv, d)       int8  page-mean codes
      r8_c     (L, NB, n_kv, page, r) int8  per-key coordinates (int4: (.., page, r/2),
               low nibble = even column, as in the reference)
    then n_kv scale blocks of 64 bytes (fp16 halves), head h at n_kv * VM + 64 h:
      Vk_scale (L, NB, n_kv, r)       half 0..r-1
      c_scale  (L, NB, n_kv, page)    half 8..23 (c_grain "page" / "tensor")
      c_scale_f32 (L, NB, n_kv)       fp32 at bytes 16..19 (c_grain "page_f32": one fp32 c
               scale per page, config 2's per-page fp32 scale; halves 10..23 zero)
      mu_scale (L, NB, n_kv)          half 24; the other halves are zero
  r8_tag   (L, NB, n_kv, TAGW)  bf16  NaN-init content tag (separate)

A block's records are contiguous and the score kernel's loads each read 64 r contiguous
Vk bytes of every page they touch, fed straight into int8 matrix-core instructions (the
quad record's reasoning, :mod:`amass.selection.quad_state`).  ``reference_Vk`` /
``load_reference`` convert Vk between this and the reference layout.

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
        if vk_grain not in ("col", "tensor") or c_grain not in ("page", "tensor", "page_f32"):
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
        if D != 128 or page != 16 or not 1 <= r <= 8 or (4 in (vk_bits, c_bits) and r % 2):
            raise ValueError("the packed r8 record holds r <= 8 columns of d = 128 and "
                             "16-token pages (r even for int4 codes)")
        cb = D // 2 if vk_bits == 4 else D
        rc = r // 2 if c_bits == 4 else r
        vb, cbytes = r * cb, page * rc
        vm = vb + D + cbytes                              # Vk + mu + c bytes per head
        self.rec_bytes = vm + 64                          # + the head's scale block
        self.r8_rec = torch.zeros(L, NB, n_kv * self.rec_bytes, device=device, dtype=i8)
        recs = self.r8_rec[..., :n_kv * vm].unflatten(-1, (n_kv, vm))
        meta = self.r8_rec[..., n_kv * vm:].unflatten(-1, (n_kv, 64)).view(f16)
        self.r8_Vk = recs[..., :vb].unflatten(-1, (r, cb))
        self.r8_mu = recs[..., vb:vb + D]
        self.r8_c = recs[..., vb + D:].unflatten(-1, (page, rc))
        self.Vk_scale = meta[..., 0:r]
        self.c_scale = meta[..., 8:8 + page]
        self.c_scale_f32 = meta.view(f32)[..., 4]
        self.mu_scale = meta[..., 24]
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
        return self.r8_rec[0].numel() + 2 * self.r8_tag[0].numel()

    def layer_state(self, layer: int):
        """(mu, mu_scale, Vk, Vk_scale, c, c_scale, tag) of ``layer`` (views; Vk tiled,
        :meth:`reference_Vk` gives the reference layout).  c_scale is per token: for
        c_grain "page_f32" the page's fp32 scale broadcast over its tokens (a copy)."""
        return (self.r8_mu[layer], self.mu_scale[layer], self.r8_Vk[layer],
                self.Vk_scale[layer], self.r8_c[layer], self.token_c_scale(layer),
                self.r8_tag[layer])

    def token_c_scale(self, layer: int) -> torch.Tensor:
        """The c scale of every token (L=layer: (NB, n_kv, page)): the stored fp16 slots,
        or the fp32 per-page scale repeated over the page."""
        if self.c_grain == "page_f32":
            cs = self.c_scale_f32[layer]
            return cs[..., None].expand(*cs.shape, self.page)
        return self.c_scale[layer]

    def load_reference(self, layer: int, mu, mu_scale, Vk, Vk_scale, c, c_scale) -> None:
        """Write one layer's summaries given in the reference layout
        (``selection/state.py:35-112``: r8_Vk (NB, n_kv, d, r[/2]))."""
        from .quad_state import v_to_device
        dev = self.r8_rec.device
        self.r8_mu[layer].copy_(torch.as_tensor(mu).to(dev))
        self.mu_scale[layer].copy_(torch.as_tensor(mu_scale).to(dev))
        self.r8_Vk[layer].copy_(v_to_device(torch.as_tensor(Vk).to(dev), self.vk_bits,
                                            tiled=True))
        self.Vk_scale[layer].copy_(torch.as_tensor(Vk_scale).to(dev))
        self.r8_c[layer].copy_(torch.as_tensor(c).to(dev))
        if self.c_grain == "page_f32":      # c_scale (NB, n_kv) fp32 per page
            self.c_scale_f32[layer].copy_(torch.as_tensor(c_scale).to(dev))
        else:
            self.c_scale[layer].copy_(torch.as_tensor(c_scale).to(dev))

    def reference_Vk(self, layer: int) -> torch.Tensor:
        """r8_Vk of ``layer`` in the reference layout (NB, n_kv, d, r[/2])."""
        from .quad_state import v_to_reference
        return v_to_reference(self.r8_Vk[layer], self.vk_bits, tiled=True)
