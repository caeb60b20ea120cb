"""QuadState -- persistent buffers of the quad (Gaussian-MGF quadratic) selector.

The reference (``selection/quad_state.py:36-151``) keeps five slabs per layer; this
build packs them into one block-keyed buffer and exposes the reference's names as views
into it.  Per (layer, block), REC = r' * CB + 176 bytes per kv head:

  quad_rec   (L, NB, n_kv * REC)  int8, per block:
    n_kv records of VM = r' * CB + 128 bytes, head h at h * VM:
      quad_V   (L, NB, n_kv, r', CB) int8  (r' * CB bytes) tiled for the score kernel's
               column groups: 16 bytes per (K-step t, d group kg, column k) at
               ((t * 4 + kg) * r' + k) * 16, byte i = code[64 t + 16 kg + i]; int8 CB = d,
               int4 CB = d/2 with byte i of (kg, k) = code[16 kg + i] | code[16 kg + i + 64] << 4
               (the reference keeps (.., d, r') with two columns per int4 byte)
      quad_mu  (L, NB, n_kv, d)      int8  page-mean codes
    then n_kv scale blocks of 48 bytes (fp16 halves), head h at n_kv * VM + 48 h:
      V_scale  (L, NB, n_kv, r')     half 0..r'-1
      quad_sig2(L, NB, n_kv, r')     half 8..8+r'-1 (eigenvalues of the centred key scatter)
      mu_scale (L, NB, n_kv)         half 16; the other halves are zero
  quad_tag   (L, NB, n_kv, TAGW)  bf16  NaN-init content tag (separate)

Every V / mu record is whole 128-byte lines and a block's n_kv records are contiguous.
The tiled V lets the gfx950 score kernel feed an int8 matrix-core instruction whose 16
columns are 16 / r' pages x r' ranks with loads that each read 64 r' contiguous bytes
of every page they touch.  ``v_to_device`` / ``v_to_reference`` convert V between this
and the reference layout; ``load_reference`` and ``reference_V`` use them.  CLSE and
the r8 records keep V in the same tiled order.

CLSE (``coords="lse"``, the reference's ``score="clse"``) keeps the per-key coordinates
and the residual scatter energy instead of sig2, in its own record
(AMASS_CLSE_REC_BYTES = VQ + TB per head): the n_kv heads' ``[quad_V tiled | quad_mu]``
(VQ = r' * CB + 128 bytes, whole lines, as above), then per head a tail of
TB = 16 * rc + 16 * ceil((36 + 2 r') / 16) bytes at n_kv * VQ + TB * h:
``quad_c (page, rc)`` (rc = r' or r'/2 bytes per token row), then fp16 halves c_scale
0..15 (``c_grain="page"``: one scale per (block, head), kept in all 16 halves and exposed
as half 0), V_scale at half 16, mu_scale at half 16 + r' and quad_resid at half
17 + r', zero to the end (320 bytes per head at r' = 2 with int4 V and c, against 336 in
the r8 layout with its 64-byte scale block); ``quad_sig2`` is None there.

Per-step outputs are those of :class:`R8State`; combine="nrm" adds score_h
(R, n_kv, G, MP) and score_tmax (R, n_kv, G, ceil(MP / 16)), the per-16-page-tile
per-head maxima the score launch writes beside score_h for the fused nrm combine, and
unit_tickets (R * n_kv,), the zero-at-rest counters of the per-unit pipeline.
"""
from __future__ import annotations

import torch

from .state import TAGW


def _unpack_pairs(packed: torch.Tensor) -> torch.Tensor:
    b = packed.view(torch.uint8).to(torch.int32)
    lo, hi = b & 0xF, (b >> 4) & 0xF
    lo = torch.where(lo >= 8, lo - 16, lo)
    hi = torch.where(hi >= 8, hi - 16, hi)
    return lo, hi


def _tile(col: torch.Tensor, v_bits: int) -> torch.Tensor:
    """Column-major (..., r', CB) -> the quad kernel's tiled bytes, same shape: 16 bytes
    per (K-step t, d group kg, column k) at ((t * 4 + kg) * r' + k) * 16, d = 64 t + 16 kg
    + i (int4: byte i of (kg, k) packs d = 16 kg + i and d + 64, so t is folded)."""
    *lead, r, cb = col.shape
    nl = len(lead)
    if v_bits == 8:
        t = col.reshape(*lead, r, 2, 4, 16).permute(*range(nl), nl + 1, nl + 2, nl, nl + 3)
    else:
        t = col.reshape(*lead, r, 4, 16).permute(*range(nl), nl + 1, nl, nl + 2)
    return t.reshape(*lead, r, cb).contiguous()


def _untile(tiled: torch.Tensor, v_bits: int) -> torch.Tensor:
    """Inverse of :func:`_tile`."""
    *lead, r, cb = tiled.shape
    nl = len(lead)
    if v_bits == 8:
        c = tiled.reshape(*lead, 2, 4, r, 16).permute(*range(nl), nl + 2, nl, nl + 1, nl + 3)
    else:
        c = tiled.reshape(*lead, 4, r, 16).permute(*range(nl), nl + 1, nl, nl + 2)
    return c.reshape(*lead, r, cb).contiguous()


def v_to_device(v_ref: torch.Tensor, v_bits: int, tiled: bool = False) -> torch.Tensor:
    """Reference quad_V (..., d, r') int8 or (..., d, r'/2) packed int4 (lo nibble = even
    column) -> the kernel layout: column-major (..., r', d) int8 or (..., r', d/2) packed
    halves (r8, CLSE), or those bytes tiled for the quad kernel (``tiled``)."""
    if v_bits == 8:
        col = v_ref.transpose(-1, -2).contiguous()
        return _tile(col, v_bits) if tiled else col
    lo, hi = _unpack_pairs(v_ref)                       # columns 2c, 2c+1
    code = torch.stack([lo, hi], dim=-1).flatten(-2)    # (..., d, r')
    code = code.transpose(-1, -2)                       # (..., r', d)
    half = code.shape[-1] // 2
    packed = (code[..., :half] & 0xF) | ((code[..., half:] & 0xF) << 4)
    col = packed.to(torch.uint8).view(torch.int8).contiguous()
    return _tile(col, v_bits) if tiled else col


def v_to_reference(v_dev: torch.Tensor, v_bits: int, tiled: bool = False) -> torch.Tensor:
    """Inverse of :func:`v_to_device`."""
    if tiled:
        v_dev = _untile(v_dev, v_bits)
    if v_bits == 8:
        return v_dev.transpose(-1, -2).contiguous()
    lo, hi = _unpack_pairs(v_dev)                       # d = j, j + d/2
    code = torch.cat([lo, hi], dim=-1)                  # (..., r', d)
    code = code.transpose(-1, -2)                       # (..., d, r')
    packed = (code[..., 0::2] & 0xF) | ((code[..., 1::2] & 0xF) << 4)
    return packed.to(torch.uint8).view(torch.int8).contiguous()


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
        if coords not in ("none", "lse"):
            raise ValueError(f"coords must be 'none' or 'lse', got {coords!r}")
        if coords == "lse" and (c_bits not in (4, 8) or c_grain not in ("token", "page")
                                or (c_bits == 4 and rank % 2)):
            raise ValueError(f"CLSE coords: c_bits 4|8, c_grain token|page (got {c_bits}, "
                             f"{c_grain!r}; int4 needs an even rank)")
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
        self.v_tiled = True                               # the score kernels' V layout
        self.combine = combine
        self.device = device
        i8, f16, bf16 = torch.int8, torch.float16, torch.bfloat16
        i32, f32, f64 = torch.int32, torch.float32, torch.float64
        if r > 8 or D != 128 or (coords == "lse" and page != 16):
            raise ValueError("the packed quad record holds r' <= 8 columns of d = 128 "
                             "(and 16-token pages with CLSE coordinates)")
        cb = D // 2 if v_bits == 4 else D
        vb = r * cb
        vm = vb + D                                       # V + mu bytes per head
        if coords == "lse":
            rc = r // 2 if c_bits == 4 else r             # c bytes per token row
            tb = page * rc + 16 * ((36 + 2 * r + 15) // 16)   # the head's tail
        else:
            tb = 48                                       # the head's scale block
        self.rec_bytes = vm + tb
        self.quad_rec = torch.zeros(L, NB, n_kv * self.rec_bytes, device=device, dtype=i8)
        recs = self.quad_rec[..., :n_kv * vm].unflatten(-1, (n_kv, vm))
        tails = self.quad_rec[..., n_kv * vm:].unflatten(-1, (n_kv, tb))
        self.quad_V = recs[..., :vb].unflatten(-1, (r, cb))
        self.quad_mu = recs[..., vb:vb + D]
        self.quad_tag = torch.full((L, NB, n_kv, tagw), float("nan"), device=device, dtype=bf16)
        if coords == "lse":
            self.quad_c = tails[..., :page * rc].unflatten(-1, (page, rc))
            sp = tails[..., page * rc:].view(f16)         # the tail's scale halves
            self._c_scale16 = sp[..., 0:page]
            self.c_scale = self._c_scale16 if c_grain == "token" else sp[..., 0]
            self.V_scale = sp[..., 16:16 + r]
            self.mu_scale = sp[..., 16 + r]
            self.quad_resid = sp[..., 17 + r]
            self.quad_sig2 = None
        else:
            meta = tails.view(f16)
            self.V_scale = meta[..., 0:r]
            self.quad_sig2 = meta[..., 8:8 + r]
            self.mu_scale = meta[..., 16]
            self.quad_c = self.c_scale = self.quad_resid = self._c_scale16 = None
        self.score = torch.empty(R, n_kv, MP, device=device, dtype=f32)
        self.page_table = torch.empty(R, n_kv, MP, device=device, dtype=i32)
        self.page_cnt = torch.zeros(R, n_kv, device=device, dtype=i32)
        self.n_sel = torch.zeros(R, n_kv, device=device, dtype=i32)
        if combine == "nrm":
            self.score_h = torch.empty(R, n_kv, G, MP, device=device, dtype=f32)
            self.score_tmax = torch.empty(R, n_kv, G, (MP + 15) // 16, device=device,
                                          dtype=f32)
            # the per-unit pipeline's tickets (several workgroups per unit): zero at rest
            self.unit_tickets = torch.zeros(R * n_kv, device=device, dtype=i32)
        else:
            self.score_h = self.score_tmax = self.unit_tickets = None
        self.n_pages = torch.zeros(R, device=device, dtype=i32)
        self.n_sel_hi = torch.zeros(R, device=device, dtype=i32)
        self.b_fix = torch.ones(R, device=device, dtype=i32)
        self.budget64 = torch.tensor([self.budget], device=device, dtype=f64)

    def bytes_per_layer(self) -> int:
        return self.quad_rec[0].numel() + 2 * self.quad_tag[0].numel()

    def layer_state(self, layer: int):
        """(mu, mu_scale, V, V_scale, sig2, tag) views of ``layer`` (V tiled)."""
        sig2 = self.quad_sig2[layer] if self.quad_sig2 is not None else None   # None: CLSE
        return (self.quad_mu[layer], self.mu_scale[layer], self.quad_V[layer],
                self.V_scale[layer], sig2, self.quad_tag[layer])

    def load_reference(self, layer: int, mu, mu_scale, V, V_scale, sig2=None, c=None,
                       c_scale=None, resid=None) -> None:
        """Write one layer's summaries given in the reference layout
        (``selection/quad_state.py:36-151``: quad_V (NB, n_kv, d, r'[/2]); CLSE adds
        quad_c (NB, n_kv, page, r'[/2]), c_scale (token: (NB, n_kv, page), page:
        (NB, n_kv)) and quad_resid (NB, n_kv))."""
        dev = self.quad_mu.device
        t = lambda x: torch.as_tensor(x).to(dev)  # noqa: E731
        self.quad_mu[layer].copy_(t(mu))
        self.mu_scale[layer].copy_(t(mu_scale))
        self.quad_V[layer].copy_(v_to_device(t(V), self.v_bits, tiled=self.v_tiled))
        self.V_scale[layer].copy_(t(V_scale))
        if self.coords == "lse":
            self.quad_c[layer].copy_(t(c))
            cs = t(c_scale)
            self._c_scale16[layer].copy_(cs if self.c_grain == "token"
                                         else cs[..., None].expand_as(self._c_scale16[layer]))
            self.quad_resid[layer].copy_(t(resid))
        else:
            self.quad_sig2[layer].copy_(t(sig2))

    def reference_V(self, layer: int) -> torch.Tensor:
        """quad_V of ``layer`` in the reference layout (NB, n_kv, d, r'[/2])."""
        return v_to_reference(self.quad_V[layer], self.v_bits, tiled=self.v_tiled)
