"""Quantisation rules of the hot path (test oracle).

q_limbs   -- the 2-limb int8 query code of the reference's int kernels
             (selection/quad_score_cuda.py:902-935, selection/score_cuda.py:182-215):
             qs = max(amax|q|, 1e-12)/16383, qi = rn(q/qs) in [-16383, 16383],
             hi = rn(qi/128) in [-127, 127], lo = qi - 128 hi  (so 128 hi + lo == qi).
             The reference divides with --use_fast_math; this build fixes the rounding as
             m = max(amax, 1e-12), qs = m/16383 and inv = 16383/m (IEEE fp32 divides) and
             qi = rn(fp32(q * inv)).
quant     -- summary codes (selection/build.py:297-301): lvl = 2^(bits-1)-1,
             s = max(amax/lvl, 1e-8) fp32, code = clip(rint(x/s), -lvl, lvl).
pack_i4   -- selection/build.py:304-312: byte = lo nibble (even column) | hi << 4.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32


def bf16_round(x) -> np.ndarray:
    """Round float32 values to bf16 (nearest even), returned as float32."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32)


def q_limbs(q):
    """q (..., d) -> (qi int64, hi int64, lo int64, qs float32) per the reference recipe."""
    q = np.asarray(q, np.float32)
    m = np.maximum(np.abs(q).max(axis=-1), F32(1e-12)).astype(np.float32)
    qs = (m / F32(16383)).astype(np.float32)
    inv = (F32(16383) / m).astype(np.float32)
    qi = np.clip(np.rint((q * inv[..., None]).astype(np.float32)), -16383, 16383).astype(np.int64)
    hi = np.clip(np.rint(qi.astype(np.float32) * F32(0.0078125)), -127, 127).astype(np.int64)
    lo = np.clip(qi - 128 * hi, -127, 127)
    return qi, hi, lo, qs


def quant(x, axis, bits: int = 8):
    """(code int8, scale fp32 with keepdims) -- selection/build.py:297-301."""
    x = np.asarray(x, np.float32)
    lvl = F32((1 << (bits - 1)) - 1)
    s = np.maximum(np.abs(x).max(axis=axis, keepdims=True) / lvl, F32(1e-8)).astype(np.float32)
    code = np.clip(np.rint(x / s), -lvl, lvl).astype(np.int8)
    return code, s


def pack_i4(code):
    """(..., r) int8 in [-7, 7] -> (..., r/2) int8; lo nibble = even column."""
    c = np.asarray(code).astype(np.int32) & 0xF
    return (c[..., 0::2] | (c[..., 1::2] << 4)).astype(np.uint8).view(np.int8)


def unpack_i4(packed):
    """Inverse of pack_i4 -> (..., r) int8."""
    b = np.asarray(packed).view(np.uint8).astype(np.int32)
    lo, hi = b & 0xF, (b >> 4) & 0xF
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    out = np.stack([lo, hi], axis=-1)
    return out.reshape(*b.shape[:-1], b.shape[-1] * 2).astype(np.int8)


def codes(v, bits: int):
    """Stored V/Vk/c code tensor -> signed int8 codes (unpacking int4)."""
    return unpack_i4(v) if bits == 4 else np.asarray(v, np.int8)
