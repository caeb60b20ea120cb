"""quad_V layouts of the gfx950 score kernels vs the reference layout (column-major for
r8 / CLSE records, tiled for the quad kernel).

The kernel reads quad_V as (.., r', d) int8 or (.., r', d/2) int4 with byte
j = code[j] | code[j + d/2] << 4; the reference stores (.., d, r') int8 or (.., d, r'/2)
int4 with two columns per byte (selection/build.py:304-312).  The converters must be
exact inverses and place every code where the kernel's lane mapping expects it.
"""
import numpy as np
import pytest
import torch

import oracle.quant as oq
from amass.selection import QuadState
from amass.selection.quad_state import v_to_device, v_to_reference


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("r", [2, 4, 8])
def test_round_trip_and_positions(bits, r):
    g = torch.Generator().manual_seed(r * 10 + bits)
    lvl = 127 if bits == 8 else 7
    code = torch.randint(-lvl, lvl + 1, (3, 2, 128, r), generator=g, dtype=torch.int8)
    ref = code if bits == 8 else torch.from_numpy(oq.pack_i4(code.numpy()))
    dev = v_to_device(ref, bits)
    assert torch.equal(v_to_reference(dev, bits), ref)
    if bits == 8:
        assert dev.shape == (3, 2, r, 128)
        assert torch.equal(dev[1, 1, r - 1, 77], code[1, 1, 77, r - 1])
    else:
        assert dev.shape == (3, 2, r, 64)
        b = int(dev[2, 0, r - 1, 5].view(torch.uint8))
        lo, hi = b & 0xF, b >> 4
        lo, hi = (lo - 16 if lo >= 8 else lo), (hi - 16 if hi >= 8 else hi)
        assert lo == int(code[2, 0, 5, r - 1]) and hi == int(code[2, 0, 69, r - 1])


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("r", [2, 4, 8])
def test_tiled_round_trip_and_positions(bits, r):
    """The quad kernel's tiled V: 16 bytes per (K-step t, d group kg, column k) at
    ((t * 4 + kg) * r + k) * 16, byte i = code[64 t + 16 kg + i] (int4: t folded into the
    nibbles of (kg, k)); every code checked against that formula."""
    g = torch.Generator().manual_seed(r * 10 + bits + 1)
    lvl = 127 if bits == 8 else 7
    code = torch.randint(-lvl, lvl + 1, (2, 3, 128, r), generator=g, dtype=torch.int8)
    ref = code if bits == 8 else torch.from_numpy(oq.pack_i4(code.numpy()))
    dev = v_to_device(ref, bits, tiled=True)
    assert torch.equal(v_to_reference(dev, bits, tiled=True), ref)
    flat = dev.reshape(2, 3, -1).view(torch.uint8).to(torch.int32)
    for d in range(128):
        for k in range(r):
            t, kg, i = d // 64, (d % 64) // 16, d % 16
            if bits == 8:
                got = flat[..., ((t * 4 + kg) * r + k) * 16 + i]
                got = torch.where(got >= 128, got - 256, got)
            else:
                b = flat[..., (kg * r + k) * 16 + i]
                nib = (b >> (4 * t)) & 0xF
                got = torch.where(nib >= 8, nib - 16, nib)
            assert torch.equal(got, code[..., d, k].to(torch.int32)), (d, k)


def test_state_load_reference_round_trip():
    st = QuadState("cpu", num_layers=2, num_blocks=5, n_kv=2, G=4, head_dim=128, page=16,
                   max_reqs=1, max_pages=4, rank=4, v_bits=4)
    rng = np.random.default_rng(0)
    code = rng.integers(-7, 8, (5, 2, 128, 4)).astype(np.int8)
    V = oq.pack_i4(code)
    mu = rng.integers(-127, 128, (5, 2, 128)).astype(np.int8)
    h = np.ones((5, 2), np.float16)
    st.load_reference(1, mu, h, V, np.ones((5, 2, 4), np.float16),
                      np.ones((5, 2, 4), np.float16))
    assert np.array_equal(st.reference_V(1).numpy(), V)
    assert not st.quad_V[0].any()



@pytest.mark.parametrize("v_bits,r", [(8, 8), (4, 8), (8, 4), (4, 2), (8, 2)])
def test_quad_record_positions(v_bits, r):
    """The packed quad record (include/amass_hip.h, AMASS_QUAD_REC_BYTES): per block the
    n_kv heads' [V tiled | mu] at h * VM (whole 128-byte lines), then 48-byte fp16 scale
    blocks at n_kv * VM + 48 h with V_scale at half 0, sig2 at half 8, mu_scale at half 16
    and zeros to the end.  Every field is checked at that offset in the raw buffer."""
    n_kv, NB = 3, 4
    st = QuadState("cpu", num_layers=1, num_blocks=NB, n_kv=n_kv, G=4, head_dim=128,
                   page=16, max_reqs=1, max_pages=4, rank=r, v_bits=v_bits)
    cb = 128 if v_bits == 8 else 64
    vm = r * cb + 128
    rec_bytes = r * cb + 176                                # AMASS_QUAD_REC_BYTES
    assert vm % 128 == 0 and st.rec_bytes == rec_bytes == vm + 48
    assert st.quad_rec.shape[-1] == n_kv * rec_bytes
    rng = np.random.default_rng(r * 10 + v_bits)
    lv = 127 if v_bits == 8 else 7
    vcode = rng.integers(-lv, lv + 1, (NB, n_kv, 128, r)).astype(np.int8)
    V = vcode if v_bits == 8 else oq.pack_i4(vcode)
    mu = rng.integers(-127, 128, (NB, n_kv, 128)).astype(np.int8)
    mus = (rng.random((NB, n_kv)) + 0.5).astype(np.float16)
    vs = (rng.random((NB, n_kv, r)) + 0.5).astype(np.float16)
    sg = (rng.random((NB, n_kv, r)) + 0.5).astype(np.float16)
    st.load_reference(0, mu, mus, V, vs, sg)
    raw = st.quad_rec[0].numpy().view(np.uint8)
    for b in range(NB):
        for h in range(n_kv):
            base = h * vm
            if v_bits == 8:               # d = 77: K-step 1, d group 0, byte 13
                off = ((1 * 4 + 0) * r + (r - 1)) * 16 + 13
                assert raw[b, base + off].view(np.int8) == vcode[b, h, 77, r - 1]
            assert np.array_equal(raw[b, base + r * cb: base + vm].view(np.int8), mu[b, h])
            meta = raw[b, n_kv * vm + 48 * h: n_kv * vm + 48 * (h + 1)].view(np.float16)
            assert np.array_equal(meta[:r], vs[b, h]) and not meta[r:8].any()
            assert np.array_equal(meta[8:8 + r], sg[b, h]) and not meta[8 + r:16].any()
            assert meta[16] == mus[b, h] and not meta[17:].any()


@pytest.mark.parametrize("vk_bits,c_bits,r", [(8, 8, 8), (4, 4, 8), (8, 4, 4), (4, 8, 4)])
def test_r8_record_positions(vk_bits, c_bits, r):
    """The packed r8 record (include/amass_hip.h, AMASS_R8_REC_BYTES): per block the n_kv
    heads' [Vk tiled | mu | c rows], then 64-byte fp16 scale blocks with Vk_scale
    at half 0, c_scale at halves 8..23, mu_scale at half 24.  Bytes are checked at their
    documented offsets in the raw buffer, so a view that drifts from the kernel's
    addressing fails here."""
    from amass.selection import R8State
    n_kv, NB = 2, 3
    st = R8State("cpu", num_layers=1, num_blocks=NB, n_kv=n_kv, G=4, head_dim=128, page=16,
                 max_reqs=1, max_pages=4, rank=r, vk_bits=vk_bits, c_bits=c_bits)
    cb = 128 if vk_bits == 8 else 64
    crow = r * c_bits // 8
    vm = r * cb + 128 + 16 * crow
    rec_bytes = r * cb + 128 + 2 * r * c_bits + 64          # AMASS_R8_REC_BYTES
    assert st.rec_bytes == rec_bytes == vm + 64 and st.r8_rec.shape[-1] == n_kv * rec_bytes
    rng = np.random.default_rng(r + vk_bits)
    lv = 127 if vk_bits == 8 else 7
    vcode = rng.integers(-lv, lv + 1, (NB, n_kv, 128, r)).astype(np.int8)
    Vk = vcode if vk_bits == 8 else oq.pack_i4(vcode)
    lc = 127 if c_bits == 8 else 7
    ccode = rng.integers(-lc, lc + 1, (NB, n_kv, 16, r)).astype(np.int8)
    c = ccode if c_bits == 8 else oq.pack_i4(ccode)
    mu = rng.integers(-127, 128, (NB, n_kv, 128)).astype(np.int8)
    mus = rng.random((NB, n_kv)).astype(np.float16)
    vks = rng.random((NB, n_kv, r)).astype(np.float16)
    cs = rng.random((NB, n_kv, 16)).astype(np.float16)
    st.load_reference(0, mu, mus, Vk, vks, c, cs)
    assert np.array_equal(st.reference_Vk(0).numpy(), Vk)
    raw = st.r8_rec[0].numpy().view(np.uint8)               # (NB, n_kv * REC)
    b, h, k, j, t = 2, 1, r - 1, 77, 13
    base = h * vm
    if vk_bits == 8:                  # d = 77: K-step 1, d group 0, byte 13
        off = ((1 * 4 + 0) * r + k) * 16 + 13
        assert raw[b, base + off].view(np.int8) == vcode[b, h, j, k]
    else:                             # d = 13 and 77 share byte 13 of (kg 0, column k)
        byte = int(raw[b, base + k * 16 + 13])
        lo, hi = byte & 0xF, byte >> 4
        assert (lo - 16 if lo >= 8 else lo) == vcode[b, h, 13, k]
        assert (hi - 16 if hi >= 8 else hi) == vcode[b, h, 13 + 64, k]
    assert raw[b, base + r * cb + j].view(np.int8) == mu[b, h, j]
    crow_bytes = raw[b, base + r * cb + 128 + t * crow: base + r * cb + 128 + (t + 1) * crow]
    assert np.array_equal(crow_bytes.view(np.int8), c[b, h, t])
    meta = raw[b, n_kv * vm + 64 * h: n_kv * vm + 64 * (h + 1)].view(np.float16)
    assert np.array_equal(meta[:r], vks[b, h]) and np.array_equal(meta[8:24], cs[b, h])
    assert meta[24] == mus[b, h] and not meta[25:].any()


def test_r8_page_f32_scale_position():
    """c_grain "page_f32" (the per-page fp32 c scale): one fp32 per (block, head) at bytes
    16..19 of the head's scale block, halves 10..23 zero; token_c_scale repeats it."""
    from amass.selection import R8State
    n_kv, NB, r = 2, 3, 8
    st = R8State("cpu", num_layers=1, num_blocks=NB, n_kv=n_kv, G=4, head_dim=128, page=16,
                 max_reqs=1, max_pages=4, rank=r, c_grain="page_f32")
    rng = np.random.default_rng(5)
    Vk = rng.integers(-127, 128, (NB, n_kv, 128, r)).astype(np.int8)
    c = rng.integers(-127, 128, (NB, n_kv, 16, r)).astype(np.int8)
    mu = rng.integers(-127, 128, (NB, n_kv, 128)).astype(np.int8)
    mus = rng.random((NB, n_kv)).astype(np.float16)
    vks = rng.random((NB, n_kv, r)).astype(np.float16)
    cs = (rng.random((NB, n_kv)) * 1e-3 + 1e-7).astype(np.float32)   # not fp16-exact
    st.load_reference(0, mu, mus, Vk, vks, c, cs)
    vm = r * 128 + 128 + 16 * r
    raw = st.r8_rec[0].numpy().view(np.uint8)
    for b in range(NB):
        for h in range(n_kv):
            blk = raw[b, n_kv * vm + 64 * h: n_kv * vm + 64 * (h + 1)]
            assert blk[16:20].view(np.float32)[0] == cs[b, h]
            assert not blk[20:48].any()
            assert blk[48:50].view(np.float16)[0] == mus[b, h]
    tcs = st.token_c_scale(0).numpy()
    assert tcs.shape == (NB, n_kv, 16) and np.array_equal(tcs, np.repeat(cs[..., None], 16, -1))


@pytest.mark.parametrize("v_bits,c_bits,r", [(4, 4, 2), (8, 4, 2), (4, 8, 4), (8, 8, 8),
                                             (4, 4, 8)])
@pytest.mark.parametrize("c_grain", ["token", "page"])
def test_clse_record_positions(v_bits, c_bits, r, c_grain):
    """The packed CLSE record (include/amass_hip.h, AMASS_CLSE_REC_BYTES): per block the
    n_kv heads' [V tiled | mu] at h * VQ (whole 128-byte lines), then per head a tail of
    TB bytes at n_kv * VQ + TB * h: the c rows, then fp16 c_scale[0..16), V_scale at
    half 16, mu_scale at half 16 + r', the residual at half 17 + r', zeros to the end.
    Every field is checked at that byte offset in the raw buffer."""
    n_kv, NB = 3, 4
    st = QuadState("cpu", num_layers=1, num_blocks=NB, n_kv=n_kv, G=4, head_dim=128,
                   page=16, max_reqs=1, max_pages=4, rank=r, v_bits=v_bits, coords="lse",
                   c_bits=c_bits, c_grain=c_grain)
    cb = 128 if v_bits == 8 else 64
    vq = r * cb + 128
    crow = r * c_bits // 8
    tb = 16 * crow + 16 * ((36 + 2 * r + 15) // 16)
    rec_bytes = r * cb + 128 + 2 * r * c_bits + 16 * ((36 + 2 * r + 15) // 16)  # the macro
    assert vq % 128 == 0 and tb % 16 == 0
    assert st.rec_bytes == rec_bytes == vq + tb and st.quad_rec.shape[-1] == n_kv * rec_bytes
    if (v_bits, c_bits, r) == (4, 4, 2):
        assert rec_bytes == 320                     # the reference's default CLSE record
    rng = np.random.default_rng(r * 100 + v_bits * 10 + c_bits)
    lv, lc = (127 if v_bits == 8 else 7), (127 if c_bits == 8 else 7)
    vcode = rng.integers(-lv, lv + 1, (NB, n_kv, 128, r)).astype(np.int8)
    V = vcode if v_bits == 8 else oq.pack_i4(vcode)
    ccode = rng.integers(-lc, lc + 1, (NB, n_kv, 16, r)).astype(np.int8)
    c = ccode if c_bits == 8 else oq.pack_i4(ccode)
    mu = rng.integers(-127, 128, (NB, n_kv, 128)).astype(np.int8)
    mus = (rng.random((NB, n_kv)) + 0.5).astype(np.float16)
    vs = (rng.random((NB, n_kv, r)) + 0.5).astype(np.float16)
    cs = (rng.random((NB, n_kv, 16) if c_grain == "token" else (NB, n_kv)) + 0.5
          ).astype(np.float16)
    res = (rng.random((NB, n_kv)) + 0.5).astype(np.float16)
    st.load_reference(0, mu, mus, V, vs, c=c, c_scale=cs, resid=res)
    assert np.array_equal(st.reference_V(0).numpy(), V)
    raw = st.quad_rec[0].numpy().view(np.uint8)             # (NB, n_kv * REC)
    for b in range(NB):
        for h in range(n_kv):
            base = h * vq
            if v_bits == 8:               # d = 77: K-step 1, d group 0, byte 13
                off = ((1 * 4 + 0) * r + (r - 1)) * 16 + 13
                assert raw[b, base + off].view(np.int8) == vcode[b, h, 77, r - 1]
            assert np.array_equal(raw[b, base + r * cb: base + r * cb + 128].view(np.int8),
                                  mu[b, h])
            tail = raw[b, n_kv * vq + tb * h: n_kv * vq + tb * (h + 1)]
            assert np.array_equal(tail[:16 * crow].reshape(16, crow).view(np.int8), c[b, h])
            halves = tail[16 * crow:].view(np.float16)
            want_cs = cs[b, h] if c_grain == "token" else np.full(16, cs[b, h], np.float16)
            assert np.array_equal(halves[:16], want_cs)
            assert np.array_equal(halves[16:16 + r], vs[b, h])
            assert halves[16 + r] == mus[b, h] and halves[17 + r] == res[b, h]
            assert not halves[18 + r:].any()
    # the views the kernels' inputs are read back through
    assert np.array_equal(st.quad_c[0].numpy(), c)
    assert np.array_equal(st.V_scale[0].numpy(), vs) and np.array_equal(st.quad_resid[0].numpy(), res)
    assert np.array_equal(st.mu_scale[0].numpy(), mus)


def test_record_span_guard():
    """The score kernels address a layer's records with 32-bit offsets: the wrappers accept
    a record buffer of up to 4 GiB per layer and refuse a larger one (meta tensors, so
    nothing is allocated)."""
    from amass.selection.score import check_rec_span
    check_rec_span(torch.empty(1 << 20, 4096, dtype=torch.int8, device="meta"))   # 4 GiB
    check_rec_span(torch.empty(32768, 9600, dtype=torch.int8, device="meta"))    # config 1
    with pytest.raises(ValueError, match="4 GiB"):
        check_rec_span(torch.empty((1 << 20) + 1, 4096, dtype=torch.int8, device="meta"))
