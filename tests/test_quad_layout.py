"""Column-major quad_V layout of the gfx950 score kernel vs the reference layout.

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
