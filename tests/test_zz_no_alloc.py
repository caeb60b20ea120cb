"""The allocation-free decode entry point (amass_sparse_decode_noalloc, no counterpart in
the reference) against amass_sparse_decode, through the C-ABI.

Both run the same kernels with the same plan; only the split-K partials live elsewhere
(the library's file-scope device array instead of the state's buffers), so the outputs
must be bit-identical.  Two calls in a row, the second with a smaller batch (its merge
must not see the first call's partials), for every decode path.  The library's default
split (128) at config 1's batch geometry (32 requests x 8 kv heads x G 4) needs more
partial slots than the array holds: the entry point lowers the split to the 63 that fit,
and the output still equals the allocating entry's (the plan splits a unit into 8 there).
A batch for which fewer than 3 slots fit is refused with AMASS_ERR_CAPACITY before
anything runs.
"""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle.decode as odec
import oracle.select as osel
from amass import _hip
from amass.attention import ensure_stage_b_buffers
from amass.attention.decode import ResidentVSource, _decode_args, _split_kv
from amass.bench.synth import make_case
from helpers import announce, npf

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCRATCH_BYTES = 32 * 1024 * 1024      # AMASS_DECODE_SCRATCH_BYTES


class _St:
    pass


def _setup(B, ctx, frac, seed):
    case = make_case(B=B, ctx=ctx, n_kv=8, G=4, heavy=0.0, table="perm", seed=seed)
    MP = case.max_pages
    sc = torch.randn(B, 8, MP, generator=torch.Generator().manual_seed(seed)).numpy()
    npg, nsh, bfix = osel.derive(case.seq_lens.numpy(), frac, 16, 1, 1)
    tab, cnt, _ = osel.select(sc, npg, nsh, bfix, sink=1, max_pages=MP, mode=0)
    st = _St()
    st.max_reqs, st.n_kv, st.G, st.D = B, 8, 4, 128
    st.page_table = torch.from_numpy(tab).to(DEV)
    st.page_cnt = torch.from_numpy(cnt).to(DEV)
    ensure_stage_b_buffers(st, DEV)
    kv = case.kv_cache.to(DEV)
    dev = dict(q=case.q.to(DEV), kv=kv, bt=case.block_table.to(DEV),
               sl=case.seq_lens.to(DEV))
    return case, st, dev, tab, cnt


def _args(case, st, dev, out, path):
    k, _ = _split_kv(dev["kv"])
    return _decode_args(dev["q"], k, ResidentVSource(dev["kv"]), dev["bt"], dev["sl"], st,
                        out, case.scale, case.q.shape[0], dense=False, path=path)


def _both(case, st, dev, path):
    """(out of amass_sparse_decode, out of amass_sparse_decode_noalloc) on one stream."""
    lib = _hip.load_library()
    stream = _hip.current_stream(dev["q"].device)
    outs = []
    for name in ("amass_sparse_decode", "amass_sparse_decode_noalloc"):
        out = torch.full((case.q.shape[0], 32, 128), float("nan"), dtype=torch.bfloat16,
                         device=DEV)
        a = _args(case, st, dev, out, path)
        if name.endswith("noalloc"):
            a.m_part = a.l_part = a.acc_part = None       # ignored by this entry point
        _hip.check(getattr(lib, name)(C.byref(a), C.c_void_p(stream)), name)
        outs.append(out)
    torch.cuda.synchronize()
    return outs


@pytest.mark.parametrize("path", ["auto", "split", "fused"])
def test_noalloc_decode_matches_allocating_entry(path):
    announce(f"no-alloc decode, path={path}: B=8 then B=3")
    big = _setup(8, (3000, 9000), 0.6, seed=101)
    small = _setup(3, (500, 2000), 0.3, seed=102)
    for case, st, dev, tab, cnt in (big, small):
        B = case.q.shape[0]
        need = 4 * B * 8 * st.split * 4 * (2 + 128) + 256
        assert need <= SCRATCH_BYTES
        ref, got = _both(case, st, dev, path)
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"B={B}"
        want = odec.attend(npf(case.q), npf(case.kv_cache[:, 0]), npf(case.kv_cache[:, 1]),
                           case.block_table.numpy(), case.seq_lens.numpy(), tab, cnt,
                           scale=case.scale, G=4)
        assert np.allclose(npf(got), want, atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("path", ["auto", "split"])
def test_noalloc_decode_at_the_default_split_of_a_full_batch(path):
    announce(f"no-alloc decode, path={path}: B=32 at split 128 (63 slots fit)")
    case, st, dev, tab, cnt = _setup(32, 4096, 0.9, seed=104)
    assert st.split == 128
    assert 4 * 32 * 8 * 128 * 4 * (2 + 128) > SCRATCH_BYTES      # the default does not fit
    ref, got = _both(case, st, dev, path)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    # and again with a smaller batch right after (no leftover partials are read)
    case, st, dev, tab, cnt = _setup(5, (500, 3000), 0.5, seed=105)
    ref, got = _both(case, st, dev, path)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_noalloc_decode_refuses_oversized_partials():
    announce("no-alloc decode: capacity check")
    B = 700                               # 700 * 8 * 4 slots per split: only 2 fit
    case, st, dev, _, _ = _setup(B, (16, 64), 0.5, seed=103)
    out = torch.zeros(B, 32, 128, dtype=torch.bfloat16, device=DEV)
    a = _args(case, st, dev, out, "split")
    assert (SCRATCH_BYTES - 256) // (4 * B * 8 * 4 * (2 + 128)) < 3
    lib = _hip.load_library()
    rc = lib.amass_sparse_decode_noalloc(C.byref(a), C.c_void_p(_hip.current_stream()))
    assert rc == -6                       # AMASS_ERR_CAPACITY, nothing launched
    torch.cuda.synchronize()
    assert not out.any()
