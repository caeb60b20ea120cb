"""GPU parity of the sparse / dense paged decode against the fp64 oracle.

Bar: outputs within 2e-2 absolute / 1e-2 relative of the fp64 softmax
attention.  Covers split-K + merge, the fused single pass, the dense baseline, G = 4 / 8,
partial last pages whose unused slots hold NaN (must be masked), padded rows (zero
output), empty and single-page selections.
"""
import numpy as np
import pytest
import torch

import oracle.decode as odec
import oracle.select as osel
from amass.attention import ensure_stage_b_buffers
from amass.attention.decode import ResidentVSource, dense_paged_decode, sparse_paged_decode_batched
from amass.bench.synth import make_case
from helpers import announce, npf, npi

pytestmark = pytest.mark.gpu
DEV = "cuda"
ATOL, RTOL = 2e-2, 1e-2


class _St:
    pass


def _case(B, G, seed, partial=True, n_kv=8):
    case = make_case(B=B, ctx=(200, 3000), n_kv=n_kv, G=G, heavy=0.0, table="perm", seed=seed)
    sl = case.seq_lens.clone()
    if partial:
        sl = sl - torch.arange(B, dtype=torch.int32) % 13   # ragged partial last pages
        sl = torch.clamp(sl, min=1)
        # poison the unused token slots of every request's last page
        for r in range(B):
            n = int(sl[r])
            last = (n - 1) // 16
            blk = int(case.block_table[r, last])
            t0 = n - last * 16
            if t0 < 16:
                case.kv_cache[blk, :, t0:] = float("nan")
    case.seq_lens = sl.to(torch.int32)
    return case


def _selection(case, frac, seed, empty_unit=False):
    B, n_kv, MP = case.q.shape[0], case.n_kv, case.max_pages
    gen = torch.Generator().manual_seed(seed)
    sc = torch.randn(B, n_kv, MP, generator=gen).numpy()
    npg, nsh, bfix = osel.derive(case.seq_lens.numpy(), frac, 16, 1, 1)
    tab, cnt, _ = osel.select(sc, npg, nsh, bfix, sink=1, max_pages=MP, mode=0)
    if empty_unit:
        cnt[0, 0] = 0
        tab[0, 0, :] = -1
    return tab, cnt


def _st(case, tab, cnt):
    st = _St()
    st.max_reqs, st.n_kv, st.G, st.D = case.q.shape[0], case.n_kv, case.G, case.d
    st.page_table = torch.from_numpy(tab).to(DEV)
    st.page_cnt = torch.from_numpy(cnt).to(DEV)
    ensure_stage_b_buffers(st, DEV)
    return st


def _np_inputs(case):
    return (npf(case.q), npf(case.kv_cache[:, 0]), npf(case.kv_cache[:, 1]),
            npi(case.block_table), npi(case.seq_lens))


@pytest.mark.parametrize("G", [4, 8])
@pytest.mark.parametrize("path", ["split", "fused"])
@pytest.mark.parametrize("frac", [0.05, 0.5])
def test_sparse_decode(G, path, frac):
    announce(f"sparse decode G={G} path={path} frac={frac}")
    case = _case(5, G, seed=G * 10 + int(frac * 100))
    tab, cnt = _selection(case, frac, seed=1, empty_unit=True)
    q, K, V, bt, sl = _np_inputs(case)
    ref = odec.attend(q, K, V, bt, sl, tab, cnt, scale=case.scale, G=G)
    kv = case.kv_cache.to(DEV)
    st = _st(case, tab, cnt)
    out = torch.full((5, 8 * G, 128), float("nan"), dtype=torch.bfloat16, device=DEV)
    sparse_paged_decode_batched(case.q.to(DEV), kv, case.block_table.to(DEV),
                                case.seq_lens.to(DEV), st, out, ResidentVSource(kv),
                                scale=case.scale, path=path)
    torch.cuda.synchronize()
    got = npf(out)
    assert np.isfinite(got).all()
    assert np.allclose(got, ref, atol=ATOL, rtol=RTOL), float(np.abs(got - ref).max())
    # the empty unit (req 0, kv-head 0) writes zeros
    assert np.all(got[0, :G] == 0)


@pytest.mark.parametrize("n_kv,G", [(1, 8), (2, 2), (4, 1), (16, 4)])
@pytest.mark.parametrize("path", ["auto", "split", "fused"])
def test_sparse_decode_head_layouts(n_kv, G, path):
    """Workgroups of fewer than 8 kv heads, two head groups, GQA groups 1 and 2."""
    announce(f"sparse decode heads n_kv={n_kv} G={G} path={path}")
    case = _case(3, G, seed=70 + n_kv + G, n_kv=n_kv)
    tab, cnt = _selection(case, 0.3, seed=2)
    q, K, V, bt, sl = _np_inputs(case)
    ref = odec.attend(q, K, V, bt, sl, tab, cnt, scale=case.scale, G=G)
    kv = case.kv_cache.to(DEV)
    st = _st(case, tab, cnt)
    out = torch.full((3, n_kv * G, 128), float("nan"), dtype=torch.bfloat16, device=DEV)
    sparse_paged_decode_batched(case.q.to(DEV), kv, case.block_table.to(DEV),
                                case.seq_lens.to(DEV), st, out, ResidentVSource(kv),
                                scale=case.scale, path=path)
    torch.cuda.synchronize()
    got = npf(out)
    assert np.isfinite(got).all()
    assert np.allclose(got, ref, atol=ATOL, rtol=RTOL), float(np.abs(got - ref).max())


@pytest.mark.parametrize("G", [4, 8])
@pytest.mark.parametrize("path", ["split", "fused", "auto"])
def test_dense_decode(G, path):
    announce(f"dense decode G={G} path={path}")
    case = _case(4, G, seed=40 + G)
    q, K, V, bt, sl = _np_inputs(case)
    ref = odec.attend(q, K, V, bt, sl, scale=case.scale, G=G, dense=True)
    kv = case.kv_cache.to(DEV)
    st = _St()
    st.max_reqs, st.n_kv, st.G, st.D = 4, 8, G, 128
    ensure_stage_b_buffers(st, DEV)
    out = torch.zeros((4, 8 * G, 128), dtype=torch.bfloat16, device=DEV)
    dense_paged_decode(case.q.to(DEV), kv, case.block_table.to(DEV), case.seq_lens.to(DEV),
                       st, out, scale=case.scale, path=path)
    torch.cuda.synchronize()
    got = npf(out)
    assert np.allclose(got, ref, atol=ATOL, rtol=RTOL), float(np.abs(got - ref).max())


@pytest.mark.parametrize("ctx", [4096, 16384])
def test_dense_decode_one_long_request(ctx):
    """path "auto" with one request of many pages (config 0's dense baseline shape and
    beyond): the plan splits the few long units over many workgroups (LSE partials and
    the merge) instead of one workgroup per head; matches the fp64 oracle."""
    announce(f"dense decode one request ctx={ctx}")
    case = make_case(B=1, ctx=(ctx, ctx), n_kv=8, G=4, heavy=0.0, table="perm", seed=90)
    q, K, V, bt, sl = _np_inputs(case)
    ref = odec.attend(q, K, V, bt, sl, scale=case.scale, G=4, dense=True)
    kv = case.kv_cache.to(DEV)
    st = _St()
    st.max_reqs, st.n_kv, st.G, st.D = 1, 8, 4, 128
    ensure_stage_b_buffers(st, DEV)
    out = torch.full((1, 32, 128), float("nan"), dtype=torch.bfloat16, device=DEV)
    dense_paged_decode(case.q.to(DEV), kv, case.block_table.to(DEV), case.seq_lens.to(DEV),
                       st, out, scale=case.scale, path="auto")
    torch.cuda.synchronize()
    got = npf(out)
    assert np.isfinite(got).all()
    assert np.allclose(got, ref, atol=ATOL, rtol=RTOL), float(np.abs(got - ref).max())


def test_split_equals_fused_and_padded_rows():
    announce("split vs fused, padded rows")
    case = _case(4, 4, seed=77, partial=False)
    case.seq_lens[3] = 0
    tab, cnt = _selection(case, 0.2, seed=2)
    cnt[3] = 0
    tab[3] = -1
    kv = case.kv_cache.to(DEV)
    st = _st(case, tab, cnt)
    outs = []
    for path in ("split", "fused"):
        out = torch.full((4, 32, 128), 7.0, dtype=torch.bfloat16, device=DEV)
        sparse_paged_decode_batched(case.q.to(DEV), kv, case.block_table.to(DEV),
                                    case.seq_lens.to(DEV), st, out, ResidentVSource(kv),
                                    scale=case.scale, path=path)
        outs.append(npf(out))
    torch.cuda.synchronize()
    assert np.all(outs[0][3] == 0) and np.all(outs[1][3] == 0)
    assert np.allclose(outs[0], outs[1], atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("frac", [0.02, 0.9])
def test_auto_plan_layouts(frac):
    """path "auto" plans on the device: a latency-bound batch (2 % of the pages) runs one
    workgroup per (request, head) with the waves merged in LDS; a bandwidth-bound ragged
    batch (90 %, more than 16 pages per resident workgroup) runs the balanced split layout
    (one wave per head, LSE partials, the merge launch).  Both match the fp64 oracle."""
    announce(f"auto plan layouts frac={frac}")
    B, G = 8, 4
    case = make_case(B=B, ctx=(4000, 24000), n_kv=8, G=G, heavy=0.0, table="perm", seed=61)
    tab, cnt = _selection(case, frac, seed=6, empty_unit=True)
    q, K, V, bt, sl = _np_inputs(case)
    ref = odec.attend(q, K, V, bt, sl, tab, cnt, scale=case.scale, G=G)
    kv = case.kv_cache.to(DEV)
    st = _st(case, tab, cnt)
    out = torch.full((B, 8 * G, 128), float("nan"), dtype=torch.bfloat16, device=DEV)
    sparse_paged_decode_batched(case.q.to(DEV), kv, case.block_table.to(DEV),
                                case.seq_lens.to(DEV), st, out, ResidentVSource(kv),
                                scale=case.scale, path="auto")
    torch.cuda.synchronize()
    got = npf(out)
    assert np.isfinite(got).all()
    assert np.allclose(got, ref, atol=ATOL, rtol=RTOL), float(np.abs(got - ref).max())
    assert np.all(got[0, :G] == 0)


@pytest.mark.parametrize("dense", [False, True])
def test_split_merge_repeatable_across_launches_and_graph_replays(dense):
    """Split-K partials + merge launch: eager launches and HIP-graph replays (with eager
    work between them) give bit-identical outputs that match the fp64 oracle."""
    announce(f"split-K repeatability, dense={dense}")
    case = _case(3, 8, seed=91)
    tab, cnt = _selection(case, 0.9, seed=3)
    q, K, V, bt, sl = _np_inputs(case)
    ref = odec.attend(q, K, V, bt, sl, None if dense else tab, None if dense else cnt,
                      scale=case.scale, G=8, dense=dense)
    kv = case.kv_cache.to(DEV)
    st = _st(case, tab, cnt)
    qd, btd, sld = case.q.to(DEV), case.block_table.to(DEV), case.seq_lens.to(DEV)
    out = torch.zeros((3, 64, 128), dtype=torch.bfloat16, device=DEV)

    def step():
        if dense:
            dense_paged_decode(qd, kv, btd, sld, st, out, scale=case.scale, path="split")
        else:
            sparse_paged_decode_batched(qd, kv, btd, sld, st, out, ResidentVSource(kv),
                                        scale=case.scale, path="split")
    step()
    torch.cuda.synchronize()
    first = out.clone()
    got = npf(first)
    assert np.allclose(got, ref, atol=ATOL, rtol=RTOL), float(np.abs(got - ref).max())
    step()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), first.view(torch.int16))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), first.view(torch.int16))
        step()                                   # eager launch between replays
        torch.cuda.synchronize()


def test_decode_rejects_inconsistent_geometry():
    """The host side refuses a query / cache / state mismatch before any launch (the
    kernels index the state's partials, tables and counts with these values), and the
    library refuses K or V views that are not 16-byte aligned."""
    announce("decode geometry checks")
    from amass._hip import AmassError
    case = _case(3, 4, seed=5, partial=False)
    tab, cnt = _selection(case, 0.3, seed=2)
    kv = case.kv_cache.to(DEV)
    st = _st(case, tab, cnt)
    q, bt, sl = case.q.to(DEV), case.block_table.to(DEV), case.seq_lens.to(DEV)
    out = torch.zeros((3, 32, 128), dtype=torch.bfloat16, device=DEV)
    run = lambda q_, kv_, out_, st_: sparse_paged_decode_batched(  # noqa: E731
        q_, kv_, bt, sl, st_, out_, ResidentVSource(kv_), scale=case.scale)
    run(q, kv, out, st)                                   # consistent: runs
    torch.cuda.synchronize()
    st.max_reqs = 2                                       # more requests than the state
    with pytest.raises(ValueError, match="max_reqs"):
        run(q, kv, out, st)
    st.max_reqs = 3
    st.G = 8                                              # state built for another group
    with pytest.raises(ValueError, match="geometry"):
        run(q, kv, out, st)
    st.G = 4
    with pytest.raises(ValueError, match="query heads"):
        run(q[:, :30], kv, out, st)
    # a cache view one element off its 16-byte alignment
    flat = torch.empty(kv.numel() + 8, dtype=torch.bfloat16, device=DEV)
    bad = flat.as_strided(kv.shape, kv.stride(), 1)
    bad.copy_(kv)
    with pytest.raises(AmassError):
        run(q, bad, out, st)
    torch.cuda.synchronize()
