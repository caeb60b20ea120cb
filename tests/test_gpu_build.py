"""GPU parity of the HIP page-summary builder (amass_summary_build) against the float64
oracle (oracle/build.py, pinned in tests/test_build_oracle.py).

The builder's fp32 Jacobi eigh and the oracle's float64 LAPACK eigh agree to rounding, so
codes may differ by one step where a value sits on a rounding boundary, and eigenvectors
are compared up to sign and only where the eigenvalue is separated from its neighbours
(a near-repeated eigenvalue leaves its eigenvectors free to rotate; the scores built from
them are insensitive to that).  Bars: tags exact; mu codes within 1 (>= 99 % exact);
scales within 2e-3 relative; sig2 within 2e-3 relative (+1e-4 of the page's largest);
V / Vk codes of separated columns within 1 after sign alignment (>= 97 % exact); c codes
within 1 (>= 97 % exact) on separated columns of the token rows whose scale agrees (a
token's scale is the max over all its coordinates, so an unstable column can move it;
>= 80 % of the rows agree); with a "tensor" V grain only heads whose columns are all
separated are compared; the quad / r8 scores computed by the oracle from the HIP-built
and from the oracle-built summaries within 2e-2 * max(|s|, 1) (with a scale shared by all
columns, pages whose keys span fewer than r directions are left out: there the reference
formula divides rounding noise by sqrt(1e-10) in any precision; with any grain, pages
whose r-th and (r+1)-th eigenvalues are within 1e-3 of the largest are left out: their
top-r subspace is not fixed at fp32 resolution; both exclusions stay under 5 % of the
page-heads).  Two pages are crafted: a constant page (zero centred keys) gives zero V
codes and its score (the mu term alone) is checked separately, for every grain; the
near-rank-1 page (one direction plus bf16 rounding noise) stays out of the score check:
its r-1 trailing directions are rounding noise at ~1e-6 of the largest eigenvalue, the
fp32 eigensolver's own resolution, so no fp32 builder reproduces the float64 basis there.
The graph-captured tail rebuild restores corrupted records bit for bit.
"""
import numpy as np
import pytest
import torch

import oracle.build as ob
import oracle.quant as oq
import oracle.score as osc
from amass.bench.synth import make_case
from amass.selection import QuadState, R8State
from amass.selection.quad_build import quad_build_refresh, quad_build_tail
from helpers import announce, npf, npi

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(seed):
    case = make_case(B=3, ctx=(600, 1500), n_kv=8, G=4, heavy=0.05, table="perm", seed=seed,
                     device=DEV)
    K = case.kv_cache
    b0, b1 = int(case.block_table[0, 1]), int(case.block_table[1, 2])
    K[b0, 0] = K[b0, 0, 3]                          # page 1 of request 0: constant keys
    gen = torch.Generator(device=DEV)
    gen.manual_seed(seed + 104729)                  # independent of the global RNG's state
    x = torch.randn(16, 1, 1, device=DEV, generator=gen)   # page 2 of request 1: rank 1
    K[b1, 0] = (K[b1, 0, :1] + x * torch.randn(1, 8, 128, device=DEV, generator=gen)
                ).to(torch.bfloat16)
    return case, b0


def _blocks(case):
    return np.unique(np.concatenate([npi(case.block_table[r, :int(case.seq_lens[r]) // 16])
                                     for r in range(case.q.shape[0])]))


def _separated(S2_all, rank, gap=0.05):
    """(N, n_kv, rank) mask: eigenvalue separated from both neighbours by > gap (relative)."""
    ev = np.sort(S2_all, axis=-1)[..., -rank:]
    full = np.sort(S2_all, axis=-1)
    lo = full[..., -rank - 1:-1]
    hi = np.concatenate([full[..., -rank + 1:], np.full(full.shape[:-1] + (1,), np.inf)],
                        axis=-1)
    scale = np.maximum(full[..., -1:], 1e-30)
    return ((ev - lo) > gap * scale) & ((hi - ev) > gap * scale)


def _col_check(ref_codes, got_codes, sep):
    """Sign-aligned code comparison of the separated columns (axis -2 = d or token)."""
    ref = ref_codes.astype(np.float64)
    got = got_codes.astype(np.float64)
    sgn = np.sign((ref * got).sum(axis=-2, keepdims=True))
    sgn[sgn == 0] = 1
    diff = np.abs(got * sgn - ref)
    m = np.broadcast_to(sep[..., None, :], diff.shape)
    d = diff[m]
    assert d.size and d.max() <= 1 and (d == 0).mean() >= 0.97, (d.max(), (d == 0).mean())
    return sgn


def _deficient(S2_all, rank):
    """(N, n_kv) pages whose centred keys span fewer than `rank` directions: their
    null-space columns are dc^T u / sqrt(1e-10), rounding noise times 1e5 in any
    precision (the reference's fp32 builder included), so a scale shared across columns
    is set by noise on both sides."""
    ev = np.sort(S2_all, axis=-1)
    return ev[..., -rank] <= 1e-6 * ev[..., -1]


def _ill_posed(S2_all, rank, gap=1e-3):
    """(N, n_kv) pages whose r-th and (r+1)-th eigenvalues lie within `gap` of the largest:
    the top-r subspace is not fixed by the data to fp32 resolution (the fp32 Jacobi moves
    eigenvalues by ~1e-6 of the largest), so any fp32 builder may pick another basis of
    the near-degenerate pair and the score built from it differs from the float64 one."""
    ev = np.sort(S2_all, axis=-1)
    return (ev[..., -rank] - ev[..., -rank - 1]) <= gap * np.maximum(ev[..., -1], 1e-30)


def _score_mask(case, blocks, bad, nsh):
    """(R, n_kv, MP) True where the scored page's (block, head) is not in `bad`."""
    remap = {int(b): i for i, b in enumerate(blocks)}
    bt = npi(case.block_table)
    R, n_kv = bt.shape[0], bad.shape[1]
    m = np.zeros((R, n_kv, case.max_pages), bool)
    for r in range(R):
        for p in range(nsh[r]):
            m[r, :, p] = ~bad[remap[int(bt[r, p])]]
    return m


def _check_constant_page(case, blocks, const_blk, nsh, ok):
    """The constant page's score (zero centred keys: the mu term alone) agrees for every
    kv head, whatever the grain (the ill-posed / deficient masks leave it out)."""
    one = np.zeros((blocks.size, ok.shape[1]), bool)
    one[int(np.searchsorted(blocks, const_blk))] = True
    at = _score_mask(case, blocks, ~one, nsh)
    assert at.any() and np.all(ok[at])


def _rel(got, ref, tol, abs_tol=0.0):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    assert np.all(np.abs(got - ref) <= tol * np.abs(ref) + abs_tol), \
        float(np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)))


@pytest.mark.parametrize("rank,v_bits,v_grain", [(8, 8, "col"), (8, 4, "col"), (2, 8, "col"),
                                                 (4, 4, "tensor")])
def test_quad_summary_build(rank, v_bits, v_grain):
    announce(f"HIP builder quad r'={rank} v_bits={v_bits} grain={v_grain}")
    case, const_blk = _case(20 + rank + v_bits)
    NB = case.kv_cache.shape[0]
    st = QuadState(DEV, num_layers=1, num_blocks=NB, n_kv=8, G=4, head_dim=128, page=16,
                   max_reqs=3, max_pages=case.max_pages, rank=rank, v_bits=v_bits,
                   v_grain=v_grain, combine="nrm")
    n = quad_build_refresh(st, 0, case.K, case.block_table, case.seq_lens, 3, force=True)
    torch.cuda.synchronize()
    blocks = _blocks(case)
    assert n == blocks.size
    K = npf(case.K)[blocks]
    ref = ob.quad_summary(K, rank, v_bits, v_grain)
    dc = ob.page_factors(K, 16)[1]
    S2_all = np.linalg.eigvalsh(dc @ dc.swapaxes(-1, -2))
    tag = npi(st.quad_tag[0].view(torch.int16))[blocks]
    last = npi(case.K[torch.from_numpy(blocks).to(DEV)][:, 15, :, :8].contiguous().view(torch.int16))
    assert np.array_equal(tag, last)
    mu = npi(st.quad_mu[0])[blocks].astype(int)
    dm = np.abs(mu - ref["mu"].astype(int))
    assert dm.max() <= 1 and (dm == 0).mean() >= 0.99
    _rel(npf(st.mu_scale[0])[blocks], ref["mu_scale"], 2e-3)
    sig2 = npf(st.quad_sig2[0])[blocks]
    # stored as fp16 (the 1e-10 clamp of a zero eigenvalue is 0 there)
    _rel(sig2, ref["sig2"].astype(np.float16), 2e-3, 1e-4 * ref["sig2"][..., -1:])
    sep = _separated(S2_all, rank)
    if v_grain == "tensor":            # one scale over all columns: every column must be stable
        sep = sep & sep.all(axis=-1, keepdims=True)
    V = oq.codes(npi(st.reference_V(0))[blocks], v_bits)
    _col_check(oq.codes(ref["V"], v_bits), V, sep)
    vs = npf(st.V_scale[0])[blocks]
    if v_grain == "tensor":
        assert np.all(vs == vs[..., :1])
    else:
        _rel(vs[sep], ref["V_scale"][sep], 2e-3)
    # the constant page: zero centred keys -> zero V codes, sig2 = fp16(1e-10) = 0
    ci = int(np.searchsorted(blocks, const_blk))
    assert not V[ci].any() and not sig2[ci].any()
    # downstream: the oracle's score from both summaries
    bt = npi(case.block_table)
    nsh = np.array([int(s) // 16 - 1 for s in npi(case.seq_lens)])
    remap = np.full(NB, -1, np.int64)
    remap[blocks] = np.arange(blocks.size)
    btl = remap[bt.clip(0)].clip(0).astype(np.int32)
    q = npf(case.q)
    kw = dict(scale=case.scale, page=16, G=4, v_bits=v_bits, max_pages=case.max_pages,
              combine="max")
    s_hip = osc.quad_score(q, npi(st.quad_mu[0])[blocks], npf(st.mu_scale[0])[blocks],
                           npi(st.reference_V(0))[blocks], vs, sig2, btl, nsh, **kw)
    s_ref = osc.quad_score(q, ref["mu"], ref["mu_scale"], ref["V"], ref["V_scale"],
                           ref["sig2"], btl, nsh, **kw)
    bad = _ill_posed(S2_all, rank)
    if v_grain == "tensor":
        bad |= _deficient(S2_all, rank)
    assert bad.mean() < 0.05, bad.mean()
    mask = _score_mask(case, blocks, bad, nsh)
    ok = np.abs(s_hip - s_ref) <= 2e-2 * np.maximum(np.abs(s_ref), 1)
    assert np.all(ok | ~mask), float(np.nanmax(np.where(mask, np.abs(s_hip - s_ref), 0)))
    _check_constant_page(case, blocks, const_blk, nsh, ok)


@pytest.mark.parametrize("rank,vk_bits,c_bits,vk_grain,c_grain",
                         [(8, 8, 8, "col", "page"), (8, 4, 4, "col", "page"),
                          (4, 8, 4, "tensor", "tensor"), (8, 8, 8, "col", "page_f32")])
def test_r8_summary_build(rank, vk_bits, c_bits, vk_grain, c_grain):
    announce(f"HIP builder r8 r={rank} vk={vk_bits} c={c_bits} {vk_grain}/{c_grain}")
    from amass.selection.build import r8_build_refresh
    case, const_blk = _case(40 + rank + c_bits)
    NB = case.kv_cache.shape[0]
    st = R8State(DEV, num_layers=1, num_blocks=NB, n_kv=8, G=4, head_dim=128, page=16,
                 max_reqs=3, max_pages=case.max_pages, rank=rank, vk_bits=vk_bits,
                 c_bits=c_bits, vk_grain=vk_grain, c_grain=c_grain)
    r8_build_refresh(st, 0, case.K, case.block_table, case.seq_lens, 3, force=True)
    torch.cuda.synchronize()
    blocks = _blocks(case)
    K = npf(case.K)[blocks]
    ref = ob.r8_summary(K, rank, vk_bits, c_bits, vk_grain, c_grain)
    dc = ob.page_factors(K, 16)[1]
    sep = _separated(np.linalg.eigvalsh(dc @ dc.swapaxes(-1, -2)), rank)
    if vk_grain == "tensor":           # one scale over all columns: every column must be stable
        sep = sep & sep.all(axis=-1, keepdims=True)
    mu = npi(st.r8_mu[0])[blocks].astype(int)
    assert np.abs(mu - ref["mu"].astype(int)).max() <= 1
    Vk = oq.codes(npi(st.reference_Vk(0))[blocks], vk_bits)
    sgn = _col_check(oq.codes(ref["Vk"], vk_bits), Vk, sep)
    c = oq.codes(npi(st.r8_c[0])[blocks], c_bits).astype(np.float64) * sgn  # same column signs
    cref = oq.codes(ref["c"], c_bits).astype(np.float64)
    cs = npf(st.token_c_scale(0))[blocks]
    if c_grain != "page":
        assert np.all(cs == cs[..., :1])
    if c_grain == "page_f32":         # stored fp32, not rounded to fp16
        assert not np.all(cs == cs.astype(np.float16).astype(np.float32))
    # a token's scale is the max over its r coordinates: rows whose scale agrees, columns
    # that are separated
    same = np.abs(cs - ref["c_scale"]) <= 2e-3 * ref["c_scale"]
    assert same.mean() >= 0.8, same.mean()
    m = sep[..., None, :] & same[..., :, None]
    dcod = np.abs(c - cref)[m]
    assert dcod.size and dcod.max() <= 1 and (dcod == 0).mean() >= 0.97
    # downstream r8 score from both summaries
    bt = npi(case.block_table)
    nsh = np.array([int(s) // 16 - 1 for s in npi(case.seq_lens)])
    remap = np.full(NB, -1, np.int64)
    remap[blocks] = np.arange(blocks.size)
    btl = remap[bt.clip(0)].clip(0).astype(np.int32)
    kw = dict(scale=case.scale, page=16, G=4, vk_bits=vk_bits, c_bits=c_bits,
              max_pages=case.max_pages)
    q, sl = npf(case.q), npi(case.seq_lens)
    s_hip = osc.r8_score(q, npi(st.r8_mu[0])[blocks], npf(st.mu_scale[0])[blocks],
                         npi(st.reference_Vk(0))[blocks], npf(st.Vk_scale[0])[blocks],
                         npi(st.r8_c[0])[blocks], cs, btl, sl, nsh, **kw)
    s_ref = osc.r8_score(q, ref["mu"], ref["mu_scale"], ref["Vk"], ref["Vk_scale"], ref["c"],
                         ref["c_scale"], btl, sl, nsh, **kw)
    S2_all = np.linalg.eigvalsh(dc @ dc.swapaxes(-1, -2))
    bad = _ill_posed(S2_all, rank)
    if vk_grain == "tensor":
        bad |= _deficient(S2_all, rank)
    assert bad.mean() < 0.05, bad.mean()
    mask = _score_mask(case, blocks, bad, nsh)
    ok = np.abs(s_hip - s_ref) <= 2e-2 * np.maximum(np.abs(s_ref), 1)
    assert np.all(ok | ~mask), float(np.nanmax(np.where(mask, np.abs(s_hip - s_ref), 0)))
    _check_constant_page(case, blocks, const_blk, nsh, ok)


def test_tail_rebuild_graph_replay():
    """quad_build_tail (every request's last finalised page, all layers) is sync-free:
    captured in a HIP graph and replayed after the records were corrupted, it restores
    them bit for bit (the build is a pure function of the K bytes)."""
    announce("HIP builder: tail rebuild in a graph")
    case, _ = _case(77)
    NB = case.kv_cache.shape[0]
    st = QuadState(DEV, num_layers=2, num_blocks=NB, n_kv=8, G=4, head_dim=128, page=16,
                   max_reqs=3, max_pages=case.max_pages, rank=8, combine="nrm")
    K2 = [case.K, case.K]
    quad_build_tail(st, K2, case.block_table, case.seq_lens, 3)
    torch.cuda.synchronize()
    want = st.quad_rec.clone()
    tail = [int(case.block_table[r, int(case.seq_lens[r]) // 16 - 1]) for r in range(3)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        quad_build_tail(st, K2, case.block_table, case.seq_lens, 3)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        quad_build_tail(st, K2, case.block_table, case.seq_lens, 3)
    for _ in range(3):
        st.quad_rec[:, tail] = 77
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(st.quad_rec, want)
