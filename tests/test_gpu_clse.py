"""GPU parity of the CLSE score (amass_clse_score) and of the CLSE summary build.

CLSE (reference selection/quad_score.py:156-393) = the quad storage + per-key coordinates
+ the residual energy.  Bars: int32 d-contractions bit-exact (comb_out vs int64 brute
force); scores within 1e-3 * max(|ref|, 1) of the float64 oracle with unquantised q
(the 1e-3 bar for the score kernels), per head (combine "nrm") and group max ("max");
the HIP builder's resid within 2e-3 relative (+1e-4 of the page's trace), c codes within
one step on separated columns, and the scores from its summaries within 2e-2 of the
oracle-built ones; select_pages_clse + decode end to end against the oracle.
"""
import numpy as np
import pytest
import torch

import oracle.build as ob
import oracle.decode as odec
import oracle.score as osc
import oracle.select as osel
from amass.attention.decode import ResidentVSource, sparse_paged_decode_batched
from amass.bench.synth import build_quad_state, make_case
from amass.selection import derive_page_params, select_pages_clse
from amass.selection.quad_score import clse_score
from helpers import announce, case_to, npf, npi, rel_err, to_device

pytestmark = pytest.mark.gpu
DEV = "cuda"

CASES = [  # rank, v_bits, c_bits, c_grain, G, combine
    (2, 8, 4, "token", 4, "max"), (2, 4, 4, "token", 4, "nrm"), (2, 8, 8, "page", 8, "nrm"),
    (8, 8, 4, "token", 4, "nrm"), (8, 4, 8, "page", 4, "max"), (4, 8, 4, "token", 8, "max"),
    (2, 8, 4, "token", 1, "max"), (4, 4, 4, "page", 2, "nrm"),
]


def _oracle_inputs(case, st):
    mu, mus, _, Vs, _sg, _ = st.layer_state(0)
    cs = st.c_scale[0]
    return dict(q=npf(case.q), mu=npi(mu), mu_scale=npf(mus), V=npi(st.reference_V(0)),
                V_scale=npf(Vs), c=npi(st.quad_c[0]), c_scale=npf(cs),
                resid=npf(st.quad_resid[0]), block_table=npi(case.block_table),
                seq_lens=npi(case.seq_lens), n_sel_hi=npi(st.n_sel_hi))


@pytest.mark.parametrize("rank,v_bits,c_bits,c_grain,G,combine", CASES)
def test_clse_score_vs_oracle(rank, v_bits, c_bits, c_grain, G, combine):
    announce(f"CLSE r'={rank} v={v_bits} c={c_bits} {c_grain} G={G} {combine}")
    B = 3
    case = make_case(B=B, ctx=(300, 1400), n_kv=8, G=G, heavy=0.05, table="perm",
                     seed=60 + rank + G)
    st = build_quad_state(case, rank=rank, v_bits=v_bits, combine=combine, coords="lse",
                          c_bits=c_bits, c_grain=c_grain, budget=0.05)
    to_device(st, DEV)
    case_to(case, DEV)
    derive_page_params(st, case.seq_lens, B)
    MP = st.max_pages
    comb = torch.zeros(B, 8, MP, G, rank + 1, dtype=torch.int32, device=DEV)
    clse_score(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale, comb_out=comb)
    torch.cuda.synchronize()
    inp = _oracle_inputs(case, st)
    nsh = inp["n_sel_hi"]
    ref_comb = osc.quad_comb(inp["q"], inp["mu"], inp["V"], inp["block_table"], nsh, G=G,
                             v_bits=v_bits, max_pages=MP)
    got_comb = npi(comb).astype(np.int64)
    ref = osc.clse_score(inp["q"], inp["mu"], inp["mu_scale"], inp["V"], inp["V_scale"],
                         inp["c"], inp["c_scale"], inp["resid"], inp["block_table"],
                         inp["seq_lens"], nsh, scale=case.scale, page=16, G=G, v_bits=v_bits,
                         c_bits=c_bits, max_pages=MP, combine=combine)
    got = npf(st.score_h if combine == "nrm" else st.score)
    for r in range(B):
        n = int(nsh[r])
        assert np.array_equal(got_comb[r, :, :n], ref_comb[r, :, :n])
        if combine == "nrm":
            assert rel_err(got[r, :, :, :n], ref[r, :, :, :n]) <= 1e-3
        else:
            assert rel_err(got[r, :, :n], ref[r, :, :n]) <= 1e-3


@pytest.mark.parametrize("rank,c_bits,c_grain", [(2, 4, "token"), (8, 8, "page")])
def test_clse_summary_build(rank, c_bits, c_grain):
    announce(f"HIP builder CLSE r'={rank} c={c_bits} {c_grain}")
    B = 3
    case = make_case(B=B, ctx=(600, 1500), n_kv=8, G=4, heavy=0.05, table="perm", seed=88,
                     device=DEV)
    st = build_quad_state(case, rank=rank, v_bits=8, combine="max", coords="lse",
                          c_bits=c_bits, c_grain=c_grain, budget=0.05)
    torch.cuda.synchronize()
    fin = np.unique(np.concatenate([npi(case.block_table[r, :int(case.seq_lens[r]) // 16])
                                    for r in range(B)]))
    K = npf(case.K)[fin]
    ref = ob.clse_summary(K, rank, 8, c_bits, c_grain)
    dc = ob.page_factors(K, 16)[1]
    trace = (dc * dc).sum(axis=(-2, -1))
    resid = npf(st.quad_resid[0])[fin]
    assert np.all(np.abs(resid - ref["resid"].astype(np.float16)) <=
                  2e-3 * np.abs(ref["resid"]) + 1e-4 * trace)
    cs = npf(st.c_scale[0])[fin]
    assert cs.shape == ref["c_scale"].shape
    # the downstream score from the HIP-built and from the oracle-built summaries
    derive_page_params(st, case.seq_lens, B)
    nsh = npi(st.n_sel_hi)
    NB = case.kv_cache.shape[0]
    remap = np.full(NB, 0, np.int64)
    remap[fin] = np.arange(fin.size)
    btl = remap[npi(case.block_table).clip(0)].astype(np.int32)
    kw = dict(scale=case.scale, page=16, G=4, v_bits=8, c_bits=c_bits,
              max_pages=case.max_pages)
    q, sl = npf(case.q), npi(case.seq_lens)
    s_hip = osc.clse_score(q, npi(st.quad_mu[0])[fin], npf(st.mu_scale[0])[fin],
                           npi(st.reference_V(0))[fin], npf(st.V_scale[0])[fin],
                           npi(st.quad_c[0])[fin], cs, resid, btl, sl, nsh, **kw)
    s_ref = osc.clse_score(q, ref["mu"], ref["mu_scale"], ref["V"], ref["V_scale"], ref["c"],
                           ref["c_scale"], ref["resid"], btl, sl, nsh, **kw)
    for r in range(B):
        a, b = s_hip[r, :, :nsh[r]], s_ref[r, :, :nsh[r]]
        assert np.all(np.abs(a - b) <= 2e-2 * np.maximum(np.abs(b), 1)), np.abs(a - b).max()


def test_select_pages_clse_end_to_end():
    """The reference's default score (clse, r'=2, int4 coordinates per token, nrm combine)
    through selection (coverage 0.95) and the sparse decode, against the oracle."""
    announce("CLSE end to end: score -> nrm + coverage -> decode")
    B = 4
    case = make_case(B=B, ctx=(800, 3000), n_kv=8, G=4, heavy=0.05, table="perm", seed=91,
                     device=DEV, boost="keynorm")
    st = build_quad_state(case, rank=2, v_bits=4, combine="nrm", coords="lse", c_bits=4,
                          c_grain="token", coverage=0.95)
    derive_page_params(st, case.seq_lens, B)
    select_pages_clse(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale,
                      derive=False)
    out = torch.zeros(B, 32, 128, dtype=torch.bfloat16, device=DEV)
    sparse_paged_decode_batched(case.q, case.kv_cache, case.block_table, case.seq_lens, st,
                                out, ResidentVSource(case.kv_cache), scale=case.scale)
    torch.cuda.synchronize()
    inp = _oracle_inputs(case, st)
    nsh = inp["n_sel_hi"]
    ref_h = osc.clse_score(inp["q"], inp["mu"], inp["mu_scale"], inp["V"], inp["V_scale"],
                           inp["c"], inp["c_scale"], inp["resid"], inp["block_table"],
                           inp["seq_lens"], nsh, scale=case.scale, page=16, G=4, v_bits=4,
                           c_bits=4, max_pages=st.max_pages, combine="nrm")
    for r in range(B):
        n = int(nsh[r])
        assert rel_err(npf(st.score_h[r, :, :, :n]), ref_h[r, :, :, :n]) <= 1e-3
    tab, cnt, _ = osel.select(npf(st.score), npi(st.n_pages), nsh, npi(st.b_fix), sink=1,
                              max_pages=st.max_pages, mode=1, coverage=0.95, score_kind=1)
    assert np.array_equal(npi(st.page_table), tab) and np.array_equal(npi(st.page_cnt), cnt)
    frac = cnt.sum() / (npi(st.n_pages).sum() * 8)
    assert frac < 0.5, frac                 # the boosted pages concentrate the mass
    ref = odec.attend(inp["q"], npf(case.kv_cache[:, 0]), npf(case.kv_cache[:, 1]),
                      inp["block_table"], inp["seq_lens"], tab, cnt, scale=case.scale, G=4)
    assert np.allclose(npf(out), ref, atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("n_kv,G", [(1, 8), (2, 2), (4, 1), (16, 4)])
@pytest.mark.parametrize("rank,v_bits,c_bits,c_grain", [(2, 4, 4, "token"), (8, 8, 8, "page")])
def test_clse_head_layouts(n_kv, G, rank, v_bits, c_bits, c_grain):
    """Fewer than 8 kv heads per workgroup, two head groups, GQA groups 1 and 2, with the
    summaries written by the HIP builder (device K): contractions exact, per-head scores
    within 1e-3 of the oracle."""
    announce(f"CLSE heads n_kv={n_kv} G={G} r'={rank}")
    B = 2
    case = make_case(B=B, ctx=(300, 900), n_kv=n_kv, G=G, heavy=0.05, table="perm",
                     seed=90 + n_kv + G + rank, device=DEV)
    st = build_quad_state(case, rank=rank, v_bits=v_bits, combine="nrm", coords="lse",
                          c_bits=c_bits, c_grain=c_grain, budget=0.05)
    derive_page_params(st, case.seq_lens, B)
    MP = st.max_pages
    comb = torch.zeros(B, n_kv, MP, G, rank + 1, dtype=torch.int32, device=DEV)
    clse_score(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale, comb_out=comb)
    torch.cuda.synchronize()
    inp = _oracle_inputs(case, st)
    nsh = inp["n_sel_hi"]
    ref_comb = osc.quad_comb(inp["q"], inp["mu"], inp["V"], inp["block_table"], nsh, G=G,
                             v_bits=v_bits, max_pages=MP)
    ref = osc.clse_score(inp["q"], inp["mu"], inp["mu_scale"], inp["V"], inp["V_scale"],
                         inp["c"], inp["c_scale"], inp["resid"], inp["block_table"],
                         inp["seq_lens"], nsh, scale=case.scale, page=16, G=G, v_bits=v_bits,
                         c_bits=c_bits, max_pages=MP, combine="nrm")
    got_comb = npi(comb).astype(np.int64)
    got = npf(st.score_h)
    for r in range(B):
        n = int(nsh[r])
        assert np.array_equal(got_comb[r, :, :n], ref_comb[r, :, :n])
        assert rel_err(got[r, :, :, :n], ref[r, :, :, :n]) <= 1e-3
