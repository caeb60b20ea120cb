"""End-to-end Stage A + Stage B on GPU vs the oracle chain, and HIP-graph replay.

Config 0 of BASELINE.json (B=1, ctx 4096, 8B GQA, quad r'=8 summary, fixed 5% -> b=13)
and a small coverage-0.95 batch: the GPU selection must equal the oracle selection on the
GPU's own scores, the scores must match the oracle within 1e-3, and the attention output
must match the fp64 attention over the GPU-selected pages within 2e-2 / 1e-2.  The whole
step is captured in a HIP graph and every replay must equal the eager result.
"""
import numpy as np
import pytest
import torch

import oracle.decode as odec
import oracle.score as osc
import oracle.select as osel
from amass.attention.decode import ResidentVSource, sparse_paged_decode_batched
from amass.bench.synth import build_quad_state, config_case, make_case
from amass.selection import derive_page_params, select_pages_quad
from helpers import announce, case_to, npf, npi, rel_err, to_device

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _step(st, case, out, path="auto"):
    B = case.q.shape[0]
    select_pages_quad(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale,
                      derive=False)
    sparse_paged_decode_batched(case.q, case.kv_cache, case.block_table, case.seq_lens, st,
                                out, ResidentVSource(case.kv_cache), scale=case.scale,
                                path=path)


def _check(case, st, out, *, mode, cov, kind):
    B, MP, G = case.q.shape[0], st.max_pages, case.G
    nsh = npi(st.n_sel_hi)
    mu, mus, _, Vs, sg, _ = st.layer_state(0)
    V = st.reference_V(0)
    ref_h = osc.quad_score(npf(case.q), npi(mu), npf(mus), npi(V), npf(Vs), npf(sg),
                           npi(case.block_table), nsh, scale=case.scale, page=16, G=G,
                           v_bits=st.v_bits, max_pages=MP, combine="nrm")
    ref_s = osc.nrm_combine(ref_h, nsh)
    sc = npf(st.score)
    for r in range(B):
        assert rel_err(sc[r, :, :nsh[r]], ref_s[r, :, :nsh[r]]) <= 1e-3
    tab, cnt, _ = osel.select(sc, npi(st.n_pages), nsh, npi(st.b_fix), sink=1, max_pages=MP,
                              mode=mode, coverage=cov, tie_mode=0, score_kind=kind)
    assert np.array_equal(npi(st.page_table), tab) and np.array_equal(npi(st.page_cnt), cnt)
    ref = odec.attend(npf(case.q), npf(case.kv_cache[:, 0]), npf(case.kv_cache[:, 1]),
                      npi(case.block_table), npi(case.seq_lens), tab, cnt, scale=case.scale,
                      G=G)
    got = npf(out)
    assert np.allclose(got, ref, atol=2e-2, rtol=1e-2), float(np.abs(got - ref).max())


def test_config0_end_to_end():
    announce("config 0 end to end")
    case = config_case(0, seed=0)
    st = build_quad_state(case, rank=8, v_bits=8, combine="nrm", budget=0.05)
    to_device(st, DEV)
    case_to(case, DEV)
    derive_page_params(st, case.seq_lens, 1)
    out = torch.zeros(1, 32, 128, dtype=torch.bfloat16, device=DEV)
    _step(st, case, out)
    torch.cuda.synchronize()
    assert int(st.b_fix[0]) == 13
    assert (npi(st.page_cnt) == 13 + 2).all()      # b + sink + window
    _check(case, st, out, mode=0, cov=1.0, kind=1)


def test_coverage_batch_and_graph_replay():
    announce("coverage batch + graph replay")
    case = make_case(B=4, ctx=(1000, 3000), n_kv=8, G=4, heavy=0.05, seed=4)
    st = build_quad_state(case, rank=8, v_bits=4, combine="nrm", coverage=0.95)
    to_device(st, DEV)
    case_to(case, DEV)
    derive_page_params(st, case.seq_lens, 4)
    out = torch.zeros(4, 32, 128, dtype=torch.bfloat16, device=DEV)
    _step(st, case, out, path="split")
    torch.cuda.synchronize()
    _check(case, st, out, mode=1, cov=0.95, kind=1)
    eager = out.clone()
    eager_tab = st.page_table.clone()
    # capture score + select + decode (split path) in one HIP graph
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _step(st, case, out, path="split")
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _step(st, case, out, path="split")
    for i in range(4):
        out.zero_()
        st.page_table.fill_(-5)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        assert torch.equal(st.page_table, eager_tab), f"replay {i}"


def _replay_matches_eager(step, outs):
    """Capture `step` in one HIP graph, replay it four times (the outputs poisoned before
    each replay, eager work in between) and compare every replay with the eager run."""
    step()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for i in range(4):
        for o in outs:
            o.fill_(-5 if o.dtype == torch.int32 else float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), f"replay {i}"


@pytest.mark.parametrize("score", ["r8", "clse"])
def test_r8_and_clse_steps_graph_replay(score):
    """The r8 (top-b) and CLSE (coverage) steps -- score, select, decode -- replayed from
    one HIP graph equal the eager step bit for bit."""
    announce(f"{score} step graph replay")
    from amass.bench.synth import build_r8_state
    from amass.selection import select_pages_clse, select_pages_r8
    case = make_case(B=3, ctx=(1500, 4000), n_kv=8, G=4, heavy=0.05, seed=12)
    if score == "r8":
        st = build_r8_state(case, rank=8, vk_bits=8, c_bits=8, budget=0.05)
    else:
        st = build_quad_state(case, rank=2, v_bits=4, combine="nrm", coverage=0.95,
                              coords="lse", c_bits=4, c_grain="token")
    to_device(st, DEV)
    case_to(case, DEV)
    B = 3
    derive_page_params(st, case.seq_lens, B)
    out = torch.zeros(B, 32, 128, dtype=torch.bfloat16, device=DEV)
    sel = select_pages_r8 if score == "r8" else select_pages_clse

    def step():
        sel(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale, derive=False)
        sparse_paged_decode_batched(case.q, case.kv_cache, case.block_table, case.seq_lens,
                                    st, out, ResidentVSource(case.kv_cache), scale=case.scale)

    _replay_matches_eager(step, [out, st.page_table, st.page_cnt])
