"""The fp32 PyTorch restatement of the score -> select -> attend path (oracle/torch_path.py,
the CPU baseline bench.py times) against the pinned numpy oracle on seeded cases: scores
within 1e-4 * max(|ref|, 1), page tables and counts identical given the same scores (top-b
and coverage nucleus), attention within 1e-4."""
import numpy as np
import pytest
import torch

import oracle.decode as odec
import oracle.score as osc
import oracle.select as osel
import oracle.torch_path as tp
from amass.bench.synth import build_quad_state, make_case
from helpers import npf, npi, rel_err


@pytest.mark.parametrize("v_bits,boost", [(8, "sigma"), (4, "keynorm")])
def test_torch_path_matches_numpy_oracle(v_bits, boost):
    case = make_case(B=3, ctx=(700, 2000), n_kv=8, G=4, heavy=0.05, table="perm", seed=17,
                     boost=boost)
    st = build_quad_state(case, rank=8, v_bits=v_bits, combine="nrm", coverage=0.95)
    mu, mus, _, Vs, sg, _ = st.layer_state(0)
    V = st.reference_V(0)
    B, MP = 3, case.max_pages
    npg, nsh, bfix = tp.derive(case.seq_lens, 0.05, 16, 1, 1)
    onpg, onsh, obfix = osel.derive(npi(case.seq_lens), 0.05, 16, 1, 1)
    assert np.array_equal(npg.numpy(), onpg) and np.array_equal(nsh.numpy(), onsh)
    assert np.array_equal(bfix.numpy(), obfix)
    q = case.q.float()
    sh = tp.quad_score(q, mu, mus, V, Vs, sg, case.block_table, nsh, scale=case.scale,
                       page=16, G=4, v_bits=v_bits, max_pages=MP)
    ref_h = osc.quad_score(npf(case.q), npi(mu), npf(mus), npi(V), npf(Vs), npf(sg),
                           npi(case.block_table), onsh, scale=case.scale, page=16, G=4,
                           v_bits=v_bits, max_pages=MP, combine="nrm")
    for r in range(B):
        n = int(onsh[r])
        assert rel_err(sh[r, :, :, :n].numpy(), ref_h[r, :, :, :n]) <= 1e-4
    sc = tp.nrm_combine(sh, nsh)
    ref_s = osc.nrm_combine(sh.double().numpy(), onsh)
    for r in range(B):
        n = int(onsh[r])
        assert rel_err(sc[r, :, :n].numpy(), ref_s[r, :, :n]) <= 1e-5
    for mode in (0, 1):
        tab, cnt = tp.select(sc, npg, nsh, bfix, sink=1, max_pages=MP, mode=mode,
                             coverage=0.95, score_kind=1)
        otab, ocnt, _ = osel.select(sc.numpy(), onpg, onsh, obfix, sink=1, max_pages=MP,
                                    mode=mode, coverage=0.95, score_kind=1)
        assert np.array_equal(tab.numpy(), otab) and np.array_equal(cnt.numpy(), ocnt)
    K, Vc = case.kv_cache[:, 0], case.kv_cache[:, 1]
    out = tp.attend(q, K, Vc, case.block_table, case.seq_lens, tab, cnt, scale=case.scale,
                    G=4)
    ref = odec.attend(npf(case.q), npf(K), npf(Vc), npi(case.block_table),
                      npi(case.seq_lens), otab, ocnt, scale=case.scale, G=4)
    assert np.allclose(out.numpy(), ref, atol=1e-4, rtol=1e-4)


def test_torch_select_log_masses_and_empty_units():
    """score_kind 0 (log-mass scores) with a forced tie, and a request with seq_len 0."""
    rng = np.random.default_rng(3)
    sc = rng.normal(size=(2, 2, 40)).astype(np.float32)
    sc[0, 0, 5] = sc[0, 0, 9] = sc[0, 0].max() + 1          # a tie at the top
    npg = np.array([40, 0]); nsh = np.array([39, -1]); b = np.array([4, 1])
    for mode in (0, 1):
        tab, cnt = tp.select(torch.from_numpy(sc), npg, nsh, b, sink=1, max_pages=40,
                             mode=mode, coverage=0.9, score_kind=0)
        otab, ocnt, _ = osel.select(sc, npg, nsh, b, sink=1, max_pages=40, mode=mode,
                                    coverage=0.9, score_kind=0)
        assert np.array_equal(tab.numpy(), otab) and np.array_equal(cnt.numpy(), ocnt)


def test_torch_exp_det_is_the_oracle_exp_det():
    x = np.concatenate([np.linspace(-90, 0, 200001, dtype=np.float32),
                        np.array([0.0, -0.0, -1e-30, -79.99], np.float32)])
    got = tp.exp_det(torch.from_numpy(x)).numpy()
    assert np.array_equal(got.view(np.uint32), osel.exp_det(x).view(np.uint32))
