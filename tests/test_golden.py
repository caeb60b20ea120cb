"""The committed golden fixtures (tests/golden/*.npz, written by make_golden.py).

CPU: the oracle, rerun on each fixture's inputs, still gives the frozen outputs
(bit-exact for integer / index outputs, 1e-12 relative for float64 ones).
GPU: the HIP path, fed the same inputs through the C-ABI, matches the frozen outputs to
the parity bars: int32 contractions and page sets bit-exact, quad scores 1e-3 relative,
r8 scores 1e-3, attention 2e-2 abs / 1e-2 rel, tier maps bit-exact.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

import make_golden as mg

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DEV = "cuda"


def _load(name):
    z = np.load(os.path.join(HERE, f"{name}.npz"))
    inp = {k[3:]: z[k] for k in z.files if k.startswith("in_")}
    out = {k[4:]: z[k] for k in z.files if k.startswith("out_")}
    return inp, out


def _same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape and a.dtype.kind == b.dtype.kind
    if a.dtype.kind == "f":
        assert np.allclose(a, b, rtol=1e-12, atol=1e-300, equal_nan=True)
    else:
        assert np.array_equal(a, b)


@pytest.mark.parametrize("name", sorted(mg.CASES))
def test_oracle_reproduces_fixture(name):
    inp, out = _load(name)
    fresh_in = mg.CASES[name][0]()
    for k, v in inp.items():
        _same(fresh_in[k], v)
    fresh = mg.CASES[name][1](inp)
    assert set(fresh) == set(out)
    for k, v in out.items():
        _same(fresh[k], v)


# --------------------------------------------------------------------------- GPU
def _t(x, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x))
    return (t if dtype is None else t.to(dtype)).to(DEV)


def _rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float((np.abs(np.asarray(got, np.float64) - ref) / np.maximum(np.abs(ref), 1)).max())


@pytest.mark.gpu
@pytest.mark.parametrize("name,rank,v_bits", [("quad_i8", 8, 8), ("quad_i4_r4", 4, 4)])
def test_gpu_quad_fixture(name, rank, v_bits):
    import torch
    from amass.selection import QuadState  # noqa: F401
    from amass.selection.quad_score import nrm_combine, quad_score_launch
    from helpers import announce, npf, npi
    announce(f"golden {name}")
    inp, out = _load(name)
    R, H, d = inp["q"].shape
    NB, n_kv = inp["mu"].shape[:2]
    G = H // n_kv
    MP = inp["block_table"].shape[1]
    for combine in ("max", "nrm"):
        st = QuadState(DEV, num_layers=1, num_blocks=NB, n_kv=n_kv, G=G, head_dim=d, page=16,
                       max_reqs=R, max_pages=MP, rank=rank, v_bits=v_bits, combine=combine)
        st.load_reference(0, inp["mu"], inp["mu_scale"], inp["V"], inp["V_scale"], inp["sig2"])
        st.n_sel_hi.copy_(_t(inp["n_sel_hi"]))
        comb = torch.zeros(R, n_kv, MP, G, rank + 1, dtype=torch.int32, device=DEV)
        quad_score_launch(st, 0, _t(inp["q"], torch.bfloat16), _t(inp["block_table"]), R,
                          1 / np.sqrt(128), comb_out=comb)
        if combine == "nrm":
            nrm_combine(st, R)
        torch.cuda.synchronize()
        for r in range(R):
            n = int(inp["n_sel_hi"][r])
            assert np.array_equal(npi(comb)[r, :, :n], out["comb"][r, :, :n])
            if combine == "max":
                assert _rel(npf(st.score)[r, :, :n], out["score_max"][r, :, :n]) <= 1e-3
            else:
                assert _rel(npf(st.score_h)[r, :, :, :n], out["score_h"][r, :, :, :n]) <= 1e-3
                assert _rel(npf(st.score)[r, :, :n], out["nrm"][r, :, :n]) <= 1e-3


@pytest.mark.gpu
def test_gpu_r8_fixture():
    import torch
    from amass.selection import R8State
    from amass.selection.score import r8_score
    from helpers import announce, npf
    announce("golden r8")
    inp, out = _load("r8")
    R, H, d = inp["q"].shape
    NB, n_kv = inp["mu"].shape[:2]
    MP = inp["block_table"].shape[1]
    st = R8State(DEV, num_layers=1, num_blocks=NB, n_kv=n_kv, G=H // n_kv, head_dim=d,
                 page=16, max_reqs=R, max_pages=MP, rank=8)
    st.load_reference(0, *(_t(inp[k]) for k in ("mu", "mu_scale", "Vk", "Vk_scale", "c",
                                                 "c_scale")))
    st.n_sel_hi.copy_(_t(inp["n_sel_hi"]))
    r8_score(st, 0, _t(inp["q"], torch.bfloat16), _t(inp["block_table"]), _t(inp["seq_lens"]),
             R, 1 / np.sqrt(128))
    torch.cuda.synchronize()
    for r in range(R):
        n = int(inp["n_sel_hi"][r])
        assert _rel(npf(st.score)[r, :, :n], out["score"][r, :, :n]) <= 1e-3


@pytest.mark.gpu
def test_gpu_select_fixture():
    from amass.selection import QuadState, coverage_select, topb_select
    from helpers import announce, npi
    announce("golden select")
    inp, out = _load("select")
    R, n_kv, MP = inp["score"].shape
    for key in sorted(k[:-4] for k in out if k.endswith("_tab")):
        mode, tie, kind = (int(key[1]), int(key[4]), int(key[7]))
        st = QuadState(DEV, num_layers=1, num_blocks=4, n_kv=n_kv, G=4, head_dim=128, page=16,
                       max_reqs=R, max_pages=MP, rank=2, combine="nrm" if kind else "max")
        sc = np.abs(inp["score"]) if kind == 1 else inp["score"]
        st.score.copy_(_t(sc))
        st.n_pages.copy_(_t(inp["n_pages"]))
        st.n_sel_hi.copy_(_t(inp["n_sel_hi"]))
        st.b_fix.copy_(_t(inp["b_fix"]))
        tm = ["index", "all"][tie]
        if mode == 0:
            topb_select(st, R, tie_mode=tm)
        else:
            coverage_select(st, R, 0.9, tie_mode=tm)
        assert np.array_equal(npi(st.page_table), out[key + "_tab"]), key
        assert np.array_equal(npi(st.page_cnt), out[key + "_cnt"]), key
        if tie == 0:
            assert np.array_equal(npi(st.n_sel), out[key + "_nsel"]), key


@pytest.mark.gpu
def test_gpu_decode_fixture():
    import torch
    from amass.attention.decode import (ResidentVSource, dense_paged_decode,
                                        ensure_stage_b_buffers, sparse_paged_decode_batched)
    from amass.selection import QuadState
    from helpers import announce, npf
    announce("golden decode")
    inp, out = _load("decode")
    R, H, d = inp["q"].shape
    NB, P, n_kv, _ = inp["K"].shape
    kv = torch.stack([_t(inp["K"], torch.bfloat16), _t(inp["V"], torch.bfloat16)], dim=1)
    q = _t(inp["q"], torch.bfloat16)
    bt, sl = _t(inp["block_table"]), _t(inp["seq_lens"])
    st = QuadState(DEV, num_layers=1, num_blocks=NB, n_kv=n_kv, G=H // n_kv, head_dim=d,
                   page=P, max_reqs=R, max_pages=NB, rank=2)
    st.page_table.copy_(_t(inp["page_table"]))
    st.page_cnt.copy_(_t(inp["page_cnt"]))
    ensure_stage_b_buffers(st, DEV)
    for path in ("split", "fused"):
        o = torch.zeros(R, H, d, dtype=torch.bfloat16, device=DEV)
        sparse_paged_decode_batched(q, kv, bt, sl, st, o, ResidentVSource(kv),
                                    scale=1 / np.sqrt(128), path=path)
        torch.cuda.synchronize()
        assert np.allclose(npf(o), out["sparse"], atol=2e-2, rtol=1e-2), path
    o = torch.zeros(R, H, d, dtype=torch.bfloat16, device=DEV)
    dense_paged_decode(q, kv, bt, sl, st, o, scale=1 / np.sqrt(128))
    torch.cuda.synchronize()
    assert np.allclose(npf(o), out["dense"], atol=2e-2, rtol=1e-2)


@pytest.mark.gpu
def test_gpu_tier_fixture():
    import torch
    from amass.tier import Tier
    from helpers import announce, npi
    announce("golden tier")
    inp, out = _load("tier")
    steps, R, n_kv, MP = inp["page_tables"].shape
    NB, S = int(inp["NB"][0]), int(inp["slots"][0])
    tier = Tier(num_layers=1, num_blocks=NB, n_kv=n_kv, page=16, d=128, hot_slots=S,
                max_reqs=R, max_pages=MP, device=DEV, v_blocks=4)
    kv_v = torch.zeros(NB, 16, n_kv, 128, dtype=torch.bfloat16, device=DEV)
    tier.flush_layer(0, kv_v)
    res = tier.residency
    res.clock.fill_(0)                  # the fixture's plan starts from clock 0
    bt, sl = _t(inp["block_table"]), _t(inp["seq_lens"])
    for s in range(steps):
        res.gather_plan(0, _t(inp["page_tables"][s]), _t(inp["page_cnts"][s]), bt, sl, R)
        torch.cuda.synchronize()
        assert np.array_equal(npi(res.page2slot[0]).astype(np.int64), out[f"s{s}_page2slot"])
        assert np.array_equal(npi(res.slot2page[0]).astype(np.int64), out[f"s{s}_slot2page"])
        assert np.array_equal(npi(res.lru_clock[0]).astype(np.int64), out[f"s{s}_lru"])
