"""GPU parity of the quad and r8 page-score kernels against the CPU oracle.

Bar: the int32 d-contractions (comb_out) are bit-exact against int64 brute force; quad
scores within |d| <= 1e-3 * max(|ref|, 1) of the fp64 oracle with unquantised q (the
Triton reference semantics, tolerance 1e-3 relative) and within 2e-5 of the
oracle that uses the 2-limb q code; nrm-combined scores within 1e-4 relative; r8 scores
within 1e-3 likewise.
"""
import numpy as np
import pytest
import torch

import oracle.score as osc
import oracle.select as osel
from amass.bench.synth import build_quad_state, build_r8_state, make_case
from amass.selection import derive_page_params, nrm_combine, r8_score
from amass.selection.quad_score import quad_score_launch
from helpers import announce, npf, npi, rel_err, to_device, case_to

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _quad_setup(rank, v_bits, G, combine, seed=0, B=3):
    case = make_case(B=B, ctx=(300, 1400), n_kv=8, G=G, heavy=0.05, table="perm", seed=seed)
    st = build_quad_state(case, rank=rank, v_bits=v_bits, combine=combine, budget=0.05)
    to_device(st, DEV)
    case_to(case, DEV)
    derive_page_params(st, case.seq_lens, B)
    return case, st


def _oracle_inputs(case, st):
    mu, mus, _, Vs, sg, _ = st.layer_state(0)
    V = st.reference_V(0)
    return dict(q=npf(case.q), mu=npi(mu), mu_scale=npf(mus), V=npi(V), V_scale=npf(Vs),
                sig2=npf(sg), block_table=npi(case.block_table), n_sel_hi=npi(st.n_sel_hi))


@pytest.mark.parametrize("rank,v_bits", [(2, 8), (4, 8), (8, 8), (2, 4), (4, 4), (8, 4)])
@pytest.mark.parametrize("G", [4, 8])
def test_quad_comb_exact_and_scores(rank, v_bits, G):
    announce(f"quad rank={rank} v_bits={v_bits} G={G}")
    case, st = _quad_setup(rank, v_bits, G, "max")
    B, MP = case.q.shape[0], st.max_pages
    npg, nsh, bfix = osel.derive(npi(case.seq_lens), st.budget, 16, 1, 1)
    assert np.array_equal(npi(st.n_pages), npg) and np.array_equal(npi(st.n_sel_hi), nsh)
    assert np.array_equal(npi(st.b_fix), bfix)
    comb = torch.zeros(B, 8, MP, G, rank + 1, dtype=torch.int32, device=DEV)
    st.score.fill_(float("nan"))
    quad_score_launch(st, 0, case.q, case.block_table, B, case.scale, comb_out=comb)
    torch.cuda.synchronize()
    o = _oracle_inputs(case, st)
    ref_comb = osc.quad_comb(o["q"], o["mu"], o["V"], o["block_table"], o["n_sel_hi"], G=G,
                             v_bits=v_bits, max_pages=MP)
    got = npi(comb).astype(np.int64)
    for r in range(B):
        n = int(nsh[r])
        assert np.array_equal(got[r, :, :n], ref_comb[r, :, :n]), f"comb mismatch req {r}"
    kw = dict(scale=case.scale, page=16, G=G, v_bits=v_bits, max_pages=MP)
    ref_f = osc.quad_score(**o, **kw, combine="max", q_mode="float")
    ref_l = osc.quad_score(**o, **kw, combine="max", q_mode="limbs")
    sc = npf(st.score)
    for r in range(B):
        n = int(nsh[r])
        assert rel_err(sc[r, :, :n], ref_f[r, :, :n]) <= 1e-3
        assert rel_err(sc[r, :, :n], ref_l[r, :, :n]) <= 2e-5


@pytest.mark.parametrize("rank,v_bits", [(8, 8), (2, 4)])
def test_quad_nrm(rank, v_bits):
    announce(f"quad nrm rank={rank} v_bits={v_bits}")
    case, st = _quad_setup(rank, v_bits, 4, "nrm", seed=3)
    B, MP = case.q.shape[0], st.max_pages
    quad_score_launch(st, 0, case.q, case.block_table, B, case.scale)
    nrm_combine(st, B)
    torch.cuda.synchronize()
    o = _oracle_inputs(case, st)
    ref_h = osc.quad_score(**o, scale=case.scale, page=16, G=4, v_bits=v_bits, max_pages=MP,
                           combine="nrm", q_mode="float")
    sh = npf(st.score_h)
    nsh = npi(st.n_sel_hi)
    for r in range(B):
        n = int(nsh[r])
        assert rel_err(sh[r, :, :, :n], ref_h[r, :, :, :n]) <= 1e-3
    # nrm of the GPU's own per-head scores: fp64 oracle vs the fp32 kernel
    with np.errstate(invalid="ignore"):   # pages past n_sel_hi hold unwritten bits
        ref_n = osc.nrm_combine(sh.astype(np.float64), nsh)
    sc = npf(st.score)
    for r in range(B):
        n = int(nsh[r])
        assert rel_err(sc[r, :, :n], ref_n[r, :, :n]) <= 1e-5


def test_quad_padded_rows_untouched():
    """Rows with seq_len 0 (n_sel_hi < 0) write nothing."""
    announce("quad padded rows")
    case = make_case(B=2, ctx=(200, 400), n_kv=8, G=4, seed=5)
    st = build_quad_state(case, rank=2, v_bits=8, combine="max", max_reqs=3)
    to_device(st, DEV)
    case_to(case, DEV)
    sl = torch.cat([case.seq_lens, torch.zeros(1, dtype=torch.int32, device=DEV)])
    bt = torch.cat([case.block_table, case.block_table[:1]])
    q = torch.cat([case.q, case.q[:1]])
    derive_page_params(st, sl, 3)
    st.score.fill_(123.0)
    quad_score_launch(st, 0, q, bt, 3, case.scale)
    torch.cuda.synchronize()
    assert bool((st.score[2] == 123.0).all())


R8_CASES = ([(8, vb, cb, G) for vb in (8, 4) for cb in (8, 4) for G in (1, 2, 4, 8)]
            + [(4, vb, cb, G) for vb in (8, 4) for cb in (8, 4) for G in (2, 4)])


@pytest.mark.parametrize("rank,vk_bits,c_bits,G", R8_CASES)
def test_r8_comb_exact_and_scores(rank, vk_bits, c_bits, G):
    """Every (rank, Vk bits, c bits) record layout and every token split of the kernel
    (G = 8: 16 tokens per lane, G = 4: 8, G <= 2: 4, with 8-byte c rows at r = 4 int4)."""
    announce(f"r8 rank={rank} vk={vk_bits} c={c_bits} G={G}")
    case = make_case(B=3, ctx=(300, 1400), n_kv=8, G=G, seed=11 + G + rank)
    st = build_r8_state(case, rank=rank, vk_bits=vk_bits, c_bits=c_bits)
    to_device(st, DEV)
    case_to(case, DEV)
    B, MP = 3, st.max_pages
    derive_page_params(st, case.seq_lens, B)
    comb = torch.zeros(B, 8, MP, G, rank + 1, dtype=torch.int32, device=DEV)
    r8_score(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale, comb_out=comb)
    torch.cuda.synchronize()
    mu, mus, _, Vks, c, cs, _ = st.layer_state(0)
    Vk = st.reference_Vk(0)
    nsh = npi(st.n_sel_hi)
    ref_comb = osc.r8_comb(npf(case.q), npi(mu), npi(Vk), npi(case.block_table), nsh, G=G,
                           vk_bits=vk_bits, max_pages=MP)
    got = npi(comb).astype(np.int64)
    for r in range(B):
        n = int(nsh[r])
        assert np.array_equal(got[r, :, :n], ref_comb[r, :, :n])
    ref = osc.r8_score(npf(case.q), npi(mu), npf(mus), npi(Vk), npf(Vks), npi(c), npf(cs),
                       npi(case.block_table), npi(case.seq_lens), nsh, scale=case.scale,
                       page=16, G=G, vk_bits=vk_bits, c_bits=c_bits, max_pages=MP)
    # the production instance (no comb_out) writes the same scores
    sc_comb = npf(st.score).copy()
    r8_score(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale)
    torch.cuda.synchronize()
    sc = npf(st.score)
    for r in range(B):
        n = int(nsh[r])
        assert rel_err(sc[r, :, :n], sc_comb[r, :, :n]) <= 1e-6
    for r in range(B):
        n = int(nsh[r])
        assert rel_err(sc[r, :, :n], ref[r, :, :n]) <= 1e-3


HEAD_CASES = [(1, 8), (2, 2), (4, 1), (16, 4)]


@pytest.mark.parametrize("n_kv,G", HEAD_CASES)
@pytest.mark.parametrize("rank,v_bits", [(8, 8), (2, 4)])
def test_quad_head_layouts(n_kv, G, rank, v_bits):
    """Workgroups of fewer than 8 kv heads (n_kv 1, 2, 4) and two head groups (n_kv 16),
    and GQA groups 1 and 2 (spare limb rows zero): int32 contractions exact, max scores
    within the limb oracle's 2e-5."""
    announce(f"quad heads n_kv={n_kv} G={G} rank={rank} v_bits={v_bits}")
    case = make_case(B=2, ctx=(300, 900), n_kv=n_kv, G=G, heavy=0.05, table="perm",
                     seed=31 + n_kv + G)
    st = build_quad_state(case, rank=rank, v_bits=v_bits, combine="max", budget=0.05)
    to_device(st, DEV)
    case_to(case, DEV)
    B, MP = 2, st.max_pages
    derive_page_params(st, case.seq_lens, B)
    comb = torch.zeros(B, n_kv, MP, G, rank + 1, dtype=torch.int32, device=DEV)
    quad_score_launch(st, 0, case.q, case.block_table, B, case.scale, comb_out=comb)
    torch.cuda.synchronize()
    o = _oracle_inputs(case, st)
    nsh = npi(st.n_sel_hi)
    ref_comb = osc.quad_comb(o["q"], o["mu"], o["V"], o["block_table"], o["n_sel_hi"], G=G,
                             v_bits=v_bits, max_pages=MP)
    got = npi(comb).astype(np.int64)
    ref_l = osc.quad_score(**o, scale=case.scale, page=16, G=G, v_bits=v_bits, max_pages=MP,
                           combine="max", q_mode="limbs")
    sc = npf(st.score)
    for r in range(B):
        n = int(nsh[r])
        assert np.array_equal(got[r, :, :n], ref_comb[r, :, :n]), f"comb mismatch req {r}"
        assert rel_err(sc[r, :, :n], ref_l[r, :, :n]) <= 2e-5


@pytest.mark.parametrize("n_kv,G", HEAD_CASES)
def test_r8_head_layouts(n_kv, G):
    """The r8 kernel over the same head layouts: contractions exact, scores within 1e-3 of
    the fp64 oracle."""
    announce(f"r8 heads n_kv={n_kv} G={G}")
    case = make_case(B=2, ctx=(300, 900), n_kv=n_kv, G=G, seed=41 + n_kv + G)
    st = build_r8_state(case, rank=8, vk_bits=8, c_bits=8)
    to_device(st, DEV)
    case_to(case, DEV)
    B, MP = 2, st.max_pages
    derive_page_params(st, case.seq_lens, B)
    comb = torch.zeros(B, n_kv, MP, G, 9, dtype=torch.int32, device=DEV)
    r8_score(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale, comb_out=comb)
    torch.cuda.synchronize()
    mu, mus, _, Vks, c, cs, _ = st.layer_state(0)
    Vk = st.reference_Vk(0)
    nsh = npi(st.n_sel_hi)
    ref_comb = osc.r8_comb(npf(case.q), npi(mu), npi(Vk), npi(case.block_table), nsh, G=G,
                           vk_bits=8, max_pages=MP)
    ref = osc.r8_score(npf(case.q), npi(mu), npf(mus), npi(Vk), npf(Vks), npi(c), npf(cs),
                       npi(case.block_table), npi(case.seq_lens), nsh, scale=case.scale,
                       page=16, G=G, vk_bits=8, c_bits=8, max_pages=MP)
    got = npi(comb).astype(np.int64)
    sc = npf(st.score)
    for r in range(B):
        n = int(nsh[r])
        assert np.array_equal(got[r, :, :n], ref_comb[r, :, :n])
        assert rel_err(sc[r, :, :n], ref[r, :, :n]) <= 1e-3


@pytest.mark.parametrize("vk_bits,c_bits,G", [(8, 8, 4), (8, 4, 8), (4, 8, 2)])
def test_r8_page_f32_scale(vk_bits, c_bits, G):
    """The per-page fp32 c scale (c_grain "page_f32", config 2's "per-page fp32
    scale"): int32 contractions exact (they do not depend on the scale format), scores
    within 1e-3 of the fp64 oracle fed the same fp32 scales."""
    announce(f"r8 page_f32 vk={vk_bits} c={c_bits} G={G}")
    case = make_case(B=3, ctx=(300, 1400), n_kv=8, G=G, seed=71 + G + c_bits)
    st = build_r8_state(case, rank=8, vk_bits=vk_bits, c_bits=c_bits, c_grain="page_f32")
    to_device(st, DEV)
    case_to(case, DEV)
    B, MP = 3, st.max_pages
    derive_page_params(st, case.seq_lens, B)
    comb = torch.zeros(B, 8, MP, G, 9, dtype=torch.int32, device=DEV)
    r8_score(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale, comb_out=comb)
    torch.cuda.synchronize()
    sc_comb = npf(st.score).copy()
    r8_score(st, 0, case.q, case.block_table, case.seq_lens, B, case.scale)
    torch.cuda.synchronize()
    mu, mus, _, Vks, c, cs, _ = st.layer_state(0)
    assert bool((npf(st.c_scale_f32[0]) > 0).any())
    Vk = st.reference_Vk(0)
    nsh = npi(st.n_sel_hi)
    ref_comb = osc.r8_comb(npf(case.q), npi(mu), npi(Vk), npi(case.block_table), nsh, G=G,
                           vk_bits=vk_bits, max_pages=MP)
    ref = osc.r8_score(npf(case.q), npi(mu), npf(mus), npi(Vk), npf(Vks), npi(c), npf(cs),
                       npi(case.block_table), npi(case.seq_lens), nsh, scale=case.scale,
                       page=16, G=G, vk_bits=vk_bits, c_bits=c_bits, max_pages=MP)
    got = npi(comb).astype(np.int64)
    sc = npf(st.score)
    for r in range(B):
        n = int(nsh[r])
        assert np.array_equal(got[r, :, :n], ref_comb[r, :, :n])
        assert rel_err(sc[r, :, :n], sc_comb[r, :, :n]) <= 1e-6
        assert rel_err(sc[r, :, :n], ref[r, :, :n]) <= 1e-3


@pytest.mark.parametrize("kind", ["quad", "clse"])
def test_records_beyond_2gib(kind):
    """The score kernels address records with 32-bit offsets from the layer's base (block
    * rec_sb, plus head and lane bytes, summed unsigned): records placed at block ids whose
    offsets exceed 2^31 bytes score bit for bit as the same records at low block ids."""
    from amass.selection import QuadState
    from amass.selection.quad_score import clse_score
    announce(f"records beyond 2 GiB: {kind}")
    B, MP, n_kv, G = 2, 64, 8, 4
    if kind == "quad":
        kw = dict(rank=8, v_bits=8)
    else:
        kw = dict(rank=2, v_bits=4, coords="lse", c_bits=4, c_grain="token")
    rec_block = n_kv * (8 * 128 + 176 if kind == "quad" else 2 * 64 + 128 + 16 + 48)
    hi0 = (1 << 31) // rec_block + 1                     # first block past 2 GiB
    NB = hi0 + B * MP
    st = QuadState(DEV, num_layers=1, num_blocks=NB, n_kv=n_kv, G=G, head_dim=128, page=16,
                   max_reqs=B, max_pages=MP, combine="max", **kw)
    assert st.quad_rec.stride(1) == rec_block and NB * rec_block < (1 << 32)
    g = torch.Generator(device=DEV).manual_seed(7)
    lo = torch.arange(B * MP, device=DEV)
    raw = torch.randint(-127, 128, (B * MP, st.quad_rec.shape[-1]), generator=g,
                        device=DEV, dtype=torch.int8)
    st.quad_rec[0, lo] = raw
    # finite fp16 scales over the random bytes
    half = lambda *s: (torch.rand(*s, generator=g, device=DEV) * 0.02 + 0.01).half()  # noqa: E731
    st.V_scale[0, lo] = half(B * MP, n_kv, st.r)
    st.mu_scale[0, lo] = half(B * MP, n_kv)
    if kind == "quad":
        st.quad_sig2[0, lo] = half(B * MP, n_kv, st.r)
    else:
        st._c_scale16[0, lo] = half(B * MP, n_kv, 16)
        st.quad_resid[0, lo] = half(B * MP, n_kv)
    st.quad_rec[0, hi0 + lo] = st.quad_rec[0, lo]
    q = torch.randn(B, n_kv * G, 128, generator=g, device=DEV).to(torch.bfloat16)
    sl = torch.full((B,), MP * 16, dtype=torch.int32, device=DEV)
    derive_page_params(st, sl, B)
    bt_lo = lo.view(B, MP).to(torch.int32)
    scores = []
    for bt in (bt_lo, bt_lo + hi0):
        st.score.fill_(float("nan"))
        if kind == "quad":
            quad_score_launch(st, 0, q, bt.contiguous(), B, 128 ** -0.5)
        else:
            clse_score(st, 0, q, bt.contiguous(), sl, B, 128 ** -0.5)
        torch.cuda.synchronize()
        scores.append(st.score.clone())
    nsh = int(st.n_sel_hi[0])
    assert torch.isfinite(scores[0][:, :, :nsh]).all()
    assert torch.equal(scores[0][:, :, :nsh], scores[1][:, :, :nsh])
    del st
    torch.cuda.empty_cache()
