"""Pins for the CPU oracle: closed forms, invariants, brute force and hand-worked cases.

The reference ships no tests or golden vectors for this path, so each oracle function is
checked here against something it does not restate: the mathematics the reference's
docstrings state (selection/quad_score.py:7-24, selection/score.py:3-12), a brute force
over all candidates, or a small case worked by hand.  Every check is chosen so that a
plausible slip (a dropped factor, a flipped sign or order, an off-by-one) fails it.
"""
from __future__ import annotations

import itertools
import math

import numpy as np
import pytest

import oracle.decode as odec
import oracle.quant as oq
import oracle.score as osc
import oracle.select as osel
import oracle.tier as otier
from helpers import exp_det_fused, mass_cut_case


def _hadamard(n):
    h = np.array([[1.0]])
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


# ----------------------------------------------------------------------------- quant
def test_q_limbs_identity_and_range():
    rng = np.random.default_rng(0)
    q = rng.standard_normal((64, 128)).astype(np.float32) * rng.uniform(1e-3, 30, (64, 1))
    qi, hi, lo, qs = oq.q_limbs(q)
    assert np.array_equal(128 * hi + lo, qi)
    assert np.abs(hi).max() <= 127 and np.abs(lo).max() <= 127
    assert np.abs(qi).max() == 16383
    # the amax element maps to +-16383 and every code is within half a step of q/qs
    am = np.abs(q).argmax(axis=1)
    assert np.all(np.abs(qi[np.arange(64), am]) == 16383)
    err = np.abs(qi - q.astype(np.float64) / qs[:, None].astype(np.float64))
    assert err.max() <= 0.5 + 1e-3


def test_q_limbs_zero_vector():
    qi, hi, lo, qs = oq.q_limbs(np.zeros((1, 128), np.float32))
    assert not qi.any() and not hi.any() and not lo.any() and qs[0] > 0


@pytest.mark.parametrize("bits", [8, 4])
def test_quant_round_trip(bits):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((32, 128)).astype(np.float32)
    code, s = oq.quant(x, axis=-1, bits=bits)
    lvl = (1 << (bits - 1)) - 1
    assert np.abs(code).max() == lvl
    assert np.all(np.abs(x - code * s) <= s / 2 * (1 + 1e-6))
    assert np.array_equal(np.abs(code).max(axis=-1), np.full(32, lvl))


def test_pack_i4_layout_and_round_trip():
    # lo nibble = even column: [1, -2] -> 0xE1
    assert oq.pack_i4(np.array([[1, -2]], np.int8)).view(np.uint8)[0, 0] == 0xE1
    vals = np.array(list(itertools.product(range(-7, 8), repeat=2)), np.int8)
    assert np.array_equal(oq.unpack_i4(oq.pack_i4(vals)), vals)


# ----------------------------------------------------------------------------- quad
def _structured_page(rng, d=128, P=16, r=8, lam=None):
    """A page whose centred keys span exactly r orthonormal directions with exactly
    representable int8 codes: column k = +-1/4 on a disjoint support of 16 dims."""
    V = np.zeros((d, r))
    perm = rng.permutation(d)
    for k in range(r):
        sup = perm[16 * k:16 * (k + 1)]
        V[sup, k] = rng.choice([-1.0, 1.0], 16) / 4.0
    H = _hadamard(P)[:, 1:r + 1]                 # centred, orthogonal, |col|^2 = P
    lam = rng.uniform(0.5, 3.0, r) if lam is None else lam
    A = H * np.sqrt(lam / P)                      # scatter eigenvalue of column k = lam_k
    mu_code = rng.integers(-127, 128, d).astype(np.int8)
    mu_scale = 1.0 / 64
    mu = mu_code * mu_scale
    K = mu[None, :] + A @ V.T                     # (P, d)
    return K, V, lam, mu_code, mu_scale


def _quad_from_summary(q, V, lam, mu_code, mu_scale, scale, P=16):
    d, r = V.shape
    v_code = np.rint(V * 4 * 127).astype(np.int8)[None, None]      # (1, 1, d, r)
    v_scale = np.full((1, 1, r), 1.0 / (4 * 127))
    return osc.quad_score(q[None, None].astype(np.float32), mu_code[None, None],
                          np.array([[mu_scale]]), v_code, v_scale, lam[None, None],
                          np.zeros((1, 1), np.int32), np.array([1]), scale=scale, page=P,
                          G=1, v_bits=8, max_pages=1)[0, 0, 0]


def test_quad_closed_form_from_raw_keys():
    """S = s q.mu + s^2/2 q^T Cov q, Cov = centred scatter / P, computed from the keys."""
    rng = np.random.default_rng(2)
    for _ in range(5):
        K, V, lam, mu_code, mu_scale = _structured_page(rng)
        q = (rng.standard_normal(128) * 2).astype(np.float32).astype(np.float64)
        scale = 1 / math.sqrt(128)
        mu = K.mean(axis=0)
        C = (K - mu).T @ (K - mu) / K.shape[0]
        want = scale * q @ mu + 0.5 * scale * scale * q @ C @ q
        got = _quad_from_summary(q, V, lam, mu_code, mu_scale, scale)
        assert abs(got - want) <= 1e-9 * max(1.0, abs(want))


def test_quad_eigen_sign_invariance():
    rng = np.random.default_rng(3)
    K, V, lam, mu_code, mu_scale = _structured_page(rng)
    q = rng.standard_normal(128)
    a = _quad_from_summary(q, V, lam, mu_code, mu_scale, 0.1)
    V2 = V.copy()
    V2[:, [1, 5]] *= -1
    b = _quad_from_summary(q, V2, lam, mu_code, mu_scale, 0.1)
    assert a == pytest.approx(b, rel=1e-12)


def test_quad_gaussian_page_matches_log_mean_exp():
    """For small logit spread the Gaussian-MGF score approximates log-mean-exp of the
    page's true logits to fourth order (symmetric coefficients: no third cumulant)."""
    rng = np.random.default_rng(4)
    K, V, lam, mu_code, mu_scale = _structured_page(rng, lam=np.full(8, 0.02))
    q = rng.standard_normal(128)
    scale = 1 / math.sqrt(128)
    logits = scale * K @ q
    lme = logits.max() + math.log(np.mean(np.exp(logits - logits.max())))
    got = _quad_from_summary(q, V, lam, mu_code, mu_scale, scale)
    assert abs(got - lme) < 1e-4


def test_quad_group_max_and_nrm_layout():
    rng = np.random.default_rng(5)
    R, NB, n_kv, G, d, r = 2, 6, 2, 3, 128, 4
    q = rng.standard_normal((R, n_kv * G, d)).astype(np.float32)
    mu = rng.integers(-127, 128, (NB, n_kv, d)).astype(np.int8)
    mus = rng.uniform(0.01, 0.02, (NB, n_kv)).astype(np.float32)
    V = rng.integers(-127, 128, (NB, n_kv, d, r)).astype(np.int8)
    Vs = rng.uniform(0.001, 0.01, (NB, n_kv, r)).astype(np.float32)
    sg = rng.uniform(0.1, 2, (NB, n_kv, r)).astype(np.float32)
    bt = np.array([[3, 1, 4, 0, 5, 2], [5, 4, 3, 2, 1, 0]], np.int32)
    nsh = np.array([5, 3])
    kw = dict(scale=0.09, page=16, G=G, v_bits=8, max_pages=6)
    sh = osc.quad_score(q, mu, mus, V, Vs, sg, bt, nsh, combine="nrm", **kw)
    sm = osc.quad_score(q, mu, mus, V, Vs, sg, bt, nsh, combine="max", **kw)
    assert np.isnan(sh[0, :, :, 5:]).all() and np.isnan(sh[1, :, :, 3:]).all()
    assert np.allclose(sh[0, :, :, :5].max(axis=1), sm[0, :, :5])
    # request 0, kv head 1, group member 2, logical page 2 -> block 4, by hand
    qq = q[0, 1 * G + 2].astype(np.float64)
    qh = (V[4, 1].astype(np.float64) * Vs[4, 1]).T @ qq
    want = 0.09 * (mu[4, 1] * np.float64(mus[4, 1])) @ qq + \
        0.09 ** 2 / 32 * float(np.sum(sg[4, 1].astype(np.float64) * qh * qh))
    assert sh[0, 1, 2, 2] == pytest.approx(want, rel=1e-12)


def test_comb_brute_force():
    rng = np.random.default_rng(6)
    R, NB, n_kv, G, d, r = 1, 3, 1, 2, 128, 4
    q = rng.standard_normal((R, n_kv * G, d)).astype(np.float32)
    mu = rng.integers(-127, 128, (NB, n_kv, d)).astype(np.int8)
    codes = rng.integers(-7, 8, (NB, n_kv, d, r)).astype(np.int8)
    V4 = oq.pack_i4(codes)
    bt = np.array([[2, 0, 1]], np.int32)
    comb = osc.quad_comb(q, mu, V4, bt, np.array([3]), G=G, v_bits=4, max_pages=3)
    qi = oq.q_limbs(q[0])[0]
    for p, blk in enumerate(bt[0]):
        for g in range(G):
            for c in range(r + 1):
                col = [int(mu[blk, 0, k]) if c == r else int(codes[blk, 0, k, c])
                       for k in range(d)]
                want = sum(int(qi[g, k]) * col[k] for k in range(d))
                assert comb[0, 0, p, g, c] == want


def test_limbs_score_is_float_score_on_quantised_q():
    rng = np.random.default_rng(7)
    NB, n_kv, G, d, r = 4, 1, 2, 128, 8
    q = rng.standard_normal((1, G, d)).astype(np.float32)
    mu = rng.integers(-127, 128, (NB, n_kv, d)).astype(np.int8)
    V = rng.integers(-127, 128, (NB, n_kv, d, r)).astype(np.int8)
    one = lambda *s: np.full(s, 0.01, np.float32)  # noqa: E731
    args = (mu, one(NB, n_kv), V, one(NB, n_kv, r), one(NB, n_kv, r),
            np.arange(NB, dtype=np.int32)[None], np.array([NB]))
    kw = dict(scale=0.1, page=16, G=G, v_bits=8, max_pages=NB, combine="nrm")
    qi, _, _, qs = oq.q_limbs(q)
    qhat = (qi * qs[..., None].astype(np.float64)).astype(np.float32)
    a = osc.quad_score(q, *args, q_mode="limbs", **kw)
    b = osc.quad_score(qhat, *args, q_mode="float", **kw)
    assert np.allclose(a, b, rtol=1e-6)
    # the limb score differs from the exact-q score only by the 14-bit rounding of q
    c = osc.quad_score(q, *args, q_mode="float", **kw)
    assert np.abs(a - c).max() < 1e-3 * np.abs(c).max()


def test_nrm_combine_hand_case():
    sh = np.array([[[[0.0, 1.0], [2.0, 0.0]]]])           # (R=1, kv=1, G=2, MP=2)
    out = osc.nrm_combine(sh, np.array([2]))
    assert out[0, 0, 0] == pytest.approx(math.exp(-1) + 1.0)
    assert out[0, 0, 1] == pytest.approx(1.0 + math.exp(-2))
    out1 = osc.nrm_combine(sh, np.array([1]))              # only page 0 scored
    assert out1[0, 0, 0] == pytest.approx(2.0) and np.isnan(out1[0, 0, 1])


# ----------------------------------------------------------------------------- r8
@pytest.mark.parametrize("seq_len", [48, 41])
def test_r8_equals_true_logsumexp_at_rank_r(seq_len):
    """With page rank <= r and exactly representable codes, the r8 score is the exact
    logsumexp of the page's true logits s q.k_t over its valid tokens."""
    rng = np.random.default_rng(8)
    d, r, P, NB, G = 128, 8, 16, 3, 2
    Vk = np.zeros((NB, 1, d, r), np.int8)
    c = rng.integers(-127, 128, (NB, 1, P, r)).astype(np.int8)
    mu = rng.integers(-127, 128, (NB, 1, d)).astype(np.int8)
    for b in range(NB):
        perm = rng.permutation(d)
        for k in range(r):
            Vk[b, 0, perm[16 * k:16 * (k + 1)], k] = rng.choice([-127, 127], 16)
    vks = np.full((NB, 1, r), 1.0 / 508)                  # 127/508 = 1/4: orthonormal
    cs = rng.uniform(0.002, 0.01, (NB, 1, P))
    mus = np.full((NB, 1), 1.0 / 64)
    q = rng.standard_normal((1, G, d)).astype(np.float32)
    bt = np.array([[2, 0, 1]], np.int32)
    scale = 1 / math.sqrt(d)
    got = osc.r8_score(q, mu, mus, Vk, vks, c, cs, bt, np.array([seq_len]), np.array([3]),
                       scale=scale, page=P, G=G, vk_bits=8, c_bits=8, max_pages=3)
    for p, blk in enumerate(bt[0]):
        Vf = Vk[blk, 0].astype(np.float64) * vks[blk, 0]
        K = mu[blk, 0] * mus[blk, 0] + (c[blk, 0] * cs[blk, 0][:, None]) @ Vf.T
        valid = p * P + np.arange(P) < seq_len
        best = -np.inf
        for g in range(G):
            lg = scale * K[valid] @ q[0, g].astype(np.float64)
            best = max(best, lg.max() + math.log(np.exp(lg - lg.max()).sum()))
        assert got[0, 0, p] == pytest.approx(best, rel=1e-10, abs=1e-10)


# ----------------------------------------------------------------------------- select
def test_derive_config0_known_answer():
    npg, nsh, b = osel.derive([4096], 0.05, page=16, window=1, sink=1)
    assert (int(npg[0]), int(nsh[0]), int(b[0])) == (256, 255, 13)
    npg, nsh, b = osel.derive([1, 16, 17, 33], 0.5, page=16, window=1, sink=1)
    assert list(npg) == [1, 1, 2, 3] and list(nsh) == [0, 0, 1, 2]
    assert list(b) == [1, 1, 1, 1]


def test_exp_det_accuracy():
    x = np.concatenate([np.linspace(-79.9, 0, 200001, dtype=np.float32),
                        np.array([0.0, -1e-30, -0.5, -1.0, -87.0], np.float32)])
    got = osel.exp_det(x).astype(np.float64)
    want = np.exp(x.astype(np.float64))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    m = x > -80
    assert np.all(np.abs(got[m] - want[m]) <= 4 * ulp[m])
    assert np.all(got[~m] == 0)
    assert osel.exp_det(np.float32(0.0)) == 1.0


def test_mass_cut_case_separates_fused_exp():
    """The coverage case of the GPU test for exact exp masses is sensitive: with every
    multiply-add of exp_det fused (a planted mistake, one rounding instead of two) the
    oracle's nucleus keeps one more page."""
    sc, cov = mass_cut_case(osel.exp_det)
    MP = sc.size
    npg, nsh, b = osel.derive([MP * 16], 0.05, page=16, window=1, sink=1)
    args = dict(sink=1, max_pages=MP, mode=1, coverage=cov, score_kind=0)
    _, cnt, nsel = osel.select(sc[None, None], npg, nsh, b, **args)
    assert int(nsel[0, 0]) == 11
    real = osel.exp_det
    try:
        osel.exp_det = exp_det_fused
        _, cnt_f, nsel_f = osel.select(sc[None, None], npg, nsh, b, **args)
    finally:
        osel.exp_det = real
    assert int(nsel_f[0, 0]) == 12 and int(cnt_f[0, 0]) == int(cnt[0, 0]) + 1


def test_f2u_order_preserving():
    rng = np.random.default_rng(9)
    x = np.concatenate([rng.standard_normal(1000) * 10 ** rng.uniform(-30, 30, 1000),
                        [np.inf, -np.inf, 1e-45, -1e-45, 3.4e38, -3.4e38]]).astype(np.float32)
    order_k = np.argsort(osel.f2u(x), kind="stable")
    assert np.array_equal(x[order_k], np.sort(x))
    # +0 and -0 compare equal as floats, so they must share one key (ties -> index order)
    assert osel.f2u(np.float32(-0.0)) == osel.f2u(np.float32(0.0))


def _brute_topb(sc, nh, npg, sink, b):
    S = nh - sink
    if S <= 1:
        return list(range(npg)), max(S, 0)
    b = min(max(b, 1), S)
    chosen = sorted(range(sink, nh), key=lambda p: (-float(sc[p]), p))[:b]
    keep = set(range(sink)) | set(range(nh, npg)) | set(chosen)
    return sorted(keep), b


@pytest.mark.parametrize("seed", range(6))
def test_topb_brute_force(seed):
    rng = np.random.default_rng(10 + seed)
    R, n_kv, MP = 3, 2, 40
    vals = np.array([-3.5, -1.0, 0.25, 2.0, 7.0], np.float32)     # many exact ties
    sc = vals[rng.integers(0, 5, (R, n_kv, MP))]
    npg = np.array([40, 17, 2])
    nsh = npg - 1
    bfix = np.array([5, 30, 1])
    tab, cnt, nsel = osel.select(sc, npg, nsh, bfix, sink=1, max_pages=MP, mode=0)
    for r in range(R):
        for kh in range(n_kv):
            keep, b = _brute_topb(sc[r, kh], int(nsh[r]), int(npg[r]), 1, int(bfix[r]))
            assert list(tab[r, kh, :cnt[r, kh]]) == keep
            assert (tab[r, kh, cnt[r, kh]:] == -1).all() and nsel[r, kh] == b


def test_topb_threshold_tie_mode():
    sc = np.array([[[9.0, 5.0, 3.0, 5.0, 5.0, 1.0, 0.5]]], np.float32)
    tab, cnt, nsel = osel.select(sc, np.array([7]), np.array([6]), np.array([2]), sink=1,
                                 max_pages=7, mode=0, tie_mode=1)
    # b-th (2nd) largest selectable score is 5.0 -> all three 5.0 pages, plus sink/window
    assert list(tab[0, 0, :cnt[0, 0]]) == [0, 1, 3, 4, 6] and nsel[0, 0] == 3
    tab0, cnt0, _ = osel.select(sc, np.array([7]), np.array([6]), np.array([2]), sink=1,
                                max_pages=7, mode=0, tie_mode=0)
    assert list(tab0[0, 0, :cnt0[0, 0]]) == [0, 1, 3, 6]


@pytest.mark.parametrize("seed", range(8))
@pytest.mark.parametrize("kind", [0, 1])
def test_nucleus_minimal_by_subset_enumeration(seed, kind):
    """The chosen set reaches the coverage, and no set of one fewer selectable pages does
    (checked over every subset, with float64 masses and a slack of one fixed-point unit
    per page)."""
    rng = np.random.default_rng(100 + seed)
    npg = 11
    nsh = npg - 1
    sink = 1
    sc = (rng.standard_normal(npg) * 2).astype(np.float32)
    if kind == 1:
        sc = np.abs(sc)
    cov = float(rng.uniform(0.5, 0.99))
    tab, cnt, nsel = osel.select(sc[None, None], np.array([npg]), np.array([nsh]),
                                 np.array([1]), sink=sink, max_pages=npg, mode=1,
                                 coverage=cov, score_kind=kind)
    b = int(nsel[0, 0])
    scored = sc[:nsh].astype(np.float64)
    w = np.exp(scored - scored.max()) if kind == 0 else np.clip(scored, 0, 1024)
    need = cov * w.sum() - w[:sink].sum()
    slack = (nsh + 1) * 2.0 ** -32 * (1 if kind == 0 else 1)
    kept = [p for p in tab[0, 0, :cnt[0, 0]] if sink <= p < nsh]
    assert len(kept) == b
    if need <= 0:
        assert b == 1
        return
    assert w[kept].sum() >= need - slack
    sel = range(sink, nsh)
    for sub in itertools.combinations(sel, b - 1):
        assert w[list(sub)].sum() < need + slack


def test_select_always_pages_and_short_sequences():
    sc = np.zeros((4, 1, 8), np.float32)
    npg = np.array([8, 2, 1, 0])
    nsh = npg - 1
    tab, cnt, nsel = osel.select(sc, npg, nsh, np.array([1, 1, 1, 1]), sink=1, max_pages=8)
    assert list(tab[0, 0, :cnt[0, 0]]) == [0, 1, 7]
    assert list(tab[1, 0, :cnt[1, 0]]) == [0, 1] and nsel[1, 0] == 0
    assert list(tab[2, 0, :cnt[2, 0]]) == [0] and cnt[3, 0] == 0


# ----------------------------------------------------------------------------- decode
def _kv(rng, NB, P, n_kv, d):
    K = rng.standard_normal((NB, P, n_kv, d))
    V = rng.standard_normal((NB, P, n_kv, d))
    return K, V


def test_attend_uniform_and_one_hot():
    rng = np.random.default_rng(11)
    NB, P, n_kv, d, G = 4, 16, 1, 8, 1
    K, V = _kv(rng, NB, P, n_kv, d)
    K[2] = K[2, 0]                     # every key of block 2 identical -> uniform weights
    q = rng.standard_normal((1, 1, d))
    bt = np.array([[2, 0, 1, 3]])
    pt = np.array([[[0]]])
    out = odec.attend(q, K, V, bt, np.array([10]), pt, np.array([[1]]), scale=0.3, G=G)
    assert np.allclose(out[0, 0], V[2, :10, 0].mean(axis=0))
    K2 = K.copy()
    K2[0, 5, 0] = 100 * q[0, 0]        # one dominant token in block 0 = logical page 1
    pt = np.array([[[0, 1]]])
    out = odec.attend(q, K2, V, bt, np.array([64]), pt, np.array([[2]]), scale=1.0, G=G)
    assert np.allclose(out[0, 0], V[0, 5, 0])


def test_attend_dense_equals_all_pages_selected():
    rng = np.random.default_rng(12)
    NB, P, n_kv, d, G = 6, 16, 2, 16, 2
    K, V = _kv(rng, NB, P, n_kv, d)
    q = rng.standard_normal((2, n_kv * G, d))
    bt = np.array([[5, 1, 3, 0, 2, 4], [0, 1, 2, 3, 4, 5]])
    sl = np.array([83, 40])
    pt = np.full((2, n_kv, 6), -1)
    cnt = np.zeros((2, n_kv), int)
    for r in range(2):
        n = -(-int(sl[r]) // P)
        pt[r, :, :n] = np.arange(n)
        cnt[r] = n
    a = odec.attend(q, K, V, bt, sl, scale=0.25, G=G, dense=True)
    b = odec.attend(q, K, V, bt, sl, pt, cnt, scale=0.25, G=G)
    assert np.allclose(a, b)


@pytest.mark.parametrize("split,pps_min", [(1, 1), (2, 1), (3, 2), (16, 1), (4, 8)])
def test_split_merge_invariance(split, pps_min):
    rng = np.random.default_rng(13)
    NB, P, n_kv, d, G = 8, 16, 2, 16, 3
    K, V = _kv(rng, NB, P, n_kv, d)
    q = rng.standard_normal((2, n_kv * G, d))
    bt = rng.permutation(NB)[None].repeat(2, 0)
    sl = np.array([120, 7])
    pt = np.array([[[0, 2, 5, 7, -1], [1, 3, 4, -1, -1]], [[0, -1, -1, -1, -1]] * 2])
    cnt = np.array([[4, 3], [1, 0]])
    a = odec.attend(q, K, V, bt, sl, pt, cnt, scale=0.2, G=G)
    b = odec.split_merge(q, K, V, bt, sl, pt, cnt, scale=0.2, G=G, split=split,
                         pps_min=pps_min)
    assert np.allclose(a, b, atol=1e-12)
    assert not b[1, G:].any()          # empty unit -> zeros


# ----------------------------------------------------------------------------- tier
def test_tier_plan_hand_worked_lru():
    """1 kv head, 3 slots, pages complete; worked by hand:
    step 1 touches blocks 10, 11       -> both miss, slots 0, 1 (all lru 0 < 1)
    step 2 touches 11, 12, 13          -> 11 hits slot 1 (lru 2); 12 -> slot 2 (lru 0);
                                          13 -> slot 0 (lru 1, the oldest untouched)
    step 3 touches 12, 10              -> 12 hits slot 2; 10 -> slot 1 (lru 2 < slot 0's 2?
                                          no: slot 0 lru 2, slot 1 lru 2 -> lowest index 0)
    """
    P = 16
    p2s = np.full((1, 32), -1)
    s2p = np.full((1, 3), -1)
    lru = np.zeros((1, 3), np.int64)
    bt = np.arange(32)[None]
    sl = np.array([32 * P])

    def step(pages, st):
        pt = np.array([[pages + [-1] * (8 - len(pages))]])
        return otier.plan(pt, np.array([[len(pages)]]), bt, sl, st["page2slot"],
                          st["slot2page"], st["lru"], st["clock"], page=P)

    st = dict(page2slot=p2s, slot2page=s2p, lru=lru, clock=0)
    st = step([10, 11], st)
    assert st["victims"][0][0] == [0, 1] and st["clock"] == 1
    st = step([11, 12, 13], st)
    assert st["victims"][0][0] == [2, 0]
    assert list(st["slot2page"][0]) == [13, 11, 12] and list(st["lru"][0]) == [2, 2, 2]
    st = step([12, 10], st)
    assert st["victims"][0][0] == [0]
    assert list(st["slot2page"][0]) == [10, 11, 12]
    assert st["page2slot"][0, 13] == -1 and st["page2slot"][0, 10] == 0


def test_tier_plan_incomplete_pages_and_overflow():
    P = 16
    bt = np.arange(8)[None].repeat(2, 0)
    pt = np.array([[[0, 1, 2, 3]], [[0, 1, 2, 3]]])
    cnt = np.array([[4], [4]])
    sl = np.array([3 * P + 5, 4 * P])       # request 0: page 3 incomplete -> never planned
    st = otier.plan(pt, cnt, bt, sl, np.full((1, 8), -1), np.full((1, 5), -1),
                    np.zeros((1, 5), np.int64), 0, page=P)
    assert st["miss"][0][0] == [0, 1, 2] and st["miss"][1][0] == [0, 1, 2, 3]
    # request 1's first three misses were installed by request 0 this step -> -1
    assert st["victims"][1][0] == [-1, -1, -1, 3] and not st["overflow"]
    st2 = otier.plan(pt, cnt, bt, sl, np.full((1, 8), -1), np.full((1, 2), -1),
                     np.zeros((1, 2), np.int64), 0, page=P)
    assert st2["overflow"]


def test_tier_plan_maps_stay_inverse():
    rng = np.random.default_rng(14)
    NB, S, P = 64, 12, 16
    st = dict(page2slot=np.full((2, NB), -1), slot2page=np.full((2, S), -1),
              lru=np.zeros((2, S), np.int64), clock=0)
    bt = np.stack([rng.permutation(NB) for _ in range(3)])
    sl = np.array([NB * P] * 3)
    for _ in range(10):
        pt = np.full((3, 2, 6), -1)
        cnt = np.zeros((3, 2), int)
        for r in range(3):
            for kv in range(2):
                pages = np.sort(rng.choice(20, 3, replace=False))
                pt[r, kv, :3] = pages
                cnt[r, kv] = 3
        clk0 = st["clock"]
        lru0 = st["lru"].copy()
        st = otier.plan(pt, cnt, bt, sl, st["page2slot"], st["slot2page"], st["lru"],
                        st["clock"], page=P)
        for kv in range(2):
            for s, blk in enumerate(st["slot2page"][kv]):
                if blk >= 0:
                    assert st["page2slot"][kv, blk] == s
            assert (st["page2slot"][kv] >= 0).sum() == (st["slot2page"][kv] >= 0).sum()
            # every victim slot was untouched before this step's installs
            vict = {v for r in range(3) for v in st["victims"][r][kv] if v >= 0}
            assert all(lru0[kv, v] <= clk0 for v in vict)


def _clse_page(rng, r=2, d=128, NB=2, n_kv=1):
    mu = rng.integers(-100, 100, (NB, n_kv, d)).astype(np.int8)
    mus = np.full((NB, n_kv), 0.01, np.float32)
    V = rng.integers(-127, 128, (NB, n_kv, d, r)).astype(np.int8)
    vs = rng.uniform(0.005, 0.02, (NB, n_kv, r)).astype(np.float32)
    c = rng.integers(-127, 128, (NB, n_kv, 16, r)).astype(np.int8)
    cs = rng.uniform(0.01, 0.05, (NB, n_kv, 16)).astype(np.float32)
    return mu, mus, V, vs, c, cs


def test_clse_equals_r8_at_zero_residual():
    """resid = 0 removes the iso term: CLSE is then the r8 score on the same factors
    (the r8 oracle is pinned to the exact logsumexp above)."""
    rng = np.random.default_rng(5)
    mu, mus, V, vs, c, cs = _clse_page(rng)
    q = rng.standard_normal((1, 4, 128)).astype(np.float32)
    bt, sl, nsh = np.array([[0, 1]], np.int32), np.array([29]), np.array([2])
    kw = dict(scale=128 ** -0.5, page=16, G=4, max_pages=2)
    a = osc.clse_score(q, mu, mus, V, vs, c, cs, np.zeros((2, 1)), bt, sl, nsh,
                       v_bits=8, c_bits=8, **kw)
    b = osc.r8_score(q, mu, mus, V, vs, c, cs, bt, sl, nsh, vk_bits=8, c_bits=8, **kw)
    assert np.allclose(a, b, rtol=1e-12, atol=1e-12)


def test_clse_iso_term_by_hand():
    """Constant coordinates (c = 0: every token logit 0, lse = log 16) and a V of two
    exact unit axes: S = s mu.q + log 16 + (|q|^2 - q_0^2 - q_1^2) resid s^2 / (2P(d-2))."""
    d, s = 128, 128 ** -0.5
    mu = np.zeros((1, 1, d), np.int8)
    mu[0, 0, :4] = [10, -20, 30, 0]
    mus = np.array([[0.5]], np.float32)
    V = np.zeros((1, 1, d, 2), np.int8)
    V[0, 0, 0, 0] = V[0, 0, 1, 1] = 100
    vs = np.full((1, 1, 2), 0.01, np.float32)              # unit axes e_0, e_1
    c = np.zeros((1, 1, 16, 2), np.int8)
    cs = np.ones((1, 1), np.float32)                       # page grain
    q = np.zeros((1, 1, d), np.float32)
    q[0, 0, :3] = [1.5, -2.0, 0.25]
    q[0, 0, 100] = 3.0
    resid = np.array([[7.0]])
    got = osc.clse_score(q, mu, mus, V, vs, c, cs, resid, np.array([[0]], np.int32),
                         np.array([16]), np.array([1]), scale=s, page=16, G=1, v_bits=8,
                         c_bits=8, max_pages=1)
    qmu = s * 0.5 * (10 * 1.5 + (-20) * (-2.0) + 30 * 0.25)
    iso = (0.25 ** 2 + 3.0 ** 2) * 7.0 * s * s / (2 * 16 * (d - 2))
    assert np.isclose(got[0, 0, 0], qmu + np.log(16) + iso, rtol=1e-12)


def test_clse_nrm_is_per_head_max_layout():
    rng = np.random.default_rng(6)
    mu, mus, V, vs, c, cs = _clse_page(rng, r=4, NB=3, n_kv=2)
    q = rng.standard_normal((1, 8, 128)).astype(np.float32)
    bt, sl, nsh = np.array([[2, 0, 1]], np.int32), np.array([48]), np.array([3])
    resid = rng.uniform(0, 50, (3, 2))
    kw = dict(scale=128 ** -0.5, page=16, G=4, v_bits=8, c_bits=8, max_pages=3)
    mx = osc.clse_score(q, mu, mus, V, vs, c, cs, resid, bt, sl, nsh, combine="max", **kw)
    ph = osc.clse_score(q, mu, mus, V, vs, c, cs, resid, bt, sl, nsh, combine="nrm", **kw)
    assert ph.shape == (1, 2, 4, 3) and np.allclose(ph.max(axis=2), mx)
