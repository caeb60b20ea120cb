"""Pins of the page-summary builder oracle (oracle/build.py) and of the torch host
builder against it -- CPU only.

The oracle's factors are pinned by what the linear algebra fixes, not by restating it:
a page whose centred keys have rank <= r is reconstructed exactly by U8 S8 Vk^T; the
stored eigenvalues are the squared singular values of the centred page (an independent
LAPACK routine); Vk has orthonormal columns; a hand-built rank-1 page gives its known
eigenvalue and direction.  The package's torch builder (used for host-resident K) must
match the oracle's codes up to fp32-vs-fp64 rounding at code boundaries.
"""
import numpy as np
import pytest

import oracle.build as ob
import oracle.quant as oq


def _low_rank_page(rng, rank, d=128, n_kv=2):
    """(1, 16, n_kv, d) keys mu + U diag(sig) V^T with U orthonormal and orthogonal to 1."""
    out = np.zeros((1, 16, n_kv, d))
    sigs = []
    for h in range(n_kv):
        A = rng.standard_normal((16, rank))
        A -= A.mean(axis=0)                          # columns orthogonal to the ones vector
        U, _ = np.linalg.qr(A)
        V, _ = np.linalg.qr(rng.standard_normal((d, rank)))
        sig = np.sort(rng.uniform(1.0, 9.0, rank))[::-1]
        mu = rng.standard_normal(d)
        out[0, :, h, :] = mu + (U * sig) @ V.T
        sigs.append(sig)
    return out, np.array(sigs)


@pytest.mark.parametrize("rank", [2, 4, 8])
def test_exact_reconstruction_at_rank_r(rank):
    rng = np.random.default_rng(rank)
    K, sig = _low_rank_page(rng, rank)
    mu, dc, S2r, U8, Vk = ob.page_factors(K, rank)
    recon = (U8 * np.sqrt(S2r)[..., None, :]) @ Vk.swapaxes(-1, -2)
    assert np.abs(recon - dc).max() < 1e-9
    assert np.allclose(np.sort(S2r[0], axis=-1), np.sort(sig ** 2, axis=-1), rtol=1e-10)
    gram = Vk.swapaxes(-1, -2) @ Vk
    assert np.abs(gram - np.eye(rank)).max() < 1e-10
    assert np.all(np.diff(S2r, axis=-1) >= 0)        # ascending, as eigh returns


def test_sig2_are_squared_singular_values():
    rng = np.random.default_rng(7)
    K = rng.standard_normal((5, 16, 3, 128))
    _mu, dc, S2r, _U8, _Vk = ob.page_factors(K, 8)
    sv = np.linalg.svd(dc, compute_uv=False)         # descending
    assert np.allclose(S2r, (sv[..., :8] ** 2)[..., ::-1], rtol=1e-10)


def test_rank_one_page_by_hand():
    x = np.array([3., -1., 2., 0., -4., 1., 1., -2., 0., 0., 5., -5., 1., -1., 0., 0.])
    assert x.sum() == 0
    K = np.zeros((1, 16, 1, 128))
    K[0, :, 0, :] = 0.25                              # mean
    K[0, :, 0, 5] += x
    mu, _dc, S2r, U8, Vk = ob.page_factors(K, 2)
    assert np.allclose(mu[0, 0], 0.25)
    assert np.isclose(S2r[0, 0, -1], (x ** 2).sum())
    assert S2r[0, 0, 0] == 1e-10                      # the clamp of a zero eigenvalue
    v = Vk[0, 0, :, -1]
    assert np.isclose(abs(v[5]), 1.0) and np.abs(np.delete(v, 5)).max() < 1e-12
    c = U8[0, 0, :, -1] * np.sqrt(S2r[0, 0, -1])
    assert np.allclose(np.abs(c), np.abs(x))


def test_summary_codes_follow_quant_rules():
    rng = np.random.default_rng(3)
    K = oq.bf16_round(rng.standard_normal((4, 16, 2, 128)).astype(np.float32))
    q = ob.quad_summary(K, 4, v_bits=4)
    mu, _dc, S2r, _U8, Vk = ob.page_factors(K, 4)
    code, s = oq.quant(mu.astype(np.float32), axis=-1, bits=8)
    assert np.array_equal(q["mu"], code) and np.array_equal(q["mu_scale"], s[..., 0])
    assert np.array_equal(oq.unpack_i4(q["V"]), oq.quant(Vk.astype(np.float32), -2, 4)[0])
    r = ob.r8_summary(K, 4, c_bits=8, c_grain="tensor")
    assert np.all(np.abs(r["c"]).max(axis=(-2, -1)) == 127)   # one scale per (block, head)
    assert np.all(r["c_scale"] == r["c_scale"][..., :1])


def _align(ref, got, axis=-2):
    """Flip each column of `got` to the sign that best matches `ref`."""
    sgn = np.sign((ref.astype(np.float64) * got.astype(np.float64)).sum(axis=axis, keepdims=True))
    sgn[sgn == 0] = 1
    return got * sgn, sgn


@pytest.mark.parametrize("kind", ["quad", "r8"])
def test_torch_host_builder_matches_oracle(kind):
    from amass.bench.synth import build_quad_state, build_r8_state, make_case
    case = make_case(B=2, ctx=(300, 700), n_kv=2, G=4, heavy=0.05, table="perm", seed=5)
    if kind == "quad":
        st = build_quad_state(case, rank=8, v_bits=8)
        V = st.reference_V(0).numpy()
        mu = st.quad_mu[0].numpy()
    else:
        st = build_r8_state(case, rank=8, vk_bits=8, c_bits=8)
        V = st.reference_Vk(0).numpy()
        mu = st.r8_mu[0].numpy()
    K = case.kv_cache[:, 0].float().numpy()
    blocks = np.unique(case.block_table.numpy()[:, :20].reshape(-1))
    ref = ob.quad_summary(K[blocks], 8) if kind == "quad" else ob.r8_summary(K[blocks], 8)
    assert np.abs(mu[blocks].astype(int) - ref["mu"].astype(int)).max() <= 1
    Vref = ref["V"] if kind == "quad" else ref["Vk"]
    got, _ = _align(Vref, V[blocks].astype(np.float64))
    diff = np.abs(got - Vref)
    assert diff.max() <= 2 and (diff == 0).mean() > 0.95


def test_clse_resid_is_energy_beyond_top_r():
    rng = np.random.default_rng(11)
    K = rng.standard_normal((3, 16, 2, 128))
    out = ob.clse_summary(K, 2, c_bits=8, c_grain="page")
    dc = ob.page_factors(K, 2)[1]
    sv = np.linalg.svd(dc, compute_uv=False)
    assert np.allclose(out["resid"], (sv[..., 2:] ** 2).sum(-1), rtol=1e-10)
    assert out["c_scale"].shape == (3, 2)
    tok = ob.clse_summary(K, 2, c_bits=4, c_grain="token")
    assert tok["c_scale"].shape == (3, 2, 16) and tok["c"].shape == (3, 2, 16, 1)
