"""The vLLM-ROCm boundary end to end on the GPU (vLLM itself replaced by the stand-in of
fake_vllm): register() -> wrapped backend -> metadata builder (lazy state, summary bulk
build, derive) -> impl.forward (quad score, nrm, coverage selection, sparse decode),
checked against the CPU oracle: page tables bit-exact, output within 2e-2 / 1e-2."""
import types

import numpy as np
import pytest
import torch

import fake_vllm
import oracle.decode as odec
import oracle.score as osc
import oracle.select as osel
from amass.backend import _runtime, register
from amass.bench.synth import make_case
from helpers import announce, npf, npi

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture
def vllm(monkeypatch):
    saved = fake_vllm.install()
    orig = fake_vllm.RocmPlatform.__dict__["get_attn_backend_cls"]
    monkeypatch.setattr(register, "_APPLIED", False)
    monkeypatch.setattr(register, "_WRAPPED", {})
    monkeypatch.delenv("AMASS_DISABLE", raising=False)
    monkeypatch.delenv("AMASS_CONFIG", raising=False)
    yield fake_vllm
    fake_vllm.RocmPlatform.get_attn_backend_cls = orig
    _runtime.set_config(None)
    fake_vllm.uninstall(saved)


@pytest.mark.parametrize("combine", ["nrm", "max"])
def test_backend_decode_step_matches_oracle(vllm, combine):
    announce(f"backend decode step combine={combine}")
    cfg = dict(variant="fast", score="quad", quad_rank=8, quad_v_bits=8,
               quad_combine=combine, budget=None, coverage=0.9)
    register.register(cfg)
    be = register._resolve(vllm.RocmPlatform.get_attn_backend_cls(None, 128, None,
                                                                   "auto", 16))
    case = make_case(B=3, ctx=(700, 1500), n_kv=8, G=4, heavy=0.05, table="perm", seed=21)
    kv = case.kv_cache.to(DEV)
    q = case.q.to(DEV)
    bt, sl = case.block_table.to(DEV), case.seq_lens.to(DEV)
    B = q.shape[0]
    vc = vllm.vllm_config(num_gpu_blocks=kv.shape[0], layers={"layer0": kv},
                          max_num_seqs=4, max_model_len=case.max_pages * 16)
    b = be.get_builder_cls()(vllm.kv_spec(), ["layer0"], vc, DEV)
    cam = types.SimpleNamespace(seq_lens=sl, block_table_tensor=bt, max_query_len=1,
                                seq_lens_cpu_upper_bound=sl.cpu())
    md = b.build(0, cam)
    st = md.amass
    impl = be.get_impl_cls()(32, 128, case.scale, 8)
    out = torch.zeros(B, 32 * 128, dtype=torch.bfloat16, device=DEV)
    assert impl.forward(None, q, None, None, kv, md, output=out) is out
    torch.cuda.synchronize()
    assert impl.calls == []                                     # the AMASS path ran

    # oracle: scores from the built summaries, the same nucleus, attention
    mu, mus, _, Vs, sg, _ = st.layer_state(0)
    nsh = npi(st.n_sel_hi)
    ref = osc.quad_score(npf(case.q), npi(mu), npf(mus), npi(st.reference_V(0)), npf(Vs),
                         npf(sg), npi(case.block_table), nsh, scale=case.scale, page=16,
                         G=4, v_bits=8, max_pages=st.max_pages, combine=combine)
    if combine == "nrm":
        ref = osc.nrm_combine(ref, nsh)
    sc = npf(st.score)
    for r in range(B):
        n = int(nsh[r])
        err = np.abs(sc[r, :, :n] - ref[r, :, :n]) / np.maximum(np.abs(ref[r, :, :n]), 1)
        assert err.max() <= 1e-3
    tab, cnt, _ = osel.select(sc[:B], npi(st.n_pages)[:B], nsh[:B], npi(st.b_fix)[:B],
                              sink=1, max_pages=st.max_pages, mode=1, coverage=0.9,
                              score_kind=1 if combine == "nrm" else 0)
    assert np.array_equal(npi(st.page_table)[:B], tab)
    assert np.array_equal(npi(st.page_cnt)[:B], cnt)
    want = odec.attend(npf(case.q), npf(case.kv_cache[:, 0]), npf(case.kv_cache[:, 1]),
                       npi(case.block_table), npi(case.seq_lens), tab, cnt, scale=case.scale,
                       G=4)
    got = npf(out.view(B, 32, 128))
    assert np.allclose(got, want, atol=2e-2, rtol=1e-2), float(np.abs(got - want).max())


def test_mem_v_shadow_tier_tracks_the_cache(vllm):
    """mem-v through the backend on the GPU (shadow, reference builder.py:300-330): a
    prefill step and decode steps go through the builder (tier lifecycle) and the impl
    (V write path, then the stock attention); afterwards every written token's V is held
    by the tier -- staged or flushed to the pinned pool -- equal to the engine cache's."""
    announce("backend mem-v shadow tier")
    register.register(dict(variant="mem-v", score="quad", budget=None, coverage=0.95,
                           hot_slots=64))
    be = register._resolve(vllm.RocmPlatform.get_attn_backend_cls(None, 128, None,
                                                                   "auto", 16))
    L, B, n_kv, d, page, NB, MP = 2, 3, 8, 128, 16, 48, 8
    gen = torch.Generator().manual_seed(4)
    kvs = {f"layer{i}": torch.zeros(NB, 2, page, n_kv, d, dtype=torch.bfloat16, device=DEV)
           for i in range(L)}
    vc = vllm.vllm_config(num_gpu_blocks=NB, layers=kvs, max_num_seqs=B,
                          max_model_len=MP * page)
    vc.scheduler_config.max_num_batched_tokens = 128
    b = be.get_builder_cls()(vllm.kv_spec(), list(kvs), vc, DEV)
    impl = be.get_impl_cls()(32, 128, d ** -0.5, 8)
    bt = torch.randperm(NB, generator=gen)[:B * MP].view(B, MP).to(torch.int32)
    bt_d = bt.to(DEV)
    sl = torch.zeros(B, dtype=torch.int32)
    for ql in ([40, 17, 33], [1, 1, 1], [1, 1, 1], [30, 1, 1], [1, 1, 1]):
        ql = torch.tensor(ql, dtype=torch.int32)
        sl = sl + ql
        qsl = torch.cat([torch.zeros(1, dtype=torch.int32), torch.cumsum(ql, 0).to(torch.int32)])
        n_tok = int(qsl[-1])
        cam = types.SimpleNamespace(
            seq_lens=sl.to(DEV), block_table_tensor=bt_d, max_query_len=int(ql.max()),
            seq_lens_cpu_upper_bound=sl.clone(), query_start_loc=qsl.to(DEV),
            slot_mapping=torch.full((n_tok,), -1, dtype=torch.int64, device=DEV),
            num_actual_tokens=n_tok)
        md = b.build(0, cam)
        assert md.amass_tier is not None
        for name, kv in kvs.items():
            value = torch.randn(n_tok, n_kv, d, generator=gen).to(torch.bfloat16)
            for r in range(B):                 # the engine's own cache write
                for i in range(int(ql[r])):
                    pos = int(sl[r]) - int(ql[r]) + i
                    kv[int(bt[r, pos // page]), 1, pos % page] = value[int(qsl[r]) + i].to(DEV)
            out = torch.zeros(n_tok, 32 * 128, dtype=torch.bfloat16, device=DEV)
            impl.forward(None, out, None, value.to(DEV), kv, md, output=out)
        assert impl.calls and set(impl.calls) == {"stock"}
    torch.cuda.synchronize()
    tier = md.amass_tier
    tier.assert_invariants(bt_d, sl.to(DEV), qsl.to(DEV))
    vbo = tier.staging.vbo.cpu()
    pv = tier.residency.pool_valid.cpu()
    pool = tier.pool.host
    n_staged = n_flushed = 0
    for lidx, kv in enumerate(kvs.values()):
        vp = tier.staging.v_pool[lidx].cpu()
        kvc = kv.cpu()
        for r in range(B):
            for p in range((int(sl[r]) + page - 1) // page):
                blk = int(bt[r, p])
                nt = min(page, int(sl[r]) - p * page)
                want = kvc[blk, 1, :nt]                         # (nt, n_kv, d)
                if int(vbo[blk]) >= 0:
                    got = vp[int(vbo[blk]), :nt]
                    n_staged += 1
                else:
                    assert bool((pv[lidx, :, blk] == 1).all()), (lidx, r, p)
                    got = pool[lidx, blk, :, :nt].permute(1, 0, 2)
                    n_flushed += 1
                assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (lidx, r, p)
    assert n_staged > 0 and n_flushed > 0
