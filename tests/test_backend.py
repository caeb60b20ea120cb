"""vLLM-ROCm plugin boundary on a vLLM stand-in (CPU): registration and backend
wrapping (reference backend/register.py:26-86), the impl's pure-decode gate
(backend/attn.py:31-82), graph-support declaration (backend/builder.py:81-88) and the
builder's lazy state, summary refresh gate and derive gating (builder.py:252-459).
Kernel calls are replaced by recorders; the GPU path is covered by test_gpu_backend."""
import types

import pytest
import torch

import fake_vllm
from amass import AmassConfig
from amass.backend import _runtime, attn, builder, register


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


FAST = dict(variant="fast", score="quad", quad_rank=8, quad_v_bits=8, budget=None,
            coverage=0.95)


def _backend(vllm, **cfg):
    register.register(dict(FAST, **cfg))
    path = vllm.RocmPlatform.get_attn_backend_cls(None, 128, torch.bfloat16, "auto", 16)
    return path, register._resolve(path)


def test_register_wraps_the_platform_backend(vllm):
    path, be = _backend(vllm)
    assert path == "amass.backend.register.Amass_TritonAttentionBackend"
    assert issubclass(be, vllm.TritonAttentionBackend) and be.get_name() == "TRITON_ATTN"
    impl, bld = be.get_impl_cls(), be.get_builder_cls()
    assert issubclass(impl, attn.AmassAttentionImplMixin)
    assert issubclass(impl, vllm.TritonAttentionImpl)
    assert issubclass(bld, builder.AmassMetadataBuilderMixin)
    assert issubclass(bld, vllm.TritonAttentionMetadataBuilder)
    # the same class comes back on every selection; MLA is left alone
    assert vllm.RocmPlatform.get_attn_backend_cls(None, 128, None, "auto", 16) == path
    assert vllm.RocmPlatform.get_attn_backend_cls(None, 128, None, "auto", 16,
                                                  use_mla=True) == vllm.MLA_PATH
    assert _runtime.get_config() == AmassConfig(**FAST)


def test_disable_env_makes_register_inert(vllm, monkeypatch):
    monkeypatch.setenv("AMASS_DISABLE", "1")
    register.register(FAST)
    assert vllm.RocmPlatform.get_attn_backend_cls(None, 128, None, "auto", 16) == \
        vllm.TRITON_PATH
    assert _runtime.get_config() is None


@pytest.mark.parametrize("cfg,want", [
    ({}, "UNIFORM_SINGLE_TOKEN_DECODE"),
    ({"force_eager": True}, "NEVER"),
    ({"variant": "mem-v"}, "NEVER"),
    ({"variant": "mem-kv"}, "NEVER"),
    ({"score": "clse"}, "UNIFORM_SINGLE_TOKEN_DECODE"),
    ({"score": "r8"}, "UNIFORM_SINGLE_TOKEN_DECODE"),
])
def test_cudagraph_support(vllm, cfg, want):
    _, be = _backend(vllm, **cfg)
    vc = vllm.vllm_config(num_gpu_blocks=0, layers={})
    got = be.get_builder_cls().get_cudagraph_support(vc, vllm.kv_spec())
    assert got.name == want


def test_unserved_geometry_keeps_stock(vllm):
    _, be = _backend(vllm)
    vc = vllm.vllm_config(num_gpu_blocks=0, layers={})
    assert be.get_builder_cls().get_cudagraph_support(
        vc, vllm.kv_spec(head_size=64)).name == "NEVER"


@pytest.mark.parametrize("cfg,n_q,n_kv,max_len", [
    ({"score": "clse"}, 56, 8, 4096),          # G = 7: the r8/CLSE kernels take 1, 2, 4, 8
    ({"score": "r8"}, 24, 8, 4096),            # G = 3
    ({"score": "quad"}, 96, 12, 4096),         # 12 kv heads: <= 8 or a multiple of 8
    ({"score": "r8", "r8_rank": 6}, 32, 8, 4096),
    ({"score": "quad", "quad_rank": 6}, 32, 8, 4096),
    ({}, 32, 8, 16384 * 16 + 1),               # more pages than one selection holds
])
def test_kernel_limits_keep_stock(vllm, cfg, n_q, n_kv, max_len):
    """Layers outside what the kernels accept are refused up front: no graph support,
    the builder attaches no state, so the impl calls the stock attention."""
    _, be = _backend(vllm, **cfg)
    kv = {"l0": torch.zeros(40, 2, 16, n_kv, 128, dtype=torch.bfloat16)}
    vc = vllm.vllm_config(num_gpu_blocks=40, layers=kv, max_model_len=max_len, n_q=n_q)
    bld = be.get_builder_cls()
    assert bld.get_cudagraph_support(vc, vllm.kv_spec(n_kv=n_kv)).name == "NEVER"
    b = bld(vllm.kv_spec(n_kv=n_kv), list(kv), vc, "cpu")
    assert not b._amass_enabled
    md = b.build(0, _cam(torch.tensor([33, 40]), torch.arange(8, dtype=torch.int32).view(2, 4)))
    assert getattr(md, "amass", None) is None
    impl = _impl(be, n_q=n_q, n_kv=n_kv)
    out = torch.zeros(2, n_q * 128)
    impl.forward(None, torch.zeros(2, n_q, 128), None, None, kv["l0"], md, output=out)
    assert impl.calls == ["stock"]


def test_kernel_limits_accept_the_served_shapes():
    base = AmassConfig(**FAST)
    for score, G, rank in (("quad", 7, 8), ("clse", 8, 2), ("r8", 1, 4)):
        cfg = AmassConfig(**dict(FAST, score=score, quad_rank=rank if score != "r8" else 8,
                                 r8_rank=rank if score == "r8" else 8))
        assert _runtime.unsupported_reason(cfg, head_size=128, block_size=16, G=G, n_kv=16,
                                           max_pages=16384) is None, (score, G, rank)
    assert _runtime.unsupported_reason(base, head_size=128, block_size=16, G=4) is None


def _impl(be, n_q=32, n_kv=8):
    return be.get_impl_cls()(n_q, 128, 0.088, n_kv)


def test_impl_delegates_everything_but_pure_decode(vllm, monkeypatch):
    _, be = _backend(vllm)
    calls = []
    monkeypatch.setattr(_runtime, "select", lambda *a: calls.append(("select", a)))
    monkeypatch.setattr(_runtime, "decode_dispatch", lambda *a: calls.append(("decode", a)))
    monkeypatch.setattr(attn, "ResidentVSource", lambda kv: ("vsrc", kv))
    impl = _impl(be)
    kv = torch.zeros(4, 2, 16, 8, 128)
    q = torch.zeros(3, 32, 128)
    out = torch.zeros(3, 32 * 128)
    st = types.SimpleNamespace()
    sl, bt = torch.tensor([5, 9, 17]), torch.zeros(3, 4, dtype=torch.int32)
    decode = vllm.Metadata(seq_lens=sl, block_table=bt, max_query_len=1, causal=True,
                           amass=st)
    for md in (vllm.Metadata(**dict(vars(decode), max_query_len=7)),      # prefill
               vllm.Metadata(**dict(vars(decode), amass=None)),           # no state
               vllm.Metadata(**dict(vars(decode), causal=False)),
               vllm.Metadata(**dict(vars(decode), use_cascade=True))):
        assert impl.forward(None, q, None, None, kv, md, output=out) is out
    assert impl.calls == ["stock"] * 4 and not calls
    impl.sliding_window = (128, 0)
    impl.forward(None, q, None, None, kv, decode, output=out)
    impl.sliding_window = (-1, -1)
    impl.kv_cache_dtype = "fp8"
    impl.forward(None, q, None, None, kv, decode, output=out)
    impl.kv_cache_dtype = "auto"
    assert impl.calls == ["stock"] * 6 and not calls
    assert impl.forward(None, q, None, None, kv, decode, output=out) is out
    assert [c[0] for c in calls] == ["select", "decode"]
    sel, dec = calls[0][1], calls[1][1]
    assert sel[0] is q and sel[1] is kv and sel[4] is st and sel[5] == 3 and sel[6] == 0.088
    assert dec[5].shape == (3, 32, 128) and dec[6] == ("vsrc", kv)
    assert impl.calls == ["stock"] * 6


def _cam(sl, bt, max_q=1):
    return types.SimpleNamespace(seq_lens=sl, block_table_tensor=bt, max_query_len=max_q,
                                 seq_lens_cpu_upper_bound=sl.clone())


def test_builder_lazy_state_refresh_gate_and_derive(vllm, monkeypatch):
    _, be = _backend(vllm)
    rec = []
    import amass.selection as sel
    monkeypatch.setattr(sel, "derive_page_params", lambda st, sl, n: rec.append("derive"))
    monkeypatch.setattr(sel, "quad_build_bulk", lambda *a: rec.append(("bulk", a[4], a[5])))
    monkeypatch.setattr(sel, "quad_build_delta", lambda *a: rec.append(("delta", a[4], a[5])))
    monkeypatch.setattr(sel, "quad_build_tail",
                        lambda *a: rec.append(("tail", a[5].tolist())))
    kv = {f"l{i}": torch.zeros(40, 2, 16, 8, 128, dtype=torch.bfloat16) for i in range(2)}
    vc = vllm.vllm_config(num_gpu_blocks=0, layers=kv, max_num_seqs=4, max_model_len=512)
    b = be.get_builder_cls()(vllm.kv_spec(), list(kv), vc, "cpu")
    bt = torch.arange(8, dtype=torch.int32).view(2, 4)
    md = b.build(0, _cam(torch.tensor([33, 40]), bt))
    assert not hasattr(md, "amass") and not rec                 # cache not allocated yet
    vc.cache_config.num_gpu_blocks = 40
    md = b.build(0, _cam(torch.tensor([33, 40]), bt))
    st = md.amass
    assert type(st).__name__ == "QuadState" and st.L == 2 and st.NB == 40
    assert st.coverage == 0.95 and st.r == 8 and st.max_pages == 32 and st.max_reqs == 4
    assert st._layer_of == {kv["l0"].data_ptr(): 0, kv["l1"].data_ptr(): 1}
    assert rec == [("bulk", 2, 2), "derive"]
    rec.clear()
    b.build(0, _cam(torch.tensor([34, 41]), bt))               # steady, no boundary
    assert rec == []
    b.build(0, _cam(torch.tensor([35, 42]), bt))
    assert rec == []
    want = []
    for _ in range(29):                                           # reach 64 / 71
        cur = b._amass_prev + 1
        crossed = [i for i in range(2) if int(cur[i]) % 16 == 0]
        want += [("tail", crossed)] if crossed else []
        want += ["derive"] if any(int(c) % 16 == 1 for c in cur) else []
        b.build(0, _cam(cur, bt))
    assert rec == want and ("tail", [0]) in rec and ("tail", [1]) in rec
    rec.clear()
    b.build(0, _cam(torch.tensor([65, 72]), bt))                 # 65 % 16 == 1 -> derive
    assert rec == ["derive"]
    rec.clear()
    b.build(0, _cam(torch.tensor([100, 3]), bt))                 # composition change
    assert rec == [("delta", 2, 6), "derive"]
    rec.clear()
    md = b.build(0, _cam(torch.tensor([100, 3]), bt, max_q=5))   # prefill: no state
    assert not hasattr(md, "amass") and rec == []


def test_builder_skips_refresh_during_capture(vllm, monkeypatch):
    _, be = _backend(vllm, score="r8", budget=0.05)
    rec = []
    import amass.selection as sel
    monkeypatch.setattr(sel, "derive_page_params", lambda st, sl, n: rec.append("derive"))
    monkeypatch.setattr(sel, "r8_build_bulk", lambda *a: rec.append("bulk"))
    kv = {"l0": torch.zeros(20, 2, 16, 8, 128, dtype=torch.bfloat16)}
    vc = vllm.vllm_config(num_gpu_blocks=20, layers=kv, max_model_len=256)
    b = be.get_builder_cls()(vllm.kv_spec(), list(kv), vc, "cpu")
    md = b.build_for_cudagraph_capture(_cam(torch.tensor([1, 1]),
                                            torch.zeros(2, 16, dtype=torch.int32)))
    assert type(md.amass).__name__ == "R8State" and md.amass.coverage is None
    assert rec == ["derive"]


class _RecTier:
    """Stands in for amass.tier.Tier: records the write-path calls."""

    def __init__(self, rec):
        self.rec = rec

    def begin_step(self, bt, sl, qsl, n_tok):
        self.rec.append(("begin", n_tok))

    def write_kv(self, lidx, value, n_tokens, key=None):
        self.rec.append(("write", lidx, tuple(value.shape), n_tokens))

    def bytes_report(self):
        return "rec"


def test_mem_v_runs_the_tier_in_shadow(vllm, monkeypatch):
    """mem-v (reference builder.py:243-330, attn.py:84-118): the builder allocates the tier
    lazily and runs its lifecycle on every step -- prefill and decode, over the padded
    token count -- skipping it on capture batches; the impl writes each layer's V into
    the staging pool and attends with the stock attention."""
    _, be = _backend(vllm, variant="mem-v")
    rec = []
    made = {}

    def make_tier(cfg, device, **kw):
        made.update(kw)
        return _RecTier(rec)

    monkeypatch.setattr(_runtime, "make_tier", make_tier)
    kv = {f"l{i}": torch.zeros(40, 2, 16, 8, 128, dtype=torch.bfloat16) for i in range(2)}
    vc = vllm.vllm_config(num_gpu_blocks=0, layers=kv, max_num_seqs=4, max_model_len=512)
    b = be.get_builder_cls()(vllm.kv_spec(), list(kv), vc, "cpu")
    bt = torch.arange(8, dtype=torch.int32).view(2, 4)

    def cam(sl, qsl, max_q, n_pad):
        c = _cam(torch.tensor(sl), bt, max_q)
        c.query_start_loc = torch.tensor(qsl, dtype=torch.int32)
        c.slot_mapping = torch.full((n_pad,), -1, dtype=torch.int64)
        c.num_actual_tokens = qsl[-1]
        return c

    md = b.build(0, cam([20, 9], [0, 20, 29], 20, 29))
    assert not hasattr(md, "amass_tier") and not rec              # cache not allocated
    vc.cache_config.num_gpu_blocks = 40
    md = b.build(0, cam([20, 9], [0, 20, 29], 20, 29))           # prefill step
    assert rec == [("begin", 29)] and isinstance(md.amass_tier, _RecTier)
    assert made["num_blocks"] == 40 and made["num_layers"] == 2 and made["max_pages"] == 32
    assert md.amass_tier._layer_of == {kv["l0"].data_ptr(): 0, kv["l1"].data_ptr(): 1}
    assert not hasattr(md, "amass")                               # no selection in shadow
    rec.clear()
    md = b.build(0, cam([21, 10], [0, 1, 2], 1, 4))              # decode step, padded to 4
    assert rec == [("begin", 4)]
    rec.clear()
    md_cap = b.build_for_cudagraph_capture(cam([1, 1], [0, 1, 2], 1, 2))
    assert rec == [] and isinstance(md_cap.amass_tier, _RecTier)
    impl = be.get_impl_cls()(32, 128, 0.1, 8)
    out = torch.zeros(4, 32, 128)
    value = torch.zeros(4, 8 * 128, dtype=torch.bfloat16)
    impl.forward(None, out, None, value, kv["l1"], md, out)
    assert rec == [("write", 1, (4, 8, 128), 4)] and impl.calls == ["stock"]
    assert be.get_builder_cls().get_cudagraph_support(vc, vllm.kv_spec()).name == "NEVER"


def test_k_only_kv_cache_spec_patch(vllm):
    """The opt-in K-only spec (reference register.py:90-101): a plain full-attention spec
    gets head_size_v = 0; sliding-window and asymmetric specs are refused."""
    register.patch_kv_cache_spec_k_only()
    register.patch_kv_cache_spec_k_only()                         # idempotent
    full = vllm.Attention(vllm.FullAttentionSpec(16, 8, 128, 128))
    assert full.get_kv_cache_spec(None) == vllm.FullAttentionSpec(16, 8, 128, 0)
    with pytest.raises(ValueError, match="SlidingWindowSpec"):
        vllm.Attention(vllm.SlidingWindowSpec(16, 8, 128, 4096)).get_kv_cache_spec(None)
    with pytest.raises(ValueError, match="asymmetric"):
        vllm.Attention(vllm.FullAttentionSpec(16, 8, 128, 64)).get_kv_cache_spec(None)


def test_quad_states_take_the_one_launch_route(monkeypatch):
    """_runtime.select_and_decode sends a quad state (not CLSE) through
    select_then_attend, with the layer the builder bound and the impl's arguments; r8
    and CLSE states go through select + decode_dispatch."""
    import amass.selection as sel_mod
    from amass.selection import QuadState
    calls = []
    monkeypatch.setattr(sel_mod, "select_then_attend", lambda *a: calls.append(("one", a)))
    monkeypatch.setattr(_runtime, "select", lambda *a: calls.append(("select", a)))
    monkeypatch.setattr(_runtime, "decode_dispatch", lambda *a: calls.append(("decode", a)))
    cfg = AmassConfig(**FAST)
    kv = torch.zeros(4, 2, 16, 8, 128)
    q, out, bt, sl = torch.zeros(3, 32, 128), torch.zeros(3, 32, 128), "bt", "sl"
    quad = QuadState.__new__(QuadState)
    quad.coords, quad._layer_of = "none", {kv.data_ptr(): 5}
    _runtime.select_and_decode(q, kv, bt, sl, quad, out, "vs", 3, 0.088, cfg)
    assert [c[0] for c in calls] == ["one"]
    a = calls[0][1]
    assert a[0] is quad and a[1] == 5 and a[2] is q and a[3] is kv and a[6] == 3
    assert a[7] == 0.088 and a[8] is out and a[9] == "vs"
    calls.clear()
    quad.coords = "lse"
    _runtime.select_and_decode(q, kv, bt, sl, quad, out, "vs", 3, 0.088, cfg)
    assert [c[0] for c in calls] == ["select", "decode"]


def test_unit_route_decisions(monkeypatch):
    """select_then_attend's route on a 256-CU GPU: the balanced plan (0; at one request a
    count from the row width); the attend in
    the launch when top-b bounds the kept pages by 64 (by 32 below 16 units) and V is
    resident; without it, at most 16 units with rows of at most 1024 pages; at most 512
    units."""
    import importlib
    from amass.selection import QuadState
    quad_score = importlib.import_module("amass.selection.quad_score")
    monkeypatch.setattr(quad_score, "_num_cus", lambda device: 256)

    def st(R, MP, budget=None, coverage=None, G=4, rank=8):
        s = QuadState("cpu", num_layers=1, num_blocks=2, n_kv=8, G=G, head_dim=128, page=16,
                      max_reqs=R, max_pages=MP, rank=rank, budget=budget or 0.1,
                      combine="nrm")
        s.coverage = coverage
        return s

    route = quad_score.unit_route
    assert route(st(1, 256, budget=0.05), 1, "cpu") == (2, True)       # config 0: bound 16
    assert route(st(1, 256, coverage=0.95), 1, "cpu") == (2, False)    # B = 1: from the row
    assert route(st(1, 1024, budget=0.05), 1, "cpu") == (8, False)     # bound 55, 8 units
    assert route(st(2, 1024, budget=0.05), 2, "cpu") == (0, True)      # bound 55, 16 units
    assert route(st(2, 1024, coverage=0.95), 2, "cpu") == (0, False)
    assert route(st(2, 2048, coverage=0.95), 2, "cpu") is None         # rows of 2048 pages
    assert route(st(8, 1024, budget=0.05), 8, "cpu") == (0, True)
    assert route(st(32, 1024, budget=0.05), 32, "cpu") == (0, True)
    assert route(st(64, 256, budget=0.05), 64, "cpu") == (0, True)     # 512 units
    assert route(st(4, 1024, coverage=0.95), 4, "cpu") is None         # 32 units
    assert route(st(32, 1024, coverage=0.95), 32, "cpu") is None       # config 1
    assert route(st(4, 2048, budget=0.05), 4, "cpu") is None           # bound 106
    assert route(st(128, 256, budget=0.05), 128, "cpu") is None        # 1024 units
    assert route(st(1, 4096, budget=0.05), 1, "cpu") is None           # beyond 2048 pages
    assert route(st(1, 256, budget=0.05, rank=4), 1, "cpu") is None    # r' = 8 only
    # V not resident (the mem-v tier's sources): the launch does not attend
    assert route(st(1, 256, budget=0.05), 1, "cpu", resident=False) == (2, False)
    assert route(st(8, 1024, budget=0.05), 8, "cpu", resident=False) is None
