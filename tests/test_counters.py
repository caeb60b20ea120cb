"""Host logic of the counter summaries (amass.bench.counters) and of bench.py's reading of
the committed profiles: dispatch grouping into timed launches, and a traffic and an MFMA
figure for every kernel of the config-1/2/3 workloads."""
import importlib.util
import os

import pytest

from amass.bench import counters

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_classify_names():
    c = counters.classify
    assert c("void amass::decode_kernel<0, false>(amass_decode_args)") == "sparse_decode"
    assert c("void amass::decode_kernel<0, true>(amass_decode_args)") == "dense_decode"
    assert c("amass::merge_kernel(amass_decode_args)") == "merge"
    assert c("void amass::r8_score_kernel<2, 4, 4, 4, false, true>(R8Params)") == "score"
    assert c("void amass::quad_score_kernel<8, 8, true, false>(x)") == "score"
    assert c("amass::nrm_pass_kernel(amass_select_args)") == "nrm"
    assert c("void amass::select_kernel<512, 2, true>(amass_select_args)") == "select"
    assert c("amass_calib::gather_calib_kernel(unsigned short const*)") == "calib_gather"
    assert c("void amass::unit_kernel<8, 8, 1, true>(QuadParams, amass_select_args, "
             "amass_decode_args)") == "quad_select_attend"
    assert c("amass::derive_kernel(amass_derive_args)") is None


def test_launch_grouping():
    """A decode absorbs the merges after it; an nrm pre-pass and the selection after it
    are one select launch; anything else starts a new launch."""
    d = [(1, "score", {"X": 1.0}), (2, "nrm", {"X": 2.0}), (3, "select", {"X": 3.0}),
         (4, "sparse_decode", {"X": 10.0}), (5, "merge", {"X": 1.0}),
         (6, "dense_decode", {"X": 20.0}), (7, "merge", {"X": 2.0}),
         (8, "select", {"X": 4.0}), (9, "merge", {"X": 7.0})]
    g = counters.launches(d)
    assert [x["X"] for x in g["select"]] == [5.0, 4.0]
    assert [x["X"] for x in g["sparse_decode"]] == [11.0]
    assert [x["X"] for x in g["dense_decode"]] == [22.0]
    assert [x["X"] for x in g["merge"]] == [7.0]      # a merge after no decode stays apart


@pytest.mark.parametrize("name,score", [("config1", "quad_score"), ("config2", "r8_score"),
                                        ("config2_page_f32", "r8_score"),
                                        ("config3", "quad_score"),
                                        ("config1_keynorm", "quad_score"),
                                        ("config1_clse", "clse_score")])
def test_profiles_cover_every_kernel(name, score):
    b = _bench()
    t, m = b.profiled_traffic(name), b.profiled_mfma(name)
    for k in (score, "select", "sparse_decode", "dense_decode"):
        assert t.get(k, 0) > 0, (name, k)
        assert k in m, (name, k)
    e = b.mfma_entry(100.0, m["sparse_decode"])
    assert e["type"] == "bf16" and 0 < e["frac"] < 1 and e["busy_pct"] > 0
    assert b.mfma_entry(100.0, m[score])["type"] == "i8"


def test_config0_profile_covers_the_one_launch_route():
    """Config 0 takes the one-launch route (amass_quad_select_attend); its profile carries a
    traffic and an MFMA line for that launch beside the separate kernels'."""
    b = _bench()
    t, m = b.profiled_traffic("config0"), b.profiled_mfma("config0")
    for k in ("quad_select_attend", "quad_score", "select", "sparse_decode"):
        assert t.get(k, 0) > 0, k
        assert k in m, k
