"""AmassConfig surface: same fields, defaults, validation and AMASS_CONFIG rules as the
reference (src/amass/config.py:26-165)."""
import dataclasses
import json

import pytest

from amass import AmassConfig, __version__


def test_defaults_match_reference():
    c = AmassConfig()
    assert c.variant == "mem-v" and c.coverage == 0.95 and c.budget is None
    assert c.sink_pages == 1 and c.window_pages == 1 and c.score == "clse"
    assert c.quad_rank == 2 and c.quad_v_bits == 4 and c.quad_combine == "nrm"
    assert c.hot_slots == 2048 and c.max_pool_gb == 256.0 and c.r8_rank == 8
    assert c.is_mem and not c.offload_k
    assert __version__ == "0.1.1"


def test_field_set():
    names = [f.name for f in dataclasses.fields(AmassConfig)]
    assert names == ["variant", "coverage", "budget", "table", "sink_pages", "window_pages",
                     "r8_screen", "r8_rank", "score", "quad_rank", "quad_v_bits",
                     "quad_combine", "quad_c_bits", "quad_c_grain", "hot_slots", "v_blocks",
                     "max_pool_gb", "use_cuda", "force_eager"]


@pytest.mark.parametrize("bad", [dict(variant="x"), dict(coverage=0.0), dict(coverage=1.5),
                                 dict(budget=0.0), dict(score="foo"), dict(quad_rank=0),
                                 dict(quad_v_bits=2), dict(quad_combine="sum"),
                                 dict(quad_c_bits=3), dict(quad_c_grain="x")])
def test_validation(bad):
    with pytest.raises(ValueError):
        AmassConfig(**bad)


def test_mem_kv_forces_r8_screen():
    assert AmassConfig(variant="mem-kv").r8_screen is True


def test_load_inline_and_file(monkeypatch, tmp_path):
    monkeypatch.setenv("AMASS_CONFIG", json.dumps({"variant": "fast", "score": "quad"}))
    c = AmassConfig.load({"budget": 0.05})
    assert c.variant == "fast" and c.score == "quad" and c.budget == 0.05
    p = tmp_path / "c.yaml"
    p.write_text("variant: fast\nquad_rank: 8\n")
    monkeypatch.setenv("AMASS_CONFIG", str(p))
    assert AmassConfig.load().quad_rank == 8
    monkeypatch.setenv("AMASS_CONFIG", json.dumps({"nope": 1}))
    with pytest.raises(ValueError, match="unknown AmassConfig keys"):
        AmassConfig.load()
