"""The vLLM general-plugin entry point is declared and resolves to the plugin function.

Reference: ``pyproject.toml:76-80`` declares
``[project.entry-points."vllm.general_plugins"] amass = "amass.backend.register:register"``,
which is how vLLM finds AMASS with no import in user code.  Here the declaration lives in
``amass-kv_amd/setup.cfg``; this test reads it the way setuptools does (``egg_info``) and
resolves it the way vLLM's plugin loader does (``importlib.metadata`` entry points).
"""
from __future__ import annotations

import configparser
import importlib.metadata as md
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "amass-kv_amd")


def test_setup_cfg_declares_plugin():
    cfg = configparser.ConfigParser()
    cfg.read(os.path.join(PKG, "setup.cfg"))
    eps = cfg["options.entry_points"]["vllm.general_plugins"].strip().splitlines()
    assert [e.replace(" ", "") for e in eps] == ["amass=amass.backend.register:register"]
    assert "_lib/*.so" in cfg["options.package_data"]["amass"]
    assert cfg["metadata"]["name"] == "amass-kv"


@pytest.mark.timeout(120)
def test_entry_point_resolves_through_metadata(tmp_path):
    res = subprocess.run([sys.executable, "setup.py", "-q", "egg_info", "--egg-base", str(tmp_path)],
                         cwd=PKG, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    dists = [d for d in md.distributions(path=[str(tmp_path)]) if d.metadata["Name"] == "amass-kv"]
    assert len(dists) == 1
    import amass
    assert dists[0].version == amass.__version__
    eps = [e for e in dists[0].entry_points if e.group == "vllm.general_plugins"]
    assert [e.name for e in eps] == ["amass"]
    fn = eps[0].load()
    from amass.backend.register import register
    assert fn is register
