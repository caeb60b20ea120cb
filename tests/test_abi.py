"""The C-ABI library loads without a GPU, exports every entry point include/amass_hip.h
declares, and the ctypes structs mirror the header (names, order, types, sizeof)."""
import ctypes
import os
import re

import pytest

from amass import _hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                      "include", "amass_hip.h")


def _header_text():
    with open(HEADER) as fh:
        return fh.read()


def _declared_functions():
    txt = re.sub(r"/\*.*?\*/", "", _header_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(amass_\w+)\s*\(",
                                 txt, flags=re.M)))


def _header_structs():
    txt = re.sub(r"/\*.*?\*/", "", _header_text(), flags=re.S)
    out = {}
    for body, name in re.findall(r"typedef struct \w+ \{(.*?)\} (\w+);", txt, flags=re.S):
        fields = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            m = re.match(r"((?:const\s+)?\w+\s*\**)\s*(.*)", decl)
            typ, names = m.group(1).replace(" ", ""), m.group(2)
            for nm in names.split(","):
                nm = nm.strip()
                star = nm.startswith("*")
                nm = nm.lstrip("*").strip()
                fields.append((nm, "p" if ("*" in typ or star) else typ.replace("const", "")))
        out[name] = fields
    return out


_KIND = {"p": ctypes.c_void_p, "int64_t": ctypes.c_int64, "int32_t": ctypes.c_int32,
         "float": ctypes.c_float, "double": ctypes.c_double}


def test_library_loads_and_exports_every_symbol():
    lib = _hip.load_library()
    names = _declared_functions()
    assert len(names) == 25
    for n in names:
        assert hasattr(lib, n), f"{n} declared in the header but not exported"
    assert lib.amass_abi_version() == 11


def test_struct_mirrors_header():
    lib = _hip.load_library()
    hdr = _header_structs()
    assert set(hdr) == set(_hip.STRUCTS)
    for name, (idx, st) in _hip.STRUCTS.items():
        want = [(n, _KIND[k]) for n, k in hdr[name]]
        got = [(n, t) for n, t in st._fields_]
        assert got == want, name
        assert ctypes.sizeof(st) == lib.amass_abi_struct_size(idx), name


def test_status_strings_and_null_rejection():
    lib = _hip.load_library()
    assert _hip.status_string(0) == "ok"
    assert "NULL" in _hip.status_string(-1)
    # NULL pointers are rejected on the host before any launch (no GPU touched)
    a = _hip.QuadScoreArgs()
    assert lib.amass_quad_score(ctypes.byref(a), None) == -1
    d = _hip.DecodeArgs()
    assert lib.amass_sparse_decode(ctypes.byref(d), None) == -1
    assert lib.amass_topb_select(None, None) == -1
    b = _hip.BuildArgs()
    assert lib.amass_summary_build(ctypes.byref(b), None) == -1
    assert lib.amass_host_pool_alloc(16, None, None) == -1


def test_copy_runs_checked_before_any_copy():
    """amass_tier_dma checks the whole run list before issuing a copy: a bad run after good
    ones (zero width; a pitch narrower than the row) is refused with no HIP call made."""
    lib = _hip.load_library()
    runs = (_hip.CopyRun * 2)()
    for r in runs:
        r.dst, r.src, r.dpitch, r.spitch, r.width, r.height = 0x1000, 0x2000, 256, 256, 256, 4
    runs[1].width = 0
    assert lib.amass_tier_dma(runs, 2, None) == -2
    runs[1].width, runs[1].spitch = 256, 128
    assert lib.amass_tier_dma(runs, 2, None) == -2
    assert lib.amass_tier_dma(None, 1, None) == -1
    assert lib.amass_tier_dma(runs, -1, None) == -2


def test_missing_library_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(_hip, "_LIB", None)
    with pytest.raises(_hip.AmassError, match="missing"):
        _hip.load_library(str(tmp_path / "nope.so"))


def test_product_never_imports_the_oracle():
    """The shipped package has no CPU fallback: nothing under amass-kv_amd imports oracle."""
    import re
    pkg = os.path.join(ROOT, "amass-kv_amd")
    pat = re.compile(r"^\s*(from\s+oracle\b|import\s+oracle\b)", re.M)
    for dp, _dn, fns in os.walk(pkg):
        for fn in fns:
            if fn.endswith((".py", ".hip", ".h", ".cpp")):
                with open(os.path.join(dp, fn)) as f:
                    assert not pat.search(f.read()), os.path.join(dp, fn)
