"""Per-launch HBM traffic and MFMA use of the hot path's kernels from rocprofv3 counters.

    python3 -m amass.bench.counters traffic FETCH_DB WRITE_DB --name NAME [--bench-json J]
    python3 -m amass.bench.counters mfma MFMA_DB --name NAME [--bench-json J]

Input: rocprofv3 ``--pmc`` databases of one ``bench.py --only NAME`` run per counter pass (FETCH_SIZE; WRITE_SIZE; the MFMA set SQ_VALU_MFMA_BUSY_CYCLES
SQ_INSTS_VALU_MFMA_MOPS_BF16 SQ_INSTS_VALU_MFMA_MOPS_I8 SQ_INSTS_MFMA SQ_BUSY_CYCLES
GRBM_GUI_ACTIVE MfmaUtil).  Dispatches are walked in dispatch order and grouped into the
launches bench.py times: a decode dispatch with the merge dispatches after it
(sparse_decode / dense_decode), an nrm pre-pass with the selection after it (select), a
score dispatch (named quad_score / clse_score / r8_score after the bench result), the
per-unit pipeline (quad_select_attend).

traffic: bytes per launch = 1024 * (f * FETCH_SIZE + w * WRITE_SIZE) (KiB counters), with
f and w from torch's neg over 256 MiB fp32 in the same run (reads 256 MiB, writes 256 MiB:
a plain stream).  The second calibration kernel, libamass_calib's gather (every (block,
head) K and V slice of a 2 GiB paged pool read once in random block order with the
decode's 16-byte non-temporal lane pattern), checks that scale on the decode's access
pattern: its scaled traffic over its known bytes is printed beside the hot kernels'.
Prints a table and ``traffic <kernel> <bytes>`` lines, which bench.py reads into each
kernel's ``traffic`` field.

mfma: per launch, MFMA-busy fraction (MfmaUtil: MFMA-busy cycles summed over SIMDs over
GPU-busy cycles x SIMDs; GRBM_GUI_ACTIVE is summed over the 8 XCDs, MfmaUtil uses one
XCD's) and the MFMA operations the counters report (MOPS x 512), as
``mfma <kernel> <util_percent> <bf16_ops> <i8_ops> <mfma_insts>`` lines.
"""
from __future__ import annotations

import argparse
import json
import sqlite3
import sys
from collections import defaultdict

from .profsum import short_name

NEG_BYTES = 256 << 20                 # torch.neg over 64 Mi fp32: reads and writes this
CALIB_PAGES, CALIB_KV = 32768, 8      # bench.py's calibration pool (NB, 2, 16, 8, 128) bf16
CALIB_READ = CALIB_PAGES * CALIB_KV * 2 * 16 * 128 * 2 + 4 * CALIB_PAGES


def classify(name: str) -> str | None:
    n = short_name(name)
    if "gather_calib_kernel" in n:
        return "calib_gather"
    if "neg" in n and "elementwise" in n:
        return "calib_neg"
    if "decode_kernel" in n:
        return "dense_decode" if n.rstrip().endswith("true>") else "sparse_decode"
    if "merge_kernel" in n:
        return "merge"
    if "quad_score_kernel" in n or "r8_score_kernel" in n:
        return "score"          # the CLSE score runs the r8 kernel template too
    if "nrm_pass_kernel" in n or "nrm_kernel" in n:
        return "nrm"
    if "select_kernel" in n:
        return "select"
    if "unit_kernel" in n:
        return "quad_select_attend"
    return None


def dispatches(db_path: str):
    """[(dispatch_id, class, {counter: value})] in dispatch order (known kernels only)."""
    db = sqlite3.connect(db_path)
    rows = db.execute("select kernel_name, dispatch_id, counter_name, value "
                      "from counters_collection").fetchall()
    db.close()
    per = defaultdict(lambda: defaultdict(float))
    cls = {}
    for kname, disp, cname, val in rows:
        c = classify(kname)
        if c is None:
            continue
        cls[disp] = c
        per[disp][cname] += float(val)
    return [(d, cls[d], dict(per[d])) for d in sorted(per)]


def launches(disp):
    """Group dispatches into timed launches: {kernel: [summed counters per launch]}."""
    out = defaultdict(list)
    cur_k, cur = None, None

    def close():
        if cur_k is not None:
            out[cur_k].append(cur)

    for _, c, cs in disp:
        if c == "merge" and cur_k in ("sparse_decode", "dense_decode"):
            for k, v in cs.items():
                cur[k] = cur.get(k, 0.0) + v
            continue
        if c == "select" and cur_k == "nrm":
            cur_k = "select"
            for k, v in cs.items():
                cur[k] = cur.get(k, 0.0) + v
            continue
        close()
        cur_k, cur = c, dict(cs)
    close()
    return out


def mean(xs):
    return sum(xs) / len(xs) if xs else float("nan")


def counter_mean(groups, key):
    return mean([g.get(key, 0.0) for g in groups])


def bench_result(path):
    """The workload's bench.py result (the `only` object of `bench.py --only`)."""
    with open(path) as f:
        lines = [l for l in f if l.strip().startswith("{")]
    res = json.loads(lines[-1])
    return res.get("only", res)


def bench_bytes(res):
    """Algorithmic bytes per launch that bench.py charged each kernel, keyed like the
    launch groups here (select, score, sparse_decode, dense_decode)."""
    out = {}
    for k, v in res.get("kernels", {}).items():
        key = "score" if k.endswith("_score") else ("select" if k.startswith("select") else k)
        out[key] = v.get("bytes")
    if res.get("dense_bytes"):
        out["dense_decode"] = res["dense_bytes"]
    return out


def score_name(res):
    """quad_score / r8_score / clse_score: the score kernel the workload runs."""
    return next((k for k in res.get("kernels", {}) if k.endswith("_score")), "score")


HOT = ("score", "select", "sparse_decode", "dense_decode", "quad_select_attend")


def traffic(fetch_db, write_db, name, bench_json=None):
    fl, wl = launches(dispatches(fetch_db)), launches(dispatches(write_db))
    f_neg = counter_mean(fl["calib_neg"], "FETCH_SIZE")
    w_neg = counter_mean(wl["calib_neg"], "WRITE_SIZE")
    f_gat = counter_mean(fl["calib_gather"], "FETCH_SIZE")
    fs_neg = NEG_BYTES / 1024 / f_neg
    ws = NEG_BYTES / 1024 / w_neg
    fs_gat = CALIB_READ / 1024 / f_gat
    res = bench_result(bench_json) if bench_json else {}
    alg, sname = bench_bytes(res), score_name(res)
    print(f"calibration (same run): neg 256 MiB FETCH {f_neg:.1f} KiB -> read scale "
          f"{fs_neg:.3f}; WRITE {w_neg:.1f} KiB -> write scale {ws:.3f}")
    print(f"pattern check: gather of {CALIB_READ} B (decode pattern, 2 GiB footprint) FETCH "
          f"{f_gat:.1f} KiB -> traffic / bytes = {fs_neg / fs_gat:.3f}")
    print(f"per-launch averages (KiB) and traffic = 1024 * ({fs_neg:.3f} FETCH + {ws:.3f} WRITE)")
    print(f"{'kernel':16s} {'launches':>8s} {'FETCH_SIZE':>12s} {'WRITE_SIZE':>11s} "
          f"{'traffic_B':>12s} {'algorithmic_B':>14s} {'ratio':>6s}")
    lines = []
    for k in HOT:
        if k not in fl or k not in wl:
            continue
        f, w = counter_mean(fl[k], "FETCH_SIZE"), counter_mean(wl[k], "WRITE_SIZE")
        t = int(round(1024 * (fs_neg * f + ws * w)))
        a = alg.get(k)
        ratio = f"{t / a:6.3f}" if a else "     -"
        kn = sname if k == "score" else k
        print(f"{kn:16s} {len(fl[k]):8d} {f:12.1f} {w:11.1f} {t:12d} {a or '-':>14} {ratio}")
        lines.append(f"traffic {kn} {t}")
    print("\nMachine-readable lines (read by bench.py for the kernels' traffic field):")
    print("\n".join(lines))


def mfma(db, name, bench_json=None):
    ls = launches(dispatches(db))
    sname = score_name(bench_result(bench_json)) if bench_json else "score"
    print(f"{'kernel':16s} {'launches':>8s} {'MfmaUtil%':>9s} {'MFMA_BUSY_CYC':>14s} "
          f"{'GUI_ACTIVE':>11s} {'bf16_ops':>14s} {'i8_ops':>14s} {'MFMA_insts':>11s}")
    lines = []
    for k in HOT:
        if k not in ls:
            continue
        g = ls[k]
        util = counter_mean(g, "MfmaUtil")
        busy = counter_mean(g, "SQ_VALU_MFMA_BUSY_CYCLES")
        gui = counter_mean(g, "GRBM_GUI_ACTIVE")
        bf = counter_mean(g, "SQ_INSTS_VALU_MFMA_MOPS_BF16") * 512
        i8 = counter_mean(g, "SQ_INSTS_VALU_MFMA_MOPS_I8") * 512
        ni = counter_mean(g, "SQ_INSTS_MFMA")
        kn = sname if k == "score" else k
        print(f"{kn:16s} {len(g):8d} {util:9.2f} {busy:14.0f} {gui:11.0f} {bf:14.4g} "
              f"{i8:14.4g} {ni:11.0f}")
        lines.append(f"mfma {kn} {util:.3f} {bf:.6g} {i8:.6g} {ni:.0f}")
    print("\nMachine-readable lines (read by bench.py for the roofline's mfma field):")
    print("\n".join(lines))


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("traffic")
    t.add_argument("fetch_db")
    t.add_argument("write_db")
    m = sub.add_parser("mfma")
    m.add_argument("db")
    for p in (t, m):
        p.add_argument("--name", required=True)
        p.add_argument("--bench-json")
    a = ap.parse_args(argv)
    if a.cmd == "traffic":
        traffic(a.fetch_db, a.write_db, a.name, a.bench_json)
    else:
        mfma(a.db, a.name, a.bench_json)
    return 0


if __name__ == "__main__":
    sys.exit(main())
