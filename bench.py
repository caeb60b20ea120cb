#!/usr/bin/env python3
"""Decode-step benchmark of the AMASS sparse-attention hot path on one MI355X.

Metric: sparse decode attention time per decode step per layer
(score + select + attend, HIP-graph replay) at config 1 -- B=32, ctx 16384, Llama-3.1-8B
GQA (32 q / 8 kv heads, d=128), bf16 paged KV (page 16, permuted block tables), quad
summary r'=8 int8, nrm combine, per-head coverage nucleus 0.95 -- plus HBM GB/s and the
speedup over a dense paged decode of all 1024 pages on the same GPU.

One JSON line is printed.  `value` is the sparse step time in us per layer (lower is
better); `roofline` is for the kernel with the largest share of the step, using its
algorithmic bytes per launch over its average duration measured with HIP events on the
launch stream; `cpu_baseline` times the CPU oracle (the numpy restatement of the
reference's score / select / attend path) on a bounded sample of the same workload.
Inputs are synthetic (amass.bench.synth, seeded) and resident in HBM before timing.

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline] [--quick]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "amass-kv_amd"))

PEAK_HBM = 8.0e12   # MI355X HBM3E, bytes/s


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def graph_of(fn, reps=1):
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    torch.cuda.synchronize()
    return g


def time_graph(g, steps, warmup, reps=1, batches=7):
    """Median over `batches` of the average ms per call of `steps` back-to-back replays of
    a graph holding `reps` calls (one event pair per batch on the replay stream) -- the
    reference's median-of-batches graph timing (bench/timing.py:71-117)."""
    import statistics

    import torch
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    out = []
    for _ in range(batches):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            g.replay()
        b.record()
        torch.cuda.synchronize()
        out.append(a.elapsed_time(b) / (steps * reps))
    return statistics.median(out)


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_config1.txt")


def profiled_traffic():
    """HBM bytes per launch measured by rocprofv3 (FETCH_SIZE / WRITE_SIZE, calibrated
    against a kernel of known size) for the config-1 kernels: the `traffic <kernel>
    <bytes>` lines of profiles/hbm_traffic_config1.txt, or {} when it is absent."""
    out = {}
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 3 and parts[0] == "traffic":
                    out[parts[1]] = int(parts[2])
    except OSError:
        pass
    return out


def quad_score_bytes(st, n_req, G):
    """Algorithmic HBM bytes of one quad-score launch: per scored (page, kv-head) record
    d*r'*vb/8 (V) + d (mu) + 2r' (V_scale) + 2r' (sig2) + 2 (mu_scale), plus the block
    table, q, and the per-head score write (nrm: G floats per record)."""
    nsh = st.n_sel_hi[:n_req].clamp_min(0).long()
    units = int(nsh.sum()) * st.n_kv
    rec = st.d * st.r * st.v_bits // 8 + st.d + 2 * st.r + 2 * st.r + 2
    out = 4 * (G if st.combine == "nrm" else 1)
    return units * (rec + out) + int(nsh.sum()) * 4 + n_req * st.n_kv * G * st.d * 2


def select_bytes(st, n_req, G):
    """score_h read (G floats per record) + score write + page_table + page_cnt."""
    nsh = st.n_sel_hi[:n_req].clamp_min(0).long()
    units = int(nsh.sum()) * st.n_kv
    return units * (G * 4 + 4) + n_req * st.n_kv * st.max_pages * 4 + n_req * st.n_kv * 4


def attend_bytes(cnt, n_req, n_kv, G, d=128, page=16):
    """K + V of every attended page (16*d*2 bytes each) + its page-table entry + block
    id, plus q and out."""
    pages = int(cnt[:n_req].long().sum())
    return pages * (page * d * 2 * 2 + 4 + 4) + 2 * n_req * n_kv * G * d * 2


def cpu_baseline(case, st, budget_s=15.0):
    """Time the CPU oracle chain (quad score fp64 -> nrm -> coverage select -> attend) on
    whole requests until ~budget_s of work, then scale to the full batch."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    import oracle.decode as odec
    import oracle.score as osc
    import oracle.select as osel

    f = lambda t: t.detach().float().cpu().numpy()  # noqa: E731
    i = lambda t: t.detach().cpu().numpy()          # noqa: E731
    mu, mus, _, Vs, sg, _ = st.layer_state(0)
    V = st.reference_V(0)
    host = dict(q=f(case.q), mu=i(mu), mus=f(mus), V=i(V), Vs=f(Vs), sg=f(sg),
                bt=i(case.block_table), sl=i(case.seq_lens), K=f(case.kv_cache[:, 0]),
                Vc=f(case.kv_cache[:, 1]), npg=i(st.n_pages), nsh=i(st.n_sel_hi),
                bfix=i(st.b_fix))
    B = case.q.shape[0]
    done, t_total = 0, 0.0
    with threadpool_limits(limits=1):
        while done < B and t_total < budget_s:
            r = slice(done, done + 1)
            t0 = time.perf_counter()
            sh = osc.quad_score(host["q"][r], host["mu"], host["mus"], host["V"], host["Vs"],
                                host["sg"], host["bt"][r], host["nsh"][r], scale=case.scale,
                                page=16, G=case.G, v_bits=st.v_bits, max_pages=st.max_pages,
                                combine="nrm")
            sc = osc.nrm_combine(sh, host["nsh"][r]).astype(np.float32)
            tab, cnt, _ = osel.select(sc, host["npg"][r], host["nsh"][r], host["bfix"][r],
                                      sink=1, max_pages=st.max_pages, mode=1, coverage=0.95,
                                      score_kind=1)
            odec.attend(host["q"][r], host["K"], host["Vc"], host["bt"][r], host["sl"][r],
                        tab, cnt, scale=case.scale, G=case.G)
            t_total += time.perf_counter() - t0
            done += 1
    us_full = t_total / done * B * 1e6
    return {"value": round(us_full, 1), "unit": "us/layer", "cores": 1, "kind": "port",
            "sample": f"{done} of {B} requests of config 1 (oracle: quad fp64 score, nrm, "
                      f"coverage select, fp64 attend; numpy, 1 thread), scaled x{B / done:.1f}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--boost", default="sigma", choices=["sigma", "keynorm"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--quick", action="store_true", help="headline only (for profiling)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 256 MiB read + 256 MiB write kernel (HBM counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: the hot path has no "
                                   "cross-GPU component (see DESIGN.md, sharding note); "
                                   "run with --gpus 1"}))
        sys.exit(2)

    import torch

    from amass.attention.decode import (ResidentVSource, dense_paged_decode,
                                        sparse_paged_decode_batched)
    from amass.bench.synth import build_quad_state, config_case
    from amass.selection import derive_page_params, select_pages_quad
    from amass.selection.quad_score import quad_score_launch
    from amass.selection.select import select_pages

    dev = "cuda"
    if args.copy_calibration:
        src = torch.empty(64 << 20, dtype=torch.float32, device=dev).normal_()
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)     # one elementwise kernel: reads 256 MiB, writes 256 MiB
        torch.cuda.synchronize()
        log("copy calibration: 3 x 256 MiB device copies done")
        del src, dst
    t0 = time.time()
    case = config_case(1, seed=args.seed, device=dev, boost=args.boost)
    log(f"inputs generated ({time.time() - t0:.1f}s)")
    st = build_quad_state(case, rank=8, v_bits=8, combine="nrm", coverage=0.95)
    log(f"quad summaries built ({time.time() - t0:.1f}s)")
    B, G, n_kv = case.q.shape[0], case.G, case.n_kv
    q, kv, bt, sl = case.q, case.kv_cache, case.block_table, case.seq_lens
    derive_page_params(st, sl, B)
    out = torch.zeros(B, n_kv * G, 128, dtype=torch.bfloat16, device=dev)
    out_d = torch.zeros_like(out)
    vsrc = ResidentVSource(kv)

    def sparse_step():
        select_pages_quad(st, 0, q, bt, sl, B, case.scale, derive=False)
        sparse_paged_decode_batched(q, kv, bt, sl, st, out, vsrc, scale=case.scale)

    def dense_step():
        dense_paged_decode(q, kv, bt, sl, st, out_d, scale=case.scale)

    sparse_step()
    dense_step()
    torch.cuda.synchronize()
    g_sparse = graph_of(sparse_step)
    g_dense = graph_of(dense_step)
    ms_sparse = time_graph(g_sparse, args.steps, args.warmup)
    ms_dense = time_graph(g_dense, args.steps, args.warmup)
    log(f"sparse {ms_sparse * 1e3:.1f} us, dense {ms_dense * 1e3:.1f} us")

    # ---- per-kernel durations (each kernel repeated inside one graph) ----------------
    reps = 10
    k_steps = max(5, args.steps // 5)
    g_score = graph_of(lambda: quad_score_launch(st, 0, q, bt, B, case.scale), reps)
    us_score = time_graph(g_score, k_steps, 2, reps) * 1e3
    g_sel = graph_of(lambda: select_pages(st, B, score_h=st.score_h), reps)
    us_sel = time_graph(g_sel, k_steps, 2, reps) * 1e3
    g_att = graph_of(lambda: sparse_paged_decode_batched(q, kv, bt, sl, st, out, vsrc,
                                                          scale=case.scale), reps)
    us_att = time_graph(g_att, k_steps, 2, reps) * 1e3
    torch.cuda.synchronize()
    cnt = st.page_cnt[:B]
    nsel = st.n_sel[:B].double()
    S_all = (st.n_sel_hi[:B] - st.sink_pages).clamp_min(0).double()
    frac = float(nsel.sum() / (S_all.sum() * n_kv))
    att_frac = float(cnt.double().sum() / (st.n_pages[:B].double().sum() * n_kv))
    b_score = quad_score_bytes(st, B, G)
    b_sel = select_bytes(st, B, G)
    b_att = attend_bytes(cnt, B, n_kv, G)
    b_dense = attend_bytes(st.n_pages[:B][:, None].expand(B, n_kv), B, n_kv, G)
    kernels = {
        "quad_score": dict(us=round(us_score, 2), bytes=b_score,
                           gbs=round(b_score / us_score / 1e3, 1)),
        "select_nrm_coverage": dict(us=round(us_sel, 2), bytes=b_sel,
                                    gbs=round(b_sel / us_sel / 1e3, 1)),
        "sparse_decode": dict(us=round(us_att, 2), bytes=b_att,
                              gbs=round(b_att / us_att / 1e3, 1)),
    }
    traffic = profiled_traffic()
    for k, v in kernels.items():
        v["traffic"] = traffic.get(k)
    dom = max(kernels, key=lambda k: kernels[k]["us"])
    dk = kernels[dom]
    roof = {"bound": "hbm", "kernel": dom, "achieved": round(dk["bytes"] / dk["us"] / 1e3, 1),
            "peak": PEAK_HBM / 1e9, "unit": "GB/s",
            "frac": round(dk["bytes"] / (dk["us"] * 1e-6) / PEAK_HBM, 4),
            "traffic": traffic.get(dom),
            "traffic_source": "profiles/hbm_traffic_config1.txt: rocprofv3 FETCH_SIZE x2.000 "
                              "+ WRITE_SIZE x1.000 (scales from a 256 MiB neg kernel)"
            if dom in traffic else None}
    total_bytes = b_score + b_sel + b_att
    res = {
        "metric": "sparse decode attn us/layer + HBM GB/s at B=32 ctx16k; speedup vs dense paged",
        "value": round(ms_sparse * 1e3, 2), "unit": "us/layer", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_sparse, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 score / bf16 attention", "data": "synthetic",
        "config": {"workload": "config1: B=32 ctx16384 llama3.1-8B GQA (32q/8kv, d128), "
                               "bf16 paged KV page16 permuted pool, quad r'=8 int8 nrm, "
                               "coverage 0.95, one layer",
                   "boost": f"{args.boost} (beta={case.meta['beta']:.3f})",
                   "graph": "hipGraph replay of score+select+attend"},
        "gb_s": round(total_bytes / (ms_sparse * 1e-3) / 1e9, 1),
        "dense_us": round(ms_dense * 1e3, 2),
        "dense_gb_s": round(b_dense / (ms_dense * 1e-3) / 1e9, 1),
        "speedup_vs_dense": round(ms_dense / ms_sparse, 3),
        "selected_fraction": round(frac, 4), "attended_fraction": round(att_frac, 4),
        "kernels": kernels,
        "roofline": roof,
    }
    if not args.quick:
        # secondary: fixed 5% budget at the same shape (same summaries, top-b selection)
        st.coverage = None
        st.budget = 0.05
        derive_page_params(st, sl, B)
        g_b = graph_of(sparse_step)
        ms_b = time_graph(g_b, args.steps, args.warmup)
        res["fixed_budget_5pct"] = {"us": round(ms_b * 1e3, 2),
                                    "speedup_vs_dense": round(ms_dense / ms_b, 3)}
        st.coverage = 0.95
        derive_page_params(st, sl, B)
        torch.cuda.synchronize()
        del g_b
    if not args.no_cpu_baseline:
        sparse_step()
        torch.cuda.synchronize()
        res["cpu_baseline"] = cpu_baseline(case, st)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
