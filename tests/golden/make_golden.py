"""Write the frozen oracle fixtures in this folder (run from the repository root):

    python3 tests/golden/make_golden.py

Each fixture holds small seeded inputs and the oracle's outputs for them (queries and
K/V are bf16-representable, as the kernels take them in bf16).  The
reference ships no golden vectors for this path, so these are the oracle's own answers
after it passed the closed-form, brute-force and hand-worked checks of
tests/test_oracle_pins.py; tests/test_golden.py recomputes them, so any later change to
the oracle's behaviour shows up as a fixture mismatch.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import oracle.decode as odec   # noqa: E402
import oracle.quant as oq      # noqa: E402
import oracle.score as osc     # noqa: E402
import oracle.select as osel   # noqa: E402
import oracle.tier as otier    # noqa: E402


def quad_inputs(seed=0, R=2, NB=12, n_kv=2, G=4, d=128, r=8, v_bits=8):
    rng = np.random.default_rng(seed)
    q = oq.bf16_round((rng.standard_normal((R, n_kv * G, d)) * 1.5).astype(np.float32))
    mu = rng.integers(-127, 128, (NB, n_kv, d)).astype(np.int8)
    mus = rng.uniform(0.005, 0.02, (NB, n_kv)).astype(np.float16)
    lvl = 127 if v_bits == 8 else 7
    code = rng.integers(-lvl, lvl + 1, (NB, n_kv, d, r)).astype(np.int8)
    V = code if v_bits == 8 else oq.pack_i4(code)
    Vs = rng.uniform(0.001, 0.01, (NB, n_kv, r)).astype(np.float16)
    sg = rng.uniform(0.1, 4.0, (NB, n_kv, r)).astype(np.float16)
    bt = np.stack([rng.permutation(NB) for _ in range(R)]).astype(np.int32)
    nsh = np.array([NB - 1, NB // 2], np.int32)
    return dict(q=q, mu=mu, mu_scale=mus, V=V, V_scale=Vs, sig2=sg, block_table=bt,
                n_sel_hi=nsh)


def quad_outputs(inp, G=4, v_bits=8):
    kw = dict(scale=1 / np.sqrt(128), page=16, G=G, v_bits=v_bits, max_pages=inp["block_table"].shape[1])
    args = [inp[k] for k in ("q", "mu", "mu_scale", "V", "V_scale", "sig2", "block_table",
                             "n_sel_hi")]
    a = dict(score_max=osc.quad_score(*args, combine="max", **kw),
             score_h=osc.quad_score(*args, combine="nrm", **kw),
             score_h_limbs=osc.quad_score(*args, combine="nrm", q_mode="limbs", **kw))
    a["nrm"] = osc.nrm_combine(a["score_h"], inp["n_sel_hi"])
    a["comb"] = osc.quad_comb(inp["q"], inp["mu"], inp["V"], inp["block_table"],
                              inp["n_sel_hi"], G=G, v_bits=v_bits, max_pages=kw["max_pages"])
    return a


def r8_inputs(seed=1, R=2, NB=6, n_kv=2, G=4, d=128, r=8, P=16):
    rng = np.random.default_rng(seed)
    q = oq.bf16_round(rng.standard_normal((R, n_kv * G, d)).astype(np.float32))
    mu = rng.integers(-127, 128, (NB, n_kv, d)).astype(np.int8)
    mus = rng.uniform(0.005, 0.02, (NB, n_kv)).astype(np.float16)
    Vk = rng.integers(-127, 128, (NB, n_kv, d, r)).astype(np.int8)
    vks = rng.uniform(0.001, 0.01, (NB, n_kv, r)).astype(np.float16)
    c = rng.integers(-127, 128, (NB, n_kv, P, r)).astype(np.int8)
    cs = rng.uniform(0.005, 0.02, (NB, n_kv, P)).astype(np.float16)
    bt = np.stack([rng.permutation(NB) for _ in range(R)]).astype(np.int32)
    sl = np.array([NB * P - 7, 3 * P], np.int32)
    nsh = np.array([NB - 1, 2], np.int32)
    return dict(q=q, mu=mu, mu_scale=mus, Vk=Vk, Vk_scale=vks, c=c, c_scale=cs,
                block_table=bt, seq_lens=sl, n_sel_hi=nsh)


def r8_outputs(inp, G=4):
    args = [inp[k] for k in ("q", "mu", "mu_scale", "Vk", "Vk_scale", "c", "c_scale",
                             "block_table", "seq_lens", "n_sel_hi")]
    return dict(score=osc.r8_score(*args, scale=1 / np.sqrt(128), page=16, G=G, vk_bits=8,
                                   c_bits=8, max_pages=inp["block_table"].shape[1]))


def select_inputs(seed=2, R=4, n_kv=2, MP=50):
    rng = np.random.default_rng(seed)
    sc = (np.round(rng.standard_normal((R, n_kv, MP)) * 8) / 4).astype(np.float32)
    npg = np.array([50, 23, 2, 0], np.int32)
    return dict(score=sc, n_pages=npg, n_sel_hi=(npg - 1).astype(np.int32),
                b_fix=np.array([6, 40, 1, 1], np.int32))


def select_outputs(inp):
    out = {}
    args = (inp["score"], inp["n_pages"], inp["n_sel_hi"], inp["b_fix"])
    for mode, cov in ((0, 1.0), (1, 0.9)):
        for tie in (0, 1):
            for kind in (0, 1):
                if mode == 0 and kind == 1:
                    continue
                sc = np.abs(args[0]) if kind == 1 else args[0]
                t, c, n = osel.select(sc, *args[1:], sink=1, max_pages=sc.shape[-1],
                                      mode=mode, coverage=cov, tie_mode=tie,
                                      score_kind=kind)
                key = f"m{mode}_t{tie}_k{kind}"
                out[key + "_tab"], out[key + "_cnt"], out[key + "_nsel"] = t, c, n
    npg, nsh, b = osel.derive([4096, 100, 16, 65536], 0.05, page=16, window=1, sink=1)
    out["derive"] = np.stack([npg, nsh, b])
    x = np.linspace(-85, 0, 4097, dtype=np.float32)
    out["exp_det"] = osel.exp_det(x)
    return out


def decode_inputs(seed=3, R=2, NB=6, n_kv=2, G=4, d=128, P=16):
    rng = np.random.default_rng(seed)
    import numpy as _np
    K = oq.bf16_round(rng.standard_normal((NB, P, n_kv, d)).astype(_np.float32))
    V = oq.bf16_round(rng.standard_normal((NB, P, n_kv, d)).astype(_np.float32))
    q = oq.bf16_round(rng.standard_normal((R, n_kv * G, d)).astype(_np.float32))
    bt = np.stack([rng.permutation(NB) for _ in range(R)]).astype(np.int32)
    sl = np.array([NB * P - 9, 4 * P + 1], np.int32)
    pt = np.full((R, n_kv, NB), -1, np.int32)
    cnt = np.zeros((R, n_kv), np.int32)
    for r in range(R):
        npg = -(-int(sl[r]) // P)
        for kv in range(n_kv):
            pages = np.sort(rng.choice(npg, min(4, npg), replace=False))
            pt[r, kv, :pages.size] = pages
            cnt[r, kv] = pages.size
    return dict(q=q, K=K, V=V, block_table=bt, seq_lens=sl, page_table=pt, page_cnt=cnt)


def decode_outputs(inp, G=4):
    a = [inp[k] for k in ("q", "K", "V", "block_table", "seq_lens")]
    sparse = odec.attend(*a, inp["page_table"], inp["page_cnt"], scale=1 / np.sqrt(128), G=G)
    dense = odec.attend(*a, scale=1 / np.sqrt(128), G=G, dense=True)
    return dict(sparse=sparse, dense=dense)


def tier_inputs(seed=4, R=3, n_kv=2, NB=40, S=10, P=16, steps=4):
    rng = np.random.default_rng(seed)
    bt = np.stack([rng.permutation(NB) for _ in range(R)]).astype(np.int32)
    sl = np.array([NB * P, NB * P - 3, 20 * P], np.int32)
    pts = np.full((steps, R, n_kv, 6), -1, np.int32)
    cnts = np.zeros((steps, R, n_kv), np.int32)
    for s in range(steps):
        for r in range(R):
            for kv in range(n_kv):
                pages = np.sort(rng.choice(20, 4, replace=False))
                pts[s, r, kv, :4] = pages
                cnts[s, r, kv] = 4
    return dict(block_table=bt, seq_lens=sl, page_tables=pts, page_cnts=cnts,
                slots=np.array([S]), NB=np.array([NB]))


def tier_outputs(inp):
    n_kv = inp["page_tables"].shape[2]
    NB, S = int(inp["NB"][0]), int(inp["slots"][0])
    st = dict(page2slot=np.full((n_kv, NB), -1), slot2page=np.full((n_kv, S), -1),
              lru=np.zeros((n_kv, S), np.int64), clock=0)
    out = {}
    for s in range(inp["page_tables"].shape[0]):
        st = otier.plan(inp["page_tables"][s], inp["page_cnts"][s], inp["block_table"],
                        inp["seq_lens"], st["page2slot"], st["slot2page"], st["lru"],
                        st["clock"], page=16)
        out[f"s{s}_page2slot"] = st["page2slot"]
        out[f"s{s}_slot2page"] = st["slot2page"]
        out[f"s{s}_lru"] = st["lru"]
        out[f"s{s}_fetch"] = np.array(sorted(st["fetch"]), np.int64).reshape(-1, 3)
    return out


CASES = {
    "quad_i8": (lambda: quad_inputs(), lambda i: quad_outputs(i)),
    "quad_i4_r4": (lambda: quad_inputs(seed=5, r=4, v_bits=4),
                   lambda i: quad_outputs(i, v_bits=4)),
    "r8": (r8_inputs, r8_outputs),
    "select": (select_inputs, select_outputs),
    "decode": (decode_inputs, decode_outputs),
    "tier": (tier_inputs, tier_outputs),
}


def main():
    for name, (mk_in, mk_out) in CASES.items():
        inp = mk_in()
        out = mk_out(inp)
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"),
                            **{f"in_{k}": v for k, v in inp.items()},
                            **{f"out_{k}": v for k, v in out.items()})
        print(f"wrote {name}.npz")


if __name__ == "__main__":
    main()
