"""Write tests/golden/ref_vectors.json from the reference sampler itself.

Run in a checkout where the reference source is available:

    make -C oracle            # builds oracle/_ref/libref_sample.so from the reference sample.c
    python tests/golden/make_golden.py

The reference (franzvill/quasar) ships no test vectors for its sampler, so the vectors
are produced here by its own sample.c, compiled unmodified (oracle/ref_harness.c only
adds a history preload and state read-back).  The file holds data only: seeds,
parameters, small raw logit rows (as float bit patterns) and the ids, generator states
and histories the reference returned.  Full-width rows are named by (workload, row) and
regenerated bit-exactly by the portable generator; their CRC32 is stored to pin that.

Sections:
  clamps    sample.c:47-68 stored parameters for a grid of inputs
  workload  full-width rows of the five workloads and three stress settings:
            several consecutive picks per row (history and RNG evolve)
  edge      hand-built small rows: ties, NaN, +-inf, -0, the window edge, p-ties that
            differ from greedy, ring wrap-around, V not a multiple of 4
  fuzz      random small rows with random (including out-of-range) parameters
"""
import json
import os
import struct
import sys
import zlib

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, ROOT)

from pyoracle import Oracle, RefSampler  # noqa: E402
from quasar_amd.workloads import STRESS, WORKLOADS  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ref_vectors.json")


def f32(x):
    return float(np.float32(x))


def bits_of(a):
    return [int(x) for x in np.asarray(a, dtype=np.float32).view(np.uint32)]


def run_both(ref, orc, logits_rows, params, seed, history, picks):
    """Run `picks` consecutive picks (row k % len(rows)) on the reference and on the
    restatement; assert they agree; return the reference's outcome."""
    rs, os_ = ref.sampler(), orc.sampler()
    for s in (rs, os_):
        s.config(*params, seed=seed)
        if history is not None and len(history):
            s.set_history(history)
    ids = []
    for k in range(picks):
        row = logits_rows[k % len(logits_rows)]
        a, b = rs.pick(row), os_.pick(row)
        assert a == b, ("restatement disagrees with the reference", params, k, a, b)
        ids.append(int(a))
    assert rs.rng == os_.rng
    h = rs.history()
    assert (h == os_.history()).all()
    out = {"ids": ids, "rng_after": "%016x" % rs.rng, "hist_len": int(len(h)),
           "hist_tail": [int(x) for x in h[-min(len(h), 8):]],
           "hist_crc": zlib.crc32(h.astype(np.int32).tobytes())}
    rs.close()
    os_.close()
    return out


def clamps(ref):
    grid_T = [-1.0, 0.0, 1e-3, 0.7, 2.0]
    grid_p = [-0.5, 0.0, 1e-6, 0.9, 1.0, 1.5]
    grid_k = [-5, 0, 1, 40]
    grid_m = [-0.1, 0.0, 0.05, 1.0]
    grid_rp = [0.5, 1.0, 1.1]
    grid_n = [-3, 0, 64]
    out = []
    rng = np.random.default_rng(1)
    for _ in range(120):
        args = (f32(rng.choice(grid_T)), f32(rng.choice(grid_p)), int(rng.choice(grid_k)),
                f32(rng.choice(grid_m)), f32(rng.choice(grid_rp)), int(rng.choice(grid_n)))
        s = ref.sampler()
        s.config(*args, seed=7)
        out.append({"in": list(args), "out": list(s.params())})
        s.close()
    return out


def workload_rows(ref, orc):
    plan = [("greedy_b1", [0], 2), ("full_b1", [0], 4),
            ("peaked_b256", list(range(12)) + [255], 2),
            ("studentt_b1024", list(range(12)) + [1023], 2),
            ("large_b4096", list(range(6)) + [4095], 2),
            ("nucleus_b8", [0, 1], 1), ("fullwindow_b8", [0, 1], 1),
            ("minp_only_b8", [0, 1], 2)]
    allw = dict(WORKLOADS)
    allw.update(STRESS)
    out = []
    for name, rows, picks in plan:
        w = allw[name]
        for r in rows:
            logits = orc.gen_logits(w.dist, w.sigma, w.boost, w.seed, r, 1, w.vocab)
            hist = (orc.gen_hist(w.seed, r, 1, w.hist_len, w.vocab, w.hist_pool)[0]
                    if w.hist_len else None)
            seed = int(orc.gen_row_seeds(w.seed, r, 1)[0])
            res = run_both(ref, orc, [logits[0]], w.params(), seed, hist, picks)
            res.update({"workload": name, "row": r, "picks": picks, "seed": "%016x" % seed,
                        "logits_crc": zlib.crc32(logits.tobytes()),
                        "hist_crc_in": zlib.crc32(hist.tobytes()) if hist is not None else 0})
            out.append(res)
            print(name, r, res["ids"], flush=True)
    return out


def _tiny(x, k):
    """x moved k float32 ulps toward -inf."""
    v = np.float32(x)
    for _ in range(k):
        v = np.nextafter(v, np.float32(-np.inf), dtype=np.float32)
    return float(v)


def edge_cases():
    inf, nan = float("inf"), float("nan")
    one_below = _tiny(5.0, 1)
    cases = [
        # name, logits, params (T, top_p, top_k, min_p, rp, last_n), seed, history, picks
        ("greedy_ties", [1, 3, 3, 2], (0, 1, 0, 0, 1, 0), 3, [], 1),
        ("greedy_nan_first", [nan, 3, 9, 2], (0, 1, 0, 0, 1, 0), 3, [], 1),
        ("greedy_nan_inside", [1, nan, 9, 9, nan], (0, 1, 0, 0, 1, 0), 3, [], 1),
        ("greedy_signed_zero", [-0.0, 0.0, -0.0], (0, 1, 0, 0, 1, 0), 3, [], 1),
        ("greedy_all_neg_inf", [-inf] * 6, (0, 1, 0, 0, 1, 0), 3, [], 1),
        ("greedy_all_nan", [nan] * 5, (0, 1, 0, 0, 1, 0), 3, [], 1),
        ("greedy_penalised_max", [2, 9, 8.5, -1], (0, 1, 0, 0, 1.1, 4), 3, [1], 2),
        ("greedy_negative_penalty", [-1, -2, -0.5, -3], (0, 1, 0, 0, 3.0, 4), 3, [2], 1),
        ("topk1_p_tie_vs_greedy", [one_below, 5.0, 1.0], (1, 1, 1, 0, 1, 0), 11, [], 1),
        ("greedy_p_tie_case", [one_below, 5.0, 1.0], (0, 1, 0, 0, 1, 0), 11, [], 1),
        ("window_edge", [10.0, -20.0, _tiny(-20.0, 1), 9.0, -20.0],
         (1, 1, 0, 0, 1, 0), 5, [], 4),
        ("window_edge_scaled", [10.0, 0.5, -4.0, 9.0, -4.0000005], (0.25, 1, 0, 0, 1, 0), 5, [], 3),
        ("all_equal", [0.5] * 37, (1, 1, 0, 0, 1, 0), 9, [], 6),
        ("all_equal_topk", [0.5] * 37, (1, 1, 5, 0, 1, 0), 9, [], 6),
        ("all_equal_minp1", [0.5] * 37, (1, 1, 0, 1.0, 1, 0), 9, [], 3),
        ("pos_inf", [1, inf, 3, inf, inf], (1, 1, 0, 0, 1, 0), 2, [], 2),
        ("pos_inf_topk2", [1, inf, 3, inf, inf], (1, 1, 2, 0, 1, 0), 2, [], 2),
        ("all_neg_inf_sampling", [-inf] * 7, (0.8, 0.9, 3, 0.05, 1, 0), 2, [], 2),
        ("neg_inf_and_nan", [-inf, nan, -inf, nan], (1, 1, 0, 0, 1, 0), 2, [], 2),
        ("nan_mixed_sampling", [1, nan, 2, nan, 0.5], (1, 0.9, 0, 0.05, 1, 0), 4, [], 3),
        ("penalty_signs", [3, -3, 0.0, -0.0, 2, 1], (1, 1, 0, 0, 2.0, 8), 21, [0, 1, 2, 3, 0, 1], 4),
        ("ring_wrap", [0.1 * i for i in range(23)], (0.5, 1, 0, 0, 1.5, 3), 99, [22, 21, 20, 19], 9),
        ("topp_tiny", [1, 2, 3, 4, 5], (1, 1e-6, 0, 0, 1, 0), 8, [], 3),
        ("topp_half", [1, 2, 3, 4, 5, 5], (1, 0.5, 0, 0, 1, 0), 8, [], 5),
        ("minp_one", [1, 2, 3, 4, 5, 5], (1, 1, 0, 1.0, 1, 0), 8, [], 5),
        ("topk_over_window", [1, 2, 3], (1, 1, 50, 0, 1, 0), 8, [], 3),
        ("low_temperature", [1, 2, 3, 2.999, 3], (1e-3, 1, 0, 0, 1, 0), 8, [], 3),
        ("high_temperature", [1, 2, 3, 2.999, 3], (100, 1, 0, 0, 1, 0), 8, [], 3),
        ("vocab_7", [0.3, 1.7, -2, 1.7, 0.9, 1.6, 1.65], (0.9, 0.95, 3, 0.05, 1.1, 4), 5, [1], 4),
        ("vocab_1", [2.5], (0.9, 0.9, 3, 0.05, 1.1, 4), 5, [0], 3),
    ]
    return cases


def fuzz_cases(n=120):
    rng = np.random.default_rng(20261201)
    out = []
    for c in range(n):
        V = int(rng.choice([1, 2, 3, 5, 8, 13, 31, 64, 100, 127, 128, 129, 257]))
        scale = float(rng.choice([0.1, 1.0, 3.0, 10.0, 50.0]))
        x = rng.normal(0, scale, V).astype(np.float32)
        if rng.random() < 0.5:      # coarse values make exact ties common
            x = np.round(x).astype(np.float32)
        if rng.random() < 0.3:
            sel = rng.random(V)
            x[sel < 0.03] = np.float32(-np.inf)
            x[(sel >= 0.03) & (sel < 0.06)] = np.float32(np.nan)
            x[(sel >= 0.06) & (sel < 0.09)] = np.float32(-0.0)
            if rng.random() < 0.2:
                x[sel > 0.98] = np.float32(np.inf)
        T = float(rng.choice([-1.0, 0.0, 1e-3, 0.1, 0.7, 1.0, 2.0, 100.0]))
        if not np.isfinite(x).any() and not np.isinf(x).any() and T > 0:
            x[0] = np.float32(1.0)       # an all-NaN row is unspecified when sampling
        params = (T, float(rng.choice([1.0, 0.5, 0.9, 0.99, 1e-6, 0.0, 1.5])),
                  int(rng.choice([0, -3, 1, 2, 5, 40, 1000])),
                  float(rng.choice([0.0, 0.01, 0.05, 0.5, 1.0, -1.0])),
                  float(rng.choice([1.0, 0.5, 1.1, 1.5, 3.0])),
                  int(rng.choice([0, 1, 3, 8, 64])))
        hist = rng.integers(0, V, int(rng.integers(0, 12))).tolist()
        seed = int(rng.integers(1, 2**63))
        picks = int(rng.integers(1, 5))
        out.append(("fuzz_%03d" % c, x, params, seed, hist, picks))
    return out


def main():
    ref, orc = RefSampler(), Oracle()
    data = {"about": __doc__.strip().splitlines()[0],
            "clamps": clamps(ref), "workload": workload_rows(ref, orc), "edge": [], "fuzz": []}
    for key, cases in (("edge", edge_cases()), ("fuzz", fuzz_cases())):
        for name, logits, params, seed, hist, picks in cases:
            x = np.asarray(logits, dtype=np.float32)
            params = tuple(f32(v) if i in (0, 1, 3, 4) else int(v) for i, v in enumerate(params))
            res = run_both(ref, orc, [x], params, seed, hist, picks)
            res.update({"name": name, "logits_bits": bits_of(x), "params": list(params),
                        "seed": "%016x" % seed, "history": [int(h) for h in hist],
                        "picks": picks})
            data[key].append(res)
    with open(OUT, "w") as f:
        json.dump(data, f, separators=(",", ":"))
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
