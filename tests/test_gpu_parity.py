"""GPU parity: the HIP sampler against the reference's golden vectors and against the CPU
restatement (oracle/) on the same logits.  Bar: bit-exact ids, generator states and
histories; a sampled id may differ only when the reference's uniform draw lies within
1e-6 of a CDF boundary of the kept prefix (counted, and expected to be 0 here).  Rows the
streaming kernel decides over a proven interval of the softmax denominator (PATH_CERT)
must hold the reference's denominator and normaliser inside the interval they report."""
import ctypes as C
import sys
import zlib

import numpy as np
import pytest

from helpers import expect, f32_from_bits

pytestmark = pytest.mark.gpu

BOUNDARY_TOL = 1e-6


@pytest.fixture(scope="module")
def qa():
    import quasar_amd
    quasar_amd.load()
    return quasar_amd


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def allw():
    from quasar_amd.workloads import STRESS, WORKLOADS
    return dict(WORKLOADS, **STRESS)


def batch_replay(qa, x, params, seed, history, picks):
    """One fixture case through the device batch API (B = 1, device logits)."""
    V = x.size
    b = qa.Batch(1, V, 64)
    buf = qa.DeviceBuffer.from_array(x)
    b.config(0, 1, *params, seeds=[seed])
    if history:
        b.set_history(0, np.asarray(history, dtype=np.int32))
    ids = [int(b.pick(buf.ptr, V, 1, V)[0]) for _ in range(picks)]
    rng, h = b.get_state(0)
    b.close()
    buf.free()
    h = h.astype(np.int32)
    return {"ids": ids, "rng_after": "%016x" % rng, "hist_len": int(len(h)),
            "hist_tail": [int(v) for v in h[-min(len(h), 8):]],
            "hist_crc": zlib.crc32(h.tobytes())}


def test_row_kernel_workgroups_per_cu(qa):
    """The row kernel's occupancy as designed: one 16-wavefront workgroup per CU (a row per
    CU fills the chip), two 8-wavefront ones (one row decides while the other streams)."""
    lib = qa.load()
    assert lib.qs_row_workgroups_per_cu(16) == 1
    assert lib.qs_row_workgroups_per_cu(8) == 2
    assert lib.qs_row_workgroups_per_cu(4) == qa._native.QS_EINVAL


def test_device_expf_equals_host_libm(qa, oracle):
    """The kernels' expf on gfx950 against the host C library's expf (sample.c:148) on a
    dense sample of the softmax window [-31, 0] plus special values."""
    lo = np.float32(-31.0).view(np.uint32)
    neg = np.arange(0, lo + 1, 7, dtype=np.uint32) | np.uint32(0x80000000)
    special = np.array([0.0, -0.0, 1.0, 50.0, 88.0, 88.72, 89.0, -87.0, -103.0, -103.5,
                        -104.0, -150.0, np.inf, -np.inf, np.nan], dtype=np.float32)
    x = np.concatenate([neg.view(np.float32), special]).astype(np.float32)
    dx = qa.DeviceBuffer.from_array(x)
    dy = qa.DeviceBuffer(x.nbytes)
    qa.check(qa.load().qs_expf_device(dx.ptr, dy.ptr, x.size), "qs_expf_device")
    y = dy.download(np.float32, x.size)
    ref = oracle.libm_expf(x)
    same = (y.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(y) & np.isnan(ref))
    log(f"expf checked {x.size} inputs, mismatches {int((~same).sum())}")
    assert same.all(), x[~same][:10]


def test_device_generator_bit_identical(qa, oracle, golden):
    seen = set()
    W = allw()
    for c in golden["workload"]:
        key = (c["workload"], c["row"])
        if key in seen:
            continue
        seen.add(key)
        w = W[c["workload"]]
        buf = qa.DeviceBuffer(4 * w.vocab)
        qa.gen_logits_device(buf, w.vocab, c["row"], 1, w.vocab, w.dist, w.sigma, w.boost,
                             w.seed)
        got = buf.download(np.float32, w.vocab)
        buf.free()
        assert zlib.crc32(got.tobytes()) == c["logits_crc"], key
    host = oracle.gen_logits(2, 2.0, 0.0, 99, 5, 2, 4099)
    buf = qa.DeviceBuffer(host.nbytes)
    qa.gen_logits_device(buf, 4099, 5, 2, 4099, 2, 2.0, 0.0, 99)
    assert (buf.download(np.float32, host.size).view(np.uint32)
            == host.reshape(-1).view(np.uint32)).all()


@pytest.mark.parametrize("section", ["edge", "fuzz"])
def test_golden_small_rows_batch_api(qa, golden, section):
    for c in golden[section]:
        x = f32_from_bits(c["logits_bits"])
        got = batch_replay(qa, x, c["params"], int(c["seed"], 16), c["history"], c["picks"])
        assert got == expect(c), c["name"]
    log(f"{section}: {len(golden[section])} cases bit-exact")


def test_golden_small_rows_sample_h_api(qa, golden):
    """The five-function API (host logits) on every case without a preloaded history."""
    n = 0
    for c in golden["edge"] + golden["fuzz"]:
        if c["history"]:
            continue
        x = f32_from_bits(c["logits_bits"])
        s = qa.Sampler()
        s.config(*c["params"], seed=int(c["seed"], 16))
        ids = [int(s.pick(x)) for _ in range(c["picks"])]
        s.close()
        assert ids == c["ids"], c["name"]
        n += 1
    log(f"sample.h API: {n} cases bit-exact")


def test_golden_workload_rows(qa, oracle, golden):
    W = allw()
    for c in golden["workload"]:
        w = W[c["workload"]]
        V = w.vocab
        buf = qa.DeviceBuffer(4 * V)
        qa.gen_logits_device(buf, V, c["row"], 1, V, w.dist, w.sigma, w.boost, w.seed)
        b = qa.Batch(1, V, max(1, w.repeat_last_n))
        b.config(0, 1, *w.params(), seeds=[int(c["seed"], 16)])
        if w.hist_len:
            b.set_history(0, oracle.gen_hist(w.seed, c["row"], 1, w.hist_len, V, w.hist_pool))
        ids, diags = [], []
        for _ in range(c["picks"]):
            i, d = b.pick(buf.ptr, V, 1, V, diag=True)
            ids.append(int(i[0]))
            diags.append(d[0].path)
        rng, h = b.get_state(0)
        b.close()
        buf.free()
        h = h.astype(np.int32)
        got = {"ids": ids, "rng_after": "%016x" % rng, "hist_len": int(len(h)),
               "hist_tail": [int(v) for v in h[-min(len(h), 8):]],
               "hist_crc": zlib.crc32(h.tobytes())}
        assert got == expect(c), (c["workload"], c["row"], diags)
    log(f"workload rows: {len(golden['workload'])} bit-exact")


def run_batch_vs_oracle(qa, oracle, w, rows_checked, picks=1):
    """Whole batch on the GPU, `rows_checked` rows replayed on the CPU restatement."""
    B, V = w.batch, w.vocab
    buf = qa.DeviceBuffer(4 * B * V)
    qa.gen_logits_device(buf, V, 0, B, V, w.dist, w.sigma, w.boost, w.seed)
    seeds = oracle.gen_row_seeds(w.seed, 0, B)
    b = qa.Batch(B, V, max(1, w.repeat_last_n))
    b.config(0, B, *w.params(), seeds=seeds)
    hist = oracle.gen_hist(w.seed, 0, B, w.hist_len, V, w.hist_pool) if w.hist_len else None
    if hist is not None:
        b.set_history(0, hist)
    gpu = []
    for _ in range(picks):
        ids, diag = b.pick(buf.ptr, V, B, V, diag=True)
        gpu.append((ids, diag))
    stats = {"rows": 0, "id_mismatch": 0, "tolerated": 0, "inv_mismatch": 0,
             "keep_mismatch": 0, "outside_interval": 0, "paths": {}, "inv_floats": 0}
    for r in rows_checked:
        x = buf.download(np.float32, V, offset=4 * r * V)
        s = oracle.sampler()
        s.config(*w.params(), seed=int(seeds[r]))
        if hist is not None:
            s.set_history(hist[r])
        for k in range(picks):
            want, od = s.pick_diag(x)
            ids, diag = gpu[k]
            d = diag[r]
            stats["rows"] += 1
            stats["paths"][d.path] = stats["paths"].get(d.path, 0) + 1
            if not od["greedy"]:
                inv = np.float32(od["inv"])
                if d.path == qa.PATH_CERT:
                    lo, hi = np.float32(d.inv), np.float32(d.inv_hi)
                    if not (lo <= inv <= hi and d.sum <= od["sum"] <= d.sum_hi):
                        stats["outside_interval"] += 1
                        log(f"row {r} pick {k}: sum {od['sum']!r} not in [{d.sum!r}, "
                            f"{d.sum_hi!r}] or inv {inv!r} not in [{lo!r}, {hi!r}]")
                    stats["inv_floats"] = max(stats["inv_floats"], int(hi.view(np.int32))
                                              - int(lo.view(np.int32)) + 1)
                elif np.float32(d.inv).view(np.uint32) != inv.view(np.uint32):
                    stats["inv_mismatch"] += 1
                if d.keep != od["keep"]:
                    stats["keep_mismatch"] += 1
            if int(ids[r]) != want:
                if od["bdist"] < BOUNDARY_TOL:
                    stats["tolerated"] += 1
                else:
                    stats["id_mismatch"] += 1
                    log(f"row {r} pick {k}: gpu {int(ids[r])} cpu {want} path {d.path} "
                        f"keep {d.keep}/{od['keep']} inv {d.inv!r}/{od['inv']!r}")
        if hist is not None or w.repeat_last_n:
            rng, h = b.get_state(r)
            assert rng == s.rng and (h == s.history()).all(), r
    b.close()
    buf.free()
    return stats


@pytest.mark.parametrize("name,rows,picks", [
    ("greedy_b1", None, 3),
    ("full_b1", None, 4),
    ("peaked_b256", None, 2),
    ("studentt_b1024", None, 1),
    ("nucleus_b8", None, 1),
    ("fullwindow_b8", None, 1),
    ("minp_only_b8", None, 2),
    ("peaked_tail_b64", None, 2),
])
def test_workload_batch_vs_cpu(qa, oracle, name, rows, picks):
    w = allw()[name]
    rows = list(range(w.batch)) if rows is None else rows
    st = run_batch_vs_oracle(qa, oracle, w, rows, picks)
    log(f"{name}: {st}")
    assert st["id_mismatch"] == 0
    assert st["outside_interval"] == 0
    assert st["inv_mismatch"] == 0 and st["keep_mismatch"] == 0


@pytest.mark.parametrize("name", ["large_b4096", "studentt_b1024", "peaked_b256"])
def test_workload_all_rows_threaded(qa, oracle, name):
    """One pick of every row of the large batches against the restatement run on host
    threads (orc_pick_rows_diag): ids (a mismatch only on a draw within 1e-6 of a CDF
    boundary, counted), the reference's denominator and normaliser inside the GPU's proven
    interval (certified rows) or equal (exact rows), the kept prefix, and every row's
    generator state and history afterwards."""
    from pyoracle import Params, parity_report
    w = allw()[name]
    B, V = w.batch, w.vocab
    buf = qa.DeviceBuffer(4 * B * V)
    qa.gen_logits_device(buf, V, 0, B, V, w.dist, w.sigma, w.boost, w.seed)
    seeds = np.asarray(oracle.gen_row_seeds(w.seed, 0, B), dtype=np.uint64)
    hist = oracle.gen_hist(w.seed, 0, B, w.hist_len, V, w.hist_pool) if w.hist_len else None
    b = qa.Batch(B, V, max(1, w.repeat_last_n))
    b.config(0, B, *w.params(), seeds=seeds)
    if hist is not None:
        b.set_history(0, hist)
    ids, diag = b.pick(buf.ptr, V, B, V, diag=True)
    x = buf.download(np.float32, B * V).reshape(B, V)
    p = Params(w.temperature, w.top_p, w.min_p, w.repeat_penalty, w.top_k, w.repeat_last_n)
    oids, od, _ = oracle.pick_rows_diag(p, x, B, V, hist, seeds, 16)
    rep = parity_report(ids, diag, oids, od)
    outside = sum(1 for r in range(B) if diag[r].path == qa.PATH_CERT and od["greedy"][r] == 0
                  and not (diag[r].sum <= od["sum"][r] <= diag[r].sum_hi))
    log(f"{name} all rows: {rep}, sums outside their interval {outside}")
    assert rep["rows"] == B and rep["unexplained"] == 0
    assert rep["inv_outside"] == 0 and rep["keep_mismatches"] == 0 and outside == 0
    cap = w.repeat_last_n
    for r in range(B):
        rng, h = b.get_state(r)
        assert rng == int(od["rng_after"][r]), r
        if cap:
            want = (list(hist[r]) if hist is not None else []) + [int(oids[r])]
            assert list(h) == want[-cap:], r
    b.close()
    buf.free()


def test_mixed_rows_one_batch(qa, oracle):
    """Every row of one batch with its own parameters (greedy, sampled, penalised, cuts
    on and off), coarse logits with many exact ties, three consecutive picks."""
    rng = np.random.default_rng(11)
    B, V = 48, 3001
    x = (np.round(rng.normal(0, 2.5, (B, V)) * 2) / 2).astype(np.float32)
    x[3, :] = np.float32(0.25)                      # all equal
    x[5, ::7] = np.float32(-np.inf)
    x[6, 17] = np.float32(np.nan)
    buf = qa.DeviceBuffer.from_array(x)
    b = qa.Batch(B, V, 64)
    cfgs, hists = [], []
    for r in range(B):
        cfg = (float(rng.choice([0.0, 0.3, 0.7, 1.0, 1.7])), float(rng.choice([1.0, 0.5, 0.95])),
               int(rng.choice([0, 1, 3, 40, 700])), float(rng.choice([0.0, 0.05, 0.3])),
               float(rng.choice([1.0, 1.3])), int(rng.choice([0, 8, 64])))
        seed = int(rng.integers(1, 2**62))
        b.config(r, 1, *cfg, seeds=[seed])
        h = rng.integers(0, V, 16).astype(np.int32)
        b.set_history(r, h)
        cfgs.append((cfg, seed))
        hists.append(h)
    outs = [b.pick(buf.ptr, V, B, V, diag=True) for _ in range(3)]
    for r in range(B):
        s = oracle.sampler()
        s.config(*cfgs[r][0], seed=cfgs[r][1])
        s.set_history(hists[r])
        for k in range(3):
            want = s.pick(x[r])
            assert int(outs[k][0][r]) == want, (r, k, cfgs[r], outs[k][1][r].path)
        rs, h = b.get_state(r)
        assert rs == s.rng and (h == s.history()).all()
    # the whole-window path with a top-k below the window (its top-k select before the
    # sort) is among the rows checked: ties straddle the preselection boundary
    full_topk = [(r, k) for r in range(B) for k in range(3)
                 if outs[k][1][r].path == qa.PATH_FULL and 0 < cfgs[r][0][2] < outs[k][1][r].n_window]
    log(f"whole-window rows with top-k below the window: {full_topk}")
    assert full_topk
    b.close()


def test_unaligned_rows_take_the_scalar_path(qa, oracle):
    """Row stride not a multiple of 4 floats and a base offset of one float: the scalar
    loads must give the same ids as the CPU."""
    w = allw()["full_b1"]
    V, B = 10007, 6
    stride = V + 3
    rng = np.random.default_rng(5)
    x = np.zeros((B, stride), dtype=np.float32)
    x[:, :V] = rng.normal(0, 2, (B, V)).astype(np.float32)
    buf = qa.DeviceBuffer(4 * (B * stride + 1))
    buf.upload(x, offset=4)
    b = qa.Batch(B, V, 64)
    b.config(0, B, *w.params(), seeds=np.arange(1, B + 1))
    ids = b.pick(buf.ptr + 4, stride, B, V)
    for r in range(B):
        s = oracle.sampler()
        s.config(*w.params(), seed=r + 1)
        assert int(ids[r]) == s.pick(x[r, :V]), r
    b.close()


def _full_width_rows(oracle, name, n):
    from quasar_amd.workloads import WORKLOADS
    w = WORKLOADS[name]
    return w, oracle.gen_logits(w.dist, w.sigma, w.boost, w.seed, 0, n, w.vocab)


def test_sample_h_default_sampler(qa, oracle):
    """A sampler that was never configured (sample.c:31-39: greedy, no history, the default
    generator state) picking full-width rows through the five-function API."""
    _, x = _full_width_rows(oracle, "greedy_b1", 3)
    g, o = qa.Sampler(), oracle.sampler()
    for r in (0, 1, 2, 1):
        assert g.pick(x[r]) == o.pick(x[r]), r
    rng, hist = g.get_state()
    assert rng == o.rng == 0x9E3779B97F4A7C15 and len(hist) == 0
    g.close()


@pytest.mark.parametrize("name", ["greedy_b1", "full_b1"])
def test_sample_h_full_width(qa, oracle, name):
    """The single-row workloads (V = 151,936) through quasar_sampler_pick with host logits,
    as the reference's server and generate loops call it: ids and final state."""
    w, x = _full_width_rows(oracle, name, 4)
    g, o = qa.Sampler(), oracle.sampler()
    for s in (g, o):
        s.config(*w.params(), seed=w.seed)
    ids = []
    for r in (0, 1, 2, 3, 0):
        i = g.pick(x[r])
        assert i == o.pick(x[r]), (name, r)
        ids.append(i)
    rng, hist = g.get_state()
    assert rng == o.rng and list(hist) == list(o.history()), name
    log(f"{name} via sample.h: ids {ids}")
    g.close()


def test_sample_h_device_unavailable_then_back(qa, oracle):
    """Picks the device cannot take (injected) answer with the raw argmax and are recorded
    (sample.c:113-116); the next picks run on the device again with that history, also when
    the device row existed before the failure."""
    rng = np.random.default_rng(21)
    xs = [rng.normal(0, 1.5, 3000).astype(np.float32) for _ in range(4)]
    g, o = qa.Sampler(), oracle.sampler()
    for s in (g, o):
        s.config(0.9, 0.95, 30, 0.02, 1.5, 6, 31)
    plan = [(True, 0), (True, 1), (False, 2), (False, 0), (True, 3), (False, 1), (False, 3)]
    for fail, r in plan:
        if fail:
            qa.fail_picks(1)
            o.fail_allocs(1)
        try:
            assert g.pick(xs[r]) == o.pick(xs[r]), (fail, r)
        finally:
            qa.fail_picks(0)
            o.fail_allocs(0)
    got_rng, hist = g.get_state()
    assert got_rng == o.rng and list(hist) == list(o.history())
    g.close()


def test_bounded_wait_give_up_keeps_state(qa, oracle):
    """A row whose whole-window scratch slot wait gives up (forced from the host with a
    spin limit of 0) returns -3, keeps its generator state and history, and makes
    qs_batch_synchronize report QS_EAGAIN; picked again, it gets the reference's id."""
    from quasar_amd.workloads import STRESS
    w = STRESS["fullwindow_b8"]
    V = w.vocab
    x = oracle.gen_logits(w.dist, w.sigma, w.boost, w.seed, 0, 2, V)
    buf = qa.DeviceBuffer.from_array(x)
    b = qa.Batch(1, V, 8)
    seed = 0x5EED
    b.config(0, 1, *w.params(), seeds=[seed])
    b.set_history(0, np.array([3, 5, 7], np.int32))
    before = b.get_state(0)
    b.set_spin_limit(0)
    b.pick_async(buf.ptr, V, 1, V)
    with pytest.raises(qa.QsError) as e:
        b.synchronize()
    assert e.value.rc == qa.QS_EAGAIN
    assert int(b._out.download(np.int32, 1)[0]) == -3
    after = b.get_state(0)
    assert after[0] == before[0] and list(after[1]) == list(before[1])
    b.set_spin_limit(1 << 20)
    got = int(b.pick(buf.ptr, V, 1, V)[0])
    o = oracle.sampler()
    o.config(*w.params(), seed=seed)
    o.set_history([3, 5, 7])
    assert got == o.pick(x[0])
    rng, h = b.get_state(0)
    assert rng == o.rng and list(h) == list(o.history())
    b.close()
    buf.free()


def test_bounded_wait_give_up_multi_row_retry(qa, oracle):
    """In a batch of 4 rows whose whole-window slot waits all give up (spin limit 0), every
    whole-window row returns -3 with its state kept; qs_batch_pick_rows then picks each
    such row alone and it gets the reference's id, while rows a retry does not name keep
    the state their first pick left."""
    from quasar_amd.workloads import STRESS
    w = STRESS["fullwindow_b8"]
    V, B = w.vocab, 4
    x = oracle.gen_logits(w.dist, w.sigma, w.boost, w.seed, 0, B, V)
    buf = qa.DeviceBuffer.from_array(x)
    b = qa.Batch(B, V, 8)
    seeds = [0x5EED + r for r in range(B)]
    for r in range(B):
        if r == 1:
            b.config(r, 1, 0.0, 1.0, 0, 0.0, 1.0, 8, seeds=[seeds[r]])   # greedy: no slot
        else:
            b.config(r, 1, *w.params(), seeds=[seeds[r]])
        b.set_history(r, np.array([3 + r, 5, 7], np.int32))
    before = [b.get_state(r) for r in range(B)]
    b.set_spin_limit(0)
    b.pick_async(buf.ptr, V, B, V)
    with pytest.raises(qa.QsError) as e:
        b.synchronize()
    assert e.value.rc == qa.QS_EAGAIN
    first = b._out.download(np.int32, B)
    failed = [r for r in range(B) if first[r] == -3]
    assert 1 not in failed and failed, first
    for r in failed:
        after = b.get_state(r)
        assert after[0] == before[r][0] and list(after[1]) == list(before[r][1]), r
    kept = {r: b.get_state(r) for r in range(B) if r not in failed}
    b.set_spin_limit(1 << 20)
    for r in failed:
        got = int(b.pick_rows(r, buf.ptr + 4 * V * r, V, 1, V)[0])
        o = oracle.sampler()
        o.config(*w.params(), seed=seeds[r])
        o.set_history([3 + r, 5, 7])
        assert got == o.pick(x[r]), r
        rng, h = b.get_state(r)
        assert rng == o.rng and list(h) == list(o.history()), r
    for r, st in kept.items():
        now = b.get_state(r)
        assert now[0] == st[0] and list(now[1]) == list(st[1]), r
    b.close()
    buf.free()


@pytest.mark.parametrize("mode", [0, 1, 2, 3])
@pytest.mark.parametrize("name", ["fullwindow_b8", "nucleus_b8", "minp_only_b8"])
def test_exact_path_sum_in_id_order(qa, oracle, mode, name):
    """Rows that leave the certified decision, with the recount's in-id-order sum forced
    (qs_batch_set_sum_in_order): each such row's denominator equals the restatement's
    (sample.c:147-149, ids ascending) bit for bit, and so do its id and state, under every
    mode (AUTO, split, streaming, row)."""
    from quasar_amd.workloads import STRESS
    w = STRESS[name]
    B, V = w.batch, w.vocab
    x = oracle.gen_logits(w.dist, w.sigma, w.boost, w.seed, 0, B, V)
    buf = qa.DeviceBuffer.from_array(x)
    b = qa.Batch(B, V, max(1, w.repeat_last_n))
    b.set_mode(mode)
    seeds = qa.gen_row_seeds(w.seed, 0, B)
    b.config(0, B, *w.params(), seeds=seeds)
    hist = qa.gen_history(w.seed, 0, B, w.hist_len, V, w.hist_pool) if w.hist_len else None
    if hist is not None:
        b.set_history(0, hist)
    b.set_sum_in_order(1)
    ids, diag = b.pick(buf.ptr, V, B, V, diag=True)
    exact = 0
    for r in range(B):
        s = oracle.sampler()
        s.config(*w.params(), seed=int(seeds[r]))
        if hist is not None:
            s.set_history(hist[r])
        want, od = s.pick_diag(x[r])
        assert int(ids[r]) == want, (r, int(ids[r]), want)
        if diag[r].path in (qa.PATH_FAST, qa.PATH_FULL):
            exact += 1
            assert diag[r].sum == od["sum"], (r, diag[r].sum, od["sum"])
            assert np.float32(diag[r].inv) == np.float32(od["inv"]), r
    log(f"{name} mode {mode}: {exact} of {B} rows on the exact path, sums equal")
    assert exact > 0
    b.close()
    buf.free()


def test_sample_h_state_rules(qa, oracle):
    """Config/reset/pick sequences through the five-function API: the ring keeps its
    capacity when repeat_last_n is 0 (sample.c:61-66), reset keeps the generator,
    a larger vocabulary later keeps state."""
    rng = np.random.default_rng(8)
    rows = [rng.normal(0, 1.5, 700).astype(np.float32) for _ in range(3)]
    rows.append(rng.normal(0, 1.5, 2100).astype(np.float32))
    g, o = qa.Sampler(), oracle.sampler()
    script = [("config", (0.8, 0.9, 20, 0.02, 1.4, 6, 77)), ("pick", 0), ("pick", 1),
              ("config", (0.8, 0.9, 20, 0.02, 1.4, 0, 78)), ("pick", 2), ("pick", 0),
              ("reset", None), ("pick", 1), ("pick", 3), ("pick", 3),
              ("config", (0.0, 1.0, 0, 0.0, 2.0, 3, 5)), ("pick", 3), ("pick", 3), ("pick", 0),
              ("config", (1.1, 1.0, 0, 0.0, 1.0, 9, 6)), ("pick", 2), ("pick", 3)]
    for op, arg in script:
        for s in (g, o):
            if op == "config":
                s.config(*arg[:6], seed=arg[6])
            elif op == "reset":
                s.reset()
        if op == "pick":
            assert g.pick(rows[arg]) == o.pick(rows[arg]), (op, arg)


def _run_mode(qa, mode, w, B, picks, logits_buf, seeds, hist, per_row=None):
    """Run `picks` consecutive picks of a B-row batch in one kernel mode; return ids,
    diagnostics paths and the final states of all rows."""
    V = w.vocab
    b = qa.Batch(B, V, max(1, w.repeat_last_n))
    b.set_mode(mode)
    if per_row is None:
        b.config(0, B, *w.params(), seeds=seeds)
    else:
        for r, (cfg, seed) in enumerate(per_row):
            b.config(r, 1, *cfg, seeds=[seed])
    if hist is not None:
        b.set_history(0, hist)
    ids, paths = [], []
    for _ in range(picks):
        i, d = b.pick(logits_buf.ptr, V, B, V, diag=True)
        ids.append(i.copy())
        paths.append([x.path for x in d])
    states = [b.get_state(r) for r in range(B)]
    b.close()
    return ids, paths, states


MODES = {"stream": 2, "row": 3}


@pytest.mark.parametrize("mode", sorted(MODES))
@pytest.mark.parametrize("name,B,picks", [("peaked_b256", 256, 3), ("large_b4096", 512, 2),
                                          ("studentt_b1024", 1024, 1), ("full_b1", 1, 4),
                                          ("greedy_b1", 1, 3), ("nucleus_b8", 8, 2)])
def test_mode_equals_split(qa, oracle, mode, name, B, picks):
    """The streaming kernel returns the same ids, generator states and histories as the
    split-row kernels (exact softmax denominators), pick after pick; the first pick is
    also checked on the CPU."""
    w = allw()[name]
    V = w.vocab
    buf = qa.DeviceBuffer(4 * B * V)
    qa.gen_logits_device(buf, V, 0, B, V, w.dist, w.sigma, w.boost, w.seed)
    seeds = oracle.gen_row_seeds(w.seed, 0, B)
    hist = oracle.gen_hist(w.seed, 0, B, w.hist_len, V, w.hist_pool) if w.hist_len else None
    sp_ids, sp_paths, sp_states = _run_mode(qa, qa.MODE_SPLIT, w, B, picks, buf, seeds, hist)
    pp_ids, pp_paths, pp_states = _run_mode(qa, MODES[mode], w, B, picks, buf, seeds, hist)
    for k in range(picks):
        assert (sp_ids[k] == pp_ids[k]).all(), (k, np.nonzero(sp_ids[k] != pp_ids[k])[0][:10])
    for r in range(B):
        assert sp_states[r][0] == pp_states[r][0] and (sp_states[r][1] == pp_states[r][1]).all()
    for r in sorted(set(list(range(min(B, 8))) + [B - 1])):
        x = buf.download(np.float32, V, offset=4 * r * V)
        s = oracle.sampler()
        s.config(*w.params(), seed=int(seeds[r]))
        if hist is not None:
            s.set_history(hist[r])
        assert s.pick(x) == int(pp_ids[0][r]), r
    log(f"{name} B={B}: {mode} == split over {picks} picks; paths {set(sum(pp_paths, []))}")
    buf.free()


@pytest.mark.parametrize("mode", sorted(MODES))
def test_mode_mixed_rows(qa, oracle, mode):
    """A 64-row batch at the full vocabulary where each row has its own parameters
    (greedy rows, top-k off, penalties, degenerate rows: ties, +inf, all -inf, NaN runs,
    a single NaN, signalling NaNs, a NaN in the last part's tail, a signed-zero max, one
    finite logit), through the streaming kernel, against the CPU restatement row by row
    over three picks."""
    rng = np.random.default_rng(21)
    B, V = 64, 151936
    x = rng.normal(0, 2.0, (B, V)).astype(np.float32)
    x[5, :] = np.float32(0.5)                      # all equal: ties everywhere
    x[6, 1000] = np.float32(np.inf)                # +inf max: degenerate window
    x[7, :] = np.float32(-np.inf)                  # all -inf
    x[8, ::3] = np.float32(np.nan)
    x[9, 77777] = np.float32(np.nan)               # one NaN
    snan = np.array([0x7F800001, 0xFF800001, 0x7FA00000], dtype=np.uint32).view(np.float32)
    x[10, [int(np.argmax(x[10])), 3, 151935]] = snan   # signalling NaNs, one at the max
    x[11, V - 3] = np.float32(np.nan)              # NaN in the last part's tail
    x[11, V - 1] = np.float32(9.0)
    x[12, :] = -np.abs(x[12, :]) - np.float32(1.0)  # the max is a signed zero
    x[12, 100] = np.float32(-0.0)
    x[12, 200] = np.float32(0.0)
    x[13, :] = np.float32(-np.inf)                 # one finite logit
    x[13, 4242] = np.float32(-3.0)
    buf = qa.DeviceBuffer.from_array(x)
    per_row, hists = [], []
    for r in range(B):
        cfg = (float(rng.choice([0.0, 0.5, 0.8, 1.0, 1.5])),
               float(rng.choice([1.0, 0.9, 0.5])), int(rng.choice([0, 1, 20, 40, 300])),
               float(rng.choice([0.0, 0.05, 0.2])), float(rng.choice([1.0, 1.2])),
               int(rng.choice([0, 16, 64])))
        per_row.append((cfg, int(rng.integers(1, 2**62))))
        hists.append(rng.integers(0, V, 32).astype(np.int32))
    b = qa.Batch(B, V, 64)
    b.set_mode(MODES[mode])
    for r, (cfg, seed) in enumerate(per_row):
        b.config(r, 1, *cfg, seeds=[seed])
        b.set_history(r, hists[r])
    outs = [b.pick(buf.ptr, V, B, V, diag=True) for _ in range(3)]
    for r in range(B):
        s = oracle.sampler()
        s.config(*per_row[r][0], seed=per_row[r][1])
        s.set_history(hists[r])
        for k in range(3):
            want = s.pick(x[r])
            assert int(outs[k][0][r]) == want, (r, k, per_row[r][0], outs[k][1][r].path)
        rs, h = b.get_state(r)
        assert rs == s.rng and (h == s.history()).all(), r
    b.close()
    buf.free()


def test_stream_all_greedy_rows_decided_by_last_part(qa, oracle):
    """A batch whose rows are all greedy takes the streaming kernel alone: each row's last
    part to finish reads the row's best (key, ~id) and records it (sample.c:118-134).  16
    rows at the full vocabulary (15 parts each): ties within and across parts, +inf, all
    -inf, NaNs (one at id 0), a signed-zero max, one finite logit, a maximum in the last
    part's tail, and rows whose largest logits are penalised history ids; against the CPU
    restatement over four picks (the per-row counters are reset between picks), then the
    same rows picked again in a mixed batch (the decision kernel's greedy path)."""
    rng = np.random.default_rng(33)
    B, V = 16, 151936
    x = rng.normal(0, 2.0, (B, V)).astype(np.float32)
    x[1, :] = np.float32(0.25)                     # all equal: id 0
    x[2, [20000, 90000, 140000]] = np.float32(30.0)  # equal maxima in three parts
    x[3, 1000] = np.float32(np.inf)
    x[4, :] = np.float32(-np.inf)                  # all -inf: id 0
    x[5, ::7] = np.float32(np.nan)
    x[6, 0] = np.float32(np.nan)                   # NaN at id 0: id 0
    x[7, :] = -np.abs(x[7, :]) - np.float32(1.0)   # the max is a signed zero
    x[7, 300] = np.float32(-0.0)
    x[7, 600] = np.float32(0.0)
    x[8, :] = np.float32(-np.inf)                  # one finite logit
    x[8, 123456] = np.float32(-7.0)
    x[9, V - 2] = np.float32(40.0)                 # in the last part's tail
    x[10, 5000] = np.float32(12.0)                 # penalised below the runner-up
    x[10, 6000] = np.float32(10.0)
    x[11, 7000] = np.float32(-0.5)                 # a negative max, penalised by product
    x[11, :7000] = np.minimum(x[11, :7000], np.float32(-0.6))
    x[11, 7001:] = np.minimum(x[11, 7001:], np.float32(-0.6))
    buf = qa.DeviceBuffer.from_array(x)
    per_row, hists = [], []
    for r in range(B):
        rp = 1.0 if r < 10 else 1.3
        cfg = (0.0, 0.9, 40, 0.05, rp, 64)
        h = rng.integers(0, V, 16).astype(np.int32)
        if r == 10:
            h[3] = 5000
        if r == 11:
            h[5] = 7000
        per_row.append((cfg, int(rng.integers(1, 2**62))))
        hists.append(h)
    b = qa.Batch(B, V, 64)
    for r, (cfg, seed) in enumerate(per_row):
        b.config(r, 1, *cfg, seeds=[seed])
        b.set_history(r, hists[r])
    assert b.resolve_mode(buf.ptr, V, B, V) == qa.MODE_STREAM
    outs = [b.pick(buf.ptr, V, B, V, diag=True) for _ in range(4)]
    sams = []
    for r in range(B):
        s = oracle.sampler()
        s.config(*per_row[r][0], seed=per_row[r][1])
        s.set_history(hists[r])
        for k in range(4):
            want = s.pick(x[r])
            assert int(outs[k][0][r]) == want, (r, k, want, int(outs[k][0][r]))
            assert outs[k][1][r].path == qa.PATH_GREEDY, (r, k)
        rs, h = b.get_state(r)
        assert rs == s.rng and (h == s.history()).all(), r
        sams.append(s)
    # a sampling row joins: the greedy rows go through the decision kernel instead
    b.config(B - 1, 1, 0.8, 0.95, 40, 0.05, 1.0, 64, seeds=[99])
    sams[B - 1] = oracle.sampler()
    sams[B - 1].config(0.8, 0.95, 40, 0.05, 1.0, 64, seed=99)
    ids = b.pick(buf.ptr, V, B, V)
    for r in range(B):
        assert int(ids[r]) == sams[r].pick(x[r]), r
    b.close()
    buf.free()


@pytest.mark.parametrize("mode", ["stream", "row", "greedy_stream"])
def test_random_row_configs(qa, oracle, mode):
    """24 rows at the full vocabulary with random per-row settings (temperature 0 to 1.5,
    top-k off to 300, top-p, min-p, penalties over random histories with repeats), logits
    from three shapes (normal, peaked, heavy-tailed), through the streaming kernel (its
    workgroup decision of rows of 15 parts), the row kernel, or, with every row greedy, the
    streaming kernel alone; ids and final states against the CPU restatement over two
    picks."""
    rng = np.random.default_rng({"stream": 51, "row": 52, "greedy_stream": 53}[mode])
    B, V = 24, 151936
    x = rng.normal(0, 2.0, (B, V)).astype(np.float32)
    for r in range(0, B, 3):
        x[r, int(rng.integers(0, V))] += np.float32(rng.uniform(5, 15))
    for r in range(1, B, 3):
        x[r] = (rng.standard_t(3, V) * 2.0).astype(np.float32)
    buf = qa.DeviceBuffer.from_array(x)
    per_row, hists = [], []
    for r in range(B):
        t = 0.0 if mode == "greedy_stream" else float(rng.choice([0.0, 0.3, 0.7, 1.0, 1.5]))
        cfg = (t, float(rng.choice([1.0, 0.95, 0.9, 0.5])),
               int(rng.choice([0, 1, 5, 40, 64, 100, 300])),
               float(rng.choice([0.0, 0.02, 0.1])), float(rng.choice([1.0, 1.1, 1.5])),
               int(rng.choice([0, 32, 64])))
        per_row.append((cfg, int(rng.integers(1, 2**62))))
        hists.append(rng.integers(0, 4000, 48).astype(np.int32))
    b = qa.Batch(B, V, 64)
    b.set_mode(qa.MODE_ROW if mode == "row" else qa.MODE_STREAM)
    for r, (cfg, seed) in enumerate(per_row):
        b.config(r, 1, *cfg, seeds=[seed])
        b.set_history(r, hists[r])
    outs = [b.pick(buf.ptr, V, B, V) for _ in range(2)]
    for r in range(B):
        s = oracle.sampler()
        s.config(*per_row[r][0], seed=per_row[r][1])
        s.set_history(hists[r])
        for k in range(2):
            assert int(outs[k][r]) == s.pick(x[r]), (mode, r, k, per_row[r][0])
        rs, h = b.get_state(r)
        assert rs == s.rng and (h == s.history()).all(), (mode, r)
    b.close()
    buf.free()


@pytest.mark.parametrize("mode", ["auto", "split"])
def test_history_layouts(qa, oracle, mode):
    """Histories in unusual shapes: runs of consecutive ids (several in one thread's
    registers), duplicates, ids at part and slice edges and the row's argmax itself,
    unaligned rows (scalar loads, the split path) and short odd vocabularies."""
    rng = np.random.default_rng(33)
    for V, stride, aligned in [(151936, 151936, True), (151933, 151937, False),
                               (1000, 1001, False), (4099, 4100, True)]:
        B = 12
        x = np.full((B, stride), np.float32(np.nan), dtype=np.float32)
        x[:, :V] = rng.normal(0, 2.0, (B, V)).astype(np.float32)
        hists = []
        for r in range(B):
            top = int(np.argmax(x[r, :V]))
            kind = r % 4
            if kind == 0:
                h = np.arange(min(V, 300), dtype=np.int64) + rng.integers(0, max(1, V - 300))
            elif kind == 1:
                h = rng.integers(0, 64, 200)
            elif kind == 2:
                edges = ([i for i in range(0, V, 64)][:150] + [i for i in range(0, V, 10240)]
                         + [i - 1 for i in range(10240, V, 10240)])
                h = np.array(edges + [V - 1, top], dtype=np.int64)
            else:
                h = np.array([top] * 5 + list(rng.integers(0, V, 100)), dtype=np.int64)
            hists.append((h % V).astype(np.int32))
        flat = x.reshape(-1)
        if not aligned:
            flat = np.concatenate([np.zeros(1, np.float32), flat])
        buf = qa.DeviceBuffer.from_array(flat)
        base = buf.ptr + (0 if aligned else 4)
        b = qa.Batch(B, V, 512)
        b.set_mode({"auto": qa.MODE_AUTO, "split": qa.MODE_SPLIT}[mode])
        cfgs = []
        for r in range(B):
            cfg = (0.0 if r % 5 == 0 else 0.8, 0.95, 40 if r % 3 else 0, 0.05,
                   1.3, 512)
            cfgs.append(cfg)
            b.config(r, 1, *cfg, seeds=[1000 + r])
            b.set_history(r, hists[r])
        outs = [b.pick(base, stride, B, V, diag=True) for _ in range(3)]
        for r in range(B):
            s = oracle.sampler()
            s.config(*cfgs[r], seed=1000 + r)
            s.set_history(hists[r])
            for k in range(3):
                want = s.pick(x[r, :V])
                assert int(outs[k][0][r]) == want, (V, r, k, outs[k][1][r].path)
        b.close()
        buf.free()
        log(f"{mode} history layouts V={V} stride={stride}: {B} rows x 3 picks match")
