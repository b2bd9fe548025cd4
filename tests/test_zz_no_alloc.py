"""qs_pick_noalloc (the pick whose scratch is the library's static device array) against
qs_batch_pick on the same rows: ids, generator states and histories equal, on two calls in
a row, the second over fewer rows."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


class RowConfig(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("min_p", C.c_float),
                ("repeat_penalty", C.c_float), ("top_k", C.c_int32), ("ring_cap", C.c_int32),
                ("inv_t", C.c_float), ("pad", C.c_int32)]


def test_no_alloc_pick_equals_batch_pick(oracle):
    import quasar_amd as qa
    from quasar_amd.workloads import WORKLOADS
    lib = qa._native.load()
    w = WORKLOADS["peaked_b256"]
    B, V, cap = w.batch, w.vocab, max(1, w.repeat_last_n)
    print(f"no-alloc pick: {w.name} B={B} V={V}", flush=True)
    logits = qa.DeviceBuffer(4 * B * V)
    qa.gen_logits_device(logits, V, 0, B, V, w.dist, w.sigma, w.boost, w.seed)
    seeds = np.asarray(oracle.gen_row_seeds(w.seed, 0, B), dtype=np.uint64)
    hist = oracle.gen_hist(w.seed, 0, B, w.hist_len, V, w.hist_pool)
    # the existing entry point
    bt = qa.Batch(B, V, cap)
    bt.config(0, B, *w.params(), seeds=seeds)
    bt.set_history(0, hist)
    want = [bt.pick(logits.ptr, V, B, V).copy(), bt.pick(logits.ptr, V, B // 2, V).copy()]
    want_state = [bt.get_state(r) for r in range(B)]
    bt.close()
    # the same rows' state in caller buffers
    cfg = (RowConfig * B)()
    for r in range(B):
        lib.qs_row_config_set(C.byref(cfg[r]), *w.params())
    d_cfg = qa.DeviceBuffer.from_array(np.frombuffer(bytes(cfg), dtype=np.uint8))
    d_rng = qa.DeviceBuffer.from_array(seeds)
    ring = np.zeros((B, cap), np.int32)
    ring[:, :hist.shape[1]] = hist
    d_ring = qa.DeviceBuffer.from_array(ring)
    d_len = qa.DeviceBuffer.from_array(np.full(B, hist.shape[1], np.int32))
    d_head = qa.DeviceBuffer.from_array(np.zeros(B, np.int32))
    d_out = qa.DeviceBuffer(4 * B)
    got = []
    for n in (B, B // 2):
        rc = lib.qs_pick_noalloc(logits.ptr, V, n, V, d_cfg.ptr, d_rng.ptr, d_ring.ptr, cap,
                                 d_len.ptr, d_head.ptr, d_out.ptr, None)
        assert rc == 0, lib.qs_last_error()
        qa.check(lib.qs_device_synchronize(), "sync")
        got.append(d_out.download(np.int32, n))
    for g, wnt in zip(got, want):
        assert np.array_equal(g, wnt)
    rng = d_rng.download(np.uint64, B)
    ring = d_ring.download(np.int32, B * cap).reshape(B, cap)
    ln = d_len.download(np.int32, B)
    hd = d_head.download(np.int32, B)
    for r in range(B):
        seq = [int(ring[r, (hd[r] + i) % cap]) for i in range(ln[r])]
        assert int(rng[r]) == want_state[r][0] and seq == list(want_state[r][1]), r
    # beyond the static scratch: refused before any launch
    assert lib.qs_pick_noalloc(logits.ptr, V, 300, V, d_cfg.ptr, d_rng.ptr, d_ring.ptr, cap,
                               d_len.ptr, d_head.ptr, d_out.ptr, None) == qa._native.QS_EINVAL
    for buf in (logits, d_cfg, d_rng, d_ring, d_len, d_head, d_out):
        buf.free()


def test_no_alloc_pick_clamps_caller_ring_state(oracle):
    """Row configs that ask for a longer ring than the call passes, and history lengths and
    heads outside the ring: the kernels use a capacity of at most the ring stride (none
    without a ring), a length in [0, cap] and a head in [0, cap) (0 when outside).  The picks
    equal qs_batch_pick's on the history that clamped state describes, and the state left
    behind is in range."""
    import quasar_amd as qa
    from quasar_amd.workloads import WORKLOADS
    lib = qa._native.load()
    w = WORKLOADS["peaked_b256"]
    B, V, S = 64, w.vocab, 8
    print(f"no-alloc ring clamp: {w.name} B={B} V={V} stride {S}", flush=True)
    logits = qa.DeviceBuffer(4 * B * V)
    qa.gen_logits_device(logits, V, 0, B, V, w.dist, w.sigma, w.boost, w.seed)
    seeds = np.asarray(oracle.gen_row_seeds(w.seed, 0, B), dtype=np.uint64)
    hist = oracle.gen_hist(w.seed, 0, B, S, V, w.hist_pool)       # the 8 slots' ids
    params = list(w.params())
    cfg = (RowConfig * B)()
    for r in range(B):
        lib.qs_row_config_set(C.byref(cfg[r]), *params)              # ring capacity 256 > 8
    assert cfg[0].ring_cap == w.repeat_last_n > S
    d_cfg = qa.DeviceBuffer.from_array(np.frombuffer(bytes(cfg), dtype=np.uint8))
    d_out = qa.DeviceBuffer(4 * B)
    bad_len = np.array([1000, -7, 2**31 - 1, 9] * (B // 4), np.int32)
    bad_head = np.array([-5, 8, 1 << 20, -2**31] * (B // 4), np.int32)
    for with_ring in (False, True):
        # the existing entry point on the history the clamped state describes
        p = list(params)
        p[5] = S if with_ring else 0                                 # repeat_last_n
        bt = qa.Batch(B, V, S)
        bt.config(0, B, *p, seeds=seeds)
        if with_ring:
            # length clamps to 8 (or 0 for -7); the head to 0
            bt.set_history(0, hist)
            for r in range(1, B, 4):
                bt.set_history(r, hist[r:r + 1, :0])
        want = [bt.pick(logits.ptr, V, B, V).copy(), bt.pick(logits.ptr, V, B, V).copy()]
        want_state = [bt.get_state(r) for r in range(B)]
        bt.close()
        d_rng = qa.DeviceBuffer.from_array(seeds)
        d_ring = qa.DeviceBuffer.from_array(np.ascontiguousarray(hist)) if with_ring else None
        d_len = qa.DeviceBuffer.from_array(bad_len.copy())
        d_head = qa.DeviceBuffer.from_array(bad_head.copy())
        got = []
        for _ in range(2):
            rc = lib.qs_pick_noalloc(logits.ptr, V, B, V, d_cfg.ptr, d_rng.ptr,
                                     d_ring.ptr if d_ring else None, S if with_ring else 0,
                                     d_len.ptr, d_head.ptr, d_out.ptr, None)
            assert rc == 0, lib.qs_last_error()
            qa.check(lib.qs_device_synchronize(), "sync")
            got.append(d_out.download(np.int32, B))
        for g, wnt in zip(got, want):
            assert np.array_equal(g, wnt), with_ring
        rng = d_rng.download(np.uint64, B)
        ln = d_len.download(np.int32, B)
        hd = d_head.download(np.int32, B)
        assert all(int(rng[r]) == want_state[r][0] for r in range(B))
        if with_ring:
            ring = d_ring.download(np.int32, B * S).reshape(B, S)
            assert ((ln >= 0) & (ln <= S) & (hd >= 0) & (hd < S)).all()
            for r in range(B):
                seq = [int(ring[r, (hd[r] + i) % S]) for i in range(ln[r])]
                assert seq == list(want_state[r][1]), r
            d_ring.free()
        else:                                                        # nothing recorded
            assert np.array_equal(ln, bad_len) and np.array_equal(hd, bad_head)
        for buf in (d_rng, d_len, d_head):
            buf.free()
    for buf in (logits, d_cfg, d_out):
        buf.free()
