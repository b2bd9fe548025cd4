"""The mixture-of-experts router's choice (forward_cpu.c:165-172, 296-304): the CPU
restatement pinned by an independent numpy computation, by the exact rational sum of the
host-libm numerators within the float summation bound, by exhaustive tie/NaN/inf
placements on 1-8 experts against the rule IEEE arithmetic fixes, and by sorting exact
rationals of the probabilities (CPU); then the device kernel behind qs_router_topk
against it, bit for bit (GPU)."""
import numpy as np
import pytest


def numpy_choice(oracle, x, n_used, norm):
    """The same arithmetic done another way: float32 numpy with the host libm expf, a
    float32 running sum (np.cumsum adds in order), and the choice as a stable sort on
    (-p, index).  Rows must be NaN-free and not all -inf."""
    mx = np.float32(np.max(x))
    e = oracle.libm_expf(x - mx)
    s = np.cumsum(e, dtype=np.float32)[-1]
    p = e * (np.float32(1.0) / s)
    order = np.lexsort((np.arange(x.size), -p))[:n_used]
    wt = p[order].astype(np.float32)
    if norm:
        sm = np.cumsum(wt, dtype=np.float32)[-1]
        if sm > 0:
            wt = wt / sm
    return order.astype(np.int32), wt.astype(np.float32), p


def rows(seed, t, e, scale=3.0):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((t, e)) * scale).astype(np.float32)
    x[0, :] = np.float32(1.25)                       # all equal: lowest indices first
    top = np.float32(x[1].max() + 1)
    for j in (5, 9, 40):                             # a three-way tie at the top
        if j < e:
            x[1, j] = top
    x[2, :] = np.round(x[2, :])                      # many ties
    if e > 7:
        x[3, 7] = -np.inf                            # probability 0
    return x


@pytest.mark.parametrize("e,u", [(128, 8), (64, 4), (256, 64), (100, 7), (1, 1), (8, 8)])
@pytest.mark.parametrize("norm", [0, 1])
def test_oracle_matches_numpy(oracle, e, u, norm):
    x = rows(11 + e + u, 24, e)
    idx, wt = oracle.router_topk(x, u, norm)
    for t in range(x.shape[0]):
        ni, nw, p = numpy_choice(oracle, x[t], u, norm)
        assert (idx[t] == ni).all(), (t, idx[t], ni)
        assert (wt[t].view(np.uint32) == nw.view(np.uint32)).all(), t
        # invariants: probabilities sum to 1, the first choice is the first arg-max of the
        # logits, choices descend, normalised weights sum to 1
        assert abs(float(np.sum(p, dtype=np.float64)) - 1.0) < 1e-5
        assert p[idx[t][0]] == p.max()
        assert (np.diff(p[idx[t]]) <= 0).all()
        if norm:
            assert abs(float(np.sum(wt[t], dtype=np.float64)) - 1.0) < 1e-5


def test_oracle_edge_rows(oracle):
    """All-equal rows take the lowest indices.  A NaN logit anywhere makes the float sum,
    and so every probability, NaN (forward_cpu.c:169-171); so does a row of -inf.  The
    reference's scan then finds nothing and reads index -1: expert -1, weight 0."""
    x = np.zeros((4, 16), dtype=np.float32)
    x[1, 3] = np.nan
    x[1, 0] = np.float32(2.0)
    x[2, 0] = np.nan
    x[3, :] = -np.inf
    idx, wt = oracle.router_topk(x, 4, 0)
    assert list(idx[0]) == [0, 1, 2, 3] and np.allclose(wt[0], 1 / 16)
    assert list(idx[1]) == [-1] * 4 and (wt[1] == 0).all()
    assert list(idx[2]) == [-1] * 4 and (wt[2] == 0).all()
    assert list(idx[3]) == [-1] * 4 and (wt[3] == 0).all()


U24 = 2.0 ** -24


@pytest.mark.parametrize("e", [8, 64, 128, 256])
def test_oracle_sum_within_summation_bound(oracle, e):
    """The restatement's float sum of the numerators (forward_cpu.c:168-169) lies within the
    recursive-summation bound of the exact sum of the host-libm numerators expf(x - max):
    |fl - S| <= (n - 1) u S / (1 - (n - 1) u), u = 2^-24 (a dropped term, a wrong shift or a
    product in place of a sum fails it); each probability within 3 u of e_i / S, their sum
    within the bound of 1, and larger logits never less probable."""
    from fractions import Fraction
    rng = np.random.default_rng(e)
    for t in range(40):
        x = (rng.standard_normal(e) * (3.0 if t % 2 else 0.5)).astype(np.float32)
        p, sm = oracle.router_probs(x)
        num = oracle.libm_expf(x - np.float32(x.max()))
        S = sum(Fraction(float(v)) for v in num)
        g = (e - 1) * U24 / (1 - (e - 1) * U24)
        assert abs(Fraction(float(sm)) - S) <= g * S, (t, float(sm), float(S))
        for i in range(e):
            exact = Fraction(float(num[i])) / S
            assert abs(Fraction(float(p[i])) - exact) <= (3 * U24 + 2 * g) * exact, (t, i)
        tot = sum(Fraction(float(v)) for v in p)
        assert abs(tot - 1) <= (e + 3) * U24 + 2 * g
        order = np.argsort(x, kind="stable")
        assert (np.diff(p[order]) >= 0).all()


def _brute_choice(x, n_used):
    """The rule the reference's scans implement, from IEEE arithmetic rather than its code:
    a NaN or +inf logit, or a row of -inf, makes the float sum and so every probability NaN
    (inf - inf, NaN + anything), and no probability beats -1e30: every slot is expert -1;
    otherwise probabilities order as their logits (expf and the product by one positive
    normaliser are monotone), the lowest index first among equals, -inf logits last (p 0)."""
    if any(np.isnan(v) or v == np.inf for v in x) or all(v == -np.inf for v in x):
        return [-1] * n_used
    return sorted(range(len(x)), key=lambda i: (-x[i], i))[:n_used]


@pytest.mark.parametrize("n,alphabet", [(1, 6), (2, 6), (3, 6), (4, 6), (5, 5), (6, 5),
                                        (7, 4), (8, 4)])
def test_oracle_exhaustive_small_rows(oracle, n, alphabet):
    """Every placement of -inf, -2, 0, 1, NaN and +inf (ties included) over 1-8 experts, for
    every n_used, against the brute-force rule; weights are 0 exactly for -1 slots and -inf
    logits, positive otherwise, non-increasing by slot, and with normalisation sum to 1
    within (n_used + 2) u."""
    import itertools
    vals = [-np.inf, 0.0, 1.0, np.nan, -2.0, np.inf][:alphabet]
    rows_ = np.array(list(itertools.product(vals, repeat=n)), dtype=np.float32)
    for u in range(1, n + 1):
        for norm in (0, 1):
            idx, wt = oracle.router_topk(rows_, u, norm)
            for r in range(rows_.shape[0]):
                x = [float(v) for v in rows_[r]]
                want = _brute_choice(x, u)
                assert list(idx[r]) == want, (x, u, list(idx[r]), want)
                w = wt[r]
                for s, i in enumerate(want):
                    assert (w[s] == 0) == (i < 0 or x[i] == -np.inf), (x, u, norm, list(w))
                assert (np.diff(w) <= 0).all(), (x, u, list(w))
                if norm and w.sum() > 0:
                    assert abs(float(np.sum(w, dtype=np.float64)) - 1.0) <= (u + 2) * U24


@pytest.mark.parametrize("e,u", [(16, 4), (64, 8), (128, 8), (256, 64)])
def test_oracle_choice_against_rational_sort(oracle, e, u):
    """The choice equals the n_used first of the probabilities sorted as exact rationals,
    descending, the lowest index first among equal ones (rows with many float ties)."""
    from fractions import Fraction
    rng = np.random.default_rng(100 + e)
    x = np.round(rng.standard_normal((30, e)) * 2.0, 1).astype(np.float32)
    idx, _ = oracle.router_topk(x, u, 0)
    for t in range(x.shape[0]):
        p, _ = oracle.router_probs(x[t])
        want = sorted(range(e), key=lambda i: (-Fraction(float(p[i])), i))[:u]
        assert list(idx[t]) == want, t


@pytest.mark.gpu
@pytest.mark.parametrize("e,u", [(128, 8), (64, 4), (256, 64), (100, 7), (1, 1), (60, 60)])
@pytest.mark.parametrize("norm", [0, 1])
def test_device_equals_oracle(oracle, e, u, norm):
    import quasar_amd as qa
    t = 1000
    x = rows(5 * e + u, t, e)
    x[4, :] = np.nan                       # every probability NaN
    x[5, min(3, e - 1)] = np.nan           # one NaN logit: the sum, so every p, is NaN
    x[6, 0] = np.nan                       # NaN at element 0 (the starting max)
    x[7, :] = -np.inf
    x[8, :] = np.float32(3.0e38)           # huge equal logits
    x[9, 1 % e] = np.inf
    buf = qa.DeviceBuffer.from_array(x)
    di = qa.DeviceBuffer(4 * t * u)
    dw = qa.DeviceBuffer(4 * t * u)
    qa.router_topk(buf, t, e, u, norm, di, dw)
    gi = di.download(np.int32, t * u).reshape(t, u)
    gw = dw.download(np.float32, t * u).reshape(t, u)
    oi, ow = oracle.router_topk(x, u, norm)
    bad = np.nonzero((gi != oi).any(axis=1) | (gw.view(np.uint32) != ow.view(np.uint32)).any(axis=1))[0]
    assert bad.size == 0, (bad[:5], gi[bad[:1]], oi[bad[:1]], gw[bad[:1]], ow[bad[:1]])
    for b_ in (buf, di, dw):
        b_.free()


@pytest.mark.gpu
def test_device_row_stride_and_arguments(oracle):
    """Rows read at a stride wider than the expert count; out-of-range arguments are
    rejected before any launch."""
    import quasar_amd as qa
    from quasar_amd import _native
    t, e, u, stride = 37, 128, 8, 160
    x = rows(3, t, stride)
    buf = qa.DeviceBuffer.from_array(x)
    di, dw = qa.DeviceBuffer(4 * t * u), qa.DeviceBuffer(4 * t * u)
    qa.router_topk(buf, t, e, u, 1, di, dw, row_stride=stride)
    oi, ow = oracle.router_topk(np.ascontiguousarray(x[:, :e]), u, 1)
    assert (di.download(np.int32, t * u).reshape(t, u) == oi).all()
    assert (dw.download(np.float32, t * u).reshape(t, u).view(np.uint32) == ow.view(np.uint32)).all()
    lib = _native.load()
    for args in [(t, 0, u), (t, 257, u), (t, e, 0), (t, e, 65), (t, 4, 5)]:
        assert lib.qs_router_topk(buf.ptr, stride, args[0], args[1], args[2], 0, di.ptr,
                                  dw.ptr, None) == -22
    for b_ in (buf, di, dw):
        b_.free()
