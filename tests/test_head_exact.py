"""The output layer at the reference's arithmetic (qs_batch_head_exact_logits,
qs_batch_pick_head_exact) and its CPU restatement (orc_head.c).

The restatement is pinned first, on the CPU: its dequantization bit for bit against the
reference's own quant.c built from source (oracle/_ref, where the source is present), the
binary16 widening against numpy's for all 65536 patterns, Q6_K rows built from known
six-bit values, scales and d against (d sc)(q - 32) in float32, and its sum by cases the
mathematics fixes: exact small-integer rows, a row whose sequential float sum differs from
every other order, a product rounded before its sum (an FMA gives another value), and the
recursive-summation bound on random rows.

On the GPU: every logit equals the restatement's bit for bit (NaN for NaN) for the four
types at several shapes, up to the vocabulary of 151,936 at n_embd 2048 (Q6_K, as the
reference's model stores its output matrix) and 1 to 8 rows; the fused pick's ids, states
and histories equal qs_batch_pick's on the logits the same call wrote, and the restatement's
sampler on those logits; arguments outside the limits are refused before any launch."""
import sys

import numpy as np
import pytest

import pyoracle
from pyoracle import RefQuant

F32, F16, Q8_0, Q6_K = 0, 1, 8, 14
TYPES = {F32: "F32", F16: "F16", Q8_0: "Q8_0", Q6_K: "Q6_K"}


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def row_bytes(wtype, E):
    return {F32: 4 * E, F16: 2 * E, Q8_0: E // 32 * 34, Q6_K: E // 256 * 210}[wtype]


def half_bits(x):
    return np.atleast_1d(np.asarray(x, dtype=np.float16)).view(np.uint16)


def make_weights(rng, wtype, E, V):
    """V GGUF rows of E elements of `wtype` (the file's bytes), values of a trained
    matrix's size: N(0, 1/E) for F32/F16, per-block scales near 2^-7 for Q8_0 and Q6_K."""
    if wtype == F32:
        return rng.normal(0.0, 1.0 / np.sqrt(E), (V, E)).astype(np.float32).view(np.uint8)
    if wtype == F16:
        return rng.normal(0.0, 1.0 / np.sqrt(E), (V, E)).astype(np.float16).view(np.uint8)
    if wtype == Q8_0:
        nb = E // 32
        blk = np.zeros((V, nb, 34), np.uint8)
        d = (rng.uniform(0.5, 1.5, (V, nb)) / 128 / np.sqrt(E)).astype(np.float16)
        blk[:, :, 0:2] = d.view(np.uint8).reshape(V, nb, 2)
        blk[:, :, 2:] = rng.integers(-128, 128, (V, nb, 32)).astype(np.int8).view(np.uint8)
        return blk.reshape(V, nb * 34)
    nb = E // 256
    blk = rng.integers(0, 256, (V, nb, 210)).astype(np.uint8)
    d = (rng.uniform(0.5, 1.5, (V, nb)) / 2048 / np.sqrt(E)).astype(np.float16)
    blk[:, :, 208:210] = d.view(np.uint8).reshape(V, nb, 2)
    return blk.reshape(V, nb * 210)


def q6k_encode(q, sc, d):
    """One Q6_K super-block's 210 bytes from 256 six-bit values q (0..63), 16 int8 scales
    and d (float16): the GGUF block layout, the inverse of quant.c's dequant_q6_K."""
    b = np.zeros(210, np.uint8)
    ql, qh = b[0:128], b[128:192]
    for h in range(2):
        for l in range(32):
            e = [128 * h + 32 * qd + l for qd in range(4)]
            ql[64 * h + l] = (q[e[0]] & 15) | ((q[e[2]] & 15) << 4)
            ql[64 * h + 32 + l] = (q[e[1]] & 15) | ((q[e[3]] & 15) << 4)
            qh[32 * h + l] = sum(((q[e[qd]] >> 4) & 3) << (2 * qd) for qd in range(4))
    b[192:208] = np.asarray(sc, np.int8).view(np.uint8)
    b[208:210] = half_bits(d).view(np.uint8)
    return b


def same_bits(got, want):
    """Bit-equal float32 arrays, NaN matching NaN (payloads aside)."""
    g = np.ascontiguousarray(got, np.float32)
    w = np.ascontiguousarray(want, np.float32)
    gn, wn = np.isnan(g), np.isnan(w)
    return bool(np.array_equal(gn, wn) and
                np.array_equal(g.view(np.uint32)[~gn], w.view(np.uint32)[~wn]))


# ---------------------------------------------------------------- the restatement, on the CPU

@pytest.mark.parametrize("wtype", [F32, F16, Q8_0, Q6_K])
def test_dequant_equals_the_reference_quant_c(oracle, wtype):
    """orc_dequant_row against quasar_dequant_row built from the reference's quant.c, on
    random rows including inf, NaN and subnormal binary16 scales."""
    if not RefQuant.available():
        pytest.skip("oracle/_ref/libref_quant.so not built (the reference source is absent)")
    ref = RefQuant()
    rng = np.random.default_rng(wtype + 1)
    E = 512
    for trial in range(40):
        w = rng.integers(0, 256, row_bytes(wtype, E)).astype(np.uint8)
        if trial % 4 == 1 and wtype in (Q8_0, Q6_K):
            off = 0 if wtype == Q8_0 else 208
            w[off:off + 2] = half_bits(np.inf).view(np.uint8)
        if trial % 4 == 2 and wtype == Q6_K:
            w[208:210] = np.array([0x01, 0x00], np.uint8)       # the least subnormal
        got = oracle.dequant_row(wtype, w, E)
        want = ref.dequant_row(wtype, w, E)
        assert same_bits(got, want), (TYPES[wtype], trial)


def test_half_widening_against_numpy(oracle):
    """All 65536 binary16 patterns (as an F16 row) widen as numpy's float16 -> float32."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.dequant_row(F16, bits.view(np.uint8), 65536)
    assert same_bits(got, bits.view(np.float16).astype(np.float32))


def test_q6k_rows_from_known_values(oracle):
    """Super-blocks encoded from chosen q, scales and d decode to (d sc)(q - 32) rounded
    in float32, for every element position (the block layout's index mapping)."""
    rng = np.random.default_rng(5)
    for trial in range(20):
        q = rng.integers(0, 64, 256)
        if trial == 0:
            q = np.arange(256) % 64
        sc = rng.integers(-128, 128, 16)
        d = np.float16(rng.uniform(-2, 2) * 2.0 ** int(rng.integers(-14, 4)))
        got = oracle.dequant_row(Q6_K, q6k_encode(q, sc, d), 256)
        is_ = np.arange(256) // 128 * 8 + (np.arange(256) % 32) // 16 + 2 * ((np.arange(256) % 128) // 32)
        want = (np.float32(d) * sc[is_].astype(np.float32)) * (q - 32).astype(np.float32)
        assert same_bits(got, want.astype(np.float32)), trial


def test_q8_0_rows_from_known_values(oracle):
    rng = np.random.default_rng(6)
    q = rng.integers(-128, 128, (4, 32))
    d = np.float16(rng.uniform(-1, 1, 4))
    w = np.zeros((4, 34), np.uint8)
    w[:, 0:2] = half_bits(d).view(np.uint8).reshape(4, 2)
    w[:, 2:] = q.astype(np.int8).view(np.uint8)
    got = oracle.dequant_row(Q8_0, w.reshape(-1), 128)
    want = (d.astype(np.float32)[:, None] * q.astype(np.float32)).reshape(-1)
    assert same_bits(got, want)


def test_gemv_small_integers_are_exact(oracle):
    """Integer weights and inputs whose every partial sum is an integer below 2^24: the
    logits are the integer dot products."""
    rng = np.random.default_rng(7)
    E, V, B = 256, 300, 3
    w = rng.integers(-8, 9, (V, E))
    x = rng.integers(-8, 9, (B, E))
    got = oracle.head_gemv(F32, w.astype(np.float32).view(np.uint8), x.astype(np.float32), V)
    assert np.array_equal(got, (x @ w.T).astype(np.float32))


def test_gemv_sums_in_k_order(oracle):
    """Unit weights against x = (2^24, 1, -2^24, 1): in k order 2^24 + 1 rounds (a tie, to
    even) to 2^24, then 0, then 1; reversed, the sum is 2 (exact), pairwise 1 + 0... = 1
    as well, so a second row tells them apart: x = (1, 2^24, 1, -2^24) gives 0 in k order
    (both ones absorbed), 2 reversed and 1 pairwise."""
    w = np.ones((1, 4), np.float32)
    x = np.array([[2.0 ** 24, 1.0, -2.0 ** 24, 1.0], [1.0, 2.0 ** 24, 1.0, -2.0 ** 24]],
                 np.float32)
    got = oracle.head_gemv(F32, w.view(np.uint8), x, 1)
    assert got[0, 0] == 1.0 and got[1, 0] == 0.0, got


def test_gemv_rounds_each_product(oracle):
    """w = (1, 1 + 2^-12), x = (-1, 1 + 2^-12): the product 1 + 2^-11 + 2^-24 rounds (a tie,
    to even) to 1 + 2^-11 before the sum, so the logit is 2^-11; a fused multiply-add would
    keep 2^-11 + 2^-24."""
    a = np.float32(1 + 2.0 ** -12)
    w = np.array([[1.0, a]], np.float32)
    x = np.array([[-1.0, a]], np.float32)
    got = oracle.head_gemv(F32, w.view(np.uint8), x, 1)
    assert got[0, 0] == np.float32(2.0 ** -11)


@pytest.mark.parametrize("wtype", [F32, F16, Q8_0, Q6_K])
def test_gemv_within_the_recursive_summation_bound(oracle, wtype):
    """|logit - exact dot product of the dequantized row| <= gamma_E sum |w x| (E products
    and E - 1 sums, each rounded by at most 2^-24 relative)."""
    rng = np.random.default_rng(8 + wtype)
    E, V, B = 512, 200, 2
    wb = make_weights(rng, wtype, E, V)
    x = rng.normal(0, 1, (B, E)).astype(np.float32)
    got = oracle.head_gemv(wtype, wb, x, V).astype(np.float64)
    wd = np.stack([oracle.dequant_row(wtype, wb[v], E) for v in range(V)]).astype(np.float64)
    exact = x.astype(np.float64) @ wd.T
    mag = np.abs(x.astype(np.float64)) @ np.abs(wd).T
    u = 2.0 ** -24
    gamma = 2 * E * u / (1 - 2 * E * u)
    assert np.all(np.abs(got - exact) <= gamma * mag + 1e-300)


def test_exact_layer_symbols_and_sizes():
    """The library exports the exact layer's entry points; the packed size matches the GGUF
    bytes for the quantized types (same bits, another order) and is 0 for types or shapes
    not taken."""
    import quasar_amd as qa
    lib = qa.load()
    for name in ("qs_head_exact_packed_bytes", "qs_batch_head_exact_pack",
                 "qs_batch_head_exact_logits", "qs_batch_pick_head_exact",
                 "qs_batch_time_head_exact"):
        assert hasattr(lib, name), name
    assert qa.head_exact_packed_bytes(Q6_K, 2048, 151936) == 151936 * 8 * 210 + (
        2374 * 64 - 151936) * 8 * 210
    assert qa.head_exact_packed_bytes(F32, 64, 1000) == 1024 * 256
    assert qa.head_exact_packed_bytes(2, 2048, 1000) == 0         # Q4_0: not taken
    assert qa.head_exact_packed_bytes(Q6_K, 2000, 1000) == 0      # not a multiple of 256
    assert qa.head_exact_packed_bytes(F16, 8, 1000) == 0          # below 16


# ---------------------------------------------------------------- the GPU

@pytest.fixture(scope="module")
def qa():
    import quasar_amd
    quasar_amd.load()
    return quasar_amd


def upload_exact(qa, bt, wtype, wb, E, V):
    dw = qa.DeviceBuffer.from_array(np.ascontiguousarray(wb).reshape(-1))
    dp = qa.DeviceBuffer(qa.head_exact_packed_bytes(wtype, E, V))
    bt.head_exact_pack(wtype, dw.ptr, E, V, dp.ptr)
    bt.synchronize()
    dw.free()
    return dp


def run_logits(qa, wtype, wb, x, V):
    B, E = x.shape
    bt = qa.Batch(8, V, 1)
    dp = upload_exact(qa, bt, wtype, wb, E, V)
    dx = qa.DeviceBuffer.from_array(np.ascontiguousarray(x, np.float32))
    dl = qa.DeviceBuffer(4 * B * V)
    bt.head_exact_logits(wtype, dp.ptr, dx.ptr, E, B, V, dl.ptr)
    bt.synchronize()
    got = dl.download(np.float32, B * V).reshape(B, V)
    bt.close()
    for b in (dp, dx, dl):
        b.free()
    return got


EXACT_SHAPES = [
    (F32, 64, 1000, 1), (F32, 272, 4100, 3), (F32, 16, 100, 8),
    (F16, 128, 2052, 2), (F16, 1024, 50000, 8),
    (Q8_0, 96, 1000, 1), (Q8_0, 2048, 32768, 5),
    (Q6_K, 256, 1000, 1), (Q6_K, 512, 10004, 4), (Q6_K, 256, 64, 7),
    (Q6_K, 2048, 151936, 1), (Q6_K, 2048, 151936, 8),
]


@pytest.mark.gpu
@pytest.mark.parametrize("wtype,E,V,B", EXACT_SHAPES)
def test_exact_logits_bit_for_bit(qa, oracle, wtype, E, V, B):
    rng = np.random.default_rng(E * 7 + V + B)
    wb = make_weights(rng, wtype, E, V)
    x = rng.normal(0, 1, (B, E)).astype(np.float32)
    log(f"exact logits {TYPES[wtype]} E {E} V {V} B {B}")
    got = run_logits(qa, wtype, wb, x, V)
    want = oracle.head_gemv(wtype, wb, x, V)
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))
    assert same_bits(got, want), (bad[0][:4], bad[1][:4], got[bad][:4], want[bad][:4])


@pytest.mark.gpu
def test_exact_logits_non_finite(qa, oracle):
    """inf and NaN scales and weights, infinite and NaN hidden elements, sums that overflow:
    the same inf, -inf and NaN positions and every finite logit bit for bit."""
    rng = np.random.default_rng(21)
    for wtype, E, V in ((Q6_K, 512, 3000), (F16, 64, 3000), (Q8_0, 64, 3000)):
        wb = make_weights(rng, wtype, E, V).copy()
        if wtype == Q6_K:
            wb[5, 208:210] = half_bits(np.inf).view(np.uint8)      # d = inf (NaN where sc 0)
            wb[9, 210 + 208:210 + 210] = half_bits(np.nan).view(np.uint8)
            wb[11, 208:210] = half_bits(65504.0).view(np.uint8)    # sums overflow
        elif wtype == F16:
            wb.view(np.uint16)[5, 3] = 0x7C00                     # +inf
            wb.view(np.uint16)[9, 0] = 0x7E00                     # NaN
            wb.view(np.uint16)[11, :] = 0x7BFF                    # 65504 everywhere
        else:
            wb[5, 0:2] = half_bits(-np.inf).view(np.uint8)
            wb[9, 34:36] = half_bits(np.nan).view(np.uint8)
            wb[11, 0:2] = half_bits(65504.0).view(np.uint8)
        x = rng.normal(0, 1, (4, E)).astype(np.float32)
        x[1, 7] = np.inf
        x[2, 3] = np.nan
        x[3, :] = 3.0e38
        got = run_logits(qa, wtype, wb, x, V)
        want = oracle.head_gemv(wtype, wb, x, V)
        assert np.isinf(want).any() and np.isnan(want).any()
        assert same_bits(got, want), TYPES[wtype]


ROWS = [
    # (temperature, top_p, top_k, min_p, repeat_penalty, repeat_last_n)
    (0.8, 0.95, 40, 0.05, 1.1, 64),
    (0.0, 1.0, 0, 0.0, 1.3, 32),
    (1.0, 0.9, 0, 0.0, 1.0, 0),
    (0.6, 0.95, 200, 0.02, 1.3, 64),
    (0.7, 1.0, 1, 0.0, 1.0, 0),
    (1.2, 0.5, 64, 0.1, 1.2, 16),
]


def exact_pick_case(qa, oracle, wtype, E, V, B, picks, seed, x_scale=1.0):
    rng = np.random.default_rng(seed)
    wb = make_weights(rng, wtype, E, V)
    x = rng.normal(0, 1, (B, E)).astype(np.float32) * np.float32(x_scale)
    if B > 3:
        x[3] = 0.0                                 # every logit 0: ties across every tile
    fused, plain = qa.Batch(B, V, 64), qa.Batch(B, V, 64)
    dp = upload_exact(qa, fused, wtype, wb, E, V)
    dx = qa.DeviceBuffer.from_array(x)
    dl = qa.DeviceBuffer(4 * B * V)
    cfgs = []
    for r in range(B):
        cfg = ROWS[r % len(ROWS)]
        sd = int(rng.integers(1, 2**62))
        hist = rng.integers(0, V, 48).astype(np.int32)
        for bt in (fused, plain):
            bt.config(r, 1, *cfg, seeds=[sd])
            bt.set_history(r, hist)
        cfgs.append((cfg, sd, hist))
    samplers = []
    for cfg, sd, hist in cfgs:
        s = oracle.sampler()
        s.config(*cfg, seed=sd)
        s.set_history(hist)
        samplers.append(s)
    want_logits = oracle.head_gemv(wtype, wb, x, V)
    paths = {}
    for k in range(picks):
        ids_f, diag = fused.pick_head_exact(wtype, dp.ptr, dx.ptr, E, B, V, dl.ptr, diag=True)
        logits = dl.download(np.float32, B * V).reshape(B, V)
        assert same_bits(logits, want_logits), k
        buf = qa.DeviceBuffer.from_array(logits)
        ids_p = plain.pick(buf.ptr, V, B, V)
        buf.free()
        for d in diag:
            paths[d.path] = paths.get(d.path, 0) + 1
        bad = np.nonzero(ids_f != ids_p)[0]
        assert bad.size == 0, (k, bad[:8], ids_f[bad[:8]], ids_p[bad[:8]])
        for r in range(B):
            want = samplers[r].pick(want_logits[r])
            assert int(ids_f[r]) == want, (k, r, int(ids_f[r]), want)
    for r in range(B):
        assert fused.get_state(r)[0] == plain.get_state(r)[0], r
        assert (fused.get_state(r)[1] == plain.get_state(r)[1]).all(), r
    log(f"exact pick {TYPES[wtype]} B {B} E {E} V {V}: {picks} picks identical; paths {paths}")
    fused.close()
    plain.close()
    for b in (dp, dx, dl):
        b.free()


@pytest.mark.gpu
@pytest.mark.parametrize("B", [1, 2, 5, 8])
def test_exact_pick_full_vocabulary(qa, oracle, B):
    exact_pick_case(qa, oracle, Q6_K, 2048, 151936, B, 3, 30 + B, x_scale=4.0)


@pytest.mark.gpu
def test_exact_pick_small_vocab_partial_tile(qa, oracle):
    exact_pick_case(qa, oracle, F16, 64, 1000, 7, 4, 41, x_scale=8.0)


@pytest.mark.gpu
def test_exact_pick_q8_0(qa, oracle):
    exact_pick_case(qa, oracle, Q8_0, 256, 20000, 3, 3, 42, x_scale=8.0)


@pytest.mark.gpu
def test_exact_rejects_arguments_outside_the_limits(qa):
    """Refused before any launch (QS_EINVAL), the batch usable afterwards."""
    E, V = 256, 1000
    rng = np.random.default_rng(4)
    wb = make_weights(rng, Q6_K, E, V)
    bt = qa.Batch(16, V, 8)
    dp = upload_exact(qa, bt, Q6_K, wb, E, V)
    dx = qa.DeviceBuffer(4 * 16 * 2048 + 16)
    dl = qa.DeviceBuffer(4 * 16 * V + 16)
    bad = [
        (2, E, 1, V, dx.ptr, dl.ptr),              # Q4_0
        (Q6_K, 255, 1, V, dx.ptr, dl.ptr),         # n_embd not a multiple of 256
        (Q6_K, E, 9, V, dx.ptr, dl.ptr),           # more rows than 8
        (Q6_K, E, 0, V, dx.ptr, dl.ptr),
        (F32, 4096, 5, V, dx.ptr, dl.ptr),         # rows x n_embd above 16384
        (Q6_K, E, 1, 998 + 1, dx.ptr, dl.ptr),     # vocab not a multiple of 4
        (Q6_K, E, 1, 2000, dx.ptr, dl.ptr),        # beyond the batch's vocabulary
        (Q6_K, E, 1, V, dx.ptr + 4, dl.ptr),       # misaligned hidden rows
        (Q6_K, E, 1, V, dx.ptr, dl.ptr + 4),       # misaligned logits
    ]
    for i, (wt, e, n, v, px, pl) in enumerate(bad):
        with pytest.raises(qa.QsError) as ei:
            bt.head_exact_logits(wt, dp.ptr, px, e, n, v, pl)
        assert ei.value.rc == -22, i
        with pytest.raises(qa.QsError):
            bt.pick_head_exact(wt, dp.ptr, px, e, n, v, pl)
    with pytest.raises(qa.QsError):
        bt.head_exact_pack(2, dp.ptr, E, V, dp.ptr)
    x = rng.normal(0, 1, (2, E)).astype(np.float32)
    dx2 = qa.DeviceBuffer.from_array(x)
    bt.config(0, 2, 0.0, 1.0, 0, 0.0, 1.0, 0, seeds=[1, 2])
    ids = bt.pick_head_exact(Q6_K, dp.ptr, dx2.ptr, E, 2, V, dl.ptr)
    logits = dl.download(np.float32, 2 * V).reshape(2, V)
    assert list(ids) == [int(np.argmax(logits[0])), int(np.argmax(logits[1]))]
    bt.close()
    for b in (dp, dx, dl, dx2):
        b.free()
