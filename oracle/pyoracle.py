"""ctypes bindings for the CPU checker libraries (TEST INFRASTRUCTURE ONLY).

Loaded only by tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg,
always as the checker or the timed CPU baseline, never on the product path.

* ``Oracle``      - oracle/liboracle.so: the C restatement of the reference sampler
                    (sample.c:31-179), plus host builds of the product's generator and
                    libm-compatible expf.
* ``RefSampler``  - oracle/_ref/libref_sample.so: the reference's own sample.c compiled
                    by oracle/Makefile (present only where that source was available at
                    build time; it is a built file and travels with the tree).
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libref_sample.so")


class Params(C.Structure):
    """Same layout as orc_params / ref_params."""
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("min_p", C.c_float),
                ("repeat_penalty", C.c_float), ("top_k", C.c_int32),
                ("repeat_last_n", C.c_int32)]


class Diag(C.Structure):
    """orc_diag."""
    _fields_ = [("id", C.c_int32), ("greedy", C.c_int32), ("n_window", C.c_int32),
                ("keep_topk", C.c_int32), ("keep_topp", C.c_int32), ("keep", C.c_int32),
                ("rank", C.c_int32), ("pad", C.c_int32),
                ("maxl", C.c_float), ("msc", C.c_float), ("inv", C.c_float), ("p0", C.c_float),
                ("sum", C.c_double), ("rsum", C.c_double), ("u", C.c_double),
                ("bdist", C.c_double), ("rng_after", C.c_uint64)]

    def as_dict(self):
        return {f: getattr(self, f) for f, _ in self._fields_ if f != "pad"}


_F = C.POINTER(C.c_float)
_I = C.POINTER(C.c_int32)
_U = C.POINTER(C.c_uint64)

# orc_diag as a numpy record (one per row from pick_rows_diag)
DIAG_DTYPE = np.dtype([(n, {C.c_int32: "<i4", C.c_float: "<f4", C.c_double: "<f8",
                            C.c_uint64: "<u8"}[t]) for n, t in Diag._fields_])
assert DIAG_DTYPE.itemsize == C.sizeof(Diag)


def _fptr(a):
    return a.ctypes.data_as(_F)


def _iptr(a):
    return a.ctypes.data_as(_I)


def _uptr(a):
    return a.ctypes.data_as(_U)


def _sampler_protos(lib, prefix):
    vp = C.c_void_p
    getattr(lib, prefix + "new").restype = vp
    getattr(lib, prefix + "new").argtypes = []
    getattr(lib, prefix + "free").argtypes = [vp]
    getattr(lib, prefix + "config").argtypes = [vp, C.c_float, C.c_float, C.c_int, C.c_float,
                                               C.c_float, C.c_int, C.c_uint64]
    getattr(lib, prefix + "reset").argtypes = [vp]
    getattr(lib, prefix + "pick").argtypes = [vp, _F, C.c_int]
    getattr(lib, prefix + "pick").restype = C.c_int


class _SamplerBase:
    """Stateful sampler mirroring sample.h (new / config / reset / pick / free)."""

    def __init__(self, lib, prefix, hooks):
        self._lib, self._p, self._h = lib, prefix, hooks
        self._s = getattr(lib, prefix + "new")()
        if not self._s:
            raise MemoryError("sampler_new returned NULL")

    def close(self):
        if self._s:
            getattr(self._lib, self._p + "free")(self._s)
            self._s = None

    __del__ = close

    def config(self, temperature=0.0, top_p=1.0, top_k=0, min_p=0.0, repeat_penalty=1.0,
               repeat_last_n=0, seed=1):
        getattr(self._lib, self._p + "config")(self._s, temperature, top_p, int(top_k), min_p,
                                               repeat_penalty, int(repeat_last_n),
                                               int(seed) & 0xFFFFFFFFFFFFFFFF)

    def reset(self):
        getattr(self._lib, self._p + "reset")(self._s)

    def pick(self, logits):
        a = np.ascontiguousarray(logits, dtype=np.float32)
        return getattr(self._lib, self._p + "pick")(self._s, _fptr(a), a.size)

    def set_history(self, ids):
        a = np.ascontiguousarray(ids, dtype=np.int32)
        getattr(self._lib, self._h + "set_history")(self._s, _iptr(a), a.size)

    def history(self, cap=1 << 16):
        out = np.zeros(cap, dtype=np.int32)
        n = getattr(self._lib, self._h + "get_history")(self._s, _iptr(out), cap)
        return out[:min(n, cap)].copy()

    def params(self):
        """Stored parameters after the config clamps: (temperature, top_p, min_p,
        repeat_penalty, top_k, repeat_last_n, ring capacity)."""
        f = np.zeros(4, dtype=np.float32)
        i = np.zeros(3, dtype=np.int32)
        getattr(self._lib, self._h + "get_params")(self._s, _fptr(f), _iptr(i))
        return tuple(float(x) for x in f) + tuple(int(x) for x in i)

    @property
    def rng(self):
        return getattr(self._lib, self._h + "get_rng")(self._s)

    @rng.setter
    def rng(self, v):
        getattr(self._lib, self._h + "set_rng")(self._s, int(v) & 0xFFFFFFFFFFFFFFFF)

    def fail_allocs(self, on):
        """While on, the scratch allocations fail (the out-of-memory branch, sample.c:113)."""
        self._fail(self._s, int(bool(on)))


def _hook_protos(lib, h):
    vp = C.c_void_p
    getattr(lib, h + "set_history").argtypes = [vp, _I, C.c_int]
    getattr(lib, h + "get_history").argtypes = [vp, _I, C.c_int]
    getattr(lib, h + "get_history").restype = C.c_int
    getattr(lib, h + "get_rng").argtypes = [vp]
    getattr(lib, h + "get_rng").restype = C.c_uint64
    getattr(lib, h + "set_rng").argtypes = [vp, C.c_uint64]
    getattr(lib, h + "get_params").argtypes = [vp, _F, _I]


def _rows_protos(fn):
    fn.argtypes = [C.POINTER(Params), _F, C.c_long, C.c_int, C.c_int, _I, C.c_int, _U, _I,
                   C.c_int]
    fn.restype = C.c_double


def _pick_rows(fn, params, logits, n_rows, n_vocab, hist, seeds, n_threads):
    """Shared body of the threaded CPU drivers; returns (ids, seconds)."""
    logits = np.asarray(logits, dtype=np.float32)
    assert logits.flags.c_contiguous and logits.ndim == 2 and logits.shape[0] >= n_rows
    stride = logits.shape[1]
    seeds = np.ascontiguousarray(seeds, dtype=np.uint64)
    if hist is None:
        hist = np.zeros((n_rows, 0), dtype=np.int32)
    hist = np.ascontiguousarray(hist, dtype=np.int32)
    out = np.zeros(n_rows, dtype=np.int32)
    secs = fn(C.byref(params), _fptr(logits), stride, n_rows, n_vocab, _iptr(hist),
              hist.shape[1] if hist.ndim == 2 else 0, _uptr(seeds), _iptr(out), n_threads)
    return out, secs


class Oracle:
    """The C restatement (liboracle.so)."""

    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (run `make -C oracle`)")
        self.lib = lib = C.CDLL(path)
        _sampler_protos(lib, "orc_sampler_")
        _hook_protos(lib, "orc_sampler_")
        lib.orc_sampler_fail_scratch.argtypes = [C.c_void_p, C.c_int]
        _rows_protos(lib.orc_pick_rows)
        lib.orc_pick_rows_diag.argtypes = [C.POINTER(Params), _F, C.c_long, C.c_int, C.c_int,
                                           _I, C.c_int, _U, _I, C.c_void_p, C.c_int]
        lib.orc_pick_rows_diag.restype = C.c_double
        lib.orc_sampler_pick_diag.argtypes = [C.c_void_p, _F, C.c_int, C.POINTER(Diag)]
        lib.orc_sampler_pick_diag.restype = C.c_int
        lib.orc_xorshift64.argtypes = [_U]
        lib.orc_xorshift64.restype = C.c_uint64
        lib.orc_rng_unit.argtypes = [_U]
        lib.orc_rng_unit.restype = C.c_double
        lib.orc_gen_logits.argtypes = [C.c_int32, C.c_float, C.c_float, C.c_uint64, C.c_long,
                                       C.c_int, C.c_int, _F, C.c_long]
        lib.orc_gen_hist.argtypes = [C.c_uint64, C.c_long, C.c_int, C.c_int, C.c_int, C.c_int,
                                     _I]
        lib.orc_gen_row_seed.argtypes = [C.c_uint64, C.c_long]
        lib.orc_gen_row_seed.restype = C.c_uint64
        lib.orc_product_expf.argtypes = [C.c_float]
        lib.orc_product_expf.restype = C.c_float
        lib.orc_libm_expf_array.argtypes = [_F, _F, C.c_long]
        lib.orc_check_expf_range.argtypes = [C.c_float, C.c_float, C.c_int]
        lib.orc_check_expf_range.restype = C.c_long
        lib.orc_router_topk.argtypes = [_F, C.c_long, C.c_int, C.c_int, C.c_int, C.c_int, _I,
                                        _F]
        lib.orc_router_probs.argtypes = [_F, C.c_int, _F, _F]
        lib.orc_head_row_bytes.argtypes = [C.c_int, C.c_int]
        lib.orc_head_row_bytes.restype = C.c_long
        lib.orc_dequant_row.argtypes = [C.c_int, C.c_void_p, _F, C.c_int]
        lib.orc_head_gemv.argtypes = [C.c_int, C.c_void_p, _F, C.c_int, C.c_int, C.c_int, _F,
                                      C.c_int]

    def router_topk(self, logits, n_used, norm_topk):
        """forward_cpu.c:165-172, 296-304 on each row of `logits` (tokens x experts):
        (idx, wt), each tokens x n_used."""
        a = np.ascontiguousarray(logits, dtype=np.float32)
        t, e = a.shape
        idx = np.zeros((t, n_used), dtype=np.int32)
        wt = np.zeros((t, n_used), dtype=np.float32)
        self.lib.orc_router_topk(_fptr(a), e, t, e, n_used, 1 if norm_topk else 0, _iptr(idx),
                                 _fptr(wt))
        return idx, wt

    def router_probs(self, x):
        """(p, the float sum of the numerators) of one row's softmax (forward_cpu.c:165-172)."""
        a = np.ascontiguousarray(x, dtype=np.float32)
        p = np.zeros(a.size, dtype=np.float32)
        sm = np.zeros(1, dtype=np.float32)
        self.lib.orc_router_probs(_fptr(a), a.size, _fptr(p), _fptr(sm))
        return p, sm[0]

    def head_row_bytes(self, wtype, n):
        return int(self.lib.orc_head_row_bytes(wtype, n))

    def dequant_row(self, wtype, src, n):
        """quasar_dequant_row restated (quant.c): n floats from the bytes of one row."""
        b = np.ascontiguousarray(src, dtype=np.uint8)
        out = np.zeros(n, dtype=np.float32)
        self.lib.orc_dequant_row(wtype, b.ctypes.data, _fptr(out), n)
        return out

    def head_gemv(self, wtype, w_bytes, x, V, n_threads=8):
        """forward_cpu.c:140-147: logits [nx][V] from V GGUF rows of `wtype` and x [nx][E]."""
        xb = np.ascontiguousarray(x, dtype=np.float32)
        nx, E = xb.shape
        wb = np.ascontiguousarray(w_bytes, dtype=np.uint8)
        assert wb.size >= V * self.head_row_bytes(wtype, E)
        y = np.zeros((nx, V), dtype=np.float32)
        self.lib.orc_head_gemv(wtype, wb.ctypes.data, _fptr(xb), nx, E, V, _fptr(y), n_threads)
        return y

    def pick_rows_diag(self, params, logits, n_rows, n_vocab, hist, seeds, n_threads=1):
        """orc_pick_rows_diag: (ids, diag records (DIAG_DTYPE), seconds)."""
        logits = np.asarray(logits, dtype=np.float32)
        assert logits.flags.c_contiguous and logits.ndim == 2 and logits.shape[0] >= n_rows
        seeds = np.ascontiguousarray(seeds, dtype=np.uint64)
        if hist is None:
            hist = np.zeros((n_rows, 0), dtype=np.int32)
        hist = np.ascontiguousarray(hist, dtype=np.int32)
        out = np.zeros(n_rows, dtype=np.int32)
        diag = np.zeros(n_rows, dtype=DIAG_DTYPE)
        secs = self.lib.orc_pick_rows_diag(
            C.byref(params), _fptr(logits), logits.shape[1], n_rows, n_vocab, _iptr(hist),
            hist.shape[1] if hist.ndim == 2 else 0, _uptr(seeds), _iptr(out),
            diag.ctypes.data_as(C.c_void_p), n_threads)
        return out, diag, secs

    def sampler(self):
        s = _SamplerBase(self.lib, "orc_sampler_", "orc_sampler_")
        s._fail = self.lib.orc_sampler_fail_scratch
        lib = self.lib

        def pick_diag(logits):
            a = np.ascontiguousarray(logits, dtype=np.float32)
            d = Diag()
            lib.orc_sampler_pick_diag(s._s, _fptr(a), a.size, C.byref(d))
            return d.id, d.as_dict()
        s.pick_diag = pick_diag
        return s

    def pick_rows(self, params, logits, n_rows, n_vocab, hist, seeds, n_threads=1):
        return _pick_rows(self.lib.orc_pick_rows, params, logits, n_rows, n_vocab, hist, seeds,
                          n_threads)

    def xorshift64(self, state):
        st = np.array([state], dtype=np.uint64)
        out = self.lib.orc_xorshift64(_uptr(st))
        return out, int(st[0])

    def rng_unit(self, state):
        st = np.array([state], dtype=np.uint64)
        u = self.lib.orc_rng_unit(_uptr(st))
        return u, int(st[0])

    def gen_logits(self, dist, sigma, boost, seed, row0, n_rows, n_vocab):
        out = np.empty((n_rows, n_vocab), dtype=np.float32)
        self.lib.orc_gen_logits(dist, sigma, boost, seed, row0, n_rows, n_vocab, _fptr(out),
                                n_vocab)
        return out

    def gen_hist(self, seed, row0, n_rows, hist_n, n_vocab, pool=0):
        out = np.empty((n_rows, hist_n), dtype=np.int32)
        self.lib.orc_gen_hist(seed, row0, n_rows, hist_n, n_vocab, pool, _iptr(out))
        return out

    def gen_row_seeds(self, seed, row0, n_rows):
        return np.array([self.lib.orc_gen_row_seed(seed, row0 + r) for r in range(n_rows)],
                        dtype=np.uint64)

    def product_expf(self, x):
        return self.lib.orc_product_expf(float(x))

    def libm_expf(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty_like(x)
        self.lib.orc_libm_expf_array(_fptr(x), _fptr(y), x.size)
        return y

    def check_expf_range(self, lo, hi, n_threads=8):
        return self.lib.orc_check_expf_range(lo, hi, n_threads)


class RefSampler:
    """The reference's own sample.c built into oracle/_ref (see oracle/Makefile)."""

    def __init__(self, path=REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (needs the reference source)")
        self.lib = lib = C.CDLL(path)
        _sampler_protos(lib, "quasar_sampler_")
        _hook_protos(lib, "ref_")
        _rows_protos(lib.ref_pick_rows)

    @staticmethod
    def available(path=REF_SO):
        return os.path.exists(path)

    def sampler(self):
        s = _SamplerBase(self.lib, "quasar_sampler_", "ref_")
        fail = self.lib.ref_fail_allocs
        fail.argtypes = [C.c_int]
        s._fail = lambda _s, on: fail(on)      # process-wide in the reference's build
        return s

    def pick_rows(self, params, logits, n_rows, n_vocab, hist, seeds, n_threads=1):
        return _pick_rows(self.lib.ref_pick_rows, params, logits, n_rows, n_vocab, hist, seeds,
                          n_threads)


BOUNDARY_TOL = 1e-6     # a draw this close to a CDF boundary may pick the neighbour
PATH_CERT = 4           # qs_pick_diag.path of rows decided over a proven interval


def parity_report(gpu_ids, gpu_diag, orc_ids, orc_diag):
    """Compare one pick of many rows: the product's ids and qs_pick_diag records against
    the restatement's ids and DIAG_DTYPE records.  Returns counts:
      rows, id_mismatches, boundary_rows (draws within BOUNDARY_TOL of a CDF boundary),
      unexplained (mismatches on rows that are not boundary rows: must be 0),
      inv_outside (rows whose reference normaliser lies outside the GPU's: proven interval
      for certified rows, the exact value otherwise), keep_mismatches (kept prefix length),
      and the rows per decision path."""
    gpu_ids = np.asarray(gpu_ids)
    n = len(gpu_ids)
    mism = gpu_ids[:n] != orc_ids[:n]
    sampled = orc_diag["greedy"][:n] == 0
    boundary = sampled & (orc_diag["bdist"][:n] < BOUNDARY_TOL)
    inv_out = keep_mis = 0
    paths = {}
    for r in range(n):
        d = gpu_diag[r]
        paths[int(d.path)] = paths.get(int(d.path), 0) + 1
        if not sampled[r]:
            continue
        o = orc_diag[r]
        if d.path == PATH_CERT:
            if not (np.float32(d.inv) <= np.float32(o["inv"]) <= np.float32(d.inv_hi)):
                inv_out += 1
        elif np.float32(d.inv).view(np.uint32) != np.float32(o["inv"]).view(np.uint32):
            inv_out += 1
        if int(d.keep) != int(o["keep"]):
            keep_mis += 1
    return {"rows": int(n), "id_mismatches": int(mism.sum()),
            "boundary_rows": int(boundary.sum()), "unexplained": int((mism & ~boundary).sum()),
            "inv_outside": int(inv_out), "keep_mismatches": int(keep_mis),
            "paths": {str(k): v for k, v in sorted(paths.items())}}


REF_QUANT_SO = os.path.join(os.path.dirname(REF_SO), "libref_quant.so")


class RefQuant:
    """The reference's own quant.c built into oracle/_ref (quasar_dequant_row)."""

    def __init__(self, path=REF_QUANT_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (needs the reference source)")
        self.lib = C.CDLL(path)
        self.lib.quasar_dequant_row.argtypes = [C.c_uint32, C.c_void_p, _F, C.c_int]
        self.lib.q_fp16_to_fp32.argtypes = [C.c_uint16]
        self.lib.q_fp16_to_fp32.restype = C.c_float

    @staticmethod
    def available(path=REF_QUANT_SO):
        return os.path.exists(path)

    def dequant_row(self, wtype, src, n):
        b = np.ascontiguousarray(src, dtype=np.uint8)
        out = np.zeros(n, dtype=np.float32)
        self.lib.quasar_dequant_row(wtype, b.ctypes.data, _fptr(out), n)
        return out
