"""quasar_amd - the reference token sampler (sample.c) on MI355X.

Python mirror of the C ABI in include/quasar_sampler.h:

* ``Sampler``  - the reference's five-function API (sample.h:14-29): ``config``,
                 ``reset``, ``pick`` on host logits, one token per call.
* ``Batch``    - the device-resident extension: B rows of device logits picked in one
                 enqueue, generator states and histories kept on the device.
* ``DeviceBuffer``, ``gen_logits_device`` - plumbing for tests and the benchmark.

Every pick runs the HIP kernels of quasar_amd/csrc/qs_batch.hip; importing the package
does not load the library, using any of these classes does (and fails loudly if it has
not been built).
"""
import ctypes as C

import numpy as np

from . import _native
from ._native import (MODE_AUTO, MODE_ROW, MODE_SPLIT, MODE_STREAM, PATH_CERT, PATH_EMPTY, PATH_FAST,
                      PATH_FULL, PATH_GREEDY, QS_EAGAIN, WTYPE_F16, WTYPE_F32, WTYPE_Q6_K,
                      WTYPE_Q8_0, PickDiag, QsError, check, load)

__all__ = ["Sampler", "Batch", "DeviceBuffer", "gen_logits_device", "device_info",
           "head_exact_packed_bytes", "WTYPE_F32", "WTYPE_F16", "WTYPE_Q8_0", "WTYPE_Q6_K",
           "PickDiag", "QsError", "PATH_GREEDY", "PATH_FAST", "PATH_FULL", "PATH_EMPTY",
           "PATH_CERT", "MODE_AUTO", "MODE_SPLIT", "MODE_STREAM", "MODE_ROW", "gen_row_seeds", "gen_history", "QS_EAGAIN"]


class DeviceBuffer:
    """A device allocation (qs_device_alloc) with numpy upload/download."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = load().qs_device_alloc(self.nbytes)
        if not self.ptr:
            raise QsError("qs_device_alloc(%d) failed: %s"
                          % (self.nbytes, load().qs_last_error().decode()))

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a, offset=0):
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        check(load().qs_memcpy_h2d(self.ptr + offset, a.ctypes.data, a.nbytes), "h2d")

    def download(self, dtype, count, offset=0):
        out = np.empty(count, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        check(load().qs_memcpy_d2h(out.ctypes.data, self.ptr + offset, out.nbytes), "d2h")
        return out

    def free(self):
        if self.ptr:
            load().qs_device_free(self.ptr)
            self.ptr = None

    __del__ = free


def gen_logits_device(buf, row_stride, row0, n_rows, n_vocab, dist, sigma, boost, seed,
                      offset_rows=0):
    """Fill rows [row0, row0+n_rows) of a workload distribution into `buf` on the GPU."""
    check(load().qs_gen_logits_device(buf.ptr + 4 * offset_rows * row_stride, row_stride,
                                      row0, n_rows, n_vocab, dist, sigma, boost, seed),
          "qs_gen_logits_device")


def gen_row_seeds(seed, row0, n_rows):
    """The synthetic workloads' sampler seeds of rows [row0, row0 + n_rows) (uint64)."""
    out = np.zeros(n_rows, dtype=np.uint64)
    check(load().qs_gen_row_seeds(seed, row0, n_rows,
                                  out.ctypes.data_as(C.POINTER(C.c_uint64))), "qs_gen_row_seeds")
    return out


def gen_history(seed, row0, n_rows, hist_n, n_vocab, pool=0):
    """The synthetic workloads' history ids of rows [row0, row0 + n_rows): int32 [n_rows,
    hist_n], oldest first."""
    out = np.zeros((n_rows, hist_n), dtype=np.int32)
    check(load().qs_gen_history(seed, row0, n_rows, hist_n, n_vocab, pool,
                                out.ctypes.data_as(C.POINTER(C.c_int32))), "qs_gen_history")
    return out


def router_topk(logits, n_tokens, n_expert, n_used, norm_topk, idx, wt, row_stride=None):
    """The mixture-of-experts router's choice (qs_router_topk) for n_tokens rows of router
    logits in DeviceBuffer `logits`; slots into DeviceBuffers `idx` (int32) and `wt`
    (float32), n_used per token.  Waits for the device."""
    lib = load()
    check(lib.qs_router_topk(logits.ptr, row_stride or n_expert, n_tokens, n_expert, n_used,
                             1 if norm_topk else 0, idx.ptr, wt.ptr, None), "qs_router_topk")
    check(lib.qs_device_synchronize(), "qs_device_synchronize")


def router_time(logits, n_tokens, n_expert, n_used, norm_topk, idx, wt, iters):
    """Milliseconds for `iters` back-to-back router_topk calls (qs_router_time)."""
    ms = C.c_float()
    check(load().qs_router_time(logits.ptr, n_expert, n_tokens, n_expert, n_used,
                                1 if norm_topk else 0, idx.ptr, wt.ptr, iters, C.byref(ms)),
          "qs_router_time")
    return ms.value


def time_row_reads(logits_ptrs, row_stride, n_rows, n_vocab, iters):
    """The row pick's loads alone (qs_time_row_reads): `iters` launches of a kernel with the
    row kernel's launch shape, chunks and loads that only adds up the rows, launch i reading
    logits_ptrs[i % len].  Returns the elapsed milliseconds of all launches."""
    if isinstance(logits_ptrs, int):
        logits_ptrs = [logits_ptrs]
    arr = (C.c_void_p * len(logits_ptrs))(*logits_ptrs)
    sink = DeviceBuffer(4 * n_rows)
    ms = C.c_float(0)
    try:
        check(load().qs_time_row_reads(arr, len(logits_ptrs), row_stride, n_rows, n_vocab,
                                       sink.ptr, iters, C.byref(ms)), "qs_time_row_reads")
    finally:
        sink.free()
    return ms.value


def copy_device(dst, src, nbytes, iters=1, kind=0):
    """`iters` streaming copies of nbytes from src to dst (DeviceBuffers): a kernel of known
    memory traffic for calibrating hardware counters; kind 0 plain 16-byte loads, 1
    nontemporal raw buffer loads, 2 buffer loads into LDS, 3 plain 4-byte loads
    (qs_copy_device_kind)."""
    check(load().qs_copy_device_kind(dst.ptr, src.ptr, nbytes, iters, kind),
          "qs_copy_device_kind")


def head_packed_bytes(n_embd, n_vocab):
    """Bytes of the packed output matrix (qs_head_packed_bytes; 0 for sizes not taken)."""
    return int(load().qs_head_packed_bytes(n_embd, n_vocab))


def head_exact_packed_bytes(wtype, n_embd, n_vocab):
    """Bytes of the exact output layer's packed matrix (qs_head_exact_packed_bytes; 0 for a
    type or size not taken)."""
    return int(load().qs_head_exact_packed_bytes(wtype, n_embd, n_vocab))


def device_info():
    name = C.create_string_buffer(256)
    mem = C.c_size_t(0)
    ncu = C.c_int(0)
    check(load().qs_device_info(name, 256, C.byref(mem), C.byref(ncu)), "qs_device_info")
    return name.value.decode(), mem.value, ncu.value


class Sampler:
    """sample.h on the GPU: one quasar_sampler (host logits in, one id out)."""

    def __init__(self):
        self._lib = load()
        self._s = self._lib.quasar_sampler_new()
        if not self._s:
            raise MemoryError("quasar_sampler_new returned NULL")

    def close(self):
        if getattr(self, "_s", None):
            self._lib.quasar_sampler_free(self._s)
            self._s = None

    __del__ = close

    def config(self, temperature=0.0, top_p=1.0, top_k=0, min_p=0.0, repeat_penalty=1.0,
               repeat_last_n=0, seed=1):
        self._lib.quasar_sampler_config(self._s, temperature, top_p, int(top_k), min_p,
                                        repeat_penalty, int(repeat_last_n),
                                        int(seed) & 0xFFFFFFFFFFFFFFFF)

    def reset(self):
        self._lib.quasar_sampler_reset(self._s)

    def pick(self, logits):
        a = np.ascontiguousarray(logits, dtype=np.float32)
        return self._lib.quasar_sampler_pick(self._s, a.ctypes.data_as(C.POINTER(C.c_float)),
                                             a.size)

    def get_state(self, cap=4096):
        """(generator state, history oldest first) through qs_sampler_get_state."""
        rng = C.c_uint64()
        h = np.zeros(max(1, cap), dtype=np.int32)
        n = C.c_int()
        check(self._lib.qs_sampler_get_state(self._s, C.byref(rng),
                                             h.ctypes.data_as(C.POINTER(C.c_int32)), cap,
                                             C.byref(n)), "qs_sampler_get_state")
        return rng.value, h[:n.value].copy()


def fail_picks(n):
    """The next n quasar_sampler_pick calls find the device unavailable (tests)."""
    check(load().qs_debug_fail_picks(int(n)), "qs_debug_fail_picks")


class Batch:
    """qs_batch: rows of device logits picked together, state on the device."""

    def __init__(self, max_rows, max_vocab, max_last_n=0):
        self._lib = load()
        self.max_rows, self.max_vocab, self.max_last_n = max_rows, max_vocab, max_last_n
        self._b = self._lib.qs_batch_new(max_rows, max_vocab, max_last_n)
        if not self._b:
            raise QsError("qs_batch_new failed: " + self._lib.qs_last_error().decode())
        self._out = DeviceBuffer(4 * max_rows)
        self._diag = DeviceBuffer(C.sizeof(PickDiag) * max_rows)

    def close(self):
        if getattr(self, "_b", None):
            self._lib.qs_batch_free(self._b)
            self._b = None

    __del__ = close

    def config(self, row0, n_rows, temperature=0.0, top_p=1.0, top_k=0, min_p=0.0,
               repeat_penalty=1.0, repeat_last_n=0, seeds=None):
        sp = None
        if seeds is not None:
            seeds = np.ascontiguousarray(np.asarray(seeds, dtype=np.uint64).reshape(-1))
            assert seeds.size == n_rows
            sp = seeds.ctypes.data_as(C.POINTER(C.c_uint64))
        check(self._lib.qs_batch_config(self._b, row0, n_rows, temperature, top_p, int(top_k),
                                        min_p, repeat_penalty, int(repeat_last_n), sp),
              "qs_batch_config")

    def reset(self, row0, n_rows):
        check(self._lib.qs_batch_reset(self._b, row0, n_rows), "qs_batch_reset")

    def set_mode(self, mode):
        """MODE_AUTO, MODE_SPLIT (split-row kernels) or MODE_STREAM (the streaming kernel
        and the per-row decision kernel); see quasar_sampler.h."""
        check(self._lib.qs_batch_set_mode(self._b, int(mode)), "qs_batch_set_mode")

    def resolve_mode(self, logits_ptr, row_stride, n_rows, n_vocab):
        """The mode (MODE_SPLIT or MODE_STREAM) a pick with these arguments uses."""
        m = self._lib.qs_batch_resolve_mode(self._b, logits_ptr, row_stride, n_rows, n_vocab)
        check(m if m < 0 else 0, "qs_batch_resolve_mode")
        return m

    def set_history(self, row0, ids):
        ids = np.ascontiguousarray(np.asarray(ids, dtype=np.int32))
        if ids.ndim == 1:
            ids = ids.reshape(1, -1)
        n_rows, n = ids.shape
        check(self._lib.qs_batch_set_history(self._b, row0, n_rows,
                                             ids.ctypes.data_as(C.POINTER(C.c_int32)), n),
              "qs_batch_set_history")

    def set_state(self, row, rng, hist):
        h = np.ascontiguousarray(np.asarray(hist, dtype=np.int32).reshape(-1))
        check(self._lib.qs_batch_set_state(self._b, row, int(rng) & 0xFFFFFFFFFFFFFFFF,
                                           h.ctypes.data_as(C.POINTER(C.c_int32)), h.size),
              "qs_batch_set_state")

    def get_state(self, row):
        cap = max(1, self.max_last_n)
        hist = np.zeros(cap, dtype=np.int32)
        rng = C.c_uint64(0)
        n = C.c_int(0)
        check(self._lib.qs_batch_get_state(self._b, row, C.byref(rng),
                                           hist.ctypes.data_as(C.POINTER(C.c_int32)), cap,
                                           C.byref(n)),
              "qs_batch_get_state")
        return int(rng.value), hist[:n.value].copy()

    def pick_async(self, logits_ptr, row_stride, n_rows, n_vocab, diag=False):
        check(self._lib.qs_batch_pick(self._b, logits_ptr, row_stride, n_rows, n_vocab,
                                      self._out.ptr, self._diag.ptr if diag else None),
              "qs_batch_pick")

    def pick(self, logits_ptr, row_stride, n_rows, n_vocab, diag=False):
        """Pick rows [0, n_rows); returns ids (and a list of PickDiag when diag)."""
        self.pick_async(logits_ptr, row_stride, n_rows, n_vocab, diag)
        self.synchronize()
        ids = self._out.download(np.int32, n_rows)
        if not diag:
            return ids
        raw = self._diag.download(np.uint8, C.sizeof(PickDiag) * n_rows)
        d = (PickDiag * n_rows).from_buffer_copy(raw.tobytes())
        return ids, list(d)

    def pick_rows(self, row0, logits_ptr, row_stride, n_rows, n_vocab, diag=False):
        """Pick the batch's rows [row0, row0 + n_rows) from logits rows 0 .. n_rows - 1
        (qs_batch_pick_rows); returns ids (and a list of PickDiag when diag)."""
        check(self._lib.qs_batch_pick_rows(self._b, row0, logits_ptr, row_stride, n_rows,
                                           n_vocab, self._out.ptr,
                                           self._diag.ptr if diag else None),
              "qs_batch_pick_rows")
        self.synchronize()
        ids = self._out.download(np.int32, n_rows)
        if not diag:
            return ids
        raw = self._diag.download(np.uint8, C.sizeof(PickDiag) * n_rows)
        return ids, list((PickDiag * n_rows).from_buffer_copy(raw.tobytes()))

    def synchronize(self):
        check(self._lib.qs_batch_synchronize(self._b), "qs_batch_synchronize")

    def set_sum_in_order(self, always):
        """Exact-path rows sum their denominator in id order always (1) or where needed (0)
        (qs_batch_set_sum_in_order)."""
        check(self._lib.qs_batch_set_sum_in_order(self._b, int(always)),
              "qs_batch_set_sum_in_order")

    def set_spin_limit(self, attempts):
        """Attempts a row makes at a whole-window scratch slot (qs_batch_set_spin_limit)."""
        check(self._lib.qs_batch_set_spin_limit(self._b, int(attempts)),
              "qs_batch_set_spin_limit")

    def time_stream_kernel(self, logits_ptrs, row_stride, n_rows, n_vocab, iters):
        """Milliseconds of the pick's dominant kernel summed over `iters` picks: each timed
        from an event before the pick to one between its two kernels (the streaming
        kernels) or after it (the row kernel, the whole pick)."""
        if isinstance(logits_ptrs, int):
            logits_ptrs = [logits_ptrs]
        arr = (C.c_void_p * len(logits_ptrs))(*logits_ptrs)
        ms = C.c_float()
        check(self._lib.qs_batch_time_kernels(self._b, arr, len(logits_ptrs), row_stride,
                                              n_rows, n_vocab, self._out.ptr, iters,
                                              C.byref(ms)), "qs_batch_time_kernels")
        return ms.value

    def head_pack(self, weight_ptr, n_embd, n_vocab, packed_ptr):
        """The output matrix into the output layer's tile order (qs_batch_head_pack),
        asynchronous; packed_ptr holds head_packed_bytes(n_embd, n_vocab) bytes."""
        check(self._lib.qs_batch_head_pack(self._b, weight_ptr, n_embd, n_vocab, packed_ptr),
              "qs_batch_head_pack")

    def head_logits(self, hidden_ptr, weight_ptr, n_embd, n_rows, n_vocab, logits_ptr):
        """The output layer alone (qs_batch_head_logits), asynchronous."""
        check(self._lib.qs_batch_head_logits(self._b, hidden_ptr, weight_ptr, n_embd, n_rows,
                                             n_vocab, logits_ptr), "qs_batch_head_logits")

    def pick_head(self, hidden_ptr, weight_ptr, n_embd, n_rows, n_vocab, logits_ptr,
                  diag=False):
        """The output layer and the pick of rows [0, n_rows) (qs_batch_pick_head); returns
        ids (and a list of PickDiag when diag)."""
        check(self._lib.qs_batch_pick_head(self._b, hidden_ptr, weight_ptr, n_embd, n_rows,
                                           n_vocab, logits_ptr, self._out.ptr,
                                           self._diag.ptr if diag else None),
              "qs_batch_pick_head")
        self.synchronize()
        ids = self._out.download(np.int32, n_rows)
        if not diag:
            return ids
        raw = self._diag.download(np.uint8, C.sizeof(PickDiag) * n_rows)
        return ids, list((PickDiag * n_rows).from_buffer_copy(raw.tobytes()))

    def time_head(self, hidden_ptr, weight_ptr, n_embd, n_rows, n_vocab, logits_ptr, iters,
                  fused):
        """Milliseconds of `iters` output-layer calls (qs_batch_time_head): fused picks
        (fused=True or 1), the layer then a pick (False or 0), the layer alone (2)."""
        ms = C.c_float(0)
        check(self._lib.qs_batch_time_head(self._b, hidden_ptr, weight_ptr, n_embd, n_rows,
                                           n_vocab, logits_ptr, self._out.ptr, iters,
                                           int(fused), C.byref(ms)),
              "qs_batch_time_head")
        return ms.value

    def head_exact_pack(self, wtype, weight_ptr, n_embd, n_vocab, packed_ptr):
        """The GGUF output matrix (rows of type wtype) into the exact output layer's layout
        (qs_batch_head_exact_pack), asynchronous; packed_ptr holds
        head_exact_packed_bytes(wtype, n_embd, n_vocab) bytes."""
        check(self._lib.qs_batch_head_exact_pack(self._b, wtype, weight_ptr, n_embd, n_vocab,
                                                 packed_ptr), "qs_batch_head_exact_pack")

    def head_exact_logits(self, wtype, packed_ptr, xn_ptr, n_embd, n_rows, n_vocab,
                          logits_ptr):
        """The output layer at the reference's arithmetic alone (qs_batch_head_exact_logits),
        asynchronous."""
        check(self._lib.qs_batch_head_exact_logits(self._b, wtype, packed_ptr, xn_ptr, n_embd,
                                                   n_rows, n_vocab, logits_ptr),
              "qs_batch_head_exact_logits")

    def pick_head_exact(self, wtype, packed_ptr, xn_ptr, n_embd, n_rows, n_vocab, logits_ptr,
                        diag=False):
        """That output layer and the pick of rows [0, n_rows) (qs_batch_pick_head_exact);
        returns ids (and a list of PickDiag when diag)."""
        check(self._lib.qs_batch_pick_head_exact(self._b, wtype, packed_ptr, xn_ptr, n_embd,
                                                 n_rows, n_vocab, logits_ptr, self._out.ptr,
                                                 self._diag.ptr if diag else None),
              "qs_batch_pick_head_exact")
        self.synchronize()
        ids = self._out.download(np.int32, n_rows)
        if not diag:
            return ids
        raw = self._diag.download(np.uint8, C.sizeof(PickDiag) * n_rows)
        return ids, list((PickDiag * n_rows).from_buffer_copy(raw.tobytes()))

    def time_head_exact(self, wtype, packed_ptr, xn_ptr, n_embd, n_rows, n_vocab, logits_ptr,
                        iters, fused):
        """Milliseconds of `iters` calls (qs_batch_time_head_exact): fused picks (1), the
        layer then a pick (0), the layer alone (2)."""
        ms = C.c_float(0)
        check(self._lib.qs_batch_time_head_exact(self._b, wtype, packed_ptr, xn_ptr, n_embd,
                                                 n_rows, n_vocab, logits_ptr, self._out.ptr,
                                                 iters, int(fused), C.byref(ms)),
              "qs_batch_time_head_exact")
        return ms.value

    def time_picks(self, logits_ptrs, row_stride, n_rows, n_vocab, iters):
        """Time `iters` picks on the batch's stream; pick i reads logits_ptrs[i % len]
        (a single pointer is allowed).  Returns milliseconds."""
        if isinstance(logits_ptrs, int):
            logits_ptrs = [logits_ptrs]
        arr = (C.c_void_p * len(logits_ptrs))(*logits_ptrs)
        ms = C.c_float(0)
        check(self._lib.qs_batch_time_picks(self._b, arr, len(logits_ptrs), row_stride, n_rows,
                                            n_vocab, self._out.ptr, iters, C.byref(ms)),
              "qs_batch_time_picks")
        return ms.value

    @property
    def stream(self):
        return self._lib.qs_batch_stream(self._b)
