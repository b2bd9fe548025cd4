"""ctypes binding of quasar_amd/lib/libquasar_sampler.so (include/quasar_sampler.h).

The library is the product: every pick runs on the GPU.  Loading fails loudly when the
library has not been built (``python -c "import __graft_entry__ as g; g.build()"`` or
``make -C quasar_amd/csrc``); there is no CPU fallback.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libquasar_sampler.so")

QS_EINVAL, QS_ENOMEM, QS_EDEVICE = -22, -12, -5
QS_EAGAIN = -11
PATH_GREEDY, PATH_FAST, PATH_FULL, PATH_EMPTY, PATH_CERT = 0, 1, 2, 3, 4
MODE_AUTO, MODE_SPLIT, MODE_STREAM, MODE_ROW = 0, 1, 2, 3
WTYPE_F32, WTYPE_F16, WTYPE_Q8_0, WTYPE_Q6_K = 0, 1, 8, 14   # GGUF tensor types
HEAD_EXACT_MAX_ROWS, HEAD_EXACT_MAX_EMBD = 8, 16384


class PickDiag(C.Structure):
    """qs_pick_diag."""
    _fields_ = [("id", C.c_int32), ("path", C.c_int32), ("n_window", C.c_int32),
                ("n_cand", C.c_int32), ("keep_topk", C.c_int32), ("keep_topp", C.c_int32),
                ("keep", C.c_int32), ("rank", C.c_int32), ("maxl", C.c_float),
                ("msc", C.c_float), ("inv", C.c_float), ("inv_hi", C.c_float),
                ("p0", C.c_float), ("fallback", C.c_int32), ("sum", C.c_double),
                ("sum_hi", C.c_double), ("rsum", C.c_double), ("u", C.c_double)]


# (name, restype, argtypes) for every function of include/quasar_sampler.h
_vp, _i, _i64, _u64, _f, _sz = C.c_void_p, C.c_int, C.c_int64, C.c_uint64, C.c_float, C.c_size_t
PROTOS = [
    ("quasar_sampler_new", _vp, []),
    ("quasar_sampler_free", None, [_vp]),
    ("quasar_sampler_config", None, [_vp, _f, _f, _i, _f, _f, _i, _u64]),
    ("quasar_sampler_reset", None, [_vp]),
    ("quasar_sampler_pick", _i, [_vp, C.POINTER(C.c_float), _i]),
    ("qs_sampler_get_state", _i, [_vp, C.POINTER(C.c_uint64), C.POINTER(C.c_int32), _i,
                                  C.POINTER(C.c_int)]),
    ("qs_debug_fail_picks", _i, [_i]),
    ("qs_batch_new", _vp, [_i, _i, _i]),
    ("qs_batch_free", None, [_vp]),
    ("qs_batch_config", _i, [_vp, _i, _i, _f, _f, _i, _f, _f, _i, C.POINTER(C.c_uint64)]),
    ("qs_batch_reset", _i, [_vp, _i, _i]),
    ("qs_batch_set_history", _i, [_vp, _i, _i, C.POINTER(C.c_int32), _i]),
    ("qs_batch_pick", _i, [_vp, _vp, _i64, _i, _i, _vp, _vp]),
    ("qs_batch_pick_rows", _i, [_vp, _i, _vp, _i64, _i, _i, _vp, _vp]),
    ("qs_batch_set_state", _i, [_vp, _i, _u64, C.POINTER(C.c_int32), _i]),
    ("qs_batch_set_mode", _i, [_vp, _i]),
    ("qs_batch_resolve_mode", _i, [_vp, _vp, _i64, _i, _i]),
    ("qs_batch_synchronize", _i, [_vp]),
    ("qs_batch_get_state", _i, [_vp, _i, C.POINTER(C.c_uint64), C.POINTER(C.c_int32), _i,
                                C.POINTER(C.c_int)]),
    ("qs_batch_stream", _vp, [_vp]),
    ("qs_row_config_set", None, [_vp, _f, _f, _i, _f, _f, _i]),
    ("qs_pick_noalloc", _i, [_vp, _i64, _i, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp]),
    ("qs_batch_set_spin_limit", _i, [_vp, _i]),
    ("qs_batch_set_sum_in_order", _i, [_vp, _i]),
    ("qs_last_error", C.c_char_p, []),
    ("qs_device_alloc", _vp, [_sz]),
    ("qs_device_free", None, [_vp]),
    ("qs_memcpy_h2d", _i, [_vp, _vp, _sz]),
    ("qs_memcpy_d2h", _i, [_vp, _vp, _sz]),
    ("qs_device_synchronize", _i, []),
    ("qs_device_info", _i, [C.c_char_p, _i, C.POINTER(C.c_size_t), C.POINTER(C.c_int)]),
    ("qs_gen_logits_device", _i, [_vp, _i64, _i64, _i, _i, _i, _f, _f, _u64]),
    ("qs_gen_row_seeds", _i, [_u64, _i64, _i, C.POINTER(C.c_uint64)]),
    ("qs_gen_history", _i, [_u64, _i64, _i, _i, _i, _i, C.POINTER(C.c_int32)]),
    ("qs_batch_time_picks", _i, [_vp, C.POINTER(_vp), _i, _i64, _i, _i, _vp, _i,
                                 C.POINTER(C.c_float)]),
    ("qs_batch_time_kernels", _i, [_vp, C.POINTER(_vp), _i, _i64, _i, _i, _vp, _i,
                                   C.POINTER(C.c_float)]),
    ("qs_timeline_read", _i, [_i, C.POINTER(C.c_uint64), _i]),
    ("qs_row_workgroups_per_cu", _i, [_i]),
    ("qs_expf_device", _i, [_vp, _vp, _i64]),
    ("qs_copy_device", _i, [_vp, _vp, _sz, _i]),
    ("qs_copy_device_kind", _i, [_vp, _vp, _sz, _i, _i]),
    ("qs_time_row_reads", _i, [C.POINTER(_vp), _i, _i64, _i, _i, _vp, _i, C.POINTER(C.c_float)]),
    ("qs_router_topk", _i, [_vp, _i64, _i, _i, _i, _i, _vp, _vp, _vp]),
    ("qs_router_time", _i, [_vp, _i64, _i, _i, _i, _i, _vp, _vp, _i, C.POINTER(C.c_float)]),
    ("qs_head_packed_bytes", _sz, [_i, _i]),
    ("qs_batch_head_pack", _i, [_vp, _vp, _i, _i, _vp]),
    ("qs_batch_head_logits", _i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    ("qs_batch_pick_head", _i, [_vp, _vp, _vp, _i, _i, _i, _vp, _vp, _vp]),
    ("qs_batch_time_head", _i, [_vp, _vp, _vp, _i, _i, _i, _vp, _vp, _i, _i,
                                C.POINTER(C.c_float)]),
    ("qs_head_exact_packed_bytes", _sz, [_i, _i, _i]),
    ("qs_batch_head_exact_pack", _i, [_vp, _i, _vp, _i, _i, _vp]),
    ("qs_batch_head_exact_logits", _i, [_vp, _i, _vp, _vp, _i, _i, _i, _vp]),
    ("qs_batch_pick_head_exact", _i, [_vp, _i, _vp, _vp, _i, _i, _i, _vp, _vp, _vp]),
    ("qs_batch_time_head_exact", _i, [_vp, _i, _vp, _vp, _i, _i, _i, _vp, _vp, _i, _i,
                                      C.POINTER(C.c_float)]),
]

_lib = None


def load(path=LIB_PATH):
    """Load the library once and declare every prototype; raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: the GPU sampler has not been built "
            "(run __graft_entry__.build() or `make -C quasar_amd/csrc`)")
    lib = C.CDLL(path)
    for name, res, args in PROTOS:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


class QsError(RuntimeError):
    """A failed library call; rc is its return code (QS_EINVAL, QS_EAGAIN, ...)."""

    def __init__(self, msg, rc=0):
        super().__init__(msg)
        self.rc = rc


def check(rc, what):
    if rc != 0:
        msg = load().qs_last_error().decode(errors="replace")
        raise QsError(f"{what} failed ({rc}): {msg}", rc)
