"""The measurement aids bench.py reports beside a pick: the row kernel's loads alone
(qs_time_row_reads)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def qa():
    import quasar_amd
    quasar_amd.load()
    return quasar_amd


def test_row_reads_time_and_write_nothing(qa):
    """Rows of the headline's width read at the row kernel's shape: a positive time, no
    write to the sink (it keeps its sentinel), and QS_EINVAL for inputs the row kernel does
    not take (a misaligned row pointer, a vocabulary not a multiple of 4)."""
    B, V = 8, 151936
    rng = np.random.default_rng(3)
    x = rng.normal(0, 2, (B, V)).astype(np.float32)
    buf = qa.DeviceBuffer.from_array(x)
    sink = qa.DeviceBuffer.from_array(np.full(B, 7.0, dtype=np.float32))
    lib = qa.load()
    ms = C.c_float(0)
    arr = (C.c_void_p * 1)(buf.ptr)
    assert lib.qs_time_row_reads(arr, 1, V, B, V, sink.ptr, 20, C.byref(ms)) == 0
    assert ms.value > 0.0
    assert (sink.download(np.float32, B) == 7.0).all()
    bad = (C.c_void_p * 1)(buf.ptr + 4)
    assert lib.qs_time_row_reads(bad, 1, V, B, V, sink.ptr, 1, C.byref(ms)) == qa._native.QS_EINVAL
    assert lib.qs_time_row_reads(arr, 1, V, B, V - 2, sink.ptr, 1, C.byref(ms)) == qa._native.QS_EINVAL
    assert qa.time_row_reads([buf.ptr], V, B, V, 5) > 0.0
    sink.free()
    buf.free()
