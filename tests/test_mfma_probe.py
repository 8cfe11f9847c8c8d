"""The matrix-core ceiling probe bench.py reports beside the published peak
(lib/libkvpprobe.so, measurement only)."""

import ctypes
from pathlib import Path

import pytest

LIB = Path(__file__).resolve().parent.parent / "cuda-kv-persistence_amd" / "lib" / "libkvpprobe.so"
PEAK = 2516.6  # MI355X dense bf16 TFLOP/s


def _probe():
    lib = ctypes.CDLL(str(LIB))
    fn = lib.kvpprobe_mfma_bf16
    fn.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                   ctypes.POINTER(ctypes.c_double)]
    fn.restype = ctypes.c_int
    return fn


def test_probe_library_loads_and_exports_its_entry_point():
    assert LIB.exists(), "build first (make -C cuda-kv-persistence_amd)"
    _probe()


def test_probe_rejects_bad_arguments():
    fn = _probe()
    tf, ms = ctypes.c_double(), ctypes.c_double()
    assert fn(0, 1, ctypes.byref(tf), ctypes.byref(ms)) != 0
    assert fn(10, 0, ctypes.byref(tf), ctypes.byref(ms)) != 0
    assert fn(10, 1, None, ctypes.byref(ms)) != 0


@pytest.mark.gpu
def test_probe_rate_is_positive_and_below_the_published_peak():
    import torch
    torch.cuda.init()
    fn = _probe()
    tf, ms = ctypes.c_double(), ctypes.c_double()
    assert fn(4000, 3, ctypes.byref(tf), ctypes.byref(ms)) == 0
    assert ms.value > 0.0
    assert 0.2 * PEAK < tf.value <= 1.02 * PEAK
