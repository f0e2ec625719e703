"""The calibration library (libmi_calib.so, the copy ceilings bench.py reads the bandwidth kernels
against) loads without a GPU, describes its launch shapes, and rejects on the host every launch
its kernels could not run in bounds -- in particular the copies to or from scattered 32 KiB
units, which need a power-of-two number of whole units (no GPU call is made here)."""

import ctypes
from pathlib import Path

import pytest

LIB = Path(__file__).resolve().parents[1] / "mini_infra_qwen3_amd" / "libmi_calib.so"


@pytest.fixture(scope="module")
def calib():
    if not LIB.exists():
        pytest.skip("libmi_calib.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(str(LIB))
    lib.calib_num_variants.restype = ctypes.c_int32
    lib.calib_variant.argtypes = [ctypes.c_int32, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32),
                                  ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int32)]
    lib.calib_variant.restype = ctypes.c_int32
    lib.calib_groups.argtypes = [ctypes.c_int64, ctypes.c_int32]
    lib.calib_groups.restype = ctypes.c_int64
    lib.calib_stream.argtypes = [ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                 ctypes.c_int32, ctypes.c_void_p]
    lib.calib_stream.restype = ctypes.c_int32
    return lib


def variants(lib):
    out = []
    for v in range(lib.calib_num_variants()):
        t, f, sp, st = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64(), ctypes.c_int32()
        assert lib.calib_variant(v, ctypes.byref(t), ctypes.byref(f), ctypes.byref(sp), ctypes.byref(st)) == 0
        out.append((t.value, f.value, sp.value, st.value))
    return out


def test_launch_shapes(calib):
    shapes = variants(calib)
    assert len(shapes) == 27
    for threads, in_flight, span, stream in shapes:
        assert threads in (64, 128, 256, 512, 1024) and in_flight in (1, 2, 4, 8)
        assert span % (16 * threads) == 0 and span & (span - 1) == 0  # whole 16-byte pieces, power of two
        assert stream in (0, 1)
    assert sum(st for *_, st in shapes) == 7  # streaming-store forms
    bad = ctypes.c_int32()
    assert calib.calib_variant(27, ctypes.byref(bad), ctypes.byref(bad), ctypes.byref(ctypes.c_int64()),
                               ctypes.byref(bad)) == -1


def test_groups(calib):
    shapes = variants(calib)
    for v, (_, _, span, _) in enumerate(shapes):
        assert calib.calib_groups(2 << 30, v) == (2 << 30) // span
    assert calib.calib_groups(0, 0) == -1  # empty
    assert calib.calib_groups(100, 0) == -1  # not whole 16-byte pieces
    assert calib.calib_groups(1 << 20, -1) == -1


def test_stream_rejects_before_any_device_call(calib):
    dummy = 1 << 12  # aligned, never dereferenced: every call below fails its host checks
    shapes = variants(calib)
    small = next(v for v, s in enumerate(shapes) if s[2] <= 32 << 10)
    large = next(v for v, s in enumerate(shapes) if s[2] > 32 << 10)
    cases = [
        (5, dummy, dummy, dummy, 2 << 30, small),           # unknown shape
        (0, None, dummy, dummy, 2 << 30, small),            # copy without destination
        (1, dummy, dummy, None, 2 << 30, small),            # read without sink
        (0, dummy + 8, dummy, dummy, 2 << 30, small),       # misaligned
        (3, dummy, dummy, dummy, 3 * (32 << 10), small),    # 3 units: not a power of two
        (4, dummy, dummy, dummy, (32 << 10) + 4096, small),  # not whole units
        (3, dummy, dummy, dummy, 2 << 30, large),           # spans larger than a unit
        (0, dummy, dummy, dummy, 2 << 30, 99),              # unknown variant
    ]
    for shape, dst, src, sink, nbytes, v in cases:
        assert calib.calib_stream(shape, dst, src, sink, nbytes, v, None) == -1, (shape, nbytes, v)
