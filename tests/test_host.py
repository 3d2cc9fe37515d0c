"""CPU tests of the C++ host layer (include/qmm_host.h): the weight quantizers behind QTensor::quantize produce
the oracle's bytes, QTensor validates its shapes, and errors come back as messages.  No GPU calls."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
import qmm

_host = None


def host():
    global _host
    if _host is None:
        L = C.CDLL(qmm.HOST_LIB_PATH)
        vp, i64 = C.c_void_p, C.c_int64
        L.qmm_host_last_error.restype = C.c_char_p
        L.qmm_quantize_cpu.argtypes = [C.c_uint32, vp, i64, vp]
        L.qmm_dequantize_cpu.argtypes = [C.c_uint32, vp, i64, vp]
        L.qmm_qtensor_from_data.argtypes = [C.c_uint32, vp, i64, i64, i64, i64, C.c_int, C.POINTER(vp)]
        L.qmm_qtensor_quantize.argtypes = [C.c_uint32, vp, i64, i64, i64, C.c_int, C.POINTER(vp)]
        L.qmm_qtensor_free.argtypes = [vp]
        L.qmm_qtensor_storage_bytes.argtypes = [vp]
        L.qmm_qtensor_storage_bytes.restype = i64
        _host = L
    return _host


def quantize(gtype, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // O.BLOCK_SIZE[gtype] * O.TYPE_SIZE[gtype], dtype=np.uint8)
    assert host().qmm_quantize_cpu(gtype, x.ctypes.data, x.size, out.ctypes.data) == 0
    return out


@pytest.mark.parametrize("gtype", [O.Q8_0, O.Q4K, O.Q6K, O.Q8K, O.Q4_0, O.Q5_0, O.Q5K])
@pytest.mark.parametrize("sigma", [0.02, 1.0])
def test_host_quantizer_matches_the_oracle_bytes(gtype, sigma):
    rng = np.random.default_rng(31 + gtype)
    x = (rng.standard_normal((64, 2048)) * sigma).astype(np.float32)
    x[3, :256] = 0.0
    x[5, 17] = 40 * sigma
    assert np.array_equal(quantize(gtype, x), O.quantize(gtype, x).reshape(-1))


def test_host_f16_matches_numpy_through_q8_0_scales():
    rng = np.random.default_rng(32)
    x = (rng.standard_normal(32 * 4096) * 10.0 ** rng.integers(-7, 4, 32 * 4096)).astype(np.float32)
    q = O.blocks(O.Q8_0, quantize(O.Q8_0, x))
    amax = np.abs(x.reshape(-1, 32)).max(axis=1)
    want = (amax / np.float32(127.0)).astype(np.float32).astype(np.float16).view(np.uint16)
    assert np.array_equal(q["d"], want)


@pytest.mark.parametrize("gtype", [O.Q8_0, O.Q4K, O.Q6K, O.Q4_0, O.Q5_0, O.Q5K])
def test_host_dequantize_matches_the_oracle(gtype):
    rng = np.random.default_rng(33)
    x = (rng.standard_normal(4096) * 0.02).astype(np.float32)
    q = O.quantize(gtype, x)
    y = np.zeros(4096, np.float32)
    assert host().qmm_dequantize_cpu(gtype, q.ctypes.data, 4096, y.ctypes.data) == 0
    assert np.array_equal(y, O.dequantize(gtype, q, 4096))


def test_qtensor_shape_checks():
    L = host()
    h = C.c_void_p()
    data = np.zeros(144 * 4, np.uint8)
    assert L.qmm_qtensor_from_data(12, data.ctypes.data, data.size, 1, 2, 512, -1, C.byref(h)) == 0
    assert L.qmm_qtensor_storage_bytes(h) == 576
    L.qmm_qtensor_free(h)
    assert L.qmm_qtensor_from_data(12, data.ctypes.data, data.size, 1, 2, 300, -1, C.byref(h)) == -1
    assert b"multiple of 256" in L.qmm_host_last_error()
    assert L.qmm_qtensor_from_data(12, data.ctypes.data, 100, 1, 2, 512, -1, C.byref(h)) == -1
    assert b"bytes" in L.qmm_host_last_error()
    assert L.qmm_qtensor_from_data(99, data.ctypes.data, data.size, 1, 2, 512, -1, C.byref(h)) == -1
    assert b"unknown dtype" in L.qmm_host_last_error()
