"""GPU parity of the dequantizers (QCudaStorage::dequantize, get_rows) and the exact Q8_0 matvec through the C ABI.
Dequantized f32 values must equal the oracle's to_float bit for bit; f16 / bf16 outputs are those values rounded
to nearest even.  The exact matvec is held to the north-star bound (max rel. error <= 1e-3) and to f32 rounding of
its terms (1e-5 * sum|terms|) against a float64 sum over the dequantized weights."""
import numpy as np
import pytest

import oracle as O
import qmm
from helpers import assert_parity, weights

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda"


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def bf16_rne(x32: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bits, round to nearest even (NaN-free inputs)."""
    u = x32.astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def quantized(gtype, n, k, seed, sigma=0.02):
    rng = np.random.default_rng(seed)
    w = weights(rng, n, k, sigma)
    if gtype != O.Q8_0:
        w[0, :256] = 0.0  # an all-zero superblock (d = dmin = 0)
    return O.quantize(gtype, w).reshape(-1)


@pytest.mark.parametrize("gtype", [O.Q8_0, O.Q4K, O.Q6K])
@pytest.mark.parametrize("n,k", [(1, 256), (7, 512), (64, 4096)])
def test_dequantize_f32_is_bit_exact(gtype, n, k):
    wq = quantized(gtype, n, k, seed=n * 31 + k + gtype)
    want = O.dequantize(gtype, wq, n * k)
    got = qmm.dequantize(gtype, to_dev(wq), n * k).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("gtype", [O.Q8_0, O.Q4K, O.Q6K])
def test_dequantize_f16_bf16_round_the_f32_values(gtype):
    n, k = 16, 1024
    wq = quantized(gtype, n, k, seed=5 + gtype, sigma=2.0)  # wide range: exercises f16 rounding and subnormals less
    want = O.dequantize(gtype, wq, n * k)
    dev = to_dev(wq)
    h = qmm.dequantize(gtype, dev, n * k, out_dtype=torch.float16).cpu().numpy()
    assert np.array_equal(h.view(np.uint16), want.astype(np.float16).view(np.uint16))
    b = qmm.dequantize(gtype, dev, n * k, out_dtype=torch.bfloat16).view(torch.int16).cpu().numpy()
    assert np.array_equal(b.view(np.uint16), bf16_rne(want))


@pytest.mark.parametrize("gtype", [O.Q8_0, O.Q4K, O.Q6K])
def test_get_rows_gathers_dequantized_rows(gtype):
    n, k = 40, 512
    wq = quantized(gtype, n, k, seed=9 + gtype)
    row_bytes = k // O.BLOCK_SIZE[gtype] * O.TYPE_SIZE[gtype]
    # rows padded to a longer stride, as a QTensor's device buffer may be
    nb01 = row_bytes + 2 * O.TYPE_SIZE[gtype]
    padded = np.zeros((n, nb01), np.uint8)
    padded[:, :row_bytes] = wq.reshape(n, row_bytes)
    ids = np.array([3, 0, 39, 3, 17], dtype=np.uint32)
    got = qmm.get_rows(gtype, to_dev(padded.reshape(-1)), to_dev(ids), k, nb01).cpu().numpy()
    full = O.dequantize(gtype, wq, n * k).reshape(n, k)
    assert np.array_equal(got.view(np.uint32), full[ids].view(np.uint32))


@pytest.mark.parametrize("b", [1, 2, 3, 8])
@pytest.mark.parametrize("n,k", [(1, 32), (37, 96), (300, 4096), (64, 14336)])
def test_exact_q8_0_matvec_f32(b, n, k):
    rng = np.random.default_rng(b * 13 + n + k)
    wq = quantized(O.Q8_0, n, k, seed=b + n + k)
    x = rng.standard_normal((b, k)).astype(np.float32)
    wd = O.dequantize(O.Q8_0, wq, n * k).reshape(n, k).astype(np.float64)
    want = x.astype(np.float64) @ wd.T
    term = np.abs(x.astype(np.float64)) @ np.abs(wd).T
    got = qmm.q8_0_exact(to_dev(wq), to_dev(x), n).cpu().numpy()
    assert_parity(got, want, term, what=f"exact b={b} {n}x{k}")


@pytest.mark.parametrize("b", [1, 5])
def test_exact_q8_0_matvec_bf16(b):
    n, k = 200, 1024
    rng = np.random.default_rng(77 + b)
    wq = quantized(O.Q8_0, n, k, seed=3 + b)
    xt = to_dev(rng.standard_normal((b, k)).astype(np.float32)).to(torch.bfloat16)
    x = xt.float().cpu().numpy().astype(np.float64)
    wd = O.dequantize(O.Q8_0, wq, n * k).reshape(n, k).astype(np.float64)
    want = x @ wd.T
    got = qmm.q8_0_exact(to_dev(wq), xt, n).float().cpu().numpy()
    # f32 sums, then one bf16 rounding of the output (relative 2^-9)
    assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + 1e-5 * (np.abs(x) @ np.abs(wd).T))


def test_qtensor_dequantize_on_device_through_the_host_api():
    import ctypes
    H = ctypes.CDLL(qmm.HOST_LIB_PATH)
    H.qmm_host_last_error.restype = ctypes.c_char_p
    H.qmm_qtensor_from_data.argtypes = [ctypes.c_uint32, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                        ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.POINTER(ctypes.c_void_p)]
    H.qmm_qtensor_dequantize_device.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p]
    H.qmm_qtensor_free.argtypes = [ctypes.c_void_p]
    n, k = 24, 768
    wq = quantized(O.Q4K, n, k, seed=41)
    t = ctypes.c_void_p()
    assert H.qmm_qtensor_from_data(O.Q4K, wq.ctypes.data, wq.size, 1, n, k, 0, ctypes.byref(t)) == 0, \
        H.qmm_host_last_error()
    out = torch.empty(n * k, dtype=torch.bfloat16, device=DEV)
    rc = H.qmm_qtensor_dequantize_device(t, out.data_ptr(), qmm.BF16, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, H.qmm_host_last_error()
    torch.cuda.synchronize()
    H.qmm_qtensor_free(t)
    want = bf16_rne(O.dequantize(O.Q4K, wq, n * k))
    assert np.array_equal(out.view(torch.int16).cpu().numpy().view(np.uint16), want)
