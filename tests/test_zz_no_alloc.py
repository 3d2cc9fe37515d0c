"""qmm_qmatmul_forward_noalloc (the QMatMul::forward that allocates nothing) against the entry point it varies, the
host's qmm_qmatmul_forward: the same routes and kernels, so the same bits, on consecutive calls whose second input is
smaller than the first (the shared scratch keeps the first call's bytes), and against the oracle's CPU QMatMul at the
north-star bound.  An input beyond the scratch is refused before anything is launched."""
import ctypes

import numpy as np
import pytest

import oracle as O
import qmm
from helpers import acts, assert_parity, weights

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DTYPE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 30}


def noalloc():
    f = qmm.lib().qmm_qmatmul_forward_noalloc
    f.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_uint32,
                  ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
    f.restype = ctypes.c_int
    return f


def host_forward(h, x, n):
    H = qmm.host()
    out = torch.full((x.shape[0], n), float("nan"), dtype=x.dtype, device="cuda")
    rc = H.qmm_qmatmul_forward(h, x.data_ptr(), DTYPE[x.dtype], x.shape[0], out.data_ptr(),
                               torch.cuda.current_stream().cuda_stream)
    assert rc == 0, H.qmm_host_last_error()
    return out


# (weight type, n, k, activation dtype, row counts of consecutive calls): the prefill route with split K (300 and 40
# rows: planes in the scratch's fixup part), the decode route through the scratch (24 rows on the few-row kernel, 9), the one-launch matvec
# (2 rows, no scratch); Q6_K at K = 14336 with bf16 activations; Q8_0 and Q5_K with f16
CASES = [(O.Q4K, 4096, 4096, torch.float32, (300, 40, 24, 9, 2)),
         (O.Q6K, 1024, 14336, torch.bfloat16, (64, 5)),
         (O.Q8_0, 2048, 4096, torch.float16, (20, 3)),
         (O.Q5K, 512, 2048, torch.float32, (33, 17))]


@pytest.mark.parametrize("gtype,n,k,dtype,rows", CASES)
def test_noalloc_forward_matches_qmatmul_forward(gtype, n, k, dtype, rows):
    rng = np.random.default_rng(900 + gtype)
    wq = O.quantize(gtype, weights(rng, n, k))
    H = qmm.host()
    h = ctypes.c_void_p()
    assert H.qmm_qtensor_from_data(gtype, wq.ctypes.data, wq.size, 1, n, k, 0, ctypes.byref(h)) == 0
    f = noalloc()
    try:
        w = H.qmm_qtensor_device_ptr(h)
        for m in rows:
            print(f"noalloc type {gtype} n={n} k={k} rows={m} {dtype}", flush=True)
            x32 = acts(rng, m, k)
            x = torch.from_numpy(x32).cuda().to(dtype)
            got = torch.full((m, n), float("nan"), dtype=dtype, device="cuda")
            rc = f(w, gtype, n, k, x.data_ptr(), DTYPE[dtype], m, got.data_ptr(), torch.cuda.current_stream().cuda_stream)
            assert rc == 0, qmm.last_error()
            ref = host_forward(h, x, n)
            torch.cuda.synchronize()
            g, r = got.cpu(), ref.cpu()
            assert torch.equal(g.view(torch.int16 if dtype != torch.float32 else torch.int32),
                               r.view(torch.int16 if dtype != torch.float32 else torch.int32)), f"rows={m}"
            if dtype == torch.float32:
                assert_parity(g.numpy(), O.matmul(gtype, x32, wq, n), what=f"rows={m}")
    finally:
        H.qmm_qtensor_free(h)


def test_noalloc_refuses_inputs_beyond_its_scratch():
    f = noalloc()
    n, k, m = 256, 14336, 4096  # 4096 x 14336 activations as Q8_K need 65.4 MB > 16 MiB
    w = torch.zeros(n * k // 256 * 144 + 4096, dtype=torch.uint8, device="cuda")
    x = torch.zeros((m, k), dtype=torch.float32, device="cuda")
    y = torch.full((m, n), 7.0, dtype=torch.float32, device="cuda")
    rc = f(w.data_ptr(), O.Q4K, n, k, x.data_ptr(), 0, m, y.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == -1 and "scratch" in qmm.last_error()
    qmm.lib().qmm_clear_error()
    torch.cuda.synchronize()
    assert torch.all(y == 7.0)  # nothing launched
