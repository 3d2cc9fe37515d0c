"""A GGUF file's quantized tensors loaded onto the GPU by the host layer (Content::tensor) and run through
QMatMul::forward and QTensor::dequantize_on_device: results match the oracle on the file's bytes."""
import ctypes

import numpy as np
import pytest

import gguf_writer as G
import oracle as O
import qmm
from helpers import assert_parity, terms

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("gtype,n,k,rows", [(O.Q4K, 96, 1024, 1), (O.Q6K, 64, 512, 5), (O.Q8_0, 48, 256, 40),
                                            (O.Q4K, 130, 2048, 100), (O.Q5K, 64, 512, 40), (O.Q4_0, 48, 256, 3),
                                            (O.Q5_0, 40, 96, 17)])
def test_gguf_weight_runs_through_qmatmul(tmp_path, gtype, n, k, rows):
    rng = np.random.default_rng(n + k + rows)
    wq = O.quantize(gtype, (rng.standard_normal((n, k)) * 0.02).astype(np.float32)).reshape(-1)
    path = tmp_path / "m.gguf"
    G.write(path, [("general.architecture", G.STRING, "llama")],
            [("blk.0.ffn_up.weight", [n, k], gtype, wq.tobytes()), ("norm", [k], 0, np.ones(k, np.float32).tobytes())])
    H = qmm.host()
    x = rng.standard_normal((rows, k)).astype(np.float32)
    with qmm.GgufFile(str(path)) as g:
        w = g.load_tensor("blk.0.ffn_up.weight", 0)
    try:
        xs = torch.from_numpy(x).cuda()
        ys = torch.empty((rows, n), dtype=torch.float32, device="cuda")
        rc = H.qmm_qmatmul_forward(w, xs.data_ptr(), qmm.F32, rows, ys.data_ptr(),
                                   torch.cuda.current_stream().cuda_stream)
        assert rc == 0, H.qmm_host_last_error()
        torch.cuda.synchronize()
        want = O.matmul(gtype, x, wq, n)
        assert_parity(ys.cpu().numpy(), want, terms(gtype, x, wq, n), what="gguf qmatmul")
        out = torch.empty(n * k, dtype=torch.float32, device="cuda")
        H.qmm_qtensor_dequantize_device.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p]
        rc = H.qmm_qtensor_dequantize_device(w, out.data_ptr(), qmm.F32, torch.cuda.current_stream().cuda_stream)
        assert rc == 0, H.qmm_host_last_error()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint32), O.dequantize(gtype, wq, n * k).view(np.uint32))
    finally:
        H.qmm_qtensor_free(w)
