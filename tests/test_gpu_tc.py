"""GPU parity of the tensor-core matvec entries through the C ABI, called as the reference's fast_mmvq::plain calls
them for 1..16 rows of a Q4_K / Q6_K weight (crates/inference-quant/src/gguf/fast_mmvq.rs:505-513, 1897-1930):
launch_mmvq_tc_quantize_<src> into a scratch buffer of exactly the reference's size ((k / 32) * 288 bytes per
8-row half, fast_mmvq.rs:92-93, 1903-1908), then launch_mmvq_tc_gguf_<t>_<dt>_plain with each of the reference's
configs.  The quantizer's d and qs are BlockQ8K::from_float's, byte for byte; nothing is written past the
reference's scratch size; outputs match the oracle's CPU QMatMul within the north-star tolerance."""
import numpy as np
import pytest

import oracle as O
import qmm
from helpers import acts, assert_parity, terms, weights

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda"
GUARD = 4096


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def guarded(nbytes):
    """A scratch buffer of nbytes followed by a guard region of 0xA5 bytes."""
    buf = torch.full((nbytes + GUARD,), 0xA5, dtype=torch.uint8, device=DEV)
    return buf, buf[:nbytes]


@pytest.mark.parametrize("rows", [1, 7, 8, 9, 16])
@pytest.mark.parametrize("src", ["f32", "f16", "bf16"])
def test_tc_quantizer_is_bit_exact_and_fits_the_reference_scratch(rows, src):
    k = 4096
    rng = np.random.default_rng(40 + rows)
    x = acts(rng, rows, k)
    x[0, 256:512] = 0.0
    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[src]
    xt = to_dev(x).to(tdt)
    buf, scratch = guarded(qmm.tc_scratch_bytes(k, rows))
    qmm.tc_quantize(xt, out=scratch)
    got = buf.cpu().numpy()
    assert np.all(got[qmm.tc_scratch_bytes(k, rows):] == 0xA5), "wrote past the reference's scratch size"
    want = O.blocks(O.Q8K, O.quantize(O.Q8K, xt.float().cpu().numpy()))
    blk = got[:rows * k // 256 * 260].reshape(-1, 260)
    assert np.array_equal(blk[:, :4].copy().view("<f4").reshape(-1), want["d"])
    assert np.array_equal(blk[:, 4:].view(np.int8), want["qs"])


CASES = [(O.Q4K, 512, 1024), (O.Q4K, 300, 4096), (O.Q4K, 14336, 4096), (O.Q6K, 256, 512), (O.Q6K, 4096, 14336),
         (O.Q6K, 77, 2048)]


@pytest.mark.parametrize("gtype,n,k", CASES)
@pytest.mark.parametrize("b", [1, 2, 3, 4, 8, 9, 16])
def test_tc_matvec_matches_the_cpu_qmatmul(gtype, n, k, b):
    rng = np.random.default_rng(7000 + 10 * gtype + b + n % 97)
    wq = O.quantize(gtype, weights(rng, n, k))
    x = acts(rng, b, k)
    x[:, ::64] *= 60.0
    buf, scratch = guarded(qmm.tc_scratch_bytes(k, b))
    qmm.tc_quantize(to_dev(x), out=scratch)
    cfg = 0 if b <= 8 else 3
    got = qmm.mmvq_tc(gtype, to_dev(wq), scratch, k, n, b, cfg=cfg).cpu().numpy()
    assert np.all(buf[-GUARD:].cpu().numpy() == 0xA5)
    idx = np.arange(n) if n <= 512 else np.r_[0:48, n // 2:n // 2 + 16, n - 48:n]  # sampled rows of tall weights
    want = O.matmul(gtype, x, wq[idx], len(idx))
    assert_parity(got[:, idx], want, what=f"t{gtype} {n}x{k} b{b}")


@pytest.mark.parametrize("gtype", [O.Q4K, O.Q6K])
@pytest.mark.parametrize("out", ["f16", "bf16"])
def test_tc_matvec_half_outputs_and_dst_stride(gtype, out):
    rng = np.random.default_rng(11)
    n, k, b = 200, 1024, 5
    wq = O.quantize(gtype, weights(rng, n, k))
    x = acts(rng, b, k)
    tdt = {"f16": torch.float16, "bf16": torch.bfloat16}[out]
    dst = torch.full((b, 256), 7.0, dtype=tdt, device=DEV)
    qmm.mmvq_tc(gtype, to_dev(wq), qmm.tc_quantize(to_dev(x).to(tdt)), k, n, b, out=dst)
    want = O.matmul(gtype, torch.from_numpy(x).to(tdt).float().numpy(), wq, n)  # the reference widens x to f32
    got = dst.float().cpu().numpy()
    ulp = {"f16": 2.0 ** -11, "bf16": 2.0 ** -8}[out]  # the f32 result rounded once to the half type
    assert np.all(np.abs(got[:, :n] - want) <= 1e-3 * np.abs(want).max() + ulp * np.abs(want))
    assert np.all(got[:, n:] == 7.0)


@pytest.mark.parametrize("n,bs", [(1024, (1, 2)), (12288, (5, 16))])
def test_tc_matvec_equals_the_plain_entry_bit_for_bit(n, bs):
    """Same weights and activations through the plain pair (Q8_K decode layout) and the tensor-core pair, at shapes
    where both run the same kernel form (the persistent matvec below the few-row threshold; the 32x32 few-row form
    for weights of at least 384 32-row tiles -- narrower plain calls take the 16x16 form, which sums in another
    order): the integer dots and their scaling are the same, so the outputs are identical."""
    rng = np.random.default_rng(12)
    k = 4096
    for gtype in (O.Q4K, O.Q6K):
        wq = to_dev(O.quantize(gtype, weights(rng, n, k)))
        for b in bs:
            x = to_dev(acts(rng, b, k))
            plain = qmm.qmatmul_decode(gtype, wq, x, n)
            tc = qmm.mmvq_tc(gtype, wq, qmm.tc_quantize(x), k, n, b)
            assert torch.equal(plain, tc), (gtype, b)


def test_tc_rejects_k_not_a_multiple_of_256():
    L = qmm.lib()
    L.qmm_clear_error()
    L.launch_mmvq_tc_quantize_f32(None, None, 300, 1, None)
    assert "multiple of 256" in qmm.last_error()
    L.qmm_clear_error()
