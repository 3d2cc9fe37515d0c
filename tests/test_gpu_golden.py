"""GPU path against the committed golden fixtures (tests/golden/): activation blocks bit-exact, matvec / matmul /
indexed MoE outputs within the north-star tolerance, through the C ABI."""
import os

import numpy as np
import pytest

import oracle as O
import qmm
from helpers import assert_parity, decode_act_blocks, terms

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TYPES = {O.Q8_0: "q8_0", O.Q4K: "q4_k", O.Q6K: "q6_k"}


def load(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("gtype", list(TYPES))
def test_decode_against_fixture(gtype):
    g = load(f"qmatmul_{TYPES[gtype]}.npz")
    n, k = int(g["n"]), int(g["k"])
    w = g["w_bytes"].reshape(-1)
    for b in (1, 2, 4, 16):
        x = g["x"][:b]
        vy, kp = qmm.quantize_decode(gtype, dev(x))
        blocks = decode_act_blocks(gtype, vy.cpu().numpy(), b, kp, k)
        assert np.array_equal(blocks, g["xq_bytes"][:b].reshape(-1)), f"b={b}"
        y = qmm.mmvq(gtype, dev(w), vy, k, n, b, kp).cpu().numpy()
        assert_parity(y, g["y"][:b], terms(gtype, x, w, n), what=f"{TYPES[gtype]} b={b}")


@pytest.mark.parametrize("gtype", list(TYPES))
def test_prefill_against_fixture(gtype):
    g = load(f"qmatmul_{TYPES[gtype]}.npz")
    n = int(g["n"])
    w = g["w_bytes"].reshape(-1)
    y = qmm.qmatmul_prefill(gtype, dev(w), dev(g["x"]), n).cpu().numpy()
    assert_parity(y, g["y"], terms(gtype, g["x"], w, n), what=TYPES[gtype])


def test_indexed_moe_against_fixture():
    g = load("indexed_moe_q4_k.npz")
    n = int(g["n"])
    y = qmm.indexed_moe(O.Q4K, dev(g["w_bytes"].reshape(-1)), dev(g["x"]), dev(g["ids"]), n)
    assert_parity(y.cpu().numpy(), g["y"], what="indexed moe")
