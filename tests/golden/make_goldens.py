"""Writes the committed golden fixtures of tests/golden/ from the C oracle (oracle/oracle.c), the restatement
of the reference CPU QMatMul that tests/test_oracle.py pins.  The reference has no golden vectors for Q8_0 /
Q4_K / Q6_K (its fixtures cover the IQ and ik types only), so these are the oracle's own outputs on seeded
inputs, kept small, and a regression pin for the oracle and for the GPU path.

Each fixture (numpy .npz, no pickles) holds for one weight type:
  w_bytes   the quantized weight [N, K] as GGUF blocks (uint8), from N(0, 0.02) values
  x         activations [M, K] f32 ~ N(0, 1), column 0 of every 64 scaled by 60 (outliers)
  xq_bytes  the activations quantized to the matmul's activation blocks (Q8_K or Q8_0), [M, K / bs] blocks
  y         the CPU QMatMul output [M, N] f32
and, for the MoE fixture, ids / route outputs of the indexed forward.

Run from the repository root:  python tests/golden/make_goldens.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle as O  # noqa: E402

SEED = 20260601
SHAPES = {O.Q8_0: (48, 512), O.Q4K: (64, 512), O.Q6K: (48, 768)}
M = 33


def make(gtype):
    n, k = SHAPES[gtype]
    rng = np.random.default_rng(SEED + gtype)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((M, k)).astype(np.float32)
    x[:, ::64] *= 60.0
    wq = O.quantize(gtype, w)
    xq = O.quantize(O.ACT_TYPE[gtype], x)
    y = O.matmul(gtype, x, wq, n)
    return {"w_bytes": wq, "x": x, "xq_bytes": xq, "y": y.astype(np.float32),
            "n": np.int64(n), "k": np.int64(k), "gtype": np.int64(gtype)}


def make_moe():
    e, n, k, tokens, topk = 3, 32, 512, 5, 2
    rng = np.random.default_rng(SEED + 99)
    w = (rng.standard_normal((e * n, k)) * 0.02).astype(np.float32)
    wq = O.quantize(O.Q4K, w)
    x = rng.standard_normal((tokens, 1, k)).astype(np.float32)
    ids = np.array([[0, 2], [2, 1], [1, 1], [0, 0], [2, 0]], dtype=np.uint32)
    y = O.indexed_moe(O.Q4K, wq, e, n, k, x, ids)
    return {"w_bytes": wq, "x": x, "ids": ids, "y": np.asarray(y, np.float32), "experts": np.int64(e),
            "n": np.int64(n), "k": np.int64(k)}


def main():
    names = {O.Q8_0: "q8_0", O.Q4K: "q4_k", O.Q6K: "q6_k"}
    for gtype, name in names.items():
        np.savez_compressed(os.path.join(HERE, f"qmatmul_{name}.npz"), **make(gtype))
    np.savez_compressed(os.path.join(HERE, "indexed_moe_q4_k.npz"), **make_moe())


if __name__ == "__main__":
    main()
