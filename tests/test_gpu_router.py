"""GPU parity of the MoE router (moe_router_topk_{f32,bf16,f16}) against the oracle's restatement of the reference
kernel: expert ids exactly, weights to float32 rounding of the exponentials (rtol 2e-6)."""
import numpy as np
import pytest

import oracle as O
import qmm

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def run(logits, top_k, score_mode, weight_mode, renorm, bias=None, escale=None, clamp=None, norm_min=0.0,
        scale=1.0, dtype=torch.float32):
    x = torch.from_numpy(logits).cuda().to(dtype)
    xs = x.float().cpu().numpy()  # the values the kernel sees
    b = torch.from_numpy(bias).cuda() if bias is not None else None
    e = torch.from_numpy(escale).cuda() if escale is not None else None
    w, ids = qmm.router_topk(x, top_k, score_mode, weight_mode, renorm, b, e, clamp, norm_min, scale)
    torch.cuda.synchronize()
    ww, wi = O.router_topk(xs, top_k, score_mode, weight_mode, renorm, bias, escale, clamp, norm_min, scale)
    return w.cpu().numpy(), ids.cpu().numpy().astype(np.uint32), ww, wi


@pytest.mark.parametrize("n_experts", [8, 60, 64, 128, 256, 576, 1000])
@pytest.mark.parametrize("top_k", [1, 2, 8])
@pytest.mark.parametrize("score_mode,weight_mode,renorm", [(1, 0, True), (1, 0, False), (2, 0, True), (0, 1, False),
                                                           (2, 2, True)])
def test_router_matches_the_oracle(n_experts, top_k, score_mode, weight_mode, renorm):
    rng = np.random.default_rng(n_experts * 7 + top_k * 3 + score_mode + 5 * weight_mode)
    logits = rng.standard_normal((37, n_experts)).astype(np.float32) * 3
    bias = rng.standard_normal(n_experts).astype(np.float32) * 0.1 if score_mode == 2 else None
    w, ids, ww, wi = run(logits, top_k, score_mode, weight_mode, renorm, bias=bias, norm_min=1e-20, scale=2.5)
    assert np.array_equal(ids, wi)
    assert np.allclose(w, ww, rtol=2e-6, atol=1e-30)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_router_half_inputs_ties_nan_and_expert_scale(dtype):
    rng = np.random.default_rng(3)
    logits = rng.standard_normal((16, 64)).astype(np.float32)
    logits[0, 5] = logits[0, 9] = 9.0            # a tie: expert 5 first
    logits[1, 3] = np.nan                         # never picked before a finite score
    escale = (rng.random(64).astype(np.float32) + 0.5)
    w, ids, ww, wi = run(logits, 4, 1, 0, True, escale=escale, dtype=dtype)
    assert ids[0, 0] == 5 and ids[0, 1] == 9 and 3 not in ids[1]
    assert np.array_equal(ids, wi) and np.allclose(w, ww, rtol=2e-6)
    w, ids, ww, wi = run(logits, 3, 0, 0, False, clamp=(-0.5, 0.5), dtype=dtype)
    assert np.array_equal(ids, wi) and np.array_equal(w, ww)


def test_router_rejects_bad_arguments():
    x = torch.zeros((2, 8), device="cuda")
    with pytest.raises(qmm.QmmError, match="top_k"):
        qmm.router_topk(x, 9)
    with pytest.raises(qmm.QmmError, match="score_mode"):
        qmm.router_topk(x, 2, score_mode=3)
