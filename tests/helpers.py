"""Shared data generators and parity checks for the GPU tests (seeded; the oracle is the checker)."""
import numpy as np

import oracle as O


def weights(rng, n, k, sigma=0.02):
    return (rng.standard_normal((n, k)) * sigma).astype(np.float32)


def acts(rng, m, k):
    return rng.standard_normal((m, k)).astype(np.float32)


def patterned(n, salt=0):
    """The reference's deterministic fixture pattern (fast_mmq.rs:1580-1804): ((i*37 + salt*19) % 211)/105 - 1."""
    i = np.arange(n, dtype=np.int64)
    return (((i * 37 + salt * 19) % 211) / 105.0 - 1.0).astype(np.float32)


def terms(gtype, x, wq, n):
    """Per-output sum of |dequantized activation * dequantized weight| (the scale of the rounding error)."""
    import test_oracle as T
    m, k = x.shape
    a = T.NP_DEQUANT[O.ACT_TYPE[gtype]](O.quantize(O.ACT_TYPE[gtype], x)).reshape(m, k)
    w = T.NP_DEQUANT[gtype](wq).reshape(n, k)
    return np.abs(a) @ np.abs(w).T


def assert_parity(got, want, term=None, rel=1e-3, term_tol=1e-5, what=""):
    """max|got - want| <= rel * max|want| (fp32 accumulation, identical integer dots);
    and, per element, |got - want| <= term_tol * sum|terms| (only the f32 summation order differs)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.all(np.isfinite(got)), what
    err = np.max(np.abs(got - want)) if got.size else 0.0
    scale = max(np.max(np.abs(want)) if want.size else 0.0, 1e-30)
    assert err <= rel * scale, f"{what}: max|d|={err:.3e} max|ref|={scale:.3e} rel={err / scale:.3e}"
    if term is not None:
        bad = np.abs(got - want) > term_tol * term + 1e-30
        assert not bad.any(), f"{what}: {bad.sum()} elements beyond {term_tol} * sum|terms|"
    return err / scale
