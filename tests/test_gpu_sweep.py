"""Randomised parity sweep of the batched tail-biting encode against the C
oracle (quantize.py:323-354 restated): every K, six target distributions --
Gaussian, exact codebook values (ties at every step), a coarse grid, heavy
tails, codebook values with zeroed columns, tiny costs -- and, per
distribution, the reference's default pivot/margin and two random ones.
The encoder picks its code path (grouping, fused or separate passes) as it
does in production.  Every sequence must match bit for bit.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hb():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import hip_backend
    return hip_backend


def _targets(rng, lut, n, kind):
    if kind == "gauss":
        return rng.standard_normal((n, 256)).astype(np.float32)
    if kind == "codebook":
        return lut[rng.integers(0, 65536, (n, 256))].astype(np.float32)
    if kind == "grid":
        return (np.round(rng.standard_normal((n, 256)) * 4) / 4).astype(np.float32)
    if kind == "student":
        return (rng.standard_t(3, (n, 256)) * 1.5).astype(np.float32)
    if kind == "codebook0":
        X = lut[rng.integers(0, 65536, (n, 256))].astype(np.float32)
        X[:, ::7] = 0.0
        return X
    return (rng.standard_normal((n, 256)) * 1e-3).astype(np.float32)


@pytest.mark.parametrize("defer,K", [("0", K) for K in range(2, 8)]
                         + [("1", K) for K in range(4, 8)])
def test_tailbite_sweep(hb, oracle_mod, mul1_lut, K, defer, monkeypatch):
    """defer "1": the deferred-argmin encode (K >= 4) on the same sweep."""
    monkeypatch.setenv("XTQ_VIT_DEFER", defer)
    rng = np.random.default_rng(9000 + K)
    n, bad = 64, []
    for kind in ("gauss", "codebook", "grid", "student", "codebook0", "tiny"):
        cases = ((128, 0), (int(rng.integers(0, 256)), 16),
                 (int(rng.integers(0, 256)), int(rng.integers(1, 120))))
        for pivot, margin in cases:
            print(f"case K={K} {kind} pivot={pivot} margin={margin}", flush=True)
            X = _targets(rng, mul1_lut, n, kind)
            want = oracle_mod.tailbite(X, mul1_lut, K, 16, pivot=pivot, margin=margin,
                                       nthreads=8)
            st, _ = hb.tailbite(torch.from_numpy(X).cuda(), K, pivot, margin)
            nb = int((st.cpu().numpy() != want).any(axis=1).sum())
            if nb:
                bad.append((kind, pivot, margin, nb))
    assert not bad, f"sequences differing from the oracle: {bad}"
