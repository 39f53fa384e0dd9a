"""xtq_vit_tailbite_dev_noalloc, the tail-bite entry that allocates nothing
(its scratch is a fixed array in the library's code object), called through
the C-ABI: bit-identical to xtq_vit_tailbite_dev on two calls in a row, the
second with fewer sequences than the first (the array keeps the first call's
contents), on both the fused and the separate-pass schedules; a batch of
exactly the array's capacity runs and one beyond it is refused with status 5;
a NaN target gives status 11 and the next call starts clean; a stream under
graph capture is refused with status 13 and the capture stays usable (the
entry is synchronous)."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

# sequences one call can take: (256 MiB - 512 B) // (bp bytes + 12) per K
CAPACITY = {2: 257, 3: 257, 4: 513, 5: 513, 6: 1027, 7: 2055}


@pytest.fixture(scope="module")
def hb():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import hip_backend
    lib = hip_backend.lib()
    assert lib.xtq_vit_init() == 0          # set-up: the no-allocation entry never does it
    return hip_backend


def _noalloc(hb, X, K, pivot, margin):
    n = X.shape[0]
    st = torch.full((n, 256), -1, dtype=torch.int32, device=X.device)
    tr = torch.zeros(n, 16 * K, dtype=torch.int16, device=X.device)
    rc = hb.lib().xtq_vit_tailbite_dev_noalloc(
        ctypes.c_void_p(X.data_ptr()), n, K, b"mul1", margin, pivot,
        ctypes.c_void_p(st.data_ptr()), ctypes.c_void_p(tr.data_ptr()),
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    return rc, st, tr


@pytest.mark.parametrize("K,n1,n2,pivot,margin", [(4, 500, 77, 147, 16), (2, 257, 100, 128, 0),
                                                  (7, 2000, 1100, 5, 16)])
def test_noalloc_matches_tailbite_dev(hb, K, n1, n2, pivot, margin):
    rng = np.random.default_rng(100 + K)
    for n in (n1, n2):                       # the second call is smaller
        X = torch.from_numpy(rng.standard_normal((n, 256)).astype(np.float32)).cuda()
        print(f"case noalloc K={K} n={n} pivot={pivot} margin={margin}", flush=True)
        rc, st, tr = _noalloc(hb, X, K, pivot, margin)
        assert rc == 0
        ref_st, ref_tr = hb.tailbite(X, K, pivot, margin, states=True, trellis=True)
        assert torch.equal(st, ref_st)
        assert torch.equal(tr, ref_tr)


def test_noalloc_capacity_and_nan(hb):
    lib = hb.lib()
    fake = ctypes.c_void_p(16)               # never dereferenced: refused first
    rng = np.random.default_rng(7)
    for K, cap in CAPACITY.items():
        assert lib.xtq_vit_tailbite_dev_noalloc(fake, cap + 1, K, b"mul1", 0, 128, fake, None,
                                                None) == 5
        # the documented capacity itself is accepted
        X = torch.from_numpy(rng.standard_normal((cap, 256)).astype(np.float32)).cuda()
        print(f"case noalloc capacity K={K} n={cap}", flush=True)
        rc, st, tr = _noalloc(hb, X, K, 128, 0)
        assert rc == 0
        ref_st, ref_tr = hb.tailbite(X, K, 128, 0, states=True, trellis=True)
        assert torch.equal(st, ref_st) and torch.equal(tr, ref_tr)
    X = torch.randn(cap_small := 40, 256, device="cuda")
    X[7, 3] = float("nan")
    rc, _, _ = _noalloc(hb, X, 5, 128, 0)
    assert rc == 11
    X[7, 3] = 0.25
    rc, st, tr = _noalloc(hb, X, 5, 128, 0)
    assert rc == 0
    ref_st, ref_tr = hb.tailbite(X, 5, 128, 0, states=True, trellis=True)
    assert torch.equal(st, ref_st) and torch.equal(tr, ref_tr)
    assert cap_small <= CAPACITY[5]


def test_noalloc_refuses_graph_capture(hb):
    X = torch.from_numpy(np.random.default_rng(9).standard_normal((64, 256)).astype(
        np.float32)).cuda()
    a = torch.arange(4096, dtype=torch.float32, device="cuda")
    st = torch.zeros(64, 256, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    print("case noalloc under graph capture", flush=True)
    with torch.cuda.graph(g, stream=s):
        y = a * 2.0 + 1.0
        rc = hb.lib().xtq_vit_tailbite_dev_noalloc(
            ctypes.c_void_p(X.data_ptr()), 64, 4, b"mul1", 0, 128, ctypes.c_void_p(st.data_ptr()),
            None, ctypes.c_void_p(s.cuda_stream))
    assert rc == 13
    assert not st.any()                         # nothing was enqueued
    for _ in range(3):                          # the capture is intact and replays
        a.add_(1.0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, a * 2.0 + 1.0)
    rc, st, tr = _noalloc(hb, X, 4, 128, 0)     # and the entry still works eagerly
    assert rc == 0
    ref_st, ref_tr = hb.tailbite(X, 4, 128, 0, states=True, trellis=True)
    assert torch.equal(st, ref_st) and torch.equal(tr, ref_tr)
