"""Host threads sharing the library: calls from two threads at once (ctypes
releases the GIL) serialise on the library's lock and share its scratch,
and each returns what the same call returns alone.  The reference's ctypes
transport makes the same kind of call from its own threads
(quantize.py:473-505)."""
import threading

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

PIVOT, MARGIN = 128, 0


@pytest.fixture(scope="module")
def hb():
    import hip_backend
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    hip_backend.lib()
    return hip_backend


def _run_threads(workers):
    errors = []

    def wrap(fn):
        def run():
            try:
                fn()
            except BaseException as e:          # reported by the main thread
                errors.append(repr(e))
        return run

    threads = [threading.Thread(target=wrap(f)) for f in workers]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
        assert not t.is_alive(), "a worker thread did not finish"
    assert not errors, errors


def test_host_entry_from_two_threads(hb):
    """xtq_vit_run (host pointers, the reference's entry) from two threads
    with different batch sizes, so that the second grows the host staging
    while the first may be using it."""
    L = hb.lib()
    rng = np.random.default_rng(11)
    Xs = [rng.standard_normal((n, 256)).astype(np.float32) for n in (300, 1100)]
    want = []
    for X in Xs:
        out = np.empty((X.shape[0], 256), dtype=np.int32)
        assert L.xtq_vit_run(X.ctypes.data, X.shape[0], b"mul1", MARGIN, PIVOT,
                             out.ctypes.data) == 0
        want.append(out)

    def worker(X, w):
        def run():
            out = np.empty((X.shape[0], 256), dtype=np.int32)
            for _ in range(6):
                out.fill(-1)
                rc = L.xtq_vit_run(X.ctypes.data, X.shape[0], b"mul1", MARGIN, PIVOT,
                                   out.ctypes.data)
                assert rc == 0, rc
                assert np.array_equal(out, w)
        return run

    _run_threads([worker(X, w) for X, w in zip(Xs, want)])


def test_device_entries_from_two_threads_on_two_streams(hb):
    """The device-pointer tail-bite from two threads, each on its own torch
    stream, at different K: the library orders their use of its scratch."""
    torch.manual_seed(12)
    jobs = [(torch.randn(700, 256, device="cuda"), 4), (torch.randn(2100, 256, device="cuda"), 6)]
    want = []
    for X, K in jobs:
        st, tr = hb.tailbite(X, K, PIVOT, MARGIN, states=True, trellis=True)
        torch.cuda.synchronize()
        want.append((st.clone(), tr.clone()))

    def worker(X, K, w):
        def run():
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for _ in range(4):
                    st, tr = hb.tailbite(X, K, PIVOT, MARGIN, states=True, trellis=True)
                    s.synchronize()
                    assert torch.equal(st, w[0]) and torch.equal(tr, w[1])
        return run

    _run_threads([worker(X, K, w) for (X, K), w in zip(jobs, want)])
    torch.cuda.synchronize()
