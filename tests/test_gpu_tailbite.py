"""GPU parity of the HIP tail-biting encoder, decode and pack kernels.

Every check compares libexl3vit.so (called through its C-ABI via ctypes)
with the reference's golden vectors or the CPU oracle on identical inputs,
bit for bit.  Reference semantics: quantize.py:218-415.
"""
import os

import numpy as np
import pytest
import torch

from conftest import load_golden

pytestmark = pytest.mark.gpu

PIVOTS = (0, 128, 147, 255)
MARGINS = (0, 16)


@pytest.fixture(scope="module")
def hb():
    import hip_backend
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    hip_backend.lib()
    return hip_backend


@pytest.fixture(scope="module")
def xq(hb):
    import quantize
    return quantize


def _run(hb, X: np.ndarray, K: int, pivot: int, margin: int, trellis=False):
    Xd = torch.from_numpy(np.ascontiguousarray(X, dtype=np.float32)).cuda()
    st, tr = hb.tailbite(Xd, K, pivot, margin, states=True, trellis=trellis)
    torch.cuda.synchronize()
    return st.cpu().numpy(), (tr.cpu().numpy() if tr is not None else None)


@pytest.mark.parametrize("K", range(2, 8))
def test_golden_tailbite(hb, K):
    """States equal the reference's own quantize_seq_tailbite on Gaussian and
    tie-heavy targets for every margin/pivot in the fixture."""
    g = load_golden("tailbite.npz")
    X = g[f"X_K{K}"]
    for m in MARGINS:
        for p in PIVOTS:
            print(f"case K={K} margin={m} pivot={p}", flush=True)
            st, tr = _run(hb, X, K, p, m, trellis=(m == 0 and p == 128))
            np.testing.assert_array_equal(st, g[f"S_K{K}_m{m}_p{p}"],
                                          err_msg=f"K={K} m={m} p={p}")
            if tr is not None:
                np.testing.assert_array_equal(tr, g[f"P_K{K}"])


TIE_CASES = ((128, 0), (147, 16), (0, 0), (255, 16))


@pytest.mark.parametrize("group,K", [(g, K) for g in ("auto", "1", "2", "4", "8", "fused")
                                     for K in range(2, 8)]
                         + [(g, K) for g in ("d1", "d4", "d8") for K in range(4, 8)])
def test_golden_ties(hb, K, group, monkeypatch):
    """The reference's quantize_seq_tailbite and viterbi() on 24 tie-forcing
    sequences per K (exact codebook values, codebook midpoints, constant
    runs, a 0.25 grid, sparse values, +-8 beyond the codebook), through every
    code path: the library's own choice, separate pass launches at 1, 2, 4 or
    8 sequences per workgroup, the fused launch, the deferred argmin."""
    if group != "auto":
        monkeypatch.setenv("XTQ_VIT_DEFER", "1" if group.startswith("d") else "0")
        monkeypatch.setenv("XTQ_VIT_FUSED", "1" if group == "fused" else "0")
        if group != "fused":
            monkeypatch.setenv("XTQ_VIT_GROUP", group.lstrip("d"))
    g = load_golden("ties.npz")
    X = g[f"X_K{K}"]
    for p, m in TIE_CASES:
        print(f"case ties K={K} group={group} pivot={p} margin={m}", flush=True)
        st, _ = _run(hb, X, K, p, m)
        np.testing.assert_array_equal(st, g[f"S_K{K}_m{m}_p{p}"], err_msg=f"K={K} m={m} p={p}")
    if group == "auto":
        Xd = torch.from_numpy(X).cuda()
        ov = torch.from_numpy(g[f"VPov_K{K}"]).cuda()
        np.testing.assert_array_equal(hb.viterbi(Xd, K, overlap=ov).cpu().numpy(),
                                      g[f"VP_K{K}"])
        vb = hb.viterbi(Xd[:, :200].contiguous(), K, back_from=60)
        np.testing.assert_array_equal(vb.cpu().numpy(), g[f"VB_K{K}"])


@pytest.mark.parametrize("K", range(2, 8))
def test_golden_viterbi_runs(hb, K):
    """Single Viterbi runs equal the reference's viterbi(): free with full
    traceback, truncated with back_from, and pinned to given overlaps."""
    g = load_golden("tailbite.npz")
    X = torch.from_numpy(g[f"X_K{K}"]).cuda()
    print(f"case K={K} free", flush=True)
    np.testing.assert_array_equal(hb.viterbi(X, K).cpu().numpy(), g[f"V_K{K}"])
    print(f"case K={K} back_from", flush=True)
    vb = hb.viterbi(X[:, :150].contiguous(), K, back_from=100)
    np.testing.assert_array_equal(vb.cpu().numpy(), g[f"VB_K{K}"])
    print(f"case K={K} pinned", flush=True)
    ov = torch.from_numpy(g[f"VPov_K{K}"]).cuda()
    np.testing.assert_array_equal(hb.viterbi(X, K, overlap=ov).cpu().numpy(), g[f"VP_K{K}"])


@pytest.mark.parametrize("K", (2, 5, 7))
def test_short_runs_vs_oracle(hb, oracle_mod, mul1_lut, K):
    """Runs shorter than a tile (T = 1, 2, 17, 255) and pinned short runs."""
    rng = np.random.default_rng(50 + K)
    for T in (1, 2, 17, 255):
        X = rng.standard_normal((5, T)).astype(np.float32)
        print(f"case K={K} T={T}", flush=True)
        got = hb.viterbi(torch.from_numpy(X).cuda(), K).cpu().numpy()
        np.testing.assert_array_equal(got, oracle_mod.viterbi(X, mul1_lut, K, 16))
        ov = rng.integers(0, 1 << (16 - K), 5).astype(np.int32)
        got = hb.viterbi(torch.from_numpy(X).cuda(), K,
                         overlap=torch.from_numpy(ov)).cpu().numpy()
        np.testing.assert_array_equal(got, oracle_mod.viterbi(X, mul1_lut, K, 16, overlap=ov))
        if T > 1:
            got = hb.viterbi(torch.from_numpy(X).cuda(), K, back_from=T // 2).cpu().numpy()
            np.testing.assert_array_equal(
                got, oracle_mod.viterbi(X, mul1_lut, K, 16, back_from=T // 2))


# the deferred-argmin paths ("d*") exist for K >= 4 only
@pytest.mark.parametrize("group,K", [(g, K) for g in ("1", "2", "4", "8", "fused")
                                     for K in range(2, 8)]
                         + [(g, K) for g in ("d1", "d2", "d4", "d8") for K in range(4, 8)])
def test_oracle_random(hb, oracle_mod, mul1_lut, K, group, monkeypatch):
    """Random Gaussian and tie-heavy batches against the oracle, with each
    code path forced: separate pass launches at 1, 2, 4 or 8 sequences per
    workgroup, the fused two-pass launch, or (K >= 4, "d*") the
    deferred-argmin forward and its recomputing traceback at 1, 2, 4 or 8
    sequences per workgroup; odd batch sizes included."""
    monkeypatch.setenv("XTQ_VIT_DEFER", "1" if group.startswith("d") else "0")
    if group == "fused":
        monkeypatch.setenv("XTQ_VIT_FUSED", "1")
    else:
        monkeypatch.setenv("XTQ_VIT_FUSED", "0")
        monkeypatch.setenv("XTQ_VIT_GROUP", group.lstrip("d"))
    rng = np.random.default_rng(1000 * K + (9 if group == "fused" else int(group.lstrip("d"))))
    n = 7
    X = rng.standard_normal((n, 256)).astype(np.float32)
    X[1] = mul1_lut[rng.integers(0, 65536, 256)]          # exact codebook values
    X[2] = 0.0                                             # all ties at step 0
    X[3] *= 40.0                                           # large costs
    X[4] = np.round(X[4] * 2) / 2                          # coarse grid
    for pivot, margin in ((128, 0), (3, 16), (250, 16), (200, 100), (0, 0), (0, 1),
                          (255, 0)):
        print(f"case K={K} group={group} pivot={pivot} margin={margin}", flush=True)
        want = oracle_mod.tailbite(X, mul1_lut, K, 16, pivot=pivot, margin=margin)
        got, tr = _run(hb, X, K, pivot, margin, trellis=True)
        np.testing.assert_array_equal(got, want)
        np.testing.assert_array_equal(tr, oracle_mod.pack(want, K))


@pytest.mark.parametrize("K", range(2, 8))
def test_lane_traceback_vs_oracle(hb, oracle_mod, mul1_lut, K, monkeypatch):
    """The one-lane-per-sequence traceback (forced at any batch size) equals
    the oracle for tail-bites (both passes), full Viterbi runs and back_from,
    with a partly filled last workgroup."""
    monkeypatch.setenv("XTQ_VIT_FUSED", "0")
    monkeypatch.setenv("XTQ_VIT_TB_LANES", "0")
    rng = np.random.default_rng(700 + K)
    n = 70
    X = rng.standard_normal((n, 256)).astype(np.float32)
    X[5] = mul1_lut[rng.integers(0, 65536, 256)]
    X[6] = 0.0
    for pivot, margin in ((128, 0), (147, 16), (3, 100)):
        print(f"case lanes K={K} pivot={pivot} margin={margin}", flush=True)
        got, tr = _run(hb, X, K, pivot, margin, trellis=True)
        want = oracle_mod.tailbite(X, mul1_lut, K, 16, pivot=pivot, margin=margin)
        np.testing.assert_array_equal(got, want)
        np.testing.assert_array_equal(tr, oracle_mod.pack(want, K))
    Xd = torch.from_numpy(X).cuda()
    np.testing.assert_array_equal(hb.viterbi(Xd, K).cpu().numpy(),
                                  oracle_mod.viterbi(X, mul1_lut, K, 16))
    np.testing.assert_array_equal(hb.viterbi(Xd[:, :200].contiguous(), K, back_from=77).cpu().numpy(),
                                  oracle_mod.viterbi(X[:, :200], mul1_lut, K, 16, back_from=77))


@pytest.mark.parametrize("K,n", [(4, 320), (6, 320), (5, 384), (7, 64), (2, 257)])
def test_fused_ldlq_sized_batches(hb, oracle_mod, mul1_lut, K, n, monkeypatch):
    """Batch sizes of the BlockLDLQ sweep's launches (one 16-row block: tn
    tiles), where the fused two-pass launch runs by default: identical to
    the separate-launch path and to the oracle."""
    rng = np.random.default_rng(300 + K)
    X = rng.standard_normal((n, 256)).astype(np.float32)
    X[::7] = mul1_lut[rng.integers(0, 65536, (len(X[::7]), 256))]
    print(f"case fused K={K} n={n}", flush=True)
    monkeypatch.delenv("XTQ_VIT_FUSED", raising=False)
    fused, tr = _run(hb, X, K, 128, 0, trellis=True)
    monkeypatch.setenv("XTQ_VIT_FUSED", "0")
    split, _ = _run(hb, X, K, 128, 0)
    np.testing.assert_array_equal(fused, split)
    np.testing.assert_array_equal(fused, oracle_mod.tailbite(X, mul1_lut, K, 16, pivot=128,
                                                             margin=0, nthreads=8))
    np.testing.assert_array_equal(tr, oracle_mod.pack(fused, K))


@pytest.mark.parametrize("K", (2, 4, 7))
def test_batch_position_invariance(hb, K):
    """A sequence encodes identically wherever it sits in a large batch
    (chunking and grouping never mix sequences)."""
    rng = np.random.default_rng(7 + K)
    n = 2100
    X = rng.standard_normal((n, 256)).astype(np.float32)
    print(f"case K={K} n={n}", flush=True)
    st_all, _ = _run(hb, X, K, 147, 16)
    idx = np.array([0, 1, 2, 511, 1024, 1500, 2098, 2099])
    st_few, _ = _run(hb, X[idx], K, 147, 16)
    np.testing.assert_array_equal(st_all[idx], st_few)
    # tail-bite wrap invariant on the whole batch (verify_viterbi.py:61-64)
    SP = 1 << (16 - K)
    assert ((st_all[:, 0] >> K) == (st_all[:, -1] & (SP - 1))).all()


@pytest.mark.parametrize("K", (4, 5, 6, 7))
def test_deferred_chunks(hb, oracle_mod, mul1_lut, K, monkeypatch):
    """The deferred-argmin encode over a batch split into three chunks (a
    small XTQ_VIT_DEFER_SCRATCH) with a partial last one equals the
    key-argmin encode of the same batch, and each chunk's first and last 16
    tiles equal the oracle (tie-heavy rows included)."""
    rng = np.random.default_rng(60 + K)
    n = 2 * 1024 + 300
    X = rng.standard_normal((n, 256)).astype(np.float32)
    X[::97] = mul1_lut[rng.integers(0, 65536, (len(X[::97]), 256))]
    X[5::211] = 0.0
    Xd = torch.from_numpy(X).cuda()
    monkeypatch.setenv("XTQ_VIT_DEFER", "0")
    print(f"case K={K} n={n} key argmin", flush=True)
    ref, ref_tr = hb.tailbite(Xd, K, 147, 16, trellis=True)
    monkeypatch.setenv("XTQ_VIT_DEFER", "1")
    per = hb.scratch_per_seq(K)       # backpointer bytes; the minima rows are larger
    monkeypatch.setenv("XTQ_VIT_DEFER_SCRATCH", str(1024 * 255 * (1 << (16 - K)) * 4 + 4096))
    ch, deferred = hb.chunk_seqs(n, K)
    assert deferred and per > 0
    print(f"case K={K} n={n} deferred argmin, chunks of {ch}", flush=True)
    got, tr = hb.tailbite(Xd, K, 147, 16, trellis=True)
    starts = list(range(0, n, ch))
    assert len(starts) >= 3 and n - starts[-1] < ch
    assert torch.equal(got, ref) and torch.equal(tr, ref_tr)
    idx = sorted({i for c0 in starts for i in list(range(c0, c0 + 16)) +
                  list(range(min(n, c0 + ch) - 16, min(n, c0 + ch)))})
    want = oracle_mod.tailbite(X[idx], mul1_lut, K, 16, pivot=147, margin=16,
                               nthreads=len(os.sched_getaffinity(0)))
    np.testing.assert_array_equal(got[idx].cpu().numpy(), want)


def test_defer_is_opt_in(hb, monkeypatch):
    """The deferred-argmin encode runs only with XTQ_VIT_DEFER=1 and K >= 4:
    unset, "0" or any other value leave every batch on the key-argmin
    forward (xtq_vit_chunk_seqs reports the path a batch would take)."""
    monkeypatch.delenv("XTQ_VIT_DEFER", raising=False)
    for K in (2, 4, 7):
        for n in (64, 8192, 348160):
            assert hb.chunk_seqs(n, K)[1] == 0
    for v, want in (("0", 0), ("yes", 0), ("1", 1)):
        monkeypatch.setenv("XTQ_VIT_DEFER", v)
        assert hb.chunk_seqs(8192, 4)[1] == want
        assert hb.chunk_seqs(8192, 3)[1] == 0


@pytest.mark.parametrize("K", (2, 4, 7))
def test_forced_chunks(hb, oracle_mod, mul1_lut, K, monkeypatch):
    """XTQ_VIT_SCRATCH is read on every call: a budget of 2048 sequences
    splits a batch of 2 x 2048 + 700 into three chunks with a partial last
    one (the full chunks take the separate-pass path with one-lane
    tracebacks, the last the fused path).  Every tile equals the unchunked
    run, and the first and last 32 tiles of each chunk equal the oracle."""
    per = hb.scratch_per_seq(K)
    rnd = 4 * torch.cuda.get_device_properties(0).multi_processor_count
    ch = 2048 if 2048 <= rnd else 2048 - 2048 % rnd
    n = 2 * 2048 + 700
    rng = np.random.default_rng(40 + K)
    X = torch.from_numpy(rng.standard_normal((n, 256)).astype(np.float32)).cuda()
    monkeypatch.delenv("XTQ_VIT_SCRATCH", raising=False)
    monkeypatch.setenv("XTQ_VIT_DEFER", "0")
    print(f"case K={K} n={n} unchunked", flush=True)
    ref, ref_tr = hb.tailbite(X, K, 147, 16, trellis=True)
    monkeypatch.setenv("XTQ_VIT_SCRATCH", str(2048 * per))
    print(f"case K={K} n={n} chunks of {ch}", flush=True)
    got, tr = hb.tailbite(X, K, 147, 16, trellis=True)
    starts = list(range(0, n, ch))
    assert len(starts) >= 3 and n - starts[-1] < ch
    assert torch.equal(got, ref) and torch.equal(tr, ref_tr)
    idx = sorted({i for c0 in starts for i in list(range(c0, c0 + 32)) +
                  list(range(min(n, c0 + ch) - 32, min(n, c0 + ch)))})
    want = oracle_mod.tailbite(X[idx].cpu().numpy(), mul1_lut, K, 16, pivot=147, margin=16,
                               nthreads=len(os.sched_getaffinity(0)))
    np.testing.assert_array_equal(got[idx].cpu().numpy(), want)


@pytest.mark.parametrize("K", range(2, 8))
def test_decode_unpack_pack(hb, oracle_mod, mul1_lut, K):
    """decode/unpack/pack kernels equal the oracle and the reference fixture."""
    g = load_golden("tailbite.npz")
    P = g[f"P_K{K}"]                                       # [6, 16K] from the reference
    tr = torch.from_numpy(P).cuda().view(2, 3, 16 * K)
    w = hb.decode(tr, K)
    np.testing.assert_array_equal(w.cpu().numpy(), g[f"D_K{K}"])
    w16 = hb.decode(tr, K, dtype=torch.float16)
    np.testing.assert_array_equal(w16.float().cpu().numpy(), g[f"D_K{K}"])
    st = hb.unpack(tr.view(-1, 16 * K), K)
    np.testing.assert_array_equal(st.cpu().numpy(), g[f"U_K{K}"])
    rp = hb.pack(st, K)
    np.testing.assert_array_equal(rp.cpu().numpy(), P)
    rng = np.random.default_rng(K)
    rnd = rng.integers(-32768, 32768, (5, 7, 16 * K)).astype(np.int16)
    w = hb.decode(torch.from_numpy(rnd).cuda(), K)
    np.testing.assert_array_equal(w.cpu().numpy(), oracle_mod.decode(rnd, mul1_lut, K))


def test_nan_target_rejected(hb):
    X = torch.randn(3, 256, device="cuda")
    X[1, 17] = float("nan")
    with pytest.raises(hb.HipViterbiError) as ei:
        hb.tailbite(X, 4, 128, 0)
    assert ei.value.rc == 11
    # the library recovers: a clean call afterwards succeeds
    st, _ = hb.tailbite(torch.randn(2, 256, device="cuda"), 4, 128, 0)
    assert st.shape == (2, 256)


def test_valu_probe_rates():
    """The roofline probe (its own library) runs and reports plausible rates:
    every probe between 0.5x and 2.5x of one wave64 instruction per SIMD per
    4 cycles."""
    import os
    import sys
    from conftest import PKG
    if os.path.join(PKG, "probe") not in sys.path:
        sys.path.insert(0, os.path.join(PKG, "probe"))
    import valu_probe
    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    base = ncu * 64 * 2.4e9
    rates = {}
    for i, name in enumerate(valu_probe.PROBES):
        r = valu_probe.rate(i)
        rates[name] = r
        print(f"probe {name}: {r / 1e12:.2f} T/s", flush=True)
        assert 0.5 * base < r < 2.5 * base, (name, r)
    # a mix at one workgroup per CU (4 waves per SIMD) issues no faster than
    # with two (8 waves per SIMD) beside it
    for mix in ("fp32-code candidate mix, grouped by opcode",
                "deferred-argmin mix (3.5 instructions per candidate), grouped by opcode"):
        assert rates[mix + ", one workgroup per CU"] < 1.05 * rates[mix], mix


def test_async_encode_and_status(hb, oracle_mod, mul1_lut):
    """Stream-ordered encodes equal the synchronous ones; a NaN target is
    reported by the next status check (and only once)."""
    rng = np.random.default_rng(11)
    X = torch.from_numpy(rng.standard_normal((40, 256)).astype(np.float32)).cuda()
    want, _ = hb.tailbite(X, 5, 147, 16)
    outs = [hb.tailbite(X[i:i + 8], 5, 147, 16, sync=False)[0] for i in range(0, 40, 8)]
    hb.status()
    np.testing.assert_array_equal(torch.cat(outs).cpu().numpy(), want.cpu().numpy())
    Xn = X.clone()
    Xn[3, 200] = float("nan")
    hb.tailbite(Xn, 5, 147, 16, sync=False)
    with pytest.raises(hb.HipViterbiError) as ei:
        hb.status()
    assert ei.value.rc == 11
    hb.status()                                      # flag cleared


def test_async_two_streams_share_scratch(hb, oracle_mod, mul1_lut):
    """Encodes issued on two streams without host waits in between (they
    share the library's backpointer scratch) each match the oracle."""
    rng = np.random.default_rng(12)
    Xa = rng.standard_normal((300, 256)).astype(np.float32)
    Xb = rng.standard_normal((700, 256)).astype(np.float32)
    da, db = torch.from_numpy(Xa).cuda(), torch.from_numpy(Xb).cuda()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(s1):
        sa, _ = hb.tailbite(da, 4, 128, 0, sync=False)
    with torch.cuda.stream(s2):
        sb, _ = hb.tailbite(db, 4, 128, 0, sync=False)
    torch.cuda.synchronize()
    hb.status()
    np.testing.assert_array_equal(sa.cpu().numpy(),
                                  oracle_mod.tailbite(Xa, mul1_lut, 4, 16, pivot=128, margin=0))
    np.testing.assert_array_equal(sb.cpu().numpy(),
                                  oracle_mod.tailbite(Xb, mul1_lut, 4, 16, pivot=128, margin=0))


def test_inf_targets_match_oracle(hb, oracle_mod, mul1_lut):
    """+-inf targets give all-inf costs; ties resolve like the reference."""
    X = np.random.default_rng(3).standard_normal((2, 256)).astype(np.float32)
    X[0, 5] = np.inf
    X[1, 100:110] = -np.inf
    want = oracle_mod.tailbite(X, mul1_lut, 4, 16, pivot=128, margin=0)
    got, _ = _run(hb, X, 4, 128, 0)
    np.testing.assert_array_equal(got, want)


def test_host_entry_matches_device(hb, mul1_lut):
    """xtq_vit_run (reference ABI, host pointers, K=4) equals the device entry."""
    import ctypes
    X = np.random.default_rng(11).standard_normal((5, 256)).astype(np.float32)
    out = np.empty((5, 256), dtype=np.int32)
    rc = hb.lib().xtq_vit_run(X.ctypes.data_as(ctypes.c_void_p), 5, b"mul1p", 16, 147,
                              out.ctypes.data_as(ctypes.c_void_p))
    assert rc == 0
    got, _ = _run(hb, X, 4, 147, 16)
    np.testing.assert_array_equal(out, got)
    out2 = np.empty((5, 256), dtype=np.int32)
    rc = hb.lib().xtq_vit_run_k(X.ctypes.data_as(ctypes.c_void_p), 5, 6, b"mul1", 0, 9,
                                out2.ctypes.data_as(ctypes.c_void_p))
    assert rc == 0
    got6, _ = _run(hb, X, 6, 9, 0)
    np.testing.assert_array_equal(out2, got6)
    rc = hb.lib().xtq_vit_run(X.ctypes.data_as(ctypes.c_void_p), 5, b"ih2x2", 0, 128,
                              out.ctypes.data_as(ctypes.c_void_p))
    assert rc == 8
    # a negative margin runs pass 1 over the whole sequence, as the
    # reference kernel does (viterbi_esimd.cpp:413-414)
    out3 = np.empty((5, 256), dtype=np.int32)
    rc = hb.lib().xtq_vit_run(X.ctypes.data_as(ctypes.c_void_p), 5, b"mul1", -7, 128,
                              out3.ctypes.data_as(ctypes.c_void_p))
    assert rc == 0
    np.testing.assert_array_equal(out3, _run(hb, X, 4, 128, 0)[0])


def test_other_codebooks(hb, oracle_mod):
    """3inst and mcg codebooks (fp16-exact) run through the same kernel."""
    X = np.random.default_rng(5).standard_normal((3, 256)).astype(np.float32)
    for name, short in (("exl3_3inst", "3inst"), ("exl3_mcg", "mcg")):
        lut = oracle_mod.code_lut(name)
        want = oracle_mod.tailbite(X, lut, 3, 16, pivot=128, margin=0)
        Xd = torch.from_numpy(X).cuda()
        st, _ = hb.tailbite(Xd, 3, 128, 0, code=short)
        np.testing.assert_array_equal(st.cpu().numpy(), want)


@pytest.mark.parametrize("group", ("1", "2", "4", "8", "fused", "d4"))
def test_1mad_vs_reference_golden(hb, oracle_mod, group, monkeypatch):
    """QTIP's 1MAD code -- fp32 table values, (bytesum - 510) / 147.8, not
    fp16-exact -- through every forward path: the reference's own states on
    Gaussian and tie-forcing targets (codes.npz) at K = 2, 4, 7, and the
    oracle with that table on random batches; the packed trellis too."""
    monkeypatch.setenv("XTQ_VIT_DEFER", "1" if group.startswith("d") else "0")
    if group == "fused":
        monkeypatch.setenv("XTQ_VIT_FUSED", "1")
    else:
        monkeypatch.setenv("XTQ_VIT_FUSED", "0")
        monkeypatch.setenv("XTQ_VIT_GROUP", group.lstrip("d"))
    g = load_golden("codes.npz")
    lut = oracle_mod.code_lut("qtip_1mad")
    rng = np.random.default_rng(77)
    for K in (2, 4, 7):
        if group.startswith("d") and K < 4:
            continue
        X = g[f"mad_X_K{K}"]
        Xd = torch.from_numpy(X).cuda()
        for p, m in ((128, 0), (147, 16)):
            print(f"case 1mad K={K} group={group} pivot={p} margin={m}", flush=True)
            st, tr = hb.tailbite(Xd, K, p, m, code="1mad", trellis=True)
            want = g[f"mad_S_K{K}_m{m}_p{p}"]
            np.testing.assert_array_equal(st.cpu().numpy(), want)
            np.testing.assert_array_equal(tr.cpu().numpy(), oracle_mod.pack(want, K))
        Xr = rng.standard_normal((9, 256)).astype(np.float32)
        Xr[1] = lut[rng.integers(0, 65536, 256)]
        st, _ = hb.tailbite(torch.from_numpy(Xr).cuda(), K, 5, 16, code="1mad")
        np.testing.assert_array_equal(st.cpu().numpy(),
                                      oracle_mod.tailbite(Xr, lut, K, 16, pivot=5, margin=16))


@pytest.mark.parametrize("K", (2, 4))
@pytest.mark.parametrize("code", ("exl3_mul1", "qtip_1mad"))
def test_gaussian_mse_on_gpu(xq, oracle_mod, code, K):
    """The reference's rate-distortion check (test_quantize.py:183-202) on the
    GPU: rms-matched Gaussian targets, 2,048 tiles through
    quantize_seq_tailbite, MSE below 3 x 2^-2K, for both codes; the decode of
    the states with the code's fp32 table matches the oracle's decode."""
    torch.manual_seed(3)
    lut = xq.get_lut(code, 16)
    lut_rms = lut.double().square().mean().sqrt().float()
    X = torch.randn(256, 2048)
    X = X / X.square().mean().sqrt() * lut_rms
    print(f"case gaussian mse {code} K={K}", flush=True)
    st = xq.quantize_seq_tailbite(X.cuda(), lut.cuda(), K, 16)
    dec = lut.cuda()[st].t().contiguous().flatten()
    mse = float((dec - X.cuda().t().reshape(-1)).square().mean() / X.square().mean())
    print(f"{code} K={K}: mse {mse:.5f} vs bound {2.0 ** (-2 * K):.5f}", flush=True)
    assert mse < 3.0 * 2.0 ** (-2 * K)
    short = {"exl3_mul1": "mul1", "qtip_1mad": "1mad"}[code]
    st32 = st.t().contiguous().to(torch.int32)[:32]
    tr = xq._hb.pack(st32, K).view(2, 16, 16 * K)
    np.testing.assert_array_equal(
        xq._hb.decode(tr, K, code=short).cpu().numpy(),
        oracle_mod.decode(tr.cpu().numpy(), oracle_mod.code_lut(code), K))


def test_verify_viterbi_readme_case(hb, oracle_mod, mul1_lut):
    """The reference's kernel-tier check (verify_viterbi.py:20-65) on its
    README case (seed 1, 64 sequences, code mul1, margin 0, pivot 128,
    README.md:181-185), through the drop-in host entry xtq_vit_run: every
    sequence exact (the reference passes at >= 99 %), decoded MSE equal, every
    sequence circular-consistent."""
    import ctypes
    nseq = 64
    X = np.random.default_rng(1).standard_normal((nseq, 256), dtype=np.float32)
    out = np.empty((nseq, 256), dtype=np.int32)
    rc = hb.lib().xtq_vit_run(X.ctypes.data_as(ctypes.c_void_p), nseq, b"mul1", 0, 128,
                              out.ctypes.data_as(ctypes.c_void_p))
    assert rc == 0
    ref = oracle_mod.tailbite(X, mul1_lut, 4, 16, pivot=128, margin=0)
    assert int((out == ref).all(axis=1).sum()) == nseq
    mse_k = float(((mul1_lut[out] - X) ** 2).mean())
    mse_r = float(((mul1_lut[ref] - X) ** 2).mean())
    assert mse_k == mse_r
    assert int(((out[:, 0] >> 4) == (out[:, -1] & ((1 << 12) - 1))).sum()) == nseq
