"""Config-scale parity on the GPU: the synthetic workloads c2..c5 at their full
sizes through quantize_linear / quantize_linear_group (BlockLDLQ and the
tail-biting encode on the GPU), and the 348,160-tile kernel workload through
the batched encoder, in the manner of the reference's whole-tensor check
(check_tensor_bitexact.py:69-123, README.md:163-166).

Every tile of every run:
  * the tail-bite wrap invariant s_0 >> K == s_255 mod 2^(16-K)
    (verify_viterbi.py:61-64);
  * pack(unpack(trellis)) == trellis (quantize.py:848-851);
  * decode(trellis) reproduces W_hat: the decoded inner tiles, taken back
    through the incoherence transform, equal quantize_linear's W_hat bit for
    bit (quantize.py:852-853, 862-866).
Sampled block rows spread over the sweep (the first row swept, which has no
feedback, the last, which has the most, and rows between; 8 rows, 16 for
c2): every tile's
states bit for bit against the C oracle on the targets the kernel computed
(the reference's per-launch dual method, quantize.py:687-717).  The batched
workload checks the first and last 64 tiles of every scratch chunk the
library processes, and a random sample, against the oracle.

Every tile, bit for bit: the headline batch, c2, c4 and c5 at K=4 are also
encoded tile by tile by the reference's own torch Viterbi (the tensor
operations of quantize.py:218-354, oracle/torch_port.py) run on the GPU, on
the same targets, and every tile's states must match -- the reference's
whole-tensor check (check_tensor_bitexact.py:69-123).  The GPU run of that
port is itself pinned to the C oracle on tie-heavy tiles for every K first.
"""
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

NTHREADS = len(os.sched_getaffinity(0))


@pytest.fixture(scope="module")
def xq():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import quantize
    return quantize


@pytest.fixture(scope="module")
def hb():
    import hip_backend
    hip_backend.lib()
    return hip_backend


@pytest.fixture(scope="module")
def wl():
    import workloads
    return workloads


def _sample_rows(tk: int, n: int):
    """n block rows in sweep order: tk-1 (swept first) .. 0 (swept last)."""
    return sorted({tk - 1 - (r * (tk - 1)) // (n - 1) for r in range(n)}, reverse=True)


def _every_tile(hb, trellis: torch.Tensor, K: int) -> torch.Tensor:
    """Wrap invariant and pack/unpack round trip on every tile; returns the
    states [ntile, 256] (device)."""
    tr = trellis.reshape(-1, 16 * K).contiguous()
    st = hb.unpack(tr, K)
    SP = 1 << (16 - K)
    wrap = (st[:, 0] >> K) == (st[:, 255] & (SP - 1))
    assert bool(wrap.all()), f"wrap invariant broken on {int((~wrap).sum())} tiles"
    assert torch.equal(hb.pack(st, K), tr), "pack(unpack(trellis)) != trellis"
    return st


def _oracle_rows(O, lut, xt: torch.Tensor, st: torch.Tensor, rows, K: int, label: str,
                 pivot: int = 128, margin: int = 0):
    """States of block rows `rows` against the C oracle on the kernel's own
    targets xt [tk, tn, 256]; st [tk, tn, 256]."""
    checked = 0
    for i in rows:
        X = xt[i].cpu().numpy()
        want = O.tailbite(X, lut, K, 16, pivot=pivot, margin=margin, nthreads=NTHREADS)
        got = st[i].cpu().numpy()
        bad = np.nonzero((got != want).any(axis=1))[0]
        assert bad.size == 0, f"{label}: block row {i}: tiles {bad[:8].tolist()} differ"
        checked += X.shape[0]
    print(f"{label}: {checked} tiles of rows {list(rows)} exact vs oracle", flush=True)
    return checked


PORT_BATCH = 16384          # tiles per torch-port launch (4 GiB of fp32 costs)


def _every_tile_vs_port(lutd, X: torch.Tensor, st: torch.Tensor, K: int, label: str,
                        pivot: int = 128, margin: int = 0) -> int:
    """States st [n, 256] of targets X [n, 256] (both on the GPU) against the
    reference's torch tail-bite run on the GPU, every tile."""
    from oracle import torch_port as TP
    n = X.shape[0]
    bad = 0
    for c0 in range(0, n, PORT_BATCH):
        c1 = min(n, c0 + PORT_BATCH)
        want = TP.tailbite(X[c0:c1].t().contiguous(), lutd, K, 16, pivot=pivot, margin=margin)
        bad += int((want.t() != st[c0:c1].long()).any(dim=1).sum())
    assert bad == 0, f"{label}: {bad} of {n} tiles differ from the reference's torch Viterbi"
    print(f"{label}: every tile ({n}) exact vs the reference's torch Viterbi on the GPU",
          flush=True)
    return n


def test_torch_port_on_gpu_vs_oracle(oracle_mod):
    """The torch port run on the GPU (the every-tile checker below) against the
    C oracle: Gaussian, exact-codebook (tie-heavy) and all-zero targets, every K,
    the default and the reference harness's pivot/margin."""
    lut = oracle_mod.code_lut("exl3_mul1")
    lutd = torch.from_numpy(lut).cuda()
    from oracle import torch_port as TP
    rng = np.random.default_rng(11)
    X = rng.standard_normal((192, 256)).astype(np.float32)
    X[:64] = lut[rng.integers(0, 65536, (64, 256))]
    X[64:80] = 0.0
    X[80:96] = np.round(X[80:96] * 4) / 4
    for K in range(2, 8):
        for pivot, margin in ((128, 0), (147, 16)):
            want = oracle_mod.tailbite(X, lut, K, 16, pivot=pivot, margin=margin,
                                       nthreads=NTHREADS)
            got = TP.tailbite(torch.from_numpy(X.T.copy()).cuda(), lutd, K, 16, pivot=pivot,
                              margin=margin).t().cpu().numpy()
            assert np.array_equal(got, want), f"torch port on the GPU != oracle (K={K}, p={pivot})"


def _reconstruct(xq, hb, r, K: int, cs: bool) -> torch.Tensor:
    """W_hat [out, in] from the member's trellis alone, on the GPU, with
    quantize_linear's own transform (quantize.py:862-866)."""
    dev = torch.device("cuda")
    tr = r["trellis"].to(dev)
    hw = hb.decode(tr, K)                                       # [in, out] inner
    h = xq.hadamard128(dev, torch.float32)
    suh, svh = r["suh"].to(dev), r["svh"].to(dev)
    if cs:
        W_hat = xq.from_inner(hw, suh, svh, h)
    else:
        W_hat = xq.from_inner(hw * r["Wscale"], suh, svh, h)
    return W_hat.t().contiguous()


def _run_config(xq, hb, O, Ws, H, Ks, cs, rows_per_run, label, every_tile=False):
    """quantize_linear_group on the GPU with the kernel's targets kept; every
    tile checked, sampled block rows against the oracle (and, with
    every_tile, every tile against the reference's torch Viterbi)."""
    lut = O.code_lut("exl3_mul1")
    dev = torch.device("cuda")
    Ws = [W.float().to(dev) for W in Ws]
    xq.ldlq_viterbi.keep_targets = True
    try:
        rs = xq.quantize_linear_group(Ws, H.to(dev), K=Ks, device="cuda", margin=0,
                                      channel_scales=cs)
        xt = xq.ldlq_viterbi.last_targets
        groups = xq.ldlq_viterbi.last_groups
        if groups is None:
            groups = [(0, xt.shape[1] * 16, Ks if isinstance(Ks, int) else Ks[0],
                       xq.ldlq_viterbi.last_trellis)]
    finally:
        xq.ldlq_viterbi.keep_targets = False
        xq.ldlq_viterbi.last_targets = None
    assert xt is not None
    tk = xt.shape[0]
    total = checked = 0
    for c0, nc, K, tr in groups:
        st = _every_tile(hb, tr, K).view(tk, nc // 16, 256)
        total += st.shape[0] * st.shape[1]
        checked += _oracle_rows(O, lut, xt[:, c0 // 16:(c0 + nc) // 16], st,
                                _sample_rows(tk, rows_per_run), K, f"{label} K={K}")
        if every_tile:
            _every_tile_vs_port(torch.from_numpy(lut).to(dev),
                                xt[:, c0 // 16:(c0 + nc) // 16].reshape(-1, 256),
                                st.reshape(-1, 256), K, f"{label} K={K}")
    Kl = [Ks] * len(Ws) if isinstance(Ks, int) else list(Ks)
    for W, r, K in zip(Ws, rs, Kl):
        assert r["trellis"].shape == (W.shape[1] // 16, W.shape[0] // 16, 16 * K)
        assert torch.equal(_reconstruct(xq, hb, r, K, cs), r["W_hat"].to(dev)), \
            f"{label}: decode of the trellis does not reproduce W_hat"
    print(f"{label}: every tile of {total} wrap/round-trip/decode checked, "
          f"{checked} vs oracle", flush=True)
    return rs


def test_c2_full_size(xq, hb, wl, oracle_mod):
    print("case c2 4096x4096 K=4", flush=True)
    w = wl.c2(device="cuda")
    _run_config(xq, hb, oracle_mod, [w["W"]], w["H"], 4, False, 16, "c2", every_tile=True)


@pytest.fixture(scope="module")
def c3(wl):
    w = wl.c3(device="cuda")
    yield w
    del w


@pytest.mark.parametrize("K", range(2, 8))
def test_c3_full_size(xq, hb, c3, oracle_mod, K):
    print(f"case c3 5120x5120 K={K}", flush=True)
    _run_config(xq, hb, oracle_mod, [c3["W"]], c3["H"], K, False, 8, f"c3 K={K}")


def test_c4_full_size(xq, hb, wl, oracle_mod):
    print("case c4 qkv K=[5,7,7] channel scales", flush=True)
    w = wl.c4(device="cuda")
    Ks = [m["K"] for m in w["members"]]
    _run_config(xq, hb, oracle_mod, [m["W"] for m in w["members"]], w["H"], Ks, True, 8,
                "c4", every_tile=True)


@pytest.fixture(scope="module")
def c5(wl):
    w = wl.c5(device="cuda")
    yield w
    del w


@pytest.mark.parametrize("K", (6, 4))
def test_c5_full_size(xq, hb, c5, oracle_mod, K):
    print(f"case c5 5120x17408 K={K}", flush=True)
    _run_config(xq, hb, oracle_mod, [c5["W"]], c5["H"], K, False, 8, f"c5 K={K}",
                every_tile=(K == 4))


def test_c5_harness_quantize(xq, hb, c5, oracle_mod):
    """The reference's whole-tensor verification path at c5's shape
    (check_tensor_bitexact.py:45-66,93-123): the weight taken to the inner
    domain and the harness-convention factor U (U^T U = G^-1 of the rotated,
    1 %-damped Hessian, built in fp64), then quantize() with seed 20261011
    (pivot 147) and margin 16 at K=4 -- the U -> L conversion, the sweep and
    the checks all on the GPU.  Every tile: wrap invariant, pack/unpack round
    trip, decode x scale == W_hat, and its states against the reference's
    torch Viterbi run on the GPU on the kernel's own targets; 8 block rows
    spread over the sweep against the C oracle."""
    seed, pivot, margin, K = 20261011, 147, 16, 4
    assert seed % 256 == pivot
    print(f"case c5 quantize() harness: U factor, seed {seed}, margin {margin}, K={K}",
          flush=True)
    dev = torch.device("cuda")
    W = c5["W"].float().to(dev)                          # [5120 out, 17408 in]
    k_in, m_out = W.shape[1], W.shape[0]
    suh = xq.sign_vec(k_in, seed, dev).half()
    svh = xq.sign_vec(m_out, seed + 1, dev).half()
    h = xq.hadamard128(dev, torch.float32)
    W_t = xq.to_inner(W.t().contiguous(), suh, svh, h).t().contiguous()   # [out, in]
    del W
    G = xq.rotate_hessian(c5["H"].float().to(dev), suh, h)
    G.diagonal().add_(0.01 * G.diagonal().mean())
    Gi = torch.cholesky_inverse(torch.linalg.cholesky(G.double()))
    del G
    U = torch.linalg.cholesky(Gi, upper=True)
    err = float((U.t() @ U - Gi).abs().max())
    del Gi
    U = U.float()
    print(f"U built on the GPU, |U^T U - G^-1| max {err:.2e}", flush=True)
    xq.ldlq_viterbi.keep_targets = True
    try:
        W_hat, packed, scale = xq.quantize(W_t, U, "exl3_mul1", K, seed, margin=margin)
        xt = xq.ldlq_viterbi.last_targets
    finally:
        xq.ldlq_viterbi.keep_targets = False
        xq.ldlq_viterbi.last_targets = None
    del U
    tk, tn = k_in // 16, m_out // 16
    assert packed.shape == (tk, tn, 16 * K) and W_hat.shape == (m_out, k_in)
    st = _every_tile(hb, packed, K).view(tk, tn, 256)
    assert torch.equal((hb.decode(packed.to(dev), K) * scale).t().contiguous(), W_hat), \
        "decode(packed) x scale does not reproduce W_hat"
    lut = oracle_mod.code_lut("exl3_mul1")
    _oracle_rows(oracle_mod, lut, xt, st, _sample_rows(tk, 8), K, "c5 harness",
                 pivot=pivot, margin=margin)
    _every_tile_vs_port(torch.from_numpy(lut).to(dev), xt.reshape(-1, 256),
                        st.reshape(-1, 256), K, "c5 harness", pivot=pivot, margin=margin)
    rel = xq.rel_mse(W_t, W_hat)
    print(f"c5 harness: rel MSE {rel:.4e}, scale {scale:.6e}", flush=True)
    assert 0.0 < rel < 0.02


def test_headline_batch_every_chunk(hb, wl, oracle_mod):
    """The benchmark's 348,160 independent K=4 tiles in one call: every tile's
    wrap invariant and pack round trip; the first and last 64 tiles of every
    scratch chunk (the chunk loop's offsets into targets, states and trellis,
    and the partial last chunk) and 4,096 random tiles against the oracle;
    every tile against the reference's torch Viterbi run on the GPU."""
    saved = {v: os.environ.pop(v, None) for v in ("XTQ_VIT_SCRATCH", "XTQ_VIT_DEFER",
                                                   "XTQ_VIT_DEFER_SCRATCH")}
    try:
        print("case headline 348160 tiles K=4 pivot 128 margin 0", flush=True)
        X = wl.c5_tiles("cuda")
        n = X.shape[0]
        assert n == 348160
        _, tr = hb.tailbite(X, 4, 128, 0, states=False, trellis=True)
        st = _every_tile(hb, tr, 4)
        ch, deferred = hb.chunk_seqs(n, 4)
        starts = list(range(0, n, ch))
        print(f"{len(starts)} chunks of {ch} (last {n - starts[-1]}), deferred argmin "
              f"{deferred}", flush=True)
        assert len(starts) >= 3 and n - starts[-1] < ch
        idx = set()
        for c0 in starts:
            c1 = min(n, c0 + ch)
            idx.update(range(c0, c0 + 64))
            idx.update(range(c1 - 64, c1))
        rng = np.random.default_rng(0)
        idx.update(rng.choice(n, 4096, replace=False).tolist())
        idx = np.array(sorted(idx))
        lut = oracle_mod.code_lut("exl3_mul1")
        want = oracle_mod.tailbite(X[torch.from_numpy(idx).cuda()].cpu().numpy(), lut, 4, 16,
                                   pivot=128, margin=0, nthreads=NTHREADS)
        got = st[torch.from_numpy(idx).cuda()].cpu().numpy()
        bad = idx[(got != want).any(axis=1)]
        assert bad.size == 0, f"tiles {bad[:8].tolist()} differ from the oracle"
        print(f"headline: {idx.size} tiles exact vs oracle, every tile wrap/round trip",
              flush=True)
        _every_tile_vs_port(torch.from_numpy(lut).cuda(), X, st, 4, "headline")
    finally:
        for v, val in saved.items():
            if val is not None:
                os.environ[v] = val
