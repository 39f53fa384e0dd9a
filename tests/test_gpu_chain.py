"""GPU tests of the column-chain BlockLDLQ schedule (xtq_ldlq_chain_dev).

The chain kernel computes every tile's targets itself, from the decoded
tiles below it in its column, and encodes them.  The tests check
  * every tile's targets bit for bit against the reference's own fp32
    sweep (quantize.py:662-686,743-744, torch CPU GEMMs) on the kernel's
    What, and against the target formula X = W[block] + L[later, block]^T
    (W - What)[later] evaluated in fp64, within the rounding bound of the
    fp32 sums -- a wrong index, sign or row range of the feedback misses it
    by orders of magnitude;
  * the whole sweep against the reference's block schedule on the CPU on
    the same inputs, What and states bit for bit;
  * every tile's states bit for bit against the oracle on those targets, and
    the packed trellis against the oracle's packing;
  * decode(trellis) == What;
  * whole-layer proxy loss against the reference's block schedule.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

U32 = 2.0 ** -24


@pytest.fixture(scope="module")
def xq():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import quantize
    return quantize


@pytest.fixture(scope="module")
def hb():
    import hip_backend
    return hip_backend


def _lfac(xq, k, seed, rho=0.5):
    import workloads as wl
    G = wl.ar1_gram(k, 2 * k, rho, seed).double()
    G.diagonal().add_(0.01 * G.diagonal().mean())
    L, _ = xq.block_LDL(G, 16)
    return L.float()


def _seq_order(T: torch.Tensor, perm: torch.Tensor) -> torch.Tensor:
    """[k, n] -> [k/16, n/16, 256]: tile (i, j) in sequence order
    x_t = tile[perm[t]] (quantize.py:684-686)."""
    k, n = T.shape
    tiles = T.reshape(k // 16, 16, n // 16, 16).permute(0, 2, 1, 3).reshape(k // 16, n // 16, 256)
    return tiles[..., perm]


def _ref_targets(Wq, Lf, hatW, perm, buf_cols=128):
    """Every tile's targets [k/16, n/16, 256] as the reference's ldlq_viterbi
    computes them (quantize.py:662-686,743-744: lazily buffered feedback,
    torch CPU GEMMs), given the final What (the error of the rows below a
    block is final when the block is swept)."""
    k, n = Wq.shape
    tk, per = k // 16, max(1, buf_cols // 16)
    W_t, hatW_t = Wq.t().contiguous(), hatW.t().contiguous()
    prod = torch.zeros(k, n)
    X = torch.empty(tk, n // 16, 256)
    for cur in range(tk, 0, -per):
        lo = max(0, cur - per)
        for i in range(cur - 1, lo - 1, -1):
            c0, c1 = 16 * i, 16 * (i + 1)
            rows = W_t[:, c0:c1].t().contiguous()
            if c1 < 16 * cur:
                err = (W_t[:, c1:16 * cur] - hatW_t[:, c1:16 * cur]).t()
                rows = rows + Lf[c1:16 * cur, c0:c1].t() @ err
            rows = rows + prod[c0:c1, :]
            X[i] = rows.view(16, n // 16, 16).permute(1, 0, 2).reshape(n // 16, 256)[:, perm]
        if lo > 0:
            err = (W_t[:, 16 * lo:16 * cur] - hatW_t[:, 16 * lo:16 * cur]).t()
            prod += Lf[16 * lo:16 * cur, :].t() @ err
    return X


def _check_targets(W, L, hatW, xt, perm):
    """xt against the fp64 formula on the kernel's What, within a rounding
    bound, and bit for bit against the reference's own fp32 sweep on the
    kernel's What (the kernel sums in that order).  Each feedback term is
    one fused multiply-add chain of at most 128 products, the chains are
    added one after another (k/128 of them) and then W: the error is below
    (128 + k/128 + 3) u times |W| + sum |L| |E| (u = 2^-24)."""
    k, n = W.shape
    if L is not None:
        assert torch.equal(xt, _ref_targets(W, L, hatW, perm)), \
            "targets differ from the reference's sweep on the same What"
    else:
        assert torch.equal(xt, _seq_order(W, perm)), "targets without feedback != W"
    W64 = W.double()
    E = (W - hatW).double()              # the kernel's fp32 E, exactly
    X64, B = W64.clone(), W64.abs()
    if L is not None:
        L64 = L.double()
        for i in range(k // 16 - 1):
            r0, r1 = 16 * i, 16 * (i + 1)
            X64[r0:r1] += L64[r1:, r0:r1].t() @ E[r1:]
            B[r0:r1] += L64[r1:, r0:r1].abs().t() @ E[r1:].abs()
    d = (xt.double() - _seq_order(X64, perm)).abs()
    lim = (128 + k / 128 + 3) * U32 * _seq_order(B, perm)
    assert (d <= lim).all(), f"worst excess {float((d - lim).max()):.3e}"
    return float(d.max())


def _check_tiles(oracle_mod, lut, K, pivot, margin, st, tr, xt, rows=None, cols=None):
    """States of the selected tiles bit-exact with the oracle on the kernel's
    own targets; trellis == oracle packing of those states."""
    xs = xt if rows is None else xt[rows][:, cols]
    ss = st if rows is None else st[rows][:, cols]
    ts = tr if rows is None else tr[rows][:, cols]
    want = oracle_mod.tailbite(xs.reshape(-1, 256).numpy(), lut, K, 16, pivot=pivot,
                               margin=margin, nthreads=8)
    np.testing.assert_array_equal(ss.reshape(-1, 256).numpy(), want)
    np.testing.assert_array_equal(ts.reshape(-1, 16 * K).numpy(), oracle_mod.pack(want, K))


@pytest.mark.parametrize("K,k,n,pivot,margin", [
    (2, 128, 64, 128, 0), (3, 64, 96, 147, 16), (4, 128, 64, 128, 0),
    (5, 96, 48, 5, 16), (6, 64, 64, 128, 0), (7, 128, 32, 250, 0)])
def test_chain_vs_oracle(xq, hb, oracle_mod, mul1_lut, K, k, n, pivot, margin):
    g = torch.Generator().manual_seed(40 + K)
    W = torch.randn(k, n, generator=g)
    L = _lfac(xq, k, K)
    print(f"case chain K={K} {k}x{n} pivot={pivot} margin={margin}", flush=True)
    hatW, st, tr, xt = hb.ldlq_chain(W.cuda(), L.cuda(), K, pivot, margin, targets=True)
    hatW, st, tr, xt = (t.cpu() for t in (hatW, st, tr, xt))
    perm = xq.tensor_core_perm()
    _check_targets(W, L, hatW, xt, perm)
    _check_tiles(oracle_mod, mul1_lut, K, pivot, margin, st, tr, xt)
    np.testing.assert_array_equal(hatW.numpy(), oracle_mod.decode(tr.numpy(), mul1_lut, K))


@pytest.mark.parametrize("name,short,K", [("exl3_3inst", "3inst", 4), ("exl3_mcg", "mcg", 6),
                                          ("qtip_1mad", "1mad", 5)])
def test_chain_other_codebooks(xq, hb, oracle_mod, name, short, K):
    """The 3inst and mcg codebooks (fp16-exact, quantize.py:64-71) and QTIP's
    1MAD code (fp32 values, quantize.py:82-86) through the chain: targets
    against the fp64 formula, states and packing against the oracle with that
    codebook's table, decode with the same table."""
    g = torch.Generator().manual_seed(60 + K)
    W = torch.randn(96, 64, generator=g)
    L = _lfac(xq, 96, K)
    lut = oracle_mod.code_lut(name)
    print(f"case chain code={short} K={K} 96x64", flush=True)
    hatW, st, tr, xt = (t.cpu() for t in hb.ldlq_chain(W.cuda(), L.cuda(), K, 128, 0,
                                                      code=short, targets=True))
    _check_targets(W, L, hatW, xt, xq.tensor_core_perm())
    _check_tiles(oracle_mod, lut, K, 128, 0, st, tr, xt)
    np.testing.assert_array_equal(hatW.numpy(), oracle_mod.decode(tr.numpy(), lut, K))


def test_chain_without_feedback(xq, hb, oracle_mod, mul1_lut):
    """L = None: every tile's targets are its own W values, and the encode is
    the plain tail-bite of each tile."""
    g = torch.Generator().manual_seed(7)
    W = torch.randn(64, 128, generator=g)
    print("case chain K=4 64x128 no feedback", flush=True)
    hatW, st, tr, xt = (t.cpu() for t in hb.ldlq_chain(W.cuda(), None, 4, 128, 0, targets=True))
    assert torch.equal(xt, _seq_order(W, xq.tensor_core_perm()))
    _check_tiles(oracle_mod, mul1_lut, 4, 128, 0, st, tr, xt)
    np.testing.assert_array_equal(hatW.numpy(), oracle_mod.decode(tr.numpy(), mul1_lut, 4))


def test_chain_one_long_column(xq, hb, oracle_mod, mul1_lut):
    """n = 16: a single chain of 32 tiles, each waiting for the one before."""
    g = torch.Generator().manual_seed(8)
    W = torch.randn(512, 16, generator=g)
    L = _lfac(xq, 512, 8, rho=0.8)
    print("case chain K=3 512x16 single column", flush=True)
    hatW, st, tr, xt = (t.cpu() for t in hb.ldlq_chain(W.cuda(), L.cuda(), 3, 128, 0,
                                                        targets=True))
    _check_targets(W, L, hatW, xt, xq.tensor_core_perm())
    _check_tiles(oracle_mod, mul1_lut, 3, 128, 0, st, tr, xt)


@pytest.mark.parametrize("k,n,K", [(1024, 16, 4), (2048, 48, 6)])
def test_chain_publish_between_launches(xq, hb, oracle_mod, mul1_lut, k, n, K):
    """Narrow weights (1 and 3 column chains for 256 workgroups): almost
    every task waits for its predecessor's flag and reads that tile's E at
    once.  Four launches in a row on different weights reuse the library's
    E scratch, so a tile read before its E was visible would return the
    previous launch's error and miss the targets bound; every tile's
    targets and states are checked in every launch."""
    L = _lfac(xq, k, 11)
    perm = xq.tensor_core_perm()
    for rep in range(4):
        g = torch.Generator().manual_seed(300 + 10 * K + rep)
        W = torch.randn(k, n, generator=g) * (1.0 + rep)
        print(f"case chain publish K={K} {k}x{n} launch {rep}", flush=True)
        hatW, st, tr, xt = (t.cpu() for t in hb.ldlq_chain(W.cuda(), L.cuda(), K, 128, 0,
                                                            targets=True))
        _check_targets(W, L, hatW, xt, perm)
        _check_tiles(oracle_mod, mul1_lut, K, 128, 0, st, tr, xt)


def test_chain_many_tasks_per_workgroup(xq, hb, oracle_mod, mul1_lut):
    """2048 tiles: several tasks per persistent workgroup; targets of every
    tile checked, states of the first and last block rows at both edges."""
    g = torch.Generator().manual_seed(9)
    W = torch.randn(256, 2048, generator=g)
    L = _lfac(xq, 256, 9)
    print("case chain K=4 256x2048", flush=True)
    hatW, st, tr, xt = (t.cpu() for t in hb.ldlq_chain(W.cuda(), L.cuda(), 4, 128, 0,
                                                        targets=True))
    _check_targets(W, L, hatW, xt, xq.tensor_core_perm())
    cols = list(range(8)) + list(range(120, 128))
    _check_tiles(oracle_mod, mul1_lut, 4, 128, 0, st, tr, xt, rows=[0, 15], cols=cols)
    np.testing.assert_array_equal(hatW.numpy(), oracle_mod.decode(tr.numpy(), mul1_lut, 4))


def test_chain_outputs_without_dump(hb):
    """Without the targets dump (per-workgroup target rows) the outputs are
    the same, and repeated launches (epochs) agree."""
    g = torch.Generator().manual_seed(10)
    W = torch.randn(128, 512, generator=g).cuda()
    L = torch.tril(0.05 * torch.randn(128, 128, generator=g), -16).cuda().contiguous()
    a = hb.ldlq_chain(W, L, 5, 128, 0, targets=True)
    for _ in range(2):
        b = hb.ldlq_chain(W, L, 5, 128, 0, targets=False)
        assert b[3] is None
        for x, y in zip(a[:3], b[:3]):
            assert torch.equal(x, y)


def test_chain_nan_rejected(hb):
    W = torch.randn(64, 64, device="cuda")
    W[40, 3] = float("nan")
    L = torch.tril(0.1 * torch.ones(64, 64), -16).cuda().contiguous()
    with pytest.raises(hb.HipViterbiError) as ei:
        hb.ldlq_chain(W, L, 4, 128, 0)
    assert ei.value.rc == 11
    hatW, *_ = hb.ldlq_chain(torch.randn(64, 64, device="cuda"), L, 4, 128, 0)
    assert torch.isfinite(hatW).all()


def test_chain_vs_block_schedule(xq, monkeypatch):
    """quantize_linear on GPU tensors with the sweep as column chains and as
    the reference's block schedule, whose feedback then runs as torch GPU
    GEMMs (rounding unlike the reference's CPU order, which the chain
    follows): the same encoder on targets that may differ by an ulp here and
    there.  Measured: every tile identical, the proxy losses equal; held to
    at most 1 % of tiles differing and a relative proxy change of 1e-5."""
    import workloads as wl
    g = torch.Generator().manual_seed(11)
    W = 0.02 * torch.randn(256, 512, generator=g)
    H = wl.ar1_gram(512, 1024, 0.5, 11)
    res = {}
    for sched in ("chain", "block"):
        monkeypatch.setattr(xq, "DEFAULT_SCHEDULE", sched)
        print(f"case quantize_linear 256x512 schedule={sched}", flush=True)
        r = xq.quantize_linear(W, H, K=4, device="cuda", margin=0)
        res[sched] = (r, xq.hessian_weighted_err(W, r["W_hat"], H))
    e_c, e_b = res["chain"][1], res["block"][1]
    same = (res["chain"][0]["trellis"] == res["block"][0]["trellis"]).all(dim=-1).float().mean()
    print(f"proxy chain {e_c:.6e} block {e_b:.6e}, identical tiles {float(same):.3f}")
    assert float(same) >= 0.99
    assert abs(e_c - e_b) <= 1e-5 * e_b


@pytest.mark.parametrize("cs,ldlq", [(False, True), (True, True), (True, False)])
def test_quantize_linear_group_matches_separate(xq, cs, ldlq):
    """Members quantized side by side in one sweep give exactly the results
    of separate quantize_linear calls (their column chains never interact)."""
    import workloads as wl
    g = torch.Generator().manual_seed(12)
    H = wl.ar1_gram(256, 512, 0.5, 12)
    Ws = [0.02 * torch.randn(128, 256, generator=g), 0.03 * torch.randn(256, 256, generator=g),
          0.02 * torch.randn(128, 256, generator=g)]
    print(f"case quantize_linear_group cs={cs} ldlq={ldlq}", flush=True)
    grp = xq.quantize_linear_group(Ws, H, K=5, device="cuda", channel_scales=cs,
                                   use_ldlq=ldlq)
    assert len(grp) == len(Ws)
    for W, r in zip(Ws, grp):
        s = xq.quantize_linear(W, H, K=5, device="cuda", channel_scales=cs, use_ldlq=ldlq)
        assert r["trellis"].shape == (256 // 16, W.shape[0] // 16, 16 * 5)
        for key in ("W_hat", "trellis", "suh", "svh"):
            assert torch.equal(r[key], s[key]), key
        assert r["Wscale"] == s["Wscale"]


def test_to_host_staging(xq):
    """The staged device-to-host and host-to-device copies equal .cpu() and
    .to("cuda") for sizes around their threshold and around and across the
    staging chunks, for several dtypes."""
    C, M = xq._STAGE_BYTES, xq._STAGE_MIN
    for nbytes, dt in ((M - 4, torch.float32), (M, torch.float32), (M + 2, torch.int16),
                       (C - 8, torch.float64), (C, torch.float32), (C + 6, torch.int16),
                       (4 * C, torch.float32), (4 * C + 4, torch.float32),
                       (9 * C + 2 * 7, torch.int16), (5 * C - 8, torch.float64)):
        n = nbytes // torch.tensor([], dtype=dt).element_size()
        t = torch.randn(n, device="cuda").to(dt) if dt.is_floating_point else \
            torch.randint(-30000, 30000, (n,), device="cuda", dtype=dt)
        h = xq._to_host(t.view(-1, 1) if n % 2 else t.view(2, -1))
        assert h.device.type == "cpu" and not h.is_pinned()
        assert torch.equal(h.view(-1), t.cpu())
        # and back through the staged host-to-device copy
        d = xq._to_device(h, torch.device("cuda"))
        assert d.is_cuda and d.shape == h.shape and torch.equal(d.view(-1), t)
    # into a given buffer (paged in beforehand) when it matches, else a new tensor
    t = torch.randn(3 * C // 4 + 5, device="cuda")
    bufs = xq._HostBuffers([(t.shape, torch.float32), (t.shape, torch.float64),
                            ((t.numel() - 1,), torch.float32)])
    for i, same in ((0, True), (1, False), (2, False)):
        b = bufs.take(i)
        h = xq._to_host(t, b)
        assert (h.data_ptr() == b.data_ptr()) == same and torch.equal(h, t.cpu())


@pytest.mark.parametrize("Ks,device", [((5, 7, 7), "cuda"), ((4, 6, 4), "cuda"),
                                       ((3, 6), "cpu")])
def test_quantize_linear_group_mixed_k(xq, Ks, device):
    """Members at different K in one call (concurrent chain launches over a
    split of the CUs on the GPU; one block sweep per K run on the CPU) give
    exactly the results of separate quantize_linear calls."""
    import workloads as wl
    g = torch.Generator().manual_seed(13)
    H = wl.ar1_gram(256, 512, 0.4, 13)
    rows = (256, 128, 128)
    Ws = [0.02 * torch.randn(rows[m], 256, generator=g) for m in range(len(Ks))]
    print(f"case quantize_linear_group K={Ks} on {device}", flush=True)
    grp = xq.quantize_linear_group(Ws, H, K=list(Ks), device=device, channel_scales=True)
    for W, Km, r in zip(Ws, Ks, grp):
        s = xq.quantize_linear(W, H, K=Km, device=device, channel_scales=True)
        assert r["K"] == Km and r["trellis"].shape == (16, W.shape[0] // 16, 16 * Km)
        for key in ("W_hat", "trellis", "suh", "svh"):
            assert torch.equal(r[key], s[key]), (Km, key)


def test_chain_groups_match_single_launches(hb, oracle_mod, mul1_lut):
    """hb.ldlq_chain over column groups of different K equals single-K calls
    on each group's columns (tiles of one column never see another's), and
    the concurrent launches encode every tile as the oracle does."""
    g = torch.Generator().manual_seed(14)
    k = 128
    W = torch.randn(k, 96, generator=g)
    L = torch.tril(0.05 * torch.randn(k, k, generator=g), -16).contiguous()
    groups = [(32, 3), (48, 7), (16, 5)]
    print("case chain groups 128x96 K=3/7/5", flush=True)
    hatW, st, trs, xt = hb.ldlq_chain(W.cuda(), L.cuda(), None, 128, 0, targets=True,
                                      groups=groups)
    c0 = 0
    for (nc, K), tr in zip(groups, trs):
        h1, s1, t1, x1 = hb.ldlq_chain(W[:, c0:c0 + nc].contiguous().cuda(), L.cuda(), K, 128,
                                       0, targets=True)
        assert torch.equal(hatW[:, c0:c0 + nc], h1)
        assert torch.equal(st[:, c0 // 16:(c0 + nc) // 16], s1)
        assert torch.equal(tr, t1)
        assert torch.equal(xt[:, c0 // 16:(c0 + nc) // 16], x1)
        want = oracle_mod.tailbite(x1.reshape(-1, 256).cpu().numpy(), mul1_lut, K, 16,
                                   pivot=128, margin=0, nthreads=8)
        np.testing.assert_array_equal(s1.reshape(-1, 256).cpu().numpy(), want)
        c0 += nc


@pytest.mark.parametrize("k,n,K,pivot,margin", [(16, 64, 4, 128, 0), (32, 16, 6, 250, 16),
                                                (48, 32, 2, 0, 255)])
def test_chain_edge_shapes(xq, hb, oracle_mod, mul1_lut, k, n, K, pivot, margin):
    """One block row (no feedback at all), one column, and margins where
    pivot + margin reaches the end of the sequence (pass 1 runs 256 steps)."""
    g = torch.Generator().manual_seed(15 + k + n)
    W = torch.randn(k, n, generator=g)
    L = torch.tril(0.1 * torch.randn(k, k, generator=g), -16).contiguous()
    print(f"case chain edge {k}x{n} K={K} pivot={pivot} margin={margin}", flush=True)
    hatW, st, tr, xt = (t.cpu() for t in hb.ldlq_chain(W.cuda(), L.cuda(), K, pivot, margin,
                                                        targets=True))
    _check_targets(W, L, hatW, xt, xq.tensor_core_perm())
    _check_tiles(oracle_mod, mul1_lut, K, pivot, margin, st, tr, xt)


@pytest.mark.parametrize("buf_cols,K,k,n", [(16, 3, 544, 240), (32, 6, 112, 144),
                                            (64, 4, 400, 96), (256, 5, 768, 160)])
def test_chain_buffer_widths(xq, hb, oracle_mod, mul1_lut, cpu8, buf_cols, K, k, n):
    """Lazy-feedback buffers other than the default 128 columns
    (quantize.py:631-636 buf_cols).  Up to 128 every tile's targets equal the
    reference's sweep with the same buffers bit for bit: each buffer's
    product has an inner dimension of at most 128, one fused multiply-add
    chain in torch's CPU sgemm.  Wider buffers are summed as one chain each
    here, while the host BLAS may split inner dimensions above 128 (on the
    AMD EPYC hosts of the GPU machines it splits 256, on others not), so
    there the targets are held to the fp64 formula within that order's
    rounding bound.  The encode of every tile is checked against the oracle
    either way."""
    g = torch.Generator().manual_seed(70 + buf_cols)
    W = torch.randn(k, n, generator=g)
    L = _lfac(xq, k, buf_cols)
    perm = xq.tensor_core_perm()
    print(f"case chain buf_cols={buf_cols} K={K} {k}x{n}", flush=True)
    hatW, st, tr, xt = (t.cpu() for t in hb.ldlq_chain(W.cuda(), L.cuda(), K, 128, 0,
                                                        targets=True, buf_cols=buf_cols))
    if buf_cols <= 128:
        assert torch.equal(xt, _ref_targets(W, L, hatW, perm, buf_cols=buf_cols))
    W64, E = W.double(), (W - hatW).double()
    X64, B = W64.clone(), W64.abs()
    L64 = L.double()
    for i in range(k // 16 - 1):
        r0, r1 = 16 * i, 16 * (i + 1)
        X64[r0:r1] += L64[r1:, r0:r1].t() @ E[r1:]
        B[r0:r1] += L64[r1:, r0:r1].abs().t() @ E[r1:].abs()
    d = (xt.double() - _seq_order(X64, perm)).abs()
    lim = (buf_cols + k / buf_cols + 3) * U32 * _seq_order(B, perm)
    assert (d <= lim).all(), f"worst excess {float((d - lim).max()):.3e}"
    _check_tiles(oracle_mod, mul1_lut, K, 128, 0, st, tr, xt)
    np.testing.assert_array_equal(hatW.numpy(), oracle_mod.decode(tr.numpy(), mul1_lut, K))


def test_chain_many_groups(hb):
    """Four column groups (one narrower than its share of the CUs) equal
    single-K launches over their columns."""
    g = torch.Generator().manual_seed(16)
    k = 96
    W = torch.randn(k, 192, generator=g).cuda()
    L = torch.tril(0.05 * torch.randn(k, k, generator=g), -16).contiguous().cuda()
    groups = [(16, 2), (96, 4), (32, 6), (48, 7)]
    print("case chain 4 groups", flush=True)
    hatW, st, trs, _ = hb.ldlq_chain(W, L, None, 147, 16, groups=groups)
    c0 = 0
    for (nc, K), tr in zip(groups, trs):
        h1, s1, t1, _ = hb.ldlq_chain(W[:, c0:c0 + nc].contiguous(), L, K, 147, 16)
        assert torch.equal(hatW[:, c0:c0 + nc], h1) and torch.equal(tr, t1)
        assert torch.equal(st[:, c0 // 16:(c0 + nc) // 16], s1)
        c0 += nc


def test_chain_targets_vs_golden_pinned_block_path(xq, hb, monkeypatch, cpu8):
    """The reference's own 128x128 AR(1) case: the block schedule with the
    torch work on the CPU reproduces the reference's golden trellis bit for
    bit, so its per-launch targets are the reference's.  The chain, fed the
    same inner weights and factor, produces those targets bit for bit, and
    so the golden trellis and the block schedule's What."""
    from conftest import load_golden
    e = load_golden("e2e_128.npz")
    W, H = torch.from_numpy(e["W"]), torch.from_numpy(e["H_ar"])
    seen, launches = {}, []
    real_ldlq, real_launch = xq.ldlq_viterbi, xq._launch

    def rec_ldlq(Wq, Lfac, *a, **kw):
        seen["Wq"], seen["Lfac"] = Wq.clone(), Lfac.clone()
        out = real_ldlq(Wq, Lfac, *a, **kw)
        seen["hatW"] = out[0].clone()
        return out

    def rec_launch(X, K, code, pivot, margin):
        launches.append(X.detach().cpu().clone())
        return real_launch(X, K, code, pivot, margin)

    monkeypatch.setattr(xq, "DEFAULT_SCHEDULE", "block")
    monkeypatch.setattr(xq, "_launch", rec_launch)
    monkeypatch.setattr(xq, "ldlq_viterbi", rec_ldlq)
    xq.ldlq_viterbi.last_trellis = None
    print("case golden 128x128 AR(1): block schedule on the CPU", flush=True)
    r = xq.quantize_linear(W, H, code="exl3_mul1", K=4, use_ldlq=True, margin=0, device="cpu")
    np.testing.assert_array_equal(r["trellis"].numpy(), e["ar_trellis"])      # pinned
    Wq, Lf = seen["Wq"], seen["Lfac"]
    Xb = torch.stack(launches[::-1])                       # [tk, tn, 256], block i first
    print("case golden 128x128 AR(1): chain on the GPU", flush=True)
    hatW, st, tr, xt = (t.cpu() for t in hb.ldlq_chain(Wq.cuda(), Lf.cuda(), 4, 128, 0,
                                                        targets=True))
    assert torch.equal(xt, Xb), "chain targets != the reference's per-launch targets"
    np.testing.assert_array_equal(tr.numpy(), e["ar_trellis"])
    assert torch.equal(hatW, seen["hatW"])


@pytest.mark.parametrize("K,shape", [(4, (4096, 4096)), (6, (2048, 1024)), (2, (1024, 512))])
def test_chain_equals_cpu_block_schedule(xq, hb, cpu8, K, shape):
    """ldlq_viterbi on the same inner weights and factor: the column chains on
    the GPU against the reference's block schedule with its torch feedback on
    the CPU (the reference's arithmetic; each launch's encode on the GPU is
    pinned separately): identical What and states for every tile, up to a
    4096x4096 weight (256 blocks of feedback, 65,536 tiles)."""
    import workloads as wl
    k, n = shape
    g = torch.Generator().manual_seed(20 + K)
    Wq = torch.randn(k, n, generator=g)
    G = wl.ar1_gram(k, 2 * k, 0.5, 20 + K)
    G.diagonal().add_(0.01 * G.diagonal().mean())
    Lf, _ = xq.block_LDL(G, 16)
    lut = xq.get_lut("exl3_mul1")
    print(f"case chain vs CPU block schedule {k}x{n} K={K}", flush=True)
    hb_, sb = xq.ldlq_viterbi(Wq, Lf, lut, K, 16, margin=0, schedule="block")
    hc, sc = xq.ldlq_viterbi(Wq.cuda(), Lf.cuda(), lut.cuda(), K, 16, margin=0,
                             schedule="chain")
    bad = int((sc.cpu() != sb).any(dim=-1).sum())
    assert bad == 0, f"{bad} of {sb.shape[0] * sb.shape[1]} tiles differ"
    assert torch.equal(hc.cpu(), hb_)


@pytest.mark.parametrize("given,runs_as", [(100, 96), (8, 16), (17, 16)])
def test_buffer_width_rounds_like_reference(xq, given, runs_as):
    """A lazy-buffer width that is not a whole number of 16-column blocks runs
    as the reference's buf_tiles = max(1, buf_cols // 16) blocks
    (quantize.py:665): on the GPU chain and the CPU block schedule alike."""
    import workloads as wl
    k, n = 384, 64
    g = torch.Generator().manual_seed(given)
    Wq = torch.randn(k, n, generator=g)
    G = wl.ar1_gram(k, 2 * k, 0.5, given)
    G.diagonal().add_(0.01 * G.diagonal().mean())
    Lf, _ = xq.block_LDL(G, 16)
    lut = xq.get_lut("exl3_mul1")
    print(f"case buf_cols {given} as {runs_as}", flush=True)
    hw, sw = xq.ldlq_viterbi(Wq.cuda(), Lf.cuda(), lut.cuda(), 4, 16, margin=0,
                             buf_cols=runs_as, schedule="chain")
    hg, sg = xq.ldlq_viterbi(Wq.cuda(), Lf.cuda(), lut.cuda(), 4, 16, margin=0,
                             buf_cols=given, schedule="chain")
    assert torch.equal(sg, sw) and torch.equal(hg, hw)
    hb_, sb = xq.ldlq_viterbi(Wq, Lf, lut, 4, 16, margin=0, buf_cols=given, schedule="block")
    assert torch.equal(sb, sw.cpu()) and torch.equal(hb_, hw.cpu())


def test_quantize_linear_1mad_chain_equals_block(xq):
    """quantize_linear with code="qtip_1mad" on the GPU (column chains) equals
    the reference's CPU block schedule bit for bit: trellis and W_hat."""
    import workloads as wl
    g = torch.Generator().manual_seed(21)
    W = 0.02 * torch.randn(128, 256, generator=g)
    H = wl.ar1_gram(256, 512, 0.5, 21)
    print("case quantize_linear 128x256 qtip_1mad K=3 chain vs CPU", flush=True)
    rg = xq.quantize_linear(W.cuda(), H.cuda(), code="qtip_1mad", K=3, device="cuda",
                            reference_arithmetic=True)
    rc = xq.quantize_linear(W, H, code="qtip_1mad", K=3, device="cpu")
    assert torch.equal(rg["trellis"], rc["trellis"])
    assert torch.equal(rg["W_hat"], rc["W_hat"])


def test_chain_factor_over_2g_elements(hb, oracle_mod, mul1_lut):
    """k = 46400: the block-LDL factor holds more than 2^31 elements (8.6 GB),
    so every index into it and into E must be 64-bit; one column chain of
    2,900 tiles.  Targets of tiles spread over the sweep against the fp64
    formula on the kernel's own What, and their encodes against the oracle."""
    k, n = 46400, 16
    assert k * k > 2 ** 31
    g = torch.Generator(device="cuda").manual_seed(17)
    W = torch.randn(k, n, device="cuda", generator=g)
    L = torch.randn(k, k, device="cuda", generator=g).mul_(0.002).tril_(-16)
    print("case chain k=46400 n=16 K=4", flush=True)
    hatW, st, tr, xt = hb.ldlq_chain(W, L, 4, 128, 0, targets=True)
    perm = torch.tensor(oracle_mod.tensor_core_perm(), device="cuda", dtype=torch.long)
    E = (W - hatW).double()
    tk = k // 16
    for i in (0, 1, tk // 2, tk - 2, tk - 1):
        r0, r1 = 16 * i, 16 * (i + 1)
        X64 = W[r0:r1].double() + L[r1:, r0:r1].double().t() @ E[r1:]
        B = W[r0:r1].double().abs() + L[r1:, r0:r1].double().abs().t() @ E[r1:].abs()
        x64 = X64.reshape(-1)[perm]
        lim = (k / 4 + 36) * U32 * B.reshape(-1)[perm]
        assert bool(((xt[i, 0].double() - x64).abs() <= lim).all()), i
        want = oracle_mod.tailbite(xt[i].cpu().numpy(), mul1_lut, 4, 16, pivot=128, margin=0)
        np.testing.assert_array_equal(st[i].cpu().numpy(), want)
    del L


def test_weight_widening_on_device_matches_host():
    """quantize_linear moves a host weight to the GPU in its own dtype and
    widens it to fp32 there: for every fp16 and bf16 bit pattern (subnormals
    included) the device conversion gives the host conversion's fp32 bits
    (NaNs: NaN either way)."""
    u = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    for dt in (torch.float16, torch.bfloat16):
        x = u.view(dt)
        host = x.float()
        dev = x.cuda().float().cpu()
        nan = torch.isnan(host)
        assert torch.equal(torch.isnan(dev), nan)
        assert torch.equal(dev[~nan].view(torch.int32), host[~nan].view(torch.int32)), dt
