"""GPU tests of the quantizer API (quantize.py mirror) on the HIP kernels.

  * end-to-end golden vectors written by the reference's own quantize_linear
    and quantize() on CPU (tests/golden/e2e_128.npz, and e2e_mid.npz: a
    1024x1024 weight, 4,096 tiles through BlockLDLQ), reproduced exactly with
    the torch work on CPU and the trellis on the GPU; the all-GPU pipeline's
    distance from them measured;
  * the reference's per-launch "dual" method (quantize.py:687-717): every
    BlockLDLQ launch's targets go to both the HIP encoder and the CPU oracle
    and the states must agree; a pipeline driven by the oracle's states gives
    the same W_hat and a proxy loss within 1e-6 relative;
  * the reference's API and quality tests (test_quantize.py:183-301).
"""
import hashlib

import numpy as np
import pytest
import torch

from conftest import load_golden

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def xq():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import quantize
    return quantize


@pytest.mark.parametrize("tag,ldlq,cs", [("id", True, False), ("ar", True, False),
                                         ("arcs", True, True), ("nold", False, False)])
def test_quantize_linear_golden(xq, cpu8, tag, ldlq, cs):
    e = load_golden("e2e_128.npz")
    W = torch.from_numpy(e["W"])
    H = torch.eye(128) if tag == "id" else torch.from_numpy(e["H_ar"])
    print(f"case quantize_linear {tag}", flush=True)
    r = xq.quantize_linear(W, H, code="exl3_mul1", K=4, use_ldlq=ldlq, margin=0,
                           channel_scales=cs, device="cpu")
    np.testing.assert_array_equal(r["trellis"].numpy(), e[f"{tag}_trellis"])
    np.testing.assert_array_equal(r["W_hat"].numpy(), e[f"{tag}_W_hat"])
    np.testing.assert_array_equal(r["suh"].float().numpy(), e[f"{tag}_suh"])
    np.testing.assert_array_equal(r["svh"].float().numpy(), e[f"{tag}_svh"])
    # Wscale is a torch CPU mean over k*n values; its reduction order (and so
    # its last bit) depends on the host CPU, not on the trellis path
    assert abs(np.float32(r["Wscale"]) - e[f"{tag}_Wscale"]) <= np.spacing(e[f"{tag}_Wscale"])
    # proxy loss: identical to the reference's W_hat evaluated on this host;
    # the stored value came from another CPU, whose fp32 einsum reduction
    # order differs in the last bits
    herr = xq.hessian_weighted_err(W, r["W_hat"], H)
    assert herr == xq.hessian_weighted_err(W, torch.from_numpy(e[f"{tag}_W_hat"]), H)
    assert herr == pytest.approx(float(e[f"{tag}_herr"]), rel=1e-5)


def _herr64(W, W_hat, H) -> float:
    """hessian_weighted_err (quantize.py:878-885) evaluated in fp64: its fp32
    einsum rounds by the host CPU's reduction order."""
    dW = (W_hat - W).double()
    H64 = H.double()
    return float(((dW @ H64) * dW).sum() / ((W.double() @ H64) * W.double()).sum())


def _kms_hessian(d: int) -> torch.Tensor:
    i = np.arange(d)
    return torch.from_numpy(np.ldexp(1.0, -np.abs(i[:, None] - i[None, :])).astype(np.float32))


@pytest.mark.parametrize("tag,K,cs", [("k4", 4, False), ("k5cs", 5, True)])
def test_quantize_linear_mid_golden(xq, cpu8, tag, K, cs):
    """The reference's quantize_linear on a 1024x1024 weight with BlockLDLQ
    (4,096 tiles, 64 feedback blocks; e2e_mid.npz): with the torch work on
    the CPU, as the reference's device="cpu" run, the trellis of every tile,
    suh, svh, Wscale and W_hat are identical and the proxy loss agrees within
    1e-6.  With channel scales this holds on hosts whose torch CPU reduction
    rounds the per-output-channel RMS as the generating host's did (a digest
    in the fixture); elsewhere the reference itself encodes the channels whose
    RMS rounds differently otherwise, and the test bounds that instead."""
    e = load_golden("e2e_mid.npz")
    W = torch.from_numpy(e["W16"].astype(np.float32))
    H = _kms_hessian(1024)
    same_host = hashlib.sha256(W.t().contiguous().square().mean(dim=0).sqrt().numpy()
                               .tobytes()).digest() == e["rout_sha256"].tobytes()
    print(f"case quantize_linear 1024x1024 {tag} device=cpu (host reduces as the "
          f"generating host: {same_host})", flush=True)
    r = xq.quantize_linear(W, H, code="exl3_mul1", K=K, use_ldlq=True, margin=0,
                           channel_scales=cs, device="cpu")
    badm = (r["trellis"].numpy() != e[f"{tag}_trellis"]).any(axis=2)
    bad = int(badm.sum())
    print(f"{tag}: {bad} tiles differ (block rows {sorted(set(np.nonzero(badm)[0].tolist()))[:10]}"
          f", cols {sorted(set(np.nonzero(badm)[1].tolist()))[:10]}); suh equal "
          f"{np.array_equal(r['suh'].float().numpy(), e[f'{tag}_suh'])} ("
          f"{int((r['suh'].float().numpy() != e[f'{tag}_suh']).sum())}), svh equal "
          f"{np.array_equal(r['svh'].float().numpy(), e[f'{tag}_svh'])} ("
          f"{int((r['svh'].float().numpy() != e[f'{tag}_svh']).sum())}), Wscale "
          f"{np.float32(r['Wscale'])!r} vs {e[f'{tag}_Wscale']!r}", flush=True)
    np.testing.assert_array_equal(r["suh"].float().numpy(), e[f"{tag}_suh"])
    np.testing.assert_array_equal(r["svh"].float().numpy(), e[f"{tag}_svh"])
    assert np.float32(r["Wscale"]) == e[f"{tag}_Wscale"]
    same_what = hashlib.sha256(r["W_hat"].contiguous().numpy().tobytes()).digest() == \
        e[f"{tag}_What_sha256"].tobytes()
    h64 = _herr64(W, r["W_hat"], H)
    herr = xq.hessian_weighted_err(W, r["W_hat"], H)
    rel = abs(h64 - float(e[f"{tag}_herr64"])) / abs(float(e[f"{tag}_herr64"]))
    print(f"{tag}: W_hat bytes identical {same_what}; proxy loss fp64 {h64:.12e} vs "
          f"{float(e[f'{tag}_herr64']):.12e} (rel {rel:.1e}); fp32 (the reference's own "
          f"einsum, host-dependent) {herr:.9e} vs {float(e[f'{tag}_herr']):.9e}", flush=True)
    if not cs or same_host:
        assert bad == 0, f"{bad} of 4096 tiles differ from the reference"
        assert same_what and rel <= 1e-12
    else:
        # one output channel's RMS rounds differently: its column of tiles
        assert bad <= 64 and len(set(np.nonzero(badm)[1].tolist())) <= 2
        assert rel <= 1e-4


# Measured on the MI355X for the default GPU pipeline against the
# reference's CPU run: differing tile share and proxy-loss change, bounded at
# twice the measurement (k4: no tile differs; the bound allows 4 of 4,096).
MID_GPU_BOUNDS = {"k4": (4 / 4096, 2e-7), "k5cs": (0.0156, 3.1e-5)}


@pytest.mark.parametrize("tag,K,cs", [("k4", 4, False), ("k5cs", 5, True)])
def test_quantize_linear_mid_on_gpu_vs_reference(xq, tag, K, cs):
    """The same weight with every step on the GPU (column-chain schedule):
    the GPU's reductions and factorisation round differently from the
    reference's CPU arithmetic (the chain's feedback follows the reference's
    order), so a few tiles' targets move by an ulp and encode differently;
    the differing share and the proxy-loss change are held to twice what
    they measure (0 % / 7.6e-8 for k4, 0.78 % / 1.5e-5 for k5cs)."""
    e = load_golden("e2e_mid.npz")
    W = torch.from_numpy(e["W16"].astype(np.float32))
    H = _kms_hessian(1024)
    print(f"case quantize_linear 1024x1024 {tag} device=cuda", flush=True)
    r = xq.quantize_linear(W.cuda(), H.cuda(), code="exl3_mul1", K=K, use_ldlq=True,
                           margin=0, channel_scales=cs, device="cuda")
    differ = float((r["trellis"].cpu().numpy() != e[f"{tag}_trellis"]).any(axis=2).mean())
    herr = _herr64(W, r["W_hat"].cpu(), H)
    rel = abs(herr - float(e[f"{tag}_herr64"])) / abs(float(e[f"{tag}_herr64"]))
    print(f"{tag}: {100 * differ:.2f} % of tiles differ from the reference's CPU run, "
          f"proxy loss {herr:.6e} vs {float(e[f'{tag}_herr']):.6e} (rel {rel:.2e})", flush=True)
    max_differ, max_rel = MID_GPU_BOUNDS[tag]
    assert differ <= max_differ and rel <= max_rel


@pytest.mark.parametrize("tag,K,cs", [("k4", 4, False), ("k5cs", 5, True)])
def test_reference_arithmetic_on_gpu_vs_golden(xq, cpu8, tag, K, cs):
    """quantize_linear on the GPU with reference_arithmetic=True (the
    reductions and the block-LDL factorisation on the host CPU, everything
    else on the GPU) against the reference's own 1024x1024 result
    (e2e_mid.npz): identical trellis, suh, svh, Wscale and W_hat, on hosts
    that reduce as the generating host did (see the device="cpu" test)."""
    e = load_golden("e2e_mid.npz")
    W = torch.from_numpy(e["W16"].astype(np.float32))
    H = _kms_hessian(1024)
    same_host = hashlib.sha256(W.t().contiguous().square().mean(dim=0).sqrt().numpy()
                               .tobytes()).digest() == e["rout_sha256"].tobytes()
    print(f"case quantize_linear 1024x1024 {tag} device=cuda reference_arithmetic", flush=True)
    r = xq.quantize_linear(W.cuda(), H.cuda(), code="exl3_mul1", K=K, use_ldlq=True, margin=0,
                           channel_scales=cs, device="cuda", reference_arithmetic=True)
    badm = (r["trellis"].numpy() != e[f"{tag}_trellis"]).any(axis=2)
    same_what = hashlib.sha256(r["W_hat"].contiguous().numpy().tobytes()).digest() == \
        e[f"{tag}_What_sha256"].tobytes()
    print(f"{tag}: {int(badm.sum())} tiles differ, W_hat identical {same_what}", flush=True)
    np.testing.assert_array_equal(r["suh"].float().numpy(), e[f"{tag}_suh"])
    np.testing.assert_array_equal(r["svh"].float().numpy(), e[f"{tag}_svh"])
    assert np.float32(r["Wscale"]) == e[f"{tag}_Wscale"]
    if not cs or same_host:
        assert int(badm.sum()) == 0 and same_what
    else:
        assert int(badm.sum()) <= 64 and len(set(np.nonzero(badm)[1].tolist())) <= 2


@pytest.mark.parametrize("cs", (False, True))
def test_reference_arithmetic_equals_cpu_pipeline(xq, cpu8, cs):
    """A 4096x4096 weight with an AR(1) Gram (65,536 tiles): the GPU pipeline
    with reference_arithmetic=True equals the reference's arithmetic with all
    torch work on the CPU (device="cpu") bit for bit -- trellis, W_hat,
    suh, svh, Wscale -- on the same host."""
    import workloads as wl
    w = wl.c2(device="cpu")
    W, H = w["W"].float(), w["H"]
    print(f"case c2 device=cpu cs={cs}", flush=True)
    rc = xq.quantize_linear(W, H, K=4, margin=0, channel_scales=cs, device="cpu")
    print(f"case c2 device=cuda reference_arithmetic cs={cs}", flush=True)
    rg = xq.quantize_linear(W.cuda(), H.cuda(), K=4, margin=0, channel_scales=cs,
                            device="cuda", reference_arithmetic=True)
    bad = int((rg["trellis"] != rc["trellis"]).any(dim=-1).sum())
    assert bad == 0, f"{bad} of 65536 tiles differ"
    for key in ("W_hat", "suh", "svh"):
        assert torch.equal(rg[key], rc[key]), key
    assert rg["Wscale"] == rc["Wscale"]


@pytest.mark.parametrize("n,k,K,code,cs,buf,rho,seed", [
    (384, 768, 7, "exl3_3inst", False, 32, 0.4673059694552129, 1198),
    (1024, 768, 7, "exl3_mcg", True, 16, 0.770254471100988, 1005),
])
def test_reference_arithmetic_damping_mean_layout(xq, cpu8, n, k, K, code, cs, buf, rho, seed):
    """Weights whose damped Gram's diagonal mean rounds differently over the
    strided diagonal view of the [k, k] matrix (the reference's
    G.diagonal().mean(), quantize.py:813) than over a contiguous copy of the
    diagonal: reference_arithmetic on the GPU must take the mean over the
    same view, or the factor, and with it the feedback of every later tile,
    differs from device="cpu" (a random sweep found one such case in 100)."""
    import workloads as wl
    g = torch.Generator().manual_seed(seed)
    W = (0.02 * torch.randn(n, k, generator=g)).half().float()
    H = wl.ar1_gram(k, k // 2, rho, seed)
    suh = xq.sign_vec(k, 20261011, "cpu").half()
    G = xq.rotate_hessian(H, suh, xq.hadamard128("cpu", torch.float32))
    assert G.diagonal().mean() != G.diagonal().contiguous().mean()    # the case this pins
    args = dict(code=code, K=K, margin=0, channel_scales=cs, buf_cols=buf)
    print(f"case damping-mean layout W {n}x{k} K={K} {code} cs={cs} buf={buf}", flush=True)
    rc = xq.quantize_linear(W, H, device="cpu", **args)
    rg = xq.quantize_linear(W.cuda(), H.cuda(), device="cuda", reference_arithmetic=True, **args)
    bad = int((rg["trellis"] != rc["trellis"]).any(dim=-1).sum())
    assert bad == 0, f"{bad} of {(k // 16) * (n // 16)} tiles differ"
    for key in ("W_hat", "suh", "svh"):
        assert torch.equal(rg[key], rc[key]), key


def test_reference_arithmetic_mixed_k_group(xq, cpu8):
    """quantize_linear_group of q/k/v-like members at K = [5, 7, 7] with
    channel scales on the GPU under reference_arithmetic (concurrent chain
    launches per K) equals each member's device="cpu" quantize_linear."""
    import workloads as wl
    g = torch.Generator().manual_seed(31)
    H = wl.ar1_gram(512, 1024, 0.5, 31)
    Ws = [0.02 * torch.randn(512, 512, generator=g), 0.03 * torch.randn(128, 512, generator=g),
          0.02 * torch.randn(128, 512, generator=g)]
    Ks = [5, 7, 7]
    print("case mixed-K group reference_arithmetic on the GPU", flush=True)
    grp = xq.quantize_linear_group([W.cuda() for W in Ws], H.cuda(), K=Ks, device="cuda",
                                   channel_scales=True, reference_arithmetic=True)
    for W, Km, r in zip(Ws, Ks, grp):
        c = xq.quantize_linear(W, H, K=Km, device="cpu", channel_scales=True)
        for key in ("trellis", "W_hat", "suh", "svh"):
            assert torch.equal(r[key], c[key]), (Km, key)
        assert r["Wscale"] == c["Wscale"]


@pytest.mark.parametrize("k,n", [(128, 64), (256, 100), (1024, 384), (4096, 4096)])
def test_hadamard_kernel_matches_cpu(xq, k, n):
    """The block-128 Hadamard kernel (had_left / had_right on GPU tensors, and
    the to_inner / from_inner / rotate_hessian built on them) reproduces the
    reference's torch CPU results bit for bit (quantize.py:134-168)."""
    g = torch.Generator().manual_seed(k + n)
    w = torch.randn(k, n, generator=g) * 0.3
    h = xq.hadamard128(None, torch.float32)
    hd = xq.hadamard128("cuda", torch.float32)
    print(f"case had128 {k}x{n}", flush=True)
    assert torch.equal(xq.had_left(w.cuda(), hd).cpu(), xq.had_left(w, h))
    if n % 128 == 0:
        assert torch.equal(xq.had_right(w.cuda(), hd).cpu(), xq.had_right(w, h))
        suh = xq.sign_vec(k, 3).half()
        svh = xq.sign_vec(n, 4).half()
        wi = xq.to_inner(w, suh, svh, h)
        assert torch.equal(xq.to_inner(w.cuda(), suh.cuda(), svh.cuda(), hd).cpu(), wi)
        assert torch.equal(xq.from_inner(wi.cuda(), suh.cuda(), svh.cuda(), hd).cpu(),
                           xq.from_inner(wi, suh, svh, h))
    if k == n:
        Hx = w @ w.t() / n
        assert torch.equal(xq.rotate_hessian(Hx.cuda(), xq.sign_vec(k, 5).cuda(), hd).cpu(),
                           xq.rotate_hessian(Hx, xq.sign_vec(k, 5), h))
    # any 128x128 matrix, not only the symmetric Hadamard: h @ w and w @ h
    hn = torch.randn(128, 128, generator=g)
    assert not torch.equal(hn, hn.t())
    want = xq.had_left(w.double(), hn.double()).float()
    got = xq.had_left(w.cuda(), hn.cuda()).cpu()
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)
    if n % 128 == 0:
        want = xq.had_right(w.double(), hn.double()).float()
        got = xq.had_right(w.cuda(), hn.cuda()).cpu()
        torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("rows", [1, 7, 37, 1000])
def test_had_right_ragged_rows(xq, rows):
    """had_right on the GPU for row counts that leave a partial wave (the
    kernel takes 8 rows per wave): each output row depends on its own input
    row only, so the rows of the CPU product of a 1024-row matrix are the
    reference (a shape whose CPU sgemm is one FMA chain per output)."""
    g = torch.Generator().manual_seed(rows)
    w = torch.randn(1024, 384, generator=g)
    h = xq.hadamard128(None, torch.float32)
    print(f"case had_right rows={rows}", flush=True)
    want = xq.had_right(w, h)[:rows]
    got = xq.had_right(w[:rows].contiguous().cuda(), h.cuda()).cpu()
    assert torch.equal(got, want)


def test_quantize_harness_golden(xq, cpu8):
    e = load_golden("e2e_128.npz")
    Wt = torch.from_numpy(e["prep_Wt"])
    U = torch.from_numpy(e["q_U"])
    print("case quantize() with U, margin 16, seed 147", flush=True)
    W_hat, packed, scale = xq.quantize(Wt, U, "exl3_mul1", 4, seed=147, margin=16)
    np.testing.assert_array_equal(packed.numpy(), e["q_packed"])
    np.testing.assert_array_equal(W_hat.numpy(), e["q_W_hat"])
    assert np.float32(scale) == e["q_scale"]
    print("case quantize() plain, K=3", flush=True)
    W_hat, packed, scale = xq.quantize(Wt[:64], None, "exl3_mul1", 3, seed=5, margin=0)
    np.testing.assert_array_equal(packed.numpy(), e["q0_packed"])
    np.testing.assert_array_equal(W_hat.numpy(), e["q0_W_hat"])


def test_module_wrappers_golden(xq):
    """quantize_seq_tailbite / viterbi / pack / unpack / decode_trellis with
    CPU tensors in and out (the trellis work still runs on the GPU)."""
    g = load_golden("tailbite.npz")
    lut = xq.get_lut("exl3_mul1")
    for K in (3, 6):
        X = torch.from_numpy(g[f"X_K{K}"].T.copy())          # [256, 6]
        st = xq.quantize_seq_tailbite(X, lut, K, 16, pivot=147, margin=16)
        assert st.dtype == torch.int64 and st.device.type == "cpu"
        np.testing.assert_array_equal(st.t().numpy(), g[f"S_K{K}_m16_p147"])
        np.testing.assert_array_equal(xq.viterbi(X, lut, K, 16).t().numpy(), g[f"V_K{K}"])
        ov = torch.from_numpy(g[f"VPov_K{K}"])
        np.testing.assert_array_equal(xq.viterbi(X, lut, K, 16, overlap=ov).t().numpy(),
                                      g[f"VP_K{K}"])
        np.testing.assert_array_equal(xq.viterbi(X[:150], lut, K, 16, back_from=100).numpy(),
                                      g[f"VB_K{K}"])
        s128 = torch.from_numpy(g[f"S_K{K}_m0_p128"].astype(np.int64))
        P = xq.pack_states(s128, K)
        np.testing.assert_array_equal(P.numpy(), g[f"P_K{K}"])
        np.testing.assert_array_equal(xq.unpack_states(P, K).numpy(), g[f"U_K{K}"])
        np.testing.assert_array_equal(
            xq.decode_trellis(P.view(2, 3, 16 * K), lut, K, 32, 48).numpy(), g[f"D_K{K}"])


def _ar1_hessian(d, n_s, rho, seed):
    g = torch.Generator().manual_seed(seed + 100)
    Z = torch.randn(n_s, d, generator=g, dtype=torch.float64)
    X = torch.empty_like(Z)
    X[:, 0] = Z[:, 0]
    c = (1 - rho * rho) ** 0.5
    for i in range(1, d):
        X[:, i] = rho * X[:, i - 1] + c * Z[:, i]
    return (X.t() @ X / n_s).float()


def test_dual_ldlq_on_gpu(xq, oracle_mod, mul1_lut, monkeypatch):
    """BlockLDLQ entirely on the GPU: every launch is bit-exact with the
    oracle on identical targets, and an oracle-driven pipeline gives the same
    W_hat and proxy loss (quantize.py:687-717 dual method)."""
    g = torch.Generator().manual_seed(1)
    W = (0.02 * torch.randn(256, 256, generator=g)).half().float()
    H = _ar1_hessian(256, 512, 0.5, 1)
    stats = {"launches": 0, "tiles": 0, "mismatch_tiles": 0}
    real = xq._launch
    monkeypatch.setattr(xq, "DEFAULT_SCHEDULE", "block")   # one launch per 16-row block

    def dual(X, K, code, pivot, margin):
        st, tr = real(X, K, code, pivot, margin)
        want = oracle_mod.tailbite(X.cpu().numpy(), mul1_lut, K, 16, pivot=pivot, margin=margin)
        stats["launches"] += 1
        stats["tiles"] += X.shape[0]
        stats["mismatch_tiles"] += int((st.cpu().numpy() != want).any(axis=1).sum())
        return st, tr

    monkeypatch.setattr(xq, "_launch", dual)
    print("case dual LDLQ 256x256 K=4 on cuda", flush=True)
    r = xq.quantize_linear(W, H, K=4, device="cuda", margin=0)
    assert stats["launches"] == 16 and stats["tiles"] == 256
    assert stats["mismatch_tiles"] == 0, stats

    def oracle_launch(X, K, code, pivot, margin):
        st = oracle_mod.tailbite(X.cpu().numpy(), mul1_lut, K, 16, pivot=pivot, margin=margin)
        tr = oracle_mod.pack(st, K)
        return (torch.from_numpy(st).to(X.device), torch.from_numpy(tr).to(X.device))

    monkeypatch.setattr(xq, "_launch", oracle_launch)
    r_o = xq.quantize_linear(W, H, K=4, device="cuda", margin=0)
    assert torch.equal(r["trellis"], r_o["trellis"])
    assert torch.equal(r["W_hat"], r_o["W_hat"])
    e_h = xq.hessian_weighted_err(W, r["W_hat"], H)
    e_o = xq.hessian_weighted_err(W, r_o["W_hat"], H)
    assert abs(e_h - e_o) <= 1e-6 * abs(e_o)


def test_ldlq_helps(xq):
    """LDLQ is no worse than plain Viterbi on the Hessian metric
    (test_quantize.py:205-219), with the sweep on the GPU."""
    torch.manual_seed(4)
    k, n = 256, 256
    A = torch.randn(k, k)
    H = A.t() @ A / k + 0.1 * torch.eye(k)
    W = (torch.randn(n, k) @ torch.linalg.cholesky(torch.linalg.inv(H)).t()).t()
    res_l = xq.quantize_linear(W.t(), H, K=4, use_ldlq=True, device="cuda")
    res_p = xq.quantize_linear(W.t(), H, K=4, use_ldlq=False, device="cuda")
    e_l = xq.hessian_weighted_err(W.t(), res_l["W_hat"], H)
    e_p = xq.hessian_weighted_err(W.t(), res_p["W_hat"], H)
    assert e_l <= e_p * 1.001, (e_l, e_p)


@pytest.mark.parametrize("K", (2, 4))
def test_quantize_api(xq, K):
    """Shapes, decode*scale == W_hat bit-exact, reproducible bitstreams and the
    MSE bound (test_quantize.py:278-301)."""
    torch.manual_seed(5)
    W = torch.randn(64, 128) * 0.03
    W_hat, packed, scale = xq.quantize(W, None, "exl3_mul1", K, seed=7)
    assert packed.shape == (128 // 16, 64 // 16, 16 * K) and packed.dtype == torch.int16
    assert W_hat.shape == W.shape
    lut = xq.get_lut("exl3_mul1")
    dec = xq.decode_trellis(packed, lut, K, 128, 64).t().contiguous() * scale
    assert torch.equal(dec, W_hat)
    _, p2, s2 = xq.quantize(W, None, "exl3_mul1", K, seed=7)
    assert torch.equal(p2, packed) and s2 == scale
    assert xq.rel_mse(W, W_hat) < 3.0 * 2.0 ** (-2 * K)


@pytest.mark.parametrize("K", (2, 4))
def test_gaussian_mse(xq, K):
    """Gaussian MSE against the rate-distortion bound (test_quantize.py:183-202)."""
    torch.manual_seed(3)
    lut = xq.get_lut("exl3_mul1")
    lut_rms = lut.double().square().mean().sqrt().float()
    X = torch.randn(256, 128)
    X = X / X.square().mean().sqrt() * lut_rms
    st = xq.quantize_seq_tailbite(X, lut, K, 16)
    dec = lut[st]
    mse = (dec - X).square().mean() / X.square().mean()
    assert mse < 3.0 * 2.0 ** (-2 * K)


def test_block_ldl_device_large(xq):
    """block_LDL of a device matrix at the size that takes the MAGMA Cholesky
    (when the build has it): L D L^T reproduces G to fp32 accuracy against
    the fp64 factor, the diagonal blocks are identities, torch's preferred
    linalg backend is restored afterwards, and a matrix that is not positive
    definite raises RuntimeError (the damping fallback relies on it)."""
    import workloads as wl
    n = xq._MAGMA_CHOL_MIN
    G = wl.ar1_gram(n, 2048, 0.5, 11, device="cuda").float()
    G.diagonal().add_(0.01 * G.diagonal().mean())
    before = torch.backends.cuda.preferred_linalg_library()
    L, D = xq.block_LDL(G.clone(), 16)
    assert torch.backends.cuda.preferred_linalg_library() == before
    L64, D64 = xq.block_LDL(G.double(), 16)
    assert float((L.double() - L64).norm() / L64.norm()) < 1e-4
    R = L.double() @ torch.block_diag(*D.double()) @ L.double().t()
    assert float((R - G.double()).norm() / G.double().norm()) < 1e-5
    m = n // 16
    diag = torch.diagonal(L.view(m, 16, m, 16), dim1=0, dim2=2).permute(2, 0, 1)
    assert torch.equal(diag, torch.eye(16, device="cuda").expand(m, 16, 16))
    B = torch.randn(n, n, device="cuda")
    with pytest.raises(RuntimeError):
        xq.block_LDL(B + B.t(), 16)
    assert torch.backends.cuda.preferred_linalg_library() == before


def test_quantize_with_U_on_device(xq, oracle_mod, mul1_lut, cpu8):
    """quantize() with a U factor on device tensors (quantize.py:944-950): the
    U -> L conversion (triangular solve, G = U^-1 U^-T, block LDL) runs on
    the GPU in fp64 and agrees with the CPU conversion to fp64 rounding; the
    sweep (column chains) encodes every tile bit-exactly for the targets the
    kernel computed.  Against the reference's golden output: the sweep's
    feedback follows the reference's order, but the scale is a device mean
    and the factor the GPU's, so a tile whose targets move by an ulp may
    encode differently; with reference_arithmetic=True (scale and U -> L on
    the host) every output equals the golden one bit for bit."""
    e = load_golden("e2e_128.npz")
    Wt = torch.from_numpy(e["prep_Wt"])
    U = torch.from_numpy(e["q_U"])
    eye = torch.eye(U.shape[0], dtype=torch.float64)
    Lc = []
    for dev in ("cpu", "cuda"):
        Uu = U.double().to(dev)
        Ui = torch.linalg.solve_triangular(Uu, eye.to(dev), upper=True)
        Lc.append(xq.block_LDL(Ui @ Ui.t(), 16)[0].cpu())
    rel = float((Lc[1] - Lc[0]).norm() / Lc[0].norm())
    print(f"U->L on the GPU vs CPU: relative difference {rel:.2e}", flush=True)
    assert rel < 1e-12
    print("case quantize() with U on cuda, margin 16, seed 147", flush=True)
    xq.ldlq_viterbi.keep_targets = True
    try:
        W_hat, packed, scale = xq.quantize(Wt.cuda(), U.cuda(), "exl3_mul1", 4, seed=147,
                                           margin=16)
        xt = xq.ldlq_viterbi.last_targets
    finally:
        xq.ldlq_viterbi.keep_targets = False
        xq.ldlq_viterbi.last_targets = None
    assert W_hat.is_cuda and packed.is_cuda
    # the scale is a device mean here: its reduction order may move the last bit
    assert abs(np.float32(scale) - e["q_scale"]) <= np.spacing(e["q_scale"])
    st = oracle_mod.unpack(packed.cpu().numpy().reshape(-1, 64), 4)
    want = oracle_mod.tailbite(xt.reshape(-1, 256).cpu().numpy(), mul1_lut, 4, 16, pivot=147,
                               margin=16)
    np.testing.assert_array_equal(st, want)
    diff_tiles = int((packed.cpu().numpy() != e["q_packed"]).any(axis=2).sum())
    e_gpu = xq.rel_mse(Wt, W_hat.cpu())
    e_ref = xq.rel_mse(Wt, torch.from_numpy(e["q_W_hat"]))
    print(f"vs golden: {diff_tiles}/64 tiles differ, rel MSE {e_gpu:.6e} vs {e_ref:.6e}",
          flush=True)
    assert diff_tiles <= 4
    assert abs(e_gpu - e_ref) <= 1e-2 * e_ref
    print("case quantize() with U on cuda, reference_arithmetic", flush=True)
    for Ud in (U.cuda(), U):                  # device or host factor
        W_hat, packed, scale = xq.quantize(Wt.cuda(), Ud, "exl3_mul1", 4, seed=147, margin=16,
                                           reference_arithmetic=True)
        assert W_hat.is_cuda and packed.is_cuda
        np.testing.assert_array_equal(packed.cpu().numpy(), e["q_packed"])
        np.testing.assert_array_equal(W_hat.cpu().numpy(), e["q_W_hat"])
        assert np.float32(scale) == e["q_scale"]


def test_factor_hessian_fallback_on_device(xq):
    """The damping fallback (quantize.py:815-835) on a device matrix that is
    not positive definite: fp32 block LDL fails, fp64 with +0 and +0.1 x
    mean(diag) fail, +1.0 x mean(diag) succeeds; the factor reproduces the
    damped matrix and equals the CPU fallback's to fp64 rounding.  A
    non-finite matrix raises."""
    n = 256
    g = torch.Generator().manual_seed(3)
    Q, _ = torch.linalg.qr(torch.randn(n, n, generator=g, dtype=torch.float64))
    lam = torch.ones(n, dtype=torch.float64)
    lam[-1] = -0.5
    G = (Q * lam) @ Q.t()
    # the damping the fallback applies to the fp32 input taken to fp64:
    # +0.1 x mean(diag), then +1.0 x the new mean(diag)
    Gd = G.float().double()
    Gd.diagonal().add_(0.1 * Gd.diagonal().mean())
    Gd.diagonal().add_(1.0 * Gd.diagonal().mean())
    out = []
    for dev in ("cpu", "cuda"):
        L = xq._factor_hessian(G.float().to(dev))
        assert L.device.type == torch.device(dev).type
        out.append(L.double().cpu())
    assert float((out[1] - out[0]).norm() / out[0].norm()) < 1e-10
    _, D = xq.block_LDL(Gd.clone().cuda(), 16)
    L = out[1]
    R = L @ torch.block_diag(*D.double().cpu()) @ L.t()
    assert float((R - Gd).norm() / Gd.norm()) < 1e-10
    bad = G.float().cuda()
    bad[3, 5] = float("nan")
    with pytest.raises(RuntimeError):
        xq._factor_hessian(bad)


def test_progress_sequence_matches_block_schedule(xq, monkeypatch):
    """The column-chain schedule reports the reference's per-block progress
    (quantize.py:666,732-734): progress(i, 512 * blocks done) for i = tk-1
    .. 0, the same calls as the block schedule makes."""
    g = torch.Generator().manual_seed(2)
    W = (0.02 * torch.randn(128, 256, generator=g)).half().float()
    H = _ar1_hessian(256, 512, 0.5, 2)
    calls = {}
    for sched in ("chain", "block"):
        monkeypatch.setattr(xq, "DEFAULT_SCHEDULE", sched)
        seen = []
        xq.quantize_linear(W, H, K=4, device="cuda", margin=0,
                           progress=lambda i, s, seen=seen: seen.append((i, s)))
        calls[sched] = [c for c in seen if c[0] != "hinv"]
    tk = 256 // 16
    assert calls["chain"] == [(i, 512 * (tk - i)) for i in range(tk - 1, -1, -1)]
    assert calls["chain"] == calls["block"]
