#!/usr/bin/env python3
"""make_golden.py -- write the golden fixtures in tests/golden/ from the reference.

Run once, in the build container only (the reference tree is not present on
the GPU host):

    python tests/golden/make_golden.py /root/reference/quantize
    python tests/golden/make_golden.py /root/reference/quantize --ties
    python tests/golden/make_golden.py /root/reference/quantize --mid
    python tests/golden/make_golden.py /root/reference/quantize --codes

It imports the reference quantizer module (quantize/quantize.py) on CPU and
records input/output vectors for the functions that closed forms, invariants
and brute force cannot pin:
  * quantize_seq_tailbite states on Gaussian and tie-heavy inputs, every K in
    2..7, margins {0, 16}, pivots {0, 128, 147, 255}   (quantize.py:323-354)
  * viterbi() free and back_from runs                   (quantize.py:218-320)
  * pack_states / unpack_states / decode_trellis        (quantize.py:360-415)
  * sign_vec values                                     (quantize.py:179-182)
  * quantize_linear on a 128x128 weight, identity and AR(1) Hessians,
    channel_scales off and on                            (quantize.py:750-875)
  * quantize() harness with a U factor, margin 16        (quantize.py:894-966)
  * prepare_incoherence                                  (quantize.py:969-1058)
--ties writes ties.npz alone: quantize_seq_tailbite on 24 sequences per K
whose results hinge on exact cost ties (six kinds, tie_forcing_inputs) at four
pivot/margin pairs, and viterbi() pinned and back_from runs on them.
--codes writes codes.npz alone: the reference's decode tables of the other
V=1 codes (exl3_3inst, exl3_mcg, qtip_1mad; quantize.py:56-97) as SHA-256
digests of their fp32 bytes with their first 64 entries, and
quantize_seq_tailbite states with the qtip_1mad table on Gaussian and
tie-forcing sequences (the six kinds of --ties) at K = 2, 4, 7, margins
{0, 16}.
--mid writes e2e_mid.npz alone: quantize_linear with BlockLDLQ on a
1024x1024 weight (4,096 tiles, 64 blocks of feedback) against the Hessian
H[i][j] = 2^-|i-j| (exact in fp32), at K=4 and at K=5 with channel scales:
trellis, suh, svh, Wscale, the proxy loss (fp32 as the reference computes it,
and in fp64), a SHA-256 digest of W_hat, and a digest of the generating host's
per-output-channel RMS reduction (channel scales depend on it).
Only data (inputs and expected outputs) is written, as compressed .npz files
loadable with numpy.load(allow_pickle=False).
"""
from __future__ import annotations

import hashlib
import os
import sys
import time

import numpy as np
import torch

OUT = os.path.dirname(os.path.abspath(__file__))


def ar1_hessian(d: int, n_s: int, rho: float, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed + 100)
    Z = torch.randn(n_s, d, generator=g, dtype=torch.float64)
    X = torch.empty_like(Z)
    X[:, 0] = Z[:, 0]
    c = (1.0 - rho * rho) ** 0.5
    for i in range(1, d):
        X[:, i] = rho * X[:, i - 1] + c * Z[:, i]
    return (X.t() @ X / n_s).float()


def tie_heavy_inputs(lut: np.ndarray, rng: np.random.Generator, n: int):
    """Targets that force exact cost ties: exact LUT values, zeros, a coarse grid."""
    X = np.empty((n, 256), dtype=np.float32)
    for q in range(n):
        kind = q % 3
        if kind == 0:
            X[q] = lut[rng.integers(0, lut.size, 256)]
        elif kind == 1:
            X[q] = 0.0
            X[q, rng.integers(0, 256, 16)] = lut[rng.integers(0, lut.size, 16)]
        else:
            X[q] = np.round(rng.standard_normal(256) * 2.0) / 2.0
    return X


def tie_forcing_inputs(lut: np.ndarray, rng: np.random.Generator, n: int):
    """Six kinds of targets, four of each, under which exactly equal path
    costs decide the result.  Large targets round fl(f - x) and the growing
    fp32 sums onto a coarse grid, so many candidates tie exactly: N(0, 3000);
    U(-1e5, 1e5); U(-1e9, 1e9) (fl(f - x) = -x for every state: every
    candidate ties at every step); exact codebook values with every fourth
    target U(-1e5, 1e5).  Plus exact codebook values and midpoints of two
    codebook values (f_a - x = -(f_b - x) exactly, equal emissions)."""
    X = np.empty((n, 256), dtype=np.float32)
    vals = np.unique(lut)
    for q in range(n):
        kind = q % 6
        if kind == 0:
            X[q] = lut[rng.integers(0, lut.size, 256)]
        elif kind == 1:
            a = rng.integers(0, vals.size - 1, 256)
            b = np.minimum(vals.size - 1, a + rng.integers(1, 4, 256))
            X[q] = (vals[a].astype(np.float64) + vals[b]) / 2.0
        elif kind == 2:
            X[q] = rng.standard_normal(256) * 3000.0
        elif kind == 3:
            X[q] = rng.uniform(-1e5, 1e5, 256)
        elif kind == 4:
            X[q] = rng.uniform(-1e9, 1e9, 256)
        else:
            X[q] = lut[rng.integers(0, lut.size, 256)]
            X[q, ::4] = rng.uniform(-1e5, 1e5, 64)
    return X


def main_ties(refdir: str):
    sys.path.insert(0, refdir)
    import quantize as xq  # the reference module, CPU only
    torch.set_num_threads(8)
    lut = xq.get_lut("exl3_mul1", 16)
    lut_np = lut.numpy().astype(np.float32)
    t0 = time.time()
    rng = np.random.default_rng(20261202)
    data = {}
    for K in range(2, 8):
        X = tie_forcing_inputs(lut_np, rng, 24)
        data[f"X_K{K}"] = X
        Xt = torch.from_numpy(X.T.copy())                # [256, 24]
        for p, m in ((128, 0), (147, 16), (0, 0), (255, 16)):
            st = xq.quantize_seq_tailbite(Xt, lut, K, 16, pivot=p, margin=m)
            data[f"S_K{K}_m{m}_p{p}"] = st.t().numpy().astype(np.int32)
        ov = torch.from_numpy((np.arange(24) * 1237) % (1 << (16 - K)))
        data[f"VPov_K{K}"] = ov.numpy().astype(np.int32)
        data[f"VP_K{K}"] = xq.viterbi(Xt, lut, K, 16, overlap=ov).t().numpy().astype(np.int32)
        data[f"VB_K{K}"] = xq.viterbi(Xt[:200], lut, K, 16, back_from=60).numpy().astype(np.int32)
        print(f"  ties K={K} done {time.time() - t0:.1f}s", flush=True)
    np.savez_compressed(os.path.join(OUT, "ties.npz"), **data)


def main_codes(refdir: str):
    sys.path.insert(0, refdir)
    import quantize as xq  # the reference module, CPU only
    torch.set_num_threads(8)
    data = {}
    for name in ("exl3_3inst", "exl3_mcg", "qtip_1mad"):
        t = xq.get_lut(name, 16).numpy().astype(np.float32)
        data[f"sha256_{name}"] = np.frombuffer(hashlib.sha256(t.tobytes()).digest(),
                                               dtype=np.uint8)
        data[f"head_{name}"] = t[:64].copy()
    lut = xq.get_lut("qtip_1mad", 16)
    lut_np = lut.numpy().astype(np.float32)
    rng = np.random.default_rng(20261203)
    t0 = time.time()
    for K in (2, 4, 7):
        g = rng.standard_normal((2, 256)).astype(np.float32)
        ties = tie_forcing_inputs(lut_np, rng, 6)
        X = np.concatenate([g, ties], 0)                 # [8, 256]
        data[f"mad_X_K{K}"] = X
        Xt = torch.from_numpy(X.T.copy())
        for p, m in ((128, 0), (147, 16)):
            st = xq.quantize_seq_tailbite(Xt, lut, K, 16, pivot=p, margin=m)
            data[f"mad_S_K{K}_m{m}_p{p}"] = st.t().numpy().astype(np.int32)
        print(f"  qtip_1mad K={K} done {time.time() - t0:.1f}s", flush=True)
    np.savez_compressed(os.path.join(OUT, "codes.npz"), **data)


def kms_hessian(d: int) -> np.ndarray:
    """H[i][j] = 2^-|i-j| (the AR(1) correlation at rho = 1/2): every entry a
    power of two, so the fp32 matrix is exact and the same on every host."""
    i = np.arange(d)
    return np.ldexp(1.0, -np.abs(i[:, None] - i[None, :])).astype(np.float32)


def main_mid(refdir: str):
    sys.path.insert(0, refdir)
    import quantize as xq  # the reference module, CPU only
    torch.set_num_threads(8)
    t0 = time.time()
    rng = np.random.default_rng(20261202)
    W16 = (0.02 * rng.standard_normal((1024, 1024))).astype(np.float16)
    H = kms_hessian(1024)
    data = {"W16": W16}
    W = torch.from_numpy(W16.astype(np.float32))
    Ht = torch.from_numpy(H)
    # the channel-scale path reduces W with torch CPU means, whose rounding
    # depends on the host CPU: a digest of this host's per-output-channel RMS
    # lets a test tell whether its own host reduces identically
    W32 = W.t().contiguous()
    data["rout_sha256"] = np.frombuffer(hashlib.sha256(
        W32.square().mean(dim=0).sqrt().numpy().tobytes()).digest(), dtype=np.uint8)
    for tag, K, cs in (("k4", 4, False), ("k5cs", 5, True)):
        r = xq.quantize_linear(W, Ht, code="exl3_mul1", K=K, use_ldlq=True, margin=0,
                               channel_scales=cs, device="cpu")
        data[f"{tag}_trellis"] = r["trellis"].numpy()
        data[f"{tag}_suh"] = r["suh"].float().numpy()
        data[f"{tag}_svh"] = r["svh"].float().numpy()
        data[f"{tag}_Wscale"] = np.float32(r["Wscale"])
        data[f"{tag}_herr"] = np.float64(xq.hessian_weighted_err(W, r["W_hat"], Ht))
        # the same proxy loss in fp64 (its fp32 einsum rounds by the host's
        # reduction order) and a digest of W_hat's bytes
        dW = (r["W_hat"] - W).double()
        H64 = Ht.double()
        data[f"{tag}_herr64"] = np.float64(((dW @ H64) * dW).sum() /
                                           ((W.double() @ H64) * W.double()).sum())
        data[f"{tag}_What_sha256"] = np.frombuffer(
            hashlib.sha256(r["W_hat"].contiguous().numpy().tobytes()).digest(), dtype=np.uint8)
        print(f"  mid {tag} done {time.time() - t0:.1f}s", flush=True)
    np.savez_compressed(os.path.join(OUT, "e2e_mid.npz"), **data)


def main(refdir: str):
    sys.path.insert(0, refdir)
    import quantize as xq  # the reference module, CPU only
    torch.set_num_threads(8)
    lut = xq.get_lut("exl3_mul1", 16)
    lut_np = lut.numpy().astype(np.float32)
    np.savez_compressed(os.path.join(OUT, "lut_mul1.npz"), lut=lut_np,
                        perm=xq.tensor_core_perm().numpy().astype(np.int32))

    # ---------------------------------------------------- tail-bite states
    t0 = time.time()
    rng = np.random.default_rng(20261011)
    pivots = (0, 128, 147, 255)
    margins = (0, 16)
    data = {}
    for K in range(2, 8):
        g = rng.standard_normal((3, 256)).astype(np.float32)
        ties = tie_heavy_inputs(lut_np, rng, 3)
        X = np.concatenate([g, ties], 0)                 # [6, 256]
        data[f"X_K{K}"] = X
        Xt = torch.from_numpy(X.T.copy())                # [256, 6]
        for m in margins:
            for p in pivots:
                st = xq.quantize_seq_tailbite(Xt, lut, K, 16, pivot=p, margin=m)
                data[f"S_K{K}_m{m}_p{p}"] = st.t().numpy().astype(np.int32)
        # plain viterbi: free, and back_from on a truncated run
        st = xq.viterbi(Xt, lut, K, 16)
        data[f"V_K{K}"] = st.t().numpy().astype(np.int32)
        sb = xq.viterbi(Xt[:150], lut, K, 16, back_from=100)
        data[f"VB_K{K}"] = sb.numpy().astype(np.int32)
        ov = torch.from_numpy((np.arange(6) * 977) % (1 << (16 - K)))
        sp = xq.viterbi(Xt, lut, K, 16, overlap=ov)
        data[f"VP_K{K}"] = sp.t().numpy().astype(np.int32)
        data[f"VPov_K{K}"] = ov.numpy().astype(np.int32)
        # pack / unpack / decode of the pass-2 states (pivot 128, margin 0)
        s128 = torch.from_numpy(data[f"S_K{K}_m0_p128"].astype(np.int64))
        packed = xq.pack_states(s128, K)
        data[f"P_K{K}"] = packed.numpy()
        data[f"U_K{K}"] = xq.unpack_states(packed, K).numpy().astype(np.int32)
        tr = packed.view(2, 3, 16 * K)
        data[f"D_K{K}"] = xq.decode_trellis(tr, lut, K, 32, 48).numpy()
        print(f"  K={K} done {time.time() - t0:.1f}s", flush=True)
    np.savez_compressed(os.path.join(OUT, "tailbite.npz"), **data)

    # ----------------------------------------------------------- sign vectors
    sv = {f"sign_{n}_{s}": xq.sign_vec(n, s).numpy().astype(np.float32)
          for n in (128, 256) for s in (20261011, 20261012, 7)}
    np.savez_compressed(os.path.join(OUT, "sign_vec.npz"), **sv)

    # ------------------------------------------------- end-to-end, 128 x 128
    e2e = {}
    g0 = torch.Generator().manual_seed(0)
    W = torch.randn(128, 128, generator=g0).half().float()
    H_ar = ar1_hessian(128, 512, 0.5, 0)
    e2e["W"] = W.numpy()
    e2e["H_ar"] = H_ar.numpy()
    cases = (("id", torch.eye(128), False, True),
             ("ar", H_ar, False, True),
             ("arcs", H_ar, True, True),
             ("nold", H_ar, False, False))
    for tag, H, cs, ldlq in cases:
        r = xq.quantize_linear(W, H, code="exl3_mul1", K=4, use_ldlq=ldlq,
                               margin=0, channel_scales=cs)
        e2e[f"{tag}_W_hat"] = r["W_hat"].numpy()
        e2e[f"{tag}_trellis"] = r["trellis"].numpy()
        e2e[f"{tag}_suh"] = r["suh"].float().numpy()
        e2e[f"{tag}_svh"] = r["svh"].float().numpy()
        e2e[f"{tag}_Wscale"] = np.float32(r["Wscale"])
        e2e[f"{tag}_herr"] = np.float64(xq.hessian_weighted_err(W, r["W_hat"], H))
        e2e[f"{tag}_relmse"] = np.float64(xq.rel_mse(W, r["W_hat"]))
        print(f"  quantize_linear {tag} done {time.time() - t0:.1f}s", flush=True)

    # quantize() harness: inner-domain weight + U factor (U^T U = G^-1)
    prep = xq.prepare_incoherence(W, H_ar, channel_scales=True)
    e2e["prep_Wt"] = prep["Wt"].numpy()
    e2e["prep_G"] = prep["G"].numpy()
    e2e["prep_suh"] = prep["suh"].numpy()
    e2e["prep_svh"] = prep["svh"].numpy()
    G = prep["G"].clone()
    G.diagonal().add_(0.01 * G.diagonal().mean())
    Gi = torch.cholesky_inverse(torch.linalg.cholesky(G.double()))
    U = torch.linalg.cholesky(Gi, upper=True).float()
    e2e["q_U"] = U.numpy()
    Wh, packed, scale = xq.quantize(prep["Wt"], U, "exl3_mul1", 4, seed=147,
                                    margin=16)
    e2e["q_W_hat"] = Wh.numpy()
    e2e["q_packed"] = packed.numpy()
    e2e["q_scale"] = np.float32(scale)
    Wh0, packed0, scale0 = xq.quantize(prep["Wt"][:64], None, "exl3_mul1", 3,
                                       seed=5, margin=0)
    e2e["q0_W_hat"] = Wh0.numpy()
    e2e["q0_packed"] = packed0.numpy()
    e2e["q0_scale"] = np.float32(scale0)
    np.savez_compressed(os.path.join(OUT, "e2e_128.npz"), **e2e)
    print(f"done {time.time() - t0:.1f}s")


if __name__ == "__main__":
    args = [a for a in sys.argv[1:] if not a.startswith("--")]
    ref = args[0] if args else "/root/reference/quantize"
    if "--ties" in sys.argv[1:]:
        main_ties(ref)
    elif "--mid" in sys.argv[1:]:
        main_mid(ref)
    elif "--codes" in sys.argv[1:]:
        main_codes(ref)
    else:
        main(ref)
