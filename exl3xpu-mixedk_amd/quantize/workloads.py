"""workloads.py -- the synthetic weight/Hessian workloads the encoder is
measured and checked on (there are no checkpoints or calibration sets here).

Every workload is fixed by a seed.  g(s) is torch.Generator("cpu") seeded
with s; weights are drawn in fp32 and rounded to fp16 (the quantizer input
dtype of the reference's harness); Hessians follow one recipe:

    X [n_s, d], X[:, 0] = Z[:, 0], X[:, i] = rho X[:, i-1] + sqrt(1-rho^2) Z[:, i]
    Z ~ N(0, 1) fp64 from g(s + 100),   H = X^T X / n_s  (fp32)

i.e. the input Gram of n_s samples with AR(1) correlation rho across input
channels, rank min(n_s, d) before the quantizer's own 1 % damping
(quantize.py:806-814).

  c1  128x128 N(0,1), H = I, K=4                    64 tiles (reference CPU size)
  c2  4096x4096 N(0,0.02), AR(1) rho=0.5, K=4        65,536 tiles
  c3  5120x5120 N(0,0.02) + 0.1 % outliers at 10 sigma, AR(1) rho=0.5, K=2..7
  c4  fused qkv: q 6144x5120 K=5, k/v 1024x5120 K=7, shared AR(1) rho=0.3,
      channel scales on; an fp16 activation x [1, 5120] for the GEMV check
  c5  17408-in x 5120-out down projection, Student-t(5) scaled to std 0.02,
      AR(1) rho=0.5 at d=17408 from n_s=4096 samples, K=6 (and K=4)

c5_tiles() gives the kernel-throughput workload: every 16x16 tile of c5's
weight after the incoherence transform and the unit-rms scale, without
BlockLDLQ feedback (348,160 independent 256-step sequences).

Shapes are nn.Linear [out, in]; H is [in, in].  `scale` shrinks every
dimension by an integer factor (multiples of 128 kept) for quick checks.
"""
from __future__ import annotations

import math

import torch


def g(s: int) -> torch.Generator:
    return torch.Generator(device="cpu").manual_seed(int(s))


def ar1_gram(d: int, n_s: int, rho: float, seed: int, device="cpu") -> torch.Tensor:
    """H = X^T X / n_s for n_s AR(1)-correlated samples of dimension d (fp32).
    Z is drawn and the recursion run on the CPU in fp64 (one rounded multiply,
    multiply and add per element, as on any device: reproducible anywhere,
    and no per-channel device launches); the Gram product runs on `device`."""
    Z = torch.randn(n_s, d, generator=g(seed + 100), dtype=torch.float64)
    Zt = Z.t().contiguous()                                 # rows = channels
    del Z
    Xt = torch.empty_like(Zt)
    Xt[0] = Zt[0]
    c = math.sqrt(1.0 - rho * rho)
    a, b = torch.empty_like(Zt[0]), torch.empty_like(Zt[0])
    for i in range(1, d):
        torch.mul(Xt[i - 1], rho, out=a)
        torch.mul(Zt[i], c, out=b)
        torch.add(a, b, out=Xt[i])
    del Zt, a, b
    Xt = Xt.to(device)
    H = (Xt @ Xt.t()) / n_s
    return H.float()


def _dim(n: int, scale: int) -> int:
    return max(128, (n // scale) // 128 * 128)


def c1() -> dict:
    W = torch.randn(128, 128, generator=g(0)).half()
    return {"name": "c1", "W": W, "H": torch.eye(128), "K": 4, "channel_scales": False}


def c2(scale: int = 1, device="cpu") -> dict:
    d = _dim(4096, scale)
    W = (0.02 * torch.randn(d, d, generator=g(1))).half()
    H = ar1_gram(d, _dim(4096, scale), 0.5, 1, device)
    return {"name": "c2", "W": W, "H": H, "K": 4, "channel_scales": False}


def c3(scale: int = 1, device="cpu") -> dict:
    d = _dim(5120, scale)
    gen = g(2)
    W = 0.02 * torch.randn(d, d, generator=gen)
    n_out = round(0.001 * d * d)
    pos = torch.randperm(d * d, generator=gen)[:n_out]
    sign = torch.where(torch.rand(n_out, generator=gen) < 0.5, -1.0, 1.0)
    W.view(-1)[pos] = 0.2 * sign
    H = ar1_gram(d, _dim(4096, scale), 0.5, 2, device)
    return {"name": "c3", "W": W.half(), "H": H, "Ks": (2, 3, 4, 5, 6, 7),
            "channel_scales": False}


def c4(scale: int = 1, device="cpu") -> dict:
    d = _dim(5120, scale)
    members = []
    for name, rows, K, s in (("q_proj", 6144, 5, 3), ("k_proj", 1024, 7, 4),
                             ("v_proj", 1024, 7, 5)):
        W = (0.02 * torch.randn(_dim(rows, scale), d, generator=g(s))).half()
        members.append({"module": f"self_attn.{name}", "W": W, "K": K})
    H = ar1_gram(d, _dim(4096, scale), 0.3, 3, device)
    x = torch.randn(1, d, generator=g(777 + 1)).half()
    return {"name": "c4", "members": members, "H": H, "x": x, "channel_scales": True}


def c5_weight(device="cpu", scale: int = 1, seed: int = 4) -> torch.Tensor:
    """Student-t(5) weight [5120 out, 17408 in] scaled to std 0.02 (the
    variance of Student-t(5) is 5/3), fp16, sampled on `device` under
    torch.manual_seed(seed)."""
    torch.manual_seed(seed)
    t = torch.distributions.StudentT(torch.tensor(5.0, device=device))
    W = t.sample((_dim(5120, scale), _dim(17408, scale))) * (0.02 / (5.0 / 3.0) ** 0.5)
    return W.half()


def c5(scale: int = 1, device="cpu") -> dict:
    W = c5_weight(device, scale)
    H = ar1_gram(W.shape[1], _dim(4096, scale), 0.5, 4, device)
    return {"name": "c5", "W": W, "H": H, "Ks": (6, 4), "channel_scales": False}


def c5_tiles(device="cuda", seed: int = 4) -> torch.Tensor:
    """The 348,160 tile targets of c5's weight without feedback: random-sign
    + Hadamard incoherence (signs from seeds 20261011 / 20261012, as
    quantize_linear), the unit-rms scale against the mul1 codebook, and each
    16x16 tile's sequence x_t = tile[perm[t]] -> [348160, 256] fp32 on
    `device` (tile (a, b) of the [17408 in, 5120 out] inner weight at row
    a * 320 + b)."""
    import quantize as xq
    dev = torch.device(device)
    W = c5_weight(dev, seed=seed).float()                    # [5120 out, 17408 in]
    out_f, in_f = W.shape
    suh = xq.sign_vec(in_f, 20261011, dev).half()
    svh = xq.sign_vec(out_f, 20261012, dev).half()
    h = xq.hadamard128(dev, torch.float32)
    Wi = xq.to_inner(W.t().contiguous(), suh, svh, h)         # [k, n]
    del W
    lut_rms = xq.get_lut("exl3_mul1").double().square().mean().sqrt().float()
    Wq = Wi / (Wi.square().mean().sqrt() / lut_rms.to(dev))
    del Wi
    tk, tn = in_f // 16, out_f // 16
    perm = xq.tensor_core_perm().to(dev)
    X = Wq.view(tk, 16, tn, 16).permute(0, 2, 1, 3).reshape(tk * tn, 256)[:, perm]
    return X.contiguous()
